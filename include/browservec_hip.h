/*
 * browservec_hip.h -- C ABI of libbrowservec_hip.so, the MI355X (gfx950)
 * implementation of BrowserVec's data-parallel search path.
 *
 * The ABI mirrors the reference's index seam: the `VectorIndex` interface
 * (src/index/flat.ts:30-40) with its duck-typed extras (queryMasked,
 * queryBatch, setNprobe, getters; src/index.ts:78-80, 352-354, 477-501,
 * 702-750), the engine's `DeviceContext` (src/engine/device.ts:3-9) and
 * `BrowserVec.rerankExact` (src/index.ts:583-594).  Plain pointers and sizes
 * only; every call returns a status code and leaves a message for
 * bv_last_error() on failure.  Host pointers are caller-owned and consumed
 * before the call returns.
 *
 * Scores follow the reference: higher is closer; cosine and dot are the dot
 * product (rows and queries arrive already normalized for cosine, as
 * Store.prepare does), l2 is the negative squared distance.  Results come
 * back in canonical order: score descending, then row ascending.
 *
 * Thread safety: one index may be used by one thread at a time (the
 * reference awaits queries serially per store, src/engine/profile.ts:11-14);
 * different indexes may be used concurrently.
 */
#ifndef BROWSERVEC_HIP_H
#define BROWSERVEC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BV_ABI_VERSION 1

/* Status codes.  The message text of BV_E_INVALID for a length mismatch is
 * the reference's: "expected <n> floats, got <m>" (src/index/flat.ts:96-98). */
#define BV_OK 0
#define BV_E_INVALID 1     /* bad argument (lengths, dims, k, null pointers)          */
#define BV_E_UNSUPPORTED 2 /* combination the reference rejects (buildIndex, index.ts:119-141) */
#define BV_E_DEVICE_LOST 3 /* "GPU device lost; re-create the store" (flat.ts:137)  */
#define BV_E_OOM 4         /* device allocation failed                             */
#define BV_E_HIP 5         /* any other HIP runtime error                          */
#define BV_E_STATE 6       /* call not valid in the current state                  */

/* Index kinds: the classes buildIndex constructs (src/index.ts:105-142). */
#define BV_KIND_FLAT 0     /* FlatIndex      src/index/flat.ts:42      */
#define BV_KIND_QUANT 1    /* QuantIndex     src/index/quant.ts:21     */
#define BV_KIND_IVF 2      /* IVFIndex       src/index/ivf.ts:51       */
#define BV_KIND_IVFQUANT 3 /* IVFQuantIndex  src/index/ivfquant.ts:33  */

/* Metric (src/types.ts `Metric`). */
#define BV_METRIC_COSINE 0
#define BV_METRIC_DOT 1
#define BV_METRIC_L2 2

/* Scorer for quantized kinds.  ASYM is the reference's (fp32 rotated query x
 * dequantized codes, src/engine/wgsl/distanceQ{8,4,1}.ts).  HAMMING (1-bit
 * only) scores P - 2*popcount(code ^ sign_bits(query)); INT8SYM (int8 only)
 * quantizes the query with quantizeRow and scores the exact int32 dot.  The
 * last two have no reference counterpart; they are integer and exact. */
#define BV_SCORER_ASYM 0
#define BV_SCORER_HAMMING 1
#define BV_SCORER_INT8SYM 2

typedef struct bv_device bv_device;
typedef struct bv_index bv_index;
typedef struct bv_graph bv_graph;

/* Index description: buildIndex's arguments (dim, metric, quantBits, quant,
 * ann, chunkRows; src/index.ts:105-113) with the QuantConfig and IVFParams
 * fields (src/types.ts:116-128, src/index/ivf.ts:29-49).  Zero means "the
 * reference default" for every optional field. */
typedef struct bv_index_desc {
    uint32_t size;          /* sizeof(bv_index_desc); 72 (no ivf_incremental) is read
                             * with ivf_incremental = 0                               */
    uint32_t kind;          /* BV_KIND_*                                             */
    uint32_t dim;           /* vector dimension (> 0)                                */
    uint32_t metric;        /* BV_METRIC_*                                           */
    uint32_t bits;          /* 0 (fp32), 8, 4, 1                                     */
    uint32_t scorer;        /* BV_SCORER_*                                           */
    uint32_t seed;          /* rotation seed; has_seed=0 -> 0x9e3779b9 (index.ts:71) */
    uint32_t has_seed;
    uint32_t rounds;        /* Hadamard rounds; 0 -> 2 (index.ts:115)                */
    uint32_t chunk_rows;    /* forced rows per chunk (reported only; one buffer here) */
    uint32_t nlist;         /* IVF: 0 -> round(sqrt(rows)) clamped [16,4096]         */
    uint32_t nprobe;        /* IVF: 0 -> tuned or 5% of nlist                        */
    uint32_t sample_size;   /* IVF reservoir; 0 -> 50000 (min 1024)                  */
    uint32_t train_size;    /* IVF k-means rows; 0 -> 16384                          */
    uint32_t iters;         /* IVF Lloyd iterations; 0 -> 8 (quant) / 8 (fp32)       */
    uint32_t ivf_seed;      /* IVF seed; has_ivf_seed=0 -> reference default         */
    uint32_t has_ivf_seed;
    float target_recall;    /* IVF: < 0 -> unset                                     */
    uint32_t ivf_incremental; /* IVF: 1 -> appends after a build assign the new rows
                               * to the current centroids and extend the lists; 0 ->
                               * the reference's rebuild on the next query
                               * (src/index/ivfquant.ts:462)                          */
} bv_index_desc;

/* Stats (the index-derived fields of `Stats`, src/types.ts:253-300, and
 * src/index.ts:702-750) plus device timings. */
typedef struct bv_index_stats {
    uint64_t rows;            /* VectorIndex.size                                     */
    uint32_t dim;
    uint32_t padded_dim;      /* quantized kinds: padToPow2(dim)                      */
    uint32_t words_per_row;   /* quantized kinds                                      */
    uint32_t bits;
    uint32_t chunk_count;     /* chunkCount getter                                    */
    uint32_t nlist;           /* nlist getter (0 until built)                         */
    uint32_t nprobe;          /* nprobe getter (0 until built)                        */
    float tuned_recall;       /* tunedRecall getter; < 0 when unset                   */
    double last_query_ms;     /* host wall time of the last query call                */
    double last_query_gpu_ms; /* device time of the last query (HIP events)           */
    double build_ms;          /* last IVF build                                       */
    uint64_t device_bytes;    /* HBM held by the index                                */
    uint64_t last_scanned_rows;
    uint64_t build_exact_rows;  /* last IVF build's final assignment: rows assigned by
                                 * the exact fp32 arithmetic alone (all of them, or
                                 * those the int8 matrix pass left open)            */
} bv_index_stats;

/* ---- errors / version ---------------------------------------------------- */
const char *bv_last_error(void); /* thread-local message of the last failure */
int bv_abi_version(void);

/* ---- device (DeviceContext, src/engine/device.ts:3-76) -------------------- */
/* acquireDevice (device.ts:22-50): open HIP device `ordinal`. */
int bv_device_open(int ordinal, bv_device **out);
/* device.destroy() (src/index.ts:753-756). */
int bv_device_close(bv_device *dev);
/* DeviceContext.lost (device.ts:68-76). */
int bv_device_is_lost(const bv_device *dev, int *lost);
/* Failure injection for tests of the error paths.  The reference's device
 * loss comes from the browser (GPUDevice.lost sets DeviceContext.lost,
 * src/engine/device.ts:68-76; queries then throw "GPU device lost; re-create
 * the store", src/index/flat.ts:137); these host-side flags force the same
 * conditions without touching the GPU. */
#define BV_INJECT_LOST 1       /* mark the device lost: every later call fails with BV_E_DEVICE_LOST */
#define BV_INJECT_APPEND_OOM 2 /* the next append fails as if a device allocation failed; the index is unchanged */
#define BV_INJECT_APPEND_LATE 3 /* the next append fails after its rows are uploaded and encoded, before its
                                 * reservoir sample and lists are committed; the index is unchanged */
int bv_debug_inject(bv_device *dev, int what);
/* Device name, compute-unit count and HBM size. */
int bv_device_info(const bv_device *dev, char *name, uint32_t name_len, uint32_t *cu_count, uint64_t *hbm_bytes);

/* ---- index lifecycle ------------------------------------------------------ */
/* buildIndex (src/index.ts:105-142): same validation and error messages. */
int bv_index_create(bv_device *dev, const bv_index_desc *desc, bv_index **out);
/* VectorIndex.destroy (flat.ts:39). */
int bv_index_destroy(bv_index *idx);
/* VectorIndex.size (flat.ts:31). */
int bv_index_size(const bv_index *idx, uint64_t *rows);

/* VectorIndex.append (flat.ts:37, quant.ts:129-140, ivfquant.ts:216-233):
 * `data` holds n_floats = count*dim prepared floats (normalized for cosine).
 * Quantized kinds rotate+quantize on the device. */
int bv_index_append(bv_index *idx, const float *data, uint64_t n_floats, uint64_t count);

/* ---- queries ---------------------------------------------------------------- */
/* VectorIndex.query (flat.ts:38): top-k of one query.  Flat kinds are exact;
 * quantized kinds return the approximate top-k by code score (the caller
 * re-ranks, as BrowserVec.query does).  *n_out = min(k, rows).  Any k on
 * flat kinds (above 1024: every row's score, then a device sort); IVF
 * kinds serve k <= 1024. */
int bv_index_query(bv_index *idx, const float *q, uint32_t k, uint32_t *rows, float *scores, uint32_t *n_out);

/* queryMasked (flat.ts:128-130, quant.ts:174-176): rows whose bit (LSB-first,
 * row r -> word r>>5) is clear never enter the top-k; *n_out may be < k. */
int bv_index_query_masked(bv_index *idx, const float *q, uint32_t k, const uint32_t *mask_words,
                          uint64_t n_words, uint32_t *rows, float *scores, uint32_t *n_out);

/* queryBatch (src/index.ts:499-501): nq queries (nq*dim floats); results
 * row-major [nq][k], n_out[nq].  Equal to looping bv_index_query: rows and
 * score bits (8 or more queries on a flat fp32 or int8 / int4 index run on
 * the matrix cores as a prefilter; the rows it keeps are scored with the
 * single-query arithmetic). */
int bv_index_query_batch(bv_index *idx, const float *queries, uint32_t nq, uint32_t k, uint32_t *rows,
                         float *scores, uint32_t *n_out);

/* setNprobe (ivfquant.ts:154-156): per-query override for the next query
 * call, consumed once (0 clears). */
int bv_index_set_nprobe(bv_index *idx, uint32_t nprobe);

/* BrowserVec.rerankExact (src/index.ts:583-594): score the candidate rows
 * with Store.dotRow's f64 arithmetic (store.ts:114-130) against the stored
 * fp32 rows and return their top-k.  Needs rows kept on the device (all
 * quantized kinds keep them). */
int bv_index_rerank(bv_index *idx, const float *q, const uint32_t *cand, uint32_t n_cand, uint32_t k,
                    uint32_t *rows, float *scores, uint32_t *n_out);

/* BrowserVec.queryRowsExact (src/index.ts:445-464): the exact score of each
 * listed row against q -- Store.dotRow (store.ts:114-130), or Store.l2Row
 * (store.ts:137-160) on an l2 index, in their f64 order, stored as f32 --
 * and the top k of them, ordered (score desc, row asc).  Any k and any
 * number of rows; a row >= size fails with BV_E_INVALID.  The reference
 * runs this on the host for filters that match few rows (and for selective
 * filters on IVF indexes); here it runs on the stored device rows. */
int bv_index_query_rows(bv_index *idx, const float *q, const uint32_t *list, uint64_t n_list, uint32_t k,
                        uint32_t *rows, float *scores, uint32_t *n_out);
/* bv_index_query_rows over the rows whose bit is set in mask_words (the
 * queryMasked layout, scoreMask.ts:23-98: bit r & 31 of word r >> 5; bits at
 * or past size are ignored, a short mask leaves the remaining rows out).  The
 * row list is built on the device from the mask. */
int bv_index_query_rows_masked(bv_index *idx, const float *q, const uint32_t *mask_words, uint64_t n_words,
                               uint32_t k, uint32_t *rows, float *scores, uint32_t *n_out);

/* BrowserVec.query's quantized path in one device round trip (index.ts:
 * 402-421): approximate top-`fetch`, then exact re-rank to top-`k`.  With
 * fetch == 0 no re-rank happens and the approximate top-k is returned.
 * queries: nq*dim floats; rows/scores [nq][k]; n_out[nq]. */
int bv_index_search(bv_index *idx, const float *queries, uint32_t nq, uint32_t fetch, uint32_t k,
                    uint32_t *rows, float *scores, uint32_t *n_out);

/* ---- device-resident variants (serving loops, benchmarks) ------------------ */
/* Same as bv_index_search with every pointer in device memory; enqueued on
 * the index's stream and returns without waiting, except for batches of 8 or
 * more queries on a flat int8/int4/fp32 index, which run on the matrix cores
 * and wait once for the batch (one overflow flag per query is read back). */
int bv_index_search_device(bv_index *idx, const float *d_queries, uint32_t nq, uint32_t fetch, uint32_t k,
                           uint32_t *d_rows, float *d_scores, uint32_t *d_n_out);

/* Query streams for bv_index_search_device (no counterpart in the
 * reference; for callers that keep several single queries in flight):
 * n = 2 to 4 lets consecutive fused calls (fewer than 8 queries per call,
 * no mask) take the index's stream and n - 1 further streams in turn, each
 * with its own scan scratch (IVF indexes: also its own probe and candidate
 * buffers), so one query's final selection overlaps the next query's scan.
 * Calls in flight may then run at once: each needs its own output buffers.
 * bv_index_sync waits for every stream; appends wait for queries still
 * running.  n = 1 (default): one stream. */
int bv_index_set_query_streams(bv_index *idx, uint32_t n);
/* bv_index_search_device for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It has no counterpart in the reference.  Every query runs the
 * fused single-query scan with its scratch in a library-owned array of
 * BV_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; the call
 * allocates nothing and launches only kernels (no memset or copy nodes).
 * Serves flat indexes and quantized indexes whose scan transforms queries
 * in-kernel (int8 / int4 / 1-bit / Hamming at padded dimensions 64..1024),
 * not IVF.  BV_E_INVALID when nq, fetch and k need more scratch than the
 * array holds (about 10.5 MB per query at 1M rows and fetch 100).  All calls
 * on one GPU share the array: calls that overlap on that GPU (other streams,
 * other threads, other indexes) race. */
#define BV_NOALLOC_SCRATCH_BYTES (64u << 20)
int bv_index_search_device_noalloc(bv_index *idx, const float *d_queries, uint32_t nq, uint32_t fetch, uint32_t k,
                                   uint32_t *d_rows, float *d_scores, uint32_t *d_n_out);
/* Append rows that already live in device memory (count*dim floats). */
int bv_index_append_device(bv_index *idx, const float *d_data, uint64_t count);
/* Wait for all work enqueued on the index's stream. */
int bv_index_sync(bv_index *idx);
/* The index's HIP stream (hipStream_t) as an opaque pointer. */
int bv_index_stream(bv_index *idx, void **stream);
/* Per-kernel device timing with HIP events on the index's stream.  enable=1
 * starts counting (and resets), enable=0 stops.  Reports the summed duration
 * and launch count of the scan kernel (the dominant one). */
int bv_index_kernel_timing(bv_index *idx, int enable, double *scan_ms, uint64_t *scan_launches);

/* ---- stats / parity exports --------------------------------------------------- */
int bv_index_get_stats(bv_index *idx, bv_index_stats *out);
/* Codes and scales of rows [row0, row0+count) (words_per_row u32 per row). */
int bv_index_export_codes(bv_index *idx, uint64_t row0, uint64_t count, uint32_t *words, float *scales);
/* The scan's score for every row for one query (rows floats): the dense
 * scores the reference's distance kernels leave in their score buffer. */
int bv_index_export_scores(bv_index *idx, const float *q, float *scores);
/* The device-rotated query (padded_dim floats), quantized kinds only. */
int bv_index_export_rotated_query(bv_index *idx, const float *q, float *rotated);

/* ---- IVF ------------------------------------------------------------------------ */
/* IVFIndex / IVFQuantIndex build (src/index/ivf.ts:191-259,
 * src/index/ivfquant.ts:248-312): k-means on the reservoir sample, final
 * assignment, CSR lists.  Queries build on demand after appends, as the
 * reference does; this entry builds now.  With desc.ivf_incremental, appends
 * after a build extend the lists instead (the new rows assigned to the
 * current centroids); this entry then retrains over the reservoir and
 * reassigns every row, giving the lists the reference would build. */
int bv_index_build(bv_index *idx);
/* The built IVF state for parity checks: centroids (nlist x D floats, D =
 * padded_dim for quantized kinds, dim for fp32), list offsets (nlist+1) and
 * list rows (rows, ascending within a list).  Any pointer may be null.
 * Stale lists are built first, as a query would; lists extended by
 * incremental appends are exported as they stand. */
int bv_index_export_ivf(bv_index *idx, float *centroids, uint32_t *list_off, uint32_t *list_rows);

/* Index section for snapshots (src/persist/format.ts:1-22, whose v2 HNSW
 * graph section is the precedent; src/index.ts:673-700 re-encodes and
 * re-trains on load instead): the codes and scales of quantized kinds and the
 * IVF state (reservoir rows and ids, centroids, CSR lists, tuned nprobe).
 * The snapshot's fp32 rows stay where the reference keeps them.
 * bv_index_save_section writes *size bytes to buf when cap >= *size; with
 * buf == NULL or a smaller cap it only reports *size. */
int bv_index_save_section(bv_index *idx, void *buf, uint64_t cap, uint64_t *size);
/* Fills an empty index from the snapshot's rows (count*dim prepared floats,
 * as append takes them) and a saved section, without encoding or training.
 * The index must have been created with the descriptor the section was saved
 * under (BV_E_INVALID otherwise).  Appends after a load continue exactly as
 * on the saved index. */
int bv_index_load_section(bv_index *idx, const float *data, uint64_t n_floats, uint64_t count, const void *section,
                          uint64_t bytes);
/* pickProbes' scores (src/index/ivfquant.ts:495-509: the f64 4-way strided
 * dot of the rotated query with every centroid, stored as f32) for nq
 * queries: scores[nq][nlist].  Batches of 8 or more run the batched probe
 * kernel, fewer the single-query one; both give the same bits. */
int bv_index_export_probe_scores(bv_index *idx, const float *queries, uint32_t nq, float *scores);

/* ---- graph search (HNSW layer 0) ------------------------------------------ */
/* HNSWGpuSearcher (src/index/hnswGpu.ts:28-244): the host's HNSW build keeps
 * the graph; this object holds the corpus rows and the flat layer-0
 * adjacency on the device and beam-searches query batches
 * (src/engine/wgsl/graphSearch.ts:62-259), one wave per query.  degree is
 * the adjacency's fixed out-degree (2M), at most 64; metric BV_METRIC_* (the
 * rows and queries arrive prepared, as for an index). */
int bv_graph_create(bv_device *dev, uint32_t dim, uint32_t metric, uint32_t degree, bv_graph **out);
int bv_graph_destroy(bv_graph *g);
/* HNSWGpuSearcher.append (hnswGpu.ts:83-109): mirror appended rows. */
int bv_graph_append(bv_graph *g, const float *data, uint64_t n_floats, uint64_t count);
/* HNSWGpuSearcher.uploadGraph (hnswGpu.ts:112-126): the layer-0 adjacency,
 * rows x degree row ids, 0xffffffff for an empty slot.  Rows past the
 * adjacency have no neighbours; ids at or past the corpus rows are skipped. */
int bv_graph_upload(bv_graph *g, const uint32_t *links, uint64_t rows);
/* HNSWGpuSearcher.search (hnswGpu.ts:134-206): beam width
 * min(max(ef, k), 256), as many expansions, seeds = entry plus up to seven
 * rows spread over the adjacency; per query the beam's ids deduped, sorted
 * by score (-distance: dot for dot / cosine, -squared distance for l2) with
 * ties in beam order, the first k: rows / scores [nq][k], n_out[nq]. */
int bv_graph_search(bv_graph *g, const float *queries, uint32_t nq, uint32_t k, uint32_t ef, uint32_t entry,
                    uint32_t *rows, float *scores, uint32_t *n_out);
/* Parity export: the raw beams ([nq][256] distances and ids, unsorted, empty
 * slots 3.4e38 / 0xffffffff) for explicit seeds, beam width and expansion
 * cap. */
int bv_graph_search_beams(bv_graph *g, const float *queries, uint32_t nq, const uint32_t *entries,
                          uint32_t n_entries, uint32_t ef, uint32_t iter_cap, float *beam_dist, uint32_t *beam_id);

#ifdef __cplusplus
}
#endif

#endif /* BROWSERVEC_HIP_H */
