// Launch interface between the host runtime (bv_api.cpp) and the gfx950
// kernels (bv_kernels.hip).  Internal to libbrowservec_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

namespace bvk {

// Code layouts the scan understands.
enum CodecId : int {
    C_F32DOT = 0,   // fp32 rows, dot / cosine        (16-byte units = 4 floats)
    C_F32L2 = 1,    // fp32 rows, negative squared l2 (16-byte units)
    C_Q8 = 2,       // int8 codes, asymmetric          (16-byte units = 16 codes)
    C_Q4 = 3,       // int4 codes, asymmetric          (16-byte units = 32 codes)
    C_Q1A = 4,      // 1-bit codes, asymmetric         (4-byte units = 32 codes)
    C_HAM = 5,      // 1-bit codes, Hamming            (16-byte units = 128 bits)
    C_I8S = 6,      // int8 codes x int8 query         (16-byte units)
    C_F32DOT_S = 7, // fp32 rows, dim % 4 != 0         (4-byte units = 1 float)
    C_F32L2_S = 8,
    C_Q1P = 9,      // 1-bit codes, asymmetric, scored through the query's int8 +
                    // int4 bit planes with an exact fp32 re-score near the
                    // bound (16-byte units = 128 codes)
    C_COUNT = 10,
    // query-level layout only (not a scan codec): int4 levels (no 1/127 scale)
    // in the int8 16-code unit layout, for the batched matrix-core scan
    C_Q4M = 16
};

constexpr int SCAN_WG = 256;      // 4 waves
constexpr int SCAN_CAP = 2048;    // LDS candidate keys per workgroup
constexpr int MAX_KPRIME = 1024;  // largest fetch the fused top-k serves
constexpr int MAX_GRID = 1024;    // workgroups per query (bound of the wave-maxima scratch)
constexpr int SCAN_GRID = 512;    // scanning workgroups per query for large row counts

// Wave maxima published per wave when a query's fetch exceeds half the
// number of waves: the threshold helper's bound, the kprime-th best of the
// published keys, needs at least kprime of them (each the key of a distinct
// row), and then forms from the waves' few best rows instead of their one.
constexpr uint32_t SCAN_PUB_MANY = 4;
inline uint32_t scan_pub_m(uint32_t kprime, uint32_t grid) {
    return 2ull * kprime > (uint64_t)grid * (SCAN_WG / 64) ? SCAN_PUB_MANY : 1u;
}

// Per-wave candidate list capacity of the fused scan for a fetch of kp:
// twice kp plus room for one grab, at least 256 keys, a multiple of 64.
inline uint32_t scan_wcap(uint32_t kp) {
    uint32_t c = 2 * kp + 64;
    if (c < 256) c = 256;
    return (c + 63) & ~63u;
}

// Per-query coordination state of the fused scan (zero before first use;
// the kernel leaves it zeroed).  Counters that many workgroups update sit in
// NGROUP groups on separate 128-byte lines: a single hot address would
// serialize every update.
constexpr int NGROUP = 32;  // counter groups
constexpr int CL = 32;      // u32 stride of one counter (128 bytes)
struct QState {
    unsigned long long tau;  // published bound: keys below it cannot be in the top-kprime
    uint32_t pad0[30];       // (every wave polls this line: the counters below live elsewhere)
    uint32_t top;            // scanning workgroups that have finished
    uint32_t fin;            // finishers (final selection + threshold helper)
    uint32_t pad1[30];
    uint32_t cc[NGROUP * CL];    // keys flushed per group region
    uint32_t dyn[NGROUP * CL];   // dynamic tickets taken per slice (may overshoot)
};

struct ScanArgs {
    const void *codes;        // row-major rows, row_bytes each
    uint64_t row_bytes;
    uint32_t units;           // units per row (W)
    uint32_t padded_dim;      // P (Hamming similarity = P - 2*popcount)
    const float *scales;      // per-row scale (quantized codecs) or null
    float scale_mul;          // constant multiplier on the row scale (int4: f32(1/7))
    const void *q;            // transformed queries, q_stride bytes apart (when qraw is null)
    uint64_t q_stride;
    const float *qraw;        // quantized codecs: fp32 queries (nq x qdim) transformed in the kernel
    uint32_t qdim;
    const float *signs;       // rotation signs (rounds x padded_dim) for qraw
    uint32_t rounds;
    const uint32_t *cand;     // indexed mode: row ids (null = rows 0..n-1)
    const uint64_t *cand_off; // per-query offsets into cand (nq+1) or null
    const uint32_t *cand_n;   // or: per-query counts, query q's ids at cand + q * cand_stride
    uint64_t cand_stride;
    const uint32_t *mask;     // row filter bits (LSB-first) or null
    uint64_t mask_bits;
    uint64_t n;               // rows per query when cand_off is null
    uint32_t kprime;          // per-query candidates kept
    uint32_t wcap;            // per-wave LDS list capacity, scan_wcap(kprime)
    uint32_t wstride;         // u64 words of LDS per wave: wcap (+ dim & ~3 re-rank staging)
    uint32_t qf_off;          // C_Q1P: LDS byte offset of the fp32 query (set at launch)
    uint32_t grid;            // scanning workgroups per query (one more runs the threshold helper)
    QState *qs;               // [nq]
    uint64_t *wmax;           // [nq][grid*4*pub_m] per-wave running maxima (zero on entry and exit)
    uint32_t pub_m;           // maxima each wave publishes: 1 (its maximum), or SCAN_PUB_MANY (the
                              // largest lane maxima) when the fetch is large next to the waves
    uint64_t *cand_keys;      // [nq][cand_cap][2] flushed (scan key, exact key) pairs
    uint64_t cand_cap;        // pairs per query: min(grid,NGROUP) regions of ceil(grid/NGROUP)*4*wcap
    uint64_t *merged;         // [nq][kprime] merged keys, descending
    uint32_t *merged_n;       // [nq]
    float *dense_out;         // optional: every row's score (query 0 only)
    const float *rr_src;      // re-rank: stored fp32 rows (N x rr_dim) or null for no re-rank
    uint32_t rr_dim;
    const float *rr_q;        // re-rank: fp32 queries, rr_q_stride floats apart
    uint64_t rr_q_stride;
    uint32_t k_out;           // when out_rows != null: top-k_out (by exact score when re-ranking)
    uint32_t *out_rows;       // [nq][k_out]
    float *out_scores;
    uint32_t *out_n;          // [nq]
    uint32_t short_tail;      // few rows per wave: every pass polls the shared bound, the flush takes
                              // a fresh read of it, and the final gather is bounded by the wave maxima
    uint32_t static_pct;      // share (%) of the row grabs assigned statically (0: the kernel's default)
    uint32_t dsteps;          // wave steps per dynamic ticket (0: the kernel's default)
    uint32_t lean;            // 1: the register-lean build of the int8 transform scan (two queries in flight)
};

// Exact keys of listed rows of a 1-bit asymmetric (C_Q1P) index, one grid
// row per query (q1p_exact_rows).
struct Q1pRowsArgs {
    const void *codes;        // N rows of row_bytes
    uint64_t row_bytes;
    uint32_t units;           // 128-code units per row
    uint32_t P;               // padded dimension
    const float *scales;      // per-row scale
    float scale_mul;
    const float *qrot;        // nq x P rotated fp32 queries
    const uint32_t *rows;     // [nq][cap] row ids
    const uint32_t *kept;     // [nq] listed rows (at most cap used)
    uint64_t cap;
    uint64_t *keys;           // [nq][cap] exact scan keys
    uint64_t nrows;           // rows of the index (listed rows are below it)
};
// Launches q1p_exact_rows in the fused scan's layout for a.units, with gx
// workgroups per query.
hipError_t launch_q1p_exact_rows(const Q1pRowsArgs &a, uint32_t nq, uint32_t gx, hipStream_t s);
// The 1-bit asymmetric form of launch_mq1_tau_exact (a.rows, a.kept, a.cap
// and a.keys unused).  kk <= 4096.
hipError_t launch_q1p_tau_exact(const Q1pRowsArgs &a, const uint64_t *merged, const uint32_t *merged_n, uint32_t kk,
                                uint64_t *tau, uint32_t nq, hipStream_t s);

// Rows per wave below which a scan takes the short tail (a wave then scans
// too few steps for the threshold helper's bound to reach it through the
// usual polling, so a flush by the wave's own bound would carry, and
// exactly re-score, most of its rows).
constexpr uint64_t SHORT_TAIL_ROWS = 256;
// The static / dynamic split of a long scan and of a short one (a short
// scan's dynamic share is handed out in finer chunks: a wave scans only a
// few steps in all).
constexpr uint32_t LONG_STATIC_PCT = 70, LONG_DSTEPS = 6;
constexpr uint32_t SHORT_STATIC_PCT = 80, SHORT_DSTEPS = 1;

struct EncodeArgs {
    const float *src;         // rows x dim
    uint64_t rows;
    uint32_t dim;
    uint32_t P;               // padToPow2(dim)
    const float *signs;       // rounds x P
    uint32_t rounds;
    uint32_t bits;            // 8, 4, 1 (codes out) or 0 (no codes)
    uint32_t *codes;          // rows x (P/per)
    float *scales;            // rows
    float *rotated;           // optional rows x P
    const int32_t *sample_slot; // optional per row: IVF reservoir slot or -1
    float *sample;            // IVF reservoir (slots x P) when sample_slot is set
    uint32_t *slow_rows;      // counter of rows that took the sequential 1-bit sum
};

struct RerankArgs {
    const float *rows;        // stored fp32 rows (original space), N x dim
    uint32_t dim;
    const float *q;           // queries (original space), q_stride floats apart
    uint64_t q_stride;
    const uint64_t *merged;   // [nq][kprime] candidate keys (row in low bits)
    const uint32_t *merged_n; // [nq]
    const uint32_t *cand_rows;// alternative: explicit candidate rows [nq][kprime]
    const uint32_t *cand_n;   // [nq] counts for cand_rows
    uint32_t kprime;
    uint32_t k_out;
    uint64_t *rr_keys;        // scratch [nq][kprime]: re-ranked (score, row) keys
    uint32_t *tickets;        // [nq]
    uint32_t *out_rows;       // [nq][k_out]
    float *out_scores;
    uint32_t *out_n;
};

struct LevelArgs {
    const float *qrot;        // nq x P rotated queries
    uint32_t P;
    int codec;                // C_Q8 or C_Q4
    unsigned char *out;       // nq x stride bytes: packed levels + QLevelTail
    uint64_t stride;
};

// ---- IVF ------------------------------------------------------------------
constexpr uint32_t IVF_MAX_NLIST = 4096;   // lists (the reference's automatic cap)
constexpr uint32_t IVF_MAX_NPROBE = IVF_MAX_NLIST;

struct IvfCopyArgs {
    const float *src;
    uint64_t src_stride;
    const uint32_t *src_idx;  // [n] source rows
    float *dst;
    uint64_t dst_stride;
    const uint32_t *dst_idx;  // [n] destination rows, or null for 0..n-1
    uint32_t n, dim;
};

struct IvfAssignArgs {
    uint64_t n;               // rows to assign
    uint32_t dim;             // product length (padded dim for codes)
    const float *rows;        // fp32 rows (bits 0)
    uint64_t row_stride;
    const uint32_t *codes;    // codes (bits 8/4/1)
    uint32_t words_per_row;
    const float *scales;
    const float *centroids;   // nlist x cen_stride
    uint32_t cen_stride;
    uint32_t nlist;
    uint32_t *out;            // [n] nearest centroid
    uint64_t *keys;           // [n] scratch of the split form (row tiles x centroid tiles), or null
};
// Row tiles below which the assignment splits the centroids over workgroups
// too (a workgroup per row tile and centroid tile, joined by a per-row
// atomic maximum) so that the grid fills the device.
constexpr uint64_t IVF_ASSIGN_SPLIT_TILES = 1024;
inline bool ivf_assign_split(uint64_t n) { return (n + 127) / 128 < IVF_ASSIGN_SPLIT_TILES; }

struct IvfProbeArgs {
    const float *centroids;   // nlist x P
    uint32_t nlist, P;
    const float *qrot;        // nq x P queries in the centroids' space
    float *scores;            // nq x nlist scratch
    uint32_t nprobe;
    uint32_t *probes;         // nq x nprobe, best first
    const uint32_t *offset;   // list offsets (nlist + 1), or null: no totals
    uint64_t *totals;         // nq: the probed lists' total size per query
    uint64_t *cand_off;       // nq + 1 candidate offsets, written here when nq == 1
};

hipError_t ivf_launch_copy_rows(const IvfCopyArgs &a, hipStream_t s);
hipError_t ivf_launch_normalize(float *m, uint32_t rows, uint32_t dim, uint32_t stride, hipStream_t s);
hipError_t ivf_launch_assign(const IvfAssignArgs &a, int bits, hipStream_t s);

// The assignment of int8 codes on the matrix cores: a pass that decides
// every row whose nearest centroid is clear by a proven margin and queues
// the others, then the exact arithmetic of ivf_assign for the queued rows.
// Scratch: the centroids' two int8 levels (nlist rounded up to 32, x 2 x P
// bytes) and scales (x 2 floats), a bound word and a queue count (two
// words), and the queue (qcap entries).
struct IvfRecheck {
    uint32_t row;
    uint32_t n;               // candidates in c, or IVF_RECHECK_ALL: every centroid
    uint32_t c[6];
};
constexpr uint32_t IVF_RECHECK_ALL = 0xffffffffu;
struct IvfMfmaScratch {
    int8_t *lev;
    float *ls;
    uint32_t *words;          // [0] bound (f32 bits), [1] queue count
    IvfRecheck *queue;
    uint32_t qcap;
};
inline bool ivf_assign_mfma_ok(int bits, uint32_t P, uint32_t nlist) {
    return bits == 8 && (P == 128 || P == 256 || P == 512 || P == 1024) && nlist >= 1 && nlist <= IVF_MAX_NLIST;
}
inline uint32_t ivf_mfma_nlist_pad(uint32_t nlist) { return (nlist + 31) & ~31u; }
inline uint32_t ivf_mfma_qcap(uint64_t n) { return (uint32_t)std::max<uint64_t>(65536, std::min<uint64_t>(n, (n + 3) / 4)); }
// levels, then the pass (out[r] for the decided rows, the queue for the rest)
hipError_t ivf_launch_assign_mfma(const IvfAssignArgs &a, const IvfMfmaScratch &m, hipStream_t s);
// the exact assignment of the first `entries` queued rows
hipError_t ivf_launch_assign_recheck(const IvfAssignArgs &a, const IvfMfmaScratch &m, uint32_t entries,
                                     hipStream_t s);
uint32_t ivf_list_blocks(uint64_t n);
// hist/base: ivf_list_blocks(n) x nlist; totals: nlist; offset: nlist+1; rows_out: n.
hipError_t ivf_launch_lists(const uint32_t *assign, uint64_t n, uint32_t nlist, uint32_t *hist, uint32_t *base,
                            uint32_t *totals, uint32_t *offset, uint32_t *rows_out, hipStream_t s);
// Lists extended by an append: for each list, its rows (old_off / old_rows),
// then the appended ones (add_off / add_rows, ids relative to add_base).
hipError_t ivf_launch_merge_lists(const uint32_t *old_off, const uint32_t *old_rows, const uint32_t *add_off,
                                  const uint32_t *add_rows, uint32_t add_base, uint32_t nlist, uint32_t *new_off,
                                  uint32_t *new_rows, hipStream_t s);
hipError_t ivf_launch_means(const float *sample, uint32_t stride, uint32_t dim, const uint32_t *offset,
                            const uint32_t *list_rows, uint32_t nlist, float *centroids, uint32_t cen_stride,
                            hipStream_t s);
hipError_t ivf_launch_probes(const IvfProbeArgs &a, uint32_t nq, hipStream_t s);
// totals: nq, as the probe launch wrote them; cand_off: nq+1 (the probe
// launch wrote it when nq == 1); cand: capacity for every query's candidates.
hipError_t ivf_launch_gather(const uint32_t *probes, uint32_t nq, uint32_t nprobe, const uint32_t *offset,
                             const uint32_t *list_rows, uint64_t *totals, uint64_t *cand_off, uint32_t *cand,
                             hipStream_t s);

// Chooses the lane layout for a codec and row size; false if unsupported.
// Batched int8 scan on the matrix cores (bv_mq.hip).  One pass scores the
// logical rows i < n (physical row i * row_step) against every query with
// v_mfma_i32_32x32x32_i8 over the three int8 query levels, and either writes
// every key densely (cand[q * cap + i]) or appends the keys at or above
// tau[q] (counted in cnt[q]; keys past cap are dropped but still counted).
constexpr int MQ_WAVES = 8;       // waves per workgroup (64 rows each)
constexpr int MQ_ROWS = 512;      // rows per workgroup tile
constexpr int MQ_QB = 32;         // queries per workgroup
constexpr uint32_t MQ_MAX_STEPS = 32;  // 32-code steps per row (P <= 1024): levels resident in LDS
constexpr uint32_t MQ_SAMPLE = 16384;  // rows of the threshold sample
struct MqArgs {
    const uint32_t *codes;    // N x W words
    const float *scales;      // N
    uint32_t W;               // words per row
    uint32_t units;           // 16-code units per row (even), P / 16
    uint64_t n;               // logical rows in this pass
    uint64_t row_step;        // physical row of logical row i = i * row_step
    int bits;                 // 8: int8 codes; 4: int4 codes (nibble n carried as n ^ 8)
    float scale_mul;          // row scale multiplier (int4: f32(1/7))
    const unsigned char *qlev;// nq x qstride bytes: packed levels (16-code units) + QLevelTail
    uint64_t qstride;
    uint32_t tail_off;        // byte offset of QLevelTail in a query's layout
    uint32_t nq;
    uint32_t qblocks;         // ceil(nq / MQ_QB)
    uint32_t groups;          // workgroups per (XCD, query block); tile stride = 8 * groups
    const uint64_t *tau;      // [nq] append threshold (null: dense pass)
    uint64_t *cand;           // [nq][cap]
    uint32_t *cnt;            // [nq] appended keys (threshold pass)
    uint64_t cap;
    // fp32 rows only.  l2: score 2 x.q - |x|^2 - |q|^2 (rsq per row, qsq per
    // query) instead of x.q.  rows_out: the threshold pass appends the ids of
    // rows whose score reaches tau's score minus slack[q] ([nq][cap] u32)
    // instead of keys: a superset of the rows that can rank in the exact scan.
    int l2;
    const float *rsq;
    const float *qsq;
    const float *slack;
    uint32_t *rows_out;
};
// Per-row squared norms of fp32 rows (f64 sums rounded to f32) and, in
// *max_bits, the largest of them (float bits, rounded up; rsq >= 0 so the
// bits order like the values).
hipError_t launch_row_sqnorms(const float *rows, uint64_t n, uint32_t dim, float *rsq, uint32_t *max_bits,
                              hipStream_t s);
// Per-query constants of the exact fp32 batch: qsq = |q|^2 and the slack
// 2E, where E bounds |matrix-core score - single-query score| for every row:
// dot 3(dim+2)u |x|max |q|, l2 4(dim+4)u (|x|max + |q|)^2 (u = 2^-24).
hipError_t launch_mq_f32_qconst(const float *q, uint32_t nq, uint32_t dim, const uint32_t *max_bits, int l2,
                                float *qsq, float *slack, hipStream_t s);
// Per query: the best kk keys of cand[q][0, min(cnt[q], cap)).  Outputs are
// optional: tau = the kk-th best key (0 when there are kk or fewer), the
// selected keys (merged, merged_n), overflow = cnt[q] > cap, and the selected
// keys ranked into (rows, scores, n) for k_out results.
struct MqSelArgs {
    const uint64_t *cand;
    const uint32_t *cnt;
    uint64_t cap;
    uint32_t kk;
    uint64_t *tau;
    uint64_t *merged;         // [nq][kk]
    uint32_t *merged_n;
    uint32_t *overflow;
    bool tau_max;             // tau[q] = max(tau[q], the kk-th best key)
    uint32_t k_out;
    uint32_t *out_rows;       // [nq][k_out]
    float *out_scores;
    uint32_t *out_n;
};
// Exact re-rank of merged[q][0, merged_n[q]) against the stored fp32 rows,
// then the top k_out (one workgroup per query).
struct MqRerankArgs {
    const float *rows;        // N x dim
    uint32_t dim;
    const float *q;           // queries, q_stride floats apart
    uint64_t q_stride;
    const uint64_t *merged;   // [nq][kprime] scan keys
    const uint32_t *merged_n;
    uint32_t kprime;
    uint32_t k_out;
    uint32_t *out_rows;       // [nq][k_out]
    float *out_scores;
    uint32_t *out_n;
};
// Level-one prefilter of int8 batches (mq1_scan): MQ1_QB queries per
// workgroup (32 per wave, in registers) scored on their first int8 level
// alone against MQ1_ROWS-row tiles staged in LDS, with per-(row, query)
// bounds from the row's code norm and the query's remaining levels.
constexpr int MQ1_QB = 256;
constexpr int MQ1_ROWS = 32;
struct Mq1Args {
    const uint32_t *codes;    // N x W words of int8 codes
    const float *scales;      // N
    const float *cn;          // N: |c|_2 of each row's codes, rounded up
    uint32_t W;               // words per row
    uint32_t units;           // 16-code units per row (even), P / 16
    uint64_t n;               // logical rows in this pass
    uint64_t row_step;        // logical row i reads row i * row_step of codes / scales / cn ...
    uint64_t row_base;        // ... and is row row_base + i * row_step in the keys
    const unsigned char *qlev;// nq x qstride bytes: packed levels (16-code units) + QLevelTail
    uint64_t qstride;
    uint32_t tail_off;
    const float *rq;          // [nq] bound of the query's levels two and three (launch_mq1_qconst)
    uint32_t nq;
    uint32_t qblocks;         // ceil(nq / MQ1_QB)
    uint32_t groups;          // workgroups per query block (about one per CU in all)
    uint32_t nwg;             // = groups (bucket count per query)
    const uint64_t *tau;      // null: dense pass (lower-bound keys into cand); else [nq] bound keys
    uint64_t *cand;           // dense: [nq][cap] lower-bound keys of logical rows;
                              // threshold: [nq][nwg][capw] lower-bound keys of kept rows, per workgroup bucket
    uint32_t *up_out;         // threshold: [nq][nwg][capw] order bits of the kept rows' upper bounds
    uint32_t *cnt;            // threshold: [nq][nwg] bucket lengths (0xffffffff: overflowed)
    uint64_t cap;
    uint32_t capw;            // threshold: entries per bucket
    float cn_const;           // mq1_scan_bits: every row's code norm (cn unused)
};
// mq1_scan over 1-bit codes (codes: W = units / 2 words of 32 bits per
// row) widened to +1 / -1 bytes in LDS; scales may be null (1); every row's
// code norm is cn_const.  16-code units per row: 8 to 64.
hipError_t launch_mq1_scan_bits(const Mq1Args &a, hipStream_t s);
// Hamming exact keys of rows[q][0, min(kept[q], cap)) over 1-bit codes (W
// words per row, 4 to 32) and the queries' bits (W words each), into
// keys[q][...]: the keys mq1_exact gives over the widened codes.
hipError_t launch_ham_exact(const uint32_t *codes, uint32_t W, const uint32_t *qbits, const unsigned char *qlev,
                            uint64_t qstride, uint32_t tail_off, const uint32_t *rows, const uint32_t *kept,
                            uint64_t cap, uint64_t *keys, uint32_t nq, hipStream_t s);
// Per query: its buckets joined into lk / uo [nq][cap] (after the list's
// cnt[q] entries when append is set) and the length in cnt[q] (0xffffffff
// when a bucket overflowed or the total exceeds cap).
hipError_t launch_mq1_compact(const uint64_t *bk, const uint32_t *bu, const uint32_t *bc, uint32_t nwg,
                              uint32_t capw, uint64_t cap, uint64_t *lk, uint32_t *uo, uint32_t *cnt, bool append,
                              uint32_t nq, hipStream_t s);
// Per query: the rows among cand[q][0, min(cnt[q], cap)) whose upper bound
// (make_key(up[q][i], row)) reaches tau[q], into rows[q][...], their number
// in kept[q].
hipError_t launch_mq1_keep(const uint64_t *cand, const uint32_t *up, const uint32_t *cnt, uint64_t cap,
                           const uint64_t *tau, uint32_t *rows, uint32_t *kept, uint32_t nq, hipStream_t s);
// Per query: the exact key (the single-query scan's three-level f64
// combine) of each of rows[q][0, kept[q]) into keys[q][...].
hipError_t launch_mq1_exact(const uint32_t *codes, uint32_t W, const float *scales, const unsigned char *qlev,
                            uint64_t qstride, uint32_t units16, const uint32_t *rows, const uint32_t *kept,
                            uint64_t cap, uint64_t *keys, uint32_t nq, hipStream_t s);
// Per query: tau[q] = max(tau[q], the smallest exact key of the rows of
// merged[q][0, kk), a list's kk best lower-bound keys (mq_select's sorted
// output); nothing when merged_n[q] < kk or a row is not below nrows.
hipError_t launch_mq1_tau_exact(const uint32_t *codes, uint32_t W, const float *scales,
                                const unsigned char *qlev, uint64_t qstride, uint32_t units16,
                                const uint64_t *merged, const uint32_t *merged_n, uint32_t kk, uint64_t nrows,
                                uint64_t *tau, uint32_t nq, hipStream_t s);
hipError_t launch_row_code_norms(const uint32_t *codes, uint64_t n, uint32_t W, float *cn, hipStream_t s);
hipError_t launch_mq1_qconst(const unsigned char *qlev, uint64_t qstride, uint32_t units, uint32_t tail_off,
                             uint32_t nq, float *rq, uint32_t *cnt, uint32_t cnt_value, hipStream_t s);
// The 1-bit asymmetric batch's query term (row term 1): |x - s1 q1|_1 plus
// the f32 summation slack, rounded up; x the rotated queries (nq x P).
hipError_t launch_mq1_qconst_l1(const float *qrot, uint32_t P, const unsigned char *qlev, uint64_t qstride,
                                uint32_t tail_off, uint32_t nq, float *rq, uint32_t *cnt, uint32_t cnt_value,
                                hipStream_t s);
hipError_t launch_mq1_scan(const Mq1Args &a, hipStream_t s);
hipError_t launch_mq_scan(const MqArgs &a, hipStream_t s);
// fp32 rows (dot / cosine): a.codes = the rows, a.W = dim, a.units = dim / 8,
// a.qlev = fp32 queries (a.qstride bytes apart).  Dimensions 32 .. 1024 in
// the set mq_f32_supported accepts (32 queries of up to 1024 floats stay in LDS).
bool mq_f32_supported(uint32_t dim);
hipError_t launch_mq_scan_f32(const MqArgs &a, hipStream_t s);
hipError_t launch_mq_rerank(const MqRerankArgs &a, uint32_t nq, hipStream_t s);
hipError_t launch_mq_select(const MqSelArgs &a, uint32_t nq, hipStream_t s);

// Zeroes `bytes` (a multiple of 4) at p with a plain kernel (no memset node,
// so the launch is safe to record in a captured graph).
hipError_t launch_zero(void *p, size_t bytes, hipStream_t s);

bool scan_supported(int codec, uint32_t units);
hipError_t launch_scan(int codec, uint32_t units, const ScanArgs &a, uint32_t nq, hipStream_t s);
hipError_t launch_encode(const EncodeArgs &a, hipStream_t s);
hipError_t launch_rerank(const RerankArgs &a, uint32_t nq, hipStream_t s);
hipError_t launch_levels(const LevelArgs &a, uint32_t nq, hipStream_t s);
// C_Q1P query layout (bit planes + Q1Tail + fp32 query) from rotated queries.
hipError_t launch_q1p_layout(const LevelArgs &a, uint32_t nq, hipStream_t s);
size_t level_stride(int codec, uint32_t P);
size_t scan_query_lds(int codec, uint32_t P);
// The fused scan's LDS per workgroup (at most: with the in-kernel query
// transform) for per-wave list stride wstride.
size_t scan_lds_bytes(int codec, uint32_t P, uint32_t wstride);
// True when the scan for this codec / row layout transforms fp32 queries itself (ScanArgs::qraw).
bool scan_prep_supported(int codec, uint32_t units, uint32_t P);

// ---- list-major IVF int8 batches (bv_mq.hip) ---------------------------------
// base[q][j]: where probe j's rows start among query q's candidates; cnt[q]:
// its candidate count; pair_count[c] += queries probing list c (zeroed first).
hipError_t launch_ivf_pairs(const uint32_t *probes, uint32_t nq, uint32_t nprobe, const uint32_t *list_off,
                            uint32_t *base, uint32_t *cnt, uint32_t *pair_count, hipStream_t s);
// The (query, base) pairs grouped by list (pair_off: exclusive scan of
// pair_count; fill zeroed first).
hipError_t launch_ivf_pair_scatter(const uint32_t *probes, const uint32_t *base, uint32_t npairs, uint32_t nprobe,
                                   const uint32_t *pair_off, uint32_t *fill, uint32_t *pair_q, uint32_t *pair_base,
                                   hipStream_t s);
// chunks[c]: list c's work items (8 of its queries each).
hipError_t launch_ivf_chunk_counts(const uint32_t *pair_count, uint32_t nlist, uint32_t *chunks, hipStream_t s);
// Every probed list's rows scored once per work item (chunk_off: exclusive
// scan of chunks): the single-query scan's key at cand[q * cap + base + i].
// bits 8 (int8 codes) or 4 (int4 codes and the int4 level layout; keys as
// the batched int4 scan forms them); scales times scale_mul (1/7 for int4).
hipError_t launch_ivf_list_scan(const uint32_t *codes, uint32_t W, uint32_t bits, const float *scales,
                                float scale_mul, const uint32_t *list_off, const uint32_t *list_rows, uint32_t nlist,
                                const uint32_t *chunk_off, uint32_t npairs, const uint32_t *pair_off,
                                const uint32_t *pair_count, const uint32_t *pair_q, const uint32_t *pair_base,
                                const unsigned char *qlev, uint64_t qstride, uint32_t units16, uint64_t *cand,
                                uint64_t cap, hipStream_t s);

// ---- Hamming batches on the int8 first-level path (bv_mq.hip) ---------------
// 1-bit codes (words 32-bit words) as +1 / -1 int8 codes (8 words out per word in).
hipError_t launch_expand_pm(const uint32_t *bits, uint64_t words, uint32_t *out, hipStream_t s);
// int4 codes (words of 8 nibbles) as signed bytes, one per code; and
// dst[i] = f32(src[i] * mul).
hipError_t launch_expand_q4(const uint32_t *nib, uint64_t words, uint32_t *out, hipStream_t s);
hipError_t launch_scale_mul(const float *src, uint64_t n, float mul, float *dst, hipStream_t s);
// Queries' 1-bit codes (P / 32 words each) as packed levels: level one +1 / -1,
// the other levels zero, tail scales (1, 0, 0).
hipError_t launch_pm_levels(const uint32_t *qbits, uint32_t nq, uint32_t P, unsigned char *qlev, uint64_t stride,
                            hipStream_t s);
hipError_t launch_fill_f32(float *p, uint64_t n, float v, hipStream_t s);

// ---- graph beam search (bv_graph.hip) ---------------------------------------
constexpr uint32_t GRAPH_EF_CAP = 256;  // beam slots (src/engine/wgsl/graphSearch.ts:32)
struct GraphArgs {
    const float *corpus;      // corpus_rows x dim, prepared rows
    uint32_t dim;
    uint64_t corpus_rows;
    const uint32_t *graph;    // graph_rows x K, 0xffffffff = empty slot
    uint32_t K;
    uint64_t graph_rows;
    const float *queries;     // nq x dim
    const uint32_t *entries;  // seed rows
    uint32_t n_entries;
    uint32_t efA;             // beam width <= GRAPH_EF_CAP
    uint32_t iter_cap;        // expansions at most
    uint32_t k;               // hits per query <= GRAPH_EF_CAP
    uint32_t out_stride;      // out_rows / out_scores entries per query (>= k)
    float *beam_dist;         // optional: [nq][GRAPH_EF_CAP] raw beam
    uint32_t *beam_id;
    uint32_t *out_rows;       // optional: [nq][k] deduped, sorted hits
    float *out_scores;
    uint32_t *out_n;          // [nq]
};
hipError_t launch_graph_beam(const GraphArgs &a, uint32_t nq, bool l2, hipStream_t s);

// ---- selection for any k; exact scan of listed rows (bv_select.hip) ---------
// Keys (make_key) of scores[0, n); rows whose mask bit is clear get key 0.
hipError_t sel_dense_keys(const float *scores, uint64_t n, const uint32_t *mask, uint64_t *keys, hipStream_t s);
// Keys of scores[i] for row list[i], i < n.
hipError_t sel_list_keys(const float *scores, const uint32_t *list, uint64_t n, uint64_t *keys, hipStream_t s);
// popc[w] = set bits of mask word w below row n.
hipError_t sel_mask_counts(const uint32_t *mask, uint64_t words, uint64_t n, uint32_t *popc, hipStream_t s);
// hipCUB exclusive sum (tmp == nullptr: only sizes tmp_bytes).
hipError_t sel_exclusive_scan(void *tmp, size_t &tmp_bytes, const uint32_t *in, uint32_t *out, uint64_t n,
                              hipStream_t s);
// The rows whose mask bit is set, ascending, at list[off[w] ...]; *list_n = their number.
hipError_t sel_mask_rows(const uint32_t *mask, uint64_t words, uint64_t n, const uint32_t *popc, const uint32_t *off,
                         uint32_t *list, uint32_t *list_n, hipStream_t s);
// Key of each listed row's exact score (Store.dotRow, or Store.l2Row when l2)
// against q; a listed row >= n sets *bad and gets key 0.
hipError_t sel_exact_row_keys(const float *raw, uint64_t n, uint32_t dim, bool l2, const float *q,
                              const uint32_t *list, uint64_t n_list, uint64_t *keys, uint32_t *bad, hipStream_t s);
// hipCUB descending radix sort of n keys (tmp == nullptr: only sizes tmp_bytes).
hipError_t sel_sort_desc(void *tmp, size_t &tmp_bytes, const uint64_t *in, uint64_t *out, uint64_t n, hipStream_t s);
// (row, score) of the first k sorted keys; *n_out = how many are not empty.
hipError_t sel_keys_to_hits(const uint64_t *sorted, uint32_t k, uint32_t *rows, float *scores, uint32_t *n_out,
                            hipStream_t s);

} // namespace bvk
