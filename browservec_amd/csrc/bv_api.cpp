// Host runtime behind include/browservec_hip.h: device handles, index objects
// holding their rows/codes in HBM, and the query pipelines that chain the
// gfx950 kernels on one HIP stream per index.
#include "../../include/browservec_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <functional>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstddef>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <thread>
#include <string>
#include <vector>

#include "bv_kernels.h"

using namespace bvk;

// ------------------------------------------------------------------ errors
static thread_local std::string g_err;

static int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

struct bv_device {
    int ordinal = 0;
    hipDeviceProp_t prop{};
    bool lost = false;
    bool inject_append_oom = false;  // bv_debug_inject: fail the next append's allocation
    bool inject_append_late = false; // bv_debug_inject: fail the next append after its rows are encoded
    void *scratch = nullptr;         // this GPU's copy of the no-allocation scratch array
};

// ------------------------------------------------- no-allocation scratch --
// The fused scan's scratch for bv_index_search_device_noalloc lives in a
// file-scope device array of BV_NOALLOC_SCRATCH_BYTES; every GPU the library
// runs on holds its own copy until the process ends.  In host code `scratch`
// names a host-side stand-in, never device memory: its device address comes
// from hipGetSymbolAddress, resolved once per device with that device
// current (bv_device_open) and used everywhere host code needs the array.
static __device__ __align__(256) unsigned char scratch[BV_NOALLOC_SCRATCH_BYTES];
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[256];  // per device ordinal; null until resolved

static void *resolve_scratch(int ordinal) {
    if (ordinal < 0 || ordinal >= 256) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[ordinal]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) == hipSuccess) g_scratch_ptr[ordinal] = ptr;
    }
    return g_scratch_ptr[ordinal];
}

static int hip_fail(bv_device *dev, hipError_t e, const char *what) {
    if (e == hipErrorOutOfMemory) return fail(BV_E_OOM, "%s: out of device memory", what);
    if (dev && (e == hipErrorIllegalAddress || e == hipErrorLaunchFailure || e == hipErrorECCNotCorrectable ||
                e == hipErrorNoDevice))
        dev->lost = true;
    return fail(BV_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIPX(dev, expr, what)                        \
    do {                                             \
        hipError_t _e = (expr);                      \
        if (_e != hipSuccess) return hip_fail((dev), _e, (what)); \
    } while (0)

// -------------------------------------------------------- device buffers
struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
    ~DevBuf() { release(); }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
    }
    // Grow to at least `bytes`, preserving the first `keep` bytes.
    hipError_t ensure(size_t bytes, size_t keep, hipStream_t s, bool geometric = true) {
        if (bytes <= cap) return hipSuccess;
        size_t ncap = geometric ? std::max(bytes, cap + cap / 2) : bytes;
        ncap = (ncap + 255) & ~size_t(255);
        void *np = nullptr;
        hipError_t e = hipMalloc(&np, ncap);
        if (e != hipSuccess) return e;
        if (p && keep) {
            e = hipMemcpyAsync(np, p, keep, hipMemcpyDeviceToDevice, s);
            if (e == hipSuccess) e = hipStreamSynchronize(s);
            if (e != hipSuccess) {
                (void)hipFree(np);
                return e;
            }
        }
        if (p) (void)hipFree(p);
        p = np;
        cap = ncap;
        return hipSuccess;
    }
    template <class T> T *as() const { return (T *)p; }
};

struct HostBuf {
    void *p = nullptr;
    size_t cap = 0;
    ~HostBuf() {
        if (p) (void)hipHostFree(p);
    }
    hipError_t ensure(size_t bytes) {
        if (bytes <= cap) return hipSuccess;
        if (p) (void)hipHostFree(p);
        p = nullptr;
        size_t ncap = std::max(bytes, cap * 2);
        hipError_t e = hipHostMalloc(&p, ncap, hipHostMallocDefault);
        if (e != hipSuccess) {
            cap = 0;
            return e;
        }
        cap = ncap;
        return hipSuccess;
    }
};

// ------------------------------------------------------------------ index
// query streams a caller may keep single queries in flight on
// (bv_index_set_query_streams)
constexpr int MAX_QUERY_STREAMS = 4;

struct bv_index {
    // Calls on one index are serialized (the Node binding runs them on worker
    // threads); the reference awaits them one at a time per store.
    mutable std::recursive_mutex mu;
    bv_device *dev = nullptr;
    bv_index_desc d{};
    uint32_t dim = 0, P = 0, words_per_row = 0, row_bytes = 0, units = 0;
    int codec = -1;
    bool quant = false;
    uint64_t rows = 0;
    hipStream_t stream = nullptr;

    DevBuf raw;      // N x dim fp32 rows (flat corpus; quantized kinds: re-rank source)
    DevBuf codes;    // N x row_bytes
    DevBuf scales;   // N floats
    DevBuf signs;    // rounds x P (+64 slack)
    DevBuf slow;     // 1-bit sequential-sum counter

    // per-call scratch
    DevBuf qin, qrot, qscan, qscale, mask;
    DevBuf qstate, wmax, cand_keys, merged, merged_n;
    DevBuf rr_keys, rr_tickets;
    DevBuf out_rows, out_scores, out_n;
    DevBuf cand, cand_n, dense;
    DevBuf mq_cand, mq_cnt, mq_tau, mq_tau2, mq_flag;  // batched matrix-core scans
    DevBuf rsq, rsq_max;                      // flat fp32: squared row norms and their maximum (float bits)
    DevBuf mq_qsq, mq_slack, mq_rows;         // exact fp32 batches: query norms, slack, surviving rows
    DevBuf cnorm, mq_rq, mq_up, mq_kept;       // flat int8 level-one batches: row code norms, query bounds, upper bounds, kept counts
    DevBuf mq_bk, mq_bu, mq_bc;               // level-one batches: per-workgroup buckets (lower keys, upper bounds, lengths)
    DevBuf sel_keys, sel_sorted, sel_tmp;     // selection by sort: keys, sorted keys, hipCUB scratch
    DevBuf pm_codes, pm_ones, pm_cn, pm_qbits; // Hamming batches: +1/-1 int8 rows, unit scales, norms, query bits
    uint64_t pm_rows = 0;                      // rows expanded into pm_codes
    DevBuf ivb_base, ivb_pcount, ivb_poff, ivb_fill, ivb_pq, ivb_pbase, ivb_tmp;  // list-major IVF batches
    DevBuf ivb_chunks, ivb_choff;             // list-major IVF batches: work items per list, their offsets
    DevBuf sel_list, sel_popc, sel_off, sel_misc;  // listed rows; mask word counts and offsets; flag + count
    HostBuf h_cnt;
    HostBuf h_rows, h_scores, h_n, h_flag;
    // host appends: rows staged through two pinned buffers on a copy stream
    hipStream_t copy_stream = nullptr;
    hipEvent_t up_ev[2] = {nullptr, nullptr};
    HostBuf up_ring[2];

    uint32_t nprobe_override = 0;

    // IVF (IVFIndex / IVFQuantIndex): reservoir sample, centroids, CSR lists
    bool ivf = false;
    uint32_t sample_cap = 0, sample_dim = 0;  // sample rows: padded dim (quant) or dim (fp32)
    uint64_t sample_filled = 0, sample_seen = 0;
    uint32_t sample_rng = 0;
    DevBuf sample;
    std::vector<uint64_t> sample_row;         // corpus row held by each reservoir slot
    uint32_t tuned_nprobe = 0;                // targetRecall tuning (0 = not tuned)
    float tuned_recall = -1.0f;
    // the tuner's own queries and outputs: a build may run inside a query
    // call, so it must not touch that call's scratch or output buffers
    DevBuf tune_q, tune_rot, tune_rows, tune_scores, tune_n;
    DevBuf ivf_qrot;                          // probe-space queries of an IVF query
    uint64_t built_rows = ~0ull;              // rows covered by the current lists
    bool retrain_due = false;                 // incremental appends since the last full build
    uint32_t nlist = 0;
    DevBuf centroids, list_off, list_rows;
    DevBuf list_off2, list_rows2;             // incremental appends: the extended lists, swapped in
    std::vector<uint32_t> list_sizes_desc;    // host: list sizes, largest first
    DevBuf ivf_idx, ivf_idx2, ivf_slot, ivf_assign, ivf_hist, ivf_base, ivf_totals, ivf_toff, ivf_trows;
    DevBuf ivf_pend;  // an append's sampled rows (rotated), scattered into `sample` once nothing can fail
    DevBuf ivf_keys;  // the split assignment's per-row keys
    DevBuf ivf_lev, ivf_ls, ivf_mwords, ivf_queue;  // the matrix-core assignment's scratch
    uint64_t ivf_exact_rows = 0;              // rows the last assignment gave the exact arithmetic alone
    uint64_t build_exact_rows = 0;            // the same, for the last build's final assignment
    DevBuf probe_scores, probes, cand_tot, cand_off;
    double build_ms = 0;
    double last_query_ms = 0, last_query_gpu_ms = 0;
    uint64_t last_scanned = 0;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    // further query streams (bv_index_set_query_streams): consecutive fused
    // queries take the index stream and these in turn, each with its own
    // scan scratch, so one query's tail overlaps the next one's scan
    struct ScanLane {
        hipStream_t stream = nullptr;
        DevBuf qstate, wmax, cand_keys, merged, merged_n;
        DevBuf ivf_qrot, probe_scores, probes, cand, cand_tot, cand_off;  // an IVF query's probes and candidates
        uint64_t mut_seen = 0;                // the ev_mut record this stream last waited on
    } lanes[MAX_QUERY_STREAMS - 1];
    uint32_t query_streams = 1, next_lane = 0;
    uint32_t lanes_pending = 0;               // bit i: lanes[i] has queries the index stream has not joined
    hipEvent_t ev_mut = nullptr;              // recorded after work that changes the index's buffers
    uint64_t mut_gen = 0;                     // counts the ev_mut records

    // kernel timing
    bool timing = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> tev;
    size_t tev_used = 0;
    double scan_ms = 0;
    uint64_t scan_launches = 0;
};

extern "C" const char *bv_last_error(void) { return g_err.c_str(); }
extern "C" int bv_abi_version(void) { return BV_ABI_VERSION; }

// ------------------------------------------------------------------ device
extern "C" int bv_device_open(int ordinal, bv_device **out) {
    if (!out) return fail(BV_E_INVALID, "out is null");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return fail(BV_E_UNSUPPORTED, "no HIP device available");
    if (ordinal < 0 || ordinal >= n) return fail(BV_E_INVALID, "device ordinal %d out of range (%d devices)", ordinal, n);
    bv_device *d = new bv_device();
    d->ordinal = ordinal;
    e = hipSetDevice(ordinal);
    if (e == hipSuccess) e = hipGetDeviceProperties(&d->prop, ordinal);
    if (e != hipSuccess) {
        delete d;
        return fail(BV_E_HIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    }
    d->scratch = resolve_scratch(ordinal);  // with this device current
    *out = d;
    return BV_OK;
}

extern "C" int bv_device_close(bv_device *dev) {
    delete dev;
    return BV_OK;
}

extern "C" int bv_device_is_lost(const bv_device *dev, int *lost) {
    if (!dev || !lost) return fail(BV_E_INVALID, "null argument");
    *lost = dev->lost ? 1 : 0;
    return BV_OK;
}

extern "C" int bv_debug_inject(bv_device *dev, int what) {
    if (!dev) return fail(BV_E_INVALID, "null device");
    switch (what) {
    case BV_INJECT_LOST: dev->lost = true; return BV_OK;
    case BV_INJECT_APPEND_OOM: dev->inject_append_oom = true; return BV_OK;
    case BV_INJECT_APPEND_LATE: dev->inject_append_late = true; return BV_OK;
    default: return fail(BV_E_INVALID, "unknown injection %d", what);
    }
}

extern "C" int bv_device_info(const bv_device *dev, char *name, uint32_t name_len, uint32_t *cu_count,
                              uint64_t *hbm_bytes) {
    if (!dev) return fail(BV_E_INVALID, "null device");
    if (name && name_len) {
        snprintf(name, name_len, "%s (%s)", dev->prop.name, dev->prop.gcnArchName);
    }
    if (cu_count) *cu_count = (uint32_t)dev->prop.multiProcessorCount;
    if (hbm_bytes) *hbm_bytes = (uint64_t)dev->prop.totalGlobalMem;
    return BV_OK;
}

// ------------------------------------------------------------------- index
static uint32_t pad_to_pow2(uint32_t n) {
    uint32_t p = 4;
    while (p < n) p <<= 1;
    return p;
}

// mulberry32 / randomSigns / Rotator signs (src/quant/prng.ts:5-22,
// src/quant/rotator.ts:44-58): computed once on the host per index.
static uint32_t mb32_next(uint32_t &a) {
    uint32_t s = a + 0x6d2b79f5u;
    a = s;
    uint32_t t = (s ^ (s >> 15)) * (1u | s);
    t = (t + (t ^ (t >> 7)) * (61u | t)) ^ t;
    return t ^ (t >> 14);
}

static void rotator_signs(uint32_t dim, uint32_t seed, uint32_t rounds, std::vector<float> &out) {
    const uint32_t P = pad_to_pow2(dim);
    out.assign((size_t)rounds * P + 64, 0.0f);
    const double inv = 1.0 / std::sqrt((double)P);
    for (uint32_t r = 0; r < rounds; r++) {
        uint32_t a = seed ^ (uint32_t)(0x9e3779b9ull * (uint64_t)(r + 1));
        for (uint32_t i = 0; i < P; i++) {
            const double draw = (double)mb32_next(a) / 4294967296.0;
            const double sgn = draw < 0.5 ? -1.0 : 1.0;
            out[(size_t)r * P + i] = (float)(sgn * inv);
        }
    }
}

extern "C" int bv_index_create(bv_device *dev, const bv_index_desc *desc, bv_index **out) {
    if (!dev || !desc || !out) return fail(BV_E_INVALID, "null argument");
    // a desc from before ivf_incremental (72 bytes) reads that field as 0
    const size_t given = desc->size;
    if (given < offsetof(bv_index_desc, ivf_incremental)) return fail(BV_E_INVALID, "bv_index_desc.size too small");
    if (dev->lost) return fail(BV_E_DEVICE_LOST, "GPU device lost; re-create the store");
    bv_index_desc d{};
    std::memcpy(&d, desc, std::min(given, sizeof(bv_index_desc)));
    if (d.dim == 0) return fail(BV_E_INVALID, "dimension must be a positive integer, got %u", d.dim);
    if (d.metric > BV_METRIC_L2) return fail(BV_E_INVALID, "unknown metric %u", d.metric);
    if (d.kind > BV_KIND_IVFQUANT) return fail(BV_E_INVALID, "unknown index kind %u", d.kind);
    const bool quant = d.kind == BV_KIND_QUANT || d.kind == BV_KIND_IVFQUANT;
    if (d.bits != 0 && d.bits != 1 && d.bits != 4 && d.bits != 8)
        return fail(BV_E_UNSUPPORTED, "quantBits %u not supported (ships 0, 1, 4, 8)", d.bits);
    if (quant && d.bits == 0) return fail(BV_E_INVALID, "quantized index kinds need bits 1, 4 or 8");
    if (!quant && d.bits != 0) return fail(BV_E_INVALID, "fp32 index kinds need bits 0");
    // buildIndex's rejections (src/index.ts:124-141)
    if ((d.kind == BV_KIND_IVF || d.kind == BV_KIND_IVFQUANT) && d.metric == BV_METRIC_L2)
        return fail(BV_E_UNSUPPORTED, "IVF supports metric cosine/dot only (l2 is later work)");
    if (d.kind == BV_KIND_QUANT && d.metric == BV_METRIC_L2)
        return fail(BV_E_UNSUPPORTED,
                    "quantized mode supports metric cosine/dot only (l2 quantization is later work)");
    if ((d.kind == BV_KIND_IVF || d.kind == BV_KIND_IVFQUANT) && d.nlist > IVF_MAX_NLIST)
        return fail(BV_E_UNSUPPORTED, "nlist %u exceeds %u", d.nlist, IVF_MAX_NLIST);
    if (d.scorer == BV_SCORER_HAMMING && d.bits != 1)
        return fail(BV_E_UNSUPPORTED, "the Hamming scorer needs 1-bit codes");
    if (d.scorer == BV_SCORER_INT8SYM && d.bits != 8)
        return fail(BV_E_UNSUPPORTED, "the int8 symmetric scorer needs int8 codes");
    if (d.scorer > BV_SCORER_INT8SYM) return fail(BV_E_INVALID, "unknown scorer %u", d.scorer);
    if (!d.has_seed) d.seed = 0x9e3779b9u;
    if (d.rounds == 0) d.rounds = 2;

    bv_index *x = new bv_index();
    x->dev = dev;
    x->d = d;
    x->dim = d.dim;
    x->quant = quant;
    if (quant) {
        x->P = pad_to_pow2(d.dim);
        if (x->P > 4096) {
            delete x;
            return fail(BV_E_UNSUPPORTED, "quantized dimension %u (padded %u) exceeds 4096", d.dim, pad_to_pow2(d.dim));
        }
        const uint32_t per = d.bits == 8 ? 4 : d.bits == 4 ? 8 : 32;
        x->words_per_row = x->P / per;
        x->row_bytes = x->words_per_row * 4;
        if (d.bits == 8) x->codec = d.scorer == BV_SCORER_INT8SYM ? C_I8S : C_Q8;
        else if (d.bits == 4) x->codec = C_Q4;
        // 1-bit asymmetric: the bit-plane prefilter from P = 128 (one 16-byte
        // unit per 128 codes), the plain fp32 sum below
        else x->codec = d.scorer == BV_SCORER_HAMMING ? C_HAM : (x->P >= 128 ? C_Q1P : C_Q1A);
        x->units = x->codec == C_Q1A ? x->row_bytes / 4 : x->row_bytes / 16;
        if (x->row_bytes < 16 && x->codec != C_Q1A) {
            delete x;
            return fail(BV_E_UNSUPPORTED, "dimension %u too small for this code layout", d.dim);
        }
    } else {
        x->P = d.dim;
        x->row_bytes = d.dim * 4;
        const bool l2 = d.metric == BV_METRIC_L2;
        if (d.dim % 4 == 0) {
            x->codec = l2 ? C_F32L2 : C_F32DOT;
            x->units = d.dim / 4;
        } else {
            x->codec = l2 ? C_F32L2_S : C_F32DOT_S;
            x->units = d.dim;
        }
    }
    if (d.kind == BV_KIND_IVF || d.kind == BV_KIND_IVFQUANT) {
        // src/index/ivf.ts:107-109, src/index/ivfquant.ts:112-124
        x->ivf = true;
        x->sample_cap = std::max<uint32_t>(1024, d.sample_size ? d.sample_size : 50000);
        x->sample_dim = quant ? x->P : d.dim;
        const uint32_t ivf_seed = d.has_ivf_seed ? d.ivf_seed : (quant ? d.seed : 0x51ed270bu);
        x->sample_rng = quant ? (ivf_seed ^ 0x85ebca6bu) : ivf_seed;
    }
    if (!scan_supported(x->codec, x->units)) {
        int c = x->codec;
        delete x;
        return fail(BV_E_UNSUPPORTED, "dimension %u not supported by the scan kernels (codec %d)", d.dim, c);
    }
    hipError_t e = hipSetDevice(dev->ordinal);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&x->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&x->ev0);
    if (e == hipSuccess) e = hipEventCreate(&x->ev1);
    if (e == hipSuccess && !quant && !x->ivf) {
        e = x->rsq_max.ensure(256, 0, x->stream, false);
        if (e == hipSuccess) e = hipMemset(x->rsq_max.p, 0, 256);
    }
    if (e == hipSuccess && quant) {
        std::vector<float> s;
        rotator_signs(d.dim, d.seed, d.rounds, s);
        e = x->signs.ensure(s.size() * 4, 0, x->stream, false);
        if (e == hipSuccess) e = hipMemcpy(x->signs.p, s.data(), s.size() * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = x->slow.ensure(256, 0, x->stream, false);
        if (e == hipSuccess) e = hipMemset(x->slow.p, 0, 256);
    }
    if (e != hipSuccess) {
        int rc = hip_fail(dev, e, "bv_index_create");
        delete x;
        return rc;
    }
    *out = x;
    return BV_OK;
}

extern "C" int bv_index_destroy(bv_index *idx) {
    if (!idx) return BV_OK;
    (void)hipSetDevice(idx->dev->ordinal);
    if (idx->stream) (void)hipStreamSynchronize(idx->stream);
    for (auto &pr : idx->tev) {
        (void)hipEventDestroy(pr.first);
        (void)hipEventDestroy(pr.second);
    }
    if (idx->ev0) (void)hipEventDestroy(idx->ev0);
    if (idx->ev1) (void)hipEventDestroy(idx->ev1);
    for (auto &l : idx->lanes) {
        if (l.stream) (void)hipStreamSynchronize(l.stream);
        if (l.stream) (void)hipStreamDestroy(l.stream);
    }
    if (idx->ev_mut) (void)hipEventDestroy(idx->ev_mut);
    if (idx->copy_stream) (void)hipStreamSynchronize(idx->copy_stream);
    for (hipEvent_t e : idx->up_ev)
        if (e) (void)hipEventDestroy(e);
    if (idx->copy_stream) (void)hipStreamDestroy(idx->copy_stream);
    if (idx->stream) (void)hipStreamDestroy(idx->stream);
    delete idx;
    return BV_OK;
}

extern "C" int bv_index_size(const bv_index *idx, uint64_t *rows) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    if (!idx || !rows) return fail(BV_E_INVALID, "null argument");
    *rows = idx->rows;
    return BV_OK;
}

static int check_live(bv_index *idx) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    if (idx->dev->lost) return fail(BV_E_DEVICE_LOST, "GPU device lost; re-create the store");
    hipError_t e = hipSetDevice(idx->dev->ordinal);
    if (e != hipSuccess) return hip_fail(idx->dev, e, "hipSetDevice");
    return BV_OK;
}

// ------------------------------------------------------------------ IVF
static double mb32_draw(uint32_t &a) { return (double)mb32_next(a) / 4294967296.0; }

// Reservoir sampling of appended rows (src/index/ivfquant.ts:235-245,
// src/index/ivf.ts:175-187): per row in order, the next free slot while the
// sample is filling, else slot floor(rng() * (seen + 1)) when below the
// capacity.  Only the last row written to a slot within the batch keeps it
// (earlier ones would be overwritten in order).  The plan is drawn on a copy
// of the sampler state; ivf_commit applies it once the append can no longer
// fail, so a failed append leaves the sample as it was.
struct ReservoirPlan {
    uint64_t filled, seen;
    uint32_t rng;
    std::vector<int32_t> slots;
};

static void ivf_plan(const bv_index *idx, uint64_t count, ReservoirPlan &pl) {
    pl.filled = idx->sample_filled;
    pl.seen = idx->sample_seen;
    pl.rng = idx->sample_rng;
    pl.slots.assign(count, -1);
    for (uint64_t i = 0; i < count; ++i) {
        if (pl.filled < idx->sample_cap) {
            pl.slots[i] = (int32_t)pl.filled++;
        } else {
            const uint64_t j = (uint64_t)std::floor(mb32_draw(pl.rng) * (double)(pl.seen + 1));
            if (j < idx->sample_cap) pl.slots[i] = (int32_t)j;
        }
        pl.seen++;
    }
    std::vector<uint8_t> taken(idx->sample_cap, 0);
    for (uint64_t i = count; i-- > 0;) {
        if (pl.slots[i] < 0) continue;
        if (taken[pl.slots[i]]) pl.slots[i] = -1;
        else taken[pl.slots[i]] = 1;
    }
}

static void ivf_commit(bv_index *idx, uint64_t base, const ReservoirPlan &pl, bool extended) {
    idx->sample_filled = pl.filled;
    idx->sample_seen = pl.seen;
    idx->sample_rng = pl.rng;
    if (idx->sample_row.size() < idx->sample_filled) idx->sample_row.resize(idx->sample_filled);
    for (uint64_t i = 0; i < pl.slots.size(); ++i)
        if (pl.slots[i] >= 0) idx->sample_row[(uint32_t)pl.slots[i]] = base + i;
    // lists are stale after any append (ivfquant.ts:462), unless the append
    // extended them (incremental mode, lists current before it)
    if (!extended) idx->built_rows = ~0ull;
}

// The matrix-core assignment of int8 codes (the final pass of a build and
// incremental appends): its scratch for n rows and nlist centroids, taken
// before anything is assigned.
static int ivf_assign_reserve(bv_index *idx, uint64_t n, uint32_t nlist) {
    const int bits = idx->quant ? (int)idx->d.bits : 0;
    const uint32_t P = idx->sample_dim;
    if (!ivf_assign_mfma_ok(bits, P, nlist) || n == 0) return BV_OK;
    hipStream_t s = idx->stream;
    const size_t pad = ivf_mfma_nlist_pad(nlist);
    HIPX(idx->dev, idx->ivf_lev.ensure(pad * 2 * P, 0, s), "scratch");
    HIPX(idx->dev, idx->ivf_ls.ensure(pad * 2 * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivf_mwords.ensure(8, 0, s), "scratch");
    HIPX(idx->dev, idx->ivf_queue.ensure((size_t)ivf_mfma_qcap(n) * sizeof(IvfRecheck), 0, s), "scratch");
    HIPX(idx->dev, idx->h_cnt.ensure(8), "pinned buffer");
    return BV_OK;
}

// The assignment of fa.n rows to the centroids (fa.out): int8 codes of a
// padded dimension the matrix pass takes go through it and the exact
// re-check of the rows it leaves open (same result as ivf_assign<8>), every
// other kind through ivf_assign.  Waits for the device.
static int ivf_assign_rows(bv_index *idx, const IvfAssignArgs &fa, int bits) {
    hipStream_t s = idx->stream;
    idx->ivf_exact_rows = fa.n;
    if (!ivf_assign_mfma_ok(bits, fa.dim, fa.nlist) || fa.n == 0) {
        HIPX(idx->dev, ivf_launch_assign(fa, bits, s), "assign kernel");
        return BV_OK;
    }
    IvfMfmaScratch m{idx->ivf_lev.as<int8_t>(), idx->ivf_ls.as<float>(), idx->ivf_mwords.as<uint32_t>(),
                     idx->ivf_queue.as<IvfRecheck>(), ivf_mfma_qcap(fa.n)};
    HIPX(idx->dev, ivf_launch_assign_mfma(fa, m, s), "assign kernel");
    uint32_t *h = (uint32_t *)idx->h_cnt.p;
    HIPX(idx->dev, hipMemcpyAsync(h, m.words + 1, 4, hipMemcpyDeviceToHost, s), "count download");
    HIPX(idx->dev, hipStreamSynchronize(s), "assign kernel");
    const uint32_t queued = h[0];
    if (queued > m.qcap) {  // more open rows than the queue holds: every row exactly
        HIPX(idx->dev, ivf_launch_assign(fa, bits, s), "assign kernel");
        return BV_OK;
    }
    HIPX(idx->dev, ivf_launch_assign_recheck(fa, m, queued, s), "assign kernel");
    idx->ivf_exact_rows = queued;
    return BV_OK;
}

// Incremental append: rows [base, base + count) assigned to the current
// centroids with the build's final-assignment arithmetic, then merged into
// the lists (each list: its rows, then the new ones, ascending).  The lists
// equal those a final assignment over every row with these centroids gives.
// The buffers ivf_extend_lists uses, allocated before an append changes
// anything.
static int ivf_extend_reserve(bv_index *idx, uint64_t base, uint64_t count) {
    const uint32_t nlist = idx->nlist;
    hipStream_t s = idx->stream;
    const uint32_t nblk = ivf_list_blocks(count);
    HIPX(idx->dev, idx->ivf_assign.ensure(count * 4, 0, s), "scratch");
    if (ivf_assign_split(count)) HIPX(idx->dev, idx->ivf_keys.ensure(count * 8, 0, s), "scratch");
    int rc = ivf_assign_reserve(idx, count, nlist);
    if (rc) return rc;
    HIPX(idx->dev, idx->ivf_hist.ensure((size_t)std::max(nblk, 1u) * nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivf_base.ensure((size_t)std::max(nblk, 1u) * nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivf_totals.ensure((size_t)nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivf_toff.ensure(((size_t)nlist + 1) * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivf_trows.ensure(count * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->list_off2.ensure(((size_t)nlist + 1) * 4, 0, s), "lists");
    HIPX(idx->dev, idx->list_rows2.ensure((base + count) * 4, 0, s), "lists");
    return BV_OK;
}

// Runs on the buffers ivf_extend_reserve allocated; the new lists are built
// in the second buffers and swapped in at the end.
static int ivf_extend_lists(bv_index *idx, uint64_t base, uint64_t count) {
    const uint32_t nlist = idx->nlist;
    hipStream_t s = idx->stream;
    IvfAssignArgs fa{};
    fa.n = count;
    fa.dim = idx->sample_dim;
    fa.centroids = idx->centroids.as<float>();
    fa.cen_stride = idx->sample_dim;
    fa.nlist = nlist;
    fa.out = idx->ivf_assign.as<uint32_t>();
    fa.keys = idx->ivf_keys.as<uint64_t>();
    if (idx->quant) {
        fa.codes = idx->codes.as<uint32_t>() + base * idx->words_per_row;
        fa.words_per_row = idx->words_per_row;
        fa.scales = idx->scales.as<float>() + base;
    } else {
        fa.rows = idx->raw.as<float>() + base * idx->dim;
        fa.row_stride = idx->dim;
    }
    int rc = ivf_assign_rows(idx, fa, idx->quant ? (int)idx->d.bits : 0);
    if (rc) return rc;
    HIPX(idx->dev, ivf_launch_lists(fa.out, count, nlist, idx->ivf_hist.as<uint32_t>(), idx->ivf_base.as<uint32_t>(),
                                    idx->ivf_totals.as<uint32_t>(), idx->ivf_toff.as<uint32_t>(),
                                    idx->ivf_trows.as<uint32_t>(), s),
         "list kernels");
    HIPX(idx->dev,
         ivf_launch_merge_lists(idx->list_off.as<uint32_t>(), idx->list_rows.as<uint32_t>(),
                                idx->ivf_toff.as<uint32_t>(), idx->ivf_trows.as<uint32_t>(), (uint32_t)base, nlist,
                                idx->list_off2.as<uint32_t>(), idx->list_rows2.as<uint32_t>(), s),
         "list merge kernel");
    std::swap(idx->list_off.p, idx->list_off2.p);
    std::swap(idx->list_off.cap, idx->list_off2.cap);
    std::swap(idx->list_rows.p, idx->list_rows2.p);
    std::swap(idx->list_rows.cap, idx->list_rows2.cap);
    std::vector<uint32_t> off(nlist + 1);
    HIPX(idx->dev, hipMemcpyAsync(off.data(), idx->list_off.p, (nlist + 1) * 4, hipMemcpyDeviceToHost, s), "download");
    HIPX(idx->dev, hipStreamSynchronize(s), "list merge");
    for (uint32_t c = 0; c < nlist; ++c) idx->list_sizes_desc[c] = off[c + 1] - off[c];
    std::sort(idx->list_sizes_desc.begin(), idx->list_sizes_desc.end(), std::greater<uint32_t>());
    idx->built_rows = base + count;
    idx->retrain_due = true;
    return BV_OK;
}

static int lanes_join(bv_index *idx);
static int lanes_mark(bv_index *idx);

// Host appends larger than one staging chunk go through two pinned buffers:
// while chunk i's rows travel to the device on the copy stream, the host
// copies chunk i + 1 into the other buffer (several threads), and the index
// stream encodes chunk i - 1 once its copy has landed.  A pageable source
// otherwise crosses PCIe at about half the rate of a pinned one.
constexpr size_t UPLOAD_CHUNK = 64ull << 20;
constexpr unsigned UPLOAD_THREADS = 8;

static int staging_ready(bv_index *idx) {
    if (!idx->copy_stream)
        HIPX(idx->dev, hipStreamCreateWithFlags(&idx->copy_stream, hipStreamNonBlocking), "copy stream");
    for (hipEvent_t &e : idx->up_ev)
        if (!e) HIPX(idx->dev, hipEventCreateWithFlags(&e, hipEventDisableTiming), "copy event");
    for (HostBuf &b : idx->up_ring) HIPX(idx->dev, b.ensure(UPLOAD_CHUNK), "pinned staging buffer");
    return BV_OK;
}

static void parallel_copy(void *dst, const void *src, size_t bytes) {
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const unsigned nt = (unsigned)std::min<size_t>(std::min(UPLOAD_THREADS, hw), std::max<size_t>(1, bytes >> 22));
    if (nt <= 1) {
        std::memcpy(dst, src, bytes);
        return;
    }
    const size_t part = (bytes / nt + 63) & ~size_t(63);
    std::vector<std::thread> th;
    th.reserve(nt);
    size_t done = 0;  // bytes handed to threads; the rest is copied here
    try {
        for (unsigned t = 0; t < nt; ++t) {
            const size_t o = (size_t)t * part;
            if (o >= bytes) break;
            const size_t len = std::min(part, bytes - o);
            th.emplace_back([=] { std::memcpy((char *)dst + o, (const char *)src + o, len); });
            done = o + len;
        }
    } catch (...) {  // no thread to be had: this thread copies what is left
    }
    if (done < bytes) std::memcpy((char *)dst + done, (const char *)src + done, bytes - done);
    for (auto &x : th) x.join();
}

// A source the caller already pinned (hipHostMalloc) is copied directly.
static bool host_pinned(const void *p) {
    hipPointerAttribute_t at{};
    if (hipPointerGetAttributes(&at, p) != hipSuccess) {
        (void)hipGetLastError();  // pageable memory: clear the lookup's error
        return false;
    }
    return at.type == hipMemoryTypeHost;
}

// Chunk rows [r0, r0 + m) from host `src` into idx->raw through staging
// buffer b; the index stream waits for the copy.
static int stage_rows(bv_index *idx, const float *src, uint64_t r0, uint64_t m, int b) {
    const size_t rb = (size_t)idx->dim * 4, bytes = m * rb;
    HIPX(idx->dev, hipEventSynchronize(idx->up_ev[b]), "staging wait");  // the buffer's last copy has landed
    parallel_copy(idx->up_ring[b].p, src, bytes);
    HIPX(idx->dev,
         hipMemcpyAsync(idx->raw.as<char>() + r0 * rb, idx->up_ring[b].p, bytes, hipMemcpyHostToDevice,
                        idx->copy_stream),
         "row upload");
    HIPX(idx->dev, hipEventRecord(idx->up_ev[b], idx->copy_stream), "copy event");
    HIPX(idx->dev, hipStreamWaitEvent(idx->stream, idx->up_ev[b], 0), "copy wait");
    return BV_OK;
}

// Append: every allocation happens first, so a failure (or an injected one)
// leaves the index exactly as it was; then the rows are copied and encoded
// into space past the index's rows.  The rows an IVF reservoir samples go to
// a staging buffer, not to their slots, so a failure at any point before the
// commit (a later staged chunk, an injected late failure) leaves the sample,
// the reservoir state and the lists as they were; the commit scatters the
// sampled rows, extends the lists (incremental mode) and advances the
// reservoir.
static int append_common(bv_index *idx, const float *data, bool device_src, uint64_t count) {
    const uint64_t base = idx->rows, total = base + count;
    const size_t rb = (size_t)idx->dim * 4;
    int jrc = lanes_join(idx);  // buffers may be reallocated below
    if (jrc) return jrc;
    if (idx->dev->inject_append_oom) {
        idx->dev->inject_append_oom = false;
        return fail(BV_E_OOM, "row buffer: out of device memory");
    }
    ReservoirPlan plan;
    std::vector<int32_t> pend_slot;         // per appended row: its staging row, or -1
    std::vector<uint32_t> src_row, dst_slot;  // the scatter: staging (or raw) row -> reservoir slot
    if (idx->ivf) {
        ivf_plan(idx, count, plan);
        pend_slot.assign(count, -1);
        for (uint64_t i = 0; i < count; ++i)
            if (plan.slots[i] >= 0) {
                pend_slot[i] = (int32_t)dst_slot.size();
                src_row.push_back(idx->quant ? (uint32_t)dst_slot.size() : (uint32_t)(base + i));
                dst_slot.push_back((uint32_t)plan.slots[i]);
            }
    }
    const size_t taken = dst_slot.size();
    const bool extend = idx->ivf && idx->built_rows == base && idx->nlist && idx->d.ivf_incremental;
    HIPX(idx->dev, idx->raw.ensure(total * rb, base * rb, idx->stream), "row buffer");
    if (idx->quant) {
        HIPX(idx->dev, idx->codes.ensure(total * idx->row_bytes, base * idx->row_bytes, idx->stream), "code buffer");
        HIPX(idx->dev, idx->scales.ensure(total * 4, base * 4, idx->stream), "scale buffer");
    }
    const bool norms = !idx->quant && !idx->ivf;  // flat fp32: the exact batch's error bound needs them
    if (norms) HIPX(idx->dev, idx->rsq.ensure(total * 4, base * 4, idx->stream), "norm buffer");
    const bool code_norms = idx->codec == C_Q8 && !idx->ivf;  // flat int8: the level-one batch bound needs them
    if (code_norms) HIPX(idx->dev, idx->cnorm.ensure(total * 4, base * 4, idx->stream), "norm buffer");
    if (idx->ivf) {
        HIPX(idx->dev, idx->sample.ensure(plan.filled * (size_t)idx->sample_dim * 4, idx->sample.cap, idx->stream),
             "sample buffer");
        HIPX(idx->dev, idx->ivf_slot.ensure(count * 4, 0, idx->stream), "scratch");
        HIPX(idx->dev, idx->ivf_idx.ensure(std::max<size_t>(taken, 1) * 4, 0, idx->stream), "scratch");
        HIPX(idx->dev, idx->ivf_idx2.ensure(std::max<size_t>(taken, 1) * 4, 0, idx->stream), "scratch");
        if (idx->quant)
            HIPX(idx->dev, idx->ivf_pend.ensure(std::max<size_t>(taken, 1) * idx->sample_dim * 4, 0, idx->stream),
                 "sample staging buffer");
        if (extend) {
            int rc = ivf_extend_reserve(idx, base, count);
            if (rc) return rc;
        }
    }
    const bool staged = !device_src && count * rb > UPLOAD_CHUNK && !host_pinned(data);
    if (staged) {
        int rc = staging_ready(idx);
        if (rc) return rc;
    } else {
        HIPX(idx->dev,
             hipMemcpyAsync(idx->raw.as<char>() + base * rb, data, count * rb,
                            device_src ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, idx->stream),
             "row upload");
    }
    if (idx->ivf) {
        HIPX(idx->dev,
             hipMemcpyAsync(idx->ivf_slot.p, pend_slot.data(), count * 4, hipMemcpyHostToDevice, idx->stream),
             "upload");
        if (taken) {
            HIPX(idx->dev, hipMemcpyAsync(idx->ivf_idx.p, src_row.data(), taken * 4, hipMemcpyHostToDevice, idx->stream),
                 "upload");
            HIPX(idx->dev,
                 hipMemcpyAsync(idx->ivf_idx2.p, dst_slot.data(), taken * 4, hipMemcpyHostToDevice, idx->stream),
                 "upload");
        }
    }
    // the rows in chunks (one chunk unless staged): upload, norms, encode
    // (sampled rows' rotations into the staging buffer)
    const uint64_t crow = staged ? std::max<uint64_t>(1, UPLOAD_CHUNK / rb) : count;
    for (uint64_t off = 0, i = 0; off < count; off += crow, ++i) {
        const uint64_t m = std::min(crow, count - off), r0 = base + off;
        if (staged) {
            int rc = stage_rows(idx, data + off * idx->dim, r0, m, (int)(i & 1));
            if (rc) {  // rows copied so far are not counted: the index keeps its size
                (void)hipStreamSynchronize(idx->copy_stream);
                (void)hipStreamSynchronize(idx->stream);
                return rc;
            }
        }
        if (norms)
            HIPX(idx->dev,
                 launch_row_sqnorms(idx->raw.as<float>() + r0 * idx->dim, m, idx->dim, idx->rsq.as<float>() + r0,
                                    idx->rsq_max.as<uint32_t>(), idx->stream),
                 "norm kernel");
        if (idx->quant) {
            EncodeArgs e{};
            e.src = idx->raw.as<float>() + r0 * idx->dim;
            e.rows = m;
            e.dim = idx->dim;
            e.P = idx->P;
            e.signs = idx->signs.as<float>();
            e.rounds = idx->d.rounds;
            e.bits = idx->d.bits;
            e.codes = idx->codes.as<uint32_t>() + r0 * idx->words_per_row;
            e.scales = idx->scales.as<float>() + r0;
            e.slow_rows = idx->slow.as<uint32_t>();
            if (idx->ivf) {
                e.sample_slot = idx->ivf_slot.as<int32_t>() + off;
                e.sample = idx->ivf_pend.as<float>();
            }
            HIPX(idx->dev, launch_encode(e, idx->stream), "encode kernel");
            if (code_norms)
                HIPX(idx->dev,
                     launch_row_code_norms(idx->codes.as<uint32_t>() + r0 * idx->words_per_row, m,
                                           idx->words_per_row, idx->cnorm.as<float>() + r0, idx->stream),
                     "norm kernel");
        }
    }
    if (idx->dev->inject_append_late) {  // (tests: a failure after the rows are encoded)
        idx->dev->inject_append_late = false;
        (void)hipStreamSynchronize(idx->stream);
        return fail(BV_E_HIP, "append: injected failure after the rows were encoded");
    }
    // commit: sampled rows to their reservoir slots, lists, reservoir state
    if (taken) {
        IvfCopyArgs c{};
        c.src = idx->quant ? idx->ivf_pend.as<float>() : idx->raw.as<float>();
        c.src_stride = idx->quant ? idx->sample_dim : idx->dim;
        c.src_idx = idx->ivf_idx.as<uint32_t>();
        c.dst = idx->sample.as<float>();
        c.dst_stride = idx->sample_dim;
        c.dst_idx = idx->ivf_idx2.as<uint32_t>();
        c.n = (uint32_t)taken;
        c.dim = idx->quant ? idx->sample_dim : idx->dim;
        HIPX(idx->dev, ivf_launch_copy_rows(c, idx->stream), "sample copy");
    }
    if (extend) {
        int rc = ivf_extend_lists(idx, base, count);
        if (rc) return rc;
    }
    if (idx->ivf) ivf_commit(idx, base, plan, extend);
    HIPX(idx->dev, hipStreamSynchronize(idx->stream), "append");
    idx->rows = total;
    if (idx->ivf_pend.cap > (64ull << 20)) idx->ivf_pend.release();  // a large staging buffer is not kept
    return lanes_mark(idx);
}

extern "C" int bv_index_append(bv_index *idx, const float *data, uint64_t n_floats, uint64_t count) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (n_floats != count * idx->dim)
        return fail(BV_E_INVALID, "expected %llu floats, got %llu", (unsigned long long)(count * idx->dim),
                    (unsigned long long)n_floats);
    if (count == 0) return BV_OK;
    if (!data) return fail(BV_E_INVALID, "data is null");
    if (idx->rows + count > 0xfffffffeull) return fail(BV_E_INVALID, "row count exceeds 2^32-2");
    return append_common(idx, data, false, count);
}

extern "C" int bv_index_append_device(bv_index *idx, const float *d_data, uint64_t count) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (count == 0) return BV_OK;
    if (!d_data) return fail(BV_E_INVALID, "data is null");
    if (idx->rows + count > 0xfffffffeull) return fail(BV_E_INVALID, "row count exceeds 2^32-2");
    return append_common(idx, d_data, true, count);
}

// IVF build (src/index/ivfquant.ts:248-312, src/index/ivf.ts:191-259):
// spherical k-means on the reservoir sample with device assignment and
// device mean update (the host only draws the init / re-seed rows from
// mulberry32, as the reference's trainer does), then every row is assigned
// (by its codes for quantized kinds) and the CSR lists are built on the
// device.
static int run_fused(bv_index *idx, const float *d_q, uint32_t nq, uint32_t kprime, uint32_t k_out, bool rerank,
                     const uint32_t *d_mask, uint64_t mask_bits, uint32_t *d_rows, float *d_scores, uint32_t *d_n,
                     bool may_alternate = false);

// nprobe auto-tune for targetRecall (src/index/ivfTune.ts:31-42,
// ivfquant.ts:322-344, ivf.ts:269-291), after a build, when no nprobe is
// configured.  For up to 32 reservoir rows spread evenly over the sample
// (pickTuneQueries), the top k+1 of every row by the index's own scores
// (probing every list scores every row) and the probe rank of each hit's
// list, skipping the first hit (the query row itself); chooseNprobe then
// takes the smallest nprobe whose share of hits probed meets the target.
// A sampled row's stored fp32 vector rotates to exactly its sample row, so
// the queries go through the ordinary query path.
static int ivf_tune(bv_index *idx, const uint32_t *d_assign) {
    idx->tuned_nprobe = 0;
    idx->tuned_recall = -1.0f;
    if (!(idx->d.target_recall >= 0.0f) || idx->d.nprobe) return BV_OK;
    const double target = std::min(1.0, std::max(0.0, (double)idx->d.target_recall));
    const uint64_t rows = idx->rows;
    const uint32_t nlist = idx->nlist;
    const uint64_t kk = std::min<uint64_t>(10, rows ? rows - 1 : 0);
    if (kk < 1 || nlist <= 1) {
        idx->tuned_nprobe = 1;
        idx->tuned_recall = 1.0f;
        return BV_OK;
    }
    const uint32_t k1 = (uint32_t)kk + 1;
    const uint64_t filled = idx->sample_filled;
    const uint32_t nq = (uint32_t)std::min<uint64_t>(filled, 32);
    hipStream_t s = idx->stream;
    const size_t rb = (size_t)idx->dim * 4;
    HIPX(idx->dev, idx->tune_q.ensure(std::max<size_t>((size_t)nq * rb, 4), 0, s), "scratch");
    for (uint32_t i = 0; i < nq; ++i) {
        const uint64_t r = idx->sample_row[(uint64_t)i * filled / nq];
        HIPX(idx->dev, hipMemcpyAsync(idx->tune_q.as<char>() + i * rb, idx->raw.as<char>() + r * rb, rb,
                                      hipMemcpyDeviceToDevice, s),
             "tune queries");
    }
    const float *d_q = idx->tune_q.as<float>();
    // the top k+1 over every row
    HIPX(idx->dev, idx->tune_rows.ensure((size_t)nq * k1 * 4, 0, s), "output buffer");
    HIPX(idx->dev, idx->tune_scores.ensure((size_t)nq * k1 * 4, 0, s), "output buffer");
    HIPX(idx->dev, idx->tune_n.ensure((size_t)nq * 4, 0, s), "output buffer");
    idx->ivf = false;
    int rc = run_fused(idx, d_q, nq, k1, k1, false, nullptr, 0, idx->tune_rows.as<uint32_t>(),
                       idx->tune_scores.as<float>(), idx->tune_n.as<uint32_t>());
    idx->ivf = true;
    if (rc) return rc;
    // probe scores of the rotated queries against every centroid
    const float *qrot = d_q;
    if (idx->quant) {
        HIPX(idx->dev, idx->tune_rot.ensure((size_t)nq * idx->P * 4, 0, s), "query buffer");
        EncodeArgs e{};
        e.src = d_q;
        e.rows = nq;
        e.dim = idx->dim;
        e.P = idx->P;
        e.signs = idx->signs.as<float>();
        e.rounds = idx->d.rounds;
        e.rotated = idx->tune_rot.as<float>();
        HIPX(idx->dev, launch_encode(e, s), "query rotate kernel");
        qrot = idx->tune_rot.as<float>();
    }
    HIPX(idx->dev, idx->probe_scores.ensure((size_t)nq * nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->probes.ensure((size_t)nq * 4, 0, s), "scratch");
    IvfProbeArgs pa{};
    pa.centroids = idx->centroids.as<float>();
    pa.nlist = nlist;
    pa.P = idx->sample_dim;
    pa.qrot = qrot;
    pa.scores = idx->probe_scores.as<float>();
    pa.nprobe = 1;
    pa.probes = idx->probes.as<uint32_t>();
    HIPX(idx->dev, ivf_launch_probes(pa, nq, s), "probe kernels");
    std::vector<uint32_t> gt((size_t)nq * k1), gtn(nq), assign(rows);
    std::vector<float> ps((size_t)nq * nlist);
    HIPX(idx->dev, hipMemcpyAsync(gt.data(), idx->tune_rows.p, gt.size() * 4, hipMemcpyDeviceToHost, s), "download");
    HIPX(idx->dev, hipMemcpyAsync(gtn.data(), idx->tune_n.p, (size_t)nq * 4, hipMemcpyDeviceToHost, s), "download");
    HIPX(idx->dev, hipMemcpyAsync(ps.data(), idx->probe_scores.p, ps.size() * 4, hipMemcpyDeviceToHost, s),
         "download");
    HIPX(idx->dev, hipMemcpyAsync(assign.data(), d_assign, rows * 4, hipMemcpyDeviceToHost, s), "download");
    HIPX(idx->dev, hipStreamSynchronize(s), "tune");
    std::vector<uint32_t> hist(nlist, 0), order(nlist), rank(nlist);
    uint64_t total = 0;
    for (uint32_t q = 0; q < nq; ++q) {
        const float *sc = ps.data() + (size_t)q * nlist;
        for (uint32_t c = 0; c < nlist; ++c) order[c] = c;
        std::stable_sort(order.begin(), order.end(), [&](uint32_t x, uint32_t y) { return sc[x] > sc[y]; });
        for (uint32_t r = 0; r < nlist; ++r) rank[order[r]] = r;
        for (uint32_t h = 1; h < gtn[q]; ++h) {
            hist[rank[assign[gt[(size_t)q * k1 + h]]]]++;
            total++;
        }
    }
    // chooseNprobe
    uint32_t np = nlist;
    double rec = 1.0;
    if (total) {
        uint64_t cum = 0;
        for (uint32_t p = 1; p <= nlist; ++p) {
            cum += hist[p - 1];
            if ((double)cum / (double)total >= target) {
                np = p;
                rec = (double)cum / (double)total;
                break;
            }
        }
    }
    idx->tuned_nprobe = np;
    idx->tuned_recall = (float)rec;
    return BV_OK;
}

static int ivf_build(bv_index *idx) {
    auto t0 = std::chrono::steady_clock::now();
    const uint64_t rows = idx->rows;
    uint32_t nlist;
    if (idx->d.nlist) {
        nlist = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(idx->d.nlist, rows));
    } else {
        const uint64_t guess = (uint64_t)std::floor(std::sqrt((double)rows) + 0.5);
        nlist = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(std::min<uint64_t>(4096, std::max<uint64_t>(16, guess)), rows));
    }
    const uint32_t seed = idx->d.has_ivf_seed ? idx->d.ivf_seed : 0x51ed270bu;
    const uint32_t iters = idx->d.iters ? idx->d.iters : 8;
    const uint32_t train = (uint32_t)std::min<uint64_t>(idx->sample_filled, idx->d.train_size ? idx->d.train_size : 16384);
    if (train == 0) return fail(BV_E_STATE, "IVF build with an empty sample");
    const uint32_t D = idx->sample_dim;
    hipStream_t s = idx->stream;
    HIPX(idx->dev, idx->centroids.ensure((size_t)nlist * D * 4, 0, s), "centroids");
    const uint64_t nmax = std::max<uint64_t>(rows, train);
    const uint32_t nblk = ivf_list_blocks(nmax);
    HIPX(idx->dev, idx->ivf_assign.ensure(nmax * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivf_hist.ensure((size_t)std::max(nblk, 1u) * nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivf_base.ensure((size_t)std::max(nblk, 1u) * nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivf_totals.ensure((size_t)nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivf_toff.ensure(((size_t)nlist + 1) * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivf_trows.ensure((size_t)train * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivf_idx.ensure((size_t)nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivf_idx2.ensure((size_t)nlist * 4, 0, s), "scratch");

    auto copy_rows = [&](const std::vector<uint32_t> &src, const std::vector<uint32_t> *dst) -> int {
        if (src.empty()) return BV_OK;
        HIPX(idx->dev, hipMemcpyAsync(idx->ivf_idx.p, src.data(), src.size() * 4, hipMemcpyHostToDevice, s), "upload");
        if (dst)
            HIPX(idx->dev, hipMemcpyAsync(idx->ivf_idx2.p, dst->data(), dst->size() * 4, hipMemcpyHostToDevice, s),
                 "upload");
        IvfCopyArgs c{};
        c.src = idx->sample.as<float>();
        c.src_stride = D;
        c.src_idx = idx->ivf_idx.as<uint32_t>();
        c.dst = idx->centroids.as<float>();
        c.dst_stride = D;
        c.dst_idx = dst ? idx->ivf_idx2.as<uint32_t>() : nullptr;
        c.n = (uint32_t)src.size();
        c.dim = D;
        HIPX(idx->dev, ivf_launch_copy_rows(c, s), "centroid copy");
        return BV_OK;
    };
    // randomInitCentroids (kmeans.ts:154-170)
    {
        uint32_t a = seed;
        std::vector<uint32_t> pick(nlist);
        for (uint32_t c = 0; c < nlist; ++c) pick[c] = (uint32_t)std::floor(mb32_draw(a) * (double)train);
        int rc = copy_rows(pick, nullptr);
        if (rc) return rc;
        HIPX(idx->dev, ivf_launch_normalize(idx->centroids.as<float>(), nlist, D, D, s), "normalize");
    }
    IvfAssignArgs ta{};
    ta.n = train;
    ta.dim = D;
    ta.rows = idx->sample.as<float>();
    ta.row_stride = D;
    ta.centroids = idx->centroids.as<float>();
    ta.cen_stride = D;
    ta.nlist = nlist;
    ta.out = idx->ivf_assign.as<uint32_t>();
    if (ivf_assign_split(train) || ivf_assign_split(rows)) {
        HIPX(idx->dev, idx->ivf_keys.ensure((size_t)std::max<uint64_t>(train, rows) * 8, 0, s), "scratch");
        ta.keys = idx->ivf_keys.as<uint64_t>();
    }
    std::vector<uint32_t> toff(nlist + 1);
    for (uint32_t it = 0; it < iters; ++it) {
        HIPX(idx->dev, ivf_launch_assign(ta, 0, s), "assign kernel");
        HIPX(idx->dev, ivf_launch_lists(ta.out, train, nlist, idx->ivf_hist.as<uint32_t>(), idx->ivf_base.as<uint32_t>(),
                                        idx->ivf_totals.as<uint32_t>(), idx->ivf_toff.as<uint32_t>(),
                                        idx->ivf_trows.as<uint32_t>(), s),
             "list kernels");
        HIPX(idx->dev, ivf_launch_means(idx->sample.as<float>(), D, D, idx->ivf_toff.as<uint32_t>(),
                                        idx->ivf_trows.as<uint32_t>(), nlist, idx->centroids.as<float>(), D, s),
             "mean kernel");
        HIPX(idx->dev, hipMemcpyAsync(toff.data(), idx->ivf_toff.p, (nlist + 1) * 4, hipMemcpyDeviceToHost, s),
             "download");
        HIPX(idx->dev, hipStreamSynchronize(s), "k-means");
        // empty clusters re-seeded in cluster order (kmeans.ts:195-199) with
        // the trainer's per-iteration seed (kmeansTrainer.ts:97)
        uint32_t a = seed + it + 1;
        std::vector<uint32_t> src, dst;
        for (uint32_t c = 0; c < nlist; ++c)
            if (toff[c + 1] == toff[c]) {
                src.push_back((uint32_t)std::floor(mb32_draw(a) * (double)train));
                dst.push_back(c);
            }
        int rc = copy_rows(src, &dst);
        if (rc) return rc;
        HIPX(idx->dev, ivf_launch_normalize(idx->centroids.as<float>(), nlist, D, D, s), "normalize");
    }
    // final assignment of every row (ivfquant.ts:291-293: by its codes)
    IvfAssignArgs fa = ta;
    fa.n = rows;
    if (idx->quant) {
        fa.rows = nullptr;
        fa.codes = idx->codes.as<uint32_t>();
        fa.words_per_row = idx->words_per_row;
        fa.scales = idx->scales.as<float>();
    } else {
        fa.rows = idx->raw.as<float>();
        fa.row_stride = idx->dim;
    }
    {
        int rc = ivf_assign_reserve(idx, rows, nlist);
        if (!rc) rc = ivf_assign_rows(idx, fa, idx->quant ? (int)idx->d.bits : 0);
        if (rc) return rc;
        idx->build_exact_rows = idx->ivf_exact_rows;
    }
    HIPX(idx->dev, idx->list_off.ensure(((size_t)nlist + 1) * 4, 0, s), "lists");
    HIPX(idx->dev, idx->list_rows.ensure(std::max<uint64_t>(rows, 1) * 4, 0, s), "lists");
    HIPX(idx->dev, ivf_launch_lists(fa.out, rows, nlist, idx->ivf_hist.as<uint32_t>(), idx->ivf_base.as<uint32_t>(),
                                    idx->ivf_totals.as<uint32_t>(), idx->list_off.as<uint32_t>(),
                                    idx->list_rows.as<uint32_t>(), s),
         "list kernels");
    std::vector<uint32_t> off(nlist + 1);
    HIPX(idx->dev, hipMemcpyAsync(off.data(), idx->list_off.p, (nlist + 1) * 4, hipMemcpyDeviceToHost, s), "download");
    HIPX(idx->dev, hipStreamSynchronize(s), "IVF build");
    idx->list_sizes_desc.resize(nlist);
    for (uint32_t c = 0; c < nlist; ++c) idx->list_sizes_desc[c] = off[c + 1] - off[c];
    std::sort(idx->list_sizes_desc.begin(), idx->list_sizes_desc.end(), std::greater<uint32_t>());
    idx->nlist = nlist;
    idx->built_rows = rows;
    idx->retrain_due = false;
    int rc = ivf_tune(idx, fa.out);
    if (rc) return rc;
    idx->build_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return BV_OK;
}

// The lazy build of the reference's first query after an append
// (ivfquant.ts:461-463).  Query entry points call it before they take any
// scratch or output pointer: the build grows and reuses buffers.
static int ensure_built(bv_index *idx) {
    if (!idx->ivf || idx->rows == 0 || idx->built_rows == idx->rows) return BV_OK;
    // (the build rewrites the lists that queries on the second stream read)
    int rc = lanes_join(idx);
    if (rc) return rc;
    rc = ivf_build(idx);
    if (rc) return rc;
    return lanes_mark(idx);
}

// nprobe for the next query (ivfquant.ts:159-162, 487-491): the per-query
// override (consumed once), else the configured one, else the tuned one,
// else 5% of nlist.
static uint32_t ivf_resolve_nprobe(bv_index *idx) {
    uint32_t n = idx->nprobe_override ? idx->nprobe_override
                 : idx->d.nprobe      ? idx->d.nprobe
                 : idx->tuned_nprobe  ? idx->tuned_nprobe
                                      : (uint32_t)std::max<double>(1.0, std::floor(idx->nlist * 0.05 + 0.5));
    idx->nprobe_override = 0;
    n = std::max<uint32_t>(1, std::min<uint32_t>(n, idx->nlist));
    return std::min<uint32_t>(n, IVF_MAX_NPROBE);
}

// Probes + gathered candidate lists for nq device queries (original space).
// Returns the per-query candidate bound used to size the scan.
// (on the second query stream, `lane`: its own buffers and stream)
static int ivf_candidates(bv_index *idx, const float *d_q, uint32_t nq, uint64_t *max_per_query,
                          bv_index::ScanLane *lane = nullptr) {
    // every query entry point builds before it takes any buffer pointer
    if (idx->built_rows != idx->rows) return fail(BV_E_STATE, "IVF lists are stale");
    hipStream_t s = lane ? lane->stream : idx->stream;
    DevBuf &b_qrot = lane ? lane->ivf_qrot : idx->ivf_qrot, &b_scores = lane ? lane->probe_scores : idx->probe_scores;
    DevBuf &b_probes = lane ? lane->probes : idx->probes, &b_cand = lane ? lane->cand : idx->cand;
    DevBuf &b_tot = lane ? lane->cand_tot : idx->cand_tot, &b_off = lane ? lane->cand_off : idx->cand_off;
    const uint32_t nprobe = ivf_resolve_nprobe(idx);
    const float *qrot = d_q;
    if (idx->quant) {  // pickProbes scores the rotated query
        HIPX(idx->dev, b_qrot.ensure((size_t)nq * idx->P * 4, 0, s), "query buffer");
        EncodeArgs e{};
        e.src = d_q;
        e.rows = nq;
        e.dim = idx->dim;
        e.P = idx->P;
        e.signs = idx->signs.as<float>();
        e.rounds = idx->d.rounds;
        e.bits = 0;
        e.rotated = b_qrot.as<float>();
        HIPX(idx->dev, launch_encode(e, s), "query rotate kernel");
        qrot = b_qrot.as<float>();
    }
    HIPX(idx->dev, b_scores.ensure((size_t)nq * idx->nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, b_probes.ensure((size_t)nq * nprobe * 4, 0, s), "scratch");
    IvfProbeArgs pa{};
    pa.centroids = idx->centroids.as<float>();
    pa.nlist = idx->nlist;
    pa.P = idx->sample_dim;
    pa.qrot = qrot;
    pa.scores = b_scores.as<float>();
    pa.nprobe = nprobe;
    pa.probes = b_probes.as<uint32_t>();
    uint64_t per = 0;
    for (uint32_t i = 0; i < nprobe && i < idx->list_sizes_desc.size(); ++i) per += idx->list_sizes_desc[i];
    HIPX(idx->dev, b_cand.ensure(std::max<uint64_t>(per * nq, 1) * 4, 0, s), "scratch");
    HIPX(idx->dev, b_tot.ensure((size_t)nq * 8, 0, s), "scratch");
    HIPX(idx->dev, b_off.ensure(((size_t)nq + 1) * 8, 0, s), "scratch");
    pa.offset = idx->list_off.as<uint32_t>();
    pa.totals = b_tot.as<uint64_t>();
    pa.cand_off = b_off.as<uint64_t>();
    HIPX(idx->dev, ivf_launch_probes(pa, nq, s), "probe kernels");
    HIPX(idx->dev, ivf_launch_gather(b_probes.as<uint32_t>(), nq, nprobe, idx->list_off.as<uint32_t>(),
                                     idx->list_rows.as<uint32_t>(), b_tot.as<uint64_t>(),
                                     b_off.as<uint64_t>(), b_cand.as<uint32_t>(), s),
         "gather kernels");
    *max_per_query = per;
    return BV_OK;
}

// ---------------------------------------------------------------- queries
// Scanning workgroups per query: at least 256 rows each, and at most
// 2 * CUs - 1 so that the scanning workgroups plus the threshold helper fit
// the device at two workgroups per CU whatever the kernel's register count.
// The fused scan's grid for n rows: one workgroup per 256 rows, at most as
// many as the device holds at once next to the threshold helper (two per
// CU, or one when a workgroup's LDS -- the per-wave lists, which grow with
// the fetch -- leaves room for one only).  The helper is the grid's last
// workgroup: with more workgroups than fit, it would start only after the
// others, the scan would run without its bound, and every wave would flush
// and exactly re-score all of its rows (measured 27 ms instead of 0.2 ms at
// fetch 1024 over 1M rows).
static uint32_t grid_for(const bv_index *idx, uint64_t n, uint32_t kprime, uint32_t rr_dim) {
    uint64_t g = (n + 255) / 256;
    const int cus = idx->dev->prop.multiProcessorCount > 0 ? idx->dev->prop.multiProcessorCount : 128;
    const size_t lds_cu = idx->dev->prop.maxSharedMemoryPerMultiProcessor > 0
                              ? (size_t)idx->dev->prop.maxSharedMemoryPerMultiProcessor
                              : (size_t)160 * 1024;
    const uint32_t wstride = scan_wcap(kprime) + ((rr_dim & ~3u) + 1) / 2 * 2;
    const size_t lds = scan_lds_bytes(idx->codec, idx->P, wstride);
    const uint64_t per_cu = std::max<uint64_t>(1, std::min<uint64_t>(2, lds_cu / std::max<size_t>(lds, 1)));
    uint64_t cap = per_cu * (uint64_t)cus - 1;
    // several query streams on a flat int8 index run the register-lean scan
    // (three workgroups per CU): each query's grid is sized so that every
    // stream's grid and threshold helper are resident at once
    if (idx->query_streams >= 2 && idx->codec == C_Q8 && !idx->ivf && lds * 3 <= lds_cu)
        cap = std::min<uint64_t>(cap, 3ull * (uint64_t)cus / idx->query_streams - 1);
    if (cap > (uint64_t)SCAN_GRID) cap = SCAN_GRID;
    if (g > cap) g = cap;
    if (g < 1) g = 1;
    return (uint32_t)g;
}

// Scratch of the fused scan for nq queries: per-query coordination state,
// per-wave maxima (both must start zeroed; the kernel leaves them zeroed),
// the flushed (scan key, exact key) pairs and the merged keys.  Byte offsets
// from one base, 256-byte aligned.
struct ScanLayout {
    size_t qstate, wmax, cand_keys, merged, merged_n, total;
    uint64_t cap;  // pairs per query
    uint32_t wcap;
    uint32_t pub_m;  // wave maxima published per wave
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static ScanLayout scan_layout(uint32_t nq, uint32_t grid, uint32_t kprime) {
    ScanLayout L{};
    const size_t slots = (size_t)grid * (SCAN_WG / 64);
    const uint64_t ng = grid < (uint32_t)NGROUP ? grid : (uint32_t)NGROUP;
    L.wcap = scan_wcap(kprime);
    L.cap = ng * ((grid + ng - 1) / ng) * (SCAN_WG / 64) * L.wcap;
    L.pub_m = scan_pub_m(kprime, grid);
    L.qstate = 0;
    L.wmax = align256(L.qstate + (size_t)nq * sizeof(QState));
    L.cand_keys = align256(L.wmax + (size_t)nq * slots * L.pub_m * 8);
    L.merged = align256(L.cand_keys + (size_t)nq * L.cap * 16);
    L.merged_n = align256(L.merged + (size_t)nq * kprime * 8);
    L.total = align256(L.merged_n + (size_t)nq * 4);
    return L;
}

static void scan_bind(const ScanLayout &L, char *base, uint32_t rr_dim, ScanArgs &a) {
    a.qs = (QState *)(base + L.qstate);
    a.wmax = (uint64_t *)(base + L.wmax);
    a.pub_m = L.pub_m;
    a.cand_keys = (uint64_t *)(base + L.cand_keys);
    a.cand_cap = L.cap;
    a.wcap = L.wcap;
    a.wstride = L.wcap + ((rr_dim & ~3u) + 1) / 2 * 2;  // list + re-rank staging (doubles)
    a.merged = (uint64_t *)(base + L.merged);
    a.merged_n = (uint32_t *)(base + L.merged_n);
}

static int scan_scratch(bv_index *idx, uint32_t nq, uint32_t grid, uint32_t kprime, uint32_t rr_dim, ScanArgs &a,
                        bv_index::ScanLane *lane = nullptr) {
    const ScanLayout L = scan_layout(nq, grid, kprime);
    DevBuf &qstate = lane ? lane->qstate : idx->qstate, &wmax = lane ? lane->wmax : idx->wmax;
    DevBuf &cand_keys = lane ? lane->cand_keys : idx->cand_keys, &merged = lane ? lane->merged : idx->merged;
    DevBuf &merged_n = lane ? lane->merged_n : idx->merged_n;
    hipStream_t s = lane ? lane->stream : idx->stream;
    {
        const size_t old = qstate.cap;
        HIPX(idx->dev, qstate.ensure((size_t)nq * sizeof(QState), 0, s), "scratch");
        if (qstate.cap != old) HIPX(idx->dev, hipMemsetAsync(qstate.p, 0, qstate.cap, s), "scratch");
    }
    {
        const size_t old = wmax.cap;
        HIPX(idx->dev, wmax.ensure(L.cand_keys - L.wmax, 0, s), "scratch");
        if (wmax.cap != old) HIPX(idx->dev, hipMemsetAsync(wmax.p, 0, wmax.cap, s), "scratch");
    }
    HIPX(idx->dev, cand_keys.ensure((size_t)nq * L.cap * 16, 0, s), "scratch");
    HIPX(idx->dev, merged.ensure((size_t)nq * kprime * 8, 0, s), "scratch");
    HIPX(idx->dev, merged_n.ensure((size_t)nq * 4, 0, s), "scratch");
    a.qs = qstate.as<QState>();
    a.wmax = wmax.as<uint64_t>();
    a.pub_m = L.pub_m;
    a.cand_keys = cand_keys.as<uint64_t>();
    a.cand_cap = L.cap;
    a.wcap = L.wcap;
    a.wstride = L.wcap + ((rr_dim & ~3u) + 1) / 2 * 2;  // list + re-rank staging (doubles)
    a.merged = merged.as<uint64_t>();
    a.merged_n = merged_n.as<uint32_t>();
    return BV_OK;
}

// Work that changes the index's buffers first waits for the second query
// stream's queries (host wait: a buffer may be freed right after), and is
// followed by ev_mut, which the second stream waits on before its next query.
static int lanes_join(bv_index *idx) {
    for (uint32_t i = 0; i < MAX_QUERY_STREAMS - 1; ++i)
        if (idx->lanes_pending & (1u << i)) HIPX(idx->dev, hipStreamSynchronize(idx->lanes[i].stream), "query stream");
    idx->lanes_pending = 0;
    return BV_OK;
}
static int lanes_mark(bv_index *idx) {
    if (!idx->lanes[0].stream) return BV_OK;
    HIPX(idx->dev, hipEventRecord(idx->ev_mut, idx->stream), "event");
    idx->mut_gen++;
    return BV_OK;
}

// Query transform for the scan: device-resident queries d_q (nq x dim) ->
// qscan (per-codec layout), and for quantized kinds qrot (nq x P).
static int prepare_queries(bv_index *idx, const float *d_q, uint32_t nq, const void **qscan, uint64_t *qstride) {
    if (!idx->quant) {
        *qscan = d_q;
        *qstride = (uint64_t)idx->dim * 4;
        return BV_OK;
    }
    const uint32_t P = idx->P;
    HIPX(idx->dev, idx->qrot.ensure((size_t)nq * P * 4, 0, idx->stream), "query buffer");
    EncodeArgs a{};
    a.src = d_q;
    a.rows = nq;
    a.dim = idx->dim;
    a.P = P;
    a.signs = idx->signs.as<float>();
    a.rounds = idx->d.rounds;
    a.rotated = idx->qrot.as<float>();
    switch (idx->codec) {
    case C_Q8:
    case C_Q4: {
        const size_t st = level_stride(idx->codec, P);
        HIPX(idx->dev, idx->qscan.ensure((size_t)nq * st, 0, idx->stream), "query buffer");
        HIPX(idx->dev, launch_encode(a, idx->stream), "query rotate kernel");
        LevelArgs la{};
        la.qrot = idx->qrot.as<float>();
        la.P = P;
        la.codec = idx->codec;
        la.out = idx->qscan.as<unsigned char>();
        la.stride = st;
        HIPX(idx->dev, launch_levels(la, nq, idx->stream), "query levels kernel");
        *qscan = idx->qscan.p;
        *qstride = st;
        return BV_OK;
    }
    case C_Q1A:
        *qscan = idx->qrot.p;
        *qstride = (uint64_t)P * 4;
        break;
    case C_Q1P: {
        const size_t st = level_stride(C_Q1P, P);
        HIPX(idx->dev, idx->qscan.ensure((size_t)nq * st, 0, idx->stream), "query buffer");
        HIPX(idx->dev, launch_encode(a, idx->stream), "query rotate kernel");
        LevelArgs la{};
        la.qrot = idx->qrot.as<float>();
        la.P = P;
        la.codec = C_Q1P;
        la.out = idx->qscan.as<unsigned char>();
        la.stride = st;
        HIPX(idx->dev, launch_q1p_layout(la, nq, idx->stream), "query bit-plane kernel");
        *qscan = idx->qscan.p;
        *qstride = st;
        return BV_OK;
    }
    case C_HAM:
    case C_I8S: {
        const uint32_t per = idx->codec == C_HAM ? 32 : 4;
        const uint32_t W = P / per;
        HIPX(idx->dev, idx->qscan.ensure((size_t)nq * W * 4, 0, idx->stream), "query buffer");
        HIPX(idx->dev, idx->qscale.ensure((size_t)nq * 4, 0, idx->stream), "query buffer");
        a.bits = idx->codec == C_HAM ? 1 : 8;
        a.codes = idx->qscan.as<uint32_t>();
        a.scales = idx->qscale.as<float>();  // the query's own scale is not used by integer scorers
        *qscan = idx->qscan.p;
        *qstride = (uint64_t)W * 4;
        break;
    }
    default:
        return fail(BV_E_STATE, "bad codec");
    }
    HIPX(idx->dev, launch_encode(a, idx->stream), "query rotate kernel");
    return BV_OK;
}

static void timing_begin(bv_index *idx, hipStream_t s = nullptr) {
    if (!idx->timing) return;
    if (idx->tev_used == idx->tev.size()) {
        // Timing-only events: no system-scope fence at the record (its L2
        // write-back would stall the next launch and show up in the timing).
        hipEvent_t a, b;
        if (hipEventCreateWithFlags(&a, hipEventDisableSystemFence) != hipSuccess) return;
        if (hipEventCreateWithFlags(&b, hipEventDisableSystemFence) != hipSuccess) {
            (void)hipEventDestroy(a);
            return;
        }
        idx->tev.push_back({a, b});
    }
    (void)hipEventRecord(idx->tev[idx->tev_used].first, s ? s : idx->stream);
}
static void timing_end(bv_index *idx, hipStream_t s = nullptr) {
    if (!idx->timing || idx->tev_used >= idx->tev.size()) return;
    (void)hipEventRecord(idx->tev[idx->tev_used].second, s ? s : idx->stream);
    idx->tev_used++;
}
static void timing_collect(bv_index *idx) {
    if (idx->tev_used == 0) return;
    (void)hipStreamSynchronize(idx->stream);
    for (auto &l : idx->lanes)
        if (l.stream) (void)hipStreamSynchronize(l.stream);
    for (size_t i = 0; i < idx->tev_used; i++) {
        float ms = 0;
        if (hipEventElapsedTime(&ms, idx->tev[i].first, idx->tev[i].second) == hipSuccess) idx->scan_ms += ms;
        idx->scan_launches++;
    }
    idx->tev_used = 0;
}

// Arguments of the fused scan shared by every caller: the rows / codes, the
// row count or candidate set, the fetch and the outputs.
static void scan_common(const bv_index *idx, const float *d_q, uint64_t n, uint32_t grid, uint32_t kprime,
                        uint32_t k_out, bool rerank, const uint32_t *d_mask, uint64_t mask_bits, uint32_t *d_rows,
                        float *d_scores, uint32_t *d_n, ScanArgs &a) {
    a.codes = idx->quant ? idx->codes.p : idx->raw.p;
    a.row_bytes = idx->row_bytes;
    a.units = idx->units;
    a.padded_dim = idx->P;
    a.scales = (idx->codec == C_Q8 || idx->codec == C_Q4 || idx->codec == C_Q1A || idx->codec == C_Q1P) ? idx->scales.as<float>() : nullptr;
    a.scale_mul = idx->codec == C_Q4 ? 1.0f / 7.0f : 1.0f;
    a.mask = d_mask;
    a.mask_bits = mask_bits;
    a.n = n;
    a.kprime = kprime;
    a.grid = grid;
    a.k_out = k_out;
    a.out_rows = d_rows;
    a.out_scores = d_scores;
    a.out_n = d_n;
    if (rerank) {
        // the scan re-ranks its fetch exactly against the stored fp32 rows
        a.rr_src = idx->raw.as<float>();
        a.rr_dim = idx->dim;
        a.rr_q = d_q;
        a.rr_q_stride = idx->dim;
    }
    // few rows per wave (IVF lists, small corpora): the short tail
    a.short_tail = n < SHORT_TAIL_ROWS * grid * (SCAN_WG / 64);
    a.static_pct = a.short_tail ? SHORT_STATIC_PCT : LONG_STATIC_PCT;
    a.dsteps = a.short_tail ? SHORT_DSTEPS : LONG_DSTEPS;
}

// The fused single-launch scan (one query per grid row): query transform,
// scan, top-kprime and exact re-rank.
static int run_fused(bv_index *idx, const float *d_q, uint32_t nq, uint32_t kprime, uint32_t k_out, bool rerank,
                     const uint32_t *d_mask, uint64_t mask_bits, uint32_t *d_rows, float *d_scores, uint32_t *d_n,
                     bool may_alternate) {
    ScanArgs a{};
    int rc = BV_OK;
    // with two query streams, every other call runs on the second one (its
    // own scan scratch; flat indexes whose scan needs no shared query buffer)
    bv_index::ScanLane *lane = nullptr;
    hipStream_t s = idx->stream;
    if (may_alternate && idx->query_streams >= 2 &&
        (!idx->quant || scan_prep_supported(idx->codec, idx->units, idx->P))) {
        a.lean = 1;  // (both queries' scans: their workgroups share CUs)
        const uint32_t li = idx->next_lane;
        idx->next_lane = (li + 1) % idx->query_streams;
        if (li > 0) {
            lane = &idx->lanes[li - 1];
            s = lane->stream;
            // (the stream is in order: one wait covers every later query on it)
            if (lane->mut_seen != idx->mut_gen) {
                HIPX(idx->dev, hipStreamWaitEvent(s, idx->ev_mut, 0), "event wait");
                lane->mut_seen = idx->mut_gen;
            }
        }
    }
    if (idx->quant && scan_prep_supported(idx->codec, idx->units, idx->P)) {
        // the scan kernel rotates and transforms the fp32 queries itself
        a.qraw = d_q;
        a.qdim = idx->dim;
        a.signs = idx->signs.as<float>();
        a.rounds = idx->d.rounds;
    } else {
        const void *qscan = nullptr;
        uint64_t qstride = 0;
        rc = prepare_queries(idx, d_q, nq, &qscan, &qstride);
        if (rc) return rc;
        a.q = qscan;
        a.q_stride = qstride;
    }
    uint64_t n = idx->rows;
    if (idx->ivf) {  // scan only the probed lists: indexed mode with per-query candidate ranges
        rc = ivf_candidates(idx, d_q, nq, &n, lane);
        if (rc) return rc;
        a.cand = (lane ? lane->cand : idx->cand).as<uint32_t>();
        a.cand_off = (lane ? lane->cand_off : idx->cand_off).as<uint64_t>();
    }
    const uint32_t grid = grid_for(idx, std::max<uint64_t>(n, 1), kprime, rerank ? idx->dim : 0);
    rc = scan_scratch(idx, nq, grid, kprime, rerank ? idx->dim : 0, a, lane);
    if (rc) return rc;
    scan_common(idx, d_q, n, grid, kprime, k_out, rerank, d_mask, mask_bits, d_rows, d_scores, d_n, a);
    timing_begin(idx, s);
    HIPX(idx->dev, launch_scan(idx->codec, idx->units, a, nq, s), "scan kernel");
    timing_end(idx, s);
    if (lane) idx->lanes_pending |= 1u << (uint32_t)(lane - idx->lanes);
    idx->last_scanned = n * nq;
    return BV_OK;
}

// ---------------------------------------------------------- batched scans
// Query batches on an int8 index take the matrix-core path: a dense pass over
// MQ_SAMPLE strided rows gives each query a pruning bound (its kprime-th best
// sample key), a pass over all rows appends the keys at or above it, and the
// best kprime per query go to the exact re-rank or straight to the output.
// Keys are the single-query scan's keys, so results equal the same queries
// run one at a time.  A query whose appended keys overflow their buffer (a
// bound left loose by the sample) is re-run through the fused scan.
constexpr uint32_t MQ_MIN_Q = 8;  // smallest batch for the matrix-core path

static bool mq_eligible(const bv_index *idx, uint32_t nq, const uint32_t *d_mask) {
    if (idx->ivf || d_mask || nq < MQ_MIN_Q || idx->rows == 0) return false;
    // fp32: dot / cosine / l2 above the sample size (smaller corpora: one fused
    // launch for the whole batch is already exact and cheap)
    if (!idx->quant)
        return (idx->codec == C_F32DOT || idx->codec == C_F32L2) && mq_f32_supported(idx->dim) &&
               idx->rows > MQ_SAMPLE;
    const uint32_t u16 = idx->P / 16;  // 16-code units per row
    const bool shape = u16 >= 2 && (u16 % 2) == 0 && u16 / 2 <= MQ_MAX_STEPS;
    // Hamming and 1-bit asymmetric: the first-level pass over +1 / -1 rows,
    // above the sample size
    if (idx->codec == C_HAM || idx->codec == C_Q1P || idx->codec == C_Q1A) return shape && idx->rows > MQ_SAMPLE;
    return (idx->codec == C_Q8 || idx->codec == C_Q4) && shape;
}

// Rotated queries split into three int8 levels in the 16-code unit layout
// the batched scan reads (int4 indexes: levels without the 1/127 scale).
static int prepare_levels16(bv_index *idx, const float *d_q, uint32_t nq, const unsigned char **qlev,
                            uint64_t *qstride, int layout = -1) {
    const uint32_t P = idx->P;
    if (layout < 0) layout = idx->codec == C_Q4 ? C_Q4M : C_Q8;
    const size_t st = level_stride(layout, P);
    HIPX(idx->dev, idx->qrot.ensure((size_t)nq * P * 4, 0, idx->stream), "query buffer");
    HIPX(idx->dev, idx->qscan.ensure((size_t)nq * st, 0, idx->stream), "query buffer");
    EncodeArgs e{};
    e.src = d_q;
    e.rows = nq;
    e.dim = idx->dim;
    e.P = P;
    e.signs = idx->signs.as<float>();
    e.rounds = idx->d.rounds;
    e.rotated = idx->qrot.as<float>();
    HIPX(idx->dev, launch_encode(e, idx->stream), "query rotate kernel");
    LevelArgs la{};
    la.qrot = idx->qrot.as<float>();
    la.P = P;
    la.codec = layout;
    la.out = idx->qscan.as<unsigned char>();
    la.stride = st;
    HIPX(idx->dev, launch_levels(la, nq, idx->stream), "query levels kernel");
    *qlev = idx->qscan.as<unsigned char>();
    *qstride = st;
    return BV_OK;
}

// Workgroups per (XCD, query block) of the persistent batched scan: about
// one workgroup per CU over the whole grid.
static uint32_t mq_groups(const bv_index *idx, uint32_t qblocks) {
    const int cus = idx->dev->prop.multiProcessorCount > 0 ? idx->dev->prop.multiProcessorCount : 256;
    const uint32_t g = (uint32_t)cus / (8u * qblocks);
    return g ? g : 1u;
}

// fp32 batches, exactly equal to single queries.  The matrix-core scan is a
// prefilter: a dense pass over MQ_SAMPLE strided rows gives each query a
// bound (its kprime-th best sample score), a pass over every row keeps the
// ids of the rows whose matrix-core score reaches the bound minus the
// slack 2E (E bounds the difference between a matrix-core score and the
// single-query scan's), and the fused scan re-scores exactly those rows in
// indexed mode with the single-query arithmetic and selects the top-k of the
// same keys.  A query whose kept rows overflow their buffer runs the fused
// scan over every row.
static int run_batched_f32(bv_index *idx, const float *d_q, uint32_t nq, uint32_t kprime, uint32_t k_out,
                           uint32_t *d_rows, float *d_scores, uint32_t *d_n) {
    const uint64_t N = idx->rows, S = MQ_SAMPLE;  // N > S (mq_eligible)
    const bool l2 = idx->codec == C_F32L2;
    uint64_t cap = std::max<uint64_t>(S, 4ull * kprime * ((N + S - 1) / S));
    cap = std::min<uint64_t>(cap, N);
    hipStream_t s = idx->stream;
    HIPX(idx->dev, idx->mq_cand.ensure((size_t)nq * std::max<uint64_t>(cap, S) * 8, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_rows.ensure((size_t)nq * cap * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_cnt.ensure((size_t)nq * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_tau.ensure((size_t)nq * 8, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_qsq.ensure((size_t)nq * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_slack.ensure((size_t)nq * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->h_cnt.ensure((size_t)nq * 4), "pinned buffer");

    timing_begin(idx);
    HIPX(idx->dev,
         launch_mq_f32_qconst(d_q, nq, idx->dim, idx->rsq_max.as<uint32_t>(), l2 ? 1 : 0, idx->mq_qsq.as<float>(),
                              idx->mq_slack.as<float>(), s),
         "query norm kernel");
    MqArgs m{};
    m.codes = idx->raw.as<uint32_t>();
    m.W = idx->dim;
    m.units = idx->dim / 8;
    m.qlev = (const unsigned char *)d_q;
    m.qstride = (uint64_t)idx->dim * 4;
    m.nq = nq;
    m.qblocks = (nq + MQ_QB - 1) / MQ_QB;
    m.groups = mq_groups(idx, m.qblocks);
    m.cand = idx->mq_cand.as<uint64_t>();
    m.cnt = idx->mq_cnt.as<uint32_t>();
    m.cap = std::max<uint64_t>(cap, S);
    m.l2 = l2 ? 1 : 0;
    m.rsq = idx->rsq.as<float>();
    m.qsq = idx->mq_qsq.as<float>();
    m.slack = idx->mq_slack.as<float>();
    // sample pass: every (approximate) key of logical rows i < S
    m.n = S;
    m.row_step = N / S;
    HIPX(idx->dev, hipMemsetD32Async((hipDeviceptr_t)idx->mq_cnt.p, (int)S, nq, s), "scratch");
    HIPX(idx->dev, launch_mq_scan_f32(m, s), "batched scan kernel");
    MqSelArgs sa{};
    sa.cand = m.cand;
    sa.cnt = m.cnt;
    sa.cap = m.cap;
    sa.kk = kprime;
    sa.tau = idx->mq_tau.as<uint64_t>();
    HIPX(idx->dev, launch_mq_select(sa, nq, s), "batched select kernel");
    // full pass: ids of every row that can rank
    HIPX(idx->dev, hipMemsetAsync(idx->mq_cnt.p, 0, (size_t)nq * 4, s), "scratch");
    m.n = N;
    m.row_step = 1;
    m.tau = idx->mq_tau.as<uint64_t>();
    m.cap = cap;
    m.rows_out = idx->mq_rows.as<uint32_t>();
    HIPX(idx->dev, launch_mq_scan_f32(m, s), "batched scan kernel");
    HIPX(idx->dev, hipMemcpyAsync(idx->h_cnt.p, idx->mq_cnt.p, (size_t)nq * 4, hipMemcpyDeviceToHost, s),
         "count download");
    HIPX(idx->dev, hipStreamSynchronize(s), "batched scan");
    const uint32_t *cnt = (const uint32_t *)idx->h_cnt.p;
    uint64_t most = 1;
    for (uint32_t i = 0; i < nq; i++) most = std::max<uint64_t>(most, std::min<uint64_t>(cnt[i], cap));
    // exact re-score of the kept rows: the fused scan in indexed mode
    ScanArgs a{};
    const uint32_t grid = grid_for(idx, most, kprime, 0);
    int rc = scan_scratch(idx, nq, grid, kprime, 0, a);
    if (rc) return rc;
    a.codes = idx->raw.p;
    a.row_bytes = idx->row_bytes;
    a.units = idx->units;
    a.padded_dim = idx->P;
    a.scale_mul = 1.0f;
    a.q = d_q;
    a.q_stride = (uint64_t)idx->dim * 4;
    a.cand = idx->mq_rows.as<uint32_t>();
    a.cand_n = idx->mq_cnt.as<uint32_t>();
    a.cand_stride = cap;
    a.n = cap;
    a.kprime = kprime;
    a.grid = grid;
    a.k_out = k_out;
    a.out_rows = d_rows;
    a.out_scores = d_scores;
    a.out_n = d_n;
    HIPX(idx->dev, launch_scan(idx->codec, idx->units, a, nq, s), "scan kernel");
    timing_end(idx);
    uint64_t scanned = N + S;
    for (uint32_t i = 0; i < nq; i++) scanned += std::min<uint64_t>(cnt[i], cap);
    idx->last_scanned = scanned;
    // queries whose kept rows overflowed: the fused scan over every row
    std::vector<uint32_t> over;
    for (uint32_t i = 0; i < nq; i++)
        if (cnt[i] > cap) over.push_back(i);
    for (uint32_t i : over) {
        rc = run_fused(idx, d_q + (size_t)i * idx->dim, 1, kprime, k_out, false, nullptr, 0,
                       d_rows + (size_t)i * k_out, d_scores + (size_t)i * k_out, d_n + i);
        if (rc) return rc;
    }
    return BV_OK;
}

// int8 batches above the sample size, exactly equal to single queries.  The
// matrix cores score every (row, query) on the query's first int8 level
// alone (mq1_scan), which reads each code from HBM once per 256 queries and
// does a third of the three-level work; the other two levels enter as a
// bound, |c|_2 |R|_2 times the row scale.  A dense pass over MQ_SAMPLE
// strided rows gives each query its kprime-th best lower-bound key (kprime
// rows have exact keys at or above it); the pass over every row keeps the
// rows whose upper bound reaches it, with their bounds (in two parts, the
// second under the bound the first part's rows give); the kprime-th best
// lower bound among those is a tighter bound, and only the rows whose upper
// bound reaches it can be in the top kprime.  Those rows get their exact
// keys with the single-query arithmetic (three exact level dots, f64
// combine), and the best kprime of them are selected and re-ranked as a
// single query's are.
// A query whose kept rows overflow their buffer runs the fused scan over
// every row.
// The codes the first-level pass reads: the index's int8 codes, or for a
// Hamming index the +1 / -1 expansion of its 1-bit codes (unit scales), whose
// int8 dots are the Hamming similarities.
struct Q8Source {
    const uint32_t *codes;
    uint32_t W;
    const float *scales, *cn;
};

// Hamming batches: the +1 / -1 rows (kept up to date with appends) and the
// queries' 1-bit codes as level one of the packed levels.
// The codes of a 1-bit or int4 index as int8 bytes (1 byte per code), kept
// current with the index's rows, for the first-level pass: 1-bit codes as
// +1 / -1 with unit row multipliers, int4 codes as their signed values with
// the multipliers f32(scale * f32(1/7)); and the rows' code norms.
static int ensure_pm_rows(bv_index *idx) {
    hipStream_t s = idx->stream;
    const uint32_t P = idx->P, W1 = idx->words_per_row;
    if (idx->pm_rows < idx->rows) {
        const uint64_t n0 = idx->pm_rows, n = idx->rows;
        HIPX(idx->dev, idx->pm_codes.ensure(n * P, n0 * P, s), "expanded code buffer");
        HIPX(idx->dev, idx->pm_ones.ensure(n * 4, n0 * 4, s), "scale buffer");
        HIPX(idx->dev, idx->pm_cn.ensure(n * 4, n0 * 4, s), "norm buffer");
        if (idx->codec == C_Q4) {
            HIPX(idx->dev,
                 launch_expand_q4(idx->codes.as<uint32_t>() + n0 * W1, (n - n0) * W1,
                                  idx->pm_codes.as<uint32_t>() + n0 * (P / 4), s),
                 "expand kernel");
            HIPX(idx->dev,
                 launch_scale_mul(idx->scales.as<float>() + n0, n - n0, 1.0f / 7.0f, idx->pm_ones.as<float>() + n0, s),
                 "scale kernel");
        } else {
            HIPX(idx->dev,
                 launch_expand_pm(idx->codes.as<uint32_t>() + n0 * W1, (n - n0) * W1,
                                  idx->pm_codes.as<uint32_t>() + n0 * (P / 4), s),
                 "expand kernel");
            HIPX(idx->dev, launch_fill_f32(idx->pm_ones.as<float>() + n0, n - n0, 1.0f, s), "fill kernel");
        }
        HIPX(idx->dev,
             launch_row_code_norms(idx->pm_codes.as<uint32_t>() + n0 * (P / 4), n - n0, P / 4,
                                   idx->pm_cn.as<float>() + n0, s),
             "norm kernel");
        idx->pm_rows = n;
    }
    return BV_OK;
}

static int prepare_pm(bv_index *idx, const float *d_q, uint32_t nq, const unsigned char **qlev, uint64_t *qstride,
                      Q8Source *src, bool widen_rows = true) {
    hipStream_t s = idx->stream;
    const uint32_t P = idx->P, W1 = idx->words_per_row;
    if (widen_rows) {
        const int rc = ensure_pm_rows(idx);
        if (rc) return rc;
    }
    const size_t st = level_stride(C_Q8, P);
    HIPX(idx->dev, idx->pm_qbits.ensure((size_t)nq * W1 * 4, 0, s), "query buffer");
    HIPX(idx->dev, idx->qscale.ensure((size_t)nq * 4, 0, s), "query buffer");
    HIPX(idx->dev, idx->qscan.ensure((size_t)nq * st, 0, s), "query buffer");
    EncodeArgs e{};
    e.src = d_q;
    e.rows = nq;
    e.dim = idx->dim;
    e.P = P;
    e.signs = idx->signs.as<float>();
    e.rounds = idx->d.rounds;
    e.bits = 1;  // the queries' bits, as the single-query Hamming scan takes them
    e.codes = idx->pm_qbits.as<uint32_t>();
    e.scales = idx->qscale.as<float>();
    HIPX(idx->dev, launch_encode(e, s), "query encode kernel");
    HIPX(idx->dev, launch_pm_levels(idx->pm_qbits.as<uint32_t>(), nq, P, idx->qscan.as<unsigned char>(), st, s),
         "query levels kernel");
    *qlev = idx->qscan.as<unsigned char>();
    *qstride = st;
    if (widen_rows) *src = Q8Source{idx->pm_codes.as<uint32_t>(), P / 4, idx->pm_ones.as<float>(), idx->pm_cn.as<float>()};
    return BV_OK;
}

// The last step of a batch whose prefilter kept, per query, a superset of
// the rows that can reach its top kprime (mq_rows, counts in mq_kept, cap
// apart; a query whose joined list overflowed, mq_cnt[q] > cap, kept none):
// the fused scan in indexed mode over the kept rows computes their
// single-query keys, selects and re-ranks, so every query returns what it
// returns alone.  Overflowed queries are re-run alone over every row.
static int finish_batched_indexed(bv_index *idx, const float *d_q, uint32_t nq, uint32_t kprime, uint32_t k_out,
                                  bool rerank, uint64_t cap, uint32_t *d_rows, float *d_scores, uint32_t *d_n) {
    hipStream_t s = idx->stream;
    uint32_t *h = (uint32_t *)idx->h_cnt.p;  // [nq] kept, then [nq] joined counts
    HIPX(idx->dev, hipMemcpyAsync(h, idx->mq_kept.p, (size_t)nq * 4, hipMemcpyDeviceToHost, s), "count download");
    HIPX(idx->dev, hipMemcpyAsync(h + nq, idx->mq_cnt.p, (size_t)nq * 4, hipMemcpyDeviceToHost, s), "count download");
    HIPX(idx->dev, hipStreamSynchronize(s), "batched scan");
    std::vector<uint32_t> kept(h, h + nq), joined(h + nq, h + 2 * (size_t)nq);
    uint64_t most = 1;
    for (uint32_t i = 0; i < nq; i++) most = std::max<uint64_t>(most, std::min<uint64_t>(kept[i], cap));
    ScanArgs a{};
    const uint32_t grid = grid_for(idx, most, kprime, rerank ? idx->dim : 0);
    int rc = scan_scratch(idx, nq, grid, kprime, rerank ? idx->dim : 0, a);
    if (rc) return rc;
    if (scan_prep_supported(idx->codec, idx->units, idx->P)) {  // the scan transforms the fp32 queries itself
        a.qraw = d_q;
        a.qdim = idx->dim;
        a.signs = idx->signs.as<float>();
        a.rounds = idx->d.rounds;
    } else {
        const void *qscan = nullptr;
        uint64_t qstride = 0;
        rc = prepare_queries(idx, d_q, nq, &qscan, &qstride);
        if (rc) return rc;
        a.q = qscan;
        a.q_stride = qstride;
    }
    scan_common(idx, d_q, most, grid, kprime, k_out, rerank, nullptr, 0, d_rows, d_scores, d_n, a);
    a.cand = idx->mq_rows.as<uint32_t>();
    a.cand_n = idx->mq_kept.as<uint32_t>();
    a.cand_stride = cap;
    HIPX(idx->dev, launch_scan(idx->codec, idx->units, a, nq, s), "scan kernel");
    timing_end(idx);
    uint64_t scanned = (idx->rows + MQ_SAMPLE) * nq;
    for (uint32_t i = 0; i < nq; i++) scanned += std::min<uint64_t>(kept[i], cap);
    idx->last_scanned = scanned;
    for (uint32_t i = 0; i < nq; i++) {
        if (joined[i] <= cap) continue;
        rc = run_fused(idx, d_q + (size_t)i * idx->dim, 1, kprime, k_out, rerank, nullptr, 0,
                       d_rows + (size_t)i * k_out, d_scores + (size_t)i * k_out, d_n + i);
        if (rc) return rc;
    }
    return BV_OK;
}

static int run_batched_q8(bv_index *idx, const float *d_q, uint32_t nq, uint32_t kprime, uint32_t k_out,
                          bool rerank, uint32_t *d_rows, float *d_scores, uint32_t *d_n) {
    const unsigned char *qlev = nullptr;
    uint64_t qstride = 0;
    Q8Source src{idx->codes.as<uint32_t>(), idx->words_per_row, idx->scales.as<float>(), idx->cnorm.as<float>()};
    // 1-bit asymmetric: the pass over the +1 / -1 expansion with the rotated
    // query's int8 level one (levels without the 1/127), the rows' own
    // scales and row term 1 (mq1_qconst_l1); the kept rows get the
    // single-query keys from q1p_exact_rows (bit-plane codes), or from the
    // fused scan in indexed mode (C_Q1A)
    const bool asym1 = idx->codec == C_Q1P || idx->codec == C_Q1A;
    // Hamming and bit-plane 1-bit codes of 128 to 1024 codes per row: the
    // pass reads the bits and widens them to +1 / -1 bytes in LDS
    // (mq1_scan_bits), so the index keeps no widened copy; every such row has
    // the code norm sqrt(P) (Hamming, rounded up as row_code_norms rounds) or
    // the row term 1 (asymmetric)
    const bool bits1 = (idx->codec == C_HAM || idx->codec == C_Q1P) && idx->P >= 128 && idx->P <= 1024;
    float cn_const = 1.0f;
    int rc = BV_OK;
    if (bits1 && idx->codec == C_HAM) {
        rc = prepare_pm(idx, d_q, nq, &qlev, &qstride, &src, false);
        src = Q8Source{idx->codes.as<uint32_t>(), idx->words_per_row, nullptr, nullptr};
        const double v = std::sqrt((double)idx->P);
        cn_const = (float)v;
        if ((double)cn_const < v) cn_const = std::nextafter(cn_const, INFINITY);
    } else if (bits1) {
        rc = prepare_levels16(idx, d_q, nq, &qlev, &qstride, C_Q4M);
        src = Q8Source{idx->codes.as<uint32_t>(), idx->words_per_row, idx->scales.as<float>(), nullptr};
    } else if (idx->codec == C_HAM) {
        rc = prepare_pm(idx, d_q, nq, &qlev, &qstride, &src);
    } else if (asym1) {
        rc = ensure_pm_rows(idx);
        if (!rc) rc = prepare_levels16(idx, d_q, nq, &qlev, &qstride, C_Q4M);
        src = Q8Source{idx->pm_codes.as<uint32_t>(), idx->P / 4, idx->scales.as<float>(), idx->pm_ones.as<float>()};
    } else if (idx->codec == C_Q4) {
        // int4: the pass over the codes' signed bytes with the query's int8
        // levels without the 1/127 (C_Q4M), the rows' multipliers
        // f32(scale * f32(1/7)) and code norms.  The exact step below then
        // forms the single-query int4 key: the byte dots are the nibble dots
        // the int4 scan recovers, combined with the same level steps.
        rc = ensure_pm_rows(idx);
        if (!rc) rc = prepare_levels16(idx, d_q, nq, &qlev, &qstride, C_Q4M);
        src = Q8Source{idx->pm_codes.as<uint32_t>(), idx->P / 4, idx->pm_ones.as<float>(), idx->pm_cn.as<float>()};
    } else {
        rc = prepare_levels16(idx, d_q, nq, &qlev, &qstride);
    }
    if (rc) return rc;
    const uint64_t N = idx->rows, S = MQ_SAMPLE;  // N > S (mq_eligible)
    // rows kept per query: those within the bounds' width of the sample's
    // bound, about 2-4x the kprime * N / S above it; room for 16x that
    uint64_t cap = std::max<uint64_t>(4 * S, 16ull * kprime * ((N + S - 1) / S));
    cap = std::min<uint64_t>(cap, N);
    hipStream_t s = idx->stream;
    const uint32_t qblocks = (nq + MQ1_QB - 1) / MQ1_QB;
    const int cus = idx->dev->prop.multiProcessorCount > 0 ? idx->dev->prop.multiProcessorCount : 256;
    const uint32_t nwg = std::min<uint32_t>(1024, std::max<uint32_t>(1, (uint32_t)cus / qblocks));
    // each workgroup's bucket of a query: room for cap / nwg entries (the
    // workgroups see evenly spread rows), at least 128
    const uint32_t capw = (uint32_t)((std::max<uint64_t>(128, (cap + nwg - 1) / nwg) + 15) & ~15ull);
    HIPX(idx->dev, idx->mq_cand.ensure((size_t)nq * std::max<uint64_t>(cap, S) * 8, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_up.ensure((size_t)nq * cap * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_bk.ensure((size_t)nq * nwg * capw * 8, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_bu.ensure((size_t)nq * nwg * capw * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_bc.ensure((size_t)nq * nwg * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_rows.ensure((size_t)nq * cap * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_cnt.ensure((size_t)nq * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_kept.ensure((size_t)nq * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_tau.ensure((size_t)nq * 8, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_tau2.ensure((size_t)nq * 8, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_rq.ensure((size_t)nq * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->h_cnt.ensure((size_t)nq * 8), "pinned buffer");
    HIPX(idx->dev, idx->merged.ensure((size_t)nq * kprime * 8, 0, s), "scratch");
    HIPX(idx->dev, idx->merged_n.ensure((size_t)nq * 4, 0, s), "scratch");
    const uint32_t units16 = idx->P / 16;

    timing_begin(idx);
    // the query bounds, and the sample pass's key count per query
    if (asym1)
        HIPX(idx->dev,
             launch_mq1_qconst_l1(idx->qrot.as<float>(), idx->P, qlev, qstride, units16 * 48, nq,
                                  idx->mq_rq.as<float>(), idx->mq_cnt.as<uint32_t>(), (uint32_t)S, s),
             "query bound kernel");
    else
        HIPX(idx->dev,
             launch_mq1_qconst(qlev, qstride, units16, units16 * 48, nq, idx->mq_rq.as<float>(),
                               idx->mq_cnt.as<uint32_t>(), (uint32_t)S, s),
             "query bound kernel");
    Mq1Args m{};
    m.codes = src.codes;
    m.scales = src.scales;
    m.cn = src.cn;
    m.W = src.W;
    m.cn_const = cn_const;
    auto scan = [&]() { return bits1 ? launch_mq1_scan_bits(m, s) : launch_mq1_scan(m, s); };
    m.units = units16;
    m.qlev = qlev;
    m.qstride = qstride;
    m.tail_off = units16 * 48;
    m.rq = idx->mq_rq.as<float>();
    m.nq = nq;
    m.qblocks = qblocks;
    m.groups = nwg;
    m.nwg = nwg;
    // sample pass: the lower-bound key of every logical row i < S
    m.n = S;
    m.row_step = N / S;
    m.cand = idx->mq_cand.as<uint64_t>();
    m.cap = S;
    HIPX(idx->dev, scan(), "batched scan kernel");
    MqSelArgs sa{};
    sa.cand = m.cand;
    sa.cnt = idx->mq_cnt.as<uint32_t>();
    sa.cap = S;
    sa.kk = kprime;
    sa.tau = idx->mq_tau.as<uint64_t>();
    // each bound is then raised to the smallest exact key of the kprime rows
    // that reach it (the kprime-th best exact key of all rows is at least
    // that), which narrows the rows the passes keep.  Hamming bounds are
    // exact already (one level, no residual); the 1-bit asymmetric keys
    // without bit planes (C_Q1A) are left to the fused scan.
    const bool q1p = idx->codec == C_Q1P;
    const bool exact_tau = (!asym1 || q1p) && idx->codec != C_HAM && kprime <= 2048;
    // the bit-plane scan's exact keys come from its re-score table over the
    // rotated queries and its own codes
    Q1pRowsArgs qa{};
    qa.codes = idx->codes.p;
    qa.row_bytes = idx->row_bytes;
    qa.units = idx->units;
    qa.P = idx->P;
    qa.scales = idx->scales.as<float>();
    qa.scale_mul = 1.0f;
    qa.qrot = idx->qrot.as<float>();
    qa.nrows = idx->rows;
    // the select writes the list's kprime best lower-bound keys, in order, to
    // merged (free until the final select), and their exact keys raise tau
    auto tighten = [&]() {
        if (q1p)
            return launch_q1p_tau_exact(qa, idx->merged.as<uint64_t>(), idx->merged_n.as<uint32_t>(), kprime,
                                        idx->mq_tau.as<uint64_t>(), nq, s);
        return launch_mq1_tau_exact(src.codes, src.W, src.scales, qlev, qstride, units16, idx->merged.as<uint64_t>(),
                                    idx->merged_n.as<uint32_t>(), kprime, idx->rows, idx->mq_tau.as<uint64_t>(), nq,
                                    s);
    };
    auto select_bound = [&](uint64_t ccap, uint64_t *tau_out) {
        sa.cap = ccap;
        sa.tau = tau_out;
        sa.merged = idx->merged.as<uint64_t>();
        sa.merged_n = idx->merged_n.as<uint32_t>();
        const hipError_t e = launch_mq_select(sa, nq, s);
        sa.merged = nullptr;
        sa.merged_n = nullptr;
        return e;
    };
    if (exact_tau) {
        HIPX(idx->dev, select_bound(S, idx->mq_tau.as<uint64_t>()), "batched select kernel");
        HIPX(idx->dev, tighten(), "batched bound kernel");
    } else {
        HIPX(idx->dev, launch_mq_select(sa, nq, s), "batched select kernel");
    }
    // the pass over every row keeps the rows whose upper bound reaches the
    // bound, into the workgroups' buckets, then one list per query.  It runs
    // in two parts: the first eighth of the rows, whose kept rows' kprime-th
    // best lower bound (a bound for the same reason) is far tighter than the
    // sample's, then the rest under the tighter of the two
    const uint64_t NA = std::max<uint64_t>(MQ1_ROWS, N / 8 / MQ1_ROWS * MQ1_ROWS);
    m.tau = idx->mq_tau.as<uint64_t>();
    m.up_out = idx->mq_bu.as<uint32_t>();
    m.cnt = idx->mq_bc.as<uint32_t>();
    m.cap = cap;
    m.capw = capw;
    m.row_step = 1;
    for (int part = 0; part < 2; ++part) {
        const uint64_t r0 = part ? NA : 0, rn = part ? N - NA : NA;
        if (rn == 0) break;
        m.n = rn;
        m.row_base = r0;
        m.codes = src.codes + r0 * src.W;
        m.scales = src.scales ? src.scales + r0 : nullptr;
        m.cn = src.cn ? src.cn + r0 : nullptr;
        m.cand = idx->mq_bk.as<uint64_t>();
        HIPX(idx->dev, scan(), "batched scan kernel");
        HIPX(idx->dev,
             launch_mq1_compact(idx->mq_bk.as<uint64_t>(), idx->mq_bu.as<uint32_t>(), idx->mq_bc.as<uint32_t>(),
                                nwg, capw, cap, idx->mq_cand.as<uint64_t>(), idx->mq_up.as<uint32_t>(),
                                idx->mq_cnt.as<uint32_t>(), part > 0, nq, s),
             "batched compact kernel");
        if (part == 0) {  // the tighter bound
            sa.cap = cap;
            if (exact_tau) {
                HIPX(idx->dev, select_bound(cap, idx->mq_tau2.as<uint64_t>()), "batched select kernel");
                HIPX(idx->dev, tighten(), "batched bound kernel");
                sa.tau = idx->mq_tau.as<uint64_t>();
            } else {
                sa.tau_max = true;
                HIPX(idx->dev, launch_mq_select(sa, nq, s), "batched select kernel");
                sa.tau_max = false;
            }
        }
    }
    m.codes = src.codes;
    m.scales = src.scales;
    m.cand = idx->mq_cand.as<uint64_t>();
    m.up_out = idx->mq_up.as<uint32_t>();
    m.cnt = idx->mq_cnt.as<uint32_t>();
    // the kprime-th best lower bound among the kept rows (raised as above),
    // and the rows whose upper bound reaches it
    sa.cap = cap;
    if (exact_tau) {
        HIPX(idx->dev, select_bound(cap, idx->mq_tau2.as<uint64_t>()), "batched select kernel");
        HIPX(idx->dev, tighten(), "batched bound kernel");
    } else {
        HIPX(idx->dev, launch_mq_select(sa, nq, s), "batched select kernel");
    }
    HIPX(idx->dev,
         launch_mq1_keep(m.cand, m.up_out, m.cnt, cap, idx->mq_tau.as<uint64_t>(), idx->mq_rows.as<uint32_t>(),
                         idx->mq_kept.as<uint32_t>(), nq, s),
         "batched keep kernel");
    if (asym1 && idx->codec != C_Q1P)
        return finish_batched_indexed(idx, d_q, nq, kprime, k_out, rerank, cap, d_rows, d_scores, d_n);
    // exact keys of those rows, the best kprime of them, and the re-rank
    if (asym1) {
        qa.rows = idx->mq_rows.as<uint32_t>();
        qa.kept = idx->mq_kept.as<uint32_t>();
        qa.cap = cap;
        qa.keys = m.cand;
        HIPX(idx->dev, launch_q1p_exact_rows(qa, nq, 8, s), "batched exact kernel");
    } else if (bits1) {  // Hamming over the bits
        HIPX(idx->dev,
             launch_ham_exact(src.codes, src.W, idx->pm_qbits.as<uint32_t>(), qlev, qstride, units16 * 48,
                              idx->mq_rows.as<uint32_t>(), idx->mq_kept.as<uint32_t>(), cap, m.cand, nq, s),
             "batched exact kernel");
    } else {
        HIPX(idx->dev,
             launch_mq1_exact(m.codes, m.W, m.scales, qlev, qstride, units16, idx->mq_rows.as<uint32_t>(),
                              idx->mq_kept.as<uint32_t>(), cap, m.cand, nq, s),
             "batched exact kernel");
    }
    MqSelArgs fa{};
    fa.cand = m.cand;
    fa.cnt = idx->mq_kept.as<uint32_t>();
    fa.cap = cap;
    fa.kk = kprime;
    fa.merged = idx->merged.as<uint64_t>();
    fa.merged_n = idx->merged_n.as<uint32_t>();
    if (!rerank) {
        fa.k_out = k_out;
        fa.out_rows = d_rows;
        fa.out_scores = d_scores;
        fa.out_n = d_n;
    }
    HIPX(idx->dev, launch_mq_select(fa, nq, s), "batched select kernel");
    if (rerank) {
        MqRerankArgs r{};
        r.rows = idx->raw.as<float>();
        r.dim = idx->dim;
        r.q = d_q;
        r.q_stride = idx->dim;
        r.merged = idx->merged.as<uint64_t>();
        r.merged_n = idx->merged_n.as<uint32_t>();
        r.kprime = kprime;
        r.k_out = k_out;
        r.out_rows = d_rows;
        r.out_scores = d_scores;
        r.out_n = d_n;
        HIPX(idx->dev, launch_mq_rerank(r, nq, s), "rerank kernel");
    }
    timing_end(idx);
    HIPX(idx->dev, hipMemcpyAsync(idx->h_cnt.p, idx->mq_cnt.p, (size_t)nq * 4, hipMemcpyDeviceToHost, s),
         "count download");
    HIPX(idx->dev, hipStreamSynchronize(s), "batched scan");
    const uint32_t *cnt = (const uint32_t *)idx->h_cnt.p;
    idx->last_scanned = (N + S) * nq;
    // queries whose kept rows overflowed their buffer: the fused scan over every row
    std::vector<uint32_t> over;
    for (uint32_t i = 0; i < nq; i++)
        if (cnt[i] > cap) over.push_back(i);
    for (uint32_t i : over) {
        rc = run_fused(idx, d_q + (size_t)i * idx->dim, 1, kprime, k_out, rerank, nullptr, 0,
                       d_rows + (size_t)i * k_out, d_scores + (size_t)i * k_out, d_n + i);
        if (rc) return rc;
    }
    return BV_OK;
}

static int run_batched(bv_index *idx, const float *d_q, uint32_t nq, uint32_t kprime, uint32_t k_out, bool rerank,
                       uint32_t *d_rows, float *d_scores, uint32_t *d_n) {
    if (!idx->quant) return run_batched_f32(idx, d_q, nq, kprime, k_out, d_rows, d_scores, d_n);
    if ((idx->codec == C_Q8 || idx->codec == C_Q4 || idx->codec == C_HAM || idx->codec == C_Q1P ||
         idx->codec == C_Q1A) &&
        idx->rows > MQ_SAMPLE)
        return run_batched_q8(idx, d_q, nq, kprime, k_out, rerank, d_rows, d_scores, d_n);
    const unsigned char *qscan = (const unsigned char *)d_q;  // fp32 rows: the queries as they are
    uint64_t qstride = (uint64_t)idx->dim * 4;
    int rc = BV_OK;
    if (idx->quant) {
        rc = prepare_levels16(idx, d_q, nq, &qscan, &qstride);
        if (rc) return rc;
    }
    const uint64_t N = idx->rows;
    const uint64_t S = std::min<uint64_t>(N, MQ_SAMPLE);
    const bool one_pass = S == N;
    // appended keys expected per query: about kprime * N / S; room for 4x that
    uint64_t cap = one_pass ? N : std::max<uint64_t>(S, 4ull * kprime * ((N + S - 1) / S));
    cap = std::min<uint64_t>(cap, N);
    HIPX(idx->dev, idx->mq_cand.ensure((size_t)nq * cap * 8, 0, idx->stream), "scratch");
    HIPX(idx->dev, idx->mq_cnt.ensure((size_t)nq * 4, 0, idx->stream), "scratch");
    HIPX(idx->dev, idx->mq_tau.ensure((size_t)nq * 8, 0, idx->stream), "scratch");
    HIPX(idx->dev, idx->mq_flag.ensure((size_t)nq * 4, 0, idx->stream), "scratch");
    HIPX(idx->dev, idx->merged.ensure((size_t)nq * kprime * 8, 0, idx->stream), "scratch");
    HIPX(idx->dev, idx->merged_n.ensure((size_t)nq * 4, 0, idx->stream), "scratch");

    MqArgs m{};
    m.codes = idx->quant ? idx->codes.as<uint32_t>() : idx->raw.as<uint32_t>();
    m.scales = idx->scales.as<float>();
    m.W = idx->quant ? idx->words_per_row : idx->dim;
    m.units = idx->quant ? idx->P / 16 : idx->dim / 8;
    m.bits = idx->codec == C_Q4 ? 4 : 8;
    m.scale_mul = idx->codec == C_Q4 ? 1.0f / 7.0f : 1.0f;
    m.qlev = qscan;
    m.qstride = qstride;
    m.tail_off = m.units * 48;  // 12 words per 16-code unit, then QLevelTail
    m.nq = nq;
    m.qblocks = (nq + MQ_QB - 1) / MQ_QB;
    m.groups = mq_groups(idx, m.qblocks);
    m.cand = idx->mq_cand.as<uint64_t>();
    m.cnt = idx->mq_cnt.as<uint32_t>();
    m.cap = cap;
    MqSelArgs sa{};
    sa.cand = m.cand;
    sa.cnt = m.cnt;
    sa.cap = cap;
    sa.kk = kprime;

    timing_begin(idx);
    // sample pass: every key of logical rows i < S (physical row i * N/S)
    m.n = S;
    m.row_step = N / S;
    m.tau = nullptr;
    HIPX(idx->dev, hipMemsetD32Async((hipDeviceptr_t)idx->mq_cnt.p, (int)S, nq, idx->stream), "scratch");
    HIPX(idx->dev, idx->quant ? launch_mq_scan(m, idx->stream) : launch_mq_scan_f32(m, idx->stream),
         "batched scan kernel");
    if (!one_pass) {
        sa.tau = idx->mq_tau.as<uint64_t>();
        HIPX(idx->dev, launch_mq_select(sa, nq, idx->stream), "batched select kernel");
        HIPX(idx->dev, hipMemsetAsync(idx->mq_cnt.p, 0, (size_t)nq * 4, idx->stream), "scratch");
        m.n = N;
        m.row_step = 1;
        m.tau = idx->mq_tau.as<uint64_t>();
        HIPX(idx->dev, idx->quant ? launch_mq_scan(m, idx->stream) : launch_mq_scan_f32(m, idx->stream),
         "batched scan kernel");
        sa.tau = nullptr;
    }
    sa.merged = idx->merged.as<uint64_t>();
    sa.merged_n = idx->merged_n.as<uint32_t>();
    sa.overflow = idx->mq_flag.as<uint32_t>();
    if (!rerank) {
        sa.k_out = k_out;
        sa.out_rows = d_rows;
        sa.out_scores = d_scores;
        sa.out_n = d_n;
    }
    HIPX(idx->dev, launch_mq_select(sa, nq, idx->stream), "batched select kernel");
    if (rerank) {
        MqRerankArgs r{};
        r.rows = idx->raw.as<float>();
        r.dim = idx->dim;
        r.q = d_q;
        r.q_stride = idx->dim;
        r.merged = idx->merged.as<uint64_t>();
        r.merged_n = idx->merged_n.as<uint32_t>();
        r.kprime = kprime;
        r.k_out = k_out;
        r.out_rows = d_rows;
        r.out_scores = d_scores;
        r.out_n = d_n;
        HIPX(idx->dev, launch_mq_rerank(r, nq, idx->stream), "rerank kernel");
    }
    timing_end(idx);
    idx->last_scanned = (N + (one_pass ? 0 : S)) * nq;
    // queries whose appended keys overflowed: the fused scan, one at a time
    HIPX(idx->dev, idx->h_flag.ensure((size_t)nq * 4), "pinned buffer");
    HIPX(idx->dev, hipMemcpyAsync(idx->h_flag.p, idx->mq_flag.p, (size_t)nq * 4, hipMemcpyDeviceToHost, idx->stream),
         "flag download");
    HIPX(idx->dev, hipStreamSynchronize(idx->stream), "batched scan");
    const uint32_t *flags = (const uint32_t *)idx->h_flag.p;
    for (uint32_t i = 0; i < nq; i++) {
        if (!flags[i]) continue;
        rc = run_fused(idx, d_q + (size_t)i * idx->dim, 1, kprime, k_out, rerank, nullptr, 0,
                       d_rows + (size_t)i * k_out, d_scores + (size_t)i * k_out, d_n + i);
        if (rc) return rc;
    }
    return BV_OK;
}

// The device pipeline shared by every query entry point.
//   d_q       : nq x dim device queries (original space)
//   kprime    : candidates kept by the scan (the fetch)
//   k_out     : results per query
//   rerank    : re-rank the kprime candidates with f64 dotRow
//   outputs   : device arrays [nq][k_out], [nq]
// IVF int8 / int4 batches, list-major: the probes of every query, then every
// probed list read once for all the queries probing it (its rows' keys
// written at their candidate positions, the single-query scan's keys), then
// each query's top-kprime and the exact re-rank, as the fused scan does
// query by query (ivfquant.ts:459-527).
constexpr uint32_t IVF_BATCH_MIN_Q = 8;

static bool ivf_batch_eligible(const bv_index *idx, uint32_t nq, const uint32_t *d_mask) {
    if (!idx->ivf || (idx->codec != C_Q8 && idx->codec != C_Q4) || d_mask || nq < IVF_BATCH_MIN_Q || idx->rows == 0 ||
        !idx->nlist)
        return false;
    const uint32_t u16 = idx->P / 16;
    return u16 >= 2 && u16 <= 64 && (u16 & (u16 - 1)) == 0;
}

static int run_ivf_batched(bv_index *idx, const float *d_q, uint32_t nq, uint32_t kprime, uint32_t k_out,
                           bool rerank, uint32_t *d_rows, float *d_scores, uint32_t *d_n) {
    hipStream_t s = idx->stream;
    const unsigned char *qlev = nullptr;
    uint64_t qstride = 0;
    int rc = prepare_levels16(idx, d_q, nq, &qlev, &qstride);  // also leaves the rotated queries in qrot
    if (rc) return rc;
    const uint32_t nprobe = ivf_resolve_nprobe(idx), nlist = idx->nlist;
    uint64_t cap = 0;  // the most candidates a query can have: its nprobe largest lists
    for (uint32_t i = 0; i < nprobe && i < idx->list_sizes_desc.size(); ++i) cap += idx->list_sizes_desc[i];
    cap = std::max<uint64_t>(cap, 1);
    const uint64_t npairs = (uint64_t)nq * nprobe;
    if (npairs > 0xffffffffull || cap > 0xffffffffull) return fail(BV_E_UNSUPPORTED, "IVF batch too large");
    HIPX(idx->dev, idx->probe_scores.ensure((size_t)nq * nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->probes.ensure(npairs * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->cand_tot.ensure((size_t)nq * 8, 0, s), "scratch");
    HIPX(idx->dev, idx->ivb_base.ensure(npairs * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivb_pq.ensure(npairs * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivb_pbase.ensure(npairs * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivb_pcount.ensure((size_t)nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivb_poff.ensure((size_t)nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivb_fill.ensure((size_t)nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivb_chunks.ensure((size_t)nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->ivb_choff.ensure((size_t)nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_cand.ensure((size_t)nq * cap * 8, 0, s), "scratch");
    HIPX(idx->dev, idx->mq_cnt.ensure((size_t)nq * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->merged.ensure((size_t)nq * kprime * 8, 0, s), "scratch");
    HIPX(idx->dev, idx->merged_n.ensure((size_t)nq * 4, 0, s), "scratch");
    size_t tb = 0;
    HIPX(idx->dev, sel_exclusive_scan(nullptr, tb, nullptr, nullptr, nlist, s), "scan sizing");
    HIPX(idx->dev, idx->ivb_tmp.ensure(std::max<size_t>(tb, 256), 0, s), "scratch");
    tb = idx->ivb_tmp.cap;

    timing_begin(idx);
    IvfProbeArgs pa{};
    pa.centroids = idx->centroids.as<float>();
    pa.nlist = nlist;
    pa.P = idx->sample_dim;
    pa.qrot = idx->qrot.as<float>();
    pa.scores = idx->probe_scores.as<float>();
    pa.nprobe = nprobe;
    pa.probes = idx->probes.as<uint32_t>();
    pa.offset = idx->list_off.as<uint32_t>();
    pa.totals = idx->cand_tot.as<uint64_t>();
    HIPX(idx->dev, ivf_launch_probes(pa, nq, s), "probe kernels");
    HIPX(idx->dev, launch_zero(idx->ivb_pcount.p, (size_t)nlist * 4, s), "scratch clear");
    HIPX(idx->dev, launch_zero(idx->ivb_fill.p, (size_t)nlist * 4, s), "scratch clear");
    HIPX(idx->dev,
         launch_ivf_pairs(idx->probes.as<uint32_t>(), nq, nprobe, idx->list_off.as<uint32_t>(),
                          idx->ivb_base.as<uint32_t>(), idx->mq_cnt.as<uint32_t>(), idx->ivb_pcount.as<uint32_t>(), s),
         "pair kernel");
    HIPX(idx->dev,
         sel_exclusive_scan(idx->ivb_tmp.p, tb, idx->ivb_pcount.as<uint32_t>(), idx->ivb_poff.as<uint32_t>(), nlist, s),
         "pair scan");
    HIPX(idx->dev,
         launch_ivf_pair_scatter(idx->probes.as<uint32_t>(), idx->ivb_base.as<uint32_t>(), (uint32_t)npairs, nprobe,
                                 idx->ivb_poff.as<uint32_t>(), idx->ivb_fill.as<uint32_t>(),
                                 idx->ivb_pq.as<uint32_t>(), idx->ivb_pbase.as<uint32_t>(), s),
         "pair scatter kernel");
    HIPX(idx->dev, launch_ivf_chunk_counts(idx->ivb_pcount.as<uint32_t>(), nlist, idx->ivb_chunks.as<uint32_t>(), s),
         "chunk kernel");
    HIPX(idx->dev,
         sel_exclusive_scan(idx->ivb_tmp.p, tb, idx->ivb_chunks.as<uint32_t>(), idx->ivb_choff.as<uint32_t>(), nlist, s),
         "chunk scan");
    HIPX(idx->dev,
         launch_ivf_list_scan(idx->codes.as<uint32_t>(), idx->words_per_row, idx->codec == C_Q4 ? 4u : 8u,
                              idx->scales.as<float>(), idx->codec == C_Q4 ? 1.0f / 7.0f : 1.0f,
                              idx->list_off.as<uint32_t>(), idx->list_rows.as<uint32_t>(), nlist,
                              idx->ivb_choff.as<uint32_t>(), (uint32_t)npairs, idx->ivb_poff.as<uint32_t>(),
                              idx->ivb_pcount.as<uint32_t>(), idx->ivb_pq.as<uint32_t>(), idx->ivb_pbase.as<uint32_t>(),
                              qlev, qstride, idx->P / 16, idx->mq_cand.as<uint64_t>(), cap, s),
         "list scan kernel");
    MqSelArgs fa{};
    fa.cand = idx->mq_cand.as<uint64_t>();
    fa.cnt = idx->mq_cnt.as<uint32_t>();
    fa.cap = cap;
    fa.kk = kprime;
    fa.merged = idx->merged.as<uint64_t>();
    fa.merged_n = idx->merged_n.as<uint32_t>();
    if (!rerank) {
        fa.k_out = k_out;
        fa.out_rows = d_rows;
        fa.out_scores = d_scores;
        fa.out_n = d_n;
    }
    HIPX(idx->dev, launch_mq_select(fa, nq, s), "batched select kernel");
    if (rerank) {
        MqRerankArgs r{};
        r.rows = idx->raw.as<float>();
        r.dim = idx->dim;
        r.q = d_q;
        r.q_stride = idx->dim;
        r.merged = idx->merged.as<uint64_t>();
        r.merged_n = idx->merged_n.as<uint32_t>();
        r.kprime = kprime;
        r.k_out = k_out;
        r.out_rows = d_rows;
        r.out_scores = d_scores;
        r.out_n = d_n;
        HIPX(idx->dev, launch_mq_rerank(r, nq, s), "rerank kernel");
    }
    timing_end(idx);
    idx->last_scanned = 0;
    return BV_OK;
}

static int run_pipeline(bv_index *idx, const float *d_q, uint32_t nq, uint32_t kprime, uint32_t k_out, bool rerank,
                        const uint32_t *d_mask, uint64_t mask_bits, uint32_t *d_rows, float *d_scores,
                        uint32_t *d_n, bool may_alternate = false) {
    if (ivf_batch_eligible(idx, nq, d_mask)) {
        int rc = lanes_join(idx);
        if (rc) return rc;
        return run_ivf_batched(idx, d_q, nq, kprime, k_out, rerank, d_rows, d_scores, d_n);
    }
    if (mq_eligible(idx, nq, d_mask)) {
        int rc = lanes_join(idx);  // the batch path shares the index stream's scratch and outputs
        if (rc) return rc;
        return run_batched(idx, d_q, nq, kprime, k_out, rerank, d_rows, d_scores, d_n);
    }
    return run_fused(idx, d_q, nq, kprime, k_out, rerank, d_mask, mask_bits, d_rows, d_scores, d_n, may_alternate);
}

// Queries per device call for query batches: the matrix-core path takes
// large batches (its scratch is about 32 * kprime * N / MQ_SAMPLE bytes per
// query); the fused scan's scratch is sized per query in flight.
static uint32_t batch_chunk(const bv_index *idx, uint32_t nq) {
    return mq_eligible(idx, nq, nullptr) ? 1024u : 64u;
}

// Host entry: upload queries (+mask), run, download.
static int host_query(bv_index *idx, const float *q, uint32_t nq, uint32_t kprime, uint32_t k_out, bool rerank,
                      const uint32_t *mask, uint64_t mask_words, uint32_t *rows, float *scores, uint32_t *n_out) {
    auto t0 = std::chrono::steady_clock::now();
    if (idx->rows == 0 || k_out == 0) {
        for (uint32_t i = 0; i < nq; i++) n_out[i] = 0;
        idx->last_query_ms = 0;
        idx->last_query_gpu_ms = 0;
        return BV_OK;
    }
    int rc = ensure_built(idx);
    if (rc) return rc;
    const size_t qbytes = (size_t)nq * idx->dim * 4;
    HIPX(idx->dev, idx->qin.ensure(qbytes, 0, idx->stream), "query buffer");
    HIPX(idx->dev, hipEventRecord(idx->ev0, idx->stream), "event");
    HIPX(idx->dev, hipMemcpyAsync(idx->qin.p, q, qbytes, hipMemcpyHostToDevice, idx->stream), "query upload");
    const uint32_t *d_mask = nullptr;
    uint64_t mask_bits = 0;
    if (mask) {
        HIPX(idx->dev, idx->mask.ensure(mask_words * 4, 0, idx->stream), "mask buffer");
        HIPX(idx->dev, hipMemcpyAsync(idx->mask.p, mask, mask_words * 4, hipMemcpyHostToDevice, idx->stream),
             "mask upload");
        d_mask = idx->mask.as<uint32_t>();
        mask_bits = mask_words * 32;
    }
    HIPX(idx->dev, idx->out_rows.ensure((size_t)nq * k_out * 4, 0, idx->stream), "output buffer");
    HIPX(idx->dev, idx->out_scores.ensure((size_t)nq * k_out * 4, 0, idx->stream), "output buffer");
    HIPX(idx->dev, idx->out_n.ensure((size_t)nq * 4, 0, idx->stream), "output buffer");
    rc = run_pipeline(idx, idx->qin.as<float>(), nq, kprime, k_out, rerank, d_mask, mask_bits,
                      idx->out_rows.as<uint32_t>(), idx->out_scores.as<float>(), idx->out_n.as<uint32_t>());
    if (rc) return rc;
    HIPX(idx->dev, idx->h_rows.ensure((size_t)nq * k_out * 4), "pinned buffer");
    HIPX(idx->dev, idx->h_scores.ensure((size_t)nq * k_out * 4), "pinned buffer");
    HIPX(idx->dev, idx->h_n.ensure((size_t)nq * 4), "pinned buffer");
    HIPX(idx->dev, hipMemcpyAsync(idx->h_rows.p, idx->out_rows.p, (size_t)nq * k_out * 4, hipMemcpyDeviceToHost,
                                  idx->stream), "result download");
    HIPX(idx->dev, hipMemcpyAsync(idx->h_scores.p, idx->out_scores.p, (size_t)nq * k_out * 4,
                                  hipMemcpyDeviceToHost, idx->stream), "result download");
    HIPX(idx->dev, hipMemcpyAsync(idx->h_n.p, idx->out_n.p, (size_t)nq * 4, hipMemcpyDeviceToHost, idx->stream),
         "result download");
    HIPX(idx->dev, hipEventRecord(idx->ev1, idx->stream), "event");
    HIPX(idx->dev, hipStreamSynchronize(idx->stream), "query");
    timing_collect(idx);
    float gms = 0;
    (void)hipEventElapsedTime(&gms, idx->ev0, idx->ev1);
    std::memcpy(rows, idx->h_rows.p, (size_t)nq * k_out * 4);
    std::memcpy(scores, idx->h_scores.p, (size_t)nq * k_out * 4);
    std::memcpy(n_out, idx->h_n.p, (size_t)nq * 4);
    idx->last_query_gpu_ms = gms;
    idx->last_query_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return BV_OK;
}

// Dense-score fallback for fetches beyond the fused top-k's capacity.
static int dense_topk(bv_index *idx, const float *q, uint32_t k, const uint32_t *mask, uint64_t mask_words,
                      uint32_t *rows, float *scores, uint32_t *n_out);
static int sorted_topk(bv_index *idx, uint64_t n_keys, uint32_t k, uint32_t *rows, float *scores, uint32_t *n_out);

extern "C" int bv_index_query(bv_index *idx, const float *q, uint32_t k, uint32_t *rows, float *scores,
                              uint32_t *n_out) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (!q || !n_out || (k && (!rows || !scores))) return fail(BV_E_INVALID, "null argument");
    const uint32_t kk = (uint32_t)std::min<uint64_t>(k, idx->rows);
    if (kk > (uint32_t)MAX_KPRIME) return dense_topk(idx, q, k, nullptr, 0, rows, scores, n_out);
    return host_query(idx, q, 1, kk, kk, false, nullptr, 0, rows, scores, n_out);
}

extern "C" int bv_index_query_masked(bv_index *idx, const float *q, uint32_t k, const uint32_t *mask_words,
                                     uint64_t n_words, uint32_t *rows, float *scores, uint32_t *n_out) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (!q || !n_out || !mask_words || (k && (!rows || !scores))) return fail(BV_E_INVALID, "null argument");
    const uint64_t need = (idx->rows + 31) / 32;
    if (n_words < need)
        return fail(BV_E_INVALID, "mask has %llu words, need %llu for %llu rows", (unsigned long long)n_words,
                    (unsigned long long)need, (unsigned long long)idx->rows);
    const uint32_t kk = (uint32_t)std::min<uint64_t>(k, idx->rows);
    if (kk > (uint32_t)MAX_KPRIME) return dense_topk(idx, q, k, mask_words, n_words, rows, scores, n_out);
    return host_query(idx, q, 1, kk, kk, false, mask_words, n_words, rows, scores, n_out);
}

extern "C" int bv_index_query_batch(bv_index *idx, const float *queries, uint32_t nq, uint32_t k, uint32_t *rows,
                                    float *scores, uint32_t *n_out) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (nq == 0) return BV_OK;
    if (!queries || !n_out || (k && (!rows || !scores))) return fail(BV_E_INVALID, "null argument");
    const uint32_t kk = (uint32_t)std::min<uint64_t>(k, idx->rows);
    if (kk > (uint32_t)MAX_KPRIME) {
        for (uint32_t i = 0; i < nq; i++) {
            rc = dense_topk(idx, queries + (size_t)i * idx->dim, k, nullptr, 0, rows + (size_t)i * k,
                            scores + (size_t)i * k, n_out + i);
            if (rc) return rc;
        }
        return BV_OK;
    }
    // chunk to bound scratch
    const uint32_t chunk = batch_chunk(idx, nq);
    for (uint32_t s0 = 0; s0 < nq; s0 += chunk) {
        const uint32_t m = std::min(chunk, nq - s0);
        std::vector<uint32_t> r((size_t)m * kk);
        std::vector<float> sc((size_t)m * kk);
        rc = host_query(idx, queries + (size_t)s0 * idx->dim, m, kk, kk, false, nullptr, 0, r.data(), sc.data(),
                        n_out + s0);
        if (rc) return rc;
        for (uint32_t i = 0; i < m; i++) {
            std::memcpy(rows + (size_t)(s0 + i) * k, r.data() + (size_t)i * kk, (size_t)kk * 4);
            std::memcpy(scores + (size_t)(s0 + i) * k, sc.data() + (size_t)i * kk, (size_t)kk * 4);
        }
    }
    return BV_OK;
}

extern "C" int bv_index_set_nprobe(bv_index *idx, uint32_t nprobe) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    if (!idx) return fail(BV_E_INVALID, "null index");
    idx->nprobe_override = nprobe;
    return BV_OK;
}

extern "C" int bv_index_search(bv_index *idx, const float *queries, uint32_t nq, uint32_t fetch, uint32_t k,
                               uint32_t *rows, float *scores, uint32_t *n_out) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (nq == 0) return BV_OK;
    if (!queries || !n_out || (k && (!rows || !scores))) return fail(BV_E_INVALID, "null argument");
    if (fetch && !idx->quant) return fail(BV_E_UNSUPPORTED, "re-rank needs a quantized index");
    const uint32_t kk = (uint32_t)std::min<uint64_t>(k, idx->rows);
    uint32_t fe = fetch ? (uint32_t)std::min<uint64_t>(std::max(fetch, kk), idx->rows) : 0;
    if (fe > (uint32_t)MAX_KPRIME || kk > (uint32_t)MAX_KPRIME)
        return fail(BV_E_UNSUPPORTED, "fetch %u exceeds the fused top-k limit %d", fe, MAX_KPRIME);
    const uint32_t chunk = batch_chunk(idx, nq);
    for (uint32_t s0 = 0; s0 < nq; s0 += chunk) {
        const uint32_t m = std::min(chunk, nq - s0);
        std::vector<uint32_t> r((size_t)m * std::max(kk, 1u));
        std::vector<float> sc((size_t)m * std::max(kk, 1u));
        rc = host_query(idx, queries + (size_t)s0 * idx->dim, m, fe ? fe : kk, kk, fe != 0, nullptr, 0, r.data(),
                        sc.data(), n_out + s0);
        if (rc) return rc;
        for (uint32_t i = 0; i < m; i++) {
            std::memcpy(rows + (size_t)(s0 + i) * k, r.data() + (size_t)i * kk, (size_t)kk * 4);
            std::memcpy(scores + (size_t)(s0 + i) * k, sc.data() + (size_t)i * kk, (size_t)kk * 4);
        }
    }
    return BV_OK;
}

extern "C" int bv_index_search_device(bv_index *idx, const float *d_queries, uint32_t nq, uint32_t fetch, uint32_t k,
                                      uint32_t *d_rows, float *d_scores, uint32_t *d_n_out) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (nq == 0) return BV_OK;
    if (!d_queries || !d_rows || !d_scores || !d_n_out) return fail(BV_E_INVALID, "null argument");
    if (fetch && !idx->quant) return fail(BV_E_UNSUPPORTED, "re-rank needs a quantized index");
    if (idx->rows == 0 || k == 0) return fail(BV_E_STATE, "empty index or k == 0");
    const uint32_t kk = (uint32_t)std::min<uint64_t>(k, idx->rows);
    const uint32_t fe = fetch ? (uint32_t)std::min<uint64_t>(std::max(fetch, kk), idx->rows) : 0;
    if (fe > (uint32_t)MAX_KPRIME || kk > (uint32_t)MAX_KPRIME)
        return fail(BV_E_UNSUPPORTED, "fetch %u exceeds the fused top-k limit %d", fe, MAX_KPRIME);
    rc = ensure_built(idx);
    if (rc) return rc;
    return run_pipeline(idx, d_queries, nq, fe ? fe : kk, kk, fe != 0, nullptr, 0, d_rows, d_scores, d_n_out, true);
}

extern "C" int bv_index_set_query_streams(bv_index *idx, uint32_t n) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (n < 1 || n > (uint32_t)MAX_QUERY_STREAMS)
        return fail(BV_E_INVALID, "query streams must be 1 to %d, got %u", MAX_QUERY_STREAMS, n);
    if (n >= 2 && !idx->ev_mut) {
        HIPX(idx->dev, hipEventCreateWithFlags(&idx->ev_mut, hipEventDisableTiming), "event");
        HIPX(idx->dev, hipEventRecord(idx->ev_mut, idx->stream), "event");
        idx->mut_gen++;
    }
    for (uint32_t i = 0; i + 1 < n; ++i)
        if (!idx->lanes[i].stream) {
            HIPX(idx->dev, hipStreamCreateWithFlags(&idx->lanes[i].stream, hipStreamNonBlocking), "query stream");
            idx->lanes[i].mut_seen = 0;  // (waits on ev_mut before its first query)
        }
    rc = lanes_join(idx);
    if (rc) return rc;
    idx->query_streams = n;
    idx->next_lane = 0;
    return BV_OK;
}

// bv_index_search_device without any device allocation: the fused scan on
// every query, its scratch carved from this GPU's copy of `scratch` (used
// through the address hipGetSymbolAddress gave, never through the name).
// The coordination state and wave maxima are cleared by a fill kernel on
// every call (the previous call may have laid the array out differently).
extern "C" int bv_index_search_device_noalloc(bv_index *idx, const float *d_queries, uint32_t nq, uint32_t fetch,
                                              uint32_t k, uint32_t *d_rows, float *d_scores, uint32_t *d_n_out) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (nq == 0) return BV_OK;
    if (!d_queries || !d_rows || !d_scores || !d_n_out) return fail(BV_E_INVALID, "null argument");
    if (fetch && !idx->quant) return fail(BV_E_UNSUPPORTED, "re-rank needs a quantized index");
    if (idx->rows == 0 || k == 0) return fail(BV_E_STATE, "empty index or k == 0");
    if (idx->ivf)
        return fail(BV_E_UNSUPPORTED, "IVF queries need list scratch and a possible build: use bv_index_search_device");
    if (idx->quant && !scan_prep_supported(idx->codec, idx->units, idx->P))
        return fail(BV_E_UNSUPPORTED, "this code layout needs a query buffer: use bv_index_search_device");
    if (!idx->dev->scratch) return fail(BV_E_HIP, "the no-allocation scratch array has no device address");
    const uint32_t kk = (uint32_t)std::min<uint64_t>(k, idx->rows);
    const uint32_t fe = fetch ? (uint32_t)std::min<uint64_t>(std::max(fetch, kk), idx->rows) : 0;
    if (fe > (uint32_t)MAX_KPRIME || kk > (uint32_t)MAX_KPRIME)
        return fail(BV_E_UNSUPPORTED, "fetch %u exceeds the fused top-k limit %d", fe, MAX_KPRIME);
    const uint32_t kprime = fe ? fe : kk;
    const bool rerank = fe != 0;
    const uint32_t grid = grid_for(idx, idx->rows, kprime, rerank ? idx->dim : 0);
    const ScanLayout L = scan_layout(nq, grid, kprime);
    if (L.total > (size_t)BV_NOALLOC_SCRATCH_BYTES)
        return fail(BV_E_INVALID, "%u queries with fetch %u need %zu bytes of scratch; the limit is %zu", nq, kprime,
                    L.total, (size_t)BV_NOALLOC_SCRATCH_BYTES);
    char *base = (char *)idx->dev->scratch;
    HIPX(idx->dev, launch_zero(base, L.cand_keys, idx->stream), "scratch clear");
    ScanArgs a{};
    if (idx->quant) {  // the scan rotates and transforms the fp32 queries itself
        a.qraw = d_queries;
        a.qdim = idx->dim;
        a.signs = idx->signs.as<float>();
        a.rounds = idx->d.rounds;
    } else {
        a.q = d_queries;
        a.q_stride = (uint64_t)idx->dim * 4;
    }
    scan_bind(L, base, rerank ? idx->dim : 0, a);
    scan_common(idx, d_queries, idx->rows, grid, kprime, kk, rerank, nullptr, 0, d_rows, d_scores, d_n_out, a);
    HIPX(idx->dev, launch_scan(idx->codec, idx->units, a, nq, idx->stream), "scan kernel");
    idx->last_scanned = idx->rows * nq;
    return BV_OK;
}

extern "C" int bv_index_sync(bv_index *idx) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    HIPX(idx->dev, hipStreamSynchronize(idx->stream), "sync");
    rc = lanes_join(idx);
    if (rc) return rc;
    return BV_OK;
}

extern "C" int bv_index_stream(bv_index *idx, void **stream) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    if (!idx || !stream) return fail(BV_E_INVALID, "null argument");
    *stream = (void *)idx->stream;
    return BV_OK;
}

extern "C" int bv_index_kernel_timing(bv_index *idx, int enable, double *scan_ms, uint64_t *scan_launches) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    if (!idx) return fail(BV_E_INVALID, "null index");
    timing_collect(idx);
    if (enable) {
        idx->timing = true;
        idx->scan_ms = 0;
        idx->scan_launches = 0;
    } else {
        idx->timing = false;
    }
    if (scan_ms) *scan_ms = idx->scan_ms;
    if (scan_launches) *scan_launches = idx->scan_launches;
    return BV_OK;
}

extern "C" int bv_index_rerank(bv_index *idx, const float *q, const uint32_t *cand, uint32_t n_cand, uint32_t k,
                               uint32_t *rows, float *scores, uint32_t *n_out) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (!q || !n_out || (n_cand && !cand) || (k && (!rows || !scores))) return fail(BV_E_INVALID, "null argument");
    if (n_cand > (uint32_t)MAX_KPRIME) return fail(BV_E_UNSUPPORTED, "at most %d re-rank candidates", MAX_KPRIME);
    for (uint32_t i = 0; i < n_cand; i++)
        if (cand[i] >= idx->rows) return fail(BV_E_INVALID, "candidate row %u out of range", cand[i]);
    const uint32_t kk = std::min(k, n_cand);
    if (kk == 0) {
        *n_out = 0;
        return BV_OK;
    }
    const size_t qb = (size_t)idx->dim * 4;
    HIPX(idx->dev, idx->qin.ensure(qb, 0, idx->stream), "query buffer");
    HIPX(idx->dev, hipMemcpyAsync(idx->qin.p, q, qb, hipMemcpyHostToDevice, idx->stream), "upload");
    HIPX(idx->dev, idx->cand.ensure((size_t)n_cand * 4, 0, idx->stream), "scratch");
    HIPX(idx->dev, hipMemcpyAsync(idx->cand.p, cand, (size_t)n_cand * 4, hipMemcpyHostToDevice, idx->stream), "upload");
    HIPX(idx->dev, idx->cand_n.ensure(4, 0, idx->stream), "scratch");
    HIPX(idx->dev, hipMemcpyAsync(idx->cand_n.p, &n_cand, 4, hipMemcpyHostToDevice, idx->stream), "upload");
    HIPX(idx->dev, idx->rr_keys.ensure((size_t)n_cand * 8, 0, idx->stream), "scratch");
    {
        const size_t old = idx->rr_tickets.cap;
        HIPX(idx->dev, idx->rr_tickets.ensure(4, 0, idx->stream), "scratch");
        if (idx->rr_tickets.cap != old)
            HIPX(idx->dev, hipMemsetAsync(idx->rr_tickets.p, 0, idx->rr_tickets.cap, idx->stream), "scratch");
    }
    HIPX(idx->dev, idx->out_rows.ensure((size_t)kk * 4, 0, idx->stream), "output");
    HIPX(idx->dev, idx->out_scores.ensure((size_t)kk * 4, 0, idx->stream), "output");
    HIPX(idx->dev, idx->out_n.ensure(4, 0, idx->stream), "output");
    RerankArgs r{};
    r.rows = idx->raw.as<float>();
    r.dim = idx->dim;
    r.q = idx->qin.as<float>();
    r.q_stride = idx->dim;
    r.cand_rows = idx->cand.as<uint32_t>();
    r.cand_n = idx->cand_n.as<uint32_t>();
    r.kprime = n_cand;
    r.k_out = kk;
    r.rr_keys = idx->rr_keys.as<uint64_t>();
    r.tickets = idx->rr_tickets.as<uint32_t>();
    r.out_rows = idx->out_rows.as<uint32_t>();
    r.out_scores = idx->out_scores.as<float>();
    r.out_n = idx->out_n.as<uint32_t>();
    HIPX(idx->dev, launch_rerank(r, 1, idx->stream), "rerank kernel");
    HIPX(idx->dev, hipMemcpyAsync(rows, idx->out_rows.p, (size_t)kk * 4, hipMemcpyDeviceToHost, idx->stream), "download");
    HIPX(idx->dev, hipMemcpyAsync(scores, idx->out_scores.p, (size_t)kk * 4, hipMemcpyDeviceToHost, idx->stream),
         "download");
    HIPX(idx->dev, hipMemcpyAsync(n_out, idx->out_n.p, 4, hipMemcpyDeviceToHost, idx->stream), "download");
    HIPX(idx->dev, hipStreamSynchronize(idx->stream), "rerank");
    return BV_OK;
}

// Exact scores of the n_list rows at idx->sel_list against q (Store.dotRow /
// Store.l2Row order), then their top k by a device sort.
static int exact_list_topk(bv_index *idx, const float *q, uint64_t n_list, uint32_t k, uint32_t *rows, float *scores,
                           uint32_t *n_out) {
    hipStream_t s = idx->stream;
    const size_t qb = (size_t)idx->dim * 4;
    HIPX(idx->dev, idx->qin.ensure(qb, 0, s), "query buffer");
    HIPX(idx->dev, hipMemcpyAsync(idx->qin.p, q, qb, hipMemcpyHostToDevice, s), "upload");
    HIPX(idx->dev, idx->sel_keys.ensure(n_list * 8, 0, s), "scratch");
    HIPX(idx->dev, idx->sel_misc.ensure(8, 0, s), "scratch");
    HIPX(idx->dev, launch_zero(idx->sel_misc.p, 4, s), "scratch clear");
    HIPX(idx->dev, sel_exact_row_keys(idx->raw.as<float>(), idx->rows, idx->dim, idx->d.metric == BV_METRIC_L2,
                                      idx->qin.as<float>(), idx->sel_list.as<uint32_t>(), n_list,
                                      idx->sel_keys.as<uint64_t>(), idx->sel_misc.as<uint32_t>(), s),
         "exact row kernel");
    uint32_t bad = 0;
    HIPX(idx->dev, hipMemcpyAsync(&bad, idx->sel_misc.p, 4, hipMemcpyDeviceToHost, s), "download");
    HIPX(idx->dev, hipStreamSynchronize(s), "exact rows");
    if (bad) return fail(BV_E_INVALID, "a listed row is out of range (the index holds %llu rows)",
                         (unsigned long long)idx->rows);
    return sorted_topk(idx, n_list, k, rows, scores, n_out);
}

static int rows_prologue(bv_index *idx, const float *q, uint32_t k, uint32_t *rows, float *scores, uint32_t *n_out) {
    if (!q || !n_out || (k && (!rows || !scores))) return fail(BV_E_INVALID, "null argument");
    if (!idx->raw.p && idx->rows) return fail(BV_E_STATE, "exact row scores need the fp32 rows on the device");
    if ((size_t)idx->dim * 4 > 96 * 1024) return fail(BV_E_UNSUPPORTED, "dimension %u above 24576", idx->dim);
    return BV_OK;
}

extern "C" int bv_index_query_rows(bv_index *idx, const float *q, const uint32_t *list, uint64_t n_list, uint32_t k,
                                   uint32_t *rows, float *scores, uint32_t *n_out) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    rc = rows_prologue(idx, q, k, rows, scores, n_out);
    if (rc) return rc;
    if (n_list && !list) return fail(BV_E_INVALID, "null argument");
    if (n_list == 0 || k == 0) {
        *n_out = 0;
        return BV_OK;
    }
    HIPX(idx->dev, idx->sel_list.ensure(n_list * 4, 0, idx->stream), "scratch");
    HIPX(idx->dev, hipMemcpyAsync(idx->sel_list.p, list, n_list * 4, hipMemcpyHostToDevice, idx->stream), "upload");
    return exact_list_topk(idx, q, n_list, k, rows, scores, n_out);
}

extern "C" int bv_index_query_rows_masked(bv_index *idx, const float *q, const uint32_t *mask_words, uint64_t n_words,
                                          uint32_t k, uint32_t *rows, float *scores, uint32_t *n_out) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    rc = rows_prologue(idx, q, k, rows, scores, n_out);
    if (rc) return rc;
    if (n_words && !mask_words) return fail(BV_E_INVALID, "null argument");
    const uint64_t words = std::min<uint64_t>(n_words, (idx->rows + 31) / 32);  // bits past the rows are ignored
    if (words == 0 || k == 0) {
        *n_out = 0;
        return BV_OK;
    }
    hipStream_t s = idx->stream;
    HIPX(idx->dev, idx->mask.ensure(words * 4, 0, s), "mask buffer");
    HIPX(idx->dev, hipMemcpyAsync(idx->mask.p, mask_words, words * 4, hipMemcpyHostToDevice, s), "upload");
    HIPX(idx->dev, idx->sel_popc.ensure(words * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->sel_off.ensure(words * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->sel_misc.ensure(8, 0, s), "scratch");
    HIPX(idx->dev, sel_mask_counts(idx->mask.as<uint32_t>(), words, idx->rows, idx->sel_popc.as<uint32_t>(), s),
         "mask count kernel");
    size_t tb = 0;
    HIPX(idx->dev, sel_exclusive_scan(nullptr, tb, nullptr, nullptr, words, s), "scan sizing");
    HIPX(idx->dev, idx->sel_tmp.ensure(std::max<size_t>(tb, 256), 0, s), "scratch");
    tb = idx->sel_tmp.cap;
    HIPX(idx->dev, sel_exclusive_scan(idx->sel_tmp.p, tb, idx->sel_popc.as<uint32_t>(), idx->sel_off.as<uint32_t>(),
                                      words, s),
         "scan");
    // the list can hold every row: sized before its length is known
    HIPX(idx->dev, idx->sel_list.ensure(words * 32 * 4, 0, s), "scratch");
    HIPX(idx->dev, sel_mask_rows(idx->mask.as<uint32_t>(), words, idx->rows, idx->sel_popc.as<uint32_t>(),
                                 idx->sel_off.as<uint32_t>(), idx->sel_list.as<uint32_t>(),
                                 idx->sel_misc.as<uint32_t>() + 1, s),
         "mask row kernel");
    uint32_t n_list = 0;
    HIPX(idx->dev, hipMemcpyAsync(&n_list, idx->sel_misc.as<uint32_t>() + 1, 4, hipMemcpyDeviceToHost, s), "download");
    HIPX(idx->dev, hipStreamSynchronize(s), "mask rows");
    if (n_list == 0) {
        *n_out = 0;
        return BV_OK;
    }
    return exact_list_topk(idx, q, n_list, k, rows, scores, n_out);
}

// Dense scores of one query for every row (the scan's score for each row),
// or with `probed` on an IVF index, for each candidate of its probed lists
// (idx->cand[0, *n_scored), in gather order).
static int dense_scores(bv_index *idx, const float *q, const uint32_t *mask, uint64_t mask_words, float *out,
                        bool probed = false, uint64_t *n_scored = nullptr) {
    const size_t qb = (size_t)idx->dim * 4;
    HIPX(idx->dev, idx->qin.ensure(qb, 0, idx->stream), "query buffer");
    HIPX(idx->dev, hipMemcpyAsync(idx->qin.p, q, qb, hipMemcpyHostToDevice, idx->stream), "upload");
    uint64_t n = idx->rows;
    if (probed) {
        uint64_t per = 0;
        int rc = ivf_candidates(idx, idx->qin.as<float>(), 1, &per);
        if (rc) return rc;
        uint64_t off[2] = {0, 0};
        HIPX(idx->dev, hipMemcpyAsync(off, idx->cand_off.p, 16, hipMemcpyDeviceToHost, idx->stream), "download");
        HIPX(idx->dev, hipStreamSynchronize(idx->stream), "candidates");
        n = off[1] - off[0];
    }
    if (n_scored) *n_scored = n;
    HIPX(idx->dev, idx->dense.ensure(std::max<uint64_t>(n, 1) * 4, 0, idx->stream), "scratch");
    const void *qscan = nullptr;
    uint64_t qstride = 0;
    const bool in_kernel = idx->quant && scan_prep_supported(idx->codec, idx->units, idx->P);
    int rc = in_kernel ? BV_OK : prepare_queries(idx, idx->qin.as<float>(), 1, &qscan, &qstride);
    if (rc) return rc;
    const uint32_t grid = grid_for(idx, std::max<uint64_t>(n, 1), 1, 0);
    const uint32_t *d_mask = nullptr;
    if (mask) {
        HIPX(idx->dev, idx->mask.ensure(mask_words * 4, 0, idx->stream), "mask buffer");
        HIPX(idx->dev, hipMemcpyAsync(idx->mask.p, mask, mask_words * 4, hipMemcpyHostToDevice, idx->stream), "upload");
        d_mask = idx->mask.as<uint32_t>();
    }
    ScanArgs a{};
    rc = scan_scratch(idx, 1, grid, 1, 0, a);
    if (rc) return rc;
    a.codes = idx->quant ? idx->codes.p : idx->raw.p;
    a.row_bytes = idx->row_bytes;
    a.units = idx->units;
    a.padded_dim = idx->P;
    a.scales = (idx->codec == C_Q8 || idx->codec == C_Q4 || idx->codec == C_Q1A || idx->codec == C_Q1P) ? idx->scales.as<float>() : nullptr;
    a.scale_mul = idx->codec == C_Q4 ? 1.0f / 7.0f : 1.0f;
    if (in_kernel) {  // the scan rotates and transforms the fp32 query itself
        a.qraw = idx->qin.as<float>();
        a.qdim = idx->dim;
        a.signs = idx->signs.as<float>();
        a.rounds = idx->d.rounds;
    } else {
        a.q = qscan;
        a.q_stride = qstride;
    }
    a.mask = d_mask;
    a.mask_bits = mask_words * 32;
    a.n = n;
    if (probed) {
        a.cand = idx->cand.as<uint32_t>();
        a.cand_off = idx->cand_off.as<uint64_t>();
    }
    a.kprime = 1;
    a.grid = grid;
    a.dense_out = idx->dense.as<float>();
    if (n == 0) return BV_OK;
    HIPX(idx->dev, launch_scan(idx->codec, idx->units, a, 1, idx->stream), "scan kernel");
    if (!out) return BV_OK;  // the scores stay in idx->dense
    HIPX(idx->dev, hipMemcpyAsync(out, idx->dense.p, idx->rows * 4, hipMemcpyDeviceToHost, idx->stream), "download");
    HIPX(idx->dev, hipStreamSynchronize(idx->stream), "dense scores");
    return BV_OK;
}

// Top min(k, n_keys) of the keys in idx->sel_keys by a descending device
// sort: the canonical order (score desc, row asc); empty keys (0) are not
// returned.  Serves any k (flat.ts:217-239 takes any k).
static int sorted_topk(bv_index *idx, uint64_t n_keys, uint32_t k, uint32_t *rows, float *scores, uint32_t *n_out) {
    hipStream_t s = idx->stream;
    const uint32_t kk = (uint32_t)std::min<uint64_t>(k, n_keys);
    if (kk == 0) {
        *n_out = 0;
        return BV_OK;
    }
    if (n_keys > 0x7fffffffull) return fail(BV_E_UNSUPPORTED, "selection over more than 2^31 - 1 rows");
    size_t tb = 0;
    HIPX(idx->dev, sel_sort_desc(nullptr, tb, nullptr, nullptr, n_keys, s), "sort sizing");
    HIPX(idx->dev, idx->sel_tmp.ensure(std::max<size_t>(tb, 256), 0, s), "scratch");
    HIPX(idx->dev, idx->sel_sorted.ensure(n_keys * 8, 0, s), "scratch");
    tb = idx->sel_tmp.cap;
    HIPX(idx->dev, sel_sort_desc(idx->sel_tmp.p, tb, idx->sel_keys.as<uint64_t>(), idx->sel_sorted.as<uint64_t>(),
                                 n_keys, s),
         "sort");
    HIPX(idx->dev, idx->out_rows.ensure((size_t)kk * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->out_scores.ensure((size_t)kk * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->out_n.ensure(4, 0, s), "scratch");
    HIPX(idx->dev, sel_keys_to_hits(idx->sel_sorted.as<uint64_t>(), kk, idx->out_rows.as<uint32_t>(),
                                    idx->out_scores.as<float>(), idx->out_n.as<uint32_t>(), s),
         "hits kernel");
    uint32_t n = 0;
    HIPX(idx->dev, hipMemcpyAsync(&n, idx->out_n.p, 4, hipMemcpyDeviceToHost, s), "download");
    HIPX(idx->dev, hipMemcpyAsync(rows, idx->out_rows.p, (size_t)kk * 4, hipMemcpyDeviceToHost, s), "download");
    HIPX(idx->dev, hipMemcpyAsync(scores, idx->out_scores.p, (size_t)kk * 4, hipMemcpyDeviceToHost, s), "download");
    HIPX(idx->dev, hipStreamSynchronize(s), "selection");
    *n_out = n;
    return BV_OK;
}

// Queries with k above the fused top-k's MAX_KPRIME: the dense scores of
// every row (IVF: of every candidate of the probed lists), then the top k by
// a device sort.
static int dense_topk(bv_index *idx, const float *q, uint32_t k, const uint32_t *mask, uint64_t mask_words,
                      uint32_t *rows, float *scores, uint32_t *n_out) {
    int rc = ensure_built(idx);
    if (rc) return rc;
    if (idx->ivf) {
        if (mask) return fail(BV_E_UNSUPPORTED, "IVF indexes take no score mask");
        uint64_t n = 0;
        rc = dense_scores(idx, q, nullptr, 0, nullptr, true, &n);
        if (rc) return rc;
        HIPX(idx->dev, idx->sel_keys.ensure(std::max<uint64_t>(n, 1) * 8, 0, idx->stream), "scratch");
        HIPX(idx->dev, sel_list_keys(idx->dense.as<float>(), idx->cand.as<uint32_t>(), n,
                                     idx->sel_keys.as<uint64_t>(), idx->stream),
             "key kernel");
        return sorted_topk(idx, n, k, rows, scores, n_out);
    }
    rc = dense_scores(idx, q, nullptr, 0, nullptr);
    if (rc) return rc;
    const uint32_t *d_mask = nullptr;
    if (mask) {
        HIPX(idx->dev, idx->mask.ensure(mask_words * 4, 0, idx->stream), "mask buffer");
        HIPX(idx->dev, hipMemcpyAsync(idx->mask.p, mask, mask_words * 4, hipMemcpyHostToDevice, idx->stream), "upload");
        d_mask = idx->mask.as<uint32_t>();
    }
    HIPX(idx->dev, idx->sel_keys.ensure(idx->rows * 8, 0, idx->stream), "scratch");
    HIPX(idx->dev, sel_dense_keys(idx->dense.as<float>(), idx->rows, d_mask, idx->sel_keys.as<uint64_t>(), idx->stream),
         "key kernel");
    return sorted_topk(idx, idx->rows, k, rows, scores, n_out);
}

// ------------------------------------------------------------ stats/exports
extern "C" int bv_index_get_stats(bv_index *idx, bv_index_stats *out) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    if (!idx || !out) return fail(BV_E_INVALID, "null argument");
    std::memset(out, 0, sizeof *out);
    out->rows = idx->rows;
    out->dim = idx->dim;
    out->padded_dim = idx->quant ? idx->P : idx->dim;
    out->words_per_row = idx->words_per_row;
    out->bits = idx->d.bits;
    uint32_t chunks = 1;
    if (idx->d.chunk_rows && idx->rows) chunks = (uint32_t)((idx->rows + idx->d.chunk_rows - 1) / idx->d.chunk_rows);
    out->chunk_count = chunks;
    out->tuned_recall = -1.0f;
    if (idx->ivf && idx->nlist) {
        out->nlist = idx->nlist;
        const uint32_t saved = idx->nprobe_override;
        out->nprobe = ivf_resolve_nprobe(idx);
        idx->nprobe_override = saved;
        out->build_ms = idx->build_ms;
        out->build_exact_rows = idx->build_exact_rows;
        out->tuned_recall = idx->tuned_recall;
    }
    out->last_query_ms = idx->last_query_ms;
    out->last_query_gpu_ms = idx->last_query_gpu_ms;
    out->device_bytes = idx->raw.cap + idx->codes.cap + idx->scales.cap + idx->sample.cap + idx->centroids.cap +
                        idx->list_off.cap + idx->list_rows.cap;
    out->last_scanned_rows = idx->last_scanned;
    return BV_OK;
}

extern "C" int bv_index_export_codes(bv_index *idx, uint64_t row0, uint64_t count, uint32_t *words, float *scales) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (!idx->quant) return fail(BV_E_STATE, "not a quantized index");
    if (row0 + count > idx->rows) return fail(BV_E_INVALID, "row range out of bounds");
    if (count == 0) return BV_OK;
    if (words)
        HIPX(idx->dev, hipMemcpy(words, idx->codes.as<char>() + row0 * idx->row_bytes, count * idx->row_bytes,
                                 hipMemcpyDeviceToHost), "download");
    if (scales)
        HIPX(idx->dev, hipMemcpy(scales, idx->scales.as<float>() + row0, count * 4, hipMemcpyDeviceToHost), "download");
    return BV_OK;
}

extern "C" int bv_index_export_scores(bv_index *idx, const float *q, float *scores) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (!q || !scores) return fail(BV_E_INVALID, "null argument");
    if (idx->rows == 0) return BV_OK;
    return dense_scores(idx, q, nullptr, 0, scores);
}

extern "C" int bv_index_export_rotated_query(bv_index *idx, const float *q, float *rotated) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (!idx->quant) return fail(BV_E_STATE, "not a quantized index");
    if (!q || !rotated) return fail(BV_E_INVALID, "null argument");
    const size_t qb = (size_t)idx->dim * 4;
    HIPX(idx->dev, idx->qin.ensure(qb, 0, idx->stream), "query buffer");
    HIPX(idx->dev, hipMemcpyAsync(idx->qin.p, q, qb, hipMemcpyHostToDevice, idx->stream), "upload");
    const void *qs = nullptr;
    uint64_t st = 0;
    rc = prepare_queries(idx, idx->qin.as<float>(), 1, &qs, &st);
    if (rc) return rc;
    HIPX(idx->dev, hipMemcpyAsync(rotated, idx->qrot.p, (size_t)idx->P * 4, hipMemcpyDeviceToHost, idx->stream),
         "download");
    HIPX(idx->dev, hipStreamSynchronize(idx->stream), "rotate");
    return BV_OK;
}

extern "C" int bv_index_build(bv_index *idx) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (!idx->ivf) return BV_OK;
    if (idx->rows == 0) return fail(BV_E_STATE, "IVF build needs rows");
    if (idx->built_rows == idx->rows && !idx->retrain_due) return BV_OK;
    return ivf_build(idx);
}

extern "C" int bv_index_export_probe_scores(bv_index *idx, const float *queries, uint32_t nq, float *scores) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (!idx->ivf) return fail(BV_E_STATE, "not an IVF index");
    if (nq == 0) return BV_OK;
    if (!queries || !scores) return fail(BV_E_INVALID, "null argument");
    if (idx->rows == 0) return fail(BV_E_STATE, "IVF build needs rows");
    rc = ensure_built(idx);
    if (rc) return rc;
    hipStream_t s = idx->stream;
    const size_t qb = (size_t)nq * idx->dim * 4;
    HIPX(idx->dev, idx->qin.ensure(qb, 0, s), "query buffer");
    HIPX(idx->dev, hipMemcpyAsync(idx->qin.p, queries, qb, hipMemcpyHostToDevice, s), "upload");
    const float *qrot = idx->qin.as<float>();
    if (idx->quant) {
        HIPX(idx->dev, idx->ivf_qrot.ensure((size_t)nq * idx->P * 4, 0, s), "query buffer");
        EncodeArgs e{};
        e.src = idx->qin.as<float>();
        e.rows = nq;
        e.dim = idx->dim;
        e.P = idx->P;
        e.signs = idx->signs.as<float>();
        e.rounds = idx->d.rounds;
        e.rotated = idx->ivf_qrot.as<float>();
        HIPX(idx->dev, launch_encode(e, s), "query rotate kernel");
        qrot = idx->ivf_qrot.as<float>();
    }
    HIPX(idx->dev, idx->probe_scores.ensure((size_t)nq * idx->nlist * 4, 0, s), "scratch");
    HIPX(idx->dev, idx->probes.ensure((size_t)nq * 4, 0, s), "scratch");
    IvfProbeArgs pa{};
    pa.centroids = idx->centroids.as<float>();
    pa.nlist = idx->nlist;
    pa.P = idx->sample_dim;
    pa.qrot = qrot;
    pa.scores = idx->probe_scores.as<float>();
    pa.nprobe = 1;
    pa.probes = idx->probes.as<uint32_t>();
    HIPX(idx->dev, ivf_launch_probes(pa, nq, s), "probe kernels");
    HIPX(idx->dev, hipMemcpyAsync(scores, idx->probe_scores.p, (size_t)nq * idx->nlist * 4, hipMemcpyDeviceToHost, s),
         "download");
    HIPX(idx->dev, hipStreamSynchronize(s), "probe scores");
    return BV_OK;
}

// ------------------------------------------------------------ index section
// A snapshot section holding what a load would otherwise re-derive: the
// codes and scales (re-encoded from the rows and the fixed seed,
// src/index.ts:673-700) and the IVF state (reservoir, centroids, CSR lists,
// tuned nprobe; rebuilt on the first query after a load).  It sits beside
// the reference snapshot's fp32 rows, as the HNSW graph section does
// (src/persist/format.ts:1-22).  Little-endian; blocks 8-byte aligned.
namespace {
constexpr uint32_t SECTION_MAGIC = 0x58495642u;  // "BVIX"
constexpr uint32_t SECTION_VERSION = 1;
struct SectionHeader {
    uint32_t magic, version, header_bytes, ivf_incremental;
    uint32_t kind, dim, metric, bits, scorer, seed, rounds;
    uint32_t nlist_desc, sample_size, train_size, iters, ivf_seed, has_ivf_seed;
    float target_recall;
    uint64_t count;
    uint32_t P, words_per_row, nlist, built;
    uint64_t built_rows;
    uint32_t sample_cap, sample_dim;
    uint64_t sample_filled, sample_seen;
    uint32_t sample_rng, tuned_nprobe;
    float tuned_recall;
    uint32_t retrain_due;
};
static_assert(sizeof(SectionHeader) % 8 == 0, "section header alignment");

inline uint64_t pad8(uint64_t n) { return (n + 7) & ~7ull; }

SectionHeader section_header(const bv_index *idx) {
    SectionHeader h{};
    h.magic = SECTION_MAGIC;
    h.version = SECTION_VERSION;
    h.header_bytes = sizeof(SectionHeader);
    h.ivf_incremental = idx->d.ivf_incremental;
    h.kind = idx->d.kind;
    h.dim = idx->d.dim;
    h.metric = idx->d.metric;
    h.bits = idx->d.bits;
    h.scorer = idx->d.scorer;
    h.seed = idx->d.seed;
    h.rounds = idx->d.rounds;
    h.nlist_desc = idx->d.nlist;
    h.sample_size = idx->d.sample_size;
    h.train_size = idx->d.train_size;
    h.iters = idx->d.iters;
    h.ivf_seed = idx->d.ivf_seed;
    h.has_ivf_seed = idx->d.has_ivf_seed;
    h.target_recall = idx->d.target_recall;
    h.count = idx->rows;
    h.P = idx->P;
    h.words_per_row = idx->words_per_row;
    h.nlist = idx->nlist;
    h.built = idx->ivf && idx->rows && idx->built_rows == idx->rows ? 1u : 0u;
    h.built_rows = h.built ? idx->built_rows : 0;
    h.sample_cap = idx->sample_cap;
    h.sample_dim = idx->sample_dim;
    h.sample_filled = idx->sample_filled;
    h.sample_seen = idx->sample_seen;
    h.sample_rng = idx->sample_rng;
    h.tuned_nprobe = idx->tuned_nprobe;
    h.tuned_recall = idx->tuned_recall;
    h.retrain_due = idx->retrain_due ? 1u : 0u;
    return h;
}

// Block sizes in section order: scales, codes (quantized kinds); reservoir
// rows, reservoir row ids (IVF); centroids, list offsets, list rows (built IVF).
std::vector<uint64_t> section_blocks(const SectionHeader &h, bool quant, bool ivf, uint32_t row_bytes) {
    std::vector<uint64_t> b;
    if (quant) {
        b.push_back(h.count * 4);
        b.push_back(h.count * row_bytes);
    }
    if (ivf) {
        b.push_back(h.sample_filled * h.sample_dim * 4);
        b.push_back(h.sample_filled * 8);
        if (h.built) {
            b.push_back((uint64_t)h.nlist * h.sample_dim * 4);
            b.push_back(((uint64_t)h.nlist + 1) * 4);
            b.push_back(h.built_rows * 4);
        }
    }
    return b;
}

uint64_t section_bytes(const std::vector<uint64_t> &blocks) {
    uint64_t n = sizeof(SectionHeader);
    for (uint64_t b : blocks) n += pad8(b);
    return n;
}
}  // namespace

extern "C" int bv_index_save_section(bv_index *idx, void *buf, uint64_t cap, uint64_t *size) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (!size) return fail(BV_E_INVALID, "null argument");
    const SectionHeader h = section_header(idx);
    const std::vector<uint64_t> blocks = section_blocks(h, idx->quant, idx->ivf, idx->row_bytes);
    const uint64_t total = section_bytes(blocks);
    *size = total;
    if (!buf || cap < total) return BV_OK;
    unsigned char *out = (unsigned char *)buf;
    std::memset(out, 0, total);
    std::memcpy(out, &h, sizeof(h));
    uint64_t at = sizeof(h);
    std::vector<const void *> src;
    if (idx->quant) {
        src.push_back(idx->scales.p);
        src.push_back(idx->codes.p);
    }
    HIPX(idx->dev, hipStreamSynchronize(idx->stream), "save");
    size_t bi = 0;
    for (; bi < src.size(); ++bi) {
        if (blocks[bi]) HIPX(idx->dev, hipMemcpy(out + at, src[bi], blocks[bi], hipMemcpyDeviceToHost), "download");
        at += pad8(blocks[bi]);
    }
    if (idx->ivf) {
        if (blocks[bi])
            HIPX(idx->dev, hipMemcpy(out + at, idx->sample.p, blocks[bi], hipMemcpyDeviceToHost), "download");
        at += pad8(blocks[bi++]);
        if (blocks[bi]) std::memcpy(out + at, idx->sample_row.data(), blocks[bi]);
        at += pad8(blocks[bi++]);
        if (h.built) {
            const void *dsrc[3] = {idx->centroids.p, idx->list_off.p, idx->list_rows.p};
            for (int j = 0; j < 3; ++j, ++bi) {
                if (blocks[bi])
                    HIPX(idx->dev, hipMemcpy(out + at, dsrc[j], blocks[bi], hipMemcpyDeviceToHost), "download");
                at += pad8(blocks[bi]);
            }
        }
    }
    return BV_OK;
}

extern "C" int bv_index_load_section(bv_index *idx, const float *data, uint64_t n_floats, uint64_t count,
                                     const void *section, uint64_t bytes) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (!section || (count && !data)) return fail(BV_E_INVALID, "null argument");
    if (idx->rows) return fail(BV_E_STATE, "a section loads into an empty index");
    if (n_floats != count * idx->dim)
        return fail(BV_E_INVALID, "expected %llu floats, got %llu", (unsigned long long)(count * idx->dim),
                    (unsigned long long)n_floats);
    SectionHeader h{};
    if (bytes < sizeof(h)) return fail(BV_E_INVALID, "index section truncated (%llu bytes)", (unsigned long long)bytes);
    std::memcpy(&h, section, sizeof(h));
    if (h.magic != SECTION_MAGIC || h.header_bytes != sizeof(h)) return fail(BV_E_INVALID, "not an index section");
    if (h.version != SECTION_VERSION) return fail(BV_E_UNSUPPORTED, "index section version %u", h.version);
    const SectionHeader mine = section_header(idx);
    if (h.kind != mine.kind || h.dim != mine.dim || h.metric != mine.metric || h.bits != mine.bits ||
        h.scorer != mine.scorer || h.seed != mine.seed || h.rounds != mine.rounds || h.nlist_desc != mine.nlist_desc ||
        h.sample_size != mine.sample_size || h.train_size != mine.train_size || h.iters != mine.iters ||
        h.ivf_seed != mine.ivf_seed || h.has_ivf_seed != mine.has_ivf_seed || h.P != mine.P ||
        h.ivf_incremental != mine.ivf_incremental ||
        h.words_per_row != mine.words_per_row || h.sample_cap != mine.sample_cap || h.sample_dim != mine.sample_dim ||
        std::memcmp(&h.target_recall, &mine.target_recall, 4) != 0)
        return fail(BV_E_INVALID, "the index section was saved from an index with a different configuration");
    if (h.count != count)
        return fail(BV_E_INVALID, "the index section holds %llu rows, got %llu", (unsigned long long)h.count,
                    (unsigned long long)count);
    if (idx->ivf && (h.sample_filled > h.sample_cap || h.sample_filled > h.count || h.sample_seen < h.sample_filled ||
                     (h.built && (h.built_rows != h.count || h.nlist == 0 || h.nlist > IVF_MAX_NLIST))))
        return fail(BV_E_INVALID, "index section: inconsistent IVF state");
    const std::vector<uint64_t> blocks = section_blocks(h, idx->quant, idx->ivf, idx->row_bytes);
    if (bytes != section_bytes(blocks))
        return fail(BV_E_INVALID, "index section has %llu bytes, expected %llu", (unsigned long long)bytes,
                    (unsigned long long)section_bytes(blocks));
    const unsigned char *in = (const unsigned char *)section;
    std::vector<uint64_t> at(blocks.size());
    uint64_t pos = sizeof(h);
    for (size_t j = 0; j < blocks.size(); ++j) {
        at[j] = pos;
        pos += pad8(blocks[j]);
    }
    if (idx->ivf && h.built) {  // the lists must be a valid CSR over the rows
        const uint32_t *off = (const uint32_t *)(in + at[blocks.size() - 2]);
        const uint32_t *lr = (const uint32_t *)(in + at[blocks.size() - 1]);
        if (off[0] != 0 || off[h.nlist] != h.built_rows) return fail(BV_E_INVALID, "index section: bad list offsets");
        for (uint32_t c = 0; c < h.nlist; ++c)
            if (off[c + 1] < off[c]) return fail(BV_E_INVALID, "index section: bad list offsets");
        for (uint64_t r = 0; r < h.built_rows; ++r)
            if (lr[r] >= h.count) return fail(BV_E_INVALID, "index section: list row out of range");
    }
    if (idx->ivf) {
        const uint64_t *sr = (const uint64_t *)(in + at[idx->quant ? 3 : 1]);
        for (uint64_t j = 0; j < h.sample_filled; ++j)
            if (sr[j] >= h.count) return fail(BV_E_INVALID, "index section: reservoir row out of range");
    }
    // every allocation first, so a failure leaves the index empty
    const size_t rb = (size_t)idx->dim * 4;
    hipStream_t s = idx->stream;
    HIPX(idx->dev, idx->raw.ensure(std::max<uint64_t>(count, 1) * rb, 0, s), "row buffer");
    const bool norms = !idx->quant && !idx->ivf;
    const bool code_norms = idx->codec == C_Q8 && !idx->ivf;
    if (norms) HIPX(idx->dev, idx->rsq.ensure(std::max<uint64_t>(count, 1) * 4, 0, s), "norm buffer");
    if (code_norms) HIPX(idx->dev, idx->cnorm.ensure(std::max<uint64_t>(count, 1) * 4, 0, s), "norm buffer");
    if (idx->quant) {
        HIPX(idx->dev, idx->scales.ensure(std::max<uint64_t>(count, 1) * 4, 0, s), "scale buffer");
        HIPX(idx->dev, idx->codes.ensure(std::max<uint64_t>(count, 1) * idx->row_bytes, 0, s), "code buffer");
    }
    if (idx->ivf) {
        HIPX(idx->dev, idx->sample.ensure(std::max<uint64_t>(h.sample_filled, 1) * idx->sample_dim * 4, 0, s),
             "sample buffer");
        if (h.built) {
            HIPX(idx->dev, idx->centroids.ensure((size_t)h.nlist * idx->sample_dim * 4, 0, s), "centroids");
            HIPX(idx->dev, idx->list_off.ensure(((size_t)h.nlist + 1) * 4, 0, s), "lists");
            HIPX(idx->dev, idx->list_rows.ensure(std::max<uint64_t>(h.built_rows, 1) * 4, 0, s), "lists");
        }
    }
    if (count) HIPX(idx->dev, hipMemcpyAsync(idx->raw.p, data, count * rb, hipMemcpyHostToDevice, s), "row upload");
    size_t bi = 0;
    if (idx->quant) {
        HIPX(idx->dev, hipMemcpyAsync(idx->scales.p, in + at[0], blocks[0], hipMemcpyHostToDevice, s), "upload");
        HIPX(idx->dev, hipMemcpyAsync(idx->codes.p, in + at[1], blocks[1], hipMemcpyHostToDevice, s), "upload");
        bi = 2;
    }
    if (norms)
        HIPX(idx->dev, launch_row_sqnorms(idx->raw.as<float>(), count, idx->dim, idx->rsq.as<float>(),
                                          idx->rsq_max.as<uint32_t>(), s),
             "norm kernel");
    if (code_norms)
        HIPX(idx->dev, launch_row_code_norms(idx->codes.as<uint32_t>(), count, idx->words_per_row,
                                             idx->cnorm.as<float>(), s),
             "norm kernel");
    if (idx->ivf) {
        if (blocks[bi])
            HIPX(idx->dev, hipMemcpyAsync(idx->sample.p, in + at[bi], blocks[bi], hipMemcpyHostToDevice, s),
                 "upload");
        ++bi;
        const uint64_t *sr = (const uint64_t *)(in + at[bi++]);
        idx->sample_row.assign(sr, sr + h.sample_filled);
        idx->sample_filled = h.sample_filled;
        idx->sample_seen = h.sample_seen;
        idx->sample_rng = h.sample_rng;
        idx->tuned_nprobe = h.tuned_nprobe;
        idx->tuned_recall = h.tuned_recall;
        if (h.built) {
            void *dst[3] = {idx->centroids.p, idx->list_off.p, idx->list_rows.p};
            for (int j = 0; j < 3; ++j, ++bi)
                if (blocks[bi])
                    HIPX(idx->dev, hipMemcpyAsync(dst[j], in + at[bi], blocks[bi], hipMemcpyHostToDevice, s),
                         "upload");
            const uint32_t *off = (const uint32_t *)(in + at[bi - 2]);
            idx->nlist = h.nlist;
            idx->list_sizes_desc.resize(h.nlist);
            for (uint32_t c = 0; c < h.nlist; ++c) idx->list_sizes_desc[c] = off[c + 1] - off[c];
            std::sort(idx->list_sizes_desc.begin(), idx->list_sizes_desc.end(), std::greater<uint32_t>());
            idx->built_rows = h.built_rows;
            idx->retrain_due = h.retrain_due != 0;
        }
    }
    HIPX(idx->dev, hipStreamSynchronize(s), "load");
    idx->rows = count;
    return lanes_mark(idx);
}

extern "C" int bv_index_export_ivf(bv_index *idx, float *centroids, uint32_t *list_off, uint32_t *list_rows) {
    if (!idx) return fail(BV_E_INVALID, "null index");
    std::lock_guard<std::recursive_mutex> lock(idx->mu);
    int rc = check_live(idx);
    if (rc) return rc;
    if (!idx->ivf) return fail(BV_E_STATE, "not an IVF index");
    if (idx->rows == 0) return fail(BV_E_STATE, "IVF lists need rows");
    rc = ensure_built(idx);  // the lists a query would probe now
    if (rc) return rc;
    if (centroids)
        HIPX(idx->dev, hipMemcpy(centroids, idx->centroids.p, (size_t)idx->nlist * idx->sample_dim * 4,
                                 hipMemcpyDeviceToHost), "download");
    if (list_off)
        HIPX(idx->dev, hipMemcpy(list_off, idx->list_off.p, ((size_t)idx->nlist + 1) * 4, hipMemcpyDeviceToHost),
             "download");
    if (list_rows && idx->rows)
        HIPX(idx->dev, hipMemcpy(list_rows, idx->list_rows.p, (size_t)idx->rows * 4, hipMemcpyDeviceToHost),
             "download");
    return BV_OK;
}


// ------------------------------------------------------------ graph search
// HNSWGpuSearcher (src/index/hnswGpu.ts:28-244): the corpus rows and the
// layer-0 adjacency the host's HNSW build hands over, and the beam search of
// a batch of queries in one launch (one wave per query).
struct bv_graph {
    mutable std::mutex mu;
    bv_device *dev = nullptr;
    hipStream_t stream = nullptr;
    uint32_t dim = 0, metric = 0, degree = 0;
    uint64_t corpus_rows = 0, graph_rows = 0;
    DevBuf corpus, graph, queries, entries, out_rows, out_scores, out_n, beam_d, beam_i;
};

namespace {
int graph_live(bv_graph *g) {
    if (!g) return fail(BV_E_INVALID, "null graph searcher");
    if (g->dev->lost) return fail(BV_E_DEVICE_LOST, "GPU device lost; re-create the store");
    hipError_t e = hipSetDevice(g->dev->ordinal);
    if (e != hipSuccess) return hip_fail(g->dev, e, "hipSetDevice");
    return BV_OK;
}

// The searcher's seeds (hnswGpu.ts:142-150): the HNSW entry, then up to
// seven rows spread evenly over the adjacency's rows.
uint32_t graph_seeds(uint32_t entry, uint64_t rows, uint32_t *out) {
    uint32_t e = 0;
    out[e++] = entry;
    const uint64_t extra = std::min<uint64_t>(7, rows);
    for (uint64_t i = 0; i < extra; i++)
        out[e++] = (uint32_t)((uint64_t)std::floor((double)(i + 1) * (double)rows / (double)(extra + 1)) % rows);
    return e;
}

int graph_run(bv_graph *g, const float *queries, uint32_t nq, const uint32_t *entries, uint32_t n_entries,
              uint32_t ef_active, uint32_t iter_cap, uint32_t k, uint32_t stride, bool beams) {
    hipStream_t s = g->stream;
    const size_t qb = (size_t)nq * g->dim * 4;
    HIPX(g->dev, g->queries.ensure(qb, 0, s), "query buffer");
    HIPX(g->dev, hipMemcpyAsync(g->queries.p, queries, qb, hipMemcpyHostToDevice, s), "upload");
    HIPX(g->dev, g->entries.ensure(std::max<size_t>(n_entries, 1) * 4, 0, s), "scratch");
    if (n_entries)
        HIPX(g->dev, hipMemcpyAsync(g->entries.p, entries, (size_t)n_entries * 4, hipMemcpyHostToDevice, s), "upload");
    GraphArgs a{};
    a.corpus = g->corpus.as<float>();
    a.dim = g->dim;
    a.corpus_rows = g->corpus_rows;
    a.graph = g->graph.as<uint32_t>();
    a.K = g->degree;
    a.graph_rows = g->graph_rows;
    a.queries = g->queries.as<float>();
    a.entries = g->entries.as<uint32_t>();
    a.n_entries = n_entries;
    a.efA = ef_active;
    a.iter_cap = iter_cap;
    if (beams) {
        HIPX(g->dev, g->beam_d.ensure((size_t)nq * GRAPH_EF_CAP * 4, 0, s), "scratch");
        HIPX(g->dev, g->beam_i.ensure((size_t)nq * GRAPH_EF_CAP * 4, 0, s), "scratch");
        a.beam_dist = g->beam_d.as<float>();
        a.beam_id = g->beam_i.as<uint32_t>();
    } else {
        HIPX(g->dev, g->out_rows.ensure((size_t)nq * std::max(stride, 1u) * 4, 0, s), "scratch");
        HIPX(g->dev, g->out_scores.ensure((size_t)nq * std::max(stride, 1u) * 4, 0, s), "scratch");
        HIPX(g->dev, g->out_n.ensure((size_t)nq * 4, 0, s), "scratch");
        a.k = k;
        a.out_stride = stride;
        a.out_rows = g->out_rows.as<uint32_t>();
        a.out_scores = g->out_scores.as<float>();
        a.out_n = g->out_n.as<uint32_t>();
    }
    HIPX(g->dev, launch_graph_beam(a, nq, g->metric == BV_METRIC_L2, s), "graph search kernel");
    return BV_OK;
}
}  // namespace

extern "C" int bv_graph_create(bv_device *dev, uint32_t dim, uint32_t metric, uint32_t degree, bv_graph **out) {
    if (!dev || !out) return fail(BV_E_INVALID, "null argument");
    if (dev->lost) return fail(BV_E_DEVICE_LOST, "GPU device lost; re-create the store");
    if (dim == 0) return fail(BV_E_INVALID, "dimension must be a positive integer, got %u", dim);
    if ((size_t)dim * 4 > 64 * 1024) return fail(BV_E_UNSUPPORTED, "graph search supports dimension <= 16384");
    if (metric > BV_METRIC_L2) return fail(BV_E_INVALID, "unknown metric %u", metric);
    if (degree == 0 || degree > 64)
        return fail(BV_E_UNSUPPORTED, "GPU graph search supports degree \xe2\x89\xa4 64 (M \xe2\x89\xa4 32), got %u", degree);
    hipError_t e = hipSetDevice(dev->ordinal);
    if (e != hipSuccess) return hip_fail(dev, e, "hipSetDevice");
    bv_graph *g = new bv_graph();
    g->dev = dev;
    g->dim = dim;
    g->metric = metric;
    g->degree = degree;
    e = hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete g;
        return hip_fail(dev, e, "hipStreamCreate");
    }
    *out = g;
    return BV_OK;
}

extern "C" int bv_graph_destroy(bv_graph *g) {
    if (!g) return BV_OK;
    (void)hipSetDevice(g->dev->ordinal);
    if (g->stream) {
        (void)hipStreamSynchronize(g->stream);
        (void)hipStreamDestroy(g->stream);
    }
    delete g;
    return BV_OK;
}

extern "C" int bv_graph_append(bv_graph *g, const float *data, uint64_t n_floats, uint64_t count) {
    if (!g) return fail(BV_E_INVALID, "null graph searcher");
    std::lock_guard<std::mutex> lock(g->mu);
    int rc = graph_live(g);
    if (rc) return rc;
    if (n_floats != count * g->dim)
        return fail(BV_E_INVALID, "expected %llu floats, got %llu", (unsigned long long)(count * g->dim),
                    (unsigned long long)n_floats);
    if (count == 0) return BV_OK;
    if (!data) return fail(BV_E_INVALID, "data is null");
    if (g->corpus_rows + count > 0xfffffffeull) return fail(BV_E_INVALID, "row count exceeds 2^32-2");
    const size_t rb = (size_t)g->dim * 4;
    HIPX(g->dev, g->corpus.ensure((g->corpus_rows + count) * rb, g->corpus_rows * rb, g->stream), "corpus buffer");
    HIPX(g->dev, hipMemcpyAsync(g->corpus.as<char>() + g->corpus_rows * rb, data, count * rb, hipMemcpyHostToDevice,
                                g->stream),
         "row upload");
    HIPX(g->dev, hipStreamSynchronize(g->stream), "append");
    g->corpus_rows += count;
    return BV_OK;
}

extern "C" int bv_graph_upload(bv_graph *g, const uint32_t *links, uint64_t rows) {
    if (!g) return fail(BV_E_INVALID, "null graph searcher");
    std::lock_guard<std::mutex> lock(g->mu);
    int rc = graph_live(g);
    if (rc) return rc;
    if (rows && !links) return fail(BV_E_INVALID, "links is null");
    if (rows > 0xfffffffeull) return fail(BV_E_INVALID, "row count exceeds 2^32-2");
    const size_t b = rows * g->degree * 4;
    HIPX(g->dev, g->graph.ensure(std::max<size_t>(b, 4), 0, g->stream), "graph buffer");
    if (b) HIPX(g->dev, hipMemcpyAsync(g->graph.p, links, b, hipMemcpyHostToDevice, g->stream), "upload");
    HIPX(g->dev, hipStreamSynchronize(g->stream), "graph upload");
    g->graph_rows = rows;
    return BV_OK;
}

extern "C" int bv_graph_search(bv_graph *g, const float *queries, uint32_t nq, uint32_t k, uint32_t ef,
                               uint32_t entry, uint32_t *rows, float *scores, uint32_t *n_out) {
    if (!g) return fail(BV_E_INVALID, "null graph searcher");
    std::lock_guard<std::mutex> lock(g->mu);
    int rc = graph_live(g);
    if (rc) return rc;
    if (nq == 0) return BV_OK;
    if (!queries || !n_out || (k && (!rows || !scores))) return fail(BV_E_INVALID, "null argument");
    if (g->corpus_rows == 0 || g->graph_rows == 0)
        return fail(BV_E_STATE, "graph search needs corpus rows and an uploaded adjacency");
    const uint32_t efA = std::min(std::max(ef, k), GRAPH_EF_CAP);
    const uint32_t kk = std::min(k, efA);
    if (kk == 0) {
        for (uint32_t i = 0; i < nq; i++) n_out[i] = 0;
        return BV_OK;
    }
    uint32_t seeds[8];
    const uint32_t ns = graph_seeds(entry, g->graph_rows, seeds);
    rc = graph_run(g, queries, nq, seeds, ns, efA, efA, kk, k, false);
    if (rc) return rc;
    HIPX(g->dev, hipMemcpyAsync(rows, g->out_rows.p, (size_t)nq * k * 4, hipMemcpyDeviceToHost, g->stream), "download");
    HIPX(g->dev, hipMemcpyAsync(scores, g->out_scores.p, (size_t)nq * k * 4, hipMemcpyDeviceToHost, g->stream),
         "download");
    HIPX(g->dev, hipMemcpyAsync(n_out, g->out_n.p, (size_t)nq * 4, hipMemcpyDeviceToHost, g->stream), "download");
    HIPX(g->dev, hipStreamSynchronize(g->stream), "graph search");
    return BV_OK;
}

extern "C" int bv_graph_search_beams(bv_graph *g, const float *queries, uint32_t nq, const uint32_t *entries,
                                     uint32_t n_entries, uint32_t ef, uint32_t iter_cap, float *beam_dist,
                                     uint32_t *beam_id) {
    if (!g) return fail(BV_E_INVALID, "null graph searcher");
    std::lock_guard<std::mutex> lock(g->mu);
    int rc = graph_live(g);
    if (rc) return rc;
    if (nq == 0) return BV_OK;
    if (!queries || !beam_dist || !beam_id || (n_entries && !entries)) return fail(BV_E_INVALID, "null argument");
    if (g->corpus_rows == 0 || g->graph_rows == 0)
        return fail(BV_E_STATE, "graph search needs corpus rows and an uploaded adjacency");
    if (ef == 0 || ef > GRAPH_EF_CAP) return fail(BV_E_INVALID, "ef must be 1..%u, got %u", GRAPH_EF_CAP, ef);
    rc = graph_run(g, queries, nq, entries, std::min(n_entries, 64u), ef, iter_cap, 0, 0, true);
    if (rc) return rc;
    const size_t b = (size_t)nq * GRAPH_EF_CAP * 4;
    HIPX(g->dev, hipMemcpyAsync(beam_dist, g->beam_d.p, b, hipMemcpyDeviceToHost, g->stream), "download");
    HIPX(g->dev, hipMemcpyAsync(beam_id, g->beam_i.p, b, hipMemcpyDeviceToHost, g->stream), "download");
    HIPX(g->dev, hipStreamSynchronize(g->stream), "graph search");
    return BV_OK;
}
