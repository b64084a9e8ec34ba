// gfx950 kernels of the IVF path: k-means build, list construction, probes.
//
//   ivf_copy_rows        row gathers (centroid init / re-seed, reservoir)
//   ivf_normalize_rows   normalizeRows (src/index/kmeans.ts:211-219)
//   ivf_assign<L>        nearest-centroid argmax over a tiled fp32 product
//                        (assign.ts / assignQ8.ts / assignQ4.ts / assignQ1.ts)
//   ivf_block_hist, ivf_list_bases, ivf_scan_offsets, ivf_scatter
//                        stable counting sort = the CSR lists
//                        (src/index/ivfquant.ts:297-305)
//   ivf_centroid_means   updateCentroids' f32 sums in row order + mean
//                        (src/index/kmeans.ts:177-209)
//   ivf_probe_scores     pickProbes' f64 four-way dot (ivfquant.ts:495-511);
//                        ivf_probe_scores_qb for batches of queries
//   ivf_probe_select     top-nprobe of the probe scores, best first, and the
//                        probed lists' total size
//   ivf_cand_offsets, ivf_gather_lists
//                        gatherCandidates (ivfquant.ts:513-527): the probed
//                        lists concatenated in probe order
#include "bv_kernels.h"
#include "bv_mfma.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bvk {

namespace {

__device__ __forceinline__ uint32_t ord_f32_i(float s) {
    s = s + 0.0f;
    uint32_t b = __float_as_uint(s);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
// larger = better: higher score, then lower index
__device__ __forceinline__ uint64_t idx_key(float s, uint32_t c) {
    return ((uint64_t)ord_f32_i(s) << 32) | (uint64_t)(0xffffffffu - c);
}

}  // namespace

// dst[dst_idx ? dst_idx[j] : j] = src[src_idx[j]], rows of `dim` floats.
__global__ __launch_bounds__(256) void ivf_copy_rows(IvfCopyArgs a) {
    const uint32_t j = blockIdx.x;
    if (j >= a.n) return;
    const float *s = a.src + (uint64_t)a.src_idx[j] * a.src_stride;
    float *d = a.dst + (uint64_t)(a.dst_idx ? a.dst_idx[j] : j) * a.dst_stride;
    for (uint32_t i = threadIdx.x; i < a.dim; i += blockDim.x) d[i] = s[i];
}

// normalizeRows: s = sequential f64 sum of m*m (each product exact in f64),
// inv = 1 / (sqrt(s) || 1), m = f32(m * inv).  One thread per row.
__global__ __launch_bounds__(256) void ivf_normalize_rows(float *m, uint32_t rows, uint32_t dim, uint32_t stride) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    float *v = m + (uint64_t)r * stride;
    double s = 0.0;
    for (uint32_t i = 0; i < dim; ++i) s = fma((double)v[i], (double)v[i], s);
    const double sq = sqrt(s);
    const double inv = 1.0 / (sq != 0.0 ? sq : 1.0);
    for (uint32_t i = 0; i < dim; ++i) v[i] = (float)((double)v[i] * inv);
}

// The same with one wave per row: the row staged in LDS with coalesced
// loads, lane 0's sequential f64 sum (element order) over it, and the scaled
// row written by every lane.  The thread-per-row form above waits on one
// scattered load per element (0.47 ms for 4096 x 1024 centroids).
// Up to four waves per workgroup, within 64 KB of LDS.
constexpr uint32_t NRM_MAX_DIM = 16384;
__global__ __launch_bounds__(256) void ivf_normalize_rows_w(float *m, uint32_t rows, uint32_t dim, uint32_t stride) {
    extern __shared__ float nbuf[];  // waves x dim
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t r = blockIdx.x * (blockDim.x >> 6) + wave;
    if (r >= rows) return;  // wave-uniform; the kernel has no workgroup barrier
    float *v = m + (uint64_t)r * stride;
    float *b = nbuf + (size_t)wave * dim;
    for (uint32_t i = lane; i < dim; i += 64) b[i] = v[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    double sum = 0.0;
    if (lane == 0) {
#pragma unroll 16
        for (uint32_t i = 0; i < dim; ++i) sum = fma((double)b[i], (double)b[i], sum);
    }
    sum = __shfl(sum, 0);
    const double sq = sqrt(sum);
    const double inv = 1.0 / (sq != 0.0 ? sq : 1.0);
    for (uint32_t i = lane; i < dim; i += 64) v[i] = (float)((double)b[i] * inv);
}

// ---------------------------------------------------------------- assign --
// Rows x centroids product in 128 x 128 tiles (256 threads, 8 x 8 outputs
// each, fp32 fused multiply-add over the dimension in order), argmax per row
// with the lowest centroid index winning ties.  The row loader dequantizes
// codes exactly as the reference's assign kernels do before the product.
// SPLIT: workgroup (x, y) takes row tile x against centroid tile y only and
// folds its rows' best (score, ~centroid) keys into a.keys with a 64-bit
// atomic maximum; the keys are unique, so the maximum over the tiles is the
// fold of the one-workgroup form, whatever the order.  ivf_assign_finish
// turns the keys into centroids.
constexpr int AT = 128;  // rows and centroids per tile
constexpr int AK = 8;    // dimension chunk per LDS stage

// dq8: for int8 codes, max(f32(b / 127), -1) of every byte b (the
// correctly rounded quotient, as the per-element division gives it), in LDS.
template <int BITS> struct RowLoader;
template <> struct RowLoader<0> {  // fp32 rows
    static __device__ __forceinline__ float get(const IvfAssignArgs &a, uint64_t r, uint32_t i, const float *) {
        return a.rows[r * a.row_stride + i];
    }
};
template <> struct RowLoader<8> {  // unpack4x8snorm(b) * scale
    static __device__ __forceinline__ float get(const IvfAssignArgs &a, uint64_t r, uint32_t i, const float *dq8) {
        const uint32_t w = a.codes[r * a.words_per_row + (i >> 2)];
        return dq8[(w >> (8 * (i & 3))) & 0xffu] * a.scales[r];
    }
};
template <> struct RowLoader<4> {  // signed nibble * (scale * f32(1/7))
    static __device__ __forceinline__ float get(const IvfAssignArgs &a, uint64_t r, uint32_t i, const float *) {
        const uint32_t w = a.codes[r * a.words_per_row + (i >> 3)];
        const int32_t n = (int32_t)((w >> (4 * (i & 7))) & 0xfu);
        const float inv7 = a.scales[r] * (1.0f / 7.0f);
        return (float)(n - 16 * (n >> 3)) * inv7;
    }
};
template <> struct RowLoader<1> {  // sign bits as +-1 (the scale multiplies the sum)
    static __device__ __forceinline__ float get(const IvfAssignArgs &a, uint64_t r, uint32_t i, const float *) {
        const uint32_t w = a.codes[r * a.words_per_row + (i >> 5)];
        return ((w >> (i & 31)) & 1u) ? 1.0f : -1.0f;
    }
};

template <int BITS, bool SPLIT>
__global__ __launch_bounds__(256) void ivf_assign(IvfAssignArgs a) {
    __shared__ float As[AK][AT + 4];
    __shared__ float Bs[AK][AT + 4];
    __shared__ float dq8[BITS == 8 ? 256 : 1];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const uint64_t r0 = (uint64_t)blockIdx.x * AT;
    if constexpr (BITS == 8) {
        dq8[tid] = fmaxf((float)(int8_t)(uint8_t)tid / 127.0f, -1.0f);
        __syncthreads();
    }
    uint64_t best[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) best[i] = 0;
    const uint32_t cbeg = SPLIT ? blockIdx.y * AT : 0u, cend = SPLIT ? cbeg + AT : a.nlist;
    for (uint32_t c0 = cbeg; c0 < cend && c0 < a.nlist; c0 += AT) {
        float acc[8][8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[i][j] = 0.0f;
        for (uint32_t k0 = 0; k0 < a.dim; k0 += AK) {
            // stage AK x AT rows and centroids: 1024 values each, 4 per thread
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int e = tid + t * 256;
                const int kk = e % AK, rr = e / AK;  // consecutive lanes read consecutive elements of a row
                const uint32_t k = k0 + kk;
                const uint64_t r = r0 + rr;
                As[kk][rr] = (r < a.n && k < a.dim) ? RowLoader<BITS>::get(a, r, k, dq8) : 0.0f;
                const uint32_t c = c0 + rr;
                Bs[kk][rr] = (c < a.nlist && k < a.dim) ? a.centroids[(uint64_t)c * a.cen_stride + k] : 0.0f;
            }
            __syncthreads();
#pragma unroll
            for (int kk = 0; kk < AK; ++kk) {
                float av[8], bv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) av[i] = As[kk][ty + 16 * i];
#pragma unroll
                for (int j = 0; j < 8; ++j) bv[j] = Bs[kk][tx + 16 * j];
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
            }
            __syncthreads();
        }
        // fold this tile into each row's running best
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint64_t b = best[i];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t c = c0 + tx + 16 * j;
                if (c < a.nlist) {
                    const float s = BITS == 1 ? acc[i][j] * a.scales[(r0 + ty + 16 * i) < a.n ? r0 + ty + 16 * i : 0]
                                              : acc[i][j];
                    const uint64_t key = idx_key(s, c);
                    b = key > b ? key : b;
                }
            }
            best[i] = b;
        }
    }
    // reduce over the 16 threads sharing each row (consecutive lanes)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint64_t b = best[i];
#pragma unroll
        for (int s = 1; s < 16; s <<= 1) {
            const uint64_t o = ((uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)(b >> 32), s) << 32) |
                               (uint32_t)__shfl_xor((int)(uint32_t)b, s);
            b = o > b ? o : b;
        }
        const uint64_t r = r0 + ty + 16 * i;
        if (tx == 0 && r < a.n) {
            if constexpr (SPLIT) atomicMax((unsigned long long *)&a.keys[r], (unsigned long long)b);
            else a.out[r] = 0xffffffffu - (uint32_t)b;
        }
    }
}

__global__ __launch_bounds__(256) void ivf_assign_keys_zero(uint64_t *keys, uint64_t n) {
    const uint64_t r = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (r < n) keys[r] = 0;
}

__global__ __launch_bounds__(256) void ivf_assign_finish(const uint64_t *keys, uint64_t n, uint32_t *out) {
    const uint64_t r = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (r < n) out[r] = 0xffffffffu - (uint32_t)keys[r];
}

// ----------------------------------------------------------------- lists --
// Stable counting sort of rows by cluster: per-block histograms, per-cluster
// running bases over the blocks, cluster offsets, then a scatter where each
// row's rank inside its block counts the earlier rows of the same cluster.
constexpr int LB = 1024;  // rows per block

__global__ __launch_bounds__(256) void ivf_block_hist(const uint32_t *assign, uint64_t n, uint32_t nlist,
                                                      uint32_t *hist) {
    extern __shared__ uint32_t h[];
    for (uint32_t c = threadIdx.x; c < nlist; c += blockDim.x) h[c] = 0;
    __syncthreads();
    const uint64_t r0 = (uint64_t)blockIdx.x * LB;
    for (uint32_t j = threadIdx.x; j < LB; j += blockDim.x)
        if (r0 + j < n) atomicAdd(&h[assign[r0 + j]], 1u);
    __syncthreads();
    for (uint32_t c = threadIdx.x; c < nlist; c += blockDim.x) hist[(uint64_t)blockIdx.x * nlist + c] = h[c];
}

// base[b][c] = sum of hist[b'][c] for b' < b; totals[c] = the full sum.
__global__ __launch_bounds__(256) void ivf_list_bases(const uint32_t *hist, uint32_t nblk, uint32_t nlist,
                                                      uint32_t *base, uint32_t *totals) {
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= nlist) return;
    uint32_t run = 0;
    uint32_t b = 0;
    for (; b + 8 <= nblk; b += 8) {
        uint32_t h[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) h[u] = hist[(uint64_t)(b + u) * nlist + c];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            base[(uint64_t)(b + u) * nlist + c] = run;
            run += h[u];
        }
    }
    for (; b < nblk; ++b) {
        base[(uint64_t)b * nlist + c] = run;
        run += hist[(uint64_t)b * nlist + c];
    }
    totals[c] = run;
}

// offset[0] = 0, offset[c+1] = offset[c] + totals[c] (one workgroup).
__global__ __launch_bounds__(256) void ivf_scan_offsets(const uint32_t *totals, uint32_t nlist, uint32_t *offset) {
    __shared__ uint32_t part[256];
    const uint32_t tid = threadIdx.x;
    const uint32_t per = (nlist + 255) / 256, c0 = tid * per;
    uint32_t s = 0;
    for (uint32_t c = c0; c < c0 + per && c < nlist; ++c) s += totals[c];
    part[tid] = s;
    __syncthreads();
    if (tid == 0) {
        uint32_t run = 0;
        for (int t = 0; t < 256; ++t) {
            const uint32_t v = part[t];
            part[t] = run;
            run += v;
        }
        offset[nlist] = run;
    }
    __syncthreads();
    uint32_t run = part[tid];
    for (uint32_t c = c0; c < c0 + per && c < nlist; ++c) {
        offset[c] = run;
        run += totals[c];
    }
}

__global__ __launch_bounds__(256) void ivf_scatter(const uint32_t *assign, uint64_t n, uint32_t nlist,
                                                   const uint32_t *offset, const uint32_t *base, uint32_t *rows_out) {
    __shared__ uint32_t cl[LB];
    const uint64_t r0 = (uint64_t)blockIdx.x * LB;
    for (uint32_t j = threadIdx.x; j < LB; j += blockDim.x) cl[j] = r0 + j < n ? assign[r0 + j] : 0xffffffffu;
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < LB; j += blockDim.x) {
        if (r0 + j >= n) continue;
        const uint32_t c = cl[j];
        uint32_t rank = 0;
        for (uint32_t i = 0; i < j; ++i) rank += cl[i] == c ? 1u : 0u;
        rows_out[offset[c] + base[(uint64_t)blockIdx.x * nlist + c] + rank] = (uint32_t)(r0 + j);
    }
}

// updateCentroids' mean: thread (c, i) adds column i of its cluster's rows in
// row order in f32 (the reference's Float32Array `+=`), then stores
// f32(sum * (1 / count)) with the reciprocal in f64.  Empty clusters are
// left for the host's re-seed.
__global__ __launch_bounds__(256) void ivf_centroid_means(const float *sample, uint32_t stride, uint32_t dim,
                                                          const uint32_t *offset, const uint32_t *list_rows,
                                                          uint32_t nlist, float *centroids, uint32_t cen_stride) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t c = (uint32_t)(t / dim), i = (uint32_t)(t % dim);
    if (c >= nlist) return;
    const uint32_t b = offset[c], e = offset[c + 1];
    if (b == e) return;
    float s = 0.0f;
    for (uint32_t j = b; j < e; ++j) s = s + sample[(uint64_t)list_rows[j] * stride + i];
    const double inv = 1.0 / (double)(e - b);
    centroids[(uint64_t)c * cen_stride + i] = (float)((double)s * inv);
}

// ---------------------------------------------------------------- probes --
// pickProbes: four f64 accumulators over the strided elements 4j+m (each
// product of two f32 exact in f64), a0 + a1 + a2 + a3, stored f32.  Four
// lanes per centroid, 16 centroids per one-wave workgroup; grid
// (ceil(nlist/16), nq).  The query sits in LDS and each lane keeps 32
// centroid loads in flight, so a 768-dim dot is six round trips to memory.
// P is at most PROBE_MAX_DIM (the scans' own limit: 4096 floats per row).
constexpr uint32_t PROBE_MAX_DIM = 4096;
__global__ __launch_bounds__(64) void ivf_probe_scores(IvfProbeArgs a) {
    extern __shared__ float qs[];  // the query, P floats
    const uint32_t qi = blockIdx.y, g = threadIdx.x >> 2, m = threadIdx.x & 3;
    const float *rq = a.qrot + (uint64_t)qi * a.P;
    for (uint32_t i = threadIdx.x; i < a.P; i += 64) qs[i] = rq[i];
    __syncthreads();
    const uint32_t c = blockIdx.x * 16 + g;
    const uint32_t vec = a.P & ~3u;
    const float *cen = a.centroids + (uint64_t)(c < a.nlist ? c : 0) * a.P;
    double acc = 0.0;
    if (c < a.nlist) {
        uint32_t i = m;
        for (; i + 124 < vec; i += 128) {  // summed in element order after the loads land
            float cv[32];
#pragma unroll
            for (int u = 0; u < 32; ++u) cv[u] = cen[i + 4 * u];
#pragma unroll
            for (int u = 0; u < 32; ++u) acc = fma((double)cv[u], (double)qs[i + 4 * u], acc);
        }
        for (; i + 28 < vec; i += 32) {
            float cv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) cv[u] = cen[i + 4 * u];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = fma((double)cv[u], (double)qs[i + 4 * u], acc);
        }
        for (; i < vec; i += 4) acc = fma((double)cen[i], (double)qs[i], acc);
    }
    const double a1 = __shfl_down(acc, 1, 4), a2 = __shfl_down(acc, 2, 4), a3 = __shfl_down(acc, 3, 4);
    if (m == 0 && c < a.nlist) {
        double s = ((acc + a1) + a2) + a3;
        for (uint32_t i = vec; i < a.P; ++i) s = fma((double)cen[i], (double)qs[i], s);  // the fp32 IVF tail
        a.scores[(uint64_t)qi * a.nlist + c] = (float)s;
    }
}

// Query batches: eight queries per 256-thread workgroup, CT centroids per
// four lanes (64 x CT centroids per workgroup), each centroid load feeding
// eight chains and each query element read from LDS feeding CT chains, in
// the same element order as ivf_probe_scores, so the scores are identical.
// The queries sit in LDS as f64, element 4j+m of query q at
// (4q+m)*(P/4+1)+j (the +1 keeps the four chains' reads in distinct banks).
// P a multiple of 128, at most 1024.
constexpr uint32_t PROBE_QB = 8;
constexpr uint32_t PROBE_QB_MAX_DIM = 1024;
template <int CT>
__global__ __launch_bounds__(256) void ivf_probe_scores_qb(IvfProbeArgs a, uint32_t nq) {
    extern __shared__ double qd[];
    const uint32_t tid = threadIdx.x, g = tid >> 2, m = tid & 3, q0 = blockIdx.y * PROBE_QB;
    const uint32_t nqb = nq - q0 < PROBE_QB ? nq - q0 : PROBE_QB;
    const uint32_t P = a.P, S = P / 4 + 1;
#pragma unroll
    for (uint32_t qq = 0; qq < PROBE_QB; ++qq) {
        const float *rq = a.qrot + (uint64_t)(q0 + (qq < nqb ? qq : 0)) * P;
        for (uint32_t e = tid; e < P; e += 256) qd[(qq * 4 + (e & 3)) * S + (e >> 2)] = (double)rq[e];
    }
    __syncthreads();
    const float *cen[CT];
    bool live[CT];
#pragma unroll
    for (int j = 0; j < CT; ++j) {
        const uint32_t c = blockIdx.x * 64 * CT + 64 * j + g;
        live[j] = c < a.nlist;
        cen[j] = a.centroids + (uint64_t)(live[j] ? c : 0) * P;
    }
    double acc[CT][PROBE_QB];
#pragma unroll
    for (int j = 0; j < CT; ++j)
#pragma unroll
        for (uint32_t qq = 0; qq < PROBE_QB; ++qq) acc[j][qq] = 0.0;
    constexpr int U = CT == 1 ? 32 : 16;  // elements i + 4u, u < U, per round trip
    for (uint32_t i = m; i < P; i += 4 * U) {  // P a multiple of 128: every element below P
        float cv[CT][U];
#pragma unroll
        for (int j = 0; j < CT; ++j)
#pragma unroll
            for (int u = 0; u < U; ++u) cv[j][u] = cen[j][i + 4 * u];
        const double *qm = qd + m * S + (i >> 2);
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (uint32_t qq = 0; qq < PROBE_QB; ++qq) {
                const double qv = qm[qq * 4 * S + u];
#pragma unroll
                for (int j = 0; j < CT; ++j) acc[j][qq] = fma((double)cv[j][u], qv, acc[j][qq]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < CT; ++j) {
        const uint32_t c = blockIdx.x * 64 * CT + 64 * j + g;
#pragma unroll
        for (uint32_t qq = 0; qq < PROBE_QB; ++qq) {
            const double a1 = __shfl_down(acc[j][qq], 1, 4), a2 = __shfl_down(acc[j][qq], 2, 4),
                         a3 = __shfl_down(acc[j][qq], 3, 4);
            if (m == 0 && live[j] && qq < nqb)
                a.scores[(uint64_t)(q0 + qq) * a.nlist + c] = (float)(((acc[j][qq] + a1) + a2) + a3);
        }
    }
}

// Best nprobe centroids of one query, best first (score desc, index asc).
// One workgroup per query; keys are unique.  A bound: the np-th best of a
// strided sample of 256 keys (at least np keys are at or above it, the
// sample's own); the keys at or above it are gathered and ranked.  When
// the bound admits too many keys (or np exceeds the sample), a bisection on
// the 64-bit keys finds the np-th key instead.
constexpr uint32_t PROBE_RANK_CAP = 1024;
__global__ __launch_bounds__(256) void ivf_probe_select(IvfProbeArgs a) {
    extern __shared__ uint64_t pk[];  // nlist keys, then up to nlist + 16 selected keys
    uint64_t *sel = pk + a.nlist;
    __shared__ uint64_t smp[256];
    __shared__ uint32_t cnt_s[4];
    __shared__ uint64_t tot_s[4];
    __shared__ uint32_t nsel;
    __shared__ uint64_t s_bound, smp_b1;
    const uint32_t qi = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *sc = a.scores + (uint64_t)qi * a.nlist;
#pragma unroll 8
    for (uint32_t c = tid; c < a.nlist; c += 256) pk[c] = idx_key(sc[c], c);
    if (tid == 0) {
        nsel = 0;
        s_bound = 0;
    }
    __syncthreads();
    const uint32_t np = a.nprobe < a.nlist ? a.nprobe : a.nlist;
    uint64_t lo = 0, hi = ~0ull;  // count(>= lo) >= np > count(>= hi) (hi unreachable)
    bool bisect = np < a.nlist;
    if (bisect && a.nlist >= 512 && np <= 64) {
        // Bounds from a strided sample of 256 keys: the sample of rank
        // np - 1 has at least np keys at or above it (about stride * np);
        // the one of rank k1 about 4 np, which keeps the all-pairs ranking
        // below small, and fewer than np only rarely (then the first).
        const uint32_t stride = a.nlist / 256;
        smp[tid] = pk[tid * stride];
        __syncthreads();
        const uint64_t mine = smp[tid];
        uint32_t r = 0;
#pragma unroll 16
        for (uint32_t j = 0; j < 256; ++j) r += smp[j] > mine ? 1u : 0u;
        uint32_t k1 = (4 * np + stride - 1) / stride;
        k1 = k1 > 0 ? k1 - 1 : 0;
        if (k1 > np - 1) k1 = np - 1;
        if (r == np - 1) s_bound = mine;
        if (r == k1) smp_b1 = mine;
        __syncthreads();
        for (int pass = 0; pass < 2; ++pass) {
            const uint64_t bound = pass == 0 ? smp_b1 : s_bound;
            uint32_t c = 0;
#pragma unroll 8
            for (uint32_t j = tid; j < a.nlist; j += 256) c += pk[j] >= bound ? 1u : 0u;
#pragma unroll
            for (int s = 1; s < 64; s <<= 1) c += __shfl_xor(c, s);
            if (lane == 0) cnt_s[wave] = c;
            __syncthreads();
            const uint32_t tot = cnt_s[0] + cnt_s[1] + cnt_s[2] + cnt_s[3];
            __syncthreads();
            if (tot >= np && tot <= PROBE_RANK_CAP) {
                lo = bound;  // rank the tot >= np keys at or above the bound below
                bisect = false;
                break;
            }
            if (k1 == np - 1) break;  // (the same bound twice)
        }
    }
    if (bisect) {
        for (int it = 0; it < 64 && hi - lo > 1; ++it) {
            const uint64_t mid = lo + ((hi - lo) >> 1);
            uint32_t c = 0;
            for (uint32_t j = tid; j < a.nlist; j += 256) c += pk[j] >= mid ? 1u : 0u;
#pragma unroll
            for (int s = 1; s < 64; s <<= 1) c += __shfl_xor(c, s);
            if (lane == 0) cnt_s[wave] = c;
            __syncthreads();
            const uint32_t tot = cnt_s[0] + cnt_s[1] + cnt_s[2] + cnt_s[3];
            __syncthreads();
            if (tot >= np) lo = mid;
            else hi = mid;
        }
    }
    // keys >= lo: exactly np of them when np < nlist (unique keys), else all
    for (uint32_t j = tid; j < a.nlist; j += 256)
        if (pk[j] >= lo) sel[atomicAdd(&nsel, 1u)] = pk[j];
    __syncthreads();
    // zeros pad the selection to a multiple of 16 (no key is 0: its low
    // word is 0xffffffff - c with c < nlist), so the rank reads run 16 wide
    const uint32_t m = nsel, mp = (m + 15) & ~15u;
    if (m + tid < mp) sel[m + tid] = 0;
    __syncthreads();
    uint64_t size = 0;  // candidates in this thread's probed lists
    for (uint32_t j = tid; j < m; j += 256) {
        const uint64_t k = sel[j];
        uint32_t r = 0;
        for (uint32_t i = 0; i < mp; i += 16) {
#pragma unroll
            for (uint32_t u = 0; u < 16; ++u) r += sel[i + u] > k ? 1u : 0u;
        }
        if (r < np) {
            const uint32_t c = 0xffffffffu - (uint32_t)k;
            a.probes[(uint64_t)qi * a.nprobe + r] = c;
            if (a.offset) size += a.offset[c + 1] - a.offset[c];
        }
    }
    if (a.offset) {  // the query's candidate count (gatherCandidates' total)
#pragma unroll
        for (int s = 1; s < 64; s <<= 1) size += __shfl_xor(size, s);
        if (lane == 0) tot_s[wave] = size;
        __syncthreads();
        if (tid == 0) {
            const uint64_t t = tot_s[0] + tot_s[1] + tot_s[2] + tot_s[3];
            a.totals[qi] = t;
            if (gridDim.x == 1) {  // one query: its offsets need no prefix pass
                a.cand_off[0] = 0;
                a.cand_off[1] = t;
            }
        }
    }
}

// cand_off[q] = sum of totals before q (one workgroup): each thread sums a
// run of queries, a scan over the 256 runs (within waves, then the four
// wave totals) places them.
__global__ __launch_bounds__(256) void ivf_cand_offsets(const uint64_t *totals, uint32_t nq, uint64_t *cand_off) {
    __shared__ uint64_t wsum[4];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t per = (nq + 255) / 256, q0 = tid * per;
    uint64_t s = 0;
    for (uint32_t q = q0; q < q0 + per && q < nq; ++q) s += totals[q];
    uint64_t x = s;  // inclusive scan within the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint64_t y = __shfl_up(x, d);
        if (lane >= (uint32_t)d) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    uint64_t run = x - s;
    for (uint32_t w = 0; w < wave; ++w) run += wsum[w];
    if (tid == 255) cand_off[nq] = run + s;
    for (uint32_t q = q0; q < q0 + per && q < nq; ++q) {
        cand_off[q] = run;
        run += totals[q];
    }
}

// gatherCandidates: the probed lists in probe order, rows ascending within
// a list.  One workgroup per (probed list, query): its position is the
// query's offset plus the sizes of the lists probed before it.
__global__ __launch_bounds__(256) void ivf_gather_lists(const uint32_t *probes, uint32_t nprobe,
                                                        const uint32_t *offset, const uint32_t *list_rows,
                                                        const uint64_t *cand_off, uint32_t *cand) {
    __shared__ uint64_t part[4];
    const uint32_t p = blockIdx.x, qi = blockIdx.y, tid = threadIdx.x;
    const uint32_t *pr = probes + (uint64_t)qi * nprobe;
    uint64_t before = 0;
    for (uint32_t i = tid; i < p; i += 256) {
        const uint32_t c = pr[i];
        before += offset[c + 1] - offset[c];
    }
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) before += __shfl_xor(before, s);
    if ((tid & 63) == 0) part[tid >> 6] = before;
    __syncthreads();
    const uint64_t w = cand_off[qi] + part[0] + part[1] + part[2] + part[3];
    const uint32_t c = pr[p];
    const uint32_t b = offset[c], e = offset[c + 1];
    for (uint32_t j = tid; j < e - b; j += 256) cand[w + j] = list_rows[b + j];
}

// ------------------------------------------------------------- launchers --
hipError_t ivf_launch_copy_rows(const IvfCopyArgs &a, hipStream_t s) {
    if (a.n == 0) return hipSuccess;
    hipLaunchKernelGGL(ivf_copy_rows, dim3(a.n), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t ivf_launch_normalize(float *m, uint32_t rows, uint32_t dim, uint32_t stride, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    if (dim >= 1 && dim <= NRM_MAX_DIM) {
        const uint32_t waves = std::max<uint32_t>(1, std::min<uint32_t>(4, NRM_MAX_DIM / dim));
        hipLaunchKernelGGL(ivf_normalize_rows_w, dim3((rows + waves - 1) / waves), dim3(waves * 64),
                           (size_t)waves * dim * 4, s, m, rows, dim, stride);
    } else
        hipLaunchKernelGGL(ivf_normalize_rows, dim3((rows + 255) / 256), dim3(256), 0, s, m, rows, dim, stride);
    return hipGetLastError();
}

template <bool SPLIT>
static hipError_t assign_bits(const IvfAssignArgs &a, int bits, dim3 grid, hipStream_t s) {
    switch (bits) {
    case 0: hipLaunchKernelGGL((ivf_assign<0, SPLIT>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((ivf_assign<8, SPLIT>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((ivf_assign<4, SPLIT>), grid, dim3(256), 0, s, a); break;
    case 1: hipLaunchKernelGGL((ivf_assign<1, SPLIT>), grid, dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t ivf_launch_assign(const IvfAssignArgs &a, int bits, hipStream_t s) {
    if (a.n == 0) return hipSuccess;
    const uint32_t tiles = (uint32_t)((a.n + AT - 1) / AT);
    if (!ivf_assign_split(a.n)) return assign_bits<false>(a, bits, dim3(tiles), s);
    if (!a.keys) return hipErrorInvalidValue;
    const uint32_t flat = (uint32_t)((a.n + 255) / 256);
    hipLaunchKernelGGL(ivf_assign_keys_zero, dim3(flat), dim3(256), 0, s, a.keys, a.n);
    hipError_t e = assign_bits<true>(a, bits, dim3(tiles, (a.nlist + AT - 1) / AT), s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(ivf_assign_finish, dim3(flat), dim3(256), 0, s, a.keys, a.n, a.out);
    return hipGetLastError();
}

// ------------------------------------------- assign on the matrix cores --
// The assignment of int8 codes (every row of a build, the rows of an
// incremental append) on v_mfma_i32_32x32x32_i8, with ivf_assign's exact
// arithmetic kept for the rows whose winner the matrix pass cannot decide.
//
// ivf_cen_levels splits each centroid into two int8 levels,
// c = s1 q1 + s2 q2 + e (s1 = max|c| / 127, s2 = max|c - s1 q1| / 127, e
// exact in f64).  For a row with codes b and scale sc > 0 the exact score
// s(c) is the fmaf chain over x_k = f32(f32(b_k / 127) sc) and c_k, and
// v(c) = s1 (b.q1) + s2 (b.q2) with exact int32 dots.  With u = 2^-24:
//   |s(c) - (sc / 127) v(c)| <= (sc / 127) |b| (|e_c| + (gamma_P + 3u) |c|)
// (the chain's P roundings, the two roundings of each x_k, Cauchy-Schwarz on
// the level residual), and the pass's f32 value of v is within 4u |b| |c| of
// v.  So with M = max over centroids of |e_c| + (gamma_P + 7u) |c|, the
// exact winner's f32 v is within W = 2 |b| M of the row's largest: a row
// with one centroid in that window is decided.  The others go to the queue:
// rows with several centroids in the window (their candidates), and rows
// whose window may hold more than a lane keeps, whose scale is not a
// positive finite number, or with a byte -128 (decoded as -1, outside the
// levels' arithmetic), for which every centroid is re-scored.

// Each lane keeps its row's best IVF_MQ_KEEP values over its half of the
// centroids.
constexpr int IVF_MQ_KEEP = 4;
constexpr int IVF_MA_WAVES = 8;                  // waves per workgroup, 32 rows each
constexpr int IVF_MA_ROWS = IVF_MA_WAVES * 32;

namespace {

__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ double wave_max_d(double v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v = fmax(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t b) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t x = ((uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)(b >> 32), o) << 32) |
                           (uint32_t)__shfl_xor((int)(uint32_t)b, o);
        b = x > b ? x : b;
    }
    return b;
}

// One wave per centroid (c < nlist rounded up to 32; the padding centroids
// get zero levels): the two int8 levels (lev[c][0..1][P]), their scales
// (ls[c][0..1]) and the bound term m_c, folded into words[0] with an atomic
// maximum of its f32 bits (a non-finite centroid makes it +inf: every row is
// then re-scored exactly).  P is a multiple of 64, at most 1024.
__global__ __launch_bounds__(64) void ivf_cen_levels(const float *cen, uint32_t stride, uint32_t nlist, uint32_t P,
                                                      int8_t *lev, float *ls, uint32_t *words) {
    const uint32_t c = blockIdx.x, lane = threadIdx.x;
    int8_t *q1 = lev + (uint64_t)c * 2 * P, *q2 = q1 + P;
    if (c >= nlist) {
        for (uint32_t i = lane; i < P; i += 64) q1[i] = q2[i] = 0;
        if (lane == 0) ls[2 * c] = ls[2 * c + 1] = 0.0f;
        return;
    }
    const uint32_t per = P / 64;
    const float *v = cen + (uint64_t)c * stride;
    float x[16];
    bool finite = true;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        x[j] = (uint32_t)j < per ? v[lane + 64 * j] : 0.0f;
        finite = finite && (fabsf(x[j]) < __builtin_inff());
    }
    float m1 = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) m1 = fmaxf(m1, fabsf(x[j]));
    m1 = wave_max_f(m1);
    const float s1 = m1 / 127.0f;
    double r1[16];
    double m2 = 0.0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        float q = s1 > 0.0f ? rintf(x[j] / s1) : 0.0f;
        q = fminf(fmaxf(q, -127.0f), 127.0f);
        if ((uint32_t)j < per) q1[lane + 64 * j] = (int8_t)(int)q;
        r1[j] = (double)x[j] - (double)s1 * (double)q;  // exact: at most 32 significant bits
        m2 = fmax(m2, fabs(r1[j]));
    }
    m2 = wave_max_d(m2);
    const float s2 = (float)(m2 / 127.0);
    double ee = 0.0, cc = 0.0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        double q = s2 > 0.0f ? rint(r1[j] / (double)s2) : 0.0;
        q = fmin(fmax(q, -127.0), 127.0);
        if ((uint32_t)j < per) q2[lane + 64 * j] = (int8_t)(int)q;
        const double e = r1[j] - (double)s2 * q;  // exact
        ee = fma(e, e, ee);
        cc = fma((double)x[j], (double)x[j], cc);
    }
    ee = wave_sum_d(ee);
    cc = wave_sum_d(cc);
    const bool all_finite = __all(finite) && s2 == s2;
    if (lane == 0) {
        ls[2 * c] = s1;
        ls[2 * c + 1] = s2;
        const double u = 0x1p-24, gamma = (double)P * u / (1.0 - (double)P * u);
        // (the sums' and square roots' own rounding: well inside 1e-12)
        const double m = (sqrt(ee) + (gamma + 7.0 * u) * sqrt(cc)) * (1.0 + 1e-12);
        const float mf = all_finite ? (float)(m * (1.0 + 0x1p-20)) : __builtin_inff();  // rounded up
        atomicMax(&words[0], __float_as_uint(mf));
    }
}

__global__ __launch_bounds__(64) void ivf_mfma_words_zero(uint32_t *words) {
    if (threadIdx.x < 2) words[threadIdx.x] = 0;
}

// The matrix pass: a workgroup of IVF_MA_WAVES waves takes 256 rows; each
// wave holds its 32 rows' codes in registers (lane l: row l % 32, units
// 2 st + l / 32 -- the B operand of K step st) for the whole launch, and the
// centroids' levels stream through four LDS buffers in half tiles (32
// centroids, one level), three in flight while one is multiplied.  The
// output of a 32 x 32 MFMA gives lane (h, c) the 16 centroids 8 (r / 4) +
// 4 h + r % 4 of its row c.
template <int S>
__global__ __launch_bounds__(IVF_MA_WAVES * 64) void ivf_assign_mfma(IvfAssignArgs a, IvfMfmaScratch m,
                                                                      uint32_t tiles) {
    constexpr uint32_t U = 2 * S;                    // 16-byte units per centroid level
    constexpr uint32_t RS = U + 1;                   // LDS stride in units (one unit of padding)
    constexpr uint32_t PER = 32 / IVF_MA_WAVES;      // centroid rows each wave loads per half tile
    __shared__ v4i tb0[32 * RS], tb1[32 * RS], tb2[32 * RS], tb3[32 * RS];
    __shared__ __attribute__((aligned(16))) float sb0[32], sb1[32], sb2[32], sb3[32];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = lane >> 5, c = lane & 31;
    const uint64_t row = (uint64_t)blockIdx.x * IVF_MA_ROWS + (uint64_t)wave * 32 + c;
    const uint64_t rowc = row < a.n ? row : a.n - 1;
    const v4i *rsrc = (const v4i *)(a.codes + rowc * a.words_per_row);
    v4i br[S];
#pragma unroll
    for (int st = 0; st < S; ++st) br[st] = rsrc[2 * st + h];
    const uint32_t nh = 2 * tiles;

    auto load_half = [&](uint32_t j, v4i *tl, float *sb) {
        const uint32_t t = j >> 1, l = j & 1;
        const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
        const uint32_t lb = lds_addr(&tl[wv * PER * RS]);
        if ((uint32_t)lane < U) {
#pragma unroll
            for (uint32_t jj = 0; jj < PER; ++jj) {
                const uint64_t cen = (uint64_t)t * 32 + wv * PER + jj;
                lds_dma16((const v4i *)(m.lev + (cen * 2 + l) * (uint64_t)(U * 16)) + lane, lb + jj * RS * 16);
            }
        }
        if (wv == 0 && lane < 32) lds_dma4(m.ls + ((uint64_t)t * 32 + lane) * 2 + l, lds_addr(sb));
    };

    float p[16];                 // the current tile's level-one terms s1 * D1
    float tv[IVF_MQ_KEEP];       // the lane's best values, descending, and their centroids
    uint32_t ti[IVF_MQ_KEEP];
#pragma unroll
    for (int i = 0; i < IVF_MQ_KEEP; ++i) tv[i] = -__builtin_inff(), ti[i] = 0xffffffffu;
    auto run_half = [&](uint32_t j, const v4i *tl, const float *sb, v4i *ntl, float *nsb) {
        // this wave's loads of half j have landed (those of j + 1 and j + 2,
        // issued after them, may still run: vmcnt counts in issue order)
        const uint32_t after = (nh - 1 - j) < 2 ? (nh - 1 - j) : 2;
        if (wave == 0) {
            if (after == 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * (PER + 1)));
            else if (after == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER + 1));
            else __builtin_amdgcn_s_waitcnt(0);
        } else {
            if (after == 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PER));
            else if (after == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER));
            else __builtin_amdgcn_s_waitcnt(0);
        }
        // every wave's loads of half j have landed and every wave is done with
        // half j - 1's buffer, which half j + 3 now takes (the barrier waits
        // for this wave's LDS reads only; the memory clobber keeps every
        // access on its side)
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (j + 3 < nh) load_half(j + 3, ntl, nsb);
        v16i e2[2] = {v16i{}, v16i{}};
        const v4i *A0 = tl + c * RS + h;
        constexpr int PF = S < 4 ? S : 4;
        v4i ar[PF];
#pragma unroll
        for (int st = 0; st < PF; ++st) ar[st] = A0[2 * st];
#pragma unroll
        for (int st = 0; st < S; ++st) {
            const v4i x = ar[st % PF];
            if (st + PF < S) ar[st % PF] = A0[2 * (st + PF)];
            e2[st & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, br[st], e2[st & 1], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        const v16i d = e2[0] + e2[1];
        // the lane's centroids come in runs of four: one 16-byte LDS read per run
        float sv[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4 s4 = *(const float4 *)&sb[8 * g + 4 * h];
            sv[4 * g] = s4.x, sv[4 * g + 1] = s4.y, sv[4 * g + 2] = s4.z, sv[4 * g + 3] = s4.w;
        }
        if ((j & 1) == 0) {
#pragma unroll
            for (int r = 0; r < 16; ++r) p[r] = sv[r] * (float)d[r];
            return;
        }
        const uint32_t c0 = (j >> 1) * 32;
        const bool full_tile = c0 + 32 <= a.nlist;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float v = fmaf(sv[r], (float)d[r], p[r]);
            const uint32_t ci = c0 + 8 * (r >> 2) + 4 * (uint32_t)h + (r & 3);
            if (v > tv[IVF_MQ_KEEP - 1] && (full_tile || ci < a.nlist)) {
                // insertion into the descending list
                float nv = v;
                uint32_t ni = ci;
#pragma unroll
                for (int i = 0; i < IVF_MQ_KEEP; ++i) {
                    const bool sw = nv > tv[i];
                    const float ov = tv[i];
                    const uint32_t oi = ti[i];
                    tv[i] = sw ? nv : ov;
                    ti[i] = sw ? ni : oi;
                    nv = sw ? ov : nv;
                    ni = sw ? oi : ni;
                }
            }
        }
    };

    load_half(0, tb0, sb0);
    if (nh > 1) load_half(1, tb1, sb1);
    if (nh > 2) load_half(2, tb2, sb2);
    for (uint32_t j = 0; j < nh; j += 4) {
        run_half(j, tb0, sb0, tb3, sb3);
        if (j + 1 >= nh) break;
        run_half(j + 1, tb1, sb1, tb0, sb0);
        if (j + 2 >= nh) break;
        run_half(j + 2, tb2, sb2, tb1, sb1);
        if (j + 3 >= nh) break;
        run_half(j + 3, tb3, sb3, tb2, sb2);
    }

    // the row's |b|^2 and any byte -128 (this lane's half of the codes)
    int nb2 = 0;
    uint32_t m128 = 0;
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t x = (uint32_t)br[st][w];
            nb2 = __builtin_amdgcn_sdot4(br[st][w], br[st][w], nb2, false);
            const uint32_t y = x ^ 0x80808080u;  // a byte 0x80 becomes zero
            m128 |= (y - 0x01010101u) & ~y & 0x80808080u;
        }
    nb2 += __shfl_xor(nb2, 32);
    const bool bad = (m128 | (uint32_t)__shfl_xor((int)m128, 32)) != 0;
    float pv[IVF_MQ_KEEP];
    uint32_t pi[IVF_MQ_KEEP];
#pragma unroll
    for (int i = 0; i < IVF_MQ_KEEP; ++i) {
        pv[i] = __shfl_xor(tv[i], 32);
        pi[i] = (uint32_t)__shfl_xor((int)ti[i], 32);
    }
    if (h != 0 || row >= a.n) return;
    const float sc = a.scales[row];
    const double vmax = fmax((double)tv[0], (double)pv[0]);
    const double W = 2.0 * sqrt((double)nb2) * (1.0 + 1e-12) * (double)__uint_as_float(m.words[0]);
    const double thr = vmax - W;
    bool all = bad || !(sc > 0.0f) || !(sc < __builtin_inff()) || !(thr > -__builtin_inf()) ||
               (double)tv[IVF_MQ_KEEP - 1] >= thr || (double)pv[IVF_MQ_KEEP - 1] >= thr;
    uint32_t cand[2 * IVF_MQ_KEEP - 2];
    uint32_t nc = 0;
#pragma unroll
    for (int i = 0; i < IVF_MQ_KEEP - 1; ++i) {
        if ((double)tv[i] >= thr) cand[nc++] = ti[i];
        if ((double)pv[i] >= thr) cand[nc++] = pi[i];
    }
    if (!all && nc == 1) {
        a.out[row] = cand[0];
        return;
    }
    const uint32_t slot = atomicAdd(&m.words[1], 1u);
    if (slot >= m.qcap) return;  // the caller sees the count and assigns every row exactly
    IvfRecheck e;
    e.row = (uint32_t)row;
    e.n = (all || nc == 0) ? IVF_RECHECK_ALL : nc;
#pragma unroll
    for (int i = 0; i < 6; ++i) e.c[i] = (uint32_t)i < nc ? cand[i] : 0u;
    m.queue[slot] = e;
}

// The queued rows, one wave each: ivf_assign<8>'s arithmetic (the row's
// values x_k = f32(f32(b_k / 127) * scale), staged in LDS, and an fmaf chain
// over k in order per centroid), over the row's candidates or every
// centroid, the lowest centroid winning ties.
constexpr int IVF_RC_WAVES = 4;
__global__ __launch_bounds__(IVF_RC_WAVES * 64) void ivf_assign_recheck(IvfAssignArgs a, IvfMfmaScratch m,
                                                                         uint32_t entries) {
    __shared__ __attribute__((aligned(16))) float xs[IVF_RC_WAVES][1024];
    __shared__ float dq8[256];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    dq8[threadIdx.x] = fmaxf((float)(int8_t)(uint8_t)threadIdx.x / 127.0f, -1.0f);
    __syncthreads();
    const uint32_t P = a.dim;
    float *x = xs[wave];
    for (uint32_t e = blockIdx.x * IVF_RC_WAVES + wave; e < entries; e += gridDim.x * IVF_RC_WAVES) {
        const IvfRecheck *q = m.queue + e;
        const uint64_t r = q->row;
        const uint32_t qn = q->n;
        const float sc = a.scales[r];
        const uint32_t *w = a.codes + r * a.words_per_row;
        for (uint32_t k = lane; k < P; k += 64) x[k] = dq8[(w[k >> 2] >> (8 * (k & 3))) & 0xffu] * sc;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const uint32_t cnt = qn == IVF_RECHECK_ALL ? a.nlist : qn;
        uint64_t best = 0;
        for (uint32_t j = lane; j < cnt; j += 64) {
            const uint32_t ci = qn == IVF_RECHECK_ALL ? j : q->c[j];
            const float4 *cv = (const float4 *)(a.centroids + (uint64_t)ci * a.cen_stride);
            float acc = 0.0f;
            for (uint32_t k4 = 0; k4 < P / 4; ++k4) {
                const float4 cc = cv[k4];
                const float4 xx = *(const float4 *)&x[4 * k4];
                acc = fmaf(xx.x, cc.x, acc);
                acc = fmaf(xx.y, cc.y, acc);
                acc = fmaf(xx.z, cc.z, acc);
                acc = fmaf(xx.w, cc.w, acc);
            }
            const uint64_t key = idx_key(acc, ci);
            best = key > best ? key : best;
        }
        best = wave_max_u64(best);
        if (lane == 0) a.out[r] = 0xffffffffu - (uint32_t)best;
        // every lane is done with x before the next entry overwrites it
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

}  // namespace

hipError_t ivf_launch_assign_mfma(const IvfAssignArgs &a, const IvfMfmaScratch &m, hipStream_t s) {
    if (!ivf_assign_mfma_ok(8, a.dim, a.nlist) || a.cen_stride % 4 != 0 || a.words_per_row != a.dim / 4)
        return hipErrorInvalidValue;
    const uint32_t pad = ivf_mfma_nlist_pad(a.nlist);
    hipLaunchKernelGGL(ivf_mfma_words_zero, dim3(1), dim3(64), 0, s, m.words);
    hipLaunchKernelGGL(ivf_cen_levels, dim3(pad), dim3(64), 0, s, a.centroids, a.cen_stride, a.nlist, a.dim, m.lev,
                       m.ls, m.words);
    if (a.n == 0) return hipGetLastError();
    const dim3 grid((uint32_t)((a.n + IVF_MA_ROWS - 1) / IVF_MA_ROWS)), block(IVF_MA_WAVES * 64);
    const uint32_t tiles = pad / 32;
    switch (a.dim) {
    case 128: hipLaunchKernelGGL(ivf_assign_mfma<4>, grid, block, 0, s, a, m, tiles); break;
    case 256: hipLaunchKernelGGL(ivf_assign_mfma<8>, grid, block, 0, s, a, m, tiles); break;
    case 512: hipLaunchKernelGGL(ivf_assign_mfma<16>, grid, block, 0, s, a, m, tiles); break;
    case 1024: hipLaunchKernelGGL(ivf_assign_mfma<32>, grid, block, 0, s, a, m, tiles); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t ivf_launch_assign_recheck(const IvfAssignArgs &a, const IvfMfmaScratch &m, uint32_t entries,
                                     hipStream_t s) {
    if (entries == 0) return hipSuccess;
    if (entries > m.qcap || a.dim > 1024 || a.dim % 4 != 0 || a.cen_stride % 4 != 0) return hipErrorInvalidValue;
    const uint32_t wgs = std::min<uint32_t>((entries + IVF_RC_WAVES - 1) / IVF_RC_WAVES, 4096);
    hipLaunchKernelGGL(ivf_assign_recheck, dim3(wgs), dim3(IVF_RC_WAVES * 64), 0, s, a, m, entries);
    return hipGetLastError();
}

uint32_t ivf_list_blocks(uint64_t n) { return (uint32_t)((n + LB - 1) / LB); }

hipError_t ivf_launch_lists(const uint32_t *assign, uint64_t n, uint32_t nlist, uint32_t *hist, uint32_t *base,
                            uint32_t *totals, uint32_t *offset, uint32_t *rows_out, hipStream_t s) {
    if (nlist == 0 || nlist > IVF_MAX_NLIST) return hipErrorInvalidValue;
    const uint32_t nblk = ivf_list_blocks(n);
    if (nblk) hipLaunchKernelGGL(ivf_block_hist, dim3(nblk), dim3(256), nlist * 4, s, assign, n, nlist, hist);
    hipLaunchKernelGGL(ivf_list_bases, dim3((nlist + 255) / 256), dim3(256), 0, s, hist, nblk, nlist, base, totals);
    hipLaunchKernelGGL(ivf_scan_offsets, dim3(1), dim3(256), 0, s, totals, nlist, offset);
    if (nblk) hipLaunchKernelGGL(ivf_scatter, dim3(nblk), dim3(256), 0, s, assign, n, nlist, offset, base, rows_out);
    return hipGetLastError();
}

namespace {
// One workgroup per list: the list's old rows, then its appended rows
// (shifted by add_base), at old_off[c] + add_off[c].
__global__ __launch_bounds__(256) void ivf_merge_lists(const uint32_t *old_off, const uint32_t *old_rows,
                                                        const uint32_t *add_off, const uint32_t *add_rows,
                                                        uint32_t add_base, uint32_t nlist, uint32_t *new_off,
                                                        uint32_t *new_rows) {
    const uint32_t c = blockIdx.x;
    const uint32_t o0 = old_off[c], o1 = old_off[c + 1], a0 = add_off[c], a1 = add_off[c + 1];
    const uint32_t dst = o0 + a0;
    if (threadIdx.x == 0) {
        new_off[c] = dst;
        if (c == nlist - 1) new_off[nlist] = o1 + a1;
    }
    for (uint32_t i = threadIdx.x; i < o1 - o0; i += 256) new_rows[dst + i] = old_rows[o0 + i];
    for (uint32_t i = threadIdx.x; i < a1 - a0; i += 256) new_rows[dst + (o1 - o0) + i] = add_base + add_rows[a0 + i];
}
}  // namespace

hipError_t ivf_launch_merge_lists(const uint32_t *old_off, const uint32_t *old_rows, const uint32_t *add_off,
                                  const uint32_t *add_rows, uint32_t add_base, uint32_t nlist, uint32_t *new_off,
                                  uint32_t *new_rows, hipStream_t s) {
    if (nlist == 0 || nlist > IVF_MAX_NLIST) return hipErrorInvalidValue;
    hipLaunchKernelGGL(ivf_merge_lists, dim3(nlist), dim3(256), 0, s, old_off, old_rows, add_off, add_rows, add_base,
                       nlist, new_off, new_rows);
    return hipGetLastError();
}

hipError_t ivf_launch_means(const float *sample, uint32_t stride, uint32_t dim, const uint32_t *offset,
                            const uint32_t *list_rows, uint32_t nlist, float *centroids, uint32_t cen_stride,
                            hipStream_t s) {
    const uint64_t t = (uint64_t)nlist * dim;
    hipLaunchKernelGGL(ivf_centroid_means, dim3((uint32_t)((t + 255) / 256)), dim3(256), 0, s, sample, stride, dim,
                       offset, list_rows, nlist, centroids, cen_stride);
    return hipGetLastError();
}

hipError_t ivf_launch_probes(const IvfProbeArgs &a, uint32_t nq, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    if (a.nlist > IVF_MAX_NLIST || a.nprobe > IVF_MAX_NPROBE || a.P > PROBE_MAX_DIM) return hipErrorInvalidValue;
    const size_t qb_lds = (size_t)PROBE_QB * 4 * (a.P / 4 + 1) * 8;
    if (nq >= PROBE_QB && a.P % 128 == 0 && a.P <= PROBE_QB_MAX_DIM && a.nlist >= 1024)
        hipLaunchKernelGGL(ivf_probe_scores_qb<4>, dim3((a.nlist + 255) / 256, (nq + PROBE_QB - 1) / PROBE_QB),
                           dim3(256), qb_lds, s, a, nq);
    else if (nq >= PROBE_QB && a.P % 128 == 0 && a.P <= PROBE_QB_MAX_DIM)
        hipLaunchKernelGGL(ivf_probe_scores_qb<1>, dim3((a.nlist + 63) / 64, (nq + PROBE_QB - 1) / PROBE_QB), dim3(256),
                           qb_lds, s, a, nq);
    else
        hipLaunchKernelGGL(ivf_probe_scores, dim3((a.nlist + 15) / 16, nq), dim3(64), (size_t)a.P * 4, s, a);
    hipLaunchKernelGGL(ivf_probe_select, dim3(nq), dim3(256), ((size_t)a.nlist * 2 + 16) * 8, s, a);
    return hipGetLastError();
}

hipError_t ivf_launch_gather(const uint32_t *probes, uint32_t nq, uint32_t nprobe, const uint32_t *offset,
                             const uint32_t *list_rows, uint64_t *totals, uint64_t *cand_off, uint32_t *cand,
                             hipStream_t s) {
    if (nq == 0) return hipSuccess;
    if (nq > 1) hipLaunchKernelGGL(ivf_cand_offsets, dim3(1), dim3(256), 0, s, totals, nq, cand_off);
    hipLaunchKernelGGL(ivf_gather_lists, dim3(nprobe, nq), dim3(256), 0, s, probes, nprobe, offset, list_rows, cand_off,
                       cand);
    return hipGetLastError();
}

}  // namespace bvk
