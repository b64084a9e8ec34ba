// Device selection for any k, and the exact scan of a caller's row list.
//
//   dense_keys      ordering key of every row of a dense score array (rows
//                   a mask leaves out get key 0)
//   list_keys       the same for the scores of listed rows
//   mask_popc /     the rows whose mask bit is set, as an ascending list
//   mask_rows       (per-word counts, an exclusive scan, then the rows)
//   exact_row_keys  Store.dotRow / Store.l2Row of each listed row in the
//                   reference's f64 order, as an ordering key
//   keys_to_hits    the first k keys of a descending sort as (row, score)
//
// Keys sort descending with hipCUB's radix sort: the canonical order (score
// desc, row asc) for any k up to the number of keys.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include "bv_device.h"
#include "bv_kernels.h"

namespace bvk {
namespace {

constexpr int SEL_BLOCK = 256;

uint32_t grid_of(uint64_t n, uint32_t per_block, uint32_t cap) {
    const uint64_t g = (n + per_block - 1) / per_block;
    return (uint32_t)(g < 1 ? 1 : (g > cap ? cap : g));
}

__global__ __launch_bounds__(SEL_BLOCK) void dense_keys(const float *scores, uint64_t n, const uint32_t *mask,
                                                        uint64_t *keys) {
    const uint64_t stride = (uint64_t)gridDim.x * SEL_BLOCK;
    for (uint64_t r = (uint64_t)blockIdx.x * SEL_BLOCK + threadIdx.x; r < n; r += stride) {
        const bool keep = !mask || ((mask[r >> 5] >> (r & 31)) & 1u);
        keys[r] = keep ? make_key(ord_f32(scores[r]), (uint32_t)r) : 0ull;
    }
}

__global__ __launch_bounds__(SEL_BLOCK) void list_keys(const float *scores, const uint32_t *list, uint64_t n,
                                                       uint64_t *keys) {
    const uint64_t stride = (uint64_t)gridDim.x * SEL_BLOCK;
    for (uint64_t i = (uint64_t)blockIdx.x * SEL_BLOCK + threadIdx.x; i < n; i += stride)
        keys[i] = make_key(ord_f32(scores[i]), list[i]);
}

// Set bits of word w below row n.
__device__ __forceinline__ uint32_t live_bits(const uint32_t *mask, uint64_t w, uint64_t n) {
    uint32_t b = mask[w];
    const uint64_t lo = w * 32;
    if (lo + 32 > n) b &= (n - lo >= 32) ? 0xffffffffu : ((1u << (uint32_t)(n - lo)) - 1u);
    return b;
}

__global__ __launch_bounds__(SEL_BLOCK) void mask_popc(const uint32_t *mask, uint64_t words, uint64_t n,
                                                       uint32_t *popc) {
    const uint64_t stride = (uint64_t)gridDim.x * SEL_BLOCK;
    for (uint64_t w = (uint64_t)blockIdx.x * SEL_BLOCK + threadIdx.x; w < words; w += stride)
        popc[w] = (uint32_t)__popc(live_bits(mask, w, n));
}

// off = exclusive scan of popc; the word's rows go to list[off[w] ...] in
// ascending order; list_n = the total.
__global__ __launch_bounds__(SEL_BLOCK) void mask_rows(const uint32_t *mask, uint64_t words, uint64_t n,
                                                       const uint32_t *popc, const uint32_t *off, uint32_t *list,
                                                       uint32_t *list_n) {
    const uint64_t stride = (uint64_t)gridDim.x * SEL_BLOCK;
    for (uint64_t w = (uint64_t)blockIdx.x * SEL_BLOCK + threadIdx.x; w < words; w += stride) {
        uint32_t b = live_bits(mask, w, n);
        uint32_t o = off[w];
        while (b) {
            const uint32_t t = (uint32_t)__ffs(b) - 1u;
            list[o++] = (uint32_t)(w * 32 + t);
            b &= b - 1u;
        }
        if (w + 1 == words) *list_n = off[w] + popc[w];
    }
}

// One lane per listed row.  Accumulator m sums elements 4j + m in order in
// f64 (dot: each f32 x f32 product is exact in f64, so fma adds it with the
// reference's single rounding; l2: the difference, its square and the sum
// each rounded, no contraction); then ((a0 + a1) + a2) + a3 and the tail
// elements in order; the score is the f32 of the sum (l2: of its negation).
// A listed row >= n sets *bad and gets key 0.
template <bool L2>
__device__ __forceinline__ void acc4(double (&a)[4], float4 x, float4 q) {
    if (L2) {
#pragma clang fp contract(off)
        const double d0 = (double)x.x - (double)q.x, d1 = (double)x.y - (double)q.y;
        const double d2 = (double)x.z - (double)q.z, d3 = (double)x.w - (double)q.w;
        a[0] = a[0] + d0 * d0;
        a[1] = a[1] + d1 * d1;
        a[2] = a[2] + d2 * d2;
        a[3] = a[3] + d3 * d3;
    } else {
        a[0] = fma((double)x.x, (double)q.x, a[0]);
        a[1] = fma((double)x.y, (double)q.y, a[1]);
        a[2] = fma((double)x.z, (double)q.z, a[2]);
        a[3] = fma((double)x.w, (double)q.w, a[3]);
    }
}

template <bool L2>
__device__ __forceinline__ double acc1(double s, float x, float q) {
    if (L2) {
#pragma clang fp contract(off)
        const double d = (double)x - (double)q;
        return s + d * d;
    }
    return fma((double)x, (double)q, s);
}

template <bool L2>
__global__ __launch_bounds__(SEL_BLOCK) void exact_row_keys(const float *raw, uint64_t n, uint32_t dim,
                                                            const float *q, const uint32_t *list, uint64_t n_list,
                                                            uint64_t *keys, uint32_t *bad) {
    extern __shared__ float qv[];
    for (uint32_t i = threadIdx.x; i < dim; i += SEL_BLOCK) qv[i] = q[i];
    __syncthreads();
    const uint32_t vec = dim & ~3u;
    const bool aligned = (dim & 3u) == 0 && (((uintptr_t)raw) & 15u) == 0;
    const uint64_t stride = (uint64_t)gridDim.x * SEL_BLOCK;
    for (uint64_t i = (uint64_t)blockIdx.x * SEL_BLOCK + threadIdx.x; i < n_list; i += stride) {
        const uint32_t row = list[i];
        if (row >= n) {
            keys[i] = 0ull;
            *bad = 1u;
            continue;
        }
        const float *x = raw + (uint64_t)row * dim;
        double a[4] = {0.0, 0.0, 0.0, 0.0};
        uint32_t j = 0;
        if (aligned) {
            const float4 *x4 = (const float4 *)x;
            const float4 *q4 = (const float4 *)qv;
            // eight 16-byte loads in flight, then summed in order
            for (; j + 32 <= vec; j += 32) {
                float4 xv[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) xv[u] = x4[j / 4 + u];
#pragma unroll
                for (int u = 0; u < 8; ++u) acc4<L2>(a, xv[u], q4[j / 4 + u]);
            }
            for (; j < vec; j += 4) acc4<L2>(a, x4[j / 4], q4[j / 4]);
        } else {
            for (; j < vec; j += 4)
                acc4<L2>(a, make_float4(x[j], x[j + 1], x[j + 2], x[j + 3]),
                         make_float4(qv[j], qv[j + 1], qv[j + 2], qv[j + 3]));
        }
        double s;
        {
#pragma clang fp contract(off)
            s = ((a[0] + a[1]) + a[2]) + a[3];
        }
        for (; j < dim; ++j) s = acc1<L2>(s, x[j], qv[j]);
        const float score = L2 ? (float)(-s) : (float)s;
        keys[i] = make_key(ord_f32(score), row);
    }
}

__global__ __launch_bounds__(SEL_BLOCK) void keys_to_hits(const uint64_t *keys, uint32_t k, uint32_t *rows,
                                                          float *scores, uint32_t *n_out) {
    for (uint32_t i = blockIdx.x * SEL_BLOCK + threadIdx.x; i < k; i += gridDim.x * SEL_BLOCK) {
        const uint64_t key = keys[i];
        if (key) {
            rows[i] = key_row(key);
            scores[i] = f32_from_ord((uint32_t)(key >> 32));
        }
        // keys are sorted descending, so the empty keys (0) come last
        if (key && (i + 1 == k || keys[i + 1] == 0ull)) *n_out = i + 1;
        if (i == 0 && !key) *n_out = 0;
    }
}

}  // namespace

hipError_t sel_dense_keys(const float *scores, uint64_t n, const uint32_t *mask, uint64_t *keys, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(dense_keys, dim3(grid_of(n, SEL_BLOCK * 4, 4096)), dim3(SEL_BLOCK), 0, s, scores, n, mask,
                       keys);
    return hipGetLastError();
}

hipError_t sel_list_keys(const float *scores, const uint32_t *list, uint64_t n, uint64_t *keys, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(list_keys, dim3(grid_of(n, SEL_BLOCK * 4, 4096)), dim3(SEL_BLOCK), 0, s, scores, list, n, keys);
    return hipGetLastError();
}

hipError_t sel_mask_counts(const uint32_t *mask, uint64_t words, uint64_t n, uint32_t *popc, hipStream_t s) {
    if (words == 0) return hipSuccess;
    hipLaunchKernelGGL(mask_popc, dim3(grid_of(words, SEL_BLOCK, 4096)), dim3(SEL_BLOCK), 0, s, mask, words, n,
                       popc);
    return hipGetLastError();
}

hipError_t sel_exclusive_scan(void *tmp, size_t &tmp_bytes, const uint32_t *in, uint32_t *out, uint64_t n,
                              hipStream_t s) {
    if (n > 0x7fffffffull) return hipErrorInvalidValue;
    return hipcub::DeviceScan::ExclusiveSum(tmp, tmp_bytes, in, out, (int)n, s);
}

hipError_t sel_mask_rows(const uint32_t *mask, uint64_t words, uint64_t n, const uint32_t *popc, const uint32_t *off,
                         uint32_t *list, uint32_t *list_n, hipStream_t s) {
    if (words == 0) return hipSuccess;
    hipLaunchKernelGGL(mask_rows, dim3(grid_of(words, SEL_BLOCK, 4096)), dim3(SEL_BLOCK), 0, s, mask, words, n, popc,
                       off, list, list_n);
    return hipGetLastError();
}

hipError_t sel_exact_row_keys(const float *raw, uint64_t n, uint32_t dim, bool l2, const float *q,
                              const uint32_t *list, uint64_t n_list, uint64_t *keys, uint32_t *bad, hipStream_t s) {
    if (n_list == 0) return hipSuccess;
    if (dim == 0 || (size_t)dim * 4 > 96 * 1024) return hipErrorInvalidValue;
    const dim3 grid(grid_of(n_list, SEL_BLOCK, 8192));
    if (l2)
        hipLaunchKernelGGL(exact_row_keys<true>, grid, dim3(SEL_BLOCK), (size_t)dim * 4, s, raw, n, dim, q, list,
                           n_list, keys, bad);
    else
        hipLaunchKernelGGL(exact_row_keys<false>, grid, dim3(SEL_BLOCK), (size_t)dim * 4, s, raw, n, dim, q, list,
                           n_list, keys, bad);
    return hipGetLastError();
}

hipError_t sel_sort_desc(void *tmp, size_t &tmp_bytes, const uint64_t *in, uint64_t *out, uint64_t n,
                         hipStream_t s) {
    if (n > 0x7fffffffull) return hipErrorInvalidValue;
    return hipcub::DeviceRadixSort::SortKeysDescending(tmp, tmp_bytes, in, out, (int)n, 0, 64, s);
}

hipError_t sel_keys_to_hits(const uint64_t *sorted, uint32_t k, uint32_t *rows, float *scores, uint32_t *n_out,
                            hipStream_t s) {
    if (k == 0) return hipSuccess;
    hipLaunchKernelGGL(keys_to_hits, dim3(grid_of(k, SEL_BLOCK, 1024)), dim3(SEL_BLOCK), 0, s, sorted, k, rows, scores,
                       n_out);
    return hipGetLastError();
}

}  // namespace bvk
