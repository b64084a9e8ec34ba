// Streaming-read ceiling for the benchmark (libbv_bench.so, loaded only by
// bench.py): a read-only kernel over a device buffer with the access the
// scans use (16-byte loads, each byte read once), so the achieved bandwidth
// of a scan can be set against what a read-only stream reaches on the same
// card.  Not part of the search library.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef unsigned int nt_u4 __attribute__((ext_vector_type(4)));

template <bool NT> __device__ __forceinline__ uint4 ld(const uint4 *p) {
    if constexpr (NT) {
        const nt_u4 x = __builtin_nontemporal_load((const nt_u4 *)p);
        return make_uint4(x.x, x.y, x.z, x.w);
    } else {
        return *p;
    }
}

// chunk == 0: grid-stride over 16-byte units, eight loads in flight per
// thread.  chunk > 0: contiguous chunks of `chunk` units handed to the
// workgroups round robin (chunk c to workgroup c % grid), the way the scans
// hand out row blocks; each thread issues eight loads of one chunk at a time.
// The XOR of everything read goes to sink[thread] so no load is dropped.
template <bool NT>
__global__ __launch_bounds__(256) void stream_read(const uint4 *p, uint64_t units, uint64_t chunk, uint32_t *sink) {
    uint32_t acc = 0;
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (chunk == 0) {
        const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
        uint64_t i = t;
        for (; i + 7 * stride < units; i += 8 * stride) {
            uint4 v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = ld<NT>(p + i + j * stride);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
        }
        for (; i < units; i += stride) {
            const uint4 v = p[i];
            acc ^= v.x ^ v.y ^ v.z ^ v.w;
        }
    } else {
        const uint64_t nchunks = (units + chunk - 1) / chunk;
        for (uint64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
            const uint64_t c0 = c * chunk, c1 = c0 + chunk < units ? c0 + chunk : units;
            uint64_t i = c0 + threadIdx.x;
            for (; i + 7 * 256 < c1; i += 8 * 256) {
                uint4 v[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = ld<NT>(p + i + j * 256);
#pragma unroll
                for (int j = 0; j < 8; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
            }
            for (; i < c1; i += 256) {
                const uint4 v = p[i];
                acc ^= v.x ^ v.y ^ v.z ^ v.w;
            }
        }
    }
    sink[t] = acc;
}

}  // namespace

// Reads `bytes` (a multiple of 16) at p once with `blocks` workgroups of 256
// threads; chunk_bytes 0 = grid-stride, else contiguous chunks of that many
// bytes (a multiple of 16) per workgroup round robin.  sink holds
// blocks * 256 words.
extern "C" int bvb_stream_read(const void *p, uint64_t bytes, int nontemporal, uint64_t chunk_bytes, uint32_t *sink,
                               uint32_t blocks, void *stream) {
    if ((bytes & 15) || (chunk_bytes & 15) || blocks == 0) return (int)hipErrorInvalidValue;
    const uint64_t units = bytes / 16, chunk = chunk_bytes / 16;
    hipStream_t s = (hipStream_t)stream;
    if (nontemporal)
        hipLaunchKernelGGL(stream_read<true>, dim3(blocks), dim3(256), 0, s, (const uint4 *)p, units, chunk, sink);
    else
        hipLaunchKernelGGL(stream_read<false>, dim3(blocks), dim3(256), 0, s, (const uint4 *)p, units, chunk, sink);
    return (int)hipGetLastError();
}
