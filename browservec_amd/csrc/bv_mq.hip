// Batched int8 scans on the gfx950 matrix cores.
//
//   mq_scan_q8   rows x queries x three int8 query levels on
//                v_mfma_i32_32x32x32_i8.  Every (row, query, level) dot is
//                an exact int32, combined per (row, query) in f64 exactly as
//                the single-query scan combines its three dots, so a batch
//                produces the same keys as the same queries scanned one at a
//                time.  Replaces the reference's per-query distanceQ8
//                dispatches + score buffers for query batches
//                (src/engine/wgsl/distanceQ8.ts:56-82, src/index/quant.ts:178-245,
//                src/index.ts:473-517).
//   mq_select    exact 64-bit radix select of each query's best kk keys.
//
// A batch runs as: a dense pass over a strided sample of the rows, whose
// kk-th best key per query is a valid pruning bound (it is the key of a real
// row, and a subset's kk-th best is never above the whole set's); a pass
// over every row that appends only the keys at or above that bound; and a
// select of the best kk appended keys.
#include "bv_kernels.h"
#include "bv_device.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bvk {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// f64 combine of the three level dots, then the row scale: the arithmetic
// of the single-query int8 scan's finalisation.
__device__ __forceinline__ uint64_t q8_key(double s0, double s1, double s2, int32_t d0, int32_t d1, int32_t d2,
                                           float scale, uint32_t row) {
    const double v = fma(s2, (double)d2, fma(s1, (double)d1, s0 * (double)d0));
    const float sc = (float)(v * (double)scale);
    return make_key(ord_f32(sc), row);
}

// Descending bitonic sort of keys[0, npow) (npow a power of two), whole
// workgroup.
__device__ void sort_desc(uint64_t *keys, uint32_t npow) {
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    for (uint32_t k = 2; k <= npow; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = tid; i < npow; i += nt) {
                const uint32_t ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t x = keys[i], y = keys[ixj];
                    const bool desc = (i & k) == 0;
                    if (desc ? (x < y) : (x > y)) {
                        keys[i] = y;
                        keys[ixj] = x;
                    }
                }
            }
            __syncthreads();
        }
    }
}

}  // namespace

// One workgroup = MQ_ROWS rows x MQ_QB queries; wave w takes rows
// [64w, 64w + 64) of the tile against all MQ_QB queries as 2 x 2 blocks of
// 32 x 32, three level accumulators each.  The K loop walks the row in
// 32-code steps: lane l supplies 16 codes (unit 2s + l/32) of row l%32 as
// the A operand and the same unit of query l%32's level bytes as the B
// operand, so both operands pair the same codes.  Accumulator register r of
// lane l holds row 8*(r/4) + 4*(l/32) + r%4, query l%32 of its block.
__global__ __launch_bounds__(256) void mq_scan_q8(MqArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = lane >> 5, c = lane & 31;
    // Dispatch is round robin over the 8 XCDs, so workgroups b, b+8, ... share
    // an XCD.  The qblocks tiles of one row tile take consecutive slots on one
    // XCD and read the same codes through its L2.
    const uint32_t b = blockIdx.x, xcd = b & 7u, slot = b >> 3;
    const uint32_t qb = slot % a.qblocks;
    const uint64_t tile = (uint64_t)(slot / a.qblocks) * 8 + xcd;
    const uint64_t t0 = tile * MQ_ROWS;
    if (t0 >= a.n) return;
    const uint64_t w0 = t0 + (uint64_t)wave * 64;

    const v4i *ap[2];
#pragma unroll
    for (int fr = 0; fr < 2; ++fr) {
        uint64_t li = w0 + fr * 32 + c;
        if (li >= a.n) li = a.n - 1;  // rows past the end load a valid row; their results are dropped
        ap[fr] = (const v4i *)(a.codes + li * a.row_step * a.W) + h;
    }
    const v4i *bp[2];
#pragma unroll
    for (int fq = 0; fq < 2; ++fq) {
        uint32_t q = qb * MQ_QB + fq * 32 + c;
        if (q >= a.nq) q = a.nq - 1;
        bp[fq] = (const v4i *)(a.qlev + (uint64_t)q * a.qstride) + h * 3;  // unit u, level l at u*3 + l
    }

    v16i acc[2][2][3];
#pragma unroll
    for (int fr = 0; fr < 2; ++fr)
#pragma unroll
        for (int fq = 0; fq < 2; ++fq)
#pragma unroll
            for (int l = 0; l < 3; ++l) acc[fr][fq][l] = v16i{};

    const uint32_t S = a.units >> 1;
    v4i A[2], B[2][3];
#pragma unroll
    for (int fr = 0; fr < 2; ++fr) A[fr] = ap[fr][0];
#pragma unroll
    for (int fq = 0; fq < 2; ++fq)
#pragma unroll
        for (int l = 0; l < 3; ++l) B[fq][l] = bp[fq][l];
    for (uint32_t s = 0; s < S; ++s) {
        const uint32_t sn = s + 1 < S ? s + 1 : s;  // the last step reloads its own operands
        v4i An[2], Bn[2][3];
#pragma unroll
        for (int fr = 0; fr < 2; ++fr) An[fr] = ap[fr][2 * sn];
#pragma unroll
        for (int fq = 0; fq < 2; ++fq)
#pragma unroll
            for (int l = 0; l < 3; ++l) Bn[fq][l] = bp[fq][6 * sn + l];
#pragma unroll
        for (int fr = 0; fr < 2; ++fr)
#pragma unroll
            for (int fq = 0; fq < 2; ++fq)
#pragma unroll
                for (int l = 0; l < 3; ++l)
                    acc[fr][fq][l] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[fr], B[fq][l], acc[fr][fq][l], 0, 0, 0);
#pragma unroll
        for (int fr = 0; fr < 2; ++fr) A[fr] = An[fr];
#pragma unroll
        for (int fq = 0; fq < 2; ++fq)
#pragma unroll
            for (int l = 0; l < 3; ++l) B[fq][l] = Bn[fq][l];
    }

#pragma unroll
    for (int fq = 0; fq < 2; ++fq) {
        const uint32_t q = qb * MQ_QB + fq * 32 + c;
        const bool qok = q < a.nq;
        const uint32_t qq = qok ? q : a.nq - 1;
        const QLevelTail *t = (const QLevelTail *)(a.qlev + (uint64_t)qq * a.qstride + a.tail_off);
        const double s0 = t->s[0], s1 = t->s[1], s2 = t->s[2];
        uint64_t *out = a.cand + (uint64_t)qq * a.cap;
        if (!a.tau) {  // dense pass: key of logical row i at out[i]
#pragma unroll
            for (int fr = 0; fr < 2; ++fr)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint64_t li = w0 + fr * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (qok && li < a.n) {
                        const uint64_t row = li * a.row_step;
                        out[li] = q8_key(s0, s1, s2, acc[fr][fq][0][r], acc[fr][fq][1][r], acc[fr][fq][2][r],
                                         a.scales[row], (uint32_t)row);
                    }
                }
            continue;
        }
        const uint64_t tau = a.tau[qq];
        uint32_t pass = 0;  // bit fr*16 + r: key at or above the bound
#pragma unroll
        for (int fr = 0; fr < 2; ++fr)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint64_t li = w0 + fr * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (qok && li < a.n) {
                    const uint64_t row = li * a.row_step;
                    const uint64_t key = q8_key(s0, s1, s2, acc[fr][fq][0][r], acc[fr][fq][1][r],
                                                acc[fr][fq][2][r], a.scales[row], (uint32_t)row);
                    if (key >= tau) pass |= 1u << (fr * 16 + r);
                }
            }
        // lanes c and c + 32 hold the same query: one reservation for both
        const uint32_t mine = __popc(pass);
        const uint32_t other = __shfl_xor(mine, 32);
        uint32_t base = 0;
        if (h == 0 && mine + other) base = atomicAdd(&a.cnt[qq], mine + other);
        base = __shfl(base, c);
        if (pass) {
            uint64_t pos = (uint64_t)base + (h ? other : 0u);
#pragma unroll
            for (int fr = 0; fr < 2; ++fr)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    if (pass & (1u << (fr * 16 + r))) {
                        const uint64_t li = w0 + fr * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                        const uint64_t row = li * a.row_step;
                        if (pos < a.cap)
                            out[pos] = q8_key(s0, s1, s2, acc[fr][fq][0][r], acc[fr][fq][1][r], acc[fr][fq][2][r],
                                              a.scales[row], (uint32_t)row);
                        ++pos;
                    }
                }
        }
    }
}

// One workgroup per query.  The kk-th best key is found digit by digit
// from the top (8 passes of 8 bits over the keys, a 256-bin histogram of
// the keys that match the digits found so far); keys are unique, so exactly
// kk keys are at or above it.
__global__ __launch_bounds__(256) void mq_select(MqSelArgs a) {
    __shared__ uint32_t hist[256];
    __shared__ uint64_t sel[MAX_KPRIME];
    __shared__ uint32_t s_digit, s_rem, s_cnt;
    const uint32_t q = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const uint32_t total = a.cnt[q];
    const uint32_t n = (uint64_t)total < a.cap ? total : (uint32_t)a.cap;
    const uint64_t *keys = a.cand + (uint64_t)q * a.cap;
    const uint32_t kk = a.kk < n ? a.kk : n;
    uint64_t T = 0;
    if (n > kk) {
        uint64_t prefix = 0;
        uint32_t rem = kk;  // rank of the wanted key from the top within the matching keys
        for (int shift = 56; shift >= 0; shift -= 8) {
            hist[tid] = 0;
            __syncthreads();
            const uint64_t hi_mask = shift == 56 ? 0ull : (~0ull << (shift + 8));
            for (uint32_t i = tid; i < n; i += 256) {
                const uint64_t k = keys[i];
                if ((k & hi_mask) == prefix) atomicAdd(&hist[(uint32_t)(k >> shift) & 255u], 1u);
            }
            __syncthreads();
            if (wave == 0) {
                // lane l holds digits 255-4l .. 252-4l; inclusive scan from the top
                uint32_t c4[4], loc = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    c4[j] = hist[255 - (4 * lane + j)];
                    loc += c4[j];
                }
                uint32_t inc = loc;
#pragma unroll
                for (int off = 1; off < 64; off <<= 1) {
                    const uint32_t v = __shfl_up(inc, off);
                    if (lane >= off) inc += v;
                }
                const uint32_t exc = inc - loc;
                const uint64_t bal = __ballot(exc < rem && rem <= inc);
                if (lane == __ffsll((unsigned long long)bal) - 1) {
                    uint32_t accum = exc;
                    for (int j = 0; j < 4; ++j) {
                        if (accum + c4[j] >= rem) {
                            s_digit = 255u - (uint32_t)(4 * lane + j);
                            s_rem = rem - accum;
                            break;
                        }
                        accum += c4[j];
                    }
                }
            }
            __syncthreads();
            prefix |= (uint64_t)s_digit << shift;
            rem = s_rem;
            __syncthreads();
        }
        T = prefix;
    }
    if (tid == 0) s_cnt = 0;
    __syncthreads();
    for (uint32_t i = tid; i < n; i += 256) {
        const uint64_t k = keys[i];
        if (k >= T && k != 0) {
            const uint32_t p = atomicAdd(&s_cnt, 1u);
            if (p < (uint32_t)MAX_KPRIME) sel[p] = k;
        }
    }
    __syncthreads();
    const uint32_t m = s_cnt < kk ? s_cnt : kk;
    if (tid == 0) {
        if (a.tau) a.tau[q] = n > kk ? T : 0ull;
        if (a.merged_n) a.merged_n[q] = m;
        if (a.overflow) a.overflow[q] = (uint64_t)total > a.cap ? 1u : 0u;
    }
    if (a.merged)
        for (uint32_t i = tid; i < m; i += 256) a.merged[(uint64_t)q * a.kk + i] = sel[i];
    if (a.out_rows) {
        uint32_t npow = 2;
        while (npow < m) npow <<= 1;
        for (uint32_t i = m + tid; i < npow; i += 256) sel[i] = 0;
        __syncthreads();
        sort_desc(sel, npow);
        const uint32_t ko = m < a.k_out ? m : a.k_out;
        for (uint32_t i = tid; i < ko; i += 256) {
            a.out_rows[(uint64_t)q * a.k_out + i] = key_row(sel[i]);
            a.out_scores[(uint64_t)q * a.k_out + i] = f32_from_ord((uint32_t)(sel[i] >> 32));
        }
        if (tid == 0) a.out_n[q] = ko;
    }
}

hipError_t launch_mq_scan(const MqArgs &a, hipStream_t s) {
    if (a.n == 0 || a.nq == 0) return hipSuccess;
    if ((a.units & 1u) || a.units == 0 || a.qblocks == 0 || (a.tiles & 7u) ||
        (uint64_t)a.tiles * MQ_ROWS < a.n || (uint64_t)a.qblocks * MQ_QB < a.nq)
        return hipErrorInvalidValue;
    const uint64_t blocks = (uint64_t)a.tiles * a.qblocks;
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mq_scan_q8, dim3((uint32_t)blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_mq_select(const MqSelArgs &a, uint32_t nq, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    if (a.kk == 0 || a.kk > (uint32_t)MAX_KPRIME) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mq_select, dim3(nq), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace bvk
