// gfx950 (CDNA4) kernels for BrowserVec's search path.
//
//   encode_rows    randomized-Hadamard rotate + int8/int4/1-bit quantize, one
//                  wave per row, FWHT in registers + cross-lane shuffles.
//                  Bit-exact with Rotator.rotateInto + quantizeRow*
//                  (src/quant/rotator.ts:61-70, src/quant/codec.ts:22-154).
//   scan_topk      streaming scan of codes / fp32 rows with the query slice
//                  held in registers, fused per-workgroup top-k in LDS and a
//                  last-workgroup merge across the grid.  Replaces the
//                  reference's distance kernels + score buffer + top-k kernel
//                  + CPU merge (src/engine/wgsl/distance*.ts, topk.ts,
//                  src/index/gpuTopk.ts:160-277).
//   rerank_topk    exact re-rank of the candidates with Store.dotRow's f64
//                  arithmetic (src/store/store.ts:114-130), then the final
//                  top-k (src/index.ts:583-594).
//
// Ordering keys: every candidate is one u64, high word = order-preserving
// bits of the score (-0 folded into +0), low word = ~row.  Larger key = better
// (higher score, then lower row), so a descending sort gives the canonical
// (score desc, row asc) order and keys are unique per row.  Key 0 = empty.
#include "bv_kernels.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bvk {

// ------------------------------------------------------------------ keys --
__device__ __forceinline__ uint32_t ord_f32(float s) {
    s = s + 0.0f;  // -0 -> +0 (round-to-nearest keeps every other value)
    uint32_t b = __float_as_uint(s);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float f32_from_ord(uint32_t o) {
    uint32_t b = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
    return __uint_as_float(b);
}
__device__ __forceinline__ uint32_t ord_i32(int32_t s) { return (uint32_t)s ^ 0x80000000u; }
__device__ __forceinline__ uint64_t make_key(uint32_t ord, uint32_t row) {
    return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - row);
}
__device__ __forceinline__ uint32_t key_row(uint64_t k) { return 0xffffffffu - (uint32_t)k; }

// ---------------------------------------------------------------- codecs --
// Each codec: Unit (what one lane loads per unit), QT/QN (query registers per
// unit), Acc (accumulator type), accumulate(), and score/ord finalisation.
template <int C> struct Codec;

template <> struct Codec<C_F32DOT> {
    using Unit = uint4; using QT = float; using Acc = float;
    static constexpr int QN = 4;
    static __device__ __forceinline__ Acc acc(Unit u, const QT *q, Acc a) {
        a = fmaf(__uint_as_float(u.x), q[0], a);
        a = fmaf(__uint_as_float(u.y), q[1], a);
        a = fmaf(__uint_as_float(u.z), q[2], a);
        a = fmaf(__uint_as_float(u.w), q[3], a);
        return a;
    }
    static __device__ __forceinline__ float score(Acc a, float) { return a; }
};
template <> struct Codec<C_F32L2> {
    using Unit = uint4; using QT = float; using Acc = float;
    static constexpr int QN = 4;
    static __device__ __forceinline__ Acc acc(Unit u, const QT *q, Acc a) {
        float d0 = __uint_as_float(u.x) - q[0], d1 = __uint_as_float(u.y) - q[1];
        float d2 = __uint_as_float(u.z) - q[2], d3 = __uint_as_float(u.w) - q[3];
        a = fmaf(d0, d0, a); a = fmaf(d1, d1, a); a = fmaf(d2, d2, a); a = fmaf(d3, d3, a);
        return a;
    }
    static __device__ __forceinline__ float score(Acc a, float) { return -a; }
};
template <> struct Codec<C_F32DOT_S> {
    using Unit = uint32_t; using QT = float; using Acc = float;
    static constexpr int QN = 1;
    static __device__ __forceinline__ Acc acc(Unit u, const QT *q, Acc a) { return fmaf(__uint_as_float(u), q[0], a); }
    static __device__ __forceinline__ float score(Acc a, float) { return a; }
};
template <> struct Codec<C_F32L2_S> {
    using Unit = uint32_t; using QT = float; using Acc = float;
    static constexpr int QN = 1;
    static __device__ __forceinline__ Acc acc(Unit u, const QT *q, Acc a) {
        float d = __uint_as_float(u) - q[0];
        return fmaf(d, d, a);
    }
    static __device__ __forceinline__ float score(Acc a, float) { return -a; }
};
// int8: q holds rotated/127 (the unpack4x8snorm scaling folded into the query).
template <> struct Codec<C_Q8> {
    using Unit = uint4; using QT = float; using Acc = float;
    static constexpr int QN = 16;
    static __device__ __forceinline__ Acc acc(Unit u, const QT *q, Acc a) {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            a = fmaf((float)(int32_t)((int32_t)(w[d] << 24) >> 24), q[4 * d + 0], a);
            a = fmaf((float)(int32_t)((int32_t)(w[d] << 16) >> 24), q[4 * d + 1], a);
            a = fmaf((float)(int32_t)((int32_t)(w[d] << 8) >> 24), q[4 * d + 2], a);
            a = fmaf((float)((int32_t)w[d] >> 24), q[4 * d + 3], a);
        }
        return a;
    }
    static __device__ __forceinline__ float score(Acc a, float scale) { return a * scale; }
};
template <> struct Codec<C_Q4> {
    using Unit = uint4; using QT = float; using Acc = float;
    static constexpr int QN = 32;
    static __device__ __forceinline__ Acc acc(Unit u, const QT *q, Acc a) {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                a = fmaf((float)((int32_t)(w[d] << (28 - 4 * j)) >> 28), q[8 * d + j], a);
        return a;
    }
    static __device__ __forceinline__ float score(Acc a, float scale) { return a * scale; }
};
template <> struct Codec<C_Q1A> {
    using Unit = uint32_t; using QT = float; using Acc = float;
    static constexpr int QN = 32;
    static __device__ __forceinline__ Acc acc(Unit u, const QT *q, Acc a) {
#pragma unroll
        for (int j = 0; j < 32; ++j) a += ((u >> j) & 1u) ? q[j] : -q[j];
        return a;
    }
    static __device__ __forceinline__ float score(Acc a, float scale) { return a * scale; }
};
template <> struct Codec<C_HAM> {
    using Unit = uint4; using QT = uint32_t; using Acc = int32_t;
    static constexpr int QN = 4;
    static __device__ __forceinline__ Acc acc(Unit u, const QT *q, Acc a) {
        return a + __popc(u.x ^ q[0]) + __popc(u.y ^ q[1]) + __popc(u.z ^ q[2]) + __popc(u.w ^ q[3]);
    }
};
template <> struct Codec<C_I8S> {
    using Unit = uint4; using QT = uint32_t; using Acc = int32_t;
    static constexpr int QN = 4;
    static __device__ __forceinline__ Acc acc(Unit u, const QT *q, Acc a) {
        a = __builtin_amdgcn_sdot4((int)u.x, (int)q[0], a, false);
        a = __builtin_amdgcn_sdot4((int)u.y, (int)q[1], a, false);
        a = __builtin_amdgcn_sdot4((int)u.z, (int)q[2], a, false);
        a = __builtin_amdgcn_sdot4((int)u.w, (int)q[3], a, false);
        return a;
    }
};

template <int C> struct IsInt { static constexpr bool v = (C == C_HAM || C == C_I8S); };

// ------------------------------------------------------- wave reductions --
// Transposing butterfly: lanes hold U partial sums (one per row group); after
// log2(U) halving exchanges and log2(LPR/U) plain ones every lane holds the
// full sum of row group bitrev(lane & (U-1)).
template <int U, int LPR, typename T> struct XReduce {
    static __device__ __forceinline__ T run(T (&v)[U], int lane) {
#pragma unroll
        for (int s = 0; (1 << s) < U; ++s) {
            const int m = 1 << s;
            const int n = U >> s;
            const int h = n >> 1;
            const bool hi = (lane & m) != 0;
#pragma unroll
            for (int j = 0; j < h; ++j) {
                T send = hi ? v[j] : v[j + h];
                T keep = hi ? v[j + h] : v[j];
                v[j] = keep + __shfl_xor(send, m);
            }
        }
#pragma unroll
        for (int m = U; m < LPR; m <<= 1) v[0] += __shfl_xor(v[0], m);
        return v[0];
    }
};

template <int U> __device__ __forceinline__ int bitrev_group(int p) {
    int r = 0;
#pragma unroll
    for (int s = 0; (1 << s) < U; ++s)
        if (p & (1 << s)) r |= (U >> (s + 1));
    return r;
}

// ------------------------------------------------------- LDS top-k state --
// Bitonic sort (descending) of keys[0, npow) by the whole workgroup.
__device__ void bitonic_desc(uint64_t *keys, uint32_t npow) {
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    for (uint32_t k = 2; k <= npow; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = tid; i < npow; i += nt) {
                uint32_t ixj = i ^ j;
                if (ixj > i) {
                    uint64_t a = keys[i], b = keys[ixj];
                    bool desc = (i & k) == 0;
                    if (desc ? (a < b) : (a > b)) {
                        keys[i] = b;
                        keys[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
}

__device__ __forceinline__ uint32_t pow2_at_least(uint32_t n) {
    uint32_t p = 2;
    while (p < n) p <<= 1;
    return p;
}

// Keep the best `kp` of keys[0, *cnt); tau becomes the kp-th best (or 0).
// Must be called by the whole workgroup; cnt/tau live in LDS.
__device__ void compact(uint64_t *keys, uint32_t *cnt, uint64_t *tau, uint32_t kp) {
    __syncthreads();
    const uint32_t n = *cnt;
    const uint32_t npow = pow2_at_least(n);
    for (uint32_t i = n + threadIdx.x; i < npow; i += blockDim.x) keys[i] = 0;
    __syncthreads();
    bitonic_desc(keys, npow);
    if (threadIdx.x == 0) {
        uint32_t m = n < kp ? n : kp;
        *cnt = m;
        *tau = (m == kp && kp > 0) ? keys[kp - 1] : 0;
    }
    __syncthreads();
}

// Wave-level append of keys for lanes where `take` holds.
__device__ __forceinline__ void wave_append(uint64_t *keys, uint32_t *cnt, bool take, uint64_t key, int lane) {
    const uint64_t ball = __ballot(take);
    if (ball == 0) return;
    const uint32_t total = __popcll(ball);
    const int leader = __ffsll((unsigned long long)ball) - 1;
    uint32_t base = 0;
    if (lane == leader) base = atomicAdd(cnt, total);
    base = __shfl(base, leader);
    if (take) {
        const uint64_t below = ball & ((lane == 0) ? 0ull : (~0ull >> (64 - lane)));
        keys[base + __popcll(below)] = key;
    }
}

// ------------------------------------------------------------ scan + top-k --
template <int C, int LPR, int UPL>
__global__ __launch_bounds__(SCAN_WG) void scan_topk(ScanArgs a) {
    using CD = Codec<C>;
    using Unit = typename CD::Unit;
    using QT = typename CD::QT;
    using Acc = typename CD::Acc;
    constexpr int U = LPR < 8 ? LPR : 8;  // row groups per lane per step
    constexpr int G = 64 / LPR;           // rows per load instruction
    constexpr int WAVES = SCAN_WG / 64;
    constexpr int RPS = U * G;            // rows per wave step

    __shared__ uint64_t keys[SCAN_CAP];
    __shared__ uint32_t cnt_s;
    __shared__ uint64_t tau_s;
    __shared__ uint32_t last_s;

    const uint32_t qi = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int slot = lane / LPR, p = lane % LPR;

    // query slice for the units this lane loads
    QT qr[UPL][CD::QN];
    const QT *qbase = (const QT *)((const char *)a.q + (uint64_t)qi * a.q_stride);
#pragma unroll
    for (int t = 0; t < UPL; ++t) {
        const uint32_t unit = p + LPR * t;
#pragma unroll
        for (int j = 0; j < CD::QN; ++j) qr[t][j] = unit < a.units ? qbase[unit * CD::QN + j] : (QT)0;
    }

    const uint32_t *cand = a.cand;
    uint64_t n = a.n;
    if (a.cand_off) {
        cand = a.cand + a.cand_off[qi];
        n = a.cand_off[qi + 1] - a.cand_off[qi];
    }
    const uint64_t r0 = (uint64_t)blockIdx.x * a.rows_per_wg;
    const uint64_t r1 = r0 + a.rows_per_wg < n ? r0 + a.rows_per_wg : n;
    const uint64_t span = r1 > r0 ? r1 - r0 : 0;
    const uint32_t steps = (uint32_t)((span + RPS - 1) / RPS);
    const uint32_t iters = (steps + WAVES - 1) / WAVES;
    constexpr uint32_t period_rows = (uint32_t)(WAVES * RPS);
    const uint32_t S = (SCAN_CAP / 2) / period_rows > 0 ? (SCAN_CAP / 2) / period_rows : 1;
    const uint32_t kp = a.kprime;

    if (tid == 0) {
        cnt_s = 0;
        tau_s = 0;
    }
    __syncthreads();
    uint64_t tau = 0;
    const int jrow = bitrev_group<U>(p & (U - 1));  // row group this lane ends up holding
    const bool rep = p < U;

    for (uint32_t it = 0; it < iters; ++it) {
        const uint32_t step = it * WAVES + wave;
        const uint64_t base = r0 + (uint64_t)step * RPS;
        // scale / global row of the row this lane will hold after the reduction
        const uint64_t myrow = base + (uint64_t)jrow * G + slot;
        const bool myvalid = rep && myrow < r1;
        uint32_t mygrow = 0;
        float myscale = 1.0f;
        if (myvalid) {
            mygrow = cand ? cand[myrow] : (uint32_t)myrow;
            if (a.scales) myscale = a.scales[mygrow] * a.scale_mul;
        }
        Acc acc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            acc[u] = (Acc)0;
            const uint64_t row = base + (uint64_t)u * G + slot;
            if (row < r1) {
                const uint64_t grow = cand ? cand[row] : row;
                const Unit *rp = (const Unit *)((const char *)a.codes + grow * a.row_bytes);
#pragma unroll
                for (int t = 0; t < UPL; ++t) {
                    const uint32_t unit = p + LPR * t;
                    if (unit < a.units) acc[u] = CD::acc(rp[unit], qr[t], acc[u]);
                }
            }
        }
        const Acc tot = XReduce<U, LPR, Acc>::run(acc, lane);
        bool take = false;
        uint64_t key = 0;
        if (myvalid) {
            uint32_t ord;
            float sc;
            if constexpr (C == C_HAM) {
                const int32_t sim = (int32_t)a.padded_dim - 2 * tot;
                ord = ord_i32(sim);
                sc = (float)sim;
            } else if constexpr (C == C_I8S) {
                ord = ord_i32(tot);
                sc = (float)tot;
            } else {
                sc = CD::score(tot, myscale);
                ord = ord_f32(sc);
            }
            if (a.dense_out && qi == 0) a.dense_out[myrow] = sc;
            bool pass = true;
            if (a.mask) pass = mygrow < a.mask_bits && ((a.mask[mygrow >> 5] >> (mygrow & 31)) & 1u);
            key = make_key(ord, mygrow);
            take = pass && key > tau;
        }
        wave_append(keys, &cnt_s, take, key, lane);
        if ((it + 1) % S == 0 || it + 1 == iters) {
            __syncthreads();
            if (it + 1 < iters && cnt_s > SCAN_CAP - S * period_rows) compact(keys, &cnt_s, &tau_s, kp);
            __syncthreads();
            tau = tau_s;
        }
    }
    compact(keys, &cnt_s, &tau_s, kp);

    // publish this workgroup's sorted top-kp
    uint64_t *mine = a.partials + ((uint64_t)qi * a.grid + blockIdx.x) * kp;
    const uint32_t have = cnt_s;
    for (uint32_t j = tid; j < kp; j += SCAN_WG) mine[j] = j < have ? keys[j] : 0;
    __threadfence();
    __syncthreads();
    if (tid == 0) last_s = atomicAdd(&a.tickets[qi], 1u) == a.grid - 1;
    __syncthreads();
    if (!last_s) return;
    __threadfence();

    // ---- last workgroup of this query: merge all partial lists --------------
    const uint64_t *lists = a.partials + (uint64_t)qi * a.grid * kp;
    if (tid == 0) {
        cnt_s = 0;
        tau_s = 0;
    }
    __syncthreads();
    // stage 1: each list's best key
    for (uint32_t g = tid; g < a.grid; g += SCAN_WG) {
        const uint64_t k0 = __builtin_nontemporal_load(&lists[(uint64_t)g * kp]);
        if (k0) keys[atomicAdd(&cnt_s, 1u)] = k0;
    }
    compact(keys, &cnt_s, &tau_s, kp);
    tau = tau_s;
    // stage 2: walk every list downwards while its keys beat tau
    const uint32_t R = (SCAN_CAP / 2) / a.grid > 0 ? ((SCAN_CAP / 2) / a.grid < 8 ? (SCAN_CAP / 2) / a.grid : 8) : 1;
    constexpr int MAXL = MAX_GRID / SCAN_WG;
    bool alive[MAXL];
#pragma unroll
    for (int m = 0; m < MAXL; ++m) alive[m] = (uint32_t)(tid + m * SCAN_WG) < a.grid;
    for (uint32_t j0 = 1; j0 < kp; j0 += R) {
        bool any = false;
#pragma unroll
        for (int m = 0; m < MAXL; ++m) {
            if (!alive[m]) continue;
            const uint32_t g = tid + m * SCAN_WG;
            for (uint32_t r = 0; r < R && j0 + r < kp; ++r) {
                const uint64_t kk = __builtin_nontemporal_load(&lists[(uint64_t)g * kp + j0 + r]);
                if (kk <= tau) {
                    alive[m] = false;
                    break;
                }
                keys[atomicAdd(&cnt_s, 1u)] = kk;
            }
            any = any || alive[m];
        }
        __syncthreads();
        if (cnt_s > SCAN_CAP / 2) compact(keys, &cnt_s, &tau_s, kp);
        tau = tau_s;
        if (!__syncthreads_or(any)) break;
    }
    compact(keys, &cnt_s, &tau_s, kp);
    const uint32_t m = cnt_s;
    uint64_t *outk = a.merged + (uint64_t)qi * kp;
    for (uint32_t j = tid; j < kp; j += SCAN_WG) outk[j] = j < m ? keys[j] : 0;
    if (tid == 0) a.merged_n[qi] = m;
    if (a.out_rows) {
        const uint32_t ko = m < a.k_out ? m : a.k_out;
        for (uint32_t j = tid; j < ko; j += SCAN_WG) {
            const uint64_t kk = keys[j];
            a.out_rows[(uint64_t)qi * a.k_out + j] = key_row(kk);
            const uint32_t o = (uint32_t)(kk >> 32);
            a.out_scores[(uint64_t)qi * a.k_out + j] =
                IsInt<C>::v ? (float)(int32_t)(o ^ 0x80000000u) : f32_from_ord(o);
        }
        if (tid == 0) a.out_n[qi] = ko;
    }
    if (tid == 0) a.tickets[qi] = 0;
}

// ---------------------------------------------------------------- encode --
// One wave per row.  Lane l holds elements [l*E, l*E+E) of the padded row.
template <int E>
__global__ __launch_bounds__(128) void encode_rows(EncodeArgs a) {
#pragma clang fp contract(off)
    extern __shared__ unsigned char smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t P = a.P;
    unsigned char *cbytes = smem + (size_t)wave * (P + 4 * P);
    float *fbuf = (float *)(cbytes + P);
    const uint32_t lanes_used = P / E;  // 64, or P when P < 64
    const uint32_t e0 = lane * E;
    const bool active = (uint32_t)lane < lanes_used;
    const uint64_t nwaves = (uint64_t)gridDim.x * (blockDim.x >> 6);

    for (uint64_t row = (uint64_t)blockIdx.x * (blockDim.x >> 6) + wave; row < a.rows; row += nwaves) {
        float x[E];
        const float *src = a.src + row * a.dim;
#pragma unroll
        for (int t = 0; t < E; ++t) {
            const uint32_t e = e0 + t;
            x[t] = (active && e < a.dim) ? src[e] : 0.0f;
        }
        for (uint32_t r = 0; r < a.rounds; ++r) {
            const float *s = a.signs + (size_t)r * P;
#pragma unroll
            for (int t = 0; t < E; ++t) x[t] = active ? x[t] * s[e0 + t] : 0.0f;
            // stages len = 1, 2, ... < E inside the lane
#pragma unroll
            for (int len = 1; len < E; len <<= 1) {
#pragma unroll
                for (int t = 0; t < E; ++t) {
                    if (!(t & len)) {
                        const float u = x[t], w = x[t + len];
                        x[t] = u + w;
                        x[t + len] = u - w;
                    }
                }
            }
            // stages len >= E across lanes (partner = lane ^ (len / E))
            for (uint32_t m = 1; m < lanes_used; m <<= 1) {
                const bool hi = (lane & m) != 0;
#pragma unroll
                for (int t = 0; t < E; ++t) {
                    const float y = __shfl_xor(x[t], (int)m);
                    x[t] = hi ? (y - x[t]) : (x[t] + y);
                }
            }
        }
        if (a.rotated && active) {
#pragma unroll
            for (int t = 0; t < E; ++t) a.rotated[row * P + e0 + t] = x[t];
        }
        if (a.qdiv && active) {
#pragma unroll
            for (int t = 0; t < E; ++t) a.qdiv[row * P + e0 + t] = x[t] / 127.0f;
        }
        if (a.bits == 0) continue;

        if (a.bits == 8 || a.bits == 4) {
            float m = 0.0f;
#pragma unroll
            for (int t = 0; t < E; ++t) {
                const float v = fabsf(x[t]);
                if (v > m) m = v;  // NaN never wins, as `a > maxAbs` in JS
            }
#pragma unroll
            for (int s = 1; s < 64; s <<= 1) {
                const float o = __shfl_xor(m, s);
                if (o > m) m = o;
            }
            const double scale = m > 0.0f ? (double)m : 1.0;
            const double inv = 1.0 / scale;
            const double levels = a.bits == 8 ? 127.0 : 7.0;
#pragma unroll
            for (int t = 0; t < E; ++t) {
                double c = (double)x[t] * inv;
                c = c < -1.0 ? -1.0 : (c > 1.0 ? 1.0 : c);
                const double y = c * levels;
                double rr = floor(y);
                if (y - rr >= 0.5) rr += 1.0;  // Math.round: ties toward +infinity
                if (rr < -levels) rr = -levels;
                if (rr > levels) rr = levels;
                const int code = (rr == rr) ? (int)rr : 0;  // NaN -> 0 (ToInt32)
                if (active) cbytes[e0 + t] = (unsigned char)(code & (a.bits == 8 ? 0xff : 0xf));
            }
            if (lane == 0) a.scales[row] = (float)scale;
        } else {  // 1-bit: signs, and mean |x| as a sequential f64 sum
            double s = 0.0;
            int emin = 1 << 20;
#pragma unroll
            for (int t = 0; t < E; ++t) {
                const float v = fabsf(x[t]);
                s += (double)v;
                if (v != 0.0f) {
                    const uint32_t b = __float_as_uint(v);
                    const int ex = (int)((b >> 23) & 0xffu);
                    const int ue = ex ? ex - 150 : -149;  // exponent of the value's ulp
                    emin = ue < emin ? ue : emin;
                }
                if (active) cbytes[e0 + t] = x[t] >= 0.0f ? 1 : 0;
            }
#pragma unroll
            for (int sh = 1; sh < 64; sh <<= 1) {
                s += __shfl_xor(s, sh);
                const int o = __shfl_xor(emin, sh);
                emin = o < emin ? o : emin;
            }
            // Every partial sum (any order) is a multiple of 2^emin no larger
            // than the total; below 2^(emin+52) all are exact in f64, so the
            // tree sum equals the reference's sequential one.  Otherwise take
            // the sequential sum literally.
            const bool exact = (s == 0.0) || (s < ldexp(1.0, emin + 52));
            if (!exact) {
                if (active) {
#pragma unroll
                    for (int t = 0; t < E; ++t) fbuf[e0 + t] = x[t];
                }
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                double seq = 0.0;
                if (lane == 0) {
                    for (uint32_t i = 0; i < P; ++i) seq += (double)fabsf(fbuf[i]);
                    if (a.slow_rows) atomicAdd(a.slow_rows, 1u);
                }
                s = __shfl(seq, 0);
            }
            if (lane == 0) a.scales[row] = s > 0.0 ? (float)(s / (double)P) : 1.0f;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // pack from LDS: word g covers `per` consecutive codes
        const uint32_t per = a.bits == 8 ? 4 : (a.bits == 4 ? 8 : 32);
        const uint32_t W = P / per, sh = a.bits == 8 ? 8 : (a.bits == 4 ? 4 : 1);
        for (uint32_t g = lane; g < W; g += 64) {
            uint32_t w = 0;
            for (uint32_t j = 0; j < per; ++j) w |= (uint32_t)cbytes[g * per + j] << (sh * j);
            a.codes[row * W + g] = w;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
}

// ---------------------------------------------------------------- rerank --
// One wave per candidate: stage the row and query in LDS, then four lanes run
// Store.dotRow's four strided f64 accumulators (store.ts:114-130).  The last
// wave of each query sorts the re-ranked scores and writes the top-k_out.
__global__ __launch_bounds__(64) void rerank_topk(RerankArgs a) {
    extern __shared__ float rsm[];
    float *rowv = rsm;
    float *qv = rsm + a.dim;
    __shared__ uint64_t keys[MAX_KPRIME];
    __shared__ uint32_t last_s;
    const uint32_t qi = blockIdx.y, c = blockIdx.x;
    const int lane = threadIdx.x;
    uint32_t m;
    uint32_t row = 0;
    bool have = false;
    if (a.merged) {
        m = a.merged_n[qi];
        if (c < m) {
            row = key_row(a.merged[(uint64_t)qi * a.kprime + c]);
            have = true;
        }
    } else {
        m = a.cand_n[qi];
        if (c < m) {
            row = a.cand_rows[(uint64_t)qi * a.kprime + c];
            have = true;
        }
    }
    if (have) {
        const float *src = a.rows + (uint64_t)row * a.dim;
        const float *qs = a.q + (uint64_t)qi * a.q_stride;
        for (uint32_t i = lane; i < a.dim; i += 64) {
            rowv[i] = src[i];
            qv[i] = qs[i];
        }
        __syncthreads();
        const uint32_t vec = a.dim & ~3u;
        double acc = 0.0;
        if (lane < 4) {
            for (uint32_t i = lane; i < vec; i += 4) acc = fma((double)rowv[i], (double)qv[i], acc);
        }
        const double a1 = __shfl(acc, 1), a2 = __shfl(acc, 2), a3 = __shfl(acc, 3);
        if (lane == 0) {
            double s = acc + a1;
            s = s + a2;
            s = s + a3;
            for (uint32_t i = vec; i < a.dim; ++i) s = fma((double)rowv[i], (double)qv[i], s);
            a.rr_scores[(uint64_t)qi * a.kprime + c] = (float)s;
            a.rr_rows[(uint64_t)qi * a.kprime + c] = row;
        }
    }
    __threadfence();
    __syncthreads();
    if (lane == 0) last_s = atomicAdd(&a.tickets[qi], 1u) == gridDim.x - 1;
    __syncthreads();
    if (!last_s) return;
    __threadfence();
    const uint32_t npow = pow2_at_least(m);
    for (uint32_t j = lane; j < npow; j += 64) {
        uint64_t kk = 0;
        if (j < m) {
            const float sc = __builtin_nontemporal_load(&a.rr_scores[(uint64_t)qi * a.kprime + j]);
            const uint32_t rw = __builtin_nontemporal_load(&a.rr_rows[(uint64_t)qi * a.kprime + j]);
            kk = make_key(ord_f32(sc), rw);
        }
        keys[j] = kk;
    }
    __syncthreads();
    bitonic_desc(keys, npow);
    const uint32_t ko = m < a.k_out ? m : a.k_out;
    for (uint32_t j = lane; j < ko; j += 64) {
        a.out_rows[(uint64_t)qi * a.k_out + j] = key_row(keys[j]);
        a.out_scores[(uint64_t)qi * a.k_out + j] = f32_from_ord((uint32_t)(keys[j] >> 32));
    }
    if (lane == 0) {
        a.out_n[qi] = ko;
        a.tickets[qi] = 0;
    }
}

// -------------------------------------------------------------- launchers --
namespace {

struct Layout {
    int lpr;
    int upl;
};

bool pick_layout(uint32_t units, Layout &L) {
    if (units == 0) return false;
    if (units >= 64) {
        const uint32_t upl = (units + 63) / 64;
        static const int ok[] = {1, 2, 3, 4, 6, 8, 12, 16};
        for (int v : ok)
            if ((uint32_t)v == upl) {
                L = {64, v};
                return true;
            }
        for (int v : ok)
            if ((uint32_t)v > upl) {
                L = {64, v};
                return true;
            }
        return false;
    }
    int lpr = 4;
    while ((uint32_t)lpr < units) lpr <<= 1;
    L = {lpr, 1};
    return true;
}

template <int C, int LPR, int UPL>
hipError_t go(const ScanArgs &a, uint32_t nq, hipStream_t s) {
    hipLaunchKernelGGL((scan_topk<C, LPR, UPL>), dim3(a.grid, nq), dim3(SCAN_WG), 0, s, a);
    return hipGetLastError();
}

template <int C>
hipError_t dispatch_layout(const Layout &L, const ScanArgs &a, uint32_t nq, hipStream_t s) {
    if (L.lpr == 64) {
        switch (L.upl) {
        case 1: return go<C, 64, 1>(a, nq, s);
        case 2: return go<C, 64, 2>(a, nq, s);
        case 3: return go<C, 64, 3>(a, nq, s);
        case 4: return go<C, 64, 4>(a, nq, s);
        case 6: return go<C, 64, 6>(a, nq, s);
        case 8: return go<C, 64, 8>(a, nq, s);
        case 12: return go<C, 64, 12>(a, nq, s);
        case 16: return go<C, 64, 16>(a, nq, s);
        default: return hipErrorInvalidValue;
        }
    }
    switch (L.lpr) {
    case 4: return go<C, 4, 1>(a, nq, s);
    case 8: return go<C, 8, 1>(a, nq, s);
    case 16: return go<C, 16, 1>(a, nq, s);
    case 32: return go<C, 32, 1>(a, nq, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool scan_supported(int codec, uint32_t units) {
    Layout L;
    if (!pick_layout(units, L)) return false;
    // register budget: at most 64 query values per lane
    static const int qn[C_COUNT] = {4, 4, 16, 32, 32, 4, 4, 1, 1};
    return codec >= 0 && codec < C_COUNT && L.upl * qn[codec] <= 64;
}

hipError_t launch_scan(int codec, uint32_t units, const ScanArgs &a, uint32_t nq, hipStream_t s) {
    Layout L;
    if (!pick_layout(units, L) || !scan_supported(codec, units)) return hipErrorInvalidValue;
    switch (codec) {
    case C_F32DOT: return dispatch_layout<C_F32DOT>(L, a, nq, s);
    case C_F32L2: return dispatch_layout<C_F32L2>(L, a, nq, s);
    case C_Q8: return dispatch_layout<C_Q8>(L, a, nq, s);
    case C_Q4: return dispatch_layout<C_Q4>(L, a, nq, s);
    case C_Q1A: return dispatch_layout<C_Q1A>(L, a, nq, s);
    case C_HAM: return dispatch_layout<C_HAM>(L, a, nq, s);
    case C_I8S: return dispatch_layout<C_I8S>(L, a, nq, s);
    case C_F32DOT_S: return dispatch_layout<C_F32DOT_S>(L, a, nq, s);
    case C_F32L2_S: return dispatch_layout<C_F32L2_S>(L, a, nq, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_encode(const EncodeArgs &a, hipStream_t s) {
    if (a.rows == 0) return hipSuccess;
    const uint32_t E = a.P >= 64 ? a.P / 64 : 1;
    const int waves = 2;
    const size_t lds = (size_t)waves * (a.P + 4 * (size_t)a.P);
    uint64_t blocks = (a.rows + waves - 1) / waves;
    if (blocks > 65536) blocks = 65536;
    dim3 grid((uint32_t)blocks), block(64 * waves);
    switch (E) {
    case 1: hipLaunchKernelGGL(encode_rows<1>, grid, block, lds, s, a); break;
    case 2: hipLaunchKernelGGL(encode_rows<2>, grid, block, lds, s, a); break;
    case 4: hipLaunchKernelGGL(encode_rows<4>, grid, block, lds, s, a); break;
    case 8: hipLaunchKernelGGL(encode_rows<8>, grid, block, lds, s, a); break;
    case 16: hipLaunchKernelGGL(encode_rows<16>, grid, block, lds, s, a); break;
    case 32: hipLaunchKernelGGL(encode_rows<32>, grid, block, lds, s, a); break;
    case 64: hipLaunchKernelGGL(encode_rows<64>, grid, block, lds, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_rerank(const RerankArgs &a, uint32_t nq, hipStream_t s) {
    const size_t lds = sizeof(float) * 2 * (size_t)a.dim;
    hipLaunchKernelGGL(rerank_topk, dim3(a.kprime, nq), dim3(64), lds, s, a);
    return hipGetLastError();
}

}  // namespace bvk
