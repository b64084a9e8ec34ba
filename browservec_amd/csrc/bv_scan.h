// Device code of the fused scan shared by the per-codec translation units
// (bv_scan_*.hip) and bv_kernels.hip: codecs, wave reductions, the LDS
// top-k, rotation / quantization building blocks, the exact re-rank
// arithmetic and scan_topk itself.  Everything here has internal linkage;
// each translation unit instantiates what it launches.
//
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
//                  src/index/gpuTopk.ts:160-189).
//   rerank_topk    exact re-rank of the candidates with Store.dotRow's f64
//                  arithmetic (src/store/store.ts:114-130), then the final
//                  top-k (src/index.ts:583-594).
//
// Ordering keys: every candidate is one u64, high word = order-preserving
// bits of the score (-0 folded into +0), low word = ~row.  Larger key = better
// (higher score, then lower row), so a descending sort gives the canonical
// (score desc, row asc) order and keys are unique per row.  Key 0 = empty.
#pragma once

#include "bv_kernels.h"
#include "bv_device.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bvk {
namespace {

// ---------------------------------------------------------------- codecs --
// Each codec: Unit (what one lane loads per unit), QT/QN (query registers per
// unit), Acc/NA (NA accumulators per row), acc() adding one unit's
// contribution, and Fin (per-query constants + score finalisation).
//
// int8 / int4 asymmetric scans use a three-level integer split of the rotated
// fp32 query, q ~= s1*q1 + s2*q2 + s3*q3 with q1..q3 int8 (each level
// quantizes the previous residual, so the residual is below 127^-3 of max|q|).
// Every level's dot with the codes is an exact int32 from v_dot4_i32_i8;
// the three are reduced across lanes exactly and combined once per row in
// f64.  This replaces per-code int->float conversion + FMA, which left the
// scan bound by VALU issue instead of HBM.
template <int C> struct Codec;

template <> struct Codec<C_F32DOT> {
    using Unit = uint4; using QT = float; using Acc = float;
    static constexpr int QN = 4, NA = 1;
    static __device__ __forceinline__ void acc(Unit u, const QT *q, Acc *a) {
        a[0] = fmaf(__uint_as_float(u.x), q[0], a[0]);
        a[0] = fmaf(__uint_as_float(u.y), q[1], a[0]);
        a[0] = fmaf(__uint_as_float(u.z), q[2], a[0]);
        a[0] = fmaf(__uint_as_float(u.w), q[3], a[0]);
    }
};
template <> struct Codec<C_F32L2> {
    using Unit = uint4; using QT = float; using Acc = float;
    static constexpr int QN = 4, NA = 1;
    static __device__ __forceinline__ void acc(Unit u, const QT *q, Acc *a) {
        float d0 = __uint_as_float(u.x) - q[0], d1 = __uint_as_float(u.y) - q[1];
        float d2 = __uint_as_float(u.z) - q[2], d3 = __uint_as_float(u.w) - q[3];
        a[0] = fmaf(d0, d0, a[0]); a[0] = fmaf(d1, d1, a[0]); a[0] = fmaf(d2, d2, a[0]); a[0] = fmaf(d3, d3, a[0]);
    }
};
template <> struct Codec<C_F32DOT_S> {
    using Unit = uint32_t; using QT = float; using Acc = float;
    static constexpr int QN = 1, NA = 1;
    static __device__ __forceinline__ void acc(Unit u, const QT *q, Acc *a) { a[0] = fmaf(__uint_as_float(u), q[0], a[0]); }
};
template <> struct Codec<C_F32L2_S> {
    using Unit = uint32_t; using QT = float; using Acc = float;
    static constexpr int QN = 1, NA = 1;
    static __device__ __forceinline__ void acc(Unit u, const QT *q, Acc *a) {
        float d = __uint_as_float(u) - q[0];
        a[0] = fmaf(d, d, a[0]);
    }
};
// int8 codes (16 per unit) x three int8 query levels: q[l*4 + d] holds the
// level-l query bytes matching code dword d.
template <> struct Codec<C_Q8> {
    using Unit = uint4; using QT = uint32_t; using Acc = int32_t;
    static constexpr int QN = 12, NA = 3;
    static __device__ __forceinline__ void acc(Unit u, const QT *q, Acc *a) {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int l = 0; l < 3; ++l) a[l] = __builtin_amdgcn_sdot4((int)w[d], (int)q[l * 4 + d], a[l], false);
    }
};
// int4 codes (32 per unit).  Each signed nibble n is moved to the high half
// of a byte, which reads as the int8 16 * n, so the level dots come out as
// exact 16 * sum(n * q).  q[l*8 + 2d] / q[l*8 + 2d + 1] hold the level-l
// query bytes for the even / odd nibbles of code dword d.
template <> struct Codec<C_Q4> {
    using Unit = uint4; using QT = uint32_t; using Acc = int32_t;
    static constexpr int QN = 24, NA = 3;
    static __device__ __forceinline__ void acc(Unit u, const QT *q, Acc *a) {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            // each nibble in the high half of a byte: the signed byte is 16 * n
            const uint32_t lo = (w[d] << 4) & 0xf0f0f0f0u, hi = w[d] & 0xf0f0f0f0u;
#pragma unroll
            for (int l = 0; l < 3; ++l) {
                a[l] = __builtin_amdgcn_sdot4((int)lo, (int)q[l * 8 + 2 * d], a[l], false);
                a[l] = __builtin_amdgcn_sdot4((int)hi, (int)q[l * 8 + 2 * d + 1], a[l], false);
            }
        }
    }
};
template <> struct Codec<C_Q1A> {
    using Unit = uint32_t; using QT = float; using Acc = float;
    static constexpr int QN = 32, NA = 1;
    static __device__ __forceinline__ void acc(Unit u, const QT *q, Acc *a) {
#pragma unroll
        for (int j = 0; j < 32; ++j) a[0] += ((u >> j) & 1u) ? q[j] : -q[j];
    }
};
template <> struct Codec<C_HAM> {
    using Unit = uint4; using QT = uint32_t; using Acc = int32_t;
    static constexpr int QN = 4, NA = 1;
    static __device__ __forceinline__ void acc(Unit u, const QT *q, Acc *a) {
        a[0] += __popc(u.x ^ q[0]) + __popc(u.y ^ q[1]) + __popc(u.z ^ q[2]) + __popc(u.w ^ q[3]);
    }
};
// 1-bit codes (128 per unit) against the query's two levels held as bit
// planes: q[p*4 + d] is bit p of the int8 level Q1 for the 32 codes of code
// dword d (p < 8), q[32 + p*4 + d] bit p of the int4 level Q2 (p < 4); both
// two's complement, so the top plane weighs -128 / -8.  The sums over the
// unit of code_bit * Q are sum_p weight_p * popcount(code & plane_p), exact
// in int32.
constexpr bool Q1P_L2 = false;  // the int4 residual level (else Q2 = 0; measured slower once the exact re-score is table-driven)
template <> struct Codec<C_Q1P> {
    using Unit = uint4; using QT = uint32_t; using Acc = int32_t;
    static constexpr int QN = Q1P_L2 ? 48 : 32, NA = 2;
    static __device__ __forceinline__ void acc(Unit u, const QT *q, Acc *a) {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int pl = 0; pl < QN / 4; ++pl) {
            int32_t c = 0;
#pragma unroll
            for (int d = 0; d < 4; ++d) c += (int32_t)__popc(w[d] & q[pl * 4 + d]);
            if (pl < 8) a[0] += pl == 7 ? -(c << 7) : (c << pl);
            else a[1] += pl == 11 ? -(c << 3) : (c << (pl - 8));
        }
    }
};
template <> struct Codec<C_I8S> {
    using Unit = uint4; using QT = uint32_t; using Acc = int32_t;
    static constexpr int QN = 4, NA = 1;
    static __device__ __forceinline__ void acc(Unit u, const QT *q, Acc *a) {
        a[0] = __builtin_amdgcn_sdot4((int)u.x, (int)q[0], a[0], false);
        a[0] = __builtin_amdgcn_sdot4((int)u.y, (int)q[1], a[0], false);
        a[0] = __builtin_amdgcn_sdot4((int)u.z, (int)q[2], a[0], false);
        a[0] = __builtin_amdgcn_sdot4((int)u.w, (int)q[3], a[0], false);
    }
};

template <int C> struct IsInt { static constexpr bool v = (C == C_HAM || C == C_I8S); };

// Row-score finalisation from the per-query constants stored after the
// query units (QLevelTail).  `ord` is the order-preserving key word.

template <int C> struct Fin {
    __device__ void load(const void *, uint32_t) {}
    template <class Acc> __device__ __forceinline__ float score(const Acc *t, float scale, uint32_t &ord) const {
        float sc;
        if constexpr (C == C_F32L2 || C == C_F32L2_S) sc = -t[0];
        else if constexpr (C == C_Q1A) sc = t[0] * scale;
        else sc = t[0];
        ord = ord_f32(sc);
        return sc;
    }
};
template <> struct Fin<C_HAM> {
    int32_t P;
    __device__ void load(const void *, uint32_t padded) { P = (int32_t)padded; }
    __device__ __forceinline__ float score(const int32_t *t, float, uint32_t &ord) const {
        const int32_t sim = P - 2 * t[0];
        ord = ord_i32(sim);
        return (float)sim;
    }
};
// The int8 level of the 1-bit asymmetric prefilter (the scan's exact
// re-score uses the fp32 query; score() is not used).
template <> struct Fin<C_Q1P> {
    double s1, s2, rsum, qabs;
    int32_t sumq1, sumq2;
    __device__ void load(const void *tail, uint32_t) {
        const Q1Tail *q = (const Q1Tail *)tail;
        s1 = q->s1;
        s2 = q->s2;
        rsum = q->rsum;
        qabs = q->qabs;
        sumq1 = q->sumq1;
        sumq2 = q->sumq2;
    }
};
template <> struct Fin<C_I8S> {
    __device__ void load(const void *, uint32_t) {}
    __device__ __forceinline__ float score(const int32_t *t, float, uint32_t &ord) const {
        ord = ord_i32(t[0]);
        return (float)t[0];
    }
};
template <> struct Fin<C_Q8> {
    double s0, s1, s2;
    __device__ void load(const void *tail, uint32_t) {
        const QLevelTail *q = (const QLevelTail *)tail;
        s0 = q->s[0]; s1 = q->s[1]; s2 = q->s[2];
    }
    __device__ __forceinline__ float score(const int32_t *t, float scale, uint32_t &ord) const {
        const double v = fma(s2, (double)t[2], fma(s1, (double)t[1], s0 * (double)t[0]));
        const float sc = (float)(v * (double)scale);
        ord = ord_f32(sc);
        return sc;
    }
};
template <> struct Fin<C_Q4> {
    double s0, s1, s2;
    __device__ void load(const void *tail, uint32_t) {
        const QLevelTail *q = (const QLevelTail *)tail;
        s0 = q->s[0]; s1 = q->s[1]; s2 = q->s[2];
    }
    // t[l] = 16 * sum(n * q_l) exactly: the shift recovers the level dot
    __device__ __forceinline__ float score(const int32_t *t, float scale, uint32_t &ord) const {
        const double v = fma(s2, (double)(t[2] >> 4), fma(s1, (double)(t[1] >> 4), s0 * (double)(t[0] >> 4)));
        const float sc = (float)(v * (double)scale);
        ord = ord_f32(sc);
        return sc;
    }
};

// ------------------------------------------------------- wave reductions --
// Cross-lane moves without LDS: DPP within 16-lane rows, and gfx950's
// v_permlane{16,32}_swap across rows / halves.  All indices are compile-time.
template <class T> __device__ __forceinline__ int as_i(T v) { return __builtin_bit_cast(int, v); }
template <class T> __device__ __forceinline__ T from_i(int v) { return __builtin_bit_cast(T, v); }

template <int CTRL, class T> __device__ __forceinline__ T dpp(T v) {
    return from_i<T>(__builtin_amdgcn_update_dpp(0, as_i(v), CTRL, 0xf, 0xf, false));
}
constexpr int DPP_XOR1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane ^ 7 within 8
constexpr int DPP_MIRROR = 0x140;      // lane ^ 15 within 16
constexpr int DPP_ROR8 = 0x128;        // lane ^ 8 within 16

// v + (v of the partner lane that differs in lane bit B), for B = 0..5.
template <int B, class T> __device__ __forceinline__ T plain_step(T v) {
    if constexpr (B == 0) return v + dpp<DPP_XOR1>(v);
    else if constexpr (B == 1) return v + dpp<DPP_XOR2>(v);
    else if constexpr (B == 2) return v + dpp<DPP_HALF_MIRROR>(v);
    else if constexpr (B == 3) return v + dpp<DPP_MIRROR>(v);
    else if constexpr (B == 4) {
        auto r = __builtin_amdgcn_permlane16_swap(as_i(v), as_i(v), false, false);
        return from_i<T>(r[0]) + from_i<T>(r[1]);
    } else {
        auto r = __builtin_amdgcn_permlane32_swap(as_i(v), as_i(v), false, false);
        return from_i<T>(r[0]) + from_i<T>(r[1]);
    }
}

// One transposing exchange on lane bit B (0..5): the lane with bit B clear
// keeps rows [0,h) and the lane with it set keeps rows [h,2h); each adds its
// partner's copy of the kept rows.  The partner of bits 3..0 is a DPP lane
// pattern that flips bit B (lane ^ 8, lane ^ 7 within 8, lane ^ 2, lane ^ 1):
// any pairing that flips bit B and keeps the higher bits leaves the lanes
// with bit B clear holding, between them, the whole group's sum.
template <int B, int H, class T> __device__ __forceinline__ void xpose_step(T *v, int lane) {
#pragma unroll
    for (int j = 0; j < H; ++j) {
        if constexpr (B == 5 || B == 4) {
            auto r = (B == 5) ? __builtin_amdgcn_permlane32_swap(as_i(v[j]), as_i(v[j + H]), false, false)
                              : __builtin_amdgcn_permlane16_swap(as_i(v[j]), as_i(v[j + H]), false, false);
            v[j] = from_i<T>(r[0]) + from_i<T>(r[1]);
        } else {
            constexpr int CTRL = B == 3 ? DPP_ROR8 : B == 2 ? DPP_HALF_MIRROR : B == 1 ? DPP_XOR2 : DPP_XOR1;
            const bool hi = (lane >> B) & 1;
            const T send = hi ? v[j] : v[j + H];
            const T keep = hi ? v[j + H] : v[j];
            v[j] = keep + dpp<CTRL>(send);
        }
    }
}

// Reduce U per-lane partials over an aligned group of LPR lanes.  Transposing
// stages use lane bits log2(LPR)-1 downwards (one per halving of U); plain
// stages cover the remaining low bits.  Afterwards every lane holds the full
// sum of row group xrow<U, LPR>(lane); lanes with the low bits clear are the
// distinct representatives.
template <int U, int LPR> struct Lg {
    static constexpr int lu = U == 1 ? 0 : U == 2 ? 1 : U == 4 ? 2 : 3;
    static constexpr int ll = LPR == 4 ? 2 : LPR == 8 ? 3 : LPR == 16 ? 4 : LPR == 32 ? 5 : 6;
    static constexpr int low = ll - lu;  // number of plain (low) bits
};

template <int U, int LPR, class T> __device__ __forceinline__ T xreduce(T (&v)[U], int lane) {
    static_assert(Lg<U, LPR>::low >= 0, "U must not exceed LPR");
    constexpr int ll = Lg<U, LPR>::ll;
    if constexpr (U >= 2) xpose_step<ll - 1, U / 2>(v, lane);
    if constexpr (U >= 4) xpose_step<ll - 2, U / 4>(v, lane);
    if constexpr (U >= 8) xpose_step<ll - 3, U / 8>(v, lane);
    T x = v[0];
    constexpr int low = Lg<U, LPR>::low;
    if constexpr (low > 0) x = plain_step<0>(x);
    if constexpr (low > 1) x = plain_step<1>(x);
    if constexpr (low > 2) x = plain_step<2>(x);
    if constexpr (low > 3) x = plain_step<3>(x);
    if constexpr (low > 4) x = plain_step<4>(x);
    if constexpr (low > 5) x = plain_step<5>(x);
    return x;
}

template <int U, int LPR> __device__ __forceinline__ int xrow(int lane) {
    constexpr int ll = Lg<U, LPR>::ll;
    int j = 0;
    if constexpr (U >= 2) j += ((lane >> (ll - 1)) & 1) ? U / 2 : 0;
    if constexpr (U >= 4) j += ((lane >> (ll - 2)) & 1) ? U / 4 : 0;
    if constexpr (U >= 8) j += ((lane >> (ll - 3)) & 1) ? U / 8 : 0;
    return j;
}

template <int U, int LPR> __device__ __forceinline__ bool xrep(int lane) {
    return (lane & ((1 << Lg<U, LPR>::low) - 1)) == 0;
}

// The value of lane ^ M (M = 1 .. 32) by DPP or a row / half swap, without
// the LDS crossbar.  xor 4 within a 16-lane row: row_shl:4 for lanes with
// bit 2 clear, row_shr:4 for the others (no lane reads outside its row).
constexpr int DPP_ROW_SHL4 = 0x104;
constexpr int DPP_ROW_SHR4 = 0x114;
// Both moves of a pair run with every lane active, and one of the two
// results is picked with integer masks: a select the compiler turned into a
// branch would run each move with half the lanes disabled, and a move that
// reads a disabled lane gets zero.
__device__ __forceinline__ int pick_bits(int lo_val, int hi_val, bool hi) {
    const int m = -(int)hi;  // all ones when hi
    return lo_val ^ ((lo_val ^ hi_val) & m);
}
template <int M> __device__ __forceinline__ float lane_xor(float x, int lane) {
    if constexpr (M == 1) return dpp<DPP_XOR1>(x);
    else if constexpr (M == 2) return dpp<DPP_XOR2>(x);
    else if constexpr (M == 4) {
        const int up = as_i(dpp<DPP_ROW_SHL4>(x)), down = as_i(dpp<DPP_ROW_SHR4>(x));
        return from_i<float>(pick_bits(up, down, (lane & 4) != 0));
    } else if constexpr (M == 8) return dpp<DPP_ROR8>(x);
    else {
        // the swap returns two copies: lanes of the lower row / half find
        // their partner in the second, the others in the first
        auto r = (M == 16) ? __builtin_amdgcn_permlane16_swap(as_i(x), as_i(x), false, false)
                           : __builtin_amdgcn_permlane32_swap(as_i(x), as_i(x), false, false);
        return from_i<float>(pick_bits(r[1], r[0], (lane & M) != 0));
    }
}

// One radix-2 FWHT stage across lanes (partner lane ^ M): the lane with bit
// M clear holds the lower element u and keeps u + w, the other keeps u - w,
// the reference's butterfly (src/quant/rotator.ts:24-36).
template <int M, int E> __device__ __forceinline__ void fwht_xlane(float (&x)[E], int lane) {
#pragma clang fp contract(off)
    const bool hi = (lane & M) != 0;
#pragma unroll
    for (int t = 0; t < E; ++t) {
        const float y = lane_xor<M>(x[t], lane);
        x[t] = hi ? (y - x[t]) : (x[t] + y);
    }
}
template <int E> __device__ __forceinline__ void fwht_xlane64(float (&x)[E], int lane) {
    fwht_xlane<1>(x, lane);
    fwht_xlane<2>(x, lane);
    fwht_xlane<4>(x, lane);
    fwht_xlane<8>(x, lane);
    fwht_xlane<16>(x, lane);
    fwht_xlane<32>(x, lane);
}

// The u64 of lane ^ M, by the same moves as lane_xor.
template <int M> __device__ __forceinline__ uint64_t lane_xor_u64(uint64_t x, int lane) {
    const float lo = lane_xor<M>(__builtin_bit_cast(float, (uint32_t)x), lane);
    const float hi = lane_xor<M>(__builtin_bit_cast(float, (uint32_t)(x >> 32)), lane);
    return ((uint64_t)__builtin_bit_cast(uint32_t, hi) << 32) | __builtin_bit_cast(uint32_t, lo);
}

// One compare-exchange stage (partner distance J, merge block size kk) of a
// bitonic sort of 128 (key, payload) pairs held two per lane: element
// lane + 64 s in k[s], v[s].  Keys are distinct; the sort is descending.
template <int J>
__device__ __forceinline__ void bitonic128_stage(uint64_t (&k)[2], uint64_t (&v)[2], int lane, uint32_t kk) {
    uint64_t pk[2], pv[2];
    if constexpr (J == 64) {
        pk[0] = k[1]; pv[0] = v[1];
        pk[1] = k[0]; pv[1] = v[0];
    } else {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            pk[t] = lane_xor_u64<J>(k[t], lane);
            pv[t] = lane_xor_u64<J>(v[t], lane);
        }
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const uint32_t e = (uint32_t)lane + 64u * t;
        const bool lower = (e & J) == 0, desc = (e & kk) == 0;
        const bool keep = (lower == desc) == (k[t] > pk[t]);  // keep the larger key iff lower == desc
        k[t] = keep ? k[t] : pk[t];
        v[t] = keep ? v[t] : pv[t];
    }
}
// Sorts the 128 pairs descending by key (the whole wave takes part).
__device__ __forceinline__ void bitonic128(uint64_t (&k)[2], uint64_t (&v)[2], int lane) {
#pragma unroll
    for (uint32_t kk = 2; kk <= 128; kk <<= 1) {
        if (kk >= 128) bitonic128_stage<64>(k, v, lane, kk);
        if (kk >= 64) bitonic128_stage<32>(k, v, lane, kk);
        if (kk >= 32) bitonic128_stage<16>(k, v, lane, kk);
        if (kk >= 16) bitonic128_stage<8>(k, v, lane, kk);
        if (kk >= 8) bitonic128_stage<4>(k, v, lane, kk);
        if (kk >= 4) bitonic128_stage<2>(k, v, lane, kk);
        bitonic128_stage<1>(k, v, lane, kk);
    }
}

// Wave-wide f64 maximum (fmax: a NaN operand never wins) and i32 sum, in
// every lane, through DPP / swaps on the 32-bit halves.
__device__ __forceinline__ double wave_fmax_f64(double v) {
#define BV_FMAX_STEP(GET)                                                        \
    {                                                                            \
        const uint64_t b = __builtin_bit_cast(uint64_t, v);                      \
        const uint32_t lo = GET((uint32_t)b), hi = GET((uint32_t)(b >> 32));     \
        v = fmax(v, __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo));      \
    }
#define BV_DPP_GET(C) [](uint32_t w) { return dpp<C>(w); }
    BV_FMAX_STEP(BV_DPP_GET(DPP_XOR1))
    BV_FMAX_STEP(BV_DPP_GET(DPP_XOR2))
    BV_FMAX_STEP(BV_DPP_GET(DPP_HALF_MIRROR))
    BV_FMAX_STEP(BV_DPP_GET(DPP_MIRROR))
#undef BV_DPP_GET
#undef BV_FMAX_STEP
    {
        const uint64_t b = __builtin_bit_cast(uint64_t, v);
        auto l = __builtin_amdgcn_permlane16_swap((int)(uint32_t)b, (int)(uint32_t)b, false, false);
        auto h = __builtin_amdgcn_permlane16_swap((int)(uint32_t)(b >> 32), (int)(uint32_t)(b >> 32), false, false);
        const double x = __builtin_bit_cast(double, ((uint64_t)(uint32_t)h[0] << 32) | (uint32_t)l[0]);
        const double y = __builtin_bit_cast(double, ((uint64_t)(uint32_t)h[1] << 32) | (uint32_t)l[1]);
        v = fmax(x, y);
    }
    {
        const uint64_t b = __builtin_bit_cast(uint64_t, v);
        auto l = __builtin_amdgcn_permlane32_swap((int)(uint32_t)b, (int)(uint32_t)b, false, false);
        auto h = __builtin_amdgcn_permlane32_swap((int)(uint32_t)(b >> 32), (int)(uint32_t)(b >> 32), false, false);
        const double x = __builtin_bit_cast(double, ((uint64_t)(uint32_t)h[0] << 32) | (uint32_t)l[0]);
        const double y = __builtin_bit_cast(double, ((uint64_t)(uint32_t)h[1] << 32) | (uint32_t)l[1]);
        v = fmax(x, y);
    }
    return v;
}
// Wave-wide f64 sum in every lane (the same pairing as wave_fmax_f64; each
// pair adds the same two values, so every lane ends with the same sum).
__device__ __forceinline__ double wave_sum_f64(double v) {
#define BV_SUM_STEP(GET)                                                         \
    {                                                                            \
        const uint64_t b = __builtin_bit_cast(uint64_t, v);                      \
        const uint32_t lo = GET((uint32_t)b), hi = GET((uint32_t)(b >> 32));     \
        v = v + __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);           \
    }
#define BV_DPP_GET(C) [](uint32_t w) { return dpp<C>(w); }
    BV_SUM_STEP(BV_DPP_GET(DPP_XOR1))
    BV_SUM_STEP(BV_DPP_GET(DPP_XOR2))
    BV_SUM_STEP(BV_DPP_GET(DPP_HALF_MIRROR))
    BV_SUM_STEP(BV_DPP_GET(DPP_MIRROR))
#undef BV_DPP_GET
#undef BV_SUM_STEP
    {
        const uint64_t b = __builtin_bit_cast(uint64_t, v);
        auto l = __builtin_amdgcn_permlane16_swap((int)(uint32_t)b, (int)(uint32_t)b, false, false);
        auto h = __builtin_amdgcn_permlane16_swap((int)(uint32_t)(b >> 32), (int)(uint32_t)(b >> 32), false, false);
        const double x = __builtin_bit_cast(double, ((uint64_t)(uint32_t)h[0] << 32) | (uint32_t)l[0]);
        const double y = __builtin_bit_cast(double, ((uint64_t)(uint32_t)h[1] << 32) | (uint32_t)l[1]);
        v = x + y;
    }
    {
        const uint64_t b = __builtin_bit_cast(uint64_t, v);
        auto l = __builtin_amdgcn_permlane32_swap((int)(uint32_t)b, (int)(uint32_t)b, false, false);
        auto h = __builtin_amdgcn_permlane32_swap((int)(uint32_t)(b >> 32), (int)(uint32_t)(b >> 32), false, false);
        const double x = __builtin_bit_cast(double, ((uint64_t)(uint32_t)h[0] << 32) | (uint32_t)l[0]);
        const double y = __builtin_bit_cast(double, ((uint64_t)(uint32_t)h[1] << 32) | (uint32_t)l[1]);
        v = x + y;
    }
    return v;
}
__device__ __forceinline__ int32_t wave_sum_i32(int32_t v) {
    v = plain_step<0>(v);
    v = plain_step<1>(v);
    v = plain_step<2>(v);
    v = plain_step<3>(v);
    v = plain_step<4>(v);
    return plain_step<5>(v);
}

// ------------------------------------------------------- LDS top-k state --
constexpr int SEL_BINS = 1024;  // histogram bins of the selection
constexpr int SEL_TMP = 1024;   // gather buffer of the selection

struct TopkLds {
    uint64_t keys[SCAN_CAP];    // candidate keys (final selection with re-rank: scan keys in
                                // [0, SCAN_CAP/2), their exact keys at the same index + SCAN_CAP/2)
    uint64_t tmp[SEL_TMP];      // selection gather buffer
    uint32_t hist[SEL_BINS];
    uint32_t red[16];           // cross-wave reduction slots
    uint32_t ovl[SCAN_WG];      // final selection: per-group flush counts, then their prefix
    uint32_t cnt, cnt2, bstar, above, flag, last, grab;
    uint64_t tau, gtau;
};

// Bitonic sort (descending) of keys[0, npow) by the whole workgroup.
__device__ void bitonic_desc(uint64_t *keys, uint32_t npow) {
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    for (uint32_t k = 2; k <= npow; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = tid; i < npow; i += nt) {
                uint32_t ixj = i ^ j;
                if (ixj > i) {
                    uint64_t x = keys[i], y = keys[ixj];
                    bool desc = (i & k) == 0;
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

__device__ __forceinline__ uint32_t pow2_at_least(uint32_t n) {
    uint32_t p = 2;
    while (p < n) p <<= 1;
    return p;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) v = max(v, (uint32_t)__shfl_xor((int)v, s));
    return v;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) v = min(v, (uint32_t)__shfl_xor((int)v, s));
    return v;
}

// #{keys in ks[0, n) greater than `mine`}; ks in LDS, read by every lane
// alike (broadcast), 16 reads in flight per batch.
__device__ __forceinline__ uint32_t count_greater(const uint64_t *ks, uint32_t n, uint64_t mine) {
    uint32_t r = 0, j = 0;
    for (; j + 16 <= n; j += 16) {
        uint64_t v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = ks[j + u];
#pragma unroll
        for (int u = 0; u < 16; ++u) r += v[u] > mine ? 1u : 0u;
    }
    for (; j < n; ++j) r += ks[j] > mine ? 1u : 0u;
    return r;
}

// Keeps the best `kk` (>= 1) of L.keys[0, n) (unique, nonzero) in
// L.keys[0, m), sorted descending, and returns m = min(n, kk).  Small inputs
// are sorted outright; larger ones are binned by the score bits over their
// actual range (1024 bins), the bin holding the kk-th key is located with a
// suffix scan, and only keys from that bin upwards are gathered and sorted.
// Whole workgroup; starts and ends with a barrier.
__device__ __noinline__ uint32_t select_topk(TopkLds &L, uint32_t n, uint32_t kk) {
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6, nwaves = nt >> 6;
    __syncthreads();
    if (n <= 256) {
        // rank by counting: key i goes to slot #{keys greater than it}
        uint64_t mine = 0;
        uint32_t rank = 0;
        if (tid < n) {
            mine = L.keys[tid];
            rank = count_greater(L.keys, n, mine);
        }
        __syncthreads();
        if (tid < n && rank < kk) L.keys[rank] = mine;
        __syncthreads();
        return n < kk ? n : kk;
    }
    if (n <= kk) {
        const uint32_t npow = pow2_at_least(n);
        for (uint32_t i = n + tid; i < npow; i += nt) L.keys[i] = 0;
        __syncthreads();
        bitonic_desc(L.keys, npow);
        return n;
    }
    // range of the high (score) words
    uint32_t mx = 0, mn = 0xffffffffu;
    for (uint32_t i = tid; i < n; i += nt) {
        const uint32_t h = (uint32_t)(L.keys[i] >> 32);
        mx = max(mx, h);
        mn = min(mn, h);
    }
    mx = wave_max_u32(mx);
    mn = wave_min_u32(mn);
    if (lane == 0) {
        L.red[wave] = mx;
        L.red[8 + wave] = mn;
    }
    for (uint32_t b = tid; b < SEL_BINS; b += nt) L.hist[b] = 0;
    __syncthreads();
    mx = 0;
    mn = 0xffffffffu;
    for (int w = 0; w < nwaves; ++w) {
        mx = max(mx, L.red[w]);
        mn = min(mn, L.red[8 + w]);
    }
    const uint32_t span = mx - mn;
    uint32_t sh = 0;
    while ((span >> sh) >= (uint32_t)SEL_BINS) ++sh;
    for (uint32_t i = tid; i < n; i += nt)
        atomicAdd(&L.hist[((uint32_t)(L.keys[i] >> 32) - mn) >> sh], 1u);
    __syncthreads();
    // b* = highest bin whose suffix count reaches kk (wave 0: 16 bins per lane)
    if (wave == 0) {
        constexpr int PER = SEL_BINS / 64;
        uint32_t loc = 0;
#pragma unroll
        for (int j = 0; j < PER; ++j) loc += L.hist[lane * PER + j];
        // inclusive suffix sum over lanes: T(l) = sum_{l' >= l} loc(l')
        uint32_t T = loc;
#pragma unroll
        for (int s = 1; s < 64; s <<= 1) {
            const uint32_t o = (uint32_t)__shfl_down((int)T, s);
            if (lane + s < 64) T += o;
        }
        const uint32_t Tnext = T - loc;  // suffix from the next lane up
        if (Tnext < kk && T >= kk) {
            uint32_t run = Tnext;
            for (int j = PER - 1; j >= 0; --j) {
                const uint32_t h = L.hist[lane * PER + j];
                if (run + h >= kk) {
                    L.bstar = lane * PER + j;
                    L.above = run + h;  // keys in bins >= b*
                    break;
                }
                run += h;
            }
        }
    }
    if (tid == 0) L.cnt2 = 0;
    __syncthreads();
    const uint32_t bstar = L.bstar, c = L.above;
    if (c <= (uint32_t)SEL_TMP) {
        for (uint32_t i = tid; i < n; i += nt) {
            const uint64_t k = L.keys[i];
            if ((((uint32_t)(k >> 32) - mn) >> sh) >= bstar) L.tmp[atomicAdd(&L.cnt2, 1u)] = k;
        }
        __syncthreads();
        if (c <= nt) {
            uint64_t mine = 0;
            uint32_t rank = 0;
            if (tid < c) {
                mine = L.tmp[tid];
                rank = count_greater(L.tmp, c, mine);
            }
            __syncthreads();
            if (tid < c && rank < kk) L.keys[rank] = mine;
            __syncthreads();
            return kk;
        }
        const uint32_t npow = pow2_at_least(c);
        for (uint32_t i = c + tid; i < npow; i += nt) L.tmp[i] = 0;
        __syncthreads();
        bitonic_desc(L.tmp, npow);
        for (uint32_t i = tid; i < kk; i += nt) L.keys[i] = L.tmp[i];
        __syncthreads();
        return kk;
    }
    // many keys share the k-th key's bin (ties): sort everything
    const uint32_t npow = pow2_at_least(n);
    for (uint32_t i = n + tid; i < npow; i += nt) L.keys[i] = 0;
    __syncthreads();
    bitonic_desc(L.keys, npow);
    return kk;
}

// Wave-level append to a shared LDS list: one atomic per wave.  Keys whose
// slot would reach `cap` are dropped (callers size cap so that only the
// threshold helper, which may use any subset, can hit it).
__device__ __forceinline__ void wave_append(uint64_t *keys, uint32_t *cnt, uint32_t cap, bool take, uint64_t key,
                                            int lane) {
    const uint64_t ball = __ballot(take);
    if (ball == 0) return;
    const uint32_t total = __popcll(ball);
    const int leader = __ffsll((unsigned long long)ball) - 1;
    uint32_t base = 0;
    if (lane == leader) base = atomicAdd(cnt, total);
    base = __shfl(base, leader);
    if (take) {
        const uint32_t below =
            __builtin_amdgcn_mbcnt_hi((uint32_t)(ball >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)ball, 0u));
        if (base + below < cap) keys[base + below] = key;
    }
}

// The maximum over the wave, in every lane: DPP moves within 16-lane rows
// (xor 1, xor 2, mirror within 8, mirror within 16) and row / half swaps,
// each step pairing every lane with one whose range it has not seen.
template <int CTRL> __device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xf, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xf, 0xf, false);
    return ((uint64_t)hi << 32) | lo;
}
template <bool HALF32> __device__ __forceinline__ uint64_t swap_max_u64(uint64_t v) {
    const int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
    auto a = HALF32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                    : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    auto b = HALF32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                    : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    const uint64_t x = ((uint64_t)(uint32_t)b[0] << 32) | (uint32_t)a[0];
    const uint64_t y = ((uint64_t)(uint32_t)b[1] << 32) | (uint32_t)a[1];
    return x > y ? x : y;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    uint64_t o;
    o = dpp_u64<DPP_XOR1>(v);
    v = o > v ? o : v;
    o = dpp_u64<DPP_XOR2>(v);
    v = o > v ? o : v;
    o = dpp_u64<DPP_HALF_MIRROR>(v);
    v = o > v ? o : v;
    o = dpp_u64<DPP_MIRROR>(v);
    v = o > v ? o : v;
    v = swap_max_u64<false>(v);
    return swap_max_u64<true>(v);
}

// wave_append for (key, companion) pairs stored at the same index.
__device__ __forceinline__ void wave_append2(uint64_t *keys, uint64_t *comp, uint32_t *cnt, uint32_t cap, bool take,
                                             uint64_t key, uint64_t c, int lane) {
    const uint64_t ball = __ballot(take);
    if (ball == 0) return;
    const uint32_t total = __popcll(ball);
    const int leader = __ffsll((unsigned long long)ball) - 1;
    uint32_t base = 0;
    if (lane == leader) base = atomicAdd(cnt, total);
    base = __shfl(base, leader);
    if (take) {
        const uint32_t i = base + __builtin_amdgcn_mbcnt_hi((uint32_t)(ball >> 32),
                                                            __builtin_amdgcn_mbcnt_lo((uint32_t)ball, 0u));
        if (i < cap) {
            keys[i] = key;
            comp[i] = c;
        }
    }
}

// ------------------------------------------------- per-wave candidate lists --
// During the scan every wave owns a private list wk[0, wc) in LDS; wc is
// wave-uniform, so appends need no atomics and no workgroup barriers.

__device__ __forceinline__ uint32_t lanes_below(uint64_t ball) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(ball >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)ball, 0u));
}
__device__ __forceinline__ uint64_t uniform_u64(uint64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ void wave_push(uint64_t *wk, uint32_t &wc, bool take, uint64_t key) {
    const uint64_t ball = __ballot(take);
    if (take) wk[wc + lanes_below(ball)] = key;
    wc += (uint32_t)__popcll(ball);
}

// Keeps the keys >= t of wk[0, wc) in place (order kept); returns the count.
// Each 64-key chunk is read by the whole wave before any lane writes, and
// writes land at or below the chunk, so the compaction is safe in place.
__device__ uint32_t wave_filter(uint64_t *wk, uint32_t wc, uint64_t t, int lane) {
    uint32_t out = 0;
    for (uint32_t j = 0; j < wc; j += 64) {
        const uint32_t i = j + lane;
        const uint64_t k = i < wc ? wk[i] : 0;
        wave_push(wk, out, i < wc && k >= t, k);
    }
    return out;
}

__device__ uint32_t wave_count_ge(const uint64_t *wk, uint32_t wc, uint64_t t, int lane) {
    uint32_t c = 0;
    for (uint32_t j = 0; j < wc; j += 64) {
        const uint32_t i = j + lane;
        c += (uint32_t)__popcll(__ballot(i < wc && wk[i] >= t));
    }
    return c;
}

// A bound t with kp <= #{keys >= t} <= target, for a list whose keys are all
// >= lo and unique, with kp <= target < wc.  Bisection on the key value: the
// count drops by at most one per unit step of t, so some t in (lo, max] has
// exactly kp keys at or above it and the search always lands in the window.
// Any such t is at most the kp-th best of the list, hence at most the
// kp-th best of the whole scan: a valid pruning bound.
__device__ uint64_t wave_bound(const uint64_t *wk, uint32_t wc, uint64_t lo, uint32_t kp, uint32_t target, int lane) {
    uint64_t mx = 0;
    for (uint32_t j = lane; j < wc; j += 64) mx = wk[j] > mx ? wk[j] : mx;
    uint64_t hi = uniform_u64(wave_max_u64(mx)) + 1;  // nothing at or above hi
    while (hi - lo > 1) {
        const uint64_t mid = lo + ((hi - lo) >> 1);
        const uint32_t c = wave_count_ge(wk, wc, mid, lane);
        if (c < kp) hi = mid;
        else if (c > target) lo = mid;
        else return mid;
    }
    return lo;
}

// ---------------------------------------------------------------- encode --
// Wave-level building blocks shared by the row encoder and the query
// transform inside the scan.  A wave holds one padded row; lane l holds
// elements [l*E, l*E+E) (E = P/64, or E = 1 with P lanes when P < 64).

// Rotator.rotateInto (src/quant/rotator.ts:61-70): per round, multiply by
// the round's signs (f32), then the in-place FWHT with len = 1, 2, 4, ...
// Butterflies within a lane first, then across lanes (partner = lane ^
// (len / E)); every butterfly is the reference's f32 (u+v, u-v).
// rotate_load issues every global read up front (the row and the signs of
// the first two rounds) so they cost one memory round trip; rotate_apply
// does the arithmetic.
template <int E> struct RotIn {
    float x[E];
    float s[2][E];
};

// Every load is unconditional, of a clamped address (rounds >= 1, and the
// sign table has rounds x P entries): a load under a condition makes the
// compiler wait for it (and, the load counter draining in order, for every
// older load) where the two paths join, instead of where the value is first
// used.  The values are masked at first use, in rotate_apply.
template <int E>
__device__ __forceinline__ void rotate_load(const float *src, uint32_t dim, uint32_t P, const float *signs,
                                            uint32_t rounds, RotIn<E> &in, int lane) {
    const uint32_t e0 = lane * E;
#pragma unroll
    for (int t = 0; t < E; ++t) {
        const uint32_t e = e0 + t;
        in.x[t] = src[e < dim ? e : dim - 1];
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const uint32_t rr = (uint32_t)r < rounds ? (uint32_t)r : 0u;
#pragma unroll
        for (int t = 0; t < E; ++t) {
            const uint32_t e = e0 + t;
            in.s[r][t] = signs[(size_t)rr * P + (e < P ? e : P - 1)];
        }
    }
}

// The rounds: the first two from the signs loaded up front, any further ones
// (never by default) from a load of their own, in a loop of their own so that
// no wait for it lands on the common path.
template <int E>
__device__ __forceinline__ void rotate_apply(RotIn<E> &in, uint32_t dim, uint32_t P, const float *signs,
                                             uint32_t rounds, float (&x)[E], int lane) {
#pragma clang fp contract(off)
    const uint32_t lanes_used = P / E;
    const uint32_t e0 = lane * E;
    const bool active = (uint32_t)lane < lanes_used;
#pragma unroll
    for (int t = 0; t < E; ++t) x[t] = (active && e0 + t < dim) ? in.x[t] : 0.0f;
    auto one_round = [&](const float (&sg)[E]) {
#pragma unroll
        for (int t = 0; t < E; ++t) x[t] = active ? x[t] * sg[t] : 0.0f;
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
        if (lanes_used == 64) {
            fwht_xlane64<E>(x, lane);
        } else {
            for (uint32_t m = 1; m < lanes_used; m <<= 1) {
                const bool hi = (lane & m) != 0;
#pragma unroll
                for (int t = 0; t < E; ++t) {
                    const float y = __shfl_xor(x[t], (int)m);
                    x[t] = hi ? (y - x[t]) : (x[t] + y);
                }
            }
        }
    };
    one_round(in.s[0]);
    if (rounds > 1) one_round(in.s[1]);
    for (uint32_t r = 2; r < rounds; ++r) {
        float sg[E];
#pragma unroll
        for (int t = 0; t < E; ++t) {
            const uint32_t e = e0 + t;
            sg[t] = signs[(size_t)r * P + (e < P ? e : P - 1)];
        }
        one_round(sg);
    }
}

template <int E>
__device__ __forceinline__ void rotate_wave(const float *src, uint32_t dim, uint32_t P, const float *signs,
                                            uint32_t rounds, float (&x)[E], int lane) {
    RotIn<E> in;
    rotate_load<E>(src, dim, P, signs, rounds, in, lane);
    rotate_apply<E>(in, dim, P, signs, rounds, x, lane);
}

// quantizeRow8 / quantizeRow4 / quantizeRow1 of a rotated row held by the
// wave (src/quant/codec.ts:22-154): codes packed LSB-first into `codes`
// (P/4, P/8 or P/32 words) and, when `scale` is set, the row scale.
// cbytes: P bytes and fbuf: 4P bytes of wave-private LDS.
template <int E>
__device__ void quantize_store_wave(const float (&x)[E], uint32_t P, uint32_t bits, unsigned char *cbytes,
                                    float *fbuf, uint32_t *codes, float *scale, uint32_t *slow_rows, int lane) {
#pragma clang fp contract(off)
    const uint32_t lanes_used = P / E;
    const uint32_t e0 = lane * E;
    const bool active = (uint32_t)lane < lanes_used;
    if (bits == 8 || bits == 4) {
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
        const double sc = m > 0.0f ? (double)m : 1.0;
        const double inv = 1.0 / sc;
        const double levels = bits == 8 ? 127.0 : 7.0;
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
            if (active) cbytes[e0 + t] = (unsigned char)(code & (bits == 8 ? 0xff : 0xf));
        }
        if (scale && lane == 0) *scale = (float)sc;
    } else {  // 1-bit: signs, and mean |x| as a sequential f64 sum
#pragma unroll
        for (int t = 0; t < E; ++t)
            if (active) cbytes[e0 + t] = x[t] >= 0.0f ? 1 : 0;
        if (scale) {
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
                    if (slow_rows) atomicAdd(slow_rows, 1u);
                }
                s = __shfl(seq, 0);
            }
            if (lane == 0) *scale = s > 0.0 ? (float)(s / (double)P) : 1.0f;
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    // pack: word g covers `per` consecutive codes
    const uint32_t per = bits == 8 ? 4 : (bits == 4 ? 8 : 32);
    const uint32_t W = P / per, sh = bits == 8 ? 8 : (bits == 4 ? 4 : 1);
    for (uint32_t g = lane; g < W; g += 64) {
        uint32_t w = 0;
        for (uint32_t j = 0; j < per; ++j) w |= (uint32_t)cbytes[g * per + j] << (sh * j);
        codes[g] = w;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

// One wave per row: rotate, optionally store the rotation, quantize + pack.
template <int E>
__global__ __launch_bounds__(128) void encode_rows(EncodeArgs a) {
    extern __shared__ unsigned char smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t P = a.P;
    unsigned char *cbytes = smem + (size_t)wave * (P + 4 * P);
    float *fbuf = (float *)(cbytes + P);
    const uint32_t lanes_used = P / E;
    const uint32_t e0 = lane * E;
    const bool active = (uint32_t)lane < lanes_used;
    const uint64_t nwaves = (uint64_t)gridDim.x * (blockDim.x >> 6);
    for (uint64_t row = (uint64_t)blockIdx.x * (blockDim.x >> 6) + wave; row < a.rows; row += nwaves) {
        float x[E];
        rotate_wave<E>(a.src + row * a.dim, a.dim, P, a.signs, a.rounds, x, lane);
        if (a.rotated && active) {
#pragma unroll
            for (int t = 0; t < E; ++t) a.rotated[row * P + e0 + t] = x[t];
        }
        if (a.sample_slot && active) {  // IVF reservoir: the rotated row goes to its sample slot
            const int32_t slot = a.sample_slot[row];
            if (slot >= 0) {
#pragma unroll
                for (int t = 0; t < E; ++t) a.sample[(uint64_t)slot * P + e0 + t] = x[t];
            }
        }
        if (a.bits == 0) continue;
        const uint32_t W = P / (a.bits == 8 ? 4 : (a.bits == 4 ? 8 : 32));
        quantize_store_wave<E>(x, P, a.bits, cbytes, fbuf, a.codes + row * W, a.scales + row, a.slow_rows, lane);
    }
}

// ---------------------------------------------------------- query levels --
// Splits a rotated query into three int8 levels (q ~= s1*q1 + s2*q2 + s3*q3,
// each level quantizing the previous residual in f64) and packs them in the
// per-unit layout the int8 / int4 scan codecs read, followed by QLevelTail.
// The wave holds the query as in rotate_wave; lv: 3P bytes of LDS.
template <int E>
__device__ void levels_wave(const float (&x)[E], uint32_t P, int codec, signed char *lv, unsigned char *out,
                            int lane) {
    const uint32_t lanes_used = P / E;
    const uint32_t e0 = lane * E;
    const bool active = (uint32_t)lane < lanes_used;
    double rd[E];
#pragma unroll
    for (int t = 0; t < E; ++t) rd[t] = active ? (double)x[t] : 0.0;
    double sl[3];
    int32_t sums[3];
#pragma unroll
    for (int l = 0; l < 3; ++l) {
        double m = 0.0;
#pragma unroll
        for (int t = 0; t < E; ++t) m = fmax(m, fabs(rd[t]));
        m = wave_fmax_f64(m);
        const double sc = m > 0.0 ? m / 127.0 : 0.0;
        const double inv = sc > 0.0 ? 1.0 / sc : 0.0;
        int32_t sum = 0;
#pragma unroll
        for (int t = 0; t < E; ++t) {
            double c = rint(rd[t] * inv);
            c = c > 127.0 ? 127.0 : (c < -127.0 ? -127.0 : c);
            rd[t] = fma(-sc, c, rd[t]);  // exact residual bookkeeping in f64
            if (active) lv[l * P + e0 + t] = (signed char)(int)c;
            sum += (int)c;
        }
        sum = wave_sum_i32(sum);
        sl[l] = sc;
        sums[l] = sum;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    uint32_t *w = (uint32_t *)out;
    const unsigned char *lb = (const unsigned char *)lv;
    uint32_t qwords;
    if (codec == C_Q8 || codec == C_Q4M) {
        const uint32_t units = P / 16;
        qwords = units * 12;
        for (uint32_t i = lane; i < qwords; i += 64) {
            const uint32_t u = i / 12, r = i % 12, l = r / 4, d = r % 4;
            const uint32_t base = l * P + 16 * u + 4 * d;
            w[i] = (uint32_t)lb[base] | ((uint32_t)lb[base + 1] << 8) | ((uint32_t)lb[base + 2] << 16) |
                   ((uint32_t)lb[base + 3] << 24);
        }
    } else {  // C_Q4
        const uint32_t units = P / 32;
        qwords = units * 24;
        for (uint32_t i = lane; i < qwords; i += 64) {
            const uint32_t u = i / 24, r = i % 24, l = r / 8, d = (r % 8) / 2, h = r % 2;
            const uint32_t base = l * P + 32 * u + 8 * d + h;
            w[i] = (uint32_t)lb[base] | ((uint32_t)lb[base + 2] << 8) | ((uint32_t)lb[base + 4] << 16) |
                   ((uint32_t)lb[base + 6] << 24);
        }
    }
    if (lane == 0) {
        QLevelTail *t = (QLevelTail *)(out + (uint64_t)qwords * 4);
        const double div = codec == C_Q8 ? 127.0 : 1.0;
        for (int l = 0; l < 3; ++l) {
            t->s[l] = sl[l] / div;
            t->sum[l] = sums[l];
        }
        t->pad = 0;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

// Standalone level split of rotated queries (nq x P): one wave per query.
template <int E>
__global__ __launch_bounds__(64) void query_levels(LevelArgs a) {
    extern __shared__ unsigned char lsm[];
    const uint32_t P = a.P, qi = blockIdx.x;
    const int lane = threadIdx.x;
    const uint32_t lanes_used = P / E, e0 = lane * E;
    float x[E];
    const float *q = a.qrot + (uint64_t)qi * P;
#pragma unroll
    for (int t = 0; t < E; ++t) x[t] = (uint32_t)lane < lanes_used ? q[e0 + t] : 0.0f;
    levels_wave<E>(x, P, a.codec, (signed char *)lsm, a.out + (uint64_t)qi * a.stride, lane);
}

// C_Q1P bit planes from the query's levels (Q1 in lv[0, P), Q2 in lv[P, 2P),
// signed bytes): word u*48 + p*4 + d holds bit p of Q1 (p < 8) or bit p - 8
// of Q2 (p >= 8) for codes 128u + 32d .. +31 (bit b = code 128u + 32d + b).
// Threads tid, tid + nt, .. build one word each.
__device__ __forceinline__ void q1p_planes(const signed char *lv, uint32_t P, uint32_t *out, uint32_t tid,
                                           uint32_t nt) {
    constexpr uint32_t W = Codec<C_Q1P>::QN;  // words per unit
    const uint32_t nw = P / 128 * W;
    for (uint32_t k = tid; k < nw; k += nt) {
        const uint32_t u = k / W, r = k % W, pl = r / 4, d = r % 4;
        const signed char *lq = pl < 8 ? lv : lv + P;
        const uint32_t sh = pl < 8 ? pl : pl - 8;
        const uint32_t *src = (const uint32_t *)(lq + 128 * u + 32 * d);
        uint32_t bits = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t w = src[j] >> sh;  // bit sh of byte b now at bit 8b
            bits |= ((w & 1u) | ((w >> 7) & 2u) | ((w >> 14) & 4u) | ((w >> 21) & 8u)) << (4 * j);
        }
        out[k] = bits;
    }
}

// The levels of a rotated query for the 1-bit prefilter: q ~= s1 * Q1 +
// s2 * Q2 with s1 = max|q| / 127, Q1 = rint(q / s1) (the rounding of the
// int8 level split's first level), s2 = s1 / 14 and Q2 = rint(r1 / s2) of
// the residual r1 = q - s1 * Q1 (|r1| <= s1 / 2, so |Q2| <= 7).  The lane's
// Q1 / Q2 go to lv[e] / lv[P + e]; it returns its sums of |q - s1 Q1 - s2 Q2|,
// |q|, Q1 and Q2.
template <int E>
__device__ __forceinline__ void q1p_level(const float (&x)[E], double s1, uint32_t P, signed char *lv, uint32_t e0,
                                          double &rs, double &qa, int32_t &sq1, int32_t &sq2) {
    const double inv = s1 > 0.0 ? 1.0 / s1 : 0.0;
    const double s2 = s1 / 14.0, inv2 = s1 > 0.0 ? 14.0 / s1 : 0.0;
    rs = 0.0;
    qa = 0.0;
    sq1 = 0;
    sq2 = 0;
#pragma unroll
    for (int t = 0; t < E; ++t) {
        const double xd = (double)x[t];
        double c = rint(xd * inv);
        c = c > 127.0 ? 127.0 : (c < -127.0 ? -127.0 : c);
        const double r1 = fma(-s1, c, xd);
        double c2 = Q1P_L2 ? rint(r1 * inv2) : 0.0;
        c2 = c2 > 7.0 ? 7.0 : (c2 < -7.0 ? -7.0 : c2);
        rs += fabs(fma(-s2, c2, r1));
        qa += fabs(xd);
        sq1 += (int32_t)c;
        sq2 += (int32_t)c2;
        lv[e0 + t] = (signed char)(int)c;
        lv[P + e0 + t] = (signed char)(int)c2;
    }
}

// C_Q1P layout: bit planes (P/128 units x QN words), Q1Tail behind them,
// the fp32 query at q1p_f_off(P).
__host__ __device__ inline size_t q1p_tail_off(uint32_t P) { return (size_t)P / 128 * Codec<C_Q1P>::QN * 4; }
__host__ __device__ inline size_t q1p_f_off(uint32_t P) { return (q1p_tail_off(P) + sizeof(Q1Tail) + 63) & ~(size_t)63; }

// The exact re-score table of the C_Q1P scan (LDS): for every 4-code nibble
// j of the query (codes 4j .. 4j+3) 16 fp32 entries, entry n =
// ((s0 q0 + s1 q1) + s2 q2) + s3 q3 with s_k = +1 if bit k of n is set, else
// -1.  Unit u's 32 nibbles start at u * Q1P_LUT_UNIT floats (the 16-float
// pad spreads the units of a wave over the LDS banks).
constexpr uint32_t Q1P_LUT_UNIT = 32 * 16 + 16;
__host__ __device__ inline size_t q1p_lut_bytes(uint32_t P) { return (size_t)(P / 128) * Q1P_LUT_UNIT * 4; }
// Builds the entries of nibbles j = tid, tid + nt, .. < P/4 from the fp32
// query q (4 consecutive floats per nibble).
__device__ __forceinline__ void q1p_lut_build(const float *q, uint32_t P, float *lut, uint32_t tid, uint32_t nt) {
#pragma clang fp contract(off)
    for (uint32_t j = tid; j < P / 4; j += nt) {
        const float q0 = q[4 * j], q1 = q[4 * j + 1], q2 = q[4 * j + 2], q3 = q[4 * j + 3];
        float *row = lut + (j / 32) * Q1P_LUT_UNIT + (j % 32) * 16;
#pragma unroll
        for (int n = 0; n < 16; ++n) {
            const float a = (n & 1) ? q0 : -q0, b = (n & 2) ? q1 : -q1, c = (n & 4) ? q2 : -q2, d = (n & 8) ? q3 : -q3;
            row[n] = ((a + b) + c) + d;
        }
    }
}

// Bytes of the scan's per-query layout for codec C at padded dimension P.
__host__ __device__ inline size_t query_layout_bytes(int codec, uint32_t P) {
    switch (codec) {
    case C_Q8:
    case C_Q4M: return ((size_t)P / 16 * 12 * 4 + sizeof(QLevelTail) + 63) & ~(size_t)63;
    case C_Q4: return ((size_t)P / 32 * 24 * 4 + sizeof(QLevelTail) + 63) & ~(size_t)63;
    case C_Q1A: return (size_t)P * 4;
    case C_Q1P: return q1p_f_off(P) + (size_t)P * 4;
    case C_HAM: return ((size_t)P / 32 * 4 + 15) & ~(size_t)15;
    case C_I8S: return ((size_t)P / 4 * 4 + 15) & ~(size_t)15;
    default: return 0;
    }
}
// LDS the in-scan query transform needs: layout + scratch.
__host__ __device__ inline size_t query_prep_lds(int codec, uint32_t P) {
    const size_t lay = query_layout_bytes(codec, P);
    // the larger of the one-wave needs and the workgroup-wide ones
    // (layout + xs + lv + reduction slots)
    const size_t wg = ((lay + 15) & ~(size_t)15) + 4 * (size_t)P + 3 * (size_t)P + 12 * 8 + 12 * 4;
    if (codec == C_Q8 || codec == C_Q4) return wg;
    if (codec == C_Q1A || codec == C_Q1P) return wg;
    if (codec == C_HAM || codec == C_I8S) return lay + 5 * (size_t)P;
    return lay;
}

// The C_Q1P layout of one rotated query per workgroup of one wave (E = P/64
// elements per lane): bit planes, Q1Tail and the fp32 query.
template <int E>
__global__ __launch_bounds__(64) void query_q1p(LevelArgs a) {
    extern __shared__ unsigned char lsm[];  // 2P bytes: the two levels
    const uint32_t P = a.P, qi = blockIdx.x;
    const int lane = threadIdx.x;
    const uint32_t e0 = (uint32_t)lane * E;
    const float *q = a.qrot + (uint64_t)qi * P;
    unsigned char *out = a.out + (uint64_t)qi * a.stride;
    float *qf = (float *)(out + q1p_f_off(P));
    float x[E];
#pragma unroll
    for (int t = 0; t < E; ++t) {
        x[t] = q[e0 + t];
        qf[e0 + t] = x[t];
    }
    double m = 0.0;
#pragma unroll
    for (int t = 0; t < E; ++t) m = fmax(m, fabs((double)x[t]));
    m = wave_fmax_f64(m);
    const double s1 = m > 0.0 ? m / 127.0 : 0.0;
    double rs, qa;
    int32_t sq1, sq2;
    q1p_level<E>(x, s1, P, (signed char *)lsm, e0, rs, qa, sq1, sq2);
    rs = wave_sum_f64(rs);
    qa = wave_sum_f64(qa);
    sq1 = wave_sum_i32(sq1);
    sq2 = wave_sum_i32(sq2);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    q1p_planes((const signed char *)lsm, P, (uint32_t *)out, (uint32_t)lane, 64);
    if (lane == 0) {
        Q1Tail *tl = (Q1Tail *)(out + q1p_tail_off(P));
        tl->s1 = s1;
        tl->s2 = Q1P_L2 ? s1 / 14.0 : 0.0;
        tl->rsum = rs;
        tl->qabs = qa;
        tl->sumq1 = sq1;
        tl->sumq2 = sq2;
    }
}

// The query transform of the quantized scans, done by one wave of every
// scanning workgroup straight from the fp32 query: rotation, then the
// codec's layout (int8 levels, rotated floats, or quantized query codes) in
// LDS at `lds`.  Byte-identical to the standalone encode + levels kernels.
template <int C, int E>
__device__ __forceinline__ void prep_query_e(const ScanArgs &a, RotIn<E> &in, unsigned char *lds, int lane) {
    const uint32_t P = a.padded_dim;
    float x[E];
    rotate_apply<E>(in, a.qdim, P, a.signs, a.rounds, x, lane);
    const size_t lay = query_layout_bytes(C, P);
    if constexpr (C == C_Q8 || C == C_Q4) {
        levels_wave<E>(x, P, C, (signed char *)(lds + lay), lds, lane);
    } else if constexpr (C == C_Q1A) {
        const uint32_t lanes_used = P / E, e0 = lane * E;
        float *f = (float *)lds;
        if ((uint32_t)lane < lanes_used) {
#pragma unroll
            for (int t = 0; t < E; ++t) f[e0 + t] = x[t];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    } else if constexpr (C == C_HAM || C == C_I8S) {
        unsigned char *cbytes = lds + lay;
        quantize_store_wave<E>(x, P, C == C_HAM ? 1 : 8, cbytes, (float *)(cbytes + P), (uint32_t *)lds, nullptr,
                               nullptr, lane);
    }
}

// Codes per scan unit, and the padded dimension / elements per lane for
// which a scan layout does its own query transform: the layout's full unit
// count (LPR * UPL units), with at most 16 elements per lane so the
// transform's registers stay below the scan loop's.
template <int C> struct UnitCodes {
    static constexpr int v = (C == C_Q8 || C == C_I8S) ? 16 : (C == C_Q4 || C == C_Q1A) ? 32
                             : (C == C_HAM || C == C_Q1P) ? 128 : 0;
};
template <int C, int LPR, int UPL> struct PrepShape {
    static constexpr int P = UnitCodes<C>::v * LPR * UPL;
    static constexpr int E = P >= 64 ? P / 64 : 1;
    // (the bit-plane layout is built only by the workgroup-wide transform)
    static constexpr bool ok = UnitCodes<C>::v > 0 && P >= 64 && E <= 16 &&
                               (C != C_Q1P || P == 256 || P == 512 || P == 1024);
};

// The same transform spread over the 4 waves of a workgroup, for the
// int8 / int4 level split and the 1-bit asym layout at P = 256 * EP
// (EP = 1, 2, 4).  Wave w holds the quarter [w*P/4, (w+1)*P/4) with EP
// consecutive elements per lane: FWHT stages len < P/4 run in registers as
// in rotate_apply, the last two (len = P/4, P/2) across waves through LDS.
// Same butterflies in the same stage order, and the level split does the
// same per-element f64 arithmetic with workgroup-wide exact max / sum, so
// the bytes equal the one-wave transform's.  Every thread takes part (the
// caller's barriers follow); LDS layout: [layout | xs: P floats | lv: 3P
// bytes | 3 x 4 double + 3 x 4 int reduction slots].
template <int EP> struct RotInWG {
    float x[EP];
    float s[2][EP];
};

__host__ __device__ inline size_t prep_wg_xs_offset(size_t lay) { return (lay + 15) & ~(size_t)15; }

// (unconditional loads of clamped addresses, as in rotate_load; the query
// is masked by the dimension at first use in prep_query_wg)
template <int EP>
__device__ __forceinline__ void rotate_load_wg(const float *src, uint32_t dim, uint32_t P, const float *signs,
                                               uint32_t rounds, RotInWG<EP> &in, int tid) {
    const uint32_t e0 = (uint32_t)tid * EP;  // quarter of wave w starts at w*64*EP = (tid - lane)*EP
#pragma unroll
    for (int t = 0; t < EP; ++t) in.x[t] = src[e0 + t < dim ? e0 + t : dim - 1];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const uint32_t rr = (uint32_t)r < rounds ? (uint32_t)r : 0u;
#pragma unroll
        for (int t = 0; t < EP; ++t) in.s[r][t] = signs[(size_t)rr * P + e0 + t];
    }
}

template <int C, int EP>
__device__ __forceinline__ void prep_query_wg(const ScanArgs &a, RotInWG<EP> &in, unsigned char *lds, int tid) {
#pragma clang fp contract(off)
    const uint32_t P = a.padded_dim;  // == 256 * EP
    const int lane = tid & 63, wave = tid >> 6;
    const uint32_t e0 = (uint32_t)tid * EP;
    const size_t lay = query_layout_bytes(C, P);
    float *xs = (float *)(lds + prep_wg_xs_offset(lay));
    float x[EP];
#pragma unroll
    for (int t = 0; t < EP; ++t) x[t] = e0 + t < a.qdim ? in.x[t] : 0.0f;
    // the rounds, as in rotate_apply: the first two from the signs loaded up
    // front, further ones in a loop of their own
    auto one_round = [&](const float (&sg)[EP]) {
#pragma unroll
        for (int t = 0; t < EP; ++t) x[t] = x[t] * sg[t];
#pragma unroll
        for (int len = 1; len < EP; len <<= 1) {
#pragma unroll
            for (int t = 0; t < EP; ++t) {
                if (!(t & len)) {
                    const float u = x[t], w = x[t + len];
                    x[t] = u + w;
                    x[t + len] = u - w;
                }
            }
        }
        fwht_xlane64<EP>(x, lane);
        // stages len = P/4 and P/2 pair elements of different waves
#pragma unroll
        for (int t = 0; t < EP; ++t) xs[e0 + t] = x[t];
        __syncthreads();
        for (uint32_t len = P / 4; len < P; len <<= 1) {
            for (uint32_t idx = tid; idx < P / 2; idx += SCAN_WG) {
                const uint32_t i = (idx / len) * (2 * len) + idx % len, j = i + len;
                const float u = xs[i], w = xs[j];
                xs[i] = u + w;
                xs[j] = u - w;
            }
            __syncthreads();
        }
#pragma unroll
        for (int t = 0; t < EP; ++t) x[t] = xs[e0 + t];
        __syncthreads();  // xs is rewritten by the next round
    };
    one_round(in.s[0]);
    if (a.rounds > 1) one_round(in.s[1]);
    for (uint32_t r = 2; r < a.rounds; ++r) {
        float sg[EP];
#pragma unroll
        for (int t = 0; t < EP; ++t) sg[t] = a.signs[(size_t)r * P + e0 + t];
        one_round(sg);
    }
    if constexpr (C == C_Q1A) {
        float *f = (float *)lds;
#pragma unroll
        for (int t = 0; t < EP; ++t) f[e0 + t] = x[t];
        return;
    } else if constexpr (C == C_Q1P) {
        // the rotated query in xs for the exact re-score table (at qf_off);
        // the levels go to bit planes + Q1Tail at lds
#pragma unroll
        for (int t = 0; t < EP; ++t) xs[e0 + t] = x[t];
        signed char *lv = (signed char *)(xs + P);  // Q1, then Q2
        double *red = (double *)(lv + 2 * P);   // [3][4]: max, sum |r|, sum |q|
        int32_t *reds = (int32_t *)(red + 12);  // [2][4]: sum Q1, sum Q2
        double m = 0.0;
#pragma unroll
        for (int t = 0; t < EP; ++t) m = fmax(m, fabs((double)x[t]));
        m = wave_fmax_f64(m);
        if (lane == 0) red[wave] = m;
        __syncthreads();
        m = fmax(fmax(red[0], red[1]), fmax(red[2], red[3]));
        const double s1 = m > 0.0 ? m / 127.0 : 0.0;
        double rs, qa;
        int32_t sq1, sq2;
        q1p_level<EP>(x, s1, P, lv, e0, rs, qa, sq1, sq2);
        rs = wave_sum_f64(rs);
        qa = wave_sum_f64(qa);
        sq1 = wave_sum_i32(sq1);
        sq2 = wave_sum_i32(sq2);
        if (lane == 0) {
            red[4 + wave] = rs;
            red[8 + wave] = qa;
            reds[wave] = sq1;
            reds[4 + wave] = sq2;
        }
        __syncthreads();
        q1p_planes(lv, P, (uint32_t *)lds, (uint32_t)tid, SCAN_WG);
        q1p_lut_build(xs, P, (float *)(lds + a.qf_off), (uint32_t)tid, SCAN_WG);
        if (tid == 0) {
            Q1Tail *tl = (Q1Tail *)(lds + q1p_tail_off(P));
            tl->s1 = s1;
            tl->s2 = Q1P_L2 ? s1 / 14.0 : 0.0;
            tl->rsum = ((red[4] + red[5]) + red[6]) + red[7];
            tl->qabs = ((red[8] + red[9]) + red[10]) + red[11];
            tl->sumq1 = reds[0] + reds[1] + reds[2] + reds[3];
            tl->sumq2 = reds[4] + reds[5] + reds[6] + reds[7];
        }
        return;
    } else {
        signed char *lv = (signed char *)(xs + P);
        double *redm = (double *)(lv + 3 * (size_t)P);  // [3][4]
        int32_t *reds = (int32_t *)(redm + 12);         // [3][4]
        double rd[EP];
#pragma unroll
        for (int t = 0; t < EP; ++t) rd[t] = (double)x[t];
        double sl[3];
#pragma unroll
        for (int l = 0; l < 3; ++l) {
            double m = 0.0;
#pragma unroll
            for (int t = 0; t < EP; ++t) m = fmax(m, fabs(rd[t]));
            m = wave_fmax_f64(m);
            if (lane == 0) redm[l * 4 + wave] = m;
            __syncthreads();
            m = fmax(fmax(redm[l * 4 + 0], redm[l * 4 + 1]), fmax(redm[l * 4 + 2], redm[l * 4 + 3]));
            const double sc = m > 0.0 ? m / 127.0 : 0.0;
            const double inv = sc > 0.0 ? 1.0 / sc : 0.0;
            int32_t sum = 0;
#pragma unroll
            for (int t = 0; t < EP; ++t) {
                double c = rint(rd[t] * inv);
                c = c > 127.0 ? 127.0 : (c < -127.0 ? -127.0 : c);
                rd[t] = fma(-sc, c, rd[t]);
                lv[l * P + e0 + t] = (signed char)(int)c;
                sum += (int)c;
            }
            sum = wave_sum_i32(sum);
            if (lane == 0) reds[l * 4 + wave] = sum;
            sl[l] = sc;
        }
        __syncthreads();
        uint32_t *w = (uint32_t *)lds;
        const unsigned char *lb = (const unsigned char *)lv;
        uint32_t qwords;
        if constexpr (C == C_Q8) {
            const uint32_t units = P / 16;
            qwords = units * 12;
            for (uint32_t i = tid; i < qwords; i += SCAN_WG) {
                const uint32_t u = i / 12, r = i % 12, l = r / 4, d = r % 4;
                const uint32_t base = l * P + 16 * u + 4 * d;
                w[i] = (uint32_t)lb[base] | ((uint32_t)lb[base + 1] << 8) | ((uint32_t)lb[base + 2] << 16) |
                       ((uint32_t)lb[base + 3] << 24);
            }
        } else {  // C_Q4
            const uint32_t units = P / 32;
            qwords = units * 24;
            for (uint32_t i = tid; i < qwords; i += SCAN_WG) {
                const uint32_t u = i / 24, r = i % 24, l = r / 8, d = (r % 8) / 2, h = r % 2;
                const uint32_t base = l * P + 32 * u + 8 * d + h;
                w[i] = (uint32_t)lb[base] | ((uint32_t)lb[base + 2] << 8) | ((uint32_t)lb[base + 4] << 16) |
                       ((uint32_t)lb[base + 6] << 24);
            }
        }
        if (tid == 0) {
            QLevelTail *tl = (QLevelTail *)(lds + (size_t)qwords * 4);
            const double div = C == C_Q8 ? 127.0 : 1.0;
#pragma unroll
            for (int l = 0; l < 3; ++l) {
                tl->s[l] = sl[l] / div;
                tl->sum[l] = reds[l * 4 + 0] + reds[l * 4 + 1] + reds[l * 4 + 2] + reds[l * 4 + 3];
            }
            tl->pad = 0;
        }
    }
}

// Which transform a scan layout uses: the workgroup-wide one for int8 /
// int4 / 1-bit asym at P = 256, 512, 1024, else the one-wave one.
template <int C, int LPR, int UPL> struct PrepWG {
    static constexpr int P = UnitCodes<C>::v * LPR * UPL;
    static constexpr bool ok = (C == C_Q8 || C == C_Q4 || C == C_Q1A || C == C_Q1P) && (P == 256 || P == 512 || P == 1024);
    static constexpr int EP = ok ? P / 256 : 1;
};

// ------------------------------------------------------------ exact score --
// Store.dotRow of one stored fp32 row with the fp32 query, by one wave
// (src/store/store.ts:114-130): four f64 accumulators over the strided
// elements 4j+m, combined as ((a0+a1)+a2)+a3, then the tail elements.  The
// wave loads row and query coalesced and stages every exact product
// x[i]*q[i] (two 24-bit significands fit a double) in `stage` (vec doubles,
// wave-private LDS), transposed so that accumulator m's terms are
// contiguous; lanes 0..3 then add them in the reference's order (adding an
// exact product rounds exactly like the reference's `acc += x*y`).  Returns
// the (score, row) key in every lane.
__device__ uint64_t exact_key_wave(const float *src, const float *qs, uint32_t dim, uint32_t row, double *stage,
                                   int lane) {
    const uint32_t vec = dim & ~3u, nv = vec >> 2;
    constexpr int B = 8;
    for (uint32_t e0 = 0; e0 < vec; e0 += 64 * B) {
        float xv[B], qv[B];
#pragma unroll
        for (int t = 0; t < B; ++t) {
            const uint32_t e = e0 + t * 64 + lane;
            xv[t] = e < vec ? src[e] : 0.0f;
            qv[t] = e < vec ? qs[e] : 0.0f;
        }
#pragma unroll
        for (int t = 0; t < B; ++t) {
            const uint32_t e = e0 + t * 64 + lane;
            if (e < vec) stage[(e & 3) * nv + (e >> 2)] = (double)xv[t] * (double)qv[t];
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    double acc = 0.0;
    if (lane < 4) {
        const double *pp = stage + (uint32_t)lane * nv;
        uint32_t j = 0;
        for (; j + 8 <= nv; j += 8) {
            double t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) t[u] = pp[j + u];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = acc + t[u];
        }
        for (; j < nv; ++j) acc = acc + pp[j];
    }
    const double a1 = __shfl(acc, 1), a2 = __shfl(acc, 2), a3 = __shfl(acc, 3);
    uint64_t key = 0;
    if (lane == 0) {
        double sum = acc + a1;
        sum = sum + a2;
        sum = sum + a3;
        for (uint32_t i = vec; i < dim; ++i) sum = fma((double)src[i], (double)qs[i], sum);
        key = make_key(ord_f32((float)sum), row);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // stage is free again
    return uniform_u64(key);
}

// Store.dotRow (src/store/store.ts:114-129) of sixteen rows at once, four
// lanes per row: lane 4c + m sums the exact products of elements 4j + m of
// row c in order (an exact f32 x f32 product added by fma rounds like the
// reference's `a_m += x*y` in f64), lane 4c combines the four as
// ((a0 + a1) + a2) + a3 and adds the tail elements in order.  x: this lane's
// row; every lane of the wave calls it; the key is valid in lanes 4c.
// qd holds the query as doubles (LDS).  Each lane issues its row loads 192 at
// a time ahead of the dependent FMA chain, so a row costs one memory round
// trip up to dim 768 (a few beyond), not one per eight elements.
template <int B>
__device__ __forceinline__ void dot_chain(const float *x, const double *qd, uint32_t vec, uint32_t &j, double &acc) {
    for (; j + 4 * (B - 1) < vec; j += 4 * B) {
        float xv[B];
#pragma unroll
        for (int u = 0; u < B; ++u) xv[u] = x[j + 4 * u];
#pragma unroll
        for (int u = 0; u < B; ++u) acc = fma((double)xv[u], qd[j + 4 * u], acc);
    }
}
__device__ __forceinline__ uint64_t exact_key_lanes4(const float *x, const double *qd, const float *q, uint32_t dim,
                                                     uint32_t row, int lane) {
    const uint32_t vec = dim & ~3u;
    double acc = 0.0;
    uint32_t j = (uint32_t)(lane & 3);
    dot_chain<192>(x, qd, vec, j, acc);
    dot_chain<16>(x, qd, vec, j, acc);
    dot_chain<1>(x, qd, vec, j, acc);
    const double a1 = __shfl_down(acc, 1), a2 = __shfl_down(acc, 2), a3 = __shfl_down(acc, 3);
    double sum = acc + a1;
    sum = sum + a2;
    sum = sum + a3;
    if ((lane & 3) == 0)
        for (uint32_t i = vec; i < dim; ++i) sum = fma((double)x[i], (double)q[i], sum);
    return make_key(ord_f32((float)sum), row);
}

// ------------------------------------------------------------ scan + top-k --
constexpr uint32_t TAU_POLL = 4;     // step pairs between reads of the shared bound
// The split between statically assigned grabs and dynamic tickets comes
// with each launch (ScanArgs::static_pct / dsteps, chosen by the host for
// long and short scans); zero takes these.
constexpr uint32_t STATIC_PCT = 70;  // share of the grabs assigned statically
constexpr uint32_t DSTEPS = 6;       // steps per dynamically assigned chunk

// A unit slot past the end of a row (layouts whose lanes overhang the row)
// must contribute nothing: zero query values do that for the dot-style codecs;
// the l2 and Hamming codecs substitute a unit equal to the query itself.
template <int C> struct Neutral {
    template <class Unit, class QT> static __device__ __forceinline__ Unit get(Unit u, const QT *, bool ok) { return u; }
};
template <> struct Neutral<C_F32L2> {
    static __device__ __forceinline__ uint4 get(uint4 u, const float *q, bool ok) {
        return ok ? u : make_uint4(__float_as_uint(q[0]), __float_as_uint(q[1]), __float_as_uint(q[2]),
                                   __float_as_uint(q[3]));
    }
};
template <> struct Neutral<C_F32L2_S> {
    static __device__ __forceinline__ uint32_t get(uint32_t u, const float *q, bool ok) {
        return ok ? u : __float_as_uint(q[0]);
    }
};
template <> struct Neutral<C_HAM> {
    static __device__ __forceinline__ uint4 get(uint4 u, const uint32_t *q, bool ok) {
        return ok ? u : make_uint4(q[0], q[1], q[2], q[3]);
    }
};

// Per-lane constants of a scan: the query slice in registers and the
// lane's place in the row layout.
template <int C, int UPL> struct ScanRegs {
    typename Codec<C>::QT qr[UPL][Codec<C>::QN];
    bool uok[UPL];
    uint32_t ucl[UPL];
    Fin<C> fin;
    const float *qf;  // C_Q1P: the exact re-score table in LDS
};

// Rows are split across LPR lanes (each lane loads UPL 16-byte or 4-byte units
// of a row; 64/LPR rows per load instruction).  Every step a wave issues all
// U*UPL loads of its U row groups before any arithmetic, then reduces the
// per-lane partial sums with the transposing butterfly.
template <int C, int LPR, int UPL> struct ScanShape {
    static constexpr int U0 = UPL >= 4 ? 2 : (UPL >= 2 ? 4 : 8);
    // one transposing stage per halving of U (at most three), and at most 32
    // rows per step so that a pass of two steps adds at most 64 keys to a
    // wave's list (the list's slack beyond twice the fetch).  (64-row steps
    // for the 8-lane layouts measured slower: 1-bit Hamming 0.31 vs 0.42 of
    // HBM peak.)
    static constexpr int UMAX = LPR >= 16 ? 8 : LPR / 2;
    static constexpr int U = U0 < UMAX ? U0 : UMAX;  // row groups per lane per step
    static constexpr int G = 64 / LPR;               // rows per load instruction
    static constexpr int WAVES = SCAN_WG / 64;
    static constexpr int RPS = U * G;                // rows per wave step
    static constexpr int GRAB_STEPS = 2;             // wave steps per work grab
    static constexpr int GRAB_ROWS = WAVES * RPS * GRAB_STEPS;
    static constexpr uint32_t WGRAB = RPS * 2;       // keys one loop iteration (two steps) can add to a wave's list
};

// Streaming loads of codes and scales are nontemporal: every byte is read
// once per query, and keeping it out of the caches' normal allocation lets
// the scan sustain a higher share of HBM bandwidth.
typedef unsigned int nt_u4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream(const uint4 *p) {
    const nt_u4 t = __builtin_nontemporal_load((const nt_u4 *)p);
    return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ uint32_t load_stream(const uint32_t *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ float load_stream(const float *p) { return __builtin_nontemporal_load(p); }

// One wave step: the U x UPL units each lane loads for RPS consecutive rows
// (candidate slots when IDX), plus the stored scale and row id of the row
// whose total this lane will hold after the reduction.  The scale stays as
// loaded until the step is scored: any arithmetic on it at load time would
// make the wave wait for every load in flight (the load counter drains in
// order), which leaves a single step in flight instead of two.
template <int C, int LPR, int UPL> struct StepData {
    typename Codec<C>::Unit d[ScanShape<C, LPR, UPL>::U][UPL];
    float scale;
    uint32_t grow;
};

// Issues the loads of the step covering rows [base, base + RPS), clipped to
// lim (> 0): rows at or past lim load row lim-1 and are dropped later.
template <int C, int LPR, int UPL, bool IDX>
__device__ __forceinline__ void load_step(const ScanArgs &a, const ScanRegs<C, UPL> &R, const uint32_t *cand,
                                          uint32_t base, uint32_t lim, StepData<C, LPR, UPL> &S, int lane) {
    using Unit = typename Codec<C>::Unit;
    using SH = ScanShape<C, LPR, UPL>;
    constexpr int U = SH::U, G = SH::G;
    const int slot = lane / LPR;
    const char *codes = (const char *)a.codes;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t row = base + (uint32_t)(u * G + slot);
        const uint32_t rc = row < lim ? row : lim - 1;
        const uint64_t grow = IDX ? (uint64_t)cand[rc] : (uint64_t)rc;
        const Unit *rp = (const Unit *)(codes + grow * a.row_bytes);
#pragma unroll
        for (int t = 0; t < UPL; ++t) S.d[u][t] = load_stream(rp + R.ucl[t]);
    }
    const uint32_t myrow = base + (uint32_t)(xrow<U, LPR>(lane) * G + slot);
    const uint32_t myrc = myrow < lim ? myrow : lim - 1;
    S.grow = IDX ? cand[myrc] : (uint32_t)myrc;
    // (a runtime condition: the unconditional form for the scaled codecs,
    // which lets the compiler schedule the load among the code loads,
    // measured 3.4 us slower per 1M-row int8 query)
    S.scale = a.scales ? load_stream(a.scales + S.grow) : 1.0f;
}

// Scores a loaded step: pushes keys >= tau to the wave's list and folds
// every eligible key into the lane's running maximum.
template <int C, int LPR, int UPL>
__device__ __forceinline__ void compute_step_gen(const ScanArgs &a, const ScanRegs<C, UPL> &R,
                                                 const StepData<C, LPR, UPL> &S, uint32_t base, uint32_t lim,
                                                 uint64_t tau, uint64_t *wk, uint32_t &wc, uint64_t &lmax, int lane) {
    using CD = Codec<C>;
    using Acc = typename CD::Acc;
    using SH = ScanShape<C, LPR, UPL>;
    constexpr int U = SH::U, G = SH::G;
    Acc acc[CD::NA][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        Acc a1[CD::NA];
#pragma unroll
        for (int m = 0; m < CD::NA; ++m) a1[m] = (Acc)0;
#pragma unroll
        for (int t = 0; t < UPL; ++t) CD::acc(Neutral<C>::get(S.d[u][t], R.qr[t], R.uok[t]), R.qr[t], a1);
#pragma unroll
        for (int m = 0; m < CD::NA; ++m) acc[m][u] = a1[m];
    }
    Acc tot[CD::NA];
#pragma unroll
    for (int m = 0; m < CD::NA; ++m) tot[m] = xreduce<U, LPR>(acc[m], lane);
    const uint32_t myrow = base + (uint32_t)(xrow<U, LPR>(lane) * G + lane / LPR);
    bool take = false;
    uint64_t key = 0;
    if (xrep<U, LPR>(lane) && myrow < lim) {
        uint32_t ord;
        const float sc = R.fin.score(tot, S.scale * a.scale_mul, ord);
        if (a.dense_out && blockIdx.y == 0) a.dense_out[myrow] = sc;
        bool pass = true;
        if (a.mask) pass = S.grow < a.mask_bits && ((a.mask[S.grow >> 5] >> (S.grow & 31)) & 1u);
        if (pass) {
            key = make_key(ord, S.grow);
            take = key >= tau;
            lmax = key > lmax ? key : lmax;
        }
    }
    wave_push(wk, wc, take, key);
}

// The next float below a finite x (bit steps; +-0 go to the negative
// smallest subnormal).
__device__ __forceinline__ float float_below(float x) {
    const uint32_t b = __float_as_uint(x);
    if ((b & 0x7fffffffu) == 0) return __uint_as_float(0x80000001u);
    return __uint_as_float((b & 0x80000000u) ? b + 1 : b - 1);
}

// A lane's part of a row's exact 1-bit asymmetric sum: its units' 32 nibble
// entries of the re-score table (q1p_lut_build) each, added in order.
template <int LPR, int UPL>
__device__ __forceinline__ float q1p_exact_partial(const ScanRegs<C_Q1P, UPL> &R, const uint4 (&d)[UPL], int pl) {
    float e = 0.0f;
#pragma unroll
    for (int t = 0; t < UPL; ++t) {
        if (!R.uok[t]) continue;
        const float *lt = R.qf + (size_t)(pl + LPR * t) * Q1P_LUT_UNIT;
        const uint32_t w[4] = {d[t].x, d[t].y, d[t].z, d[t].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
#pragma unroll
            for (int c = 0; c < 8; ++c) e += lt[(k * 8 + c) * 16 + ((w[k] >> (4 * c)) & 15u)];
        }
    }
    return e;
}

// C_Q1P: every row is scored through the levels' bit planes, exact integers
// T1, T2 = sums of Q1, Q2 over the row's set code bits.  A row group in
// which some row's bound on its exact score reaches the wave's bound is
// re-scored exactly, and only exactly scored rows enter the list, so the
// keys are those of the exact arithmetic: per unit the 32 nibble entries of
// the re-score table (q1p_lut_build) added in order, the units in order,
// then the transposing reduction, times the row scale.  Bound: the exact
// real sum is s1 (2 T1 - sum Q1) + s2 (2 T2 - sum Q2) + e with
// |e| <= sum |q - s1 Q1 - s2 Q2|, and the fp32 arithmetic differs from it by
// at most 4e-5 * sum |q| (under 512 roundings); the f64 bound takes a
// further 1e-6 margin.
template <int LPR, int UPL>
__device__ __forceinline__ void compute_step_q1p(const ScanArgs &a, const ScanRegs<C_Q1P, UPL> &R,
                                                 const StepData<C_Q1P, LPR, UPL> &S, uint32_t base, uint32_t lim,
                                                 uint64_t tau, uint64_t *wk, uint32_t &wc, uint64_t &lmax, int lane) {
    using CD = Codec<C_Q1P>;
    using SH = ScanShape<C_Q1P, LPR, UPL>;
    constexpr int U = SH::U, G = SH::G;
    int32_t acc1[U], acc2[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        int32_t a1[2] = {0, 0};
#pragma unroll
        for (int t = 0; t < UPL; ++t) CD::acc(S.d[u][t], R.qr[t], a1);  // (overhanging units: zero planes)
        acc1[u] = a1[0];
        acc2[u] = a1[1];
    }
    const int32_t T1 = xreduce<U, LPR>(acc1, lane), T2 = xreduce<U, LPR>(acc2, lane);
    // the levels' score of the row (without its scale)
    const double lev = R.fin.s1 * (double)(2 * T1 - R.fin.sumq1) + R.fin.s2 * (double)(2 * T2 - R.fin.sumq2);
    const uint32_t myrow = base + (uint32_t)(xrow<U, LPR>(lane) * G + lane / LPR);
    const bool row_ok = xrep<U, LPR>(lane) && myrow < lim;
    const float scale = S.scale * a.scale_mul;
    const double hi = (double)scale * (lev + R.fin.rsum + 4e-5 * R.fin.qabs);
    const double bound = hi + fabs(hi) * 1e-6;
    const double tau_sc = (double)f32_from_ord((uint32_t)(tau >> 32));
    const bool need = row_ok && (a.dense_out != nullptr || tau == 0 || !(bound < tau_sc));
    bool pass = true;
    if (a.mask && row_ok) pass = S.grow < a.mask_bits && ((a.mask[S.grow >> 5] >> (S.grow & 31)) & 1u);
    // Every eligible row raises the wave's maximum by a lower bound of its
    // exact key (rounded down), so the shared bound rises from the first
    // steps on without waiting for exact re-scores: the kprime-th best of the
    // published maxima is still at most the kprime-th best exact key.
    if (row_ok && pass) {
        double lo = (double)scale * (lev - R.fin.rsum - 4e-5 * R.fin.qabs);
        lo -= fabs(lo) * 1e-6;
        if (lo == lo) {  // (not NaN)
            float lf = (float)lo;
            if ((double)lf > lo) lf = float_below(lf);
            const uint64_t klo = make_key(ord_f32(lf), S.grow);
            lmax = klo > lmax ? klo : lmax;
        }
    }
    bool take = false;
    uint64_t key = 0;
    if (__ballot(need) != 0) {
        // re-score only the row groups (u) that hold a row in need: after
        // the transposing reduction lane l holds a row of group xrow(l)
        const int xr = xrow<U, LPR>(lane);
        const int pl = lane % LPR;
        float ex[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (__ballot(need && xr == u) == 0) {
                ex[u] = 0.0f;
                continue;
            }
            ex[u] = q1p_exact_partial<LPR, UPL>(R, S.d[u], pl);
        }
        const float tot = xreduce<U, LPR>(ex, lane);
        if (need) {
            const float sc = tot * scale;
            if (a.dense_out && blockIdx.y == 0) a.dense_out[myrow] = sc;
            if (pass) {
                key = make_key(ord_f32(sc), S.grow);
                take = key >= tau;
                lmax = key > lmax ? key : lmax;
            }
        }
    }
    wave_push(wk, wc, take, key);
}

template <int C, int LPR, int UPL>
__device__ __forceinline__ void compute_step(const ScanArgs &a, const ScanRegs<C, UPL> &R,
                                             const StepData<C, LPR, UPL> &S, uint32_t base, uint32_t lim,
                                             uint64_t tau, uint64_t *wk, uint32_t &wc, uint64_t &lmax, int lane) {
    if constexpr (C == C_Q1P) compute_step_q1p<LPR, UPL>(a, R, S, base, lim, tau, wk, wc, lmax, lane);
    else compute_step_gen<C, LPR, UPL>(a, R, S, base, lim, tau, wk, wc, lmax, lane);
}

// Publishes the wave's running maximum to wmax[slot] on every call, from
// every lane (one line, one value): the scan loop issues the same memory
// operations whatever the data, so that its waits stay exact.  With m > 1
// (a fetch large next to the number of waves) the m largest lane maxima go
// to m slots: the lanes hold disjoint rows, so they are distinct rows' keys.
__device__ __forceinline__ void publish_wave_max(uint64_t *wslot, uint64_t lmax, uint32_t m, int lane) {
    if (m == 1) {
        __hip_atomic_store(wslot, wave_max_u64(lmax), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    uint64_t v = lmax;
#pragma unroll
    for (uint32_t j = 0; j < SCAN_PUB_MANY; ++j) {
        const uint64_t mx = wave_max_u64(v);
        __hip_atomic_store(wslot + j, mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t hit = __ballot(v == mx);  // (mx is some lane's value: hit is not empty)
        if ((uint64_t)lane == (uint64_t)(__ffsll((unsigned long long)hit) - 1)) v = 0;
    }
}

// Cross-workgroup hand-off without cache-wide maintenance: data goes through
// relaxed device-scope atomic stores and loads (write-through / coherent
// accesses that never rely on a stale per-XCD L2 line), and the signalling
// atomic is issued only after every prior access has completed.  A device
// fence would instead write back and invalidate the whole L2 of the XCD,
// stalling every workgroup still streaming through it.
__device__ __forceinline__ void store_shared(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_shared(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T> __device__ __forceinline__ T load_shared(const T *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores_done() { __builtin_amdgcn_s_waitcnt(0); }

__device__ __forceinline__ uint64_t load_tau(const QState *qs) {
    return uniform_u64(__hip_atomic_load(&qs->tau, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// Zeroes a query's coordination state and wave maxima (run by whichever of
// the final selection and the helper finishes last).
__device__ void reset_query(const ScanArgs &a, uint32_t qi) {
    QState *qs = a.qs + qi;
    const uint32_t nw = a.grid * (SCAN_WG / 64) * a.pub_m;
    uint64_t *wm = a.wmax + (uint64_t)qi * nw;
    for (uint32_t i = threadIdx.x; i < nw; i += blockDim.x) wm[i] = 0;
    for (uint32_t r = threadIdx.x; r < (uint32_t)NGROUP; r += blockDim.x) {
        qs->cc[r * CL] = 0;
        qs->dyn[r * CL] = 0;
    }
    if (threadIdx.x == 0) {
        qs->tau = 0;
        qs->top = 0;
        qs->fin = 0;
    }
}

// Background threshold: the kprime-th best of any kprime or more wave maxima
// is the key of a real row no better than the true kprime-th best, so every
// scan may drop keys below it.  Each round gathers up to `cap` maxima at or
// above the current bound (the maxima only grow, so the bound only rises)
// and publishes the new kprime-th best.  Runs until every scanning workgroup
// has finished.
__device__ void threshold_helper(const ScanArgs &a, uint32_t qi, TopkLds &L) {
    QState *qs = a.qs + qi;
    const uint32_t nslots = a.grid * (SCAN_WG / 64) * a.pub_m;
    const uint64_t *wm = a.wmax + (uint64_t)qi * nslots;
    const uint32_t kp = a.kprime;
    const uint32_t cap = kp <= (uint32_t)SCAN_WG ? (uint32_t)SCAN_WG : (uint32_t)SCAN_CAP;
    const int tid = threadIdx.x, lane = tid & 63;
    uint64_t th = 0;
    for (int round = 0; round < (1 << 22); ++round) {
        if (tid == 0) {
            L.flag = __hip_atomic_load(&qs->top, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            L.cnt = 0;
        }
        __syncthreads();
        // every scanning workgroup has finished: nothing left to prune, and
        // the launch completes only when this workgroup exits
        if (L.flag >= a.grid) break;
        for (uint32_t i0 = 0; i0 < nslots; i0 += 8 * SCAN_WG) {
            uint64_t v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t i = i0 + j * SCAN_WG + tid;
                v[j] = i < nslots ? __hip_atomic_load(&wm[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) wave_append(L.keys, &L.cnt, cap, v[j] != 0 && v[j] >= th, v[j], lane);
        }
        __syncthreads();
        const uint32_t have = L.cnt < cap ? L.cnt : cap;
        if (have >= kp) {
            const uint32_t m = select_topk(L, have, kp);
            const uint64_t t = L.keys[m - 1];
            if (t > th) {
                th = t;
                if (tid == 0) atomicMax(&qs->tau, (unsigned long long)t);
            }
        }
        __syncthreads();
    }
}

// Fused scan + top-k (one launch per query batch).  Workgroups 0..grid-1
// take row blocks round-robin (block b goes to workgroup b % grid); each of
// their waves keeps keys at or above its running bound in a private LDS list
// and publishes its running maximum.  Workgroup `grid` is the threshold
// helper.  At the end every wave flushes its keys at or above the freshest
// bound to a global array; the last workgroup to finish selects the best
// kprime of the flushes.  Dynamic LDS: max(sizeof(TopkLds), 4 * wcap * 8).
template <int C, int LPR, int UPL, bool IDX, bool PREP>
__device__ __forceinline__ void scan_topk_body(ScanArgs a) {
    using CD = Codec<C>;
    using QT = typename CD::QT;
    using SH = ScanShape<C, LPR, UPL>;
    extern __shared__ __align__(16) unsigned char scan_smem[];
    TopkLds &L = *(TopkLds *)scan_smem;

    const uint32_t qi = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    QState *qs = a.qs + qi;
    const uint32_t kp = a.kprime;

    if (blockIdx.x == a.grid) {
        threshold_helper(a, qi, L);
        __syncthreads();
        if (tid == 0) L.last = atomicAdd(&qs->fin, 1u) == 1;
        __syncthreads();
        if (L.last) reset_query(a, qi);
        return;
    }

    const int p = lane % LPR;
    ScanRegs<C, UPL> R;
#pragma unroll
    for (int t = 0; t < UPL; ++t) {
        const uint32_t unit = p + LPR * t;
        R.uok[t] = unit < a.units;
        R.ucl[t] = R.uok[t] ? unit : a.units - 1;
    }

    const uint32_t *cand = a.cand;
    uint32_t n = (uint32_t)a.n;  // row and candidate counts stay below 2^31 (checked at launch)
    if (IDX && a.cand_off) {
        cand = a.cand + a.cand_off[qi];
        n = (uint32_t)(a.cand_off[qi + 1] - a.cand_off[qi]);
    } else if (IDX && a.cand_n) {
        cand = a.cand + (uint64_t)qi * a.cand_stride;
        n = a.cand_n[qi] < a.cand_stride ? a.cand_n[qi] : (uint32_t)a.cand_stride;
    }
    uint64_t *wslot = a.wmax + (((uint64_t)qi * a.grid + blockIdx.x) * SH::WAVES + wave) * a.pub_m;
    uint64_t lmax = 0;

    const uint32_t wcap = a.wcap;
    uint64_t *wk = (uint64_t *)scan_smem + (size_t)wave * a.wstride;  // list, then re-rank staging
    const uint32_t trig = wcap - SH::WGRAB;       // compact when the list passes this
    const uint32_t target = kp + (trig - kp) / 2;  // ... down to at most this many keys
    uint32_t wc = 0;
    uint64_t tau = 0;
    const uint32_t ng = a.grid < (uint32_t)NGROUP ? a.grid : (uint32_t)NGROUP;

    // ---- a wave's stream of steps ----
    // Static part: grabs g = blockIdx.x + gi*grid for gi < sgrabs, each wave
    // taking GRAB_STEPS steps of every grab (rows wofs + s * wstep..).
    // Dynamic part: the steps of rows [d0, n), cut into ng slices that each
    // have their own ticket counter.  A slice hands out chunks of DSTEPS
    // consecutive steps, then its last (steps % DSTEPS) steps one at a time.
    // (Handing out more of a slice's end one step at a time evens out the
    // waves' finish times but costs more than it gains: single scattered
    // steps stream worse.)  A wave whose slice runs dry moves to the slice
    // with the most tickets left.  The dynamic part absorbs speed differences between
    // workgroups (older waves win memory arbitration) and XCDs.
    const uint32_t wofs = (uint32_t)wave * SH::RPS, wstep = (uint32_t)SH::WAVES * SH::RPS;
    const uint32_t ngrabs = (n + SH::GRAB_ROWS - 1) / SH::GRAB_ROWS;
    const uint32_t spct = a.static_pct ? a.static_pct : STATIC_PCT;
    const uint32_t dsteps = a.dsteps ? a.dsteps : DSTEPS;
    const uint32_t sgrabs = (uint32_t)((uint64_t)ngrabs * spct / 100 / a.grid);  // full static grabs per workgroup
    uint32_t d0 = sgrabs * a.grid * SH::GRAB_ROWS;
    if (d0 > n) d0 = n;
    const uint32_t nsd = (n - d0 + SH::RPS - 1) / SH::RPS;  // dynamic steps
    const uint32_t per = (nsd + ng - 1) / ng;              // steps per slice
    // a slice's step count, and its chunks of DSTEPS steps (the rest are
    // single-step tickets)
    auto slice_steps = [&](uint32_t r) -> uint32_t {
        const uint32_t lo = r * per;
        return lo >= nsd ? 0 : (nsd - lo < per ? nsd - lo : per);
    };
    auto big_chunks = [&](uint32_t ls) -> uint32_t { return ls / dsteps; };
    auto slice_tickets = [&](uint32_t r) -> uint32_t {
        const uint32_t ls = slice_steps(r), nb = big_chunks(ls);
        return nb + (ls - nb * dsteps);
    };
    uint32_t gi = 0;
    uint32_t sub = 0, ds = 0, dlen = 0, slice = (blockIdx.x * SH::WAVES + wave) % ng, pend = 0;
    bool dynamic = false, has_pend = false;
    uint32_t c0 = 0, clim = 0;
    // takes the next dynamic ticket: its first row in c0 and end in clim;
    // false when every slice is exhausted
    auto take_chunk = [&]() -> bool {
        for (;;) {
            uint32_t v = pend;
            if (!has_pend && lane == 0) v = atomicAdd(&qs->dyn[slice * CL], 1u);
            has_pend = false;
            const uint32_t t = __builtin_amdgcn_readfirstlane(v);
            const uint32_t ls = slice_steps(slice), nb = big_chunks(ls);
            if (t < nb + (ls - nb * dsteps)) {
                if (lane == 0) pend = atomicAdd(&qs->dyn[slice * CL], 1u);  // next ticket in flight
                has_pend = true;
                const uint32_t st = t < nb ? t * dsteps : nb * dsteps + (t - nb);
                dlen = t < nb ? dsteps : 1;
                c0 = d0 + (slice * per + st) * SH::RPS;
                const uint32_t e = c0 + dlen * SH::RPS;
                clim = e < n ? e : n;
                return true;
            }
            // this slice is exhausted (its counter never drops): read every
            // slice's counter at once and move to the one with most left
            uint64_t rem = 0;
            if ((uint32_t)lane < ng) {
                const uint32_t c = load_shared(&qs->dyn[lane * CL]);
                const uint64_t L = slice_tickets((uint32_t)lane);
                rem = c < L ? L - c : 0;
            }
            const uint64_t best = uniform_u64(wave_max_u64((rem << 32) | (uint32_t)lane));
            if ((best >> 32) == 0) return false;
            slice = (uint32_t)best;
        }
    };
    auto next_step = [&](uint32_t &base, uint32_t &lim) -> bool {
        if (!dynamic) {
            while (gi < sgrabs) {
                const uint32_t r0 = (blockIdx.x + gi * a.grid) * SH::GRAB_ROWS;
                base = r0 + wofs + sub * wstep;
                lim = r0 + SH::GRAB_ROWS < n ? r0 + SH::GRAB_ROWS : n;
                if (++sub == (uint32_t)SH::GRAB_STEPS) {
                    sub = 0;
                    ++gi;
                }
                if (base < lim) return true;
            }
            dynamic = true;
        }
        for (;;) {
            if (ds < dlen) {
                base = c0 + ds * SH::RPS;
                ++ds;
                if (base < clim) {
                    lim = clim;
                    return true;
                }
                ds = dlen;
            }
            if (nsd == 0 || !take_chunk()) return false;
            ds = 0;
        }
    };

    using SD = StepData<C, LPR, UPL>;
    constexpr bool PIPE = SH::U * UPL * (int)(sizeof(typename CD::Unit) / 4) <= 32;  // double-buffer the loads
    SD A, B;
    uint32_t ab = 0, al = 0, bb = 0, bl = 0;
    // the query slice: transformed here by wave 0 into LDS, or read from a
    // prepared global layout.  Wave 0 issues the query and sign reads before
    // any code load, and transforms while the first code loads are in flight.
    using PS = PrepShape<C, LPR, UPL>;
    using PW = PrepWG<C, LPR, UPL>;
    RotIn<(PS::ok && !PW::ok) ? PS::E : 1> rin;
    RotInWG<PW::EP> rinw;
    const float *qsrc = a.qraw + (uint64_t)qi * a.qdim;
    if constexpr (PREP && PW::ok) {
        rotate_load_wg<PW::EP>(qsrc, a.qdim, a.padded_dim, a.signs, a.rounds, rinw, tid);
    } else if constexpr (PREP && PS::ok) {
        if (wave == 0) rotate_load<PS::E>(qsrc, a.qdim, a.padded_dim, a.signs, a.rounds, rin, lane);
    }
    // The first two steps' code loads need no query: both go out before the
    // query transform, so the memory system stays busy while it runs.  Every
    // step slot issues its loads whether or not the stream has a step for it
    // (an idle slot loads the first row of the rows, a cached line, and is
    // not scored), so every pass of the loop below issues the same memory
    // operations and the load counter, which drains in order, lets a wave
    // wait for exactly the step it scores while the other stays in flight.
    // (A query with no rows issues no loads: the first row is not there.)
    // The query slice, when it comes prepared in global memory, is read
    // before any code load: the load counter drains in order, so a read
    // issued after the code loads would make the first score wait for all of
    // them (and the compiler places that wait at the loop head, so every pass
    // would wait for both steps).  A slice the kernel transforms itself is
    // read from LDS after the transform.  Each read goes through a pointer of
    // known address space.
    auto read_query = [&](const QT *qb) {
#pragma unroll
        for (int t = 0; t < UPL; ++t) {
#pragma unroll
            for (int j = 0; j < CD::QN; ++j) R.qr[t][j] = R.uok[t] ? qb[(p + LPR * t) * CD::QN + j] : (QT)0;
        }
        R.fin.load((const char *)qb + (uint64_t)a.units * CD::QN * sizeof(QT), a.padded_dim);
    };
    if constexpr (!PREP) read_query((const QT *)((const char *)a.q + (uint64_t)qi * a.q_stride));
    if constexpr (C == C_Q1P) {
        // the exact re-score table, in LDS behind everything else (built by
        // the query transform, or here from the prepared fp32 query)
        R.qf = (const float *)(scan_smem + a.qf_off);
        if constexpr (!PREP) {
            const float *src = (const float *)((const char *)a.q + (uint64_t)qi * a.q_stride + q1p_f_off(a.padded_dim));
            q1p_lut_build(src, a.padded_dim, (float *)(scan_smem + a.qf_off), (uint32_t)tid, SCAN_WG);
            __syncthreads();
        }
    }
    // The fp32 query of the exact re-rank, read here too (dims up to 64 * RQ;
    // lane l holds elements l + 64k) and staged as doubles behind the wave's
    // list once the LDS is free, so the flush at the end of the scan starts
    // with its row loads.
    constexpr int RQ = 16;
    const uint32_t rvec = a.rr_dim & ~3u;
    const bool stail = a.short_tail != 0;
    const bool stage_q = a.rr_src != nullptr && rvec <= 64 * RQ;
    float rqv[RQ];
    if (stage_q) {
        const float *rq = a.rr_q + (uint64_t)qi * a.rr_q_stride;
#pragma unroll
        for (int k = 0; k < RQ; ++k) {
            const uint32_t i = (uint32_t)lane + 64u * k;
            rqv[k] = rq[i < rvec ? i : rvec - 1];  // (clamped: every lane loads)
        }
    }
    // The query transform and the re-rank query's staging, after the first
    // two steps' loads are issued.  The code is repeated on three paths
    // (straight-line first steps, the general first steps, no rows) rather
    // than placed after their join: at a join of paths that issued
    // different loads the compiler waits for every load in flight, which
    // would make the transform wait for both steps' codes.
    auto prologue = [&]() {
        if constexpr (PREP) {
            if constexpr (PW::ok) {
                prep_query_wg<C, PW::EP>(a, rinw, scan_smem, tid);
            } else if constexpr (PS::ok) {
                if (wave == 0) prep_query_e<C, PS::E>(a, rin, scan_smem, lane);
            }
            __syncthreads();
            read_query((const QT *)scan_smem);
            __syncthreads();  // the LDS holding it becomes the waves' lists
        }
        if (stage_q) {
            double *qd = (double *)(wk + wcap);
#pragma unroll
            for (int k = 0; k < RQ; ++k) {
                const uint32_t i = (uint32_t)lane + 64u * k;
                // (the empty asm keeps the conversion, and the wait for the
                // load, here: hoisted to the load it would wait before the
                // first code load is issued)
                float r = rqv[k];
                asm volatile("" : "+v"(r));
                if (i < rvec) qd[i] = (double)r;
            }
        }
    };
    bool ha = false, hb = false;
    static_assert(SH::GRAB_STEPS == 2, "the straight-line first steps are one grab's two steps");
    if (PIPE && sgrabs > 0) {
        // the workgroup's first static grab is full: the wave's first two
        // steps are its two steps in that grab (next_step's state moves on
        // to the second grab)
        const uint32_t r0 = blockIdx.x * SH::GRAB_ROWS;
        ab = r0 + wofs;
        al = r0 + SH::GRAB_ROWS;
        bb = ab + wstep;
        bl = al;
        gi = 1;
        ha = hb = true;
        load_step<C, LPR, UPL, IDX>(a, R, cand, ab, al, A, lane);
        load_step<C, LPR, UPL, IDX>(a, R, cand, bb, bl, B, lane);
        __builtin_amdgcn_sched_barrier(0);  // every load issued before the transform's first use of the query
        prologue();
    } else if (n > 0) {
        ha = next_step(ab, al);
        if (PIPE) load_step<C, LPR, UPL, IDX>(a, R, cand, ha ? ab : 0, ha ? al : 1, A, lane);
        hb = PIPE && ha && next_step(bb, bl);
        if (PIPE) load_step<C, LPR, UPL, IDX>(a, R, cand, hb ? bb : 0, hb ? bl : 1, B, lane);
        __builtin_amdgcn_sched_barrier(0);
        prologue();
    } else {
        prologue();
    }
    uint64_t gt = 0;      // what the previous pass read: the shared bound when it polled
    bool polled = false;
    for (uint32_t pi = 0; ha; ++pi) {
        // the loop state is wave-uniform: restated so the compiler keeps it
        // (and the stepping branches) scalar
        ab = __builtin_amdgcn_readfirstlane(ab);
        al = __builtin_amdgcn_readfirstlane(al);
        bb = __builtin_amdgcn_readfirstlane(bb);
        bl = __builtin_amdgcn_readfirstlane(bl);
        gi = __builtin_amdgcn_readfirstlane(gi);
        sub = __builtin_amdgcn_readfirstlane(sub);
        ds = __builtin_amdgcn_readfirstlane(ds);
        dlen = __builtin_amdgcn_readfirstlane(dlen);
        c0 = __builtin_amdgcn_readfirstlane(c0);
        clim = __builtin_amdgcn_readfirstlane(clim);
        slice = __builtin_amdgcn_readfirstlane(slice);
        wc = __builtin_amdgcn_readfirstlane(wc);
        hb = __builtin_amdgcn_readfirstlane((int)hb) != 0;
        dynamic = __builtin_amdgcn_readfirstlane((int)dynamic) != 0;
        has_pend = __builtin_amdgcn_readfirstlane((int)has_pend) != 0;
        tau = uniform_u64(tau);
        if constexpr (PIPE) {
            // steps alternate between A and B; the other buffer's loads are
            // in flight while one is scored
            compute_step<C, LPR, UPL>(a, R, A, ab, al, tau, wk, wc, lmax, lane);
            const bool na = hb && next_step(ab, al);
            load_step<C, LPR, UPL, IDX>(a, R, cand, na ? ab : 0, na ? al : 1, A, lane);
            if (hb) compute_step<C, LPR, UPL>(a, R, B, bb, bl, tau, wk, wc, lmax, lane);
            if (polled) {  // the bound read in the previous pass, older than B's loads
                const uint64_t ugt = uniform_u64(gt);
                tau = ugt > tau ? ugt : tau;
            }
            // one store and one load per pass: the wave's maximum, and the
            // shared bound every TAU_POLL passes (waves staggered; it is one
            // line that every wave of the grid reads) or else the wave's own
            // slot
            publish_wave_max(wslot, lmax, a.pub_m, lane);
            // (the bit-plane scan polls every pass until a bound exists: its
            // rows go through the exact re-score until then)
            // (a short scan polls every pass: its waves run only a few)
            polled = stail || (C == C_Q1P && tau == 0) || (pi + (uint32_t)wave) % TAU_POLL == 0;
            gt = __hip_atomic_load(polled ? (const uint64_t *)&qs->tau : (const uint64_t *)wslot, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            const bool nb = na && next_step(bb, bl);
            load_step<C, LPR, UPL, IDX>(a, R, cand, nb ? bb : 0, nb ? bl : 1, B, lane);
                        ha = na;
            hb = nb;
        } else {
            load_step<C, LPR, UPL, IDX>(a, R, cand, ab, al, A, lane);
            compute_step<C, LPR, UPL>(a, R, A, ab, al, tau, wk, wc, lmax, lane);
            if (next_step(ab, al)) {
                load_step<C, LPR, UPL, IDX>(a, R, cand, ab, al, A, lane);
                compute_step<C, LPR, UPL>(a, R, A, ab, al, tau, wk, wc, lmax, lane);
                ha = next_step(ab, al);
            } else {
                ha = false;
            }
            publish_wave_max(wslot, lmax, a.pub_m, lane);
            const uint64_t g = uniform_u64(__hip_atomic_load(&qs->tau, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            tau = g > tau ? g : tau;
        }
        if (wc > trig) {
            wc = wave_filter(wk, wc, tau, lane);
            if (wc > target) {
                const uint64_t t = wave_bound(wk, wc, tau, kp, target, lane);
                wc = wave_filter(wk, wc, t, lane);
                if (t > tau) {
                    tau = t;
                    if (lane == 0) atomicMax(&qs->tau, (unsigned long long)t);
                }
            }
        }
    }
    // Flush the keys at or above the wave's bound: the bound read by the last
    // pass's poll, not a fresh read (one device round trip less at the end of
    // the scan; the final selection filters by the freshest shared bound).
    if constexpr (PIPE) {
        if (polled) {
            const uint64_t ugt = uniform_u64(gt);
            tau = ugt > tau ? ugt : tau;
        }
    }
    if (stail) {  // a short scan flushes by a fresh read: the helper's bound has had the whole scan to form
        const uint64_t g = load_tau(qs);
        tau = g > tau ? g : tau;
    }
    wc = wave_filter(wk, wc, tau, lane);
    // Flushed entries are (scan key, exact key) pairs; with re-ranking on,
    // the wave scores its own candidates exactly here, while other waves of
    // the grid are still scanning.  The slot reservation is issued first and
    // read only when the pairs are stored, so its round trip overlaps the
    // re-rank's row loads.
    const uint32_t grp = blockIdx.x % ng;
    const uint64_t region = a.cand_cap / ng;  // pairs per group region
    if (wc) {
        uint32_t b0 = 0;
        if (lane == 0) b0 = atomicAdd(&qs->cc[grp * CL], wc);
        uint64_t *ck0 = a.cand_keys + 2 * ((uint64_t)qi * a.cand_cap + grp * region);
        if (a.rr_src) {
            // the query as doubles in the wave's staging area behind its list
            // (staged before the scan when the dimension allows)
            const float *rq = a.rr_q + (uint64_t)qi * a.rr_q_stride;
            double *qd = (double *)(wk + wcap);
            if (!stage_q)
                for (uint32_t i = (uint32_t)lane; i < rvec; i += 64) qd[i] = (double)rq[i];
            for (uint32_t j0 = 0; j0 < wc; j0 += 16) {  // sixteen candidates per pass
                const uint32_t j = j0 + (uint32_t)(lane >> 2);
                const bool have = j < wc;
                const uint64_t k = have ? wk[j] : 0ull;
                const uint32_t row = have ? key_row(k) : 0u;  // absent candidates read row 0
                const uint64_t ek = exact_key_lanes4(a.rr_src + (uint64_t)row * a.rr_dim, qd, rq, a.rr_dim, row, lane);
                // read the reservation only now: tied to the exact key, so the
                // compiler cannot hoist the read (and its wait for the atomic)
                // above the row loads
                uint32_t bv = b0;
                asm volatile("" : "+v"(bv) : "v"((uint32_t)ek));
                const uint32_t base = __builtin_amdgcn_readfirstlane(bv);
                if (have && (lane & 3) == 0) {
                    store_shared(&ck0[2 * (base + j)], k);
                    store_shared(&ck0[2 * (base + j) + 1], ek);
                }
            }
        } else {
            const uint32_t base = __builtin_amdgcn_readfirstlane(b0);
            for (uint32_t j = lane; j < wc; j += 64) {
                store_shared(&ck0[2 * (base + j)], wk[j]);
                store_shared(&ck0[2 * (base + j) + 1], 0ull);
            }
        }
    }
    wait_stores_done();
    __syncthreads();
    // one ticket per workgroup: the last to finish runs the final selection
    // (finishes are spread over the scan's last microseconds, so the single
    // counter is not contended)
    if (tid == 0) L.last = atomicAdd(&qs->top, 1u) == a.grid - 1;
    __syncthreads();
    if (!L.last) return;

    // ---- last scanning workgroup: select the best kprime of the flushes ----
    // One round trip reads the bound, the per-group flush counts and the
    // first SCAN_WG / ng pairs of every group region (groups rarely flush
    // more); wave 0 turns the counts into their exclusive prefix.
    const uint64_t *ckq = a.cand_keys + 2 * (uint64_t)qi * a.cand_cap;
    const uint32_t spec = SCAN_WG / ng;
    const uint32_t sg = tid % ng, ss = tid / ng;
    const uint64_t sslot = 2 * ((uint64_t)sg * region + ss);
    const uint64_t sv = load_shared(&ckq[sslot]), se = load_shared(&ckq[sslot + 1]);
    if (tid == 0) {
        L.cnt = 0;
        L.tau = load_shared(&qs->tau);
    }
    if (tid < 64) {
        const uint32_t c = (uint32_t)tid < ng ? load_shared(&qs->cc[tid * CL]) : 0u;
        uint32_t incl = c;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t o = __shfl_up(incl, d);
            incl += lane >= d ? o : 0u;
        }
        // the pairs beyond the first spec of each group: their exclusive
        // prefix in ovl[96..129) indexes one flat range for a parallel gather
        const uint32_t ex = c > spec ? c - spec : 0u;
        uint32_t xin = ex;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t o = __shfl_up(xin, d);
            xin += lane >= d ? o : 0u;
        }
        if ((uint32_t)tid < ng) {
            L.ovl[tid] = c;
            L.ovl[32 + tid] = incl - c;
            L.ovl[96 + tid] = xin - ex;
        }
        if ((uint32_t)tid == ng - 1) {
            L.ovl[32 + ng] = incl;
            L.ovl[96 + ng] = xin;
        }
    }
    __syncthreads();
    const uint32_t total = L.ovl[32 + ng];
    constexpr uint32_t CHUNK = SCAN_CAP / 2;
    if (stail && total > CHUNK) {
        // A short scan whose flushes overflow the one-pass gather (the
        // helper's bound formed late): the gather is bounded first by the
        // kp-th best wave maximum.  The maxima of distinct waves are distinct
        // rows' keys, so kp rows score at least that much and it is at most
        // the kp-th best key.  Every wave published the maximum over all its
        // rows before its workgroup took a ticket.
        const uint32_t nslots = a.grid * (SCAN_WG / 64) * a.pub_m;
        const uint64_t *wm = a.wmax + (uint64_t)qi * nslots;
        for (uint32_t i0 = 0; i0 < nslots; i0 += 8 * SCAN_WG) {
            uint64_t v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t i = i0 + j * SCAN_WG + tid;
                v[j] = i < nslots ? load_shared(&wm[i]) : 0ull;
            }
            // (beyond SCAN_CAP maxima are dropped: the kp-th best of a
            // subset is a valid bound too)
#pragma unroll
            for (int j = 0; j < 8; ++j) wave_append(L.keys, &L.cnt, SCAN_CAP, v[j] != 0, v[j], lane);
        }
        __syncthreads();
        const uint32_t nm = L.cnt < (uint32_t)SCAN_CAP ? L.cnt : (uint32_t)SCAN_CAP;
        if (nm > kp) {
            const uint32_t m0 = select_topk(L, nm, kp);
            if (tid == 0 && L.keys[m0 - 1] > L.tau) L.tau = L.keys[m0 - 1];
        }
        __syncthreads();
        if (tid == 0) L.cnt = 0;
        __syncthreads();
    }
    if (a.rr_src && total <= CHUNK) {
        // Re-rank, common case: one pass gathers the (scan key, exact key)
        // pairs at or above the bound; the fetch is the best kp scan keys,
        // found by rank counting; its exact keys are ranked for the output.
        const uint64_t th = L.tau;
        const bool sok = ss < spec && ss < L.ovl[sg];  // (threads past ng * spec read no pair)
        wave_append2(L.keys, L.keys + CHUNK, &L.cnt, CHUNK, sok && sv != 0 && sv >= th, sv, se, lane);
        // the rest of the groups that flushed more than spec pairs, all at once
        const uint32_t xtot = L.ovl[96 + ng];
        for (uint32_t i0 = 0; i0 < xtot; i0 += SCAN_WG) {
            const uint32_t i = i0 + tid;
            uint64_t v = 0, e = 0;
            if (i < xtot) {
                uint32_t lo = 0, hi = ng - 1;  // the group r with ovl[96 + r] <= i < ovl[96 + r + 1]
                while (lo < hi) {
                    const uint32_t mid = (lo + hi + 1) / 2;
                    if (L.ovl[96 + mid] <= i) lo = mid;
                    else hi = mid - 1;
                }
                const uint64_t slot = 2 * ((uint64_t)lo * region + spec + (i - L.ovl[96 + lo]));
                v = load_shared(&ckq[slot]);
                e = load_shared(&ckq[slot + 1]);
            }
            wave_append2(L.keys, L.keys + CHUNK, &L.cnt, CHUNK, v != 0 && v >= th, v, e, lane);
        }
        if (tid == 0) {
            L.gtau = 0;
            L.cnt2 = 0;
        }
        __syncthreads();
        const uint32_t nk = L.cnt;
        if (nk <= 128) {
            // Up to 128 pairs (the common case): wave 0 sorts them by scan
            // key in registers, keeps the best kp (the fetch), and sorts the
            // fetch's exact keys for the output.
            if (wave == 0) {
                uint64_t sk[2], ek[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const uint32_t e = (uint32_t)lane + 64u * t;
                    sk[t] = e < nk ? L.keys[e] : 0ull;
                    ek[t] = e < nk ? L.keys[CHUNK + e] : 0ull;
                }
                bitonic128(sk, ek, lane);
                const uint32_t mm = nk < kp ? nk : kp;
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const uint32_t e = (uint32_t)lane + 64u * t;
                    sk[t] = e < mm ? ek[t] : 0ull;  // the fetch's exact keys
                    ek[t] = 0;
                }
                bitonic128(sk, ek, lane);
                const uint32_t ko = mm < a.k_out ? mm : a.k_out;
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const uint32_t e = (uint32_t)lane + 64u * t;
                    if (e < ko) {
                        a.out_rows[(uint64_t)qi * a.k_out + e] = key_row(sk[t]);
                        a.out_scores[(uint64_t)qi * a.k_out + e] = f32_from_ord((uint32_t)(sk[t] >> 32));
                    }
                }
                if (lane == 0) {
                    a.out_n[qi] = ko;
                    a.merged_n[qi] = mm;
                }
            }
            __syncthreads();
            if (tid == 0) L.last = atomicAdd(&qs->fin, 1u) == 1;
            __syncthreads();
            if (L.last) reset_query(a, qi);
            return;
        }
        if (nk > kp) {
            for (uint32_t j = tid; j < nk; j += SCAN_WG)
                if (count_greater(L.keys, nk, L.keys[j]) == kp - 1) L.gtau = L.keys[j];
        }
        __syncthreads();
        const uint64_t T = L.gtau;  // 0 when every gathered key is in the fetch
        for (uint32_t j0 = 0; j0 < nk; j0 += SCAN_WG) {
            const uint32_t j = j0 + tid;
            const bool in = j < nk && L.keys[j] >= T;
            wave_append(L.tmp, &L.cnt2, SEL_TMP, in, in ? L.keys[CHUNK + j] : 0ull, lane);
        }
        __syncthreads();
        const uint32_t mm = L.cnt2;
        const uint32_t ko = mm < a.k_out ? mm : a.k_out;
        for (uint32_t j = tid; j < mm; j += SCAN_WG) {
            const uint64_t ek = L.tmp[j];
            const uint32_t r = count_greater(L.tmp, mm, ek);
            if (r < ko) {
                a.out_rows[(uint64_t)qi * a.k_out + r] = key_row(ek);
                a.out_scores[(uint64_t)qi * a.k_out + r] = f32_from_ord((uint32_t)(ek >> 32));
            }
        }
        if (tid == 0) {
            a.out_n[qi] = ko;
            a.merged_n[qi] = mm;
        }
        __syncthreads();
        if (tid == 0) L.last = atomicAdd(&qs->fin, 1u) == 1;
        __syncthreads();
        if (L.last) reset_query(a, qi);
        return;
    }
    for (uint32_t c0 = 0; c0 < total; c0 += CHUNK) {
        const uint64_t th = L.tau;
        const uint32_t c1 = c0 + CHUNK < total ? c0 + CHUNK : total;
        for (uint32_t i0 = c0; i0 < c1; i0 += 4 * SCAN_WG) {
            uint64_t v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t i = i0 + j * SCAN_WG + tid;
                v[j] = 0;
                if (i < c1) {
                    uint32_t r = 0;
                    while (r + 1 < ng && L.ovl[32 + r + 1] <= i) ++r;
                    v[j] = load_shared(&ckq[2 * (r * region + (i - L.ovl[32 + r]))]);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) wave_append(L.keys, &L.cnt, SCAN_CAP, v[j] != 0 && v[j] >= th, v[j], lane);
        }
        __syncthreads();
        if (L.cnt > CHUNK) {
            const uint32_t m = select_topk(L, L.cnt, kp);
            if (tid == 0) {
                L.cnt = m;
                if (m == kp && L.keys[kp - 1] > L.tau) L.tau = L.keys[kp - 1];
            }
            __syncthreads();
        }
    }
    const uint32_t m = select_topk(L, L.cnt, kp);
    uint64_t *outk = a.merged + (uint64_t)qi * kp;
    for (uint32_t j = tid; j < kp; j += SCAN_WG) outk[j] = j < m ? L.keys[j] : 0;
    if (tid == 0) a.merged_n[qi] = m;
    if (a.rr_src) {
        // the fetch set is every flushed pair whose scan key is at least the
        // m-th best; rank its exact keys and keep the best k_out
        const uint64_t T = m ? L.keys[m - 1] : ~0ull;
        __syncthreads();
        if (tid == 0) L.cnt2 = 0;
        __syncthreads();
        for (uint32_t i0 = 0; i0 < total; i0 += 4 * SCAN_WG) {
            uint64_t v[4], e[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t i = i0 + j * SCAN_WG + tid;
                v[j] = 0;
                e[j] = 0;
                if (i < total) {
                    uint32_t r = 0;
                    while (r + 1 < ng && L.ovl[32 + r + 1] <= i) ++r;
                    const uint64_t slot = 2 * (r * region + (i - L.ovl[32 + r]));
                    v[j] = load_shared(&ckq[slot]);
                    e[j] = load_shared(&ckq[slot + 1]);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) wave_append(L.tmp, &L.cnt2, SEL_TMP, v[j] != 0 && v[j] >= T, e[j], lane);
        }
        __syncthreads();
        const uint32_t mm = L.cnt2 < (uint32_t)SEL_TMP ? L.cnt2 : (uint32_t)SEL_TMP;
        const uint32_t ko = mm < a.k_out ? mm : a.k_out;
        for (uint32_t j = tid; j < mm; j += SCAN_WG) {
            const uint64_t ek = L.tmp[j];
            const uint32_t r = count_greater(L.tmp, mm, ek);
            if (r < ko) {
                a.out_rows[(uint64_t)qi * a.k_out + r] = key_row(ek);
                a.out_scores[(uint64_t)qi * a.k_out + r] = f32_from_ord((uint32_t)(ek >> 32));
            }
        }
        if (tid == 0) a.out_n[qi] = ko;
    } else if (a.out_rows) {
        const uint32_t ko = m < a.k_out ? m : a.k_out;
        for (uint32_t j = tid; j < ko; j += SCAN_WG) {
            const uint64_t kk = L.keys[j];
            a.out_rows[(uint64_t)qi * a.k_out + j] = key_row(kk);
            const uint32_t o = (uint32_t)(kk >> 32);
            a.out_scores[(uint64_t)qi * a.k_out + j] =
                IsInt<C>::v ? (float)(int32_t)(o ^ 0x80000000u) : f32_from_ord(o);
        }
        if (tid == 0) a.out_n[qi] = ko;
    }
    __syncthreads();
    if (tid == 0) L.last = atomicAdd(&qs->fin, 1u) == 1;
    __syncthreads();
    if (L.last) reset_query(a, qi);
}

template <int C, int LPR, int UPL, bool IDX, bool PREP>
__global__ __launch_bounds__(SCAN_WG) void scan_topk(ScanArgs a) {
    scan_topk_body<C, LPR, UPL, IDX, PREP>(a);
}
// The same scan with its registers held to three waves per SIMD (the int8
// transform scan: 144 VGPRs against 249, no spills), for two queries in
// flight: their workgroups then share CUs, which raised two-stream
// throughput 3.4% at a 1% slower kernel.
template <int C, int LPR, int UPL, bool IDX, bool PREP>
__global__ __launch_bounds__(SCAN_WG) __attribute__((amdgpu_waves_per_eu(3))) void scan_topk_lean(ScanArgs a) {
    scan_topk_body<C, LPR, UPL, IDX, PREP>(a);
}

// Exact keys of listed rows for the 1-bit asymmetric batch: rows[q][0,
// min(kept[q], cap)) of query q (grid row y), each row's key computed as
// compute_step_q1p computes it (the same layout, table, partial sums,
// reduction and row scale), into keys[q][i].  The re-score table is built
// from the rotated fp32 query qrot[q] in LDS; grid column x takes every
// gridDim.x-th wave step of the list.
template <int LPR, int UPL>
__global__ __launch_bounds__(SCAN_WG) void q1p_exact_rows(Q1pRowsArgs a) {
    using SH = ScanShape<C_Q1P, LPR, UPL>;
    constexpr int U = SH::U, G = SH::G;
    extern __shared__ __align__(16) unsigned char q1p_smem[];
    float *lut = (float *)q1p_smem;
    const uint32_t q = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    q1p_lut_build(a.qrot + (uint64_t)q * a.P, a.P, lut, (uint32_t)tid, SCAN_WG);
    __syncthreads();
    ScanRegs<C_Q1P, UPL> R{};
    const int pl = lane % LPR;
#pragma unroll
    for (int t = 0; t < UPL; ++t) {
        const uint32_t unit = pl + LPR * t;
        R.uok[t] = unit < a.units;
        R.ucl[t] = R.uok[t] ? unit : a.units - 1;
    }
    R.qf = lut;
    ScanArgs sa{};
    sa.codes = a.codes;
    sa.row_bytes = a.row_bytes;
    sa.scales = a.scales;
    const uint32_t n = a.kept[q] < a.cap ? a.kept[q] : (uint32_t)a.cap;
    const uint32_t *cand = a.rows + (uint64_t)q * a.cap;
    uint64_t *out = a.keys + (uint64_t)q * a.cap;
    const uint32_t stride = gridDim.x * (uint32_t)SH::WAVES * SH::RPS;
    for (uint32_t base = (blockIdx.x * SH::WAVES + (uint32_t)wave) * SH::RPS; base < n; base += stride) {
        StepData<C_Q1P, LPR, UPL> S;
        load_step<C_Q1P, LPR, UPL, true>(sa, R, cand, base, n, S, lane);
        float ex[U];
#pragma unroll
        for (int u = 0; u < U; ++u) ex[u] = q1p_exact_partial<LPR, UPL>(R, S.d[u], pl);
        const float tot = xreduce<U, LPR>(ex, lane);
        const uint32_t myrow = base + (uint32_t)(xrow<U, LPR>(lane) * G + lane / LPR);
        if (xrep<U, LPR>(lane) && myrow < n) out[myrow] = make_key(ord_f32(tot * (S.scale * a.scale_mul)), S.grow);
    }
}

// The 1-bit asymmetric counterpart of mq1_tau_exact (one workgroup per
// query): tau[q] = max(tau[q], the smallest exact key, computed as
// q1p_exact_rows computes it, of the rows of merged[q][0, kk)); nothing when
// merged_n[q] < kk.
template <int LPR, int UPL>
__global__ __launch_bounds__(SCAN_WG) void q1p_tau_exact(Q1pRowsArgs a, const uint64_t *merged,
                                                          const uint32_t *merged_n, uint32_t kk, uint64_t *tau) {
    using SH = ScanShape<C_Q1P, LPR, UPL>;
    constexpr int U = SH::U, G = SH::G;
    extern __shared__ __align__(16) unsigned char q1p_smem[];
    float *lut = (float *)q1p_smem;
    uint32_t *srow = (uint32_t *)(q1p_smem + q1p_lut_bytes(a.P));
    __shared__ uint64_t wmin[SH::WAVES];
    const uint32_t q = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (kk == 0 || merged_n[q] < kk) return;
    q1p_lut_build(a.qrot + (uint64_t)q * a.P, a.P, lut, (uint32_t)tid, SCAN_WG);
    const uint64_t *mk = merged + (uint64_t)q * kk;
    int bad = 0;
    for (uint32_t i = (uint32_t)tid; i < kk; i += SCAN_WG) {
        const uint32_t r = key_row(mk[i]);
        bad |= r >= a.nrows;
        srow[i] = r;
    }
    // (every row must be one of the index's: a list that is not is left alone)
    if (__syncthreads_or(bad)) return;
    ScanRegs<C_Q1P, UPL> R{};
    const int pl = lane % LPR;
#pragma unroll
    for (int t = 0; t < UPL; ++t) {
        const uint32_t unit = pl + LPR * t;
        R.uok[t] = unit < a.units;
        R.ucl[t] = R.uok[t] ? unit : a.units - 1;
    }
    R.qf = lut;
    ScanArgs sa{};
    sa.codes = a.codes;
    sa.row_bytes = a.row_bytes;
    sa.scales = a.scales;
    uint64_t m = ~0ull;
    for (uint32_t base = (uint32_t)wave * SH::RPS; base < kk; base += (uint32_t)SH::WAVES * SH::RPS) {
        StepData<C_Q1P, LPR, UPL> S;
        load_step<C_Q1P, LPR, UPL, true>(sa, R, srow, base, kk, S, lane);
        float ex[U];
#pragma unroll
        for (int u = 0; u < U; ++u) ex[u] = q1p_exact_partial<LPR, UPL>(R, S.d[u], pl);
        const float tot = xreduce<U, LPR>(ex, lane);
        const uint32_t myrow = base + (uint32_t)(xrow<U, LPR>(lane) * G + lane / LPR);
        if (xrep<U, LPR>(lane) && myrow < kk) {
            const uint64_t key = make_key(ord_f32(tot * (S.scale * a.scale_mul)), S.grow);
            m = key < m ? key : m;
        }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t v = __shfl_xor(m, o);
        m = v < m ? v : m;
    }
    if (lane == 0) wmin[wave] = m;
    __syncthreads();
    if (tid == 0) {
        for (int w = 0; w < SH::WAVES; ++w) m = wmin[w] < m ? wmin[w] : m;
        tau[q] = tau[q] > m ? tau[q] : m;
    }
}

// -------------------------------------------------- layouts and dispatch --
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
    // the per-wave lists must take a whole grab above the compaction target
    if (a.wcap < 2 * a.kprime + ScanShape<C, LPR, UPL>::WGRAB || (a.wcap & 63)) return hipErrorInvalidValue;
    if (a.n >= (1ull << 31)) return hipErrorInvalidValue;  // the kernel keeps row positions in 32 bits
    if (a.wstride < a.wcap || (a.rr_src && a.wstride < a.wcap + (a.rr_dim & ~3u))) return hipErrorInvalidValue;
    size_t lds = (size_t)(SCAN_WG / 64) * a.wstride * sizeof(uint64_t);
    if (lds < sizeof(TopkLds)) lds = sizeof(TopkLds);
    if (a.qraw) {
        if (!PrepShape<C, LPR, UPL>::ok || a.padded_dim != (uint32_t)PrepShape<C, LPR, UPL>::P)
            return hipErrorInvalidValue;
        const size_t need = (query_prep_lds(C, a.padded_dim) + 15) & ~(size_t)15;
        if (lds < need) lds = need;
    }
    ScanArgs b = a;
    if constexpr (C == C_Q1P) {
        // the exact re-score table, behind the lists and the transform's
        // scratch
        lds = (lds + 15) & ~(size_t)15;
        b.qf_off = (uint32_t)lds;
        lds += q1p_lut_bytes(a.padded_dim);
    }
    if (lds > 160 * 1024) return hipErrorInvalidValue;

    constexpr bool PP = PrepShape<C, LPR, UPL>::ok;  // layouts that can transform the query themselves
    if (a.cand) {
        if (PP && a.qraw)
            hipLaunchKernelGGL((scan_topk<C, LPR, UPL, true, PP>), dim3(a.grid + 1, nq), dim3(SCAN_WG), lds, s, b);
        else
            hipLaunchKernelGGL((scan_topk<C, LPR, UPL, true, false>), dim3(a.grid + 1, nq), dim3(SCAN_WG), lds, s, b);
    } else {
        if (PP && a.qraw) {
            if constexpr (C == C_Q8 && PP) {
                if (a.lean) {
                    hipLaunchKernelGGL((scan_topk_lean<C, LPR, UPL, false, true>), dim3(a.grid + 1, nq), dim3(SCAN_WG),
                                       lds, s, b);
                    return hipGetLastError();
                }
            }
            hipLaunchKernelGGL((scan_topk<C, LPR, UPL, false, PP>), dim3(a.grid + 1, nq), dim3(SCAN_WG), lds, s, b);
        } else {
            hipLaunchKernelGGL((scan_topk<C, LPR, UPL, false, false>), dim3(a.grid + 1, nq), dim3(SCAN_WG), lds, s, b);
        }
    }
    return hipGetLastError();
}

// Layouts whose query slice would exceed 64 registers per lane are never
// chosen (scan_supported rejects them), so they are not instantiated.
template <int C, int LPR, int UPL>
hipError_t go_fit(const ScanArgs &a, uint32_t nq, hipStream_t s) {
    if constexpr (UPL * Codec<C>::QN <= 64) return go<C, LPR, UPL>(a, nq, s);
    else return hipErrorInvalidValue;
}

template <int C>
hipError_t dispatch_layout(const Layout &L, const ScanArgs &a, uint32_t nq, hipStream_t s) {
    if (L.lpr == 64) {
        switch (L.upl) {
        case 1: return go_fit<C, 64, 1>(a, nq, s);
        case 2: return go_fit<C, 64, 2>(a, nq, s);
        case 3: return go_fit<C, 64, 3>(a, nq, s);
        case 4: return go_fit<C, 64, 4>(a, nq, s);
        case 6: return go_fit<C, 64, 6>(a, nq, s);
        case 8: return go_fit<C, 64, 8>(a, nq, s);
        case 12: return go_fit<C, 64, 12>(a, nq, s);
        case 16: return go_fit<C, 64, 16>(a, nq, s);
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

// One fused-scan launcher per codec, each defined in its own translation unit
// (bv_scan_<codec>.hip); lpr / upl as pick_layout chose them.
hipError_t scan_codec_f32dot(int lpr, int upl, const ScanArgs &a, uint32_t nq, hipStream_t s);
hipError_t scan_codec_f32l2(int lpr, int upl, const ScanArgs &a, uint32_t nq, hipStream_t s);
hipError_t scan_codec_q8(int lpr, int upl, const ScanArgs &a, uint32_t nq, hipStream_t s);
hipError_t scan_codec_q4(int lpr, int upl, const ScanArgs &a, uint32_t nq, hipStream_t s);
hipError_t scan_codec_q1a(int lpr, int upl, const ScanArgs &a, uint32_t nq, hipStream_t s);
hipError_t scan_codec_q1p(int lpr, int upl, const ScanArgs &a, uint32_t nq, hipStream_t s);
hipError_t scan_codec_ham(int lpr, int upl, const ScanArgs &a, uint32_t nq, hipStream_t s);
hipError_t scan_codec_i8s(int lpr, int upl, const ScanArgs &a, uint32_t nq, hipStream_t s);
hipError_t scan_codec_f32dot_s(int lpr, int upl, const ScanArgs &a, uint32_t nq, hipStream_t s);
hipError_t scan_codec_f32l2_s(int lpr, int upl, const ScanArgs &a, uint32_t nq, hipStream_t s);

}  // namespace bvk
