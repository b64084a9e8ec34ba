// Query batches on the gfx950 matrix cores.
//
//   mq_scan      int8 / int4 rows x queries x three int8 query levels on
//                v_mfma_i32_32x32x32_i8.  Every (row, query, level) dot is
//                an exact int32, combined per (row, query) in f64 exactly as
//                the single-query scan combines its three dots, so a batch
//                produces the same keys as the same queries scanned one at a
//                time.  Replaces the reference's per-query distanceQ8 /
//                distanceQ4 dispatches + score buffers for query batches
//                (src/engine/wgsl/distanceQ8.ts:56-82, distanceQ4.ts:44-78,
//                src/index/quant.ts:178-245, src/index.ts:473-517).
//   mq_scan_f32  fp32 rows x fp32 queries (dot / cosine / l2) on
//                v_mfma_f32_32x32x2f32 (src/engine/wgsl/distance.ts:24-177,
//                src/index/flat.ts:132-200 for query batches).  Its scores
//                are within a proven bound of the single-query scan's, and
//                serve as a prefilter: the rows that can rank are re-scored
//                by the single-query scan's own arithmetic, so a batch
//                returns exactly the single-query results.
//   mq_select    exact selection of each query's best kk keys.
//   mq_rerank    exact f64 re-rank of the selected candidates, 16 per wave.
//
// A batch runs as: a dense pass over a strided sample of the rows, whose
// kk-th best key per query is a valid pruning bound (it is the key of a real
// row, and a subset's kk-th best is never above the whole set's); a pass
// over every row that appends only the keys at or above that bound; and a
// select of the best kk appended keys.
#include "bv_kernels.h"
#include "bv_device.h"
#include "bv_mfma.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace bvk {

namespace {

// f64 combine of the three level dots, then the row scale: the arithmetic
// of the single-query int8 / int4 scans' finalisation (d already corrected
// for the int4 nibble offset).
__device__ __forceinline__ uint64_t q_key(double s0, double s1, double s2, int32_t d0, int32_t d1, int32_t d2,
                                          float scale, uint32_t row) {
    const double v = fma(s2, (double)d2, fma(s1, (double)d1, s0 * (double)d0));
    const float sc = (float)(v * (double)scale);
    return make_key(ord_f32(sc), row);
}

// 16 int4 codes (two words, nibble j of word g = code 8g + j) as 16 bytes
// n ^ 8 in code order: the even and odd nibbles, interleaved by byte perms.
__device__ __forceinline__ v4i unpack_q4(uint2 w) {
    const uint32_t x0 = w.x ^ 0x88888888u, x1 = w.y ^ 0x88888888u;
    const uint32_t e0 = x0 & 0x0f0f0f0fu, o0 = (x0 >> 4) & 0x0f0f0f0fu;
    const uint32_t e1 = x1 & 0x0f0f0f0fu, o1 = (x1 >> 4) & 0x0f0f0f0fu;
    v4i r;
    r[0] = (int)__builtin_amdgcn_perm(o0, e0, 0x05010400u);
    r[1] = (int)__builtin_amdgcn_perm(o0, e0, 0x07030602u);
    r[2] = (int)__builtin_amdgcn_perm(o1, e1, 0x05010400u);
    r[3] = (int)__builtin_amdgcn_perm(o1, e1, 0x07030602u);
    return r;
}

// The next float above / below a finite x (bit steps; +-0 go to the
// smallest subnormal of the right sign).
__device__ __forceinline__ float next_up(float x) {
    const uint32_t b = __float_as_uint(x);
    if ((b & 0x7fffffffu) == 0) return __uint_as_float(1u);
    return __uint_as_float((b & 0x80000000u) ? b - 1 : b + 1);
}
__device__ __forceinline__ float next_down(float x) { return -next_up(-x); }

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


// Per-query constants of the epilogue, in LDS: the level scales in f64
// (exact keys) and in f32 with the level-3 bound (prefilter), and the bound
// tau as a key and as an f32 score.
struct MqQuery {
    double s[3];
    int32_t c[3];        // int4: 8 * (sum of level l's bytes), the nibble offset's share; int8: 0
    float s0f, s1f, e3;  // e3 >= |s2 * (d2 - c2)| for any row: s2 * 127 * max|code| * P
    float tau_score;     // -inf when tau is 0
    uint64_t tau;
};

// A level dot corrected for the int4 nibble offset (int8: as is).
template <int BITS> __device__ __forceinline__ int32_t dq(int32_t d, int32_t c) {
    if constexpr (BITS == 4) return d - c;
    else return d;
}

// Keys of one wave's 64 rows x 32 queries from its accumulators: written
// densely (logical row i at cand[q][i]) or appended when at or above tau[q].
// Appending first checks an f32 upper bound of the score: the f32 sum of the
// first two level terms, plus the level-3 bound e3 and 2^-20 of the terms'
// magnitude (far above the f32 rounding of the sum and of the exact score),
// times the row scale.  Only keys whose bound reaches tau_score get the exact
// f64 combine.  sc: the scales of this wave's 64 rows (LDS).
template <int BITS>
__device__ __forceinline__ void epilogue(const MqArgs &a, const v16i (&acc)[2][3], uint64_t w0, uint32_t qb, int h,
                                         int c, const MqQuery *mq, const float *sc) {
    const bool full = w0 + 64 <= a.n;
    const uint32_t q = qb * MQ_QB + c;
    const bool qok = q < a.nq;
    const uint32_t qq = qok ? q : a.nq - 1;
    const MqQuery &Q = mq[c];
    uint64_t *out = a.cand + (uint64_t)qq * a.cap;
    if (!a.tau) {
#pragma unroll
        for (int fr = 0; fr < 2; ++fr)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t ri = fr * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                const uint64_t li = w0 + ri;
                if (qok && (full || li < a.n)) {
                    const uint64_t row = li * a.row_step;
                    out[li] = q_key(Q.s[0], Q.s[1], Q.s[2], dq<BITS>(acc[fr][0][r], Q.c[0]), dq<BITS>(acc[fr][1][r], Q.c[1]), dq<BITS>(acc[fr][2][r], Q.c[2]), sc[ri],
                                     (uint32_t)row);
                }
            }
        return;
    }
    // f32 upper bounds of all 32 keys, branch-free; the lane's rows come in
    // runs of four (r & 3), one 16-byte LDS read per run
    uint32_t maybe = 0;
#pragma unroll
    for (int fr = 0; fr < 2; ++fr) {
        float4 sv[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) sv[g] = *(const float4 *)&sc[fr * 32 + 8 * g + 4 * h];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float v4[4] = {sv[r >> 2].x, sv[r >> 2].y, sv[r >> 2].z, sv[r >> 2].w};
            const float scale = v4[r & 3];
            const float t0 = (float)dq<BITS>(acc[fr][0][r], Q.c[0]) * Q.s0f, t1 = (float)dq<BITS>(acc[fr][1][r], Q.c[1]) * Q.s1f;
            const float upper = (t0 + t1) * scale + (Q.e3 + 0x1p-20f * (fabsf(t0) + fabsf(t1))) * fabsf(scale);
            maybe |= (upper < Q.tau_score ? 0u : 1u) << (fr * 16 + r);
        }
    }
    if (!qok) maybe = 0;
    uint32_t pass = 0;  // bit fr*16 + r: key at or above the bound
    if (__ballot(maybe != 0)) {
#pragma unroll
        for (int fr = 0; fr < 2; ++fr)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t bit = 1u << (fr * 16 + r);
                if (maybe & bit) {
                    const uint32_t ri = fr * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                    const uint64_t li = w0 + ri;
                    if (full || li < a.n) {
                        const uint64_t key = q_key(Q.s[0], Q.s[1], Q.s[2], dq<BITS>(acc[fr][0][r], Q.c[0]), dq<BITS>(acc[fr][1][r], Q.c[1]),
                                                    dq<BITS>(acc[fr][2][r], Q.c[2]), sc[ri], (uint32_t)(li * a.row_step));
                        if (key >= Q.tau) pass |= bit;
                    }
                }
            }
    }
    if (!__ballot(pass != 0)) return;
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
                    const uint32_t ri = fr * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                    const uint64_t row = (w0 + ri) * a.row_step;
                    if (pos < a.cap)
                        out[pos] = q_key(Q.s[0], Q.s[1], Q.s[2], dq<BITS>(acc[fr][0][r], Q.c[0]), dq<BITS>(acc[fr][1][r], Q.c[1]), dq<BITS>(acc[fr][2][r], Q.c[2]), sc[ri],
                                          (uint32_t)row);
                    ++pos;
                }
            }
    }
}

// Bounds of one (row, query) key from its level-one dot D alone.  The exact
// key's score is f32(scale * (s0 D + s1 D1 + s2 D2)) and |s1 D1 + s2 D2| =
// |sum_i c_i R_i| <= |c|_2 |R|_2 (Cauchy-Schwarz), so with av = s0 D and
// bv = |c|_2 |R|_2 the score lies in scale * [av - bv, av + bv].  The extra
// 2^-20 |av| (and the 2^-18 already in rq) are far above every f32 rounding
// of the bound's own arithmetic and of the exact score.
__device__ __forceinline__ float mq1_upper(int32_t d, float s0f, float nr_rq, float scale) {
    const float av = (float)d * s0f;
    return fmaf(fabsf(av), 0x1p-20f, av + nr_rq) * scale;
}
__device__ __forceinline__ float mq1_lower(int32_t d, float s0f, float nr_rq, float scale) {
    const float av = (float)d * s0f;
    return fmaf(-fabsf(av), 0x1p-20f, av - nr_rq) * scale;
}

// The threshold pass keeps its entries without device-scope atomics (they
// are slow and serialize when many workgroups hit one query's counter, and
// a returning atomic would also make a wave wait for its outstanding tile
// loads).  Each tile's kept entries are staged in LDS by the wave that found
// them (a wave-private region); the waves that issue no tile loads move them
// to the workgroup's own bucket of each query, positions from LDS counters;
// mq1_compact joins the buckets into one list per query afterwards.
constexpr int MQ1_STAGE = 120;   // entries per wave per staging buffer
constexpr int MQ1_LOADERS = 4;   // waves 0..3 issue the tile loads; 4..7 move staged entries
struct Mq1Stage {
    uint64_t lk[2][MQ_WAVES][MQ1_STAGE];   // lower-bound keys, in lane order
    uint32_t uo[2][MQ_WAVES][MQ1_STAGE];   // order bits of the upper bounds
    uint16_t lo[2][MQ_WAVES][64];          // first entry of each lane
    uint16_t ln[2][MQ_WAVES][64];          // entries of each lane
    uint8_t qovf[MQ1_QB];                  // a query's entries did not all fit
};

// Inclusive prefix sum over the wave's 64 lanes in VALU (DPP row shifts
// within rows of 16, then the row broadcasts), no LDS traffic.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, false);  // row_shr:8
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false);  // row_bcast:15
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return x;
}

// Keys of one wave's 32 queries x the tile's MQ1_ROWS (32) rows.  Dense
// pass: the lower-bound key of every (row, query) (a NaN bound as order 0,
// below every key of the row).  Threshold pass: the rows whose upper bound
// reaches the query's bound are staged (buffer sb) as (lower-bound key,
// order bits of the upper bound; NaN: the largest).  Lane l holds query
// l % 32 and, in accumulator register r, tile row 8(r/4) + 4(l/32) + r%4.
// sc / cn: the tile rows' scales and code norms |c|_2 (LDS).
__device__ __forceinline__ void mq1_epilogue(const Mq1Args &a, const v16i &acc, uint64_t t0, uint32_t q,
                                             uint32_t qlocal, int h, float s0f, float rq, float tau_score,
                                             const float *sc, const float *cn, Mq1Stage &st, int sb) {
    // per-lane addresses are derived here, per tile: hoisted out of the tile
    // loop they would stay live across the matrix loop
    asm volatile("" : "+v"(q), "+v"(h));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const bool qok = q < a.nq;
    const bool full = t0 + MQ1_ROWS <= a.n;
    // the lane's rows come in runs of four: one 16-byte LDS read per run
    float sv[16], bv[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const float4 s4 = *(const float4 *)&sc[8 * g + 4 * h];
        const float4 n4 = *(const float4 *)&cn[8 * g + 4 * h];
        sv[4 * g] = s4.x, sv[4 * g + 1] = s4.y, sv[4 * g + 2] = s4.z, sv[4 * g + 3] = s4.w;
        bv[4 * g] = n4.x * rq, bv[4 * g + 1] = n4.y * rq, bv[4 * g + 2] = n4.z * rq, bv[4 * g + 3] = n4.w * rq;
    }
    auto row_of = [&](uint32_t r) { return 8 * (r >> 2) + 4 * (uint32_t)h + (r & 3); };
    if (!a.tau) {
        if (!qok) return;
        uint64_t *out = a.cand + (uint64_t)q * a.cap;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint64_t li = t0 + row_of(r);
            if (full || li < a.n) {
                const float lo = mq1_lower(acc[r], s0f, bv[r], sv[r]);
                out[li] = make_key(lo == lo ? ord_f32(lo) : 0u, (uint32_t)(a.row_base + li * a.row_step));
            }
        }
        return;
    }
    uint32_t p = 0;  // bit r: the row can reach the query's bound
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float up = mq1_upper(acc[r], s0f, bv[r], sv[r]);
        p |= (!(up < tau_score) ? 1u : 0u) << r;  // NaN: kept
    }
    if (!full) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (t0 + row_of(r) >= a.n) p &= ~(1u << r);
    }
    if (!qok) p = 0;
    // this wave's staging slots: an exclusive prefix of the lanes' counts (a
    // wave-private region: no LDS atomic, which would wait for the tile loads)
    const uint32_t mine = __popc(p);
    const uint32_t incl = wave_incl_scan(mine);
    st.lo[sb][wave][lane] = (uint16_t)(incl - mine);
    st.ln[sb][wave][lane] = (uint16_t)mine;
    if (!__builtin_amdgcn_readlane((int)incl, 63)) return;
    uint32_t pos = incl - mine;
    for (uint32_t m = p; m; m &= m - 1, ++pos) {
        if (pos >= (uint32_t)MQ1_STAGE) {
            st.qovf[qlocal] = 1;  // the query's list can no longer be complete: it falls back
            break;
        }
        const uint32_t bit = __builtin_ctz(m);
        int32_t d = 0;
        float s_ = 0.0f, b_ = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k)
            if ((uint32_t)k == bit) d = acc[k], s_ = sv[k], b_ = bv[k];
        const float lo = mq1_lower(d, s0f, b_, s_), up = mq1_upper(d, s0f, b_, s_);
        st.lk[sb][wave][pos] =
            make_key(lo == lo ? ord_f32(lo) : 0u, (uint32_t)(a.row_base + (t0 + row_of(bit)) * a.row_step));
        st.uo[sb][wave][pos] = up == up ? ord_f32(up) : 0xffffffffu;
    }
}

// 1 when a (row, query) upper bound can reach the query's bound (NaN: 1),
// as in mq1_epilogue.
__device__ __forceinline__ uint32_t mq1_reach(int32_t d, float s0f, float nr_rq, float scale, float tau_score) {
    return !(mq1_upper(d, s0f, nr_rq, scale) < tau_score) ? 1u : 0u;
}

// The staging half of mq1_epilogue for a tile whose reach bits p are formed
// (bit r: the lane's row 8(r/4) + 4h + r%4): the same slots and entries,
// each entry's scale and code norm read again from the tile's LDS.
__device__ __forceinline__ void mq1_stage(const Mq1Args &a, uint32_t p, const v16i &acc, uint64_t t0, uint32_t q,
                                          uint32_t qlocal, int h, float s0f, float rq, const float *sc,
                                          const float *cn, Mq1Stage &st, int sb) {
    // (the wave index as a scalar: the staging addresses stay in SGPRs)
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    auto row_of = [&](uint32_t r) { return 8 * (r >> 2) + 4 * (uint32_t)h + (r & 3); };
    if (t0 + MQ1_ROWS > a.n) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (t0 + row_of(r) >= a.n) p &= ~(1u << r);
    }
    if (q >= a.nq) p = 0;
    const uint32_t mine = __popc(p);
    const uint32_t incl = wave_incl_scan(mine);
    st.lo[sb][wave][lane] = (uint16_t)(incl - mine);
    st.ln[sb][wave][lane] = (uint16_t)mine;
    if (!__builtin_amdgcn_readlane((int)incl, 63)) return;
    uint32_t pos = incl - mine;
    for (uint32_t m = p; m; m &= m - 1, ++pos) {
        if (pos >= (uint32_t)MQ1_STAGE) {
            st.qovf[qlocal] = 1;  // the query's list can no longer be complete: it falls back
            break;
        }
        const uint32_t bit = __builtin_ctz(m);
        int32_t d = 0;
#pragma unroll
        for (int k = 0; k < 16; ++k)
            if ((uint32_t)k == bit) d = acc[k];
        const uint32_t rr = row_of(bit);
        const float s_ = sc[rr], b_ = cn[rr] * rq;
        const float lo = mq1_lower(d, s0f, b_, s_), up = mq1_upper(d, s0f, b_, s_);
        st.lk[sb][wave][pos] = make_key(lo == lo ? ord_f32(lo) : 0u, (uint32_t)(a.row_base + (t0 + rr) * a.row_step));
        st.uo[sb][wave][pos] = up == up ? ord_f32(up) : 0xffffffffu;
    }
}

// Staged entries of buffer fb into this workgroup's bucket of each query.
// Lane l of flushing wave f owns query f*64 + l of the block: its entries
// were staged by wave (f*64 + l) / 32, lanes c and c + 32 (c = l % 32), and
// its bucket length lives in the lane's register (len; ovf: it overflowed),
// so no atomic is needed.
__device__ __forceinline__ void mq1_flush(const Mq1Args &a, uint32_t qb, uint32_t wg, const Mq1Stage &st, int fb,
                                          int f, int lane, uint32_t &len, bool &ovf) {
    const uint32_t ql = (uint32_t)f * 64 + lane, w = ql / 32, c = ql % 32;
    const uint64_t bucket = ((uint64_t)(qb * MQ1_QB + ql) * a.nwg + wg) * a.capw;
    // the entries of lanes c and c + 32, in that order, in one loop
    const uint32_t off0 = st.lo[fb][w][c], n0 = st.ln[fb][w][c];
    const uint32_t off1 = st.lo[fb][w][c + 32], n1 = st.ln[fb][w][c + 32];
    for (uint32_t j = 0; j < n0 + n1; ++j) {
        const uint32_t i = j < n0 ? off0 + j : off1 + (j - n0);
        if (i >= (uint32_t)MQ1_STAGE) continue;  // not staged (the query is marked)
        if (len < a.capw) {
            a.cand[bucket + len] = st.lk[fb][w][i];
            a.up_out[bucket + len] = st.uo[fb][w][i];
        } else {
            ovf = true;
        }
        ++len;
    }
}

}  // namespace

// One workgroup = MQ_QB (32) queries, walking row tiles of MQ_ROWS (512)
// rows with MQ_WAVES (8) waves, two per SIMD.  The queries' three int8
// levels stay in LDS for the workgroup's lifetime (S steps x 3 levels x 1 KB,
// 96 KB at P = 1024), laid out as MFMA B operands: block (s, l) holds, at
// lane l's 16 bytes, unit 2s + l/32 of query l%32's level bytes.  Wave w
// takes rows [64w, 64w + 64) of a tile as two 32-row A operands: lane l
// supplies unit 2s + l/32 of row l%32 (int4 rows: that unit's 16 nibbles
// unpacked to bytes n ^ 8), so both operands pair the same codes.
// Accumulator register r of lane l holds row 8*(r/4) + 4*(l/32) + r%4,
// query l%32.  The codes of each wave's rows stream into two register
// groups of G steps, loads running one group ahead (into the next tile at a
// tile's end), so the K loop needs no barrier.
template <int S, int BITS>
__global__ __launch_bounds__(MQ_WAVES * 64) void mq_scan(MqArgs a) {
    using Code = typename std::conditional<BITS == 8, v4i, uint2>::type;  // 16 codes
    // Codes stream in groups of G steps: a group's loads are issued back to
    // back one group ahead, so the loads that read the same 128-byte line of
    // a row (int8: steps 4k .. 4k + 3 read line k; int4: eight steps) reach
    // L1 together and share one fill.  Issued a step at a time, the lines of
    // the 8 waves (64 KB per four int8 steps) overflow the 32 KB L1 and are
    // fetched up to four times.
    constexpr int G = S < 4 ? S : 4;
    __shared__ v4i qlds[S][3][64];
    __shared__ float srow[MQ_WAVES][64];
    __shared__ MqQuery mq[MQ_QB];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = lane >> 5, c = lane & 31;
    // Dispatch is round robin over the 8 XCDs, so workgroups b, b+8, ... share
    // an XCD.  The qblocks workgroups of one group walk the same row tiles on
    // one XCD and read the codes through its L2.
    const uint32_t b = blockIdx.x, xcd = b & 7u, slot = b >> 3;
    const uint32_t qb = slot % a.qblocks, grp = slot / a.qblocks;
    const uint64_t tstride = 8ull * a.groups;
    uint64_t tile = xcd + 8ull * grp;
    if (tile * MQ_ROWS >= a.n) return;

    // the block's query levels: 3S blocks of 1 KB, one wave instruction each
    {
        uint32_t q = qb * MQ_QB + c;
        if (q >= a.nq) q = a.nq - 1;
        const unsigned char *src = a.qlev + (uint64_t)q * a.qstride;
        for (int blk = wave; blk < S * 3; blk += MQ_WAVES) {
            const int st = blk / 3, lv = blk % 3;
            const uint32_t u = 2 * st + h;
            __builtin_amdgcn_global_load_lds((glb_void *)(src + ((uint64_t)u * 3 + lv) * 16),
                                             (lds_void *)&qlds[st][lv][0], 16, 0, 0);
        }
    }
    if (threadIdx.x < MQ_QB) {
        uint32_t q = qb * MQ_QB + threadIdx.x;
        if (q >= a.nq) q = a.nq - 1;
        const QLevelTail *t = (const QLevelTail *)(a.qlev + (uint64_t)q * a.qstride + a.tail_off);
        MqQuery &Q = mq[threadIdx.x];
        Q.s[0] = t->s[0];
        Q.s[1] = t->s[1];
        Q.s[2] = t->s[2];
        Q.s0f = (float)t->s[0];
        Q.s1f = (float)t->s[1];
#pragma unroll
        for (int l = 0; l < 3; ++l) Q.c[l] = BITS == 4 ? 8 * t->sum[l] : 0;
        Q.e3 = (float)(fabs(t->s[2]) * 127.0 * (BITS == 8 ? 127.0 : 8.0) * 16.0 * (double)a.units * 1.0000001);
        Q.tau = a.tau ? a.tau[q] : 0ull;
        Q.tau_score = Q.tau ? f32_from_ord((uint32_t)(Q.tau >> 32)) : -__builtin_inff();
    }

    auto row_ptrs = [&](uint64_t t, const Code *(&ap)[2]) {
        const uint64_t w0 = t * MQ_ROWS + (uint64_t)wave * 64;
#pragma unroll
        for (int fr = 0; fr < 2; ++fr) {
            uint64_t li = w0 + fr * 32 + c;
            if (li >= a.n) li = a.n - 1;  // rows past the end load a valid row; their results are dropped
            ap[fr] = (const Code *)(a.codes + li * a.row_step * a.W) + h;
        }
    };
    auto row_scale = [&](uint64_t t) {
        uint64_t li = t * MQ_ROWS + (uint64_t)wave * 64 + lane;
        if (li >= a.n) li = a.n - 1;
        return a.scales[li * a.row_step] * a.scale_mul;
    };
    const Code *ap[2];
    row_ptrs(tile, ap);
    Code ring[2][G][2];  // [group parity][step in group][row half]
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int fr = 0; fr < 2; ++fr) ring[0][j][fr] = ap[fr][2 * j];
    float scale = row_scale(tile);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // query levels and constants are in LDS

    for (;;) {  // row tiles
        const uint64_t ntile = tile + tstride;
        const bool more = ntile * MQ_ROWS < a.n;
        const Code *np[2];
        row_ptrs(more ? ntile : tile, np);
        v16i acc[2][3];
#pragma unroll
        for (int fr = 0; fr < 2; ++fr)
#pragma unroll
            for (int l = 0; l < 3; ++l) acc[fr][l] = v16i{};
#pragma unroll
        for (int st = 0; st < S; ++st) {
            const int gp = (st / G) & 1, j = st % G;
            if (j == 0) {  // the next group: this tile's, or the next tile's first
                const int ns = st + G;
#pragma unroll
                for (int jj = 0; jj < G; ++jj)
#pragma unroll
                    for (int fr = 0; fr < 2; ++fr) {
                        if (ns < S) ring[gp ^ 1][jj][fr] = ap[fr][2 * (ns + jj)];
                        else if (more) ring[gp ^ 1][jj][fr] = np[fr][2 * (ns - S + jj)];
                    }
            }
            v4i A[2];
#pragma unroll
            for (int fr = 0; fr < 2; ++fr) {
                if constexpr (BITS == 8) A[fr] = ring[gp][j][fr];
                else A[fr] = unpack_q4(ring[gp][j][fr]);
            }
            v4i B[3];
#pragma unroll
            for (int l = 0; l < 3; ++l) B[l] = qlds[st][l][lane];
#pragma unroll
            for (int fr = 0; fr < 2; ++fr)
#pragma unroll
                for (int l = 0; l < 3; ++l)
                    acc[fr][l] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[fr], B[l], acc[fr][l], 0, 0, 0);
            // keep each step's loads in its step: the scheduler would otherwise
            // sink the ring's loads next to their use and expose their latency
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr ((S / G) & 1) {  // one group per row: the next tile's first group is in half 1
#pragma unroll
            for (int j = 0; j < G; ++j)
#pragma unroll
                for (int fr = 0; fr < 2; ++fr) ring[0][j][fr] = ring[1][j][fr];
        }
        // this wave's 64 row scales, through wave-private LDS
        srow[wave][lane] = scale;
        if (more) scale = row_scale(ntile);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        epilogue<BITS>(a, acc, tile * MQ_ROWS + (uint64_t)wave * 64, qb, h, c, mq, srow[wave]);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (!more) break;
        ap[0] = np[0];
        ap[1] = np[1];
        tile = ntile;
    }
}

// Batched int8 prefilter on the first query level alone, on
// v_mfma_i32_32x32x32_i8, one workgroup per CU.  Each of the 8 waves holds
// one 32-query tile's level-one bytes in registers for the whole launch
// (S x 16 bytes per lane: the B operand of every K step), so a workgroup
// serves MQ1_QB = 256 queries and every code row is read from HBM once per
// 256 queries, staged in LDS and read by all 8 waves.  Tiles of MQ1_ROWS
// (32) rows rotate through four LDS buffers: three tiles stream in with
// global_load_lds (issued by waves 0..3) while one is multiplied.  LDS rows
// are one 16-byte unit longer than the codes, so the 32 rows an MFMA A
// operand reads at one unit spread over the banks, and each step's reads sit
// at a fixed offset from a per-lane base.  The matrix work is a third of a
// three-level scan; keys are not formed here: each (row, query) gets the
// bounds of mq1_upper / mq1_lower, the dense pass over a strided sample
// writes lower-bound keys (whose kk-th best per query is a valid bound: kk
// rows have exact keys at or above it), and the pass over every row keeps
// the rows whose upper bound reaches it.
template <int S, bool THR>
__global__ __launch_bounds__(MQ_WAVES * 64) void mq1_scan(Mq1Args a) {
    constexpr uint32_t U = 2 * S;     // 16-byte units per row (<= 64)
    constexpr uint32_t RS = U + 1;    // LDS row stride in units: one unit of padding
    constexpr uint32_t PER_WAVE = MQ1_ROWS / MQ1_LOADERS;  // rows each loader wave loads per tile
    // four buffers as separate LDS objects, each unrolled loop quarter naming
    // its own, so the compiler can see that pending tile loads do not touch
    // the rows being read
    __shared__ v4i tb0[MQ1_ROWS * RS], tb1[MQ1_ROWS * RS], tb2[MQ1_ROWS * RS], tb3[MQ1_ROWS * RS];
    __shared__ float sc0[MQ1_ROWS], sc1[MQ1_ROWS], sc2[MQ1_ROWS], sc3[MQ1_ROWS];
    __shared__ float cs0[MQ1_ROWS], cs1[MQ1_ROWS], cs2[MQ1_ROWS], cs3[MQ1_ROWS];
    __shared__ Mq1Stage stage;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = lane >> 5, c = lane & 31;
    const uint64_t ntiles = (a.n + MQ1_ROWS - 1) / MQ1_ROWS;
    const uint32_t qb = blockIdx.x % a.qblocks;
    const uint32_t wg = blockIdx.x / a.qblocks;  // a.nwg workgroups per query block
    const bool loader = wave < MQ1_LOADERS;
    constexpr bool thr = THR;  // (the launch picks THR from a.tau)
    for (uint32_t i = threadIdx.x; i < 2 * MQ_WAVES * 64; i += MQ_WAVES * 64)
        stage.ln[i / (MQ_WAVES * 64)][(i / 64) % MQ_WAVES][i % 64] = 0;
    if (threadIdx.x < MQ1_QB) stage.qovf[threadIdx.x] = 0;
    uint32_t blen = 0;  // flushing lanes: the owned query's bucket length
    bool bovf = false;
    // this workgroup's tiles: wg, wg + nwg, ...
    const uint64_t mine = wg < ntiles ? (ntiles - wg + a.nwg - 1) / a.nwg : 0;

    // this wave's queries: level one (unit u of a query's packed levels:
    // 48 bytes, level one first) as B operands, lane l: unit 2st + l/32
    const uint32_t qlocal = (uint32_t)wave * 32 + c;
    const uint32_t q = qb * MQ1_QB + qlocal;
    const bool wave_live = qb * MQ1_QB + (uint32_t)wave * 32 < a.nq;
    const uint32_t qc = q < a.nq ? q : a.nq - 1;
    const unsigned char *qsrc = a.qlev + (uint64_t)qc * a.qstride;
    v4i qreg[S];
#pragma unroll
    for (int st = 0; st < S; ++st) qreg[st] = *(const v4i *)(qsrc + (uint64_t)(2 * st + h) * 48);
    const QLevelTail *qt = (const QLevelTail *)(qsrc + a.tail_off);
    const float s0f = (float)qt->s[0];
    const float rq = a.rq[qc];
    const uint64_t tau = thr ? a.tau[qc] : 0ull;
    const float tau_score = tau ? f32_from_ord((uint32_t)(tau >> 32)) : -__builtin_inff();

    // tile k (the workgroup's k-th) into (tl, sc, cs) by the loader waves,
    // one load instruction per row (lanes 0 .. U-1: the row's units in
    // order), PER_WAVE rows each; the rows' scales and code norms by wave 0
    // (one dword per lane, lanes 0 .. 31)
    auto load_tile = [&](uint64_t k, v4i *tl, float *sc, float *cs) {
        const uint64_t t = wg + k * a.nwg;
        const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
        const uint32_t lb = lds_addr(&tl[wv * PER_WAVE * RS]);
        if ((uint32_t)lane < U) {
#pragma unroll
            for (uint32_t j = 0; j < PER_WAVE; ++j) {
                uint64_t li = t * MQ1_ROWS + wv * PER_WAVE + j;
                if (li >= a.n) li = a.n - 1;  // rows past the end load a valid row; their results are dropped
                lds_dma16((const v4i *)(a.codes + li * a.row_step * a.W) + lane, lb + j * RS * 16);
            }
        }
        if (wv == 0 && lane < MQ1_ROWS) {
            uint64_t li = t * MQ1_ROWS + (uint32_t)lane;
            if (li >= a.n) li = a.n - 1;
            lds_dma4(a.scales + li * a.row_step, lds_addr(sc));
            lds_dma4(a.cn + li * a.row_step, lds_addr(cs));
        }
    };
    // tile k from (tl, sc, cs), staging into buffer k & 1, while tile k + 3
    // streams into (ntl, nsc, ncs) and the previous tile's staged entries are
    // moved to the buckets
    auto run_tile = [&](uint64_t k, const v4i *tl, const float *sc, const float *cs, v4i *ntl, float *nsc,
                        float *ncs) {
        // this wave's loads of tile k have landed: the loads of the (up to
        // two) later tiles issued after them may still run (vmcnt counts in
        // issue order); the dense pass writes keys, so it waits for all
        if (loader && thr) {
            const uint64_t after = (mine - 1 - k) < 2 ? (mine - 1 - k) : 2;
            if (wave == 0) {
                if (after == 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * (PER_WAVE + 2)));
                else if (after == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER_WAVE + 2));
                else __builtin_amdgcn_s_waitcnt(0);
            } else {
                if (after == 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PER_WAVE));
                else if (after == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER_WAVE));
                else __builtin_amdgcn_s_waitcnt(0);
            }
        } else if (loader || !thr) {
            __builtin_amdgcn_s_waitcnt(0);
        }
        // every wave's loads have landed, and every wave is done with tile
        // k - 1's buffers.  The barrier waits only for this wave's LDS
        // operations: a workgroup fence on LDS would also wait for the later
        // tiles' loads into LDS (and the flushing waves' bucket stores need
        // not complete here); the memory clobber keeps every access on its
        // side of it.
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (loader) {
            if (k + 3 < mine) load_tile(k + 3, ntl, nsc, ncs);
        } else if (thr) {
            mq1_flush(a, qb, wg, stage, (int)((k + 1) & 1), wave - MQ1_LOADERS, lane, blen, bovf);
        }
        if (wave_live) {
            // two accumulators (even and odd K steps), so consecutive MFMAs
            // do not wait on each other
            v16i acc2[2] = {v16i{}, v16i{}};
            // lane l reads row l%32, unit 2st + l/32: a fixed base plus a
            // per-step constant
            const v4i *A0 = tl + c * RS + h;
            // A operands read PF steps ahead of their MFMA, so the LDS latency
            // is hidden behind the matrix work
            constexpr int PF = S < 4 ? S : 4;
            v4i ar[PF];
#pragma unroll
            for (int st = 0; st < PF; ++st) ar[st] = A0[2 * st];
#pragma unroll
            for (int st = 0; st < S; ++st) {
                const v4i x = ar[st % PF];
                if (st + PF < S) ar[st % PF] = A0[2 * (st + PF)];
                acc2[st & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, qreg[st], acc2[st & 1], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);  // keep each step's read PF steps ahead
            }
            const v16i acc = acc2[0] + acc2[1];
            mq1_epilogue(a, acc, (wg + k * a.nwg) * MQ1_ROWS, q, qlocal, h, s0f, rq, tau_score, sc, cs, stage,
                         (int)(k & 1));
        }
    };

    if constexpr (!THR) {
        if (loader) {
            if (mine > 0) load_tile(0, tb0, sc0, cs0);
            if (mine > 1) load_tile(1, tb1, sc1, cs1);
            if (mine > 2) load_tile(2, tb2, sc2, cs2);
        }
        for (uint64_t k = 0; k < mine; k += 4) {
            run_tile(k, tb0, sc0, cs0, tb3, sc3, cs3);
            if (k + 1 >= mine) break;
            run_tile(k + 1, tb1, sc1, cs1, tb0, sc0, cs0);
            if (k + 2 >= mine) break;
            run_tile(k + 2, tb2, sc2, cs2, tb1, sc1, cs1);
            if (k + 3 >= mine) break;
            run_tile(k + 3, tb3, sc3, cs3, tb2, sc2, cs2);
        }
        return;
    }

    // ---- the threshold pass: each tile's bounds are formed while the matrix
    // cores multiply the next tile ----
    // Tile k's level-one dots stay in registers (pacc) until tile k + 1's
    // K loop, which tests them against the bound between its MFMAs (the VALU
    // issues while the matrix cores run), then stages the rows that can
    // reach it.  Tile k's scales and code norms are therefore read during
    // tile k + 1: they come one tile behind its codes (the scales of tile
    // j + 2 and the codes of tile j + 3 are issued at tile j), so their
    // buffer is overwritten only after the barrier that follows that read.
    // Staged entries of tile k are moved to the buckets at tile k + 2.
    auto load_codes = [&](uint64_t k, v4i *tl) {
        const uint64_t t = wg + k * a.nwg;
        const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
        const uint32_t lb = lds_addr(&tl[wv * PER_WAVE * RS]);
        if ((uint32_t)lane < U) {
#pragma unroll
            for (uint32_t j = 0; j < PER_WAVE; ++j) {
                uint64_t li = t * MQ1_ROWS + wv * PER_WAVE + j;
                if (li >= a.n) li = a.n - 1;  // rows past the end load a valid row; their results are dropped
                lds_dma16((const v4i *)(a.codes + li * a.row_step * a.W) + lane, lb + j * RS * 16);
            }
        }
    };
    auto load_scales = [&](uint64_t k, float *sc, float *cs) {
        if (wave == 0 && lane < MQ1_ROWS) {
            uint64_t li = (wg + k * a.nwg) * MQ1_ROWS + (uint32_t)lane;
            if (li >= a.n) li = a.n - 1;
            lds_dma4(a.scales + li * a.row_step, lds_addr(sc));
            lds_dma4(a.cn + li * a.row_step, lds_addr(cs));
        }
    };
    v16i pacc = v16i{};  // the previous tile's level-one dots
    // tile k's matrix work from tl, with tile k - 1's bounds from its dots
    // and (psc, pcs); issues tile k + 3's codes into ntl and tile k + 2's
    // scales into (nsc, ncs)
    auto run_tile2 = [&](uint64_t k, const v4i *tl, const float *psc, const float *pcs, v4i *ntl, float *nsc,
                         float *ncs) {
        // tile k's codes and tile k - 1's scales have landed: both were
        // issued at tile k - 3 (or before the loop, in the same order);
        // the loads of tiles k - 2 and k - 1 may still run (vmcnt counts in
        // issue order): codes of k + 1 and k + 2, scales of k and k + 1
        if (loader) {
            const uint64_t left = mine - 1 - k;
            if (wave == 0) {
                if (left >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PER_WAVE + 4));
                else if (left == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER_WAVE + 4));
                else __builtin_amdgcn_s_waitcnt(vmcnt_imm(2));
            } else {
                if (left >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PER_WAVE));
                else if (left == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER_WAVE));
                else __builtin_amdgcn_s_waitcnt(0);
            }
        }
        // (as in run_tile: this wave's LDS operations, then the barrier)
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        // The flushing waves move staged entries first; the loader waves
        // multiply first (the matrix cores are theirs alone meanwhile) and
        // issue their loads after the K loop, while the flushing waves
        // multiply: issued at the barrier, the four loader waves' 32 KB of
        // loads kept them out of the K loop for ~1,100 cycles.
        if (!loader) mq1_flush(a, qb, wg, stage, (int)(k & 1), wave - MQ1_LOADERS, lane, blen, bovf);
        auto issue_loads = [&]() {
            if (loader) {
                if (k + 3 < mine) load_codes(k + 3, ntl);
                if (k + 2 < mine) load_scales(k + 2, nsc, ncs);
            }
        };
        if (!wave_live) issue_loads();
        if (wave_live) {
            v16i acc = v16i{};  // one chain: back-to-back MFMAs of one shape forward their sums
            const v4i *A0 = tl + c * RS + h;
            constexpr int PF = S < 4 ? S : 4;
            v4i ar[PF];
#pragma unroll
            for (int st = 0; st < PF; ++st) ar[st] = A0[2 * st];
            // element r of the lane's rows of tile k - 1 is row
            // 8(r/4) + 4h + r%4; its scale and norm are read one element ahead
            const float *psh = psc + 4 * h, *pnh = pcs + 4 * h;
            float sv = psh[0], nv = pnh[0];
            uint32_t p = 0;
#pragma unroll
            for (int st = 0; st < S; ++st) {
                const v4i x = ar[st % PF];
                if (st + PF < S) ar[st % PF] = A0[2 * (st + PF)];
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, qreg[st], acc, 0, 0, 0);
                // tile k - 1's elements [16 st / S, 16 (st + 1) / S) (tile 0
                // tests zero dots against a buffer not yet written: unused)
#pragma unroll
                for (int r = 16 * st / S; r < 16 * (st + 1) / S; ++r) {
                    float svn = 0.0f, nvn = 0.0f;
                    if (r < 15) {
                        const int rn = 8 * ((r + 1) >> 2) + ((r + 1) & 3);
                        svn = psh[rn];
                        nvn = pnh[rn];
                    }
                    p |= mq1_reach(pacc[r], s0f, nv * rq, sv, tau_score) << r;
                    // (here, between the MFMAs: not sunk to the staging below)
                    asm volatile("" : "+v"(p));
                    sv = svn;
                    nv = nvn;
                }
                __builtin_amdgcn_sched_barrier(0);  // keep each step's read PF steps ahead
            }
            issue_loads();
            if (k > 0)
                mq1_stage(a, p, pacc, (wg + (k - 1) * a.nwg) * MQ1_ROWS, q, qlocal, h, s0f, rq, psc, pcs, stage,
                          (int)((k - 1) & 1));
            pacc = acc;
        }
    };

    // before the loop, the loads of tiles -3, -2, -1 in the loop's pattern:
    // codes of 0, 1, 2 and scales of 0, 1
    if (loader) {
        if (mine > 0) load_codes(0, tb0);
        if (mine > 1) load_codes(1, tb1);
        if (mine > 0) load_scales(0, sc0, cs0);
        if (mine > 2) load_codes(2, tb2);
        if (mine > 1) load_scales(1, sc1, cs1);
    }
    for (uint64_t k = 0; k < mine; k += 4) {
        run_tile2(k, tb0, sc3, cs3, tb3, sc2, cs2);
        if (k + 1 >= mine) break;
        run_tile2(k + 1, tb1, sc0, cs0, tb0, sc3, cs3);
        if (k + 2 >= mine) break;
        run_tile2(k + 2, tb2, sc1, cs1, tb1, sc0, cs0);
        if (k + 3 >= mine) break;
        run_tile2(k + 3, tb3, sc2, cs2, tb2, sc1, cs1);
    }
    // the last tile's bounds (its scales have landed after the wait), the
    // staged entries of the last two tiles, then this workgroup's bucket
    // lengths
    if (loader) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (!loader && mine >= 2)
        mq1_flush(a, qb, wg, stage, (int)((mine - 2) & 1), wave - MQ1_LOADERS, lane, blen, bovf);
    if (wave_live && mine > 0) {
        const uint32_t lbuf = (uint32_t)((mine - 1) & 3);
        const float *lsc = lbuf == 0 ? sc0 : lbuf == 1 ? sc1 : lbuf == 2 ? sc2 : sc3;
        const float *lcs = lbuf == 0 ? cs0 : lbuf == 1 ? cs1 : lbuf == 2 ? cs2 : cs3;
        uint32_t p = 0;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t rr = 8 * (r >> 2) + 4 * (uint32_t)h + (r & 3);
            p |= mq1_reach(pacc[r], s0f, lcs[rr] * rq, lsc[rr], tau_score) << r;
        }
        mq1_stage(a, p, pacc, (wg + (mine - 1) * a.nwg) * MQ1_ROWS, q, qlocal, h, s0f, rq, lsc, lcs, stage,
                  (int)((mine - 1) & 1));
    }
    __syncthreads();
    if (!loader) {
        if (mine) mq1_flush(a, qb, wg, stage, (int)((mine - 1) & 1), wave - MQ1_LOADERS, lane, blen, bovf);
        const uint32_t ql = (uint32_t)(wave - MQ1_LOADERS) * 64 + lane, qq = qb * MQ1_QB + ql;
        if (qq < a.nq) a.cnt[(uint64_t)qq * a.nwg + wg] = bovf || stage.qovf[ql] ? 0xffffffffu : blen;
    }
}

// The first-level pass over 1-bit codes: mq1_scan over the +1 / -1 bytes of
// each row (bit set: +1, clear: -1), with the rows read as bits (P/8 bytes)
// and widened in LDS, so neither HBM nor the index holds the bytes.  The
// loader waves bring each tile's bits into a four-deep ring (one
// global_load_lds per wave and tile) three tiles ahead; at tile k every
// wave widens tile k + 1 into the other of two byte tiles (a 256-entry
// table of 8 codes per bit byte) while the matrix cores read tile k.  The
// rows' scales come with the bits (none: 1), and their code norms are the
// constant a.cn_const (every +1 / -1 row has the same norm).  The keys,
// bounds, staging and buckets are mq1_scan's.
template <int S, bool THR>
__global__ __launch_bounds__(MQ_WAVES * 64) void mq1_scan_bits(Mq1Args a) {
    constexpr uint32_t U = 2 * S;     // 16-byte units per widened row (8 <= U <= 64)
    constexpr uint32_t RS = U + 1;    // LDS row stride of the byte tiles in units
    constexpr uint32_t UB = U / 8;    // 16-byte units per row of bits
    constexpr uint32_t PER_WAVE = MQ1_ROWS / MQ1_LOADERS;
    constexpr uint32_t LN = PER_WAVE * UB;  // lanes of a loader wave's one load per tile
    static_assert(S >= 4 && LN <= 64, "1-bit rows of 128 to 1024 codes");
    __shared__ v4i tb[2][MQ1_ROWS * RS];
    __shared__ v4i bb[4][MQ1_ROWS * UB];
    __shared__ __align__(16) float scr[8][MQ1_ROWS];  // (8 deep: the threshold pass reads a tile's scales one tile late)
    __shared__ __align__(16) float ones[MQ1_ROWS];
    __shared__ __align__(16) float cnc[MQ1_ROWS];
    __shared__ uint2 lut[256];
    __shared__ Mq1Stage stage;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = lane >> 5, c = lane & 31;
    const uint64_t ntiles = (a.n + MQ1_ROWS - 1) / MQ1_ROWS;
    const uint32_t qb = blockIdx.x % a.qblocks;
    const uint32_t wg = blockIdx.x / a.qblocks;
    const bool loader = wave < MQ1_LOADERS;
    constexpr bool thr = THR;  // (the launch picks THR from a.tau)
    const bool scaled = a.scales != nullptr;
    for (uint32_t i = threadIdx.x; i < 2 * MQ_WAVES * 64; i += MQ_WAVES * 64)
        stage.ln[i / (MQ_WAVES * 64)][(i / 64) % MQ_WAVES][i % 64] = 0;
    if (threadIdx.x < MQ1_QB) stage.qovf[threadIdx.x] = 0;
    if (threadIdx.x < 256) {  // codes 8j .. 8j + 7 of a bit byte, as two words of +1 / -1 bytes
        const uint32_t b = threadIdx.x;
        uint2 e;
        e.x = 0;
        e.y = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            e.x |= (((b >> j) & 1u) ? 0x01u : 0xffu) << (8 * j);
            e.y |= (((b >> (4 + j)) & 1u) ? 0x01u : 0xffu) << (8 * j);
        }
        lut[b] = e;
    }
    if (threadIdx.x < MQ1_ROWS) {
        ones[threadIdx.x] = 1.0f;
        cnc[threadIdx.x] = a.cn_const;
    }
    uint32_t blen = 0;
    bool bovf = false;
    const uint64_t mine = wg < ntiles ? (ntiles - wg + a.nwg - 1) / a.nwg : 0;

    const uint32_t qlocal = (uint32_t)wave * 32 + c;
    const uint32_t q = qb * MQ1_QB + qlocal;
    const bool wave_live = qb * MQ1_QB + (uint32_t)wave * 32 < a.nq;
    const uint32_t qc = q < a.nq ? q : a.nq - 1;
    const unsigned char *qsrc = a.qlev + (uint64_t)qc * a.qstride;
    v4i qreg[S];
#pragma unroll
    for (int st = 0; st < S; ++st) qreg[st] = *(const v4i *)(qsrc + (uint64_t)(2 * st + h) * 48);
    const QLevelTail *qt = (const QLevelTail *)(qsrc + a.tail_off);
    const float s0f = (float)qt->s[0];
    const float rq = a.rq[qc];
    const uint64_t tau = thr ? a.tau[qc] : 0ull;
    const float tau_score = tau ? f32_from_ord((uint32_t)(tau >> 32)) : -__builtin_inff();

    // tile k's bits into ring slot k & 3 by the loader waves (lane i of wave
    // w: row w * PER_WAVE + i / UB, unit i % UB, so the tile's rows sit
    // back to back), and its scales by wave 0
    auto load_bits = [&](uint64_t k) {
        const uint64_t t = wg + k * a.nwg;
        const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
        const uint32_t lb = lds_addr(&bb[k & 3][wv * LN]);
        if ((uint32_t)lane < LN) {
            uint64_t li = t * MQ1_ROWS + wv * PER_WAVE + (uint32_t)lane / UB;
            if (li >= a.n) li = a.n - 1;  // rows past the end load a valid row; their results are dropped
            lds_dma16((const v4i *)(a.codes + li * a.row_step * a.W) + (uint32_t)lane % UB, lb);
        }
        if (scaled && wv == 0 && lane < MQ1_ROWS) {
            uint64_t li = t * MQ1_ROWS + (uint32_t)lane;
            if (li >= a.n) li = a.n - 1;
            lds_dma4(a.scales + li * a.row_step, lds_addr(&scr[k & 7][0]));
        }
    };
    // tile k's bits into byte tile k & 1: unit u of row r (codes 16u ..
    // 16u + 15) from the row's 16-bit half-word u
    auto widen = [&](uint64_t k) {
        const uint16_t *src = (const uint16_t *)&bb[k & 3][0];
        v4i *dst = &tb[k & 1][0];
        for (uint32_t i = threadIdx.x; i < MQ1_ROWS * U; i += MQ_WAVES * 64) {
            const uint32_t r = i / U, u = i % U;
            const uint32_t b16 = src[r * (UB * 8) + u];
            const uint2 lo = lut[b16 & 255u], hi = lut[b16 >> 8];
            dst[r * RS + u] = v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
        }
    };
    // this loader wave's loads of tile j have landed, with those of the
    // tiles after it (at most `after` of them) still running; the dense pass
    // writes keys, so it waits for all
    auto wait_tile = [&](uint64_t after) {
        if (loader && thr) {
            if (wave == 0 && scaled) {  // two loads per tile
                if (after >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(4));
                else if (after == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2));
                else __builtin_amdgcn_s_waitcnt(0);
            } else {
                if (after >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2));
                else if (after == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(1));
                else __builtin_amdgcn_s_waitcnt(0);
            }
        } else if (loader || !thr) {
            __builtin_amdgcn_s_waitcnt(0);
        }
    };

    if (loader) {
        if (mine > 0) load_bits(0);
        if (mine > 1) load_bits(1);
        if (mine > 2) load_bits(2);
    }
    if (mine > 0) {
        wait_tile(mine - 1 < 2 ? mine - 1 : 2);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        widen(0);
    }
    if constexpr (THR) {
        // The threshold pass as in mq1_scan: tile k - 1's bounds are tested
        // between tile k's MFMAs (its dots in pacc, its scales still in
        // their ring slot: eight deep, four tiles ahead of the loads), its
        // reaching rows staged after them and moved to the buckets at tile
        // k + 1; the loader waves multiply first and issue their loads
        // after the K loop, while the flushing waves multiply.
        v16i pacc = v16i{};
        for (uint64_t k = 0; k < mine; ++k) {
            if (k + 1 < mine) wait_tile(mine - 2 - k < 1 ? mine - 2 - k : 1);
            else wait_tile(0);
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (!loader) mq1_flush(a, qb, wg, stage, (int)(k & 1), wave - MQ1_LOADERS, lane, blen, bovf);
            if (k + 1 < mine) widen(k + 1);
            const float *psc = scaled ? &scr[(k - 1) & 7][0] : ones;  // tile k - 1's (unused at k = 0)
            if (!wave_live) {
                if (loader && k + 3 < mine) load_bits(k + 3);
                continue;
            }
            const v4i *tl = &tb[k & 1][0];
            v16i acc = v16i{};
            const v4i *A0 = tl + c * RS + h;
            constexpr int PF = S < 4 ? S : 4;
            v4i ar[PF];
#pragma unroll
            for (int st = 0; st < PF; ++st) ar[st] = A0[2 * st];
            const float *psh = psc + 4 * h, *pnh = cnc + 4 * h;
            float sv = psh[0], nv = pnh[0];
            uint32_t p = 0;
#pragma unroll
            for (int st = 0; st < S; ++st) {
                const v4i x = ar[st % PF];
                if (st + PF < S) ar[st % PF] = A0[2 * (st + PF)];
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, qreg[st], acc, 0, 0, 0);
                constexpr int EPS = S >= 16 ? 1 : 16 / S, SPE = S >= 16 ? S / 16 : 1;
#pragma unroll
                for (int e = 0; e < (st % SPE == SPE - 1 ? EPS : 0); ++e) {
                    const int r = st / SPE * EPS + e;
                    float svn = 0.0f, nvn = 0.0f;
                    if (r < 15) {
                        const int rn = 8 * ((r + 1) >> 2) + ((r + 1) & 3);
                        svn = psh[rn];
                        nvn = pnh[rn];
                    }
                    p |= mq1_reach(pacc[r], s0f, nv * rq, sv, tau_score) << r;
                    asm volatile("" : "+v"(p));  // (between the MFMAs: not sunk to the staging below)
                    sv = svn;
                    nv = nvn;
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            if (loader && k + 3 < mine) load_bits(k + 3);
            if (k > 0)
                mq1_stage(a, p, pacc, (wg + (k - 1) * a.nwg) * MQ1_ROWS, q, qlocal, h, s0f, rq, psc, cnc, stage,
                          (int)((k - 1) & 1));
            pacc = acc;
        }
        // the last tile's bounds, the staged entries of the last two tiles,
        // then this workgroup's bucket lengths
        __syncthreads();
        if (!loader && mine >= 2)
            mq1_flush(a, qb, wg, stage, (int)((mine - 2) & 1), wave - MQ1_LOADERS, lane, blen, bovf);
        if (wave_live && mine > 0) {
            const float *lsc = scaled ? &scr[(mine - 1) & 7][0] : ones;
            uint32_t p = 0;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t rr = 8 * (r >> 2) + 4 * (uint32_t)h + (r & 3);
                p |= mq1_reach(pacc[r], s0f, cnc[rr] * rq, lsc[rr], tau_score) << r;
            }
            mq1_stage(a, p, pacc, (wg + (mine - 1) * a.nwg) * MQ1_ROWS, q, qlocal, h, s0f, rq, lsc, cnc, stage,
                      (int)((mine - 1) & 1));
        }
        __syncthreads();
        if (!loader) {
            if (mine) mq1_flush(a, qb, wg, stage, (int)((mine - 1) & 1), wave - MQ1_LOADERS, lane, blen, bovf);
            const uint32_t ql = (uint32_t)(wave - MQ1_LOADERS) * 64 + lane, qq = qb * MQ1_QB + ql;
            if (qq < a.nq) a.cnt[(uint64_t)qq * a.nwg + wg] = bovf || stage.qovf[ql] ? 0xffffffffu : blen;
        }
        return;
    }
    for (uint64_t k = 0; k < mine; ++k) {
        // tile k + 1's bits have landed (every loader wave waited for its
        // own), tile k is widened, and every wave is done with tile k - 1
        if (k + 1 < mine) wait_tile(mine - 2 - k < 1 ? mine - 2 - k : 1);
        else wait_tile(0);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (loader) {
            if (k + 3 < mine) load_bits(k + 3);
        } else if (thr) {
            mq1_flush(a, qb, wg, stage, (int)((k + 1) & 1), wave - MQ1_LOADERS, lane, blen, bovf);
        }
        if (k + 1 < mine) widen(k + 1);
        if (wave_live) {
            const v4i *tl = &tb[k & 1][0];
            const float *sc = scaled ? &scr[k & 7][0] : ones;
            v16i acc2[2] = {v16i{}, v16i{}};
            const v4i *A0 = tl + c * RS + h;
            constexpr int PF = S < 4 ? S : 4;
            v4i ar[PF];
#pragma unroll
            for (int st = 0; st < PF; ++st) ar[st] = A0[2 * st];
#pragma unroll
            for (int st = 0; st < S; ++st) {
                const v4i x = ar[st % PF];
                if (st + PF < S) ar[st % PF] = A0[2 * (st + PF)];
                acc2[st & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, qreg[st], acc2[st & 1], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
            const v16i acc = acc2[0] + acc2[1];
            mq1_epilogue(a, acc, (wg + k * a.nwg) * MQ1_ROWS, q, qlocal, h, s0f, rq, tau_score, sc, cnc, stage,
                         (int)(k & 1));
        }
    }
    if (thr) {
        __syncthreads();
        if (!loader) {
            if (mine) mq1_flush(a, qb, wg, stage, (int)((mine - 1) & 1), wave - MQ1_LOADERS, lane, blen, bovf);
            const uint32_t ql = (uint32_t)(wave - MQ1_LOADERS) * 64 + lane, qq = qb * MQ1_QB + ql;
            if (qq < a.nq) a.cnt[(uint64_t)qq * a.nwg + wg] = bovf || stage.qovf[ql] ? 0xffffffffu : blen;
        }
    }
}

// One workgroup per query: the workgroups' buckets of the query joined into
// one list (bucket order; appended after the list's cnt[q] entries when
// append is set), and its length; a query with an overflowed bucket or more
// than cap entries gets length 0xffffffff (it falls back).
__global__ __launch_bounds__(1024) void mq1_compact(const uint64_t *bk, const uint32_t *bu, const uint32_t *bc,
                                                     uint32_t nwg, uint32_t capw, uint64_t cap, uint64_t *lk,
                                                     uint32_t *uo, uint32_t *cnt, int append) {
    __shared__ uint32_t off[1025];
    __shared__ uint32_t wsum[16];
    __shared__ uint32_t bad;
    const uint32_t q = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const uint32_t base = append ? cnt[q] : 0u;  // entries already in the list
    if ((uint64_t)base > cap) return;             // already overflowed
    if (tid == 0) bad = 0;
    __syncthreads();
    // bucket lengths (one thread per bucket; nwg <= 1024) and their exclusive
    // prefix: within each wave, then across the waves
    uint32_t c = 0;
    if (tid < nwg) {
        c = bc[(uint64_t)q * nwg + tid];
        if (c > capw) {
            bad = 1;
            c = 0;
        }
    }
    uint32_t incl = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(incl, o);
        if (lane >= o) incl += v;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    uint32_t before = 0;
    for (int w = 0; w < wave; ++w) before += wsum[w];
    if (tid < nwg) off[tid] = before + incl - c;
    if (tid == 1023) {
        uint32_t t = 0;
        for (int w = 0; w < 16; ++w) t += wsum[w];
        off[nwg] = t;
    }
    __syncthreads();
    const uint32_t total = base + off[nwg];
    if (bad || total > cap) {
        if (tid == 0) cnt[q] = 0xffffffffu;
        return;
    }
    // wave v copies buckets v, v + 16, ...
    for (uint32_t w = wave; w < nwg; w += 16) {
        const uint32_t n = off[w + 1] - off[w];
        const uint64_t src = ((uint64_t)q * nwg + w) * capw, dst = (uint64_t)q * cap + base + off[w];
        for (uint32_t i = lane; i < n; i += 64) {
            lk[dst + i] = bk[src + i];
            uo[dst + i] = bu[src + i];
        }
    }
    if (tid == 0) cnt[q] = total;
}

// fp32 rows x fp32 queries on v_mfma_f32_32x32x2f32: the batched
// counterpart of the fp32 flat scan.  Same structure as mq_scan: the block's
// 32 queries stay in LDS, each wave streams 64 rows.  Lane l = 32h + c
// supplies, over the four MFMA steps of chunk t, elements 8t + 4h .. 8t +
// 4h + 3 of row c (A) and of query c (B), one 16-byte load each, so both
// operands pair the same elements.  The sum runs in the matrix core's own
// order, so a score differs from the single-query scan's by rounding only:
// at most E (launch_mq_f32_qconst) for every row.  l2 scores are
// 2 x.q - |x|^2 - |q|^2 from the rows' and queries' squared norms.
// a.W = dim (floats per row), a.units = dim / 8 chunks, a.qlev = the fp32
// queries, a.qstride their byte stride.
//
// Passes: dense (every key of logical row i at cand[q][i]); threshold with
// keys (append keys at or above tau[q]); threshold with row ids (rows_out:
// append every row whose score reaches tau's score minus slack[q], which
// keeps every row the exact scan can rank: a row in the exact top-kk has
// single-query score >= the kk-th best single-query score >= tau's score
// - E, hence matrix-core score >= tau's score - 2E).
template <int CHUNKS>
__global__ __launch_bounds__(MQ_WAVES * 64) void mq_scan_f32(MqArgs a) {
    constexpr int G = CHUNKS < 4 ? CHUNKS : 4;
    __shared__ float4 qlds[CHUNKS][64];
    __shared__ uint64_t qtau[MQ_QB];
    __shared__ float qts[MQ_QB];
    __shared__ float qn2[MQ_QB];
    __shared__ float rn2[MQ_WAVES][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = lane >> 5, c = lane & 31;
    const uint32_t b = blockIdx.x, xcd = b & 7u, slot = b >> 3;
    const uint32_t qb = slot % a.qblocks, grp = slot / a.qblocks;
    const uint64_t tstride = 8ull * a.groups;
    uint64_t tile = xcd + 8ull * grp;
    if (tile * MQ_ROWS >= a.n) return;
    {
        uint32_t q = qb * MQ_QB + c;
        if (q >= a.nq) q = a.nq - 1;
        const float *src = (const float *)(a.qlev + (uint64_t)q * a.qstride);
        for (int t = wave; t < CHUNKS; t += MQ_WAVES)
            __builtin_amdgcn_global_load_lds((glb_void *)(src + 8 * t + 4 * h), (lds_void *)&qlds[t][0], 16, 0, 0);
    }
    if (threadIdx.x < MQ_QB) {
        uint32_t q = qb * MQ_QB + threadIdx.x;
        if (q >= a.nq) q = a.nq - 1;
        const uint64_t t = a.tau ? a.tau[q] : 0ull;
        qtau[threadIdx.x] = t;
        float ts = t ? f32_from_ord((uint32_t)(t >> 32)) : -__builtin_inff();
        if (a.rows_out && t) {
            // tau's score minus the slack, rounded down
            const float r = (float)((double)ts - (double)a.slack[q]);
            ts = next_down(r);
        }
        qts[threadIdx.x] = ts;
        qn2[threadIdx.x] = a.l2 ? a.qsq[q] : 0.0f;
    }
    auto row_sq = [&](uint64_t t) {
        uint64_t li = t * MQ_ROWS + (uint64_t)wave * 64 + lane;
        if (li >= a.n) li = a.n - 1;
        return a.rsq[li * a.row_step];
    };
    float rsq_next = a.l2 ? row_sq(tile) : 0.0f;
    auto row_ptrs = [&](uint64_t t, const float4 *(&ap)[2]) {
        const uint64_t w0 = t * MQ_ROWS + (uint64_t)wave * 64;
#pragma unroll
        for (int fr = 0; fr < 2; ++fr) {
            uint64_t li = w0 + fr * 32 + c;
            if (li >= a.n) li = a.n - 1;  // rows past the end load a valid row; their results are dropped
            ap[fr] = (const float4 *)((const float *)a.codes + li * a.row_step * a.W + 4 * h);
        }
    };
    const float4 *ap[2];
    row_ptrs(tile, ap);
    float4 ring[2][G][2];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int fr = 0; fr < 2; ++fr) ring[0][j][fr] = ap[fr][2 * j];
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    const uint32_t q = qb * MQ_QB + c;
    const bool qok = q < a.nq;
    const uint32_t qq = qok ? q : a.nq - 1;
    uint64_t *out = a.cand + (uint64_t)qq * a.cap;
    for (;;) {
        const uint64_t ntile = tile + tstride;
        const bool more = ntile * MQ_ROWS < a.n;
        const float4 *np[2];
        row_ptrs(more ? ntile : tile, np);
        v16f acc[2] = {v16f{}, v16f{}};
#pragma unroll
        for (int t = 0; t < CHUNKS; ++t) {
            const int gp = (t / G) & 1, j = t % G;
            if (j == 0) {
                const int nt = t + G;
#pragma unroll
                for (int jj = 0; jj < G; ++jj)
#pragma unroll
                    for (int fr = 0; fr < 2; ++fr) {
                        if (nt < CHUNKS) ring[gp ^ 1][jj][fr] = ap[fr][2 * (nt + jj)];
                        else if (more) ring[gp ^ 1][jj][fr] = np[fr][2 * (nt - CHUNKS + jj)];
                    }
            }
            const float4 B = qlds[t][lane];
            const float bv[4] = {B.x, B.y, B.z, B.w};
#pragma unroll
            for (int fr = 0; fr < 2; ++fr) {
                const float4 A = ring[gp][j][fr];
                const float av[4] = {A.x, A.y, A.z, A.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[fr] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[e], bv[e], acc[fr], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr ((CHUNKS / G) & 1) {
#pragma unroll
            for (int j = 0; j < G; ++j)
#pragma unroll
                for (int fr = 0; fr < 2; ++fr) ring[0][j][fr] = ring[1][j][fr];
        }
        // l2: the score from the dot and the squared norms (this wave's 64
        // rows' norms through wave-private LDS)
        if (a.l2) {
            rn2[wave][lane] = rsq_next;
            if (more) rsq_next = row_sq(ntile);
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            const float qs2 = qn2[c];
#pragma unroll
            for (int fr = 0; fr < 2; ++fr)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float x2 = rn2[wave][fr * 32 + 8 * (r >> 2) + 4 * h + (r & 3)];
                    acc[fr][r] = 2.0f * acc[fr][r] - x2 - qs2;
                }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        }
        // keys: dense (logical row i at out[i]), appended at or above tau, or
        // row ids appended at or above the slackened bound
        const uint64_t w0 = tile * MQ_ROWS + (uint64_t)wave * 64;
        const bool full = w0 + 64 <= a.n;
        if (a.rows_out) {
            const float ts = qts[c];
            uint32_t pass = 0;
#pragma unroll
            for (int fr = 0; fr < 2; ++fr)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint64_t li = w0 + fr * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                    // a NaN score passes: the exact scan ranks it as it ranks any key
                    if (qok && (full || li < a.n) && !(acc[fr][r] < ts)) pass |= 1u << (fr * 16 + r);
                }
            if (__ballot(pass != 0)) {
                const uint32_t mine = __popc(pass);
                const uint32_t other = __shfl_xor(mine, 32);
                uint32_t base = 0;
                if (h == 0 && mine + other) base = atomicAdd(&a.cnt[qq], mine + other);
                base = __shfl(base, c);
                if (pass) {
                    uint32_t *ro = a.rows_out + (uint64_t)qq * a.cap;
                    uint64_t pos = (uint64_t)base + (h ? other : 0u);
#pragma unroll
                    for (int fr = 0; fr < 2; ++fr)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            if (pass & (1u << (fr * 16 + r))) {
                                const uint64_t li = w0 + fr * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                                if (pos < a.cap) ro[pos] = (uint32_t)(li * a.row_step);
                                ++pos;
                            }
                }
            }
        } else if (!a.tau) {
#pragma unroll
            for (int fr = 0; fr < 2; ++fr)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint64_t li = w0 + fr * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (qok && (full || li < a.n)) out[li] = make_key(ord_f32(acc[fr][r]), (uint32_t)(li * a.row_step));
                }
        } else {
            const uint64_t tau = qtau[c];
            const float ts = qts[c];
            uint32_t pass = 0;
#pragma unroll
            for (int fr = 0; fr < 2; ++fr)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float sc = acc[fr][r];
                    if (!(sc < ts)) {
                        const uint64_t li = w0 + fr * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                        if (qok && (full || li < a.n) && make_key(ord_f32(sc), (uint32_t)(li * a.row_step)) >= tau)
                            pass |= 1u << (fr * 16 + r);
                    }
                }
            if (__ballot(pass != 0)) {
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
                        for (int r = 0; r < 16; ++r)
                            if (pass & (1u << (fr * 16 + r))) {
                                const uint64_t li = w0 + fr * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                                if (pos < a.cap) out[pos] = make_key(ord_f32(acc[fr][r]), (uint32_t)(li * a.row_step));
                                ++pos;
                            }
                }
            }
        }
        if (!more) break;
        ap[0] = np[0];
        ap[1] = np[1];
        tile = ntile;
    }
}

// One workgroup per query.  The kk-th best key is found by binning the
// keys over their actual range (2048 bins of a power-of-two width, so keys
// concentrated in a few score octaves still spread over many bins) and
// narrowing into the bin that holds it.  When the best kk keys are wanted in
// order, the narrowing stops once the keys at or above that bin's lower edge
// fit the smallest sort that holds twice kk (at least 256, at most
// SEL_CAP); those are gathered and sorted.  When only the bound is wanted,
// it goes on until the kk-th key is alone in its bin, and one more pass
// picks it out (no sort).  Keys are unique, so exactly kk keys are at or
// above the kk-th.
constexpr int SEL_THREADS = 1024;
constexpr int SEL_BINS = 2048;
constexpr int SEL_CAP = 4096;
constexpr int SEL_KPT = 16;  // keys per thread held in registers (lists up to 16,384 keys)

__global__ __launch_bounds__(SEL_THREADS) void mq_select(MqSelArgs a) {
    __shared__ uint32_t hist[SEL_BINS];
    __shared__ uint64_t sel[SEL_CAP];
    __shared__ uint64_t red[2][SEL_THREADS / 64];
    __shared__ uint32_t s_bin, s_excl, s_cnt;
    const uint32_t q = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const uint32_t total = a.cnt[q];
    if (total == 0xffffffffu) {
        // a list marked incomplete (mq1_compact): its entries were never
        // written, so nothing is selected from it and its bound is left as
        // it was; the query runs alone afterwards
        if (tid == 0) {
            if (a.merged_n) a.merged_n[q] = 0;
            if (a.overflow) a.overflow[q] = 1u;
            if (a.out_n) a.out_n[q] = 0;
        }
        return;
    }
    const uint32_t n = (uint64_t)total < a.cap ? total : (uint32_t)a.cap;
    const uint64_t *keys = a.cand + (uint64_t)q * a.cap;
    const uint32_t kk = a.kk < n ? a.kk : n;
    const bool sorted = a.merged != nullptr || a.out_rows != nullptr;
    // lists of at most SEL_KPT keys per thread are read once into registers
    // and every pass below runs over those; longer lists re-read memory
    const bool cached = n <= (uint32_t)(SEL_THREADS * SEL_KPT);
    uint64_t kr[SEL_KPT];
    if (cached) {
#pragma unroll
        for (int j = 0; j < SEL_KPT; ++j) {
            const uint32_t i = tid + (uint32_t)j * SEL_THREADS;
            kr[j] = i < n ? keys[i] : 0ull;
        }
    }
    // f(key) for every key of the list
    auto each = [&](auto f) {
        if (cached) {
#pragma unroll
            for (int j = 0; j < SEL_KPT; ++j)
                if (tid + (uint32_t)j * SEL_THREADS < n) f(kr[j]);
        } else {
            for (uint32_t i = tid; i < n; i += SEL_THREADS) f(keys[i]);
        }
    };
    uint32_t lim = 256;
    while (lim < 2 * kk && lim < (uint32_t)SEL_CAP) lim <<= 1;
    uint64_t G = 0;  // keys >= G are gathered
    uint64_t Gend = ~0ull;  // the last key of the kk-th's bin
    if (n > kk) {
        uint64_t lo = ~0ull, hi = 0;
        each([&](uint64_t k) {
            lo = k < lo ? k : lo;
            hi = k > hi ? k : hi;
        });
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint64_t l2 = __shfl_xor(lo, o), h2 = __shfl_xor(hi, o);
            lo = l2 < lo ? l2 : lo;
            hi = h2 > hi ? h2 : hi;
        }
        if (lane == 0) {
            red[0][wave] = lo;
            red[1][wave] = hi;
        }
        __syncthreads();
        lo = red[0][0];
        hi = red[1][0];
        for (int w = 1; w < SEL_THREADS / 64; ++w) {
            lo = red[0][w] < lo ? red[0][w] : lo;
            hi = red[1][w] > hi ? red[1][w] : hi;
        }
        uint32_t above = 0, rem = kk;  // keys above [lo, hi]; rank of the kk-th within [lo, hi]
        for (;;) {
            const uint64_t span = hi - lo;
            const int shift = (span >> 11) ? 64 - __clzll((long long)(span >> 11)) : 0;  // (span >> shift) < 2048
            for (uint32_t i = tid; i < SEL_BINS; i += SEL_THREADS) hist[i] = 0;
            __syncthreads();
            each([&](uint64_t k) {
                if (k >= lo && k <= hi) atomicAdd(&hist[(uint32_t)((k - lo) >> shift)], 1u);
            });
            __syncthreads();
            if (wave == 0) {
                // lane l holds bins 2047 - 32l - j (j < 32): counts from the top
                uint32_t loc = 0;
                for (int j = 0; j < 32; ++j) loc += hist[SEL_BINS - 1 - (32 * lane + j)];
                uint32_t inc = loc;
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) {
                    const uint32_t v = __shfl_up(inc, o);
                    if (lane >= o) inc += v;
                }
                const uint32_t exc = inc - loc;
                const uint64_t bal = __ballot(exc < rem && rem <= inc);
                if (lane == __ffsll((unsigned long long)bal) - 1) {
                    uint32_t acc = exc;
                    for (int j = 0; j < 32; ++j) {
                        const uint32_t bin = SEL_BINS - 1 - (32 * lane + j);
                        const uint32_t cb = hist[bin];
                        if (acc + cb >= rem) {
                            s_bin = bin;
                            s_excl = acc;
                            s_cnt = cb;
                            break;
                        }
                        acc += cb;
                    }
                }
            }
            __syncthreads();
            const uint32_t bin = s_bin, excl = s_excl, cb = s_cnt;
            __syncthreads();
            G = lo + ((uint64_t)bin << shift);
            const uint64_t w = (1ull << shift) - 1;  // the bin's last key, without wrapping past 2^64
            Gend = hi - G > w ? G + w : hi;
            if ((sorted ? above + excl + cb <= lim : cb <= 1) || shift == 0) break;
            above += excl;
            rem -= excl;
            lo = G;
            hi = Gend;
        }
    }
    if (!sorted) {
        // the bound alone: the kk-th key is the one key in [G, Gend]
        if (tid == 0) s_cnt = 0;
        __syncthreads();
        if (n > kk)
            each([&](uint64_t k) {
                if (k >= G && k <= Gend) red[0][0] = k;  // (exactly one such key)
            });
        __syncthreads();
        if (tid == 0) {
            if (a.tau) {
                const uint64_t t = n > kk ? red[0][0] : 0ull;
                a.tau[q] = a.tau_max && a.tau[q] > t ? a.tau[q] : t;
            }
            if (a.merged_n) a.merged_n[q] = kk;
            if (a.overflow) a.overflow[q] = (uint64_t)total > a.cap ? 1u : 0u;
        }
        return;
    }
    if (tid == 0) s_cnt = 0;
    __syncthreads();
    each([&](uint64_t k) {
        if (k >= G && k != 0) {
            const uint32_t p = atomicAdd(&s_cnt, 1u);
            if (p < (uint32_t)SEL_CAP) sel[p] = k;
        }
    });
    __syncthreads();
    const uint32_t got = s_cnt < (uint32_t)SEL_CAP ? s_cnt : (uint32_t)SEL_CAP;
    uint32_t npow = 2;
    while (npow < got) npow <<= 1;
    for (uint32_t i = got + tid; i < npow; i += SEL_THREADS) sel[i] = 0;
    __syncthreads();
    sort_desc(sel, npow);
    const uint32_t m = got < kk ? got : kk;
    if (tid == 0) {
        if (a.tau) {
            const uint64_t t = n > kk ? sel[kk - 1] : 0ull;
            a.tau[q] = a.tau_max && a.tau[q] > t ? a.tau[q] : t;
        }
        if (a.merged_n) a.merged_n[q] = m;
        if (a.overflow) a.overflow[q] = (uint64_t)total > a.cap ? 1u : 0u;
    }
    if (a.merged)
        for (uint32_t i = tid; i < m; i += SEL_THREADS) a.merged[(uint64_t)q * a.kk + i] = sel[i];
    if (a.out_rows) {
        const uint32_t ko = m < a.k_out ? m : a.k_out;
        for (uint32_t i = tid; i < ko; i += SEL_THREADS) {
            a.out_rows[(uint64_t)q * a.k_out + i] = key_row(sel[i]);
            a.out_scores[(uint64_t)q * a.k_out + i] = f32_from_ord((uint32_t)(sel[i] >> 32));
        }
        if (tid == 0) a.out_n[q] = ko;
    }
}

// Exact re-rank of each query's selected candidates (Store.dotRow,
// src/store/store.ts:114-130) and the final top-k_out, one workgroup per
// query.  Lane 4c + m of a wave runs accumulator m of candidate c: the f64
// sum over elements 4j + m in order (each f32 x f32 product is exact in f64,
// so fma adds it with the reference's single rounding); lanes 4c .. 4c + 3
// then combine as ((a0 + a1) + a2) + a3 and add the tail elements in order.
// Sixteen candidates per wave run at once.
constexpr int RR_THREADS = 1024;
__global__ __launch_bounds__(RR_THREADS) void mq_rerank(MqRerankArgs a) {
    extern __shared__ float qv[];  // the query, dim floats
    __shared__ uint64_t ek[MAX_KPRIME];
    const uint32_t q = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const uint32_t dim = a.dim, vec = dim & ~3u;
    const float *qs = a.q + (uint64_t)q * a.q_stride;
    for (uint32_t i = tid; i < dim; i += RR_THREADS) qv[i] = qs[i];
    __syncthreads();
    const uint32_t m = a.merged_n[q];
    const uint64_t *mk = a.merged + (uint64_t)q * a.kprime;
    const int ci = lane >> 2, ai = lane & 3;
    for (uint32_t c0 = (uint32_t)wave * 16; c0 < m; c0 += (RR_THREADS / 64) * 16) {
        const uint32_t cand = c0 + ci;
        const bool have = cand < m;
        const uint32_t row = have ? key_row(mk[cand]) : 0u;
        const float *x = a.rows + (uint64_t)row * dim;
        double acc = 0.0;
        uint32_t j = ai;
        // 32 of the lane's elements loaded at once, then summed in order
        for (; j + 124 < vec; j += 128) {
            float xv[32];
#pragma unroll
            for (int u = 0; u < 32; ++u) xv[u] = x[j + 4 * u];
#pragma unroll
            for (int u = 0; u < 32; ++u) acc = fma((double)xv[u], (double)qv[j + 4 * u], acc);
        }
        for (; j + 28 < vec; j += 32) {
            float xv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) xv[u] = x[j + 4 * u];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = fma((double)xv[u], (double)qv[j + 4 * u], acc);
        }
        for (; j < vec; j += 4) acc = fma((double)x[j], (double)qv[j], acc);
        const double a1 = __shfl_down(acc, 1), a2 = __shfl_down(acc, 2), a3 = __shfl_down(acc, 3);
        if (have && ai == 0) {
            double sum = acc + a1;
            sum = sum + a2;
            sum = sum + a3;
            for (uint32_t i = vec; i < dim; ++i) sum = fma((double)x[i], (double)qv[i], sum);
            ek[cand] = make_key(ord_f32((float)sum), row);
        }
    }
    __syncthreads();
    // rank: key i goes to slot #{keys greater than it} (keys are unique)
    const uint32_t ko = m < a.k_out ? m : a.k_out;
    for (uint32_t i = tid; i < m; i += RR_THREADS) {
        const uint64_t ki = ek[i];
        uint32_t r = 0;
        for (uint32_t j2 = 0; j2 < m; ++j2) r += ek[j2] > ki ? 1u : 0u;
        if (r < ko) {
            a.out_rows[(uint64_t)q * a.k_out + r] = key_row(ki);
            a.out_scores[(uint64_t)q * a.k_out + r] = f32_from_ord((uint32_t)(ki >> 32));
        }
    }
    if (tid == 0) a.out_n[q] = ko;
}

namespace {

// One wave per row: f64 sum of squares in element order, rounded to f32.
__global__ __launch_bounds__(256) void row_sqnorms(const float *rows, uint64_t n, uint32_t dim, float *rsq,
                                                   uint32_t *max_bits) {
    const int lane = threadIdx.x & 63;
    const uint64_t nw = (uint64_t)gridDim.x * 4;
    uint32_t mx = 0;
    for (uint64_t r = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6); r < n; r += nw) {
        const float *x = rows + r * dim;
        double s = 0.0;
        for (uint32_t i = lane; i < dim; i += 64) s = fma((double)x[i], (double)x[i], s);
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) s += __shfl_xor(s, o);
        if (lane == 0) {
            rsq[r] = (float)s;
            // the bound uses a value no smaller than any row's: round up
            const float up = next_up((float)s);
            const uint32_t b = __float_as_uint(up);
            mx = b > mx ? b : mx;
        }
    }
    if (lane == 0 && mx) atomicMax(max_bits, mx);
}

// One wave per query: |q|^2 and the slack 2E of the exact fp32 batch.
__global__ __launch_bounds__(64) void mq_f32_qconst(const float *q, uint32_t dim, const uint32_t *max_bits, int l2,
                                                    float *qsq, float *slack) {
    const int lane = threadIdx.x;
    const float *x = q + (uint64_t)blockIdx.x * dim;
    double s = 0.0;
    for (uint32_t i = lane; i < dim; i += 64) s = fma((double)x[i], (double)x[i], s);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) s += __shfl_xor(s, o);
    if (lane == 0) {
        const double u = 0x1p-24;
        const double xn = sqrt((double)__uint_as_float(*max_bits)) * (1.0 + 0x1p-20);
        const double qn = sqrt(s) * (1.0 + 0x1p-20);
        const double e = l2 ? 4.0 * (dim + 4) * u * (xn + qn) * (xn + qn) : 3.0 * (dim + 2) * u * xn * qn;
        qsq[blockIdx.x] = (float)s;
        // 2E plus room for the subnormal products a matrix core may flush
        slack[blockIdx.x] = (float)((2.0 * e + dim * 0x1p-126) * (1.0 + 0x1p-10));
    }
}

// One wave per row: |c|_2 of the int8 codes, rounded up to f32 (the exact
// sum of squares from v_dot4 of each word with itself, below 2^24; f64
// square root).
__global__ __launch_bounds__(256) void row_code_norms(const uint32_t *codes, uint64_t n, uint32_t W, float *cn) {
    const int lane = threadIdx.x & 63;
    const uint64_t nw = (uint64_t)gridDim.x * 4;
    for (uint64_t r = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6); r < n; r += nw) {
        const uint32_t *w = codes + r * W;
        int acc = 0;
        for (uint32_t i = lane; i < W; i += 64) acc = __builtin_amdgcn_sdot4((int)w[i], (int)w[i], acc, false);
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) acc += __shfl_xor(acc, o);
        if (lane == 0) {
            const double v = sqrt((double)acc);
            float f = (float)v;
            if ((double)f < v) f = next_up(f);
            cn[r] = f;
        }
    }
}

// One wave per query: rq >= |R|_2 for R = s1 q1 + s2 q2, the part of the
// query the level-one prefilter leaves out (f64 sum, 2^-18 added, rounded up
// to f32); cnt[q] = cnt_value when cnt is set (the dense pass's key count).
__global__ __launch_bounds__(64) void mq1_qconst(const unsigned char *qlev, uint64_t qstride, uint32_t units,
                                                 uint32_t tail_off, float *rq, uint32_t *cnt, uint32_t cnt_value) {
    const int lane = threadIdx.x;
    const unsigned char *src = qlev + (uint64_t)blockIdx.x * qstride;
    const QLevelTail *t = (const QLevelTail *)(src + tail_off);
    const double s1 = t->s[1], s2 = t->s[2];
    double acc = 0.0;
    for (uint32_t i = lane; i < units * 16; i += 64) {
        const uint32_t u = i >> 4, j = i & 15;
        const double r = fma(s2, (double)(int8_t)src[(u * 3 + 2) * 16 + j], s1 * (double)(int8_t)src[(u * 3 + 1) * 16 + j]);
        acc = fma(r, r, acc);
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) acc += __shfl_xor(acc, o);
    if (lane == 0) {
        const double v = sqrt(acc) * (1.0 + 0x1p-18);
        float f = (float)v;
        if ((double)f < v) f = next_up(f);
        rq[blockIdx.x] = f;
        if (cnt) cnt[blockIdx.x] = cnt_value;
    }
}

// The 1-bit asymmetric batch's query term, with the row term 1: the
// single-query score is f32(f32 sum_i (bit_i ? x_i : -x_i) * scale), x the
// rotated query.  With x = s1 q1 + r (q1 the query's int8 level one, s1 its
// step), sum_i sign_i x_i = s1 D + sum_i sign_i r_i, D the level-one dot
// with the +1 / -1 row, and |sum_i sign_i r_i| <= |r|_1.  The f32 sum in
// order differs from the exact one by at most (P - 1) 2^-24 |x|_1; rq adds
// twice that to |r|_1, then 2^-18 of the whole, rounded up to f32 (the
// bound's f32 arithmetic and the final product are covered by the bound's
// own 2^-20 |s1 D| and by the 2^-18).  Level bytes: the C_Q4M unit layout
// (level one at bytes [48u, 48u + 16) of unit u, step s[0] undivided).
__global__ __launch_bounds__(64) void mq1_qconst_l1(const float *qrot, uint32_t P, const unsigned char *qlev,
                                                    uint64_t qstride, uint32_t tail_off, float *rq, uint32_t *cnt,
                                                    uint32_t cnt_value) {
    const int lane = threadIdx.x;
    const float *x = qrot + (uint64_t)blockIdx.x * P;
    const unsigned char *src = qlev + (uint64_t)blockIdx.x * qstride;
    const QLevelTail *t = (const QLevelTail *)(src + tail_off);
    const double s1 = t->s[0];
    double r = 0.0, ax = 0.0;
    for (uint32_t i = lane; i < P; i += 64) {
        const double xi = (double)x[i];
        const double q1 = (double)(int8_t)src[(uint64_t)(i >> 4) * 48 + (i & 15)];
        r += fabs(fma(-s1, q1, xi));
        ax += fabs(xi);
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        r += __shfl_xor(r, o);
        ax += __shfl_xor(ax, o);
    }
    if (lane == 0) {
        const double v = (r + 2.0 * (double)P * 0x1p-24 * ax) * (1.0 + 0x1p-18);
        float f = (float)v;
        if ((double)f < v) f = next_up(f);
        rq[blockIdx.x] = f;
        if (cnt) cnt[blockIdx.x] = cnt_value;
    }
}

// One workgroup per query: the kept rows whose upper bound reaches tau[q]
// (the kk-th best lower-bound key among them, so every row of the exact
// top kk is among these).
__global__ __launch_bounds__(1024) void mq1_keep(const uint64_t *cand, const uint32_t *up, const uint32_t *cnt,
                                                  uint64_t cap, const uint64_t *tau, uint32_t *rows,
                                                  uint32_t *kept) {
    __shared__ uint32_t s_n;
    const uint32_t q = blockIdx.x;
    // an overflowed list (more rows than cap, or marked incomplete) keeps
    // nothing: the query runs the single-query scan instead
    const uint32_t n = (uint64_t)cnt[q] <= cap ? cnt[q] : 0u;
    const uint64_t t = tau[q];
    const uint64_t *lk = cand + (uint64_t)q * cap;
    const uint32_t *uo = up + (uint64_t)q * cap;
    uint32_t *out = rows + (uint64_t)q * cap;
    if (threadIdx.x == 0) s_n = 0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n; i += 1024) {
        const uint32_t row = key_row(lk[i]);
        if (make_key(uo[i], row) >= t) out[atomicAdd(&s_n, 1u)] = row;
    }
    __syncthreads();
    if (threadIdx.x == 0) kept[q] = s_n;
}

// Sum over the 16 lanes of a DPP row, in every lane of the row.
__device__ __forceinline__ int row16_sum(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x128, 0xf, 0xf, false);  // row_ror:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x124, 0xf, 0xf, false);  // row_ror:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x122, 0xf, 0xf, false);  // row_ror:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x121, 0xf, 0xf, false);  // row_ror:1
    return x;
}

// The exact keys of rows row_at(0 .. n-1) of one query (levels in ql,
// steps s0..s2) with the single-query scan's arithmetic (three exact int32
// level dots, f64 combine, row scale), each handed to emit(i, key) by one
// lane of the row's 16-lane group.  Sixteen lanes per row, four rows per
// group in flight (rows i, i + 64, i + 128, i + 192 of a 1024-thread
// workgroup; a slot past the end repeats row i and is not emitted): each
// load instruction reads 256 contiguous bytes of four rows.
template <int UNITS, class RowAt, class Emit>
__device__ __forceinline__ void mq1_exact_rows(const uint32_t *codes, const float *scales, const v4i *ql,
                                               double s0, double s1, double s2, uint32_t n, RowAt row_at,
                                               Emit emit) {
    constexpr int PER = UNITS < 16 ? 1 : UNITS / 16;  // units per lane (lanes >= UNITS idle when UNITS < 16)
    constexpr uint32_t W = UNITS * 4;
    const uint32_t tid = threadIdx.x;
    const int l16 = tid & 15;
    constexpr int R = 4;
    for (uint32_t i = tid >> 4; i < n; i += 64 * R) {
        uint32_t rr[R];
        const v4i *x[R];
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const uint32_t ik = i + 64 * k < n ? i + 64 * k : i;
            rr[k] = row_at(ik);
            x[k] = (const v4i *)(codes + (uint64_t)rr[k] * W);
        }
        v4i cr[R][PER];
#pragma unroll
        for (int k = 0; k < R; ++k)
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const int u = l16 + 16 * j;
                cr[k][j] = u < UNITS ? x[k][u] : v4i{};
            }
        float sc[R];
#pragma unroll
        for (int k = 0; k < R; ++k) sc[k] = scales[rr[k]];
        int d[R][3];
#pragma unroll
        for (int k = 0; k < R; ++k) d[k][0] = d[k][1] = d[k][2] = 0;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int u = l16 + 16 * j;
            if (u >= UNITS) continue;
            const v4i q0 = ql[3 * u], q1 = ql[3 * u + 1], q2 = ql[3 * u + 2];
#pragma unroll
            for (int w = 0; w < 4; ++w)
#pragma unroll
                for (int k = 0; k < R; ++k) {
                    d[k][0] = __builtin_amdgcn_sdot4(cr[k][j][w], q0[w], d[k][0], false);
                    d[k][1] = __builtin_amdgcn_sdot4(cr[k][j][w], q1[w], d[k][1], false);
                    d[k][2] = __builtin_amdgcn_sdot4(cr[k][j][w], q2[w], d[k][2], false);
                }
        }
#pragma unroll
        for (int k = 0; k < R; ++k) {
            d[k][0] = row16_sum(d[k][0]), d[k][1] = row16_sum(d[k][1]), d[k][2] = row16_sum(d[k][2]);
            if (l16 == k && i + 64 * k < n) emit(i + 64 * k, q_key(s0, s1, s2, d[k][0], d[k][1], d[k][2], sc[k], rr[k]));
        }
    }
}

// One workgroup per query: the exact key of every kept row into keys[q][i].
template <int UNITS>
__global__ __launch_bounds__(1024) void mq1_exact(const uint32_t *codes, const float *scales,
                                                   const unsigned char *qlev, uint64_t qstride,
                                                   const uint32_t *rows, const uint32_t *kept, uint64_t cap,
                                                   uint64_t *keys) {
    __shared__ v4i ql[UNITS * 3];  // the query's packed levels: unit u, level l at 3u + l
    const uint32_t q = blockIdx.x, tid = threadIdx.x;
    const unsigned char *src = qlev + (uint64_t)q * qstride;
    for (uint32_t i = tid; i < UNITS * 3; i += 1024) ql[i] = ((const v4i *)src)[i];
    const QLevelTail *t = (const QLevelTail *)(src + (uint64_t)UNITS * 48);
    const double s0 = t->s[0], s1 = t->s[1], s2 = t->s[2];
    __syncthreads();
    const uint32_t *rq = rows + (uint64_t)q * cap;
    uint64_t *out = keys + (uint64_t)q * cap;
    mq1_exact_rows<UNITS>(codes, scales, ql, s0, s1, s2, kept[q], [&](uint32_t i) { return rq[i]; },
                          [&](uint32_t i, uint64_t key) { out[i] = key; });
}

// A tighter bound from exact keys, one workgroup per query: merged[q][0,
// kk) holds the kk best lower-bound keys of a list (mq_select's sorted
// output), so they name kk distinct rows; the smallest of their exact keys
// is at most the kk-th best exact key of all rows, so tau[q] = max(tau[q],
// that key) is still a bound that every row of the exact top kk reaches, and
// it is at least the list's kk-th lower-bound key.  A list shorter than kk
// (merged_n[q] < kk) leaves tau[q] as it is.
template <int UNITS>
__global__ __launch_bounds__(1024) void mq1_tau_exact(const uint32_t *codes, const float *scales,
                                                       const unsigned char *qlev, uint64_t qstride,
                                                       const uint64_t *merged, const uint32_t *merged_n, uint32_t kk,
                                                       uint64_t nrows, uint64_t *tau) {
    __shared__ v4i ql[UNITS * 3];
    __shared__ uint64_t wmin[16];
    const uint32_t q = blockIdx.x, tid = threadIdx.x;
    if (kk == 0 || merged_n[q] < kk) return;
    const uint64_t *mk = merged + (uint64_t)q * kk;
    // (every row must be one of the index's: a list that is not is left alone)
    int bad = 0;
    for (uint32_t i = tid; i < kk; i += 1024) bad |= key_row(mk[i]) >= nrows;
    if (__syncthreads_or(bad)) return;
    const unsigned char *src = qlev + (uint64_t)q * qstride;
    for (uint32_t i = tid; i < UNITS * 3; i += 1024) ql[i] = ((const v4i *)src)[i];
    const QLevelTail *t = (const QLevelTail *)(src + (uint64_t)UNITS * 48);
    const double s0 = t->s[0], s1 = t->s[1], s2 = t->s[2];
    __syncthreads();
    uint64_t m = ~0ull;
    mq1_exact_rows<UNITS>(codes, scales, ql, s0, s1, s2, kk, [&](uint32_t i) { return key_row(mk[i]); },
                          [&](uint32_t, uint64_t key) { m = key < m ? key : m; });
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t v = __shfl_xor(m, o);
        m = v < m ? v : m;
    }
    if ((tid & 63) == 0) wmin[tid >> 6] = m;
    __syncthreads();
    if (tid == 0) {
        for (int w = 0; w < 16; ++w) m = wmin[w] < m ? wmin[w] : m;
        tau[q] = tau[q] > m ? tau[q] : m;
    }
}

// Hamming batches on 1-bit codes: the exact key of every kept row (one
// workgroup per query, a row per thread), d = P - 2 * popcount(code ^
// query bits), the +1 / -1 dot that mq1_exact gives over the widened codes,
// combined by q_key with the query's level steps and row scale 1.
template <int W>
__global__ __launch_bounds__(1024) void ham_exact(const uint32_t *codes, const uint32_t *qbits,
                                                  const unsigned char *qlev, uint64_t qstride, uint32_t tail_off,
                                                  const uint32_t *rows, const uint32_t *kept, uint64_t cap,
                                                  uint64_t *keys) {
    __shared__ uint32_t qw[W];
    const uint32_t q = blockIdx.x, tid = threadIdx.x;
    if (tid < (uint32_t)W) qw[tid] = qbits[(uint64_t)q * W + tid];
    const QLevelTail *t = (const QLevelTail *)(qlev + (uint64_t)q * qstride + tail_off);
    const double s0 = t->s[0], s1 = t->s[1], s2 = t->s[2];
    __syncthreads();
    const uint32_t n = kept[q] < cap ? kept[q] : (uint32_t)cap;
    const uint32_t *rq = rows + (uint64_t)q * cap;
    uint64_t *out = keys + (uint64_t)q * cap;
    for (uint32_t i = tid; i < n; i += 1024) {
        const uint32_t row = rq[i];
        const uint4 *x = (const uint4 *)(codes + (uint64_t)row * W);
        int pc = 0;
#pragma unroll
        for (int j = 0; j < W / 4; ++j) {
            const uint4 v = x[j];
            pc += __popc(v.x ^ qw[4 * j]) + __popc(v.y ^ qw[4 * j + 1]) + __popc(v.z ^ qw[4 * j + 2]) +
                  __popc(v.w ^ qw[4 * j + 3]);
        }
        out[i] = q_key(s0, s1, s2, 32 * W - 2 * pc, 0, 0, 1.0f, row);
    }
}

}  // namespace

namespace {
// ---- list-major IVF batches (int8) -------------------------------------------
// Each query's candidates are its probed lists' rows in probe order, then
// list order (gatherCandidates); base[q][j] is where probe j's rows start.
// One thread per query; pair_count[c] counts the queries probing list c.
__global__ __launch_bounds__(256) void ivf_pair_bases(const uint32_t *probes, uint32_t nq, uint32_t nprobe,
                                                      const uint32_t *list_off, uint32_t *base, uint32_t *cnt,
                                                      uint32_t *pair_count) {
    const uint32_t q = blockIdx.x * 256 + threadIdx.x;
    if (q >= nq) return;
    uint32_t run = 0;
    for (uint32_t j = 0; j < nprobe; ++j) {
        const uint32_t c = probes[(uint64_t)q * nprobe + j];
        base[(uint64_t)q * nprobe + j] = run;
        run += list_off[c + 1] - list_off[c];
        atomicAdd(&pair_count[c], 1u);
    }
    cnt[q] = run;
}

// The (query, base) pairs grouped by list: pair_off = exclusive scan of
// pair_count; fill[c] starts at zero.
__global__ __launch_bounds__(256) void ivf_pair_scatter(const uint32_t *probes, const uint32_t *base, uint32_t npairs,
                                                        uint32_t nprobe, const uint32_t *pair_off, uint32_t *fill,
                                                        uint32_t *pair_q, uint32_t *pair_base) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= npairs) return;
    const uint32_t c = probes[i];
    const uint32_t slot = pair_off[c] + atomicAdd(&fill[c], 1u);
    pair_q[slot] = i / nprobe;
    pair_base[slot] = base[i];
}

// List-major IVF batches: each list's rows read once for every IVF_QC
// queries probing it, the single-query scan's key (the three levels' exact
// int32 dots, combined in f64) written at the row's candidate position of
// each query.
constexpr int IVF_QC = 8;
// chunks[c] = the list's work items (IVF_QC queries each).
__global__ __launch_bounds__(256) void ivf_chunk_counts(const uint32_t *pair_count, uint32_t nlist, uint32_t *chunks) {
    const uint32_t c = blockIdx.x * 256 + threadIdx.x;
    if (c < nlist) chunks[c] = (pair_count[c] + IVF_QC - 1) / IVF_QC;
}

// One workgroup per work item: a list and up to IVF_QC of the queries
// probing it (chunk_off = exclusive scan of the lists' item counts), so a
// list probed by many queries spreads over many workgroups.  The work runs
// on v_mfma_i32_32x32x32_i8: IVF_LM_WAVES waves per workgroup,
// each taking 32-row tiles of the list.  B holds 24 columns, level l of
// query k at column 8l + k (columns 24-31 and missing queries are zero),
// staged in LDS by 16-byte unit so lane (c, h) reads column c at unit
// 2 * step + h; A is row c of the tile at the same unit (int4 rows unpacked
// to n ^ 8 bytes).  The int32 dots are exact; the three level dots of a
// (row, query) meet in a per-wave LDS tile and q_key combines them in f64,
// giving the single-query scan's key.
constexpr uint32_t IVF_LM_WAVES = 4;  // eight measured slower for int8 rows (1.58 ms against 1.35 ms at 4M x 768)
template <int UNITS, int BITS>
__global__ __launch_bounds__(IVF_LM_WAVES * 64) void ivf_list_mfma(const uint32_t *codes, const float *scales, float scale_mul,
                                                     const uint32_t *list_off, const uint32_t *list_rows,
                                                     uint32_t nlist, const uint32_t *chunk_off,
                                                     const uint32_t *pair_off, const uint32_t *pair_count,
                                                     const uint32_t *pair_q, const uint32_t *pair_base,
                                                     const unsigned char *qlev, uint64_t qstride, uint64_t *cand,
                                                     uint64_t cap) {
    static_assert(IVF_QC == 8 && UNITS % 2 == 0, "24 columns: three levels of eight queries");
    constexpr int S = UNITS / 2;                 // K steps of 32 codes
    constexpr uint32_t W = UNITS * BITS / 2;     // words per row
    __shared__ v4i bq[S][2][32];
    __shared__ int32_t stg[IVF_LM_WAVES][32][25];  // per wave: 32 rows x 24 columns (+1)
    __shared__ double qs[IVF_QC][3];
    __shared__ int32_t qc[IVF_QC][3];
    __shared__ uint32_t qid[IVF_QC], qbase[IVF_QC];
    const uint32_t item = blockIdx.x, tid = threadIdx.x;
    uint32_t lo = 0, hi = nlist;  // the list: the last c with chunk_off[c] <= item
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) / 2;
        if (chunk_off[mid] <= item) lo = mid;
        else hi = mid;
    }
    const uint32_t li = lo;
    const uint32_t np = pair_count[li], p0 = pair_off[li];
    const uint32_t pc = (item - chunk_off[li]) * IVF_QC;
    const uint32_t r0 = list_off[li], nrows = list_off[li + 1] - r0;
    if (chunk_off[li] > item || pc >= np || nrows == 0) return;  // past the last item
    const uint32_t m = np - pc < (uint32_t)IVF_QC ? np - pc : (uint32_t)IVF_QC;
    for (uint32_t i = tid; i < (uint32_t)UNITS * 32; i += IVF_LM_WAVES * 64) {
        const uint32_t u = i / 32, col = i % 32, k = col % 8, l = col / 8;
        v4i v{};
        if (l < 3 && k < m) v = ((const v4i *)(qlev + (uint64_t)pair_q[p0 + pc + k] * qstride))[3 * u + l];
        bq[u / 2][u % 2][col] = v;
    }
    if (tid < m) {
        const uint32_t q = pair_q[p0 + pc + tid];
        const QLevelTail *t = (const QLevelTail *)(qlev + (uint64_t)q * qstride + (uint64_t)UNITS * 48);
        for (int l = 0; l < 3; ++l) {
            qs[tid][l] = t->s[l];
            qc[tid][l] = BITS == 4 ? 8 * t->sum[l] : 0;
        }
        qid[tid] = q;
        qbase[tid] = pair_base[p0 + pc + tid];
    }
    __syncthreads();
    const uint32_t wave = tid >> 6, lane = tid & 63, c = lane & 31, h = lane >> 5;
    const uint32_t tiles = (nrows + 31) / 32;
    for (uint32_t t = wave; t < tiles; t += IVF_LM_WAVES) {
        const uint32_t ri = t * 32 + c;
        const uint64_t row = list_rows[r0 + (ri < nrows ? ri : nrows - 1)];  // past the end: a valid row, dropped
        v4i A[S];
        if constexpr (BITS == 8) {
            // every load of the tile is issued before the first MFMA (left to
            // itself the compiler places each load next to its MFMA and the
            // wave waits on memory once per K step)
#pragma unroll
            for (int st = 0; st < S; ++st) A[st] = ((const v4i *)(codes + row * W))[2 * st + h];
            __builtin_amdgcn_sched_barrier(0);
        } else {
            uint2 raw[S];
#pragma unroll
            for (int st = 0; st < S; ++st) raw[st] = ((const uint2 *)(codes + row * W))[2 * st + h];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int st = 0; st < S; ++st) A[st] = unpack_q4(raw[st]);
        }
        v16i acc = v16i{};
#pragma unroll
        for (int st = 0; st < S; ++st) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[st], bq[st][h][c], acc, 0, 0, 0);
        if (c < 24) {
#pragma unroll
            for (int r = 0; r < 16; ++r) stg[wave][8 * (r >> 2) + 4 * h + (r & 3)][c] = acc[r];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t p = lane + 64 * j, rr = p % 32, k = p / 32;
            const uint32_t i = t * 32 + rr;
            if (k < m && i < nrows) {
                const uint32_t rw = list_rows[r0 + i];
                const float sc = scales[rw] * scale_mul;
                cand[(uint64_t)qid[k] * cap + qbase[k] + i] =
                    q_key(qs[k][0], qs[k][1], qs[k][2], dq<BITS>(stg[wave][rr][k], qc[k][0]),
                          dq<BITS>(stg[wave][rr][8 + k], qc[k][1]), dq<BITS>(stg[wave][rr][16 + k], qc[k][2]), sc,
                          rw);
            }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
}
}  // namespace

hipError_t launch_ivf_pairs(const uint32_t *probes, uint32_t nq, uint32_t nprobe, const uint32_t *list_off,
                            uint32_t *base, uint32_t *cnt, uint32_t *pair_count, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    hipLaunchKernelGGL(ivf_pair_bases, dim3((nq + 255) / 256), dim3(256), 0, s, probes, nq, nprobe, list_off, base, cnt,
                       pair_count);
    return hipGetLastError();
}

hipError_t launch_ivf_pair_scatter(const uint32_t *probes, const uint32_t *base, uint32_t npairs, uint32_t nprobe,
                                   const uint32_t *pair_off, uint32_t *fill, uint32_t *pair_q, uint32_t *pair_base,
                                   hipStream_t s) {
    if (npairs == 0) return hipSuccess;
    hipLaunchKernelGGL(ivf_pair_scatter, dim3((npairs + 255) / 256), dim3(256), 0, s, probes, base, npairs, nprobe,
                       pair_off, fill, pair_q, pair_base);
    return hipGetLastError();
}

hipError_t launch_ivf_chunk_counts(const uint32_t *pair_count, uint32_t nlist, uint32_t *chunks, hipStream_t s) {
    if (nlist == 0) return hipSuccess;
    hipLaunchKernelGGL(ivf_chunk_counts, dim3((nlist + 255) / 256), dim3(256), 0, s, pair_count, nlist, chunks);
    return hipGetLastError();
}

hipError_t launch_ivf_list_scan(const uint32_t *codes, uint32_t W, uint32_t bits, const float *scales,
                                float scale_mul, const uint32_t *list_off, const uint32_t *list_rows, uint32_t nlist,
                                const uint32_t *chunk_off, uint32_t npairs, const uint32_t *pair_off,
                                const uint32_t *pair_count, const uint32_t *pair_q, const uint32_t *pair_base,
                                const unsigned char *qlev, uint64_t qstride, uint32_t units16, uint64_t *cand,
                                uint64_t cap, hipStream_t s) {
    if (nlist == 0 || npairs == 0) return hipSuccess;
    if ((bits != 8 && bits != 4) || W != units16 * bits / 2) return hipErrorInvalidValue;
    // work items: at most ceil(npairs / IVF_QC) + nlist (one partial chunk per list)
    const uint64_t items = ((uint64_t)npairs + IVF_QC - 1) / IVF_QC + nlist;
    if (items > 0x7fffffffull) return hipErrorInvalidValue;
#define BV_LS_CASE(U)                                                                                             \
    case U:                                                                                                        \
        if (bits == 8)                                                                                             \
            hipLaunchKernelGGL((ivf_list_mfma<U, 8>), dim3((uint32_t)items), dim3(IVF_LM_WAVES * 64), 0, s, codes, scales, \
                               scale_mul, list_off, list_rows, nlist, chunk_off, pair_off, pair_count, pair_q,    \
                               pair_base, qlev, qstride, cand, cap);                                              \
        else                                                                                                       \
            hipLaunchKernelGGL((ivf_list_mfma<U, 4>), dim3((uint32_t)items), dim3(IVF_LM_WAVES * 64), 0, s, codes, scales, \
                               scale_mul, list_off, list_rows, nlist, chunk_off, pair_off, pair_count, pair_q,    \
                               pair_base, qlev, qstride, cand, cap);                                              \
        break;
    switch (units16) {
        BV_LS_CASE(2)
        BV_LS_CASE(4)
        BV_LS_CASE(8)
        BV_LS_CASE(16)
        BV_LS_CASE(32)
        BV_LS_CASE(64)
    default: return hipErrorInvalidValue;
    }
#undef BV_LS_CASE
    return hipGetLastError();
}

hipError_t launch_mq1_exact(const uint32_t *codes, uint32_t W, const float *scales, const unsigned char *qlev,
                            uint64_t qstride, uint32_t units16, const uint32_t *rows, const uint32_t *kept,
                            uint64_t cap, uint64_t *keys, uint32_t nq, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    if (W != units16 * 4) return hipErrorInvalidValue;
#define BV_EX_CASE(U)                                                                                         \
    case U: hipLaunchKernelGGL(mq1_exact<U>, dim3(nq), dim3(1024), 0, s, codes, scales, qlev, qstride, rows, \
                               kept, cap, keys); break;
    switch (units16) {
        BV_EX_CASE(2)
        BV_EX_CASE(4)
        BV_EX_CASE(8)
        BV_EX_CASE(16)
        BV_EX_CASE(32)
        BV_EX_CASE(64)
    default: return hipErrorInvalidValue;
    }
#undef BV_EX_CASE
    return hipGetLastError();
}

hipError_t launch_mq1_tau_exact(const uint32_t *codes, uint32_t W, const float *scales,
                                const unsigned char *qlev, uint64_t qstride, uint32_t units16,
                                const uint64_t *merged, const uint32_t *merged_n, uint32_t kk, uint64_t nrows,
                                uint64_t *tau, uint32_t nq, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    if (W != units16 * 4) return hipErrorInvalidValue;
#define BV_TE_CASE(U)                                                                                          \
    case U: hipLaunchKernelGGL(mq1_tau_exact<U>, dim3(nq), dim3(1024), 0, s, codes, scales, qlev, qstride, \
                               merged, merged_n, kk, nrows, tau); break;
    switch (units16) {
        BV_TE_CASE(2)
        BV_TE_CASE(4)
        BV_TE_CASE(8)
        BV_TE_CASE(16)
        BV_TE_CASE(32)
        BV_TE_CASE(64)
    default: return hipErrorInvalidValue;
    }
#undef BV_TE_CASE
    return hipGetLastError();
}

hipError_t launch_mq1_scan_bits(const Mq1Args &a, hipStream_t s) {
    if (a.n == 0 || a.nq == 0) return hipSuccess;
    const uint32_t steps = a.units >> 1;
    if ((a.units & 1u) || steps < 4 || steps > 32 || (steps & (steps - 1)) || a.qblocks == 0 || a.groups == 0 ||
        (uint64_t)a.qblocks * MQ1_QB < a.nq || a.W * 2u != a.units || !a.cand ||
        (a.tau && (!a.up_out || !a.cnt || a.capw == 0)) || a.nwg != a.groups || !(a.cn_const >= 0.0f))
        return hipErrorInvalidValue;
    const uint64_t blocks = (uint64_t)a.groups * a.qblocks;
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    const dim3 g((uint32_t)blocks), wg(MQ_WAVES * 64);
    switch (steps) {
    case 4:
        if (a.tau) hipLaunchKernelGGL((mq1_scan_bits<4, true>), g, wg, 0, s, a);
        else hipLaunchKernelGGL((mq1_scan_bits<4, false>), g, wg, 0, s, a);
        break;
    case 8:
        if (a.tau) hipLaunchKernelGGL((mq1_scan_bits<8, true>), g, wg, 0, s, a);
        else hipLaunchKernelGGL((mq1_scan_bits<8, false>), g, wg, 0, s, a);
        break;
    case 16:
        if (a.tau) hipLaunchKernelGGL((mq1_scan_bits<16, true>), g, wg, 0, s, a);
        else hipLaunchKernelGGL((mq1_scan_bits<16, false>), g, wg, 0, s, a);
        break;
    case 32:
        if (a.tau) hipLaunchKernelGGL((mq1_scan_bits<32, true>), g, wg, 0, s, a);
        else hipLaunchKernelGGL((mq1_scan_bits<32, false>), g, wg, 0, s, a);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_ham_exact(const uint32_t *codes, uint32_t W, const uint32_t *qbits, const unsigned char *qlev,
                            uint64_t qstride, uint32_t tail_off, const uint32_t *rows, const uint32_t *kept,
                            uint64_t cap, uint64_t *keys, uint32_t nq, hipStream_t s) {
    if (nq == 0) return hipSuccess;
#define BV_HE_CASE(WW)                                                                                         \
    case WW: hipLaunchKernelGGL(ham_exact<WW>, dim3(nq), dim3(1024), 0, s, codes, qbits, qlev, qstride, tail_off, \
                                rows, kept, cap, keys); break;
    switch (W) {
        BV_HE_CASE(4)
        BV_HE_CASE(8)
        BV_HE_CASE(16)
        BV_HE_CASE(32)
    default: return hipErrorInvalidValue;
    }
#undef BV_HE_CASE
    return hipGetLastError();
}

hipError_t launch_mq1_compact(const uint64_t *bk, const uint32_t *bu, const uint32_t *bc, uint32_t nwg,
                              uint32_t capw, uint64_t cap, uint64_t *lk, uint32_t *uo, uint32_t *cnt, bool append,
                              uint32_t nq, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    if (nwg == 0 || nwg > 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mq1_compact, dim3(nq), dim3(1024), 0, s, bk, bu, bc, nwg, capw, cap, lk, uo, cnt,
                       append ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_mq1_keep(const uint64_t *cand, const uint32_t *up, const uint32_t *cnt, uint64_t cap,
                           const uint64_t *tau, uint32_t *rows, uint32_t *kept, uint32_t nq, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    hipLaunchKernelGGL(mq1_keep, dim3(nq), dim3(1024), 0, s, cand, up, cnt, cap, tau, rows, kept);
    return hipGetLastError();
}

namespace {
// 1-bit codes (bit j of word g = code 32g + j) as int8 +1 / -1 codes (byte
// j of word g = code 4g + j): the int8 dot of two such rows is
// P - 2 * popcount(a ^ b), the Hamming similarity.
__device__ __forceinline__ uint32_t pm_word(uint32_t bits4) {
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) w |= (((bits4 >> j) & 1u) ? 0x01u : 0xffu) << (8 * j);
    return w;
}

__global__ __launch_bounds__(256) void expand_pm(const uint32_t *bits, uint64_t words, uint32_t *out) {
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < words; i += stride) {
        const uint32_t b = bits[i];
        uint4 lo, hi;
        lo.x = pm_word(b), lo.y = pm_word(b >> 4), lo.z = pm_word(b >> 8), lo.w = pm_word(b >> 12);
        hi.x = pm_word(b >> 16), hi.y = pm_word(b >> 20), hi.z = pm_word(b >> 24), hi.w = pm_word(b >> 28);
        ((uint4 *)out)[2 * i] = lo;
        ((uint4 *)out)[2 * i + 1] = hi;
    }
}

// int4 codes as signed bytes, one per code (nibble j of word g -> byte
// 8g + j, value n - 16 (n >> 3)), for the first-level pass of int4 batches;
// and the rows' score multipliers f32(scale * f32(1/7)), as the
// single-query scan forms them.
__global__ __launch_bounds__(256) void expand_q4(const uint32_t *nib, uint64_t words, uint32_t *out) {
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < words; i += stride) {
        const uint32_t w = nib[i];
        uint32_t b[2] = {0, 0};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int32_t n = (int32_t)((w >> (4 * j)) & 0xfu);
            b[j >> 2] |= ((uint32_t)(n - 16 * (n >> 3)) & 0xffu) << (8 * (j & 3));
        }
        ((uint2 *)out)[i] = make_uint2(b[0], b[1]);
    }
}

__global__ __launch_bounds__(256) void scale_mul_f32(const float *src, uint64_t n, float mul, float *dst) {
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) dst[i] = src[i] * mul;
}

// A query's 1-bit code as the batched scan's packed levels: level one the
// +1 / -1 bytes, levels two and three zero, scales (1, 0, 0).
__global__ __launch_bounds__(64) void pm_levels(const uint32_t *qbits, uint32_t P, unsigned char *qlev,
                                                uint64_t stride) {
    const uint32_t q = blockIdx.x, units = P / 16;
    const uint32_t *b = qbits + (uint64_t)q * (P / 32);
    unsigned char *dst = qlev + (uint64_t)q * stride;
    for (uint32_t u = threadIdx.x; u < units; u += 64) {
        const uint32_t half = (b[u >> 1] >> (16 * (u & 1))) & 0xffffu;
        uint4 l1;
        l1.x = pm_word(half), l1.y = pm_word(half >> 4), l1.z = pm_word(half >> 8), l1.w = pm_word(half >> 12);
        uint4 *o = (uint4 *)(dst + (uint64_t)u * 48);
        o[0] = l1;
        o[1] = make_uint4(0, 0, 0, 0);
        o[2] = make_uint4(0, 0, 0, 0);
    }
    if (threadIdx.x == 0) {
        QLevelTail *t = (QLevelTail *)(dst + (uint64_t)units * 48);
        t->s[0] = 1.0;
        t->s[1] = 0.0;
        t->s[2] = 0.0;
        t->sum[0] = t->sum[1] = t->sum[2] = 0;
        t->pad = 0;
    }
}

__global__ __launch_bounds__(256) void fill_f32(float *p, uint64_t n, float v) {
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) p[i] = v;
}
}  // namespace

hipError_t launch_expand_q4(const uint32_t *nib, uint64_t words, uint32_t *out, hipStream_t s) {
    if (words == 0) return hipSuccess;
    const uint64_t blocks = std::min<uint64_t>((words + 255) / 256, 65536);
    hipLaunchKernelGGL(expand_q4, dim3((uint32_t)blocks), dim3(256), 0, s, nib, words, out);
    return hipGetLastError();
}

hipError_t launch_scale_mul(const float *src, uint64_t n, float mul, float *dst, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const uint64_t blocks = std::min<uint64_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(scale_mul_f32, dim3((uint32_t)blocks), dim3(256), 0, s, src, n, mul, dst);
    return hipGetLastError();
}

hipError_t launch_expand_pm(const uint32_t *bits, uint64_t words, uint32_t *out, hipStream_t s) {
    if (words == 0) return hipSuccess;
    uint64_t blocks = (words + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(expand_pm, dim3((uint32_t)blocks), dim3(256), 0, s, bits, words, out);
    return hipGetLastError();
}

hipError_t launch_pm_levels(const uint32_t *qbits, uint32_t nq, uint32_t P, unsigned char *qlev, uint64_t stride,
                            hipStream_t s) {
    if (nq == 0) return hipSuccess;
    if (P % 32 || stride < (uint64_t)P / 16 * 48 + sizeof(QLevelTail)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(pm_levels, dim3(nq), dim3(64), 0, s, qbits, P, qlev, stride);
    return hipGetLastError();
}

hipError_t launch_fill_f32(float *p, uint64_t n, float v, hipStream_t s) {
    if (n == 0) return hipSuccess;
    uint64_t blocks = (n + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(fill_f32, dim3((uint32_t)blocks), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

hipError_t launch_row_code_norms(const uint32_t *codes, uint64_t n, uint32_t W, float *cn, hipStream_t s) {
    if (n == 0) return hipSuccess;
    uint64_t blocks = (n + 3) / 4;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(row_code_norms, dim3((uint32_t)blocks), dim3(256), 0, s, codes, n, W, cn);
    return hipGetLastError();
}

hipError_t launch_mq1_qconst(const unsigned char *qlev, uint64_t qstride, uint32_t units, uint32_t tail_off,
                             uint32_t nq, float *rq, uint32_t *cnt, uint32_t cnt_value, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    hipLaunchKernelGGL(mq1_qconst, dim3(nq), dim3(64), 0, s, qlev, qstride, units, tail_off, rq, cnt, cnt_value);
    return hipGetLastError();
}

hipError_t launch_mq1_qconst_l1(const float *qrot, uint32_t P, const unsigned char *qlev, uint64_t qstride,
                                uint32_t tail_off, uint32_t nq, float *rq, uint32_t *cnt, uint32_t cnt_value,
                                hipStream_t s) {
    if (nq == 0) return hipSuccess;
    hipLaunchKernelGGL(mq1_qconst_l1, dim3(nq), dim3(64), 0, s, qrot, P, qlev, qstride, tail_off, rq, cnt, cnt_value);
    return hipGetLastError();
}

hipError_t launch_mq1_scan(const Mq1Args &a, hipStream_t s) {
    if (a.n == 0 || a.nq == 0) return hipSuccess;
    const uint32_t steps = a.units >> 1;
    if ((a.units & 1u) || steps == 0 || steps > MQ_MAX_STEPS || (steps & (steps - 1)) || a.qblocks == 0 ||
        a.groups == 0 || (uint64_t)a.qblocks * MQ1_QB < a.nq || a.W * 2u != a.units * 8u ||
        !a.cand || (a.tau && (!a.up_out || !a.cnt || a.capw == 0)) || a.nwg != a.groups)
        return hipErrorInvalidValue;
    const uint64_t blocks = (uint64_t)a.groups * a.qblocks;
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    const dim3 g((uint32_t)blocks), wg(MQ_WAVES * 64);
#define BV_MQ1_CASE(ST)                                                      \
    case ST:                                                                 \
        if (a.tau) hipLaunchKernelGGL((mq1_scan<ST, true>), g, wg, 0, s, a);  \
        else hipLaunchKernelGGL((mq1_scan<ST, false>), g, wg, 0, s, a);       \
        break;
    switch (steps) {
        BV_MQ1_CASE(1)
        BV_MQ1_CASE(2)
        BV_MQ1_CASE(4)
        BV_MQ1_CASE(8)
        BV_MQ1_CASE(16)
        BV_MQ1_CASE(32)
    default: return hipErrorInvalidValue;
    }
#undef BV_MQ1_CASE
    return hipGetLastError();
}

hipError_t launch_row_sqnorms(const float *rows, uint64_t n, uint32_t dim, float *rsq, uint32_t *max_bits,
                              hipStream_t s) {
    if (n == 0) return hipSuccess;
    uint64_t blocks = (n + 3) / 4;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(row_sqnorms, dim3((uint32_t)blocks), dim3(256), 0, s, rows, n, dim, rsq, max_bits);
    return hipGetLastError();
}

hipError_t launch_mq_f32_qconst(const float *q, uint32_t nq, uint32_t dim, const uint32_t *max_bits, int l2,
                                float *qsq, float *slack, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    hipLaunchKernelGGL(mq_f32_qconst, dim3(nq), dim3(64), 0, s, q, dim, max_bits, l2, qsq, slack);
    return hipGetLastError();
}

hipError_t launch_mq_scan(const MqArgs &a, hipStream_t s) {
    if (a.n == 0 || a.nq == 0) return hipSuccess;
    const uint32_t steps = a.units >> 1;
    if ((a.units & 1u) || steps == 0 || steps > MQ_MAX_STEPS || (steps & (steps - 1)) || a.qblocks == 0 ||
        a.groups == 0 || (uint64_t)a.qblocks * MQ_QB < a.nq || (a.bits != 8 && a.bits != 4) ||
        a.W * 32u != a.units * 16u * (uint32_t)a.bits)
        return hipErrorInvalidValue;
    const uint64_t blocks = 8ull * a.groups * a.qblocks;
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    const dim3 g((uint32_t)blocks), wg(MQ_WAVES * 64);
#define BV_MQ_CASE(ST)                                                                              \
    case ST:                                                                                        \
        if (a.bits == 8) hipLaunchKernelGGL((mq_scan<ST, 8>), g, wg, 0, s, a);                      \
        else hipLaunchKernelGGL((mq_scan<ST, 4>), g, wg, 0, s, a);                                  \
        break;
    switch (steps) {
        BV_MQ_CASE(1)
        BV_MQ_CASE(2)
        BV_MQ_CASE(4)
        BV_MQ_CASE(8)
        BV_MQ_CASE(16)
        BV_MQ_CASE(32)
    default: return hipErrorInvalidValue;
    }
#undef BV_MQ_CASE
    return hipGetLastError();
}

bool mq_f32_supported(uint32_t dim) {
    switch (dim) {
    case 32: case 64: case 96: case 128: case 192: case 256: case 384: case 512: case 768: case 1024: return true;
    default: return false;
    }
}

hipError_t launch_mq_scan_f32(const MqArgs &a, hipStream_t s) {
    if (a.n == 0 || a.nq == 0) return hipSuccess;
    if (!mq_f32_supported(a.W) || a.units * 8 != a.W || a.qblocks == 0 || a.groups == 0 ||
        (uint64_t)a.qblocks * MQ_QB < a.nq)
        return hipErrorInvalidValue;
    const uint64_t blocks = 8ull * a.groups * a.qblocks;
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    const dim3 g((uint32_t)blocks), wg(MQ_WAVES * 64);
    switch (a.units) {
    case 4: hipLaunchKernelGGL(mq_scan_f32<4>, g, wg, 0, s, a); break;
    case 8: hipLaunchKernelGGL(mq_scan_f32<8>, g, wg, 0, s, a); break;
    case 12: hipLaunchKernelGGL(mq_scan_f32<12>, g, wg, 0, s, a); break;
    case 16: hipLaunchKernelGGL(mq_scan_f32<16>, g, wg, 0, s, a); break;
    case 24: hipLaunchKernelGGL(mq_scan_f32<24>, g, wg, 0, s, a); break;
    case 32: hipLaunchKernelGGL(mq_scan_f32<32>, g, wg, 0, s, a); break;
    case 48: hipLaunchKernelGGL(mq_scan_f32<48>, g, wg, 0, s, a); break;
    case 64: hipLaunchKernelGGL(mq_scan_f32<64>, g, wg, 0, s, a); break;
    case 96: hipLaunchKernelGGL(mq_scan_f32<96>, g, wg, 0, s, a); break;
    case 128: hipLaunchKernelGGL(mq_scan_f32<128>, g, wg, 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_mq_select(const MqSelArgs &a, uint32_t nq, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    if (a.kk == 0 || a.kk > (uint32_t)MAX_KPRIME) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mq_select, dim3(nq), dim3(SEL_THREADS), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_mq_rerank(const MqRerankArgs &a, uint32_t nq, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    if (a.kprime == 0 || a.kprime > (uint32_t)MAX_KPRIME || a.dim == 0 || (size_t)a.dim * 4 > 96 * 1024)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(mq_rerank, dim3(nq), dim3(RR_THREADS), (size_t)a.dim * 4, s, a);
    return hipGetLastError();
}

}  // namespace bvk
