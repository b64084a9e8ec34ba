/*
 * bv_oracle.c -- CPU restatement of BrowserVec's search-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this file.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker / the CPU baseline.
 *
 * Every function names the reference file:line whose behaviour it restates.
 * The reference is TypeScript: JS numbers are IEEE f64 and a Float32Array
 * store rounds f64 -> f32 (round-to-nearest-even).  For f32 operands, f64
 * + - * / followed by that store equals the correctly rounded f32 operation,
 * so those steps are written as plain C float arithmetic.  Steps the
 * reference keeps in f64 (quantize, normalize, re-rank, probe scores) are
 * written in double.  Build with -ffp-contract=off so nothing is fused.
 *
 * Parity pins (which check holds each function) are listed in the header of
 * oracle/oracle.py; a function with no pin is marked "parity unpinned" there.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>
#include <xmmintrin.h>

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* JS numeric helpers                                                        */
/* ------------------------------------------------------------------------ */

/* ECMAScript ToInt32 (used by `|`, `&`, `<<`, `>>>`). */
static int32_t js_toint32(double x) {
    if (!isfinite(x) || x == 0.0) return 0;
    double t = trunc(x);
    double m = fmod(t, 4294967296.0);
    if (m < 0) m += 4294967296.0;
    uint32_t u = (uint32_t)m;
    return (int32_t)u;
}

/* Math.round: nearest integer, ties toward +infinity. */
static double js_round(double y) {
    if (!isfinite(y)) return y;
    double r = floor(y);
    if (y - r >= 0.5) r += 1.0;
    return r;
}

/* ------------------------------------------------------------------------ */
/* a1. mulberry32 / randomSigns  (src/quant/prng.ts:5-14, 17-22)             */
/* ------------------------------------------------------------------------ */

/* One step of mulberry32 on state `*a`; returns the u32 whose /2^32 is the
 * JS draw.  All operations are mod 2^32, matching Math.imul / |0 / >>>. */
EXPORT uint32_t bvo_mulberry32_next(uint32_t *a) {
    uint32_t s = *a + 0x6d2b79f5u;
    *a = s;
    uint32_t t = (s ^ (s >> 15)) * (1u | s);
    t = (t + (t ^ (t >> 7)) * (61u | t)) ^ t;
    return t ^ (t >> 14);
}

EXPORT double bvo_mulberry32_draw(uint32_t *a) {
    return (double)bvo_mulberry32_next(a) / 4294967296.0;
}

/* Fill `out` with n successive draws of mulberry32(seed) as f64. */
EXPORT void bvo_mulberry32_stream(uint32_t seed, uint64_t n, double *out) {
    uint32_t a = seed;
    for (uint64_t i = 0; i < n; i++) out[i] = bvo_mulberry32_draw(&a);
}

/* randomSigns: rng() < 0.5 ? -1 : 1 */
EXPORT void bvo_random_signs(uint32_t n, uint32_t seed, float *out) {
    uint32_t a = seed;
    for (uint32_t i = 0; i < n; i++) out[i] = bvo_mulberry32_draw(&a) < 0.5 ? -1.0f : 1.0f;
}

/* ------------------------------------------------------------------------ */
/* a2. padToPow2 / fwht / Rotator  (src/quant/rotator.ts:17-21,24-36,38-78)  */
/* ------------------------------------------------------------------------ */

EXPORT uint32_t bvo_pad_to_pow2(uint32_t n) {
    uint32_t p = 4;
    while (p < n) p <<= 1;
    return p;
}

/* In-place radix-2 FWHT, stages len = 1, 2, 4, ... (rotator.ts:24-36). */
EXPORT void bvo_fwht(float *a, uint32_t n) {
    for (uint32_t len = 1; len < n; len <<= 1)
        for (uint32_t i = 0; i < n; i += len << 1)
            for (uint32_t j = i; j < i + len; j++) {
                float x = a[j], y = a[j + len];
                a[j] = x + y;
                a[j + len] = x - y;
            }
}

/* Round r's sign seed: (seed ^ (0x9e3779b9 * (r + 1))) >>> 0 (rotator.ts:54).
 * The product is an exact f64 integer below 2^53 for any realistic round
 * count, so ToInt32 keeps its low 32 bits. */
EXPORT uint32_t bvo_round_seed(uint32_t seed, uint32_t r) {
    uint64_t prod = 0x9e3779b9ull * (uint64_t)(r + 1u);
    return seed ^ (uint32_t)prod;
}

/* signs[r*P + i] = f32(sign * (1 / sqrt(P)))  (rotator.ts:50-57). */
EXPORT void bvo_rotator_signs(uint32_t dim, uint32_t seed, uint32_t rounds, float *signs) {
    uint32_t P = bvo_pad_to_pow2(dim);
    double inv_scale = 1.0 / sqrt((double)P);
    for (uint32_t r = 0; r < rounds; r++) {
        float *s = signs + (size_t)r * P;
        bvo_random_signs(P, bvo_round_seed(seed, r), s);
        for (uint32_t i = 0; i < P; i++) s[i] = (float)((double)s[i] * inv_scale);
    }
}

/* rotateInto: copy, zero-pad, then per round sign-multiply + FWHT
 * (rotator.ts:61-70). dst has P entries. */
EXPORT void bvo_rotate(const float *src, uint32_t dim, const float *signs, uint32_t rounds, float *dst) {
    uint32_t P = bvo_pad_to_pow2(dim);
    memcpy(dst, src, sizeof(float) * dim);
    for (uint32_t i = dim; i < P; i++) dst[i] = 0.0f;
    for (uint32_t r = 0; r < rounds; r++) {
        const float *s = signs + (size_t)r * P;
        for (uint32_t i = 0; i < P; i++) dst[i] = dst[i] * s[i];
        bvo_fwht(dst, P);
    }
}

/* ------------------------------------------------------------------------ */
/* a3. codecs  (src/quant/codec.ts:22-54, 77-108, 136-154; dequant 57-68,    */
/*     111-122, 157-167)                                                     */
/* ------------------------------------------------------------------------ */

static int32_t snorm_code(double v, double levels) {
    /* clamp to [-1,1] (NaN passes through, as in JS), Math.round(c*levels),
     * clamp to +-levels, then ToInt32 for the final `& mask`. */
    double c = v < -1.0 ? -1.0 : (v > 1.0 ? 1.0 : v);
    double b = js_round(c * levels);
    if (b < -levels) b = -levels;
    if (b > levels) b = levels;
    return js_toint32(b);
}

static double max_abs_js(const float *x, uint32_t n) {
    double m = 0.0;
    for (uint32_t i = 0; i < n; i++) {
        double a = fabs((double)x[i]);
        if (a > m) m = a; /* NaN compares false, as `a > maxAbs` in JS */
    }
    return m;
}

/* Returns the f32 scale; words has n/4 entries. Returns -1 on bad length. */
EXPORT float bvo_quantize_row8(const float *x, uint32_t n, uint32_t *words) {
    if (n % 4 != 0) return -1.0f;
    double maxabs = max_abs_js(x, n);
    double scale = maxabs > 0 ? maxabs : 1.0;
    double inv = 1.0 / scale;
    for (uint32_t g = 0; g < n / 4; g++) {
        uint32_t w = 0;
        for (uint32_t j = 0; j < 4; j++) {
            uint32_t b = (uint32_t)snorm_code((double)x[4 * g + j] * inv, 127.0) & 0xffu;
            w |= b << (8 * j);
        }
        words[g] = w;
    }
    return (float)scale;
}

EXPORT float bvo_quantize_row4(const float *x, uint32_t n, uint32_t *words) {
    if (n % 8 != 0) return -1.0f;
    double maxabs = max_abs_js(x, n);
    double scale = maxabs > 0 ? maxabs : 1.0;
    double inv = 1.0 / scale;
    for (uint32_t g = 0; g < n / 8; g++) {
        uint32_t w = 0;
        for (uint32_t j = 0; j < 8; j++) {
            uint32_t b = (uint32_t)snorm_code((double)x[8 * g + j] * inv, 7.0) & 0xfu;
            w |= b << (4 * j);
        }
        words[g] = w;
    }
    return (float)scale;
}

EXPORT float bvo_quantize_row1(const float *x, uint32_t n, uint32_t *words) {
    if (n % 32 != 0) return -1.0f;
    double abs_sum = 0.0;
    for (uint32_t i = 0; i < n; i++) abs_sum += fabs((double)x[i]); /* sequential f64 */
    double scale = abs_sum > 0 ? abs_sum / (double)n : 1.0;
    for (uint32_t g = 0; g < n / 32; g++) {
        uint32_t w = 0;
        for (uint32_t j = 0; j < 32; j++)
            if (x[32 * g + j] >= 0.0f) w |= 1u << j;
        words[g] = w;
    }
    return (float)scale;
}

EXPORT void bvo_dequant_row8(const uint32_t *words, uint32_t nwords, float scale, float *out) {
    for (uint32_t g = 0; g < nwords; g++)
        for (uint32_t j = 0; j < 4; j++) {
            int32_t b = (int32_t)((words[g] >> (8 * j)) & 0xffu);
            if (b > 127) b -= 256;
            double v = (double)b / 127.0;
            if (v < -1.0) v = -1.0;
            out[4 * g + j] = (float)(v * (double)scale);
        }
}

EXPORT void bvo_dequant_row4(const uint32_t *words, uint32_t nwords, float scale, float *out) {
    for (uint32_t g = 0; g < nwords; g++)
        for (uint32_t j = 0; j < 8; j++) {
            int32_t b = (int32_t)((words[g] >> (4 * j)) & 0xfu);
            if (b > 7) b -= 16;
            double v = (double)b / 7.0;
            if (v < -1.0) v = -1.0;
            out[8 * g + j] = (float)(v * (double)scale);
        }
}

EXPORT void bvo_dequant_row1(const uint32_t *words, uint32_t nwords, float scale, float *out) {
    for (uint32_t g = 0; g < nwords; g++)
        for (uint32_t j = 0; j < 32; j++)
            out[32 * g + j] = (float)((((words[g] >> j) & 1u) ? 1.0 : -1.0) * (double)scale);
}

/* a4. BatchEncoder.encode (src/quant/encode.ts:54-78): rotate then quantize
 * each row in order.  bits 8/4/1.  rotated (count*P) may be NULL. */
EXPORT int bvo_encode(const float *data, uint64_t count, uint32_t dim, uint32_t seed, uint32_t rounds,
                      uint32_t bits, uint32_t *words, float *scales, float *rotated) {
    uint32_t P = bvo_pad_to_pow2(dim);
    uint32_t per = bits == 8 ? 4 : bits == 4 ? 8 : bits == 1 ? 32 : 0;
    if (!per) return -1;
    uint32_t wpr = P / per;
    float *signs = (float *)malloc(sizeof(float) * (size_t)P * (rounds ? rounds : 1));
    float *scratch = (float *)malloc(sizeof(float) * P);
    bvo_rotator_signs(dim, seed, rounds, signs);
    for (uint64_t i = 0; i < count; i++) {
        float *dst = rotated ? rotated + i * P : scratch;
        bvo_rotate(data + i * dim, dim, signs, rounds, dst);
        uint32_t *w = words + i * wpr;
        scales[i] = bits == 8 ? bvo_quantize_row8(dst, P, w)
                  : bits == 4 ? bvo_quantize_row4(dst, P, w)
                              : bvo_quantize_row1(dst, P, w);
    }
    free(signs);
    free(scratch);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* a5 / a14. Store arithmetic (src/store/store.ts:114-160, 209-217)          */
/* ------------------------------------------------------------------------ */

/* normalizeInPlace: f64 sequential sum of squares, inv = 1/sqrt, f32 store. */
EXPORT void bvo_normalize(float *v, uint32_t n) {
    double sum = 0.0;
    for (uint32_t i = 0; i < n; i++) sum += (double)v[i] * (double)v[i];
    double norm = sqrt(sum);
    if (norm > 0) {
        double inv = 1.0 / norm;
        for (uint32_t i = 0; i < n; i++) v[i] = (float)((double)v[i] * inv);
    }
}

EXPORT void bvo_normalize_many(float *v, uint64_t rows, uint32_t n) {
    for (uint64_t r = 0; r < rows; r++) bvo_normalize(v + r * n, n);
}

/* dotRow: four strided f64 accumulators, ((a0+a1)+a2)+a3, sequential tail. */
EXPORT double bvo_dot_row(const float *row, const float *q, uint32_t dim) {
    uint32_t vec = dim & ~3u;
    double a0 = 0, a1 = 0, a2 = 0, a3 = 0;
    uint32_t i = 0;
    for (; i < vec; i += 4) {
        a0 += (double)row[i] * (double)q[i];
        a1 += (double)row[i + 1] * (double)q[i + 1];
        a2 += (double)row[i + 2] * (double)q[i + 2];
        a3 += (double)row[i + 3] * (double)q[i + 3];
    }
    double acc = a0 + a1 + a2 + a3;
    for (; i < dim; i++) acc += (double)row[i] * (double)q[i];
    return acc;
}

/* l2Row: negative squared distance, same accumulator layout. */
EXPORT double bvo_l2_row(const float *row, const float *q, uint32_t dim) {
    uint32_t vec = dim & ~3u;
    double a0 = 0, a1 = 0, a2 = 0, a3 = 0;
    uint32_t i = 0;
    for (; i < vec; i += 4) {
        double d0 = (double)row[i] - (double)q[i];
        double d1 = (double)row[i + 1] - (double)q[i + 1];
        double d2 = (double)row[i + 2] - (double)q[i + 2];
        double d3 = (double)row[i + 3] - (double)q[i + 3];
        a0 += d0 * d0;
        a1 += d1 * d1;
        a2 += d2 * d2;
        a3 += d3 * d3;
    }
    double acc = a0 + a1 + a2 + a3;
    for (; i < dim; i++) {
        double d = (double)row[i] - (double)q[i];
        acc += d * d;
    }
    return -acc;
}

/* rerankExact's scoring half (src/index.ts:583-594): f32(dotRow) for each
 * candidate row. */
EXPORT void bvo_rerank_scores(const float *rows, uint32_t dim, const float *q, const uint32_t *cand,
                              uint32_t n, float *out) {
    for (uint32_t c = 0; c < n; c++) out[c] = (float)bvo_dot_row(rows + (size_t)cand[c] * dim, q, dim);
}

/* ------------------------------------------------------------------------ */
/* a6-a9. Scan scores in the reference kernels' order                        */
/* (src/engine/wgsl/distance.ts:24-44,147-191; distanceQ8.ts:56-66;        */
/*  distanceQ4.ts:44-62; distanceQ1.ts:44-67).                           */
/* WGSL leaves the rounding inside dot() implementation-defined; this        */
/* restatement fixes it as ((a0*b0 + a1*b1) + a2*b2) + a3*b3 with separate    */
/* roundings, and accumulates acc = dot + acc in group order.                */
/* ------------------------------------------------------------------------ */

static inline float dot4(float a0, float a1, float a2, float a3, const float *b) {
    float p0 = a0 * b[0], p1 = a1 * b[1], p2 = a2 * b[2], p3 = a3 * b[3];
    return ((p0 + p1) + p2) + p3;
}

/* metric: 0 cosine/dot, 2 l2 (negated). */
EXPORT void bvo_scan_f32(const float *corpus, uint64_t rows, uint32_t dim, const float *q, uint32_t metric,
                         float *out) {
    uint32_t vec = dim / 4, tail = dim % 4;
    for (uint64_t r = 0; r < rows; r++) {
        const float *c = corpus + r * dim;
        float acc = 0.0f;
        for (uint32_t g = 0; g < vec; g++) {
            const float *cg = c + 4 * g, *qg = q + 4 * g;
            if (metric == 2) {
                float d[4] = {cg[0] - qg[0], cg[1] - qg[1], cg[2] - qg[2], cg[3] - qg[3]};
                acc = dot4(d[0], d[1], d[2], d[3], d) + acc;
            } else {
                acc = dot4(cg[0], cg[1], cg[2], cg[3], qg) + acc;
            }
        }
        for (uint32_t j = 0; j < tail; j++) {
            uint32_t i = vec * 4 + j;
            if (metric == 2) {
                float d = c[i] - q[i];
                acc = d * d + acc;
            } else {
                acc = c[i] * q[i] + acc;
            }
        }
        out[r] = metric == 2 ? -acc : acc;
    }
}

static inline float unpack_snorm8(uint32_t w, uint32_t j) {
    int32_t b = (int32_t)((w >> (8 * j)) & 0xffu);
    if (b > 127) b -= 256;
    float v = (float)b / 127.0f;
    return v < -1.0f ? -1.0f : v;
}

/* int8 asymmetric scan; q is the rotated query (P floats). cand may be NULL
 * (flat) or list `rows` row ids (indexed mode, distanceQ8.ts:17-40,79-84). */
EXPORT void bvo_scan_q8(const uint32_t *codes, const float *scales, uint64_t rows, uint32_t P, const float *q,
                        const uint32_t *cand, float *out) {
    uint32_t W = P / 4;
    for (uint64_t i = 0; i < rows; i++) {
        uint64_t r = cand ? cand[i] : i;
        const uint32_t *w = codes + r * W;
        float acc = 0.0f;
        for (uint32_t g = 0; g < W; g++)
            acc = dot4(unpack_snorm8(w[g], 0), unpack_snorm8(w[g], 1), unpack_snorm8(w[g], 2),
                       unpack_snorm8(w[g], 3), q + 4 * g) + acc;
        out[i] = acc * scales[r];
    }
}

static inline float nib4(uint32_t w, uint32_t shift) {
    int32_t n = (int32_t)((w >> shift) & 0xfu);
    return (float)(n - 16 * (n >> 3));
}

EXPORT void bvo_scan_q4(const uint32_t *codes, const float *scales, uint64_t rows, uint32_t P, const float *q,
                        const uint32_t *cand, float *out) {
    uint32_t W = P / 8;
    const float inv7 = 1.0f / 7.0f;
    for (uint64_t i = 0; i < rows; i++) {
        uint64_t r = cand ? cand[i] : i;
        const uint32_t *w = codes + r * W;
        float acc = 0.0f;
        for (uint32_t g = 0; g < W; g++) {
            float d0 = dot4(nib4(w[g], 0), nib4(w[g], 4), nib4(w[g], 8), nib4(w[g], 12), q + 8 * g);
            float d1 = dot4(nib4(w[g], 16), nib4(w[g], 20), nib4(w[g], 24), nib4(w[g], 28), q + 8 * g + 4);
            acc = (d0 + d1) + acc;
        }
        out[i] = acc * (scales[r] * inv7);
    }
}

EXPORT void bvo_scan_q1(const uint32_t *codes, const float *scales, uint64_t rows, uint32_t P, const float *q,
                        const uint32_t *cand, float *out) {
    uint32_t W = P / 32;
    for (uint64_t i = 0; i < rows; i++) {
        uint64_t r = cand ? cand[i] : i;
        const uint32_t *w = codes + r * W;
        float acc = 0.0f;
        for (uint32_t g = 0; g < W; g++)
            for (uint32_t s = 0; s < 8; s++) {
                float v[4];
                for (uint32_t j = 0; j < 4; j++) v[j] = ((w[g] >> (4 * s + j)) & 1u) ? 1.0f : -1.0f;
                acc = dot4(v[0], v[1], v[2], v[3], q + 32 * g + 4 * s) + acc;
            }
        out[i] = acc * scales[r];
    }
}

/* Sign bits of a rotated query with quantizeRow1's rule (x >= 0 sets the
 * bit, codec.ts:149).  This is the query side of the Hamming scorer, which
 * has no reference counterpart. */
EXPORT void bvo_query_bits(const float *q, uint32_t P, uint32_t *bits) {
    for (uint32_t g = 0; g < P / 32; g++) {
        uint32_t w = 0;
        for (uint32_t j = 0; j < 32; j++)
            if (q[32 * g + j] >= 0.0f) w |= 1u << j;
        bits[g] = w;
    }
}

/* Hamming similarity P - 2*popcount(c ^ q): integer, exact. */
EXPORT void bvo_scan_hamming(const uint32_t *codes, uint64_t rows, uint32_t P, const uint32_t *qbits,
                             const uint32_t *cand, int32_t *out) {
    uint32_t W = P / 32;
    for (uint64_t i = 0; i < rows; i++) {
        uint64_t r = cand ? cand[i] : i;
        int32_t pc = 0;
        for (uint32_t g = 0; g < W; g++) pc += __builtin_popcount(codes[r * W + g] ^ qbits[g]);
        out[i] = (int32_t)P - 2 * pc;
    }
}

/* int8 x int8 dot of codes (both quantizeRow output): exact integer. */
EXPORT void bvo_scan_int8sym(const uint32_t *codes, uint64_t rows, uint32_t P, const uint32_t *qcodes,
                             const uint32_t *cand, int32_t *out) {
    uint32_t W = P / 4;
    for (uint64_t i = 0; i < rows; i++) {
        uint64_t r = cand ? cand[i] : i;
        int32_t acc = 0;
        for (uint32_t g = 0; g < W; g++)
            for (uint32_t j = 0; j < 4; j++) {
                int32_t a = (int8_t)((codes[r * W + g] >> (8 * j)) & 0xffu);
                int32_t b = (int8_t)((qcodes[g] >> (8 * j)) & 0xffu);
                acc += a * b;
            }
        out[i] = acc;
    }
}

/* Independent high-precision references (long double) for the closed-form
 * checks: sum_i c_i q_i and sum_i |c_i q_i|. */
EXPORT void bvo_dot_exact(const float *a, const float *b, uint64_t rows, uint32_t n, double *dot, double *mag) {
    for (uint64_t r = 0; r < rows; r++) {
        long double s = 0, m = 0;
        for (uint32_t i = 0; i < n; i++) {
            long double p = (long double)a[r * n + i] * (long double)b[i];
            s += p;
            m += p < 0 ? -p : p;
        }
        dot[r] = (double)s;
        mag[r] = (double)m;
    }
}

/* ------------------------------------------------------------------------ */
/* a19. CPU baseline: lane-exact restatement of kernel.wat dot / l2         */
/* (src/fallback/kernel.wat:6-83): f32x4 mul then add (no FMA), horizontal   */
/* (l0+l1)+(l2+l3), sequential scalar tail, l2 negated.                      */
/* ------------------------------------------------------------------------ */

EXPORT void bvo_wasm_dot(const float *data, const float *q, float *out, uint64_t rows, uint32_t dim) {
    uint32_t tail = dim & ~3u;
    for (uint64_t r = 0; r < rows; r++) {
        const float *base = data + r * dim;
        __m128 acc = _mm_setzero_ps();
        uint32_t i = 0;
        for (; i < tail; i += 4) acc = _mm_add_ps(acc, _mm_mul_ps(_mm_loadu_ps(base + i), _mm_loadu_ps(q + i)));
        float l[4];
        _mm_storeu_ps(l, acc);
        float sum = (l[0] + l[1]) + (l[2] + l[3]);
        for (; i < dim; i++) sum = sum + base[i] * q[i];
        out[r] = sum;
    }
}

EXPORT void bvo_wasm_l2(const float *data, const float *q, float *out, uint64_t rows, uint32_t dim) {
    uint32_t tail = dim & ~3u;
    for (uint64_t r = 0; r < rows; r++) {
        const float *base = data + r * dim;
        __m128 acc = _mm_setzero_ps();
        uint32_t i = 0;
        for (; i < tail; i += 4) {
            __m128 d = _mm_sub_ps(_mm_loadu_ps(base + i), _mm_loadu_ps(q + i));
            acc = _mm_add_ps(acc, _mm_mul_ps(d, d));
        }
        float l[4];
        _mm_storeu_ps(l, acc);
        float sum = (l[0] + l[1]) + (l[2] + l[3]);
        for (; i < dim; i++) {
            float d = base[i] - q[i];
            sum = sum + d * d;
        }
        out[r] = -sum;
    }
}

/* Scalar emulation of the same lane order, used to check the SSE version. */
EXPORT void bvo_wasm_dot_scalar(const float *data, const float *q, float *out, uint64_t rows, uint32_t dim) {
    uint32_t tail = dim & ~3u;
    for (uint64_t r = 0; r < rows; r++) {
        const float *base = data + r * dim;
        float l[4] = {0, 0, 0, 0};
        uint32_t i = 0;
        for (; i < tail; i += 4)
            for (uint32_t j = 0; j < 4; j++) {
                float p = base[i + j] * q[i + j];
                l[j] = l[j] + p;
            }
        float sum = (l[0] + l[1]) + (l[2] + l[3]);
        for (; i < dim; i++) sum = sum + base[i] * q[i];
        out[r] = sum;
    }
}

/* ------------------------------------------------------------------------ */
/* a12 / a13. top-k                                                          */
/* ------------------------------------------------------------------------ */

typedef struct {
    uint32_t row;
    float score;
} hit_t;

/* Stable merge sort with a JS-style comparator sign (a.score - b.score). */
static void stable_sort(hit_t *h, uint32_t n, int descending) {
    if (n < 2) return;
    hit_t *tmp = (hit_t *)malloc(sizeof(hit_t) * n);
    for (uint32_t width = 1; width < n; width <<= 1) {
        for (uint32_t lo = 0; lo < n; lo += 2 * width) {
            uint32_t mid = lo + width < n ? lo + width : n;
            uint32_t hi = lo + 2 * width < n ? lo + 2 * width : n;
            uint32_t i = lo, j = mid, k = lo;
            while (i < mid && j < hi) {
                /* take right only if strictly before left */
                int right_first = descending ? (h[j].score > h[i].score) : (h[j].score < h[i].score);
                tmp[k++] = right_first ? h[j++] : h[i++];
            }
            while (i < mid) tmp[k++] = h[i++];
            while (j < hi) tmp[k++] = h[j++];
        }
        memcpy(h, tmp, sizeof(hit_t) * n);
    }
    free(tmp);
}

/* topK exactly as src/index/flat.ts:217-239 (ref tie semantics). */
EXPORT uint32_t bvo_topk_ref(const float *scores, uint32_t n, uint32_t k, uint32_t *rows, float *out_scores) {
    uint32_t limit = k < n ? k : n;
    if (limit == 0) return 0;
    hit_t *heap = (hit_t *)malloc(sizeof(hit_t) * limit);
    uint32_t len = 0;
    for (uint32_t row = 0; row < n; row++) {
        float s = scores[row];
        if (len < limit) {
            heap[len].row = row;
            heap[len].score = s;
            len++;
            if (len == limit) stable_sort(heap, len, 0);
        } else if (s > heap[0].score) {
            heap[0].row = row;
            heap[0].score = s;
            uint32_t i = 0;
            while (i + 1 < len && heap[i].score > heap[i + 1].score) {
                hit_t t = heap[i];
                heap[i] = heap[i + 1];
                heap[i + 1] = t;
                i++;
            }
        }
    }
    stable_sort(heap, len, 1);
    for (uint32_t i = 0; i < len; i++) {
        rows[i] = heap[i].row;
        out_scores[i] = heap[i].score;
    }
    free(heap);
    return len;
}

/* mergePartials (src/index/gpuTopk.ts:160-189): skips score <= -3.4e38 (f64
 * compare) and row >= n, then the same selection as topK. */
EXPORT uint32_t bvo_merge_partials(const float *scores, const uint32_t *prow, uint32_t count, uint32_t n,
                                   uint32_t k, uint32_t *rows, float *out_scores) {
    uint32_t limit = k < n ? k : n;
    if (limit == 0) return 0;
    hit_t *heap = (hit_t *)malloc(sizeof(hit_t) * limit);
    uint32_t len = 0;
    for (uint32_t i = 0; i < count; i++) {
        float s = scores[i];
        if ((double)s <= -3.4e38) continue;
        uint32_t row = prow[i];
        if (row >= n) continue;
        if (len < limit) {
            heap[len].row = row;
            heap[len].score = s;
            len++;
            if (len == limit) stable_sort(heap, len, 0);
        } else if (s > heap[0].score) {
            heap[0].row = row;
            heap[0].score = s;
            uint32_t j = 0;
            while (j + 1 < len && heap[j].score > heap[j + 1].score) {
                hit_t t = heap[j];
                heap[j] = heap[j + 1];
                heap[j + 1] = t;
                j++;
            }
        }
    }
    stable_sort(heap, len, 1);
    for (uint32_t i = 0; i < len; i++) {
        rows[i] = heap[i].row;
        out_scores[i] = heap[i].score;
    }
    free(heap);
    return len;
}

/* Canonical top-k: order by (score desc, row asc); -0 ranks equal to +0.
 * Entries with score <= `floor` are dropped (pass -INFINITY for none). */
static int canon_cmp(const void *pa, const void *pb) {
    const hit_t *a = (const hit_t *)pa, *b = (const hit_t *)pb;
    if (a->score > b->score) return -1;
    if (a->score < b->score) return 1;
    return a->row < b->row ? -1 : (a->row > b->row ? 1 : 0);
}

EXPORT uint32_t bvo_topk_canonical(const float *scores, const uint32_t *ids, uint32_t n, uint32_t k, float floor_,
                                   uint32_t *rows, float *out_scores) {
    hit_t *h = (hit_t *)malloc(sizeof(hit_t) * (n ? n : 1));
    uint32_t m = 0;
    for (uint32_t i = 0; i < n; i++) {
        if (!(scores[i] > floor_)) continue;
        h[m].row = ids ? ids[i] : i;
        h[m].score = scores[i] + 0.0f;
        m++;
    }
    qsort(h, m, sizeof(hit_t), canon_cmp);
    uint32_t out = k < m ? k : m;
    for (uint32_t i = 0; i < out; i++) {
        rows[i] = h[i].row;
        out_scores[i] = h[i].score;
    }
    free(h);
    return out;
}

/* ------------------------------------------------------------------------ */
/* a16. k-means pieces (src/index/kmeans.ts:154-219)                         */
/* ------------------------------------------------------------------------ */

EXPORT void bvo_normalize_rows(float *m, uint32_t rows, uint32_t dim) {
    for (uint32_t r = 0; r < rows; r++) {
        float *v = m + (size_t)r * dim;
        double s = 0;
        for (uint32_t i = 0; i < dim; i++) s += (double)v[i] * (double)v[i];
        double root = sqrt(s);
        double inv = 1.0 / (root != 0.0 ? root : 1.0); /* `Math.sqrt(s) || 1` */
        for (uint32_t i = 0; i < dim; i++) v[i] = (float)((double)v[i] * inv);
    }
}

EXPORT void bvo_random_init_centroids(const float *sample, uint32_t sample_count, uint32_t nlist, uint32_t dim,
                                      uint32_t seed, float *centroids) {
    uint32_t a = seed;
    for (uint32_t c = 0; c < nlist; c++) {
        uint32_t r = (uint32_t)floor(bvo_mulberry32_draw(&a) * (double)sample_count);
        memcpy(centroids + (size_t)c * dim, sample + (size_t)r * dim, sizeof(float) * dim);
    }
    bvo_normalize_rows(centroids, nlist, dim);
}

/* updateCentroids: f32 sums in row order, c = f32(sum * (1/count)), empty
 * clusters re-seeded with mulberry32(seed) in cluster order, then
 * normalizeRows.  counts_out (nlist) may be NULL. */
EXPORT void bvo_update_centroids(const float *sample, uint32_t sample_count, const uint32_t *assign,
                                 float *centroids, uint32_t nlist, uint32_t dim, uint32_t seed, int32_t *counts_out) {
    float *sums = (float *)calloc((size_t)nlist * dim, sizeof(float));
    int32_t *counts = (int32_t *)calloc(nlist, sizeof(int32_t));
    for (uint32_t r = 0; r < sample_count; r++) {
        uint32_t c = assign[r];
        const float *x = sample + (size_t)r * dim;
        float *s = sums + (size_t)c * dim;
        for (uint32_t i = 0; i < dim; i++) s[i] = s[i] + x[i];
        counts[c]++;
    }
    uint32_t a = seed;
    for (uint32_t c = 0; c < nlist; c++) {
        float *cen = centroids + (size_t)c * dim;
        if (counts[c] == 0) {
            uint32_t r = (uint32_t)floor(bvo_mulberry32_draw(&a) * (double)sample_count);
            memcpy(cen, sample + (size_t)r * dim, sizeof(float) * dim);
        } else {
            double inv = 1.0 / (double)counts[c];
            const float *s = sums + (size_t)c * dim;
            for (uint32_t i = 0; i < dim; i++) cen[i] = (float)((double)s[i] * inv);
        }
    }
    bvo_normalize_rows(centroids, nlist, dim);
    if (counts_out) memcpy(counts_out, counts, sizeof(int32_t) * nlist);
    free(sums);
    free(counts);
}

/* fp32 assignment (src/engine/wgsl/assign.ts:31-58): argmax over centroids
 * with strict '>', so the lowest index wins ties.  order 0 = the reference
 * kernel's dot4-group order; order 1 = one sequential fused multiply-add
 * chain over i (the device kernel's order). */
/* The order-1 assignment (a fused multiply-add chain per (row, centroid) in
 * element order, strict > over centroids in index order) with eight
 * centroids per AVX2 lane group and four groups in flight: every lane runs
 * exactly the scalar fmaf chain, so the result equals the scalar loop's.
 * Used when the host CPU has AVX2 + FMA, to keep the oracle fast at 4096
 * lists x 1024 dimensions. */
__attribute__((target("avx2,fma"))) static void assign_fma_avx2(const float *rows, uint32_t nrows,
                                                                 const float *centroids, uint32_t nlist,
                                                                 uint32_t dim, uint32_t *out) {
    const uint32_t nb = (nlist + 31) / 32 * 4; /* groups of 8, a multiple of 4 */
    float *ct = (float *)aligned_alloc(32, (size_t)nb * dim * 8 * sizeof(float));
    memset(ct, 0, (size_t)nb * dim * 8 * sizeof(float));
    for (uint32_t c = 0; c < nlist; c++)
        for (uint32_t i = 0; i < dim; i++) ct[((size_t)(c / 8) * dim + i) * 8 + c % 8] = centroids[(size_t)c * dim + i];
#pragma omp parallel for schedule(dynamic, 8)
    for (uint32_t r = 0; r < nrows; r++) {
        const float *x = rows + (size_t)r * dim;
        uint32_t best_c = 0;
        float best_s = -3.4e38f;
        for (uint32_t b = 0; b < nb; b += 4) {
            __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps(), a2 = _mm256_setzero_ps(),
                   a3 = _mm256_setzero_ps();
            const float *p0 = ct + (size_t)b * dim * 8, *p1 = p0 + (size_t)dim * 8, *p2 = p1 + (size_t)dim * 8,
                        *p3 = p2 + (size_t)dim * 8;
            for (uint32_t i = 0; i < dim; i++) {
                const __m256 xi = _mm256_set1_ps(x[i]);
                a0 = _mm256_fmadd_ps(xi, _mm256_load_ps(p0 + 8 * i), a0);
                a1 = _mm256_fmadd_ps(xi, _mm256_load_ps(p1 + 8 * i), a1);
                a2 = _mm256_fmadd_ps(xi, _mm256_load_ps(p2 + 8 * i), a2);
                a3 = _mm256_fmadd_ps(xi, _mm256_load_ps(p3 + 8 * i), a3);
            }
            float s[32];
            _mm256_storeu_ps(s, a0);
            _mm256_storeu_ps(s + 8, a1);
            _mm256_storeu_ps(s + 16, a2);
            _mm256_storeu_ps(s + 24, a3);
            for (uint32_t j = 0; j < 32; j++) {
                const uint32_t c = b * 8 + j;
                if (c < nlist && s[j] > best_s) {
                    best_s = s[j];
                    best_c = c;
                }
            }
        }
        out[r] = best_c;
    }
    free(ct);
}

EXPORT void bvo_assign_f32(const float *rows, uint32_t nrows, const float *centroids, uint32_t nlist, uint32_t dim,
                           uint32_t order, uint32_t *out) {
    /* order 2: the order-1 chain on the scalar path regardless of the CPU
     * (lets the tests compare the two paths) */
    if (order == 1 && __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) {
        assign_fma_avx2(rows, nrows, centroids, nlist, dim, out);
        return;
    }
#pragma omp parallel for schedule(dynamic, 8)
    for (uint32_t r = 0; r < nrows; r++) {
        const float *x = rows + (size_t)r * dim;
        uint32_t best_c = 0;
        float best_s = -3.4e38f;
        for (uint32_t c = 0; c < nlist; c++) {
            const float *m = centroids + (size_t)c * dim;
            float acc = 0.0f;
            if (order == 0) {
                for (uint32_t g = 0; g < dim / 4; g++) acc = dot4(x[4 * g], x[4 * g + 1], x[4 * g + 2], x[4 * g + 3], m + 4 * g) + acc;
                for (uint32_t i = dim / 4 * 4; i < dim; i++) acc = x[i] * m[i] + acc;
            } else {
                for (uint32_t i = 0; i < dim; i++) acc = fmaf(x[i], m[i], acc);
            }
            if (acc > best_s) {
                best_s = acc;
                best_c = c;
            }
        }
        out[r] = best_c;
    }
}

/* Quantized assignment (assignQ8.ts:29-65, assignQ4.ts:33-72,
 * assignQ1.ts:33-76) in the reference kernels' order: the scale sits inside
 * the loop for int8/int4, after it for 1-bit. */
EXPORT void bvo_assign_quant(const uint32_t *codes, const float *scales, uint32_t nrows, uint32_t P, uint32_t bits,
                             const float *centroids, uint32_t nlist, uint32_t *out) {
    uint32_t W = bits == 8 ? P / 4 : bits == 4 ? P / 8 : P / 32;
    const float inv7c = 1.0f / 7.0f;
    for (uint32_t r = 0; r < nrows; r++) {
        const uint32_t *w = codes + (size_t)r * W;
        float scale = scales[r];
        uint32_t best_c = 0;
        float best_s = -3.4e38f;
        for (uint32_t c = 0; c < nlist; c++) {
            const float *m = centroids + (size_t)c * P;
            float acc = 0.0f;
            if (bits == 8) {
                for (uint32_t g = 0; g < W; g++) {
                    float v[4];
                    for (uint32_t j = 0; j < 4; j++) v[j] = unpack_snorm8(w[g], j) * scale;
                    acc = dot4(v[0], v[1], v[2], v[3], m + 4 * g) + acc;
                }
            } else if (bits == 4) {
                float inv7 = scale * inv7c;
                for (uint32_t g = 0; g < W; g++) {
                    float v0[4], v1[4];
                    for (uint32_t j = 0; j < 4; j++) {
                        v0[j] = nib4(w[g], 4 * j) * inv7;
                        v1[j] = nib4(w[g], 16 + 4 * j) * inv7;
                    }
                    float d0 = dot4(v0[0], v0[1], v0[2], v0[3], m + 8 * g);
                    float d1 = dot4(v1[0], v1[1], v1[2], v1[3], m + 8 * g + 4);
                    acc = (d0 + d1) + acc;
                }
            } else {
                for (uint32_t g = 0; g < W; g++)
                    for (uint32_t s = 0; s < 8; s++) {
                        float v[4];
                        for (uint32_t j = 0; j < 4; j++) v[j] = ((w[g] >> (4 * s + j)) & 1u) ? 1.0f : -1.0f;
                        acc = dot4(v[0], v[1], v[2], v[3], m + 32 * g + 4 * s) + acc;
                    }
                acc = acc * scale;
            }
            if (acc > best_s) {
                best_s = acc;
                best_c = c;
            }
        }
        out[r] = best_c;
    }
}

/* pickProbes scores (src/index/ivfquant.ts:495-511): f64 four-way strided
 * dot over P, stored f32. */
EXPORT void bvo_probe_scores(const float *centroids, uint32_t nlist, uint32_t P, const float *rq, float *out) {
    for (uint32_t c = 0; c < nlist; c++) {
        const float *m = centroids + (size_t)c * P;
        double a0 = 0, a1 = 0, a2 = 0, a3 = 0;
        for (uint32_t i = 0; i < P; i += 4) {
            a0 += (double)m[i] * (double)rq[i];
            a1 += (double)m[i + 1] * (double)rq[i + 1];
            a2 += (double)m[i + 2] * (double)rq[i + 2];
            a3 += (double)m[i + 3] * (double)rq[i + 3];
        }
        out[c] = (float)(a0 + a1 + a2 + a3);
    }
}

/* Reservoir sampling (src/index/ivfquant.ts:112-124, 235-245).  The caller
 * keeps `state` = {filled, seen, rng}; returns the slot written or -1. */
EXPORT int64_t bvo_reservoir_slot(uint32_t cap, uint64_t *filled, uint64_t *seen, uint32_t *rng) {
    int64_t slot = -1;
    if (*filled < cap) {
        slot = (int64_t)*filled;
        (*filled)++;
    } else {
        uint64_t j = (uint64_t)floor(bvo_mulberry32_draw(rng) * (double)(*seen + 1));
        if (j < cap) slot = (int64_t)j;
    }
    (*seen)++;
    return slot;
}

/* CSR build (ivfquant.ts:297-305): counts, prefix offsets, rows ascending. */
EXPORT void bvo_build_csr(const uint32_t *cluster, uint64_t rows, uint32_t nlist, int32_t *offset, int32_t *list_rows) {
    memset(offset, 0, sizeof(int32_t) * (nlist + 1));
    for (uint64_t r = 0; r < rows; r++) offset[cluster[r] + 1]++;
    for (uint32_t c = 0; c < nlist; c++) offset[c + 1] += offset[c];
    int32_t *cursor = (int32_t *)malloc(sizeof(int32_t) * (nlist ? nlist : 1));
    memcpy(cursor, offset, sizeof(int32_t) * nlist);
    for (uint64_t r = 0; r < rows; r++) list_rows[cursor[cluster[r]]++] = (int32_t)r;
    free(cursor);
}

/* chooseNprobe (src/index/ivfTune.ts:31-42).  Returns nprobe, writes recall. */
EXPORT uint32_t bvo_choose_nprobe(const uint32_t *ranks, uint32_t total, uint32_t nlist, double target,
                                  double *recall) {
    if (total == 0 || nlist <= 1) {
        *recall = 1.0;
        return nlist > 1 ? nlist : 1;
    }
    uint32_t *hist = (uint32_t *)calloc(nlist, sizeof(uint32_t));
    for (uint32_t i = 0; i < total; i++) hist[ranks[i]]++;
    uint32_t cum = 0;
    for (uint32_t p = 1; p <= nlist; p++) {
        cum += hist[p - 1];
        if ((double)cum / (double)total >= target) {
            *recall = (double)cum / (double)total;
            free(hist);
            return p;
        }
    }
    free(hist);
    *recall = 1.0;
    return nlist;
}

/* pickTuneQueries (ivfTune.ts:49-54). Returns count written. */
EXPORT uint32_t bvo_pick_tune_queries(uint32_t filled, uint32_t want, uint32_t *out) {
    uint32_t n = filled < want ? filled : want;
    for (uint32_t i = 0; i < n; i++) out[i] = (uint32_t)floor(((double)i * (double)filled) / (double)n);
    return n;
}

/* ------------------------------------------------------------------------ */
/* f4. Graph beam search over a flat fixed-degree adjacency                  */
/* (src/engine/wgsl/graphSearch.ts:62-259) and the searcher's seeds, dedup   */
/* and top-k (src/index/hnswGpu.ts:134-206).  Where the shader lets lanes    */
/* race (the visited-set inserts of one staged batch) they are taken in lane */
/* order; its reductions are restated in its own order: each lane keeps the  */
/* first strict best of slots t, t+WG, ..., then a halving tree with strict  */
/* compares.  Distances are f32, element order, multiply and add each        */
/* rounded (the shader's `acc = acc + c * q`; WGSL leaves fusing to the      */
/* compiler -- parity unpinned against a fusing backend).                    */
/* ------------------------------------------------------------------------ */
#define G_EF 256u
#define G_WG 64u
#define G_HASH 2048u
#define G_PROBES 16u
#define G_INF 3.4e38f
#define G_EMPTY 0xffffffffu

static float g_dist(const float *row, const float *q, uint32_t dim, int l2) {
    float acc = 0.0f;
    for (uint32_t i = 0; i < dim; i++) {
        if (l2) {
            const float d = row[i] - q[i];
            acc = acc + d * d;
        } else {
            acc = acc + row[i] * q[i];
        }
    }
    return l2 ? acc : -acc;
}

/* markVisited (graphSearch.ts:112-128): 1 when id was already seen. */
static int g_mark(uint32_t *vis, uint32_t id) {
    uint32_t h = (id * 2654435761u) & (G_HASH - 1u);
    for (uint32_t p = 0; p < G_PROBES; p++) {
        const uint32_t cur = vis[h];
        if (cur == id + 1u) return 1;
        if (cur == 0u) {
            vis[h] = id + 1u;
            return 0;
        }
        h = (h + 1u) & (G_HASH - 1u);
    }
    return 0; /* shed: reported unseen, not recorded */
}

/* The shader's argmin (unexpanded slots) / argmax (all active slots). */
static uint32_t g_arg(const float *val, const uint32_t *expd, uint32_t efA, int want_max, float *best_out) {
    float rv[G_WG];
    uint32_t ri[G_WG];
    for (uint32_t t = 0; t < G_WG; t++) {
        float best = want_max ? -G_INF : G_INF;
        uint32_t bi = 0;
        for (uint32_t s = t; s < efA; s += G_WG) {
            if (want_max) {
                if (val[s] > best) {
                    best = val[s];
                    bi = s;
                }
            } else if (expd[s] == 0u && val[s] < best) {
                best = val[s];
                bi = s;
            }
        }
        rv[t] = best;
        ri[t] = bi;
    }
    for (uint32_t stride = G_WG >> 1; stride; stride >>= 1)
        for (uint32_t t = 0; t < stride; t++)
            if (want_max ? rv[t + stride] > rv[t] : rv[t + stride] < rv[t]) {
                rv[t] = rv[t + stride];
                ri[t] = ri[t + stride];
            }
    *best_out = rv[0];
    return ri[0];
}

/* foldStaged (graphSearch.ts:133-165). */
static void g_fold(float *cd, uint32_t *ci, uint32_t *ce, uint32_t efA, const float *sd, const uint32_t *si,
                   uint32_t count) {
    for (uint32_t j = 0; j < count; j++) {
        float worst;
        const uint32_t slot = g_arg(cd, ce, efA, 1, &worst);
        if (sd[j] < worst) {
            cd[slot] = sd[j];
            ci[slot] = si[j];
            ce[slot] = 0u;
        }
    }
}

/* The beam of each query after the search: G_EF (dist, id) slots per query.
 * The adjacency covers graph_rows rows of a corpus of corpus_rows rows; a
 * node past graph_rows has no neighbours and an id at or past corpus_rows
 * is skipped like an empty slot (the shader relies on WebGPU's robust
 * buffer access for those). */
EXPORT void bvo_graph_search(const float *corpus, uint32_t dim, int l2, const uint32_t *graph, uint32_t K,
                             uint32_t graph_rows, uint32_t corpus_rows, const float *queries, uint32_t nq,
                             const uint32_t *entries, uint32_t n_entries, uint32_t ef, uint32_t iter_cap,
                             float *out_dist, uint32_t *out_id) {
    const uint32_t efA = ef < G_EF ? ef : G_EF;
    const uint32_t ne = n_entries < G_WG ? n_entries : G_WG;
    uint32_t *vis = (uint32_t *)malloc(G_HASH * sizeof(uint32_t));
    float cd[G_EF], sd[G_WG];
    uint32_t ci[G_EF], ce[G_EF], si[G_WG];
    for (uint32_t q = 0; q < nq; q++) {
        const float *qv = queries + (size_t)q * dim;
        memset(vis, 0, G_HASH * sizeof(uint32_t));
        for (uint32_t s = 0; s < G_EF; s++) {
            cd[s] = G_INF;
            ci[s] = G_EMPTY;
            ce[s] = 1u;
        }
        for (uint32_t t = 0; t < ne; t++) {
            const uint32_t e = entries[t];
            sd[t] = G_INF;
            si[t] = G_EMPTY;
            if (e < corpus_rows && !g_mark(vis, e)) {
                sd[t] = g_dist(corpus + (size_t)e * dim, qv, dim, l2);
                si[t] = e;
            }
        }
        g_fold(cd, ci, ce, efA, sd, si, ne);
        for (uint32_t iter = 0; iter < iter_cap; iter++) {
            float best;
            const uint32_t slot = g_arg(cd, ce, efA, 0, &best);
            if (best >= G_INF) break;
            ce[slot] = 1u;
            const uint32_t node = ci[slot];
            for (uint32_t t = 0; t < K; t++) {
                sd[t] = G_INF;
                si[t] = G_EMPTY;
                const uint32_t nb = node < graph_rows ? graph[(size_t)node * K + t] : G_EMPTY;
                if (nb < corpus_rows && !g_mark(vis, nb)) {
                    sd[t] = g_dist(corpus + (size_t)nb * dim, qv, dim, l2);
                    si[t] = nb;
                }
            }
            g_fold(cd, ci, ce, efA, sd, si, K);
        }
        memcpy(out_dist + (size_t)q * G_EF, cd, sizeof(cd));
        memcpy(out_id + (size_t)q * G_EF, ci, sizeof(ci));
    }
    free(vis);
}

/* HNSWGpuSearcher.search's seeds (hnswGpu.ts:142-150): the entry, then up to
 * seven rows spread evenly over the graph's rows.  Returns the count. */
EXPORT uint32_t bvo_graph_entries(uint32_t entry, uint32_t graph_rows, uint32_t *out) {
    uint32_t e = 0;
    out[e++] = entry;
    const uint32_t extra = graph_rows < 7u ? graph_rows : 7u;
    for (uint32_t i = 0; i < extra; i++)
        out[e++] = (uint32_t)(floor(((double)(i + 1) * (double)graph_rows) / (double)(extra + 1)) ) % graph_rows;
    return e;
}

/* The readback's dedup and top-k (hnswGpu.ts:191-203): live slots in slot
 * order, first occurrence of an id kept, score = -dist, stable sort by score
 * descending, first k.  Returns the count. */
EXPORT uint32_t bvo_graph_hits(const float *dist, const uint32_t *id, uint32_t efA, uint32_t k, uint32_t *rows,
                               float *scores) {
    uint32_t n = 0;
    uint32_t hr[G_EF];
    float hs[G_EF];
    for (uint32_t s = 0; s < efA && s < G_EF; s++) {
        const uint32_t r = id[s];
        if (r == G_EMPTY) continue;
        int dup = 0;
        for (uint32_t j = 0; j < n; j++)
            if (hr[j] == r) {
                dup = 1;
                break;
            }
        if (dup) continue;
        hr[n] = r;
        hs[n] = -dist[s];
        n++;
    }
    /* stable insertion sort, descending */
    for (uint32_t i = 1; i < n; i++) {
        const uint32_t r = hr[i];
        const float v = hs[i];
        uint32_t j = i;
        while (j > 0 && hs[j - 1] < v) {
            hs[j] = hs[j - 1];
            hr[j] = hr[j - 1];
            j--;
        }
        hs[j] = v;
        hr[j] = r;
    }
    const uint32_t m = n < k ? n : k;
    for (uint32_t i = 0; i < m; i++) {
        rows[i] = hr[i];
        scores[i] = hs[i];
    }
    return m;
}
