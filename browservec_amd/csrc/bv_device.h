// Device-side helpers shared by the gfx950 kernel files: ordering keys and
// the per-query level constants of the int8 / int4 scans.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bvk {

// Ordering keys: one u64 per candidate, high word = order-preserving bits of
// the score (-0 folded into +0), low word = ~row.  Larger key = better
// (higher score, then lower row), so a descending sort gives the canonical
// (score desc, row asc) order and keys are unique per row.  Key 0 = empty.
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

// Per-query constants stored after the packed query levels: the scale of
// each level (int8: already divided by 127) and, for int4, the sum of each
// level's query bytes.
struct QLevelTail {
    double s[3];
    int32_t sum[3];
    int32_t pad;
};

// Tail of the 1-bit asymmetric bit-plane layout: the query's two levels
// (q ~= s1 * Q1 + s2 * Q2, Q1 int8, Q2 int4), sum |q - s1 Q1 - s2 Q2|,
// sum |q|, sum Q1 and sum Q2.
struct Q1Tail {
    double s1;
    double s2;
    double rsum;
    double qabs;
    int32_t sumq1;
    int32_t sumq2;
};

}  // namespace bvk
