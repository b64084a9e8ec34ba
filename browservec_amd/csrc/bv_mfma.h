// Helpers shared by the gfx950 kernels that stage tiles through LDS for the
// matrix cores (bv_mq.hip, bv_ivf.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bvk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

// A 16-byte (dwordx4) or 4-byte global load into LDS at lds + 16 * lane (4 *
// lane), written as inline asm so that the compiler does not track it: it
// would otherwise take every later LDS read as possibly racing with it and
// wait for all outstanding LDS operations before each one.  The caller waits
// for these loads itself (vmcnt) before the LDS is read.  They set M0, which
// the compiler reserves and does not track across inline asm: no other code
// in the kernels that use them keeps a value in M0.
// lds: a wave-uniform LDS byte address (lds_addr), kept in an SGPR.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void *)p);
}
__device__ __forceinline__ void lds_dma16(const void *src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory");
}
__device__ __forceinline__ void lds_dma4(const void *src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds) : "memory");
}

// s_waitcnt immediate waiting for vmcnt <= n (n < 64) only (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8 left at their maxima).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

}  // namespace
}  // namespace bvk
