// LDS tile helpers shared by the attention kernels: swizzles of row-major
// 16-bit tiles in LDS and the asynchronous global -> LDS copy.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "index_map.h"

namespace trinix {

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

// Asynchronous global -> LDS copy (global_load_lds_dwordx4): lane l's 16
// bytes land at LDS byte address lds_base + 16*l (lds_base wave-uniform).
// Issued through asm so that the compiler's wait-count analysis
// does not see it: an LDS-writing global load makes that analysis wait for
// all LDS reads in flight (lgkmcnt(0)) at every LDS operand use.  Callers
// wait for these loads themselves (s_waitcnt vmcnt + barrier) before any
// wavefront reads the LDS they fill.
// The global address is a wave-uniform 64-bit base (SGPR pair) plus a
// per-lane 32-bit byte offset.
__device__ inline void dma_16b_s(uint32_t offset, uint64_t base, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(offset), "s"(base), "s"(lds_base) : "memory", "m0");
}

// Same with 4 bytes per lane (global_load_lds_dword): lane l's 4 bytes land
// at lds_base + 4*l.
__device__ inline void dma_4b_s(uint32_t offset, uint64_t base, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" : : "v"(offset), "s"(base), "s"(lds_base) : "memory", "m0");
}

// Wave-uniform copy of a pointer as a 64-bit SGPR value.
__device__ inline uint64_t uniform_ptr(const void* ptr) {
  const uint64_t x = (uint64_t)(uintptr_t)ptr;
  // readfirstlane returns int: widen through uint32_t (no sign extension)
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)x);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(x >> 32));
  return (uint64_t)lo | ((uint64_t)hi << 32);
}

}  // namespace trinix
