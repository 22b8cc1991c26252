// r9k_dma.h -- gfx950 helpers shared by the LDS-tiled prefill kernels: direct global -> LDS DMA
// (global_load_lds_dword / _dwordx4, completion tracked by vmcnt, which the kernels wait on explicitly), wave-uniform
// pointers and LDS addresses, and packed bf16 conversion.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace r9k {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two fp32 values to packed bf16, round to nearest even (v_cvt_pk_bf16_f32), a in the low half.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, (bf16x2){(__bf16)a, (__bf16)b});
}

// global -> LDS DMA of 16 (4) bytes per lane: lane l's bytes land at LDS address `lds` + 16 l (4 l). M0 carries the
// wave-uniform LDS base. Completion is tracked by vmcnt; the kernels wait for it explicitly.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
// The same from a wave-uniform base (SGPR pair) plus a 32-bit per-lane byte offset.
__device__ __forceinline__ void dma16s(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4s(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(lds) : "memory", "m0");
}
// A wave-uniform copy of a pointer computed from per-lane-equal values (kept in SGPRs).
__device__ __forceinline__ const uint8_t* uniform_ptr(const void* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}

}  // namespace r9k
