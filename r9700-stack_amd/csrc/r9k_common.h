// r9k_common.h -- shared device helpers for the gfx950 (CDNA4) MoE hot-path kernels.
//
// Everything here is written for wave64 CDNA4 only: 64-lane ballots, 64-bit lane masks, bf16 <-> fp32 with
// round-to-nearest-even, OCP e4m3fn encoding with the same rounding and overflow rule torch's float8_e4m3fn cast
// uses (round to nearest even; a magnitude that rounds past 448 becomes the NaN code 0x7f).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace r9k {

constexpr int WAVE = 64;

__device__ __forceinline__ float bf2f(uint16_t u) { return __uint_as_float((uint32_t)u << 16); }

// fp32 -> bf16, round to nearest even; NaN stays a quiet NaN (torch's conversion).
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// fp32 -> OCP e4m3fn byte, round to nearest even.
//   |f| <  2^-6 : subnormal grid m * 2^-9 (m = 0..8; m = 8 is the smallest normal, code 0x08)
//   |f| >= 2^-6 : 3 mantissa bits kept with RNE on the dropped 20 bits; exponent bias 7
//   rounding past 448 (the largest finite, 0x7e) or a NaN input -> 0x7f
// The sign bit is kept for zeros, so -0.0 and negative values that round to zero give 0x80.
__device__ __forceinline__ uint32_t f32_to_e4m3(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  uint32_t r;
  if (a > 0x43e80000u) {                 // > 464 (or inf / NaN): rounds past 448
    r = 0x7fu;
  } else if (a < 0x3c800000u) {          // < 2^-6: subnormal grid, exact scale by 2^9 then RNE to an integer
    r = (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);
  } else {
    const uint32_t lsb = (a >> 20) & 1u;
    r = ((a + 0x7ffffu + lsb) >> 20) - ((127u - 7u) << 3);
  }
  return sign | r;
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  const uint32_t em = b & 0x7fu;
  float mag;
  if (em == 0x7fu) mag = __uint_as_float(0x7fc00000u);
  else if (em >= 0x08u) mag = __uint_as_float((em + ((127u - 7u) << 3)) << 20);
  else mag = (float)em * 0x1p-9f;
  return (b & 0x80u) ? -mag : mag;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
  return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, o, WAVE);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o, WAVE);
    const uint64_t w = ((uint64_t)hi << 32) | lo;
    v = w > v ? w : v;
  }
  return v;
}

// Block-wide max of a float; `sh` holds one float per wave. Every thread gets the result.
template <int NT>
__device__ __forceinline__ float block_max(float v, float* sh) {
  constexpr int NW = NT / WAVE;
  v = wave_max(v);
  const int w = threadIdx.x / WAVE, l = threadIdx.x % WAVE;
  if (l == 0) sh[w] = v;
  __syncthreads();
  float r = sh[0];
#pragma unroll
  for (int i = 1; i < NW; i++) r = fmaxf(r, sh[i]);
  __syncthreads();
  return r;
}

}  // namespace r9k
