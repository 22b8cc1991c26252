// r9k_router_tile.h -- the router gate GEMM's per-lane math, shared by the standalone router kernel
// (r9k_router.hip) and the fused router + routing kernel (r9k_moe_route.hip), so both produce the same logits bit
// for bit: V_DOT2C_F32_BF16 over 16-byte chunks, then a wave transpose-sum.
#pragma once
#include "r9k_common.h"

namespace r9k {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot8(uint4 a, uint4 b, float c) {
  c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.x), __builtin_bit_cast(bf16x2, b.x), c, false);
  c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.y), __builtin_bit_cast(bf16x2, b.y), c, false);
  c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.z), __builtin_bit_cast(bf16x2, b.z), c, false);
  c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.w), __builtin_bit_cast(bf16x2, b.w), c, false);
  return c;
}

// N values (a power of two <= 64) held by every lane -> lane l returns the wave-wide sum of value l / (64 / N).
// Each halving step keeps one half of the values and trades the other half with the lane `o` away, so the work is
// N - 1 exchanges plus log2(64 / N) for the lanes that still share a value.
template <int N>
__device__ __forceinline__ float wave_transpose_sum(float (&v)[N], int lane) {
  static_assert(N >= 1 && N <= WAVE && (N & (N - 1)) == 0, "N: a power of two <= 64");
  int o = WAVE / 2;
#pragma unroll
  for (int h = N / 2; h >= 1; h /= 2) {
    const bool up = lane & o;
#pragma unroll
    for (int i = 0; i < h; i++) {
      const float send = up ? v[i] : v[i + h];
      const float keep = up ? v[i + h] : v[i];
      v[i] = keep + __shfl_xor(send, o, WAVE);
    }
    o >>= 1;
  }
  float s = v[0];
#pragma unroll
  for (; o >= 1; o >>= 1) s += __shfl_xor(s, o, WAVE);
  return s;
}

// Launch shape, measured on the gates served (E 256-512, K 2048-7168, M 1-32): many small workgroups beat few
// large ones (the loads in flight across the chip, not the bytes, bound the time), so a workgroup takes 1-2 experts x
// 1-4 tokens and 1-4 waves, each lane about `cpl` chunks of K (two at a time: the chunk loop is unrolled twice).
inline void router_shape(int M, int K, int* ept, int* mt, int* nw) {
  int cpl;
  if (M <= 2) *ept = 1, *mt = 1, cpl = 2;
  else if (M <= 4) *ept = 1, *mt = 2, cpl = 2;
  else if (M <= 8) *ept = 2, *mt = 2, cpl = 3;
  else if (M <= 16) *ept = 2, *mt = 2, cpl = 6;
  else *ept = 2, *mt = 4, cpl = 8;
  const int nch = K / 8;
  *nw = nch / (WAVE * cpl) + (nch % (WAVE * cpl) != 0);
  *nw = *nw < 1 ? 1 : (*nw > 4 ? 4 : *nw);
}

// One workgroup's EPT x MT tile of x . w^T over all of K with the first nw waves (the rest idle here): every lane of
// those waves walks the 16-byte chunks tid, tid + 64 nw, ... (two in flight), each wave transpose-sums its N = EPT x
// MT partials, and the waves' sums meet in `part` in wave order. Returns value tid (expert e0 + tid / MT, token
// m0 + tid % MT) on threads tid < N after a workgroup barrier; every thread of the workgroup must call it.
template <int EPT, int MT>
__device__ __forceinline__ float router_tile(const uint16_t* __restrict__ x, long sx, const uint16_t* __restrict__ w,
                                             long sw, int M, int E, int K, int e0, int m0, int nw,
                                             float (*part)[EPT * MT]) {
  constexpr int N = EPT * MT;
  const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
  const int nch = K / 8, nt = nw * WAVE;
  if (wave < nw) {
    float acc[N];
#pragma unroll
    for (int i = 0; i < N; i++) acc[i] = 0.f;
#pragma unroll 2
    for (int c = tid; c < nch; c += nt) {
      uint4 wv[EPT], xv[MT];
#pragma unroll
      for (int i = 0; i < EPT; i++) wv[i] = reinterpret_cast<const uint4*>(w + (long)min(e0 + i, E - 1) * sw)[c];
#pragma unroll
      for (int m = 0; m < MT; m++) xv[m] = reinterpret_cast<const uint4*>(x + (long)min(m0 + m, M - 1) * sx)[c];
#pragma unroll
      for (int i = 0; i < EPT; i++)
#pragma unroll
        for (int m = 0; m < MT; m++) acc[i * MT + m] = dot8(wv[i], xv[m], acc[i * MT + m]);
    }
    const float s = wave_transpose_sum<N>(acc, lane);
    constexpr int G = WAVE / N;             // lanes sharing one value after the transpose
    if (lane % G == 0) part[wave][lane / G] = s;
  }
  __syncthreads();
  float v = 0.f;
  if (tid < N) {
    v = part[0][tid];
    for (int q = 1; q < nw; q++) v += part[q][tid];
  }
  return v;
}

}  // namespace r9k
