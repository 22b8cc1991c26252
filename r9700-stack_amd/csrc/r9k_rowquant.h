// r9k_rowquant.h -- the per-row fp8 (e4m3) activation quant done by every workgroup of a one-launch dense GEMM
// (r9k_dense.hip, r9k_moe_nvfp4.hip): the bytes of quant_row_wave (r9k_common.h) for the M <= 4 rows of a decode-width
// linear, written into the workgroup's LDS.
#pragma once
#include "r9k_common.h"

namespace r9k {

// The workgroup quantises the activation rows MG at a time, like quant_row_wave (the same amax, 448 / amax and
// per-element encode, so the same bytes): thread t holds chunks t + T i (i < XC, T threads) of each row, read once,
// so one row's read is spread over every wave of the workgroup and the reads of the first group go out ahead of the
// weight stream instead of queueing behind it. The row maxima meet in LDS (any combination order of a max gives the
// same value), then every thread encodes its own chunks.
template <int T>
constexpr int row_chunks() { return T >= 256 ? 4 : 2; }   // K / 8 <= chunks * T: K <= 8192 at 256 threads, < 1024 at 64

template <int T, int MG, int XC>
__device__ __forceinline__ void load_row_group(const uint16_t* __restrict__ x, long ldx, int m0, int M, int nvec,
                                               int tid, uint4 (&v)[MG][XC]) {
#pragma unroll
  for (int m = 0; m < MG; m++) {
    const bool live = m0 + m < M;                    // rows past M read row M - 1 and keep zeros
    const uint4* xr = reinterpret_cast<const uint4*>(x + (size_t)(live ? m0 + m : M - 1) * ldx);
#pragma unroll
    for (int i = 0; i < XC; i++) v[m][i] = load_chunk_or_zero(xr, live ? tid + i * T : nvec, nvec);
  }
}

// Ends with a barrier: the codes and scales of the group are visible, and `red` (MG floats a wave) is free again.
template <int T, int MG, int XC>
__device__ __forceinline__ void quant_row_group(const uint4 (&v)[MG][XC], int m0, int M, int nvec, uint8_t* A,
                                                int lda, float* s_row, float* red, int tid) {
  constexpr int NW = T / WAVE;
  const int wave = tid / WAVE, lane = tid % WAVE;
  float mx[MG];
#pragma unroll
  for (int m = 0; m < MG; m++) {
    mx[m] = 0.f;
#pragma unroll
    for (int i = 0; i < XC; i++) {
      const uint32_t w[4] = {v[m][i].x, v[m][i].y, v[m][i].z, v[m][i].w};
#pragma unroll
      for (int j = 0; j < 4; j++) mx[m] = fmaxf(mx[m], fmaxf(fabsf(lo16(w[j])), fabsf(hi16(w[j]))));
    }
  }
#pragma unroll
  for (int m = 0; m < MG; m++) mx[m] = wave_max(mx[m]);
  if (lane == 0) {
#pragma unroll
    for (int m = 0; m < MG; m++) red[wave * MG + m] = mx[m];
  }
  __syncthreads();
#pragma unroll
  for (int m = 0; m < MG; m++) {
    const int row = m0 + m;
    if (row >= M) break;
    float amax = red[m];
#pragma unroll
    for (int w = 1; w < NW; w++) amax = fmaxf(amax, red[w * MG + m]);
    amax = fmaxf(amax, 1e-12f);
    const float inv = 448.f / amax;
    if (tid == 0) s_row[row] = amax / 448.f;
    uint2* qr = reinterpret_cast<uint2*>(A + (size_t)row * lda);
#pragma unroll
    for (int i = 0; i < XC; i++) {
      const int c = tid + i * T;
      if (c < nvec) qr[c] = pack8_bf16_e4m3(v[m][i], inv);
    }
  }
  __syncthreads();
}

}  // namespace r9k
