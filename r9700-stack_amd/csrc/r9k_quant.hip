// r9k_quant.hip -- per-row dynamic fp8 (OCP e4m3fn) quantisation for the MoE hot path on gfx950.
//
//   r9k_quant_rows_fp8       x bf16 [M, K] (row stride ld) -> q e4m3fn [M, K], s fp32 [M]
//   r9k_quant_rows_fp8_gate  the same, plus g[row] = bf16(sigmoid(bf16(x[row] . wg))) (shared-expert gate)
//   r9k_silu_mul_quant_fp8   gu bf16 [M, 2I] (gate | up) -> silu(gate) * up quantised per row: q [M, I], s [M]
//
// Numerics (kernels/r9k_moe_mxfp4a8.hip:1729-1741 and :517-548 of the reference define them):
//   amax = max(max_k |x_k|, 1e-12);  inv = 448 / amax  (IEEE fp32 division);  q_k = e4m3_rne(x_k * inv);
//   s = amax / 448.  x_k * inv <= 448 * (1 + 2^-23) always rounds to 448 at most, so no NaN code appears.
// The fp32 -> e4m3 encode is the explicit RNE bit routine in r9k_common.h, so the bytes are the bytes torch's
// float8_e4m3fn cast produces for the same fp32 products.
//
// Rows up to 4096 elements run one wave per row (four rows a workgroup): each lane keeps R chunks of 8 bf16
// (16 bytes) in registers (one HBM read) and the row maximum is a wave reduction, no LDS or barrier. Longer rows
// take one workgroup of QT threads per row (QR chunks a thread), and rows that do not fit or are not 16-byte
// aligned take the two-pass scalar kernel. Rows are independent, so M up to the grid limit is fine.
#include "r9k_common.h"

namespace {

using namespace r9k;

constexpr int QT = 256;     // threads per row
constexpr int QR = 4;       // 16-byte chunks per thread kept in registers: K <= 8192 on the vectorised path

constexpr int WR = 4;       // rows (waves) per workgroup of the wave-per-row kernels

// One wave per row, R 16-byte chunks per lane (K <= 512 * R). The plain quant is quant_row_wave (shared with the
// routing kernel's fused activation quant, so both give the same bytes).
template <bool GATE, int R>
__global__ void __launch_bounds__(WR * WAVE) quant_rows_wave_kernel(const uint16_t* __restrict__ x,
                                                                    uint8_t* __restrict__ q, float* __restrict__ s,
                                                                    int M, int K, long ld,
                                                                    const uint16_t* __restrict__ wg,
                                                                    float* __restrict__ g) {
  const int row = blockIdx.x * WR + threadIdx.x / WAVE, lane = threadIdx.x % WAVE, nvec = K / 8;
  if (row >= M) return;
  if constexpr (!GATE) {
    quant_row_wave<R>(x + (size_t)row * ld, K, q + (size_t)row * K, s + row, lane);
    return;
  }
  const uint4* xr = reinterpret_cast<const uint4*>(x + (size_t)row * ld);
  uint4 v[R];
  float m = 0.f, dot = 0.f;
#pragma unroll
  for (int i = 0; i < R; i++) {
    const int c = lane + i * WAVE;
    v[i] = load_chunk_or_zero(xr, c, nvec);
  }
#pragma unroll
  for (int i = 0; i < R; i++) {
    const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
    for (int j = 0; j < 4; j++) m = fmaxf(m, fmaxf(fabsf(lo16(w[j])), fabsf(hi16(w[j]))));
    if constexpr (GATE) {
      const int c = lane + i * WAVE;
      // chunks past the row are zero on both sides: their +0 terms leave the bf16 logit and its sigmoid as they are
      const uint4 gw = load_chunk_or_zero(reinterpret_cast<const uint4*>(wg), c, nvec);
      const uint32_t u[4] = {gw.x, gw.y, gw.z, gw.w};
#pragma unroll
      for (int j = 0; j < 4; j++) dot += lo16(w[j]) * lo16(u[j]) + hi16(w[j]) * hi16(u[j]);
    }
  }
  const float amax = fmaxf(wave_max(m), 1e-12f);
  if constexpr (GATE) {
    dot = wave_sum(dot);
    if (lane == 0) {
      const float logit = bf2f(f2bf(dot));                     // the router-style bf16 GEMM output
      g[row] = bf2f(f2bf(1.f / (1.f + expf(-logit))));           // bf16 sigmoid
    }
  }
  const float inv = 448.f / amax;
  if (lane == 0) s[row] = amax / 448.f;
  uint2* qr = reinterpret_cast<uint2*>(q + (size_t)row * K);
#pragma unroll
  for (int i = 0; i < R; i++) {
    const int c = lane + i * WAVE;
    if (c < nvec) {
      qr[c] = pack8_bf16_e4m3(v[i], inv);
    }
  }
}

template <bool GATE>
__global__ void __launch_bounds__(QT) quant_rows_vec_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ q,
                                                            float* __restrict__ s, int K, long ld,
                                                            const uint16_t* __restrict__ wg, float* __restrict__ g) {
  __shared__ float sh[QT / WAVE];
  __shared__ float shd[QT / WAVE];
  const int row = blockIdx.x, tid = threadIdx.x, nvec = K / 8;
  const uint4* xr = reinterpret_cast<const uint4*>(x + (size_t)row * ld);
  uint4 v[QR];
  float m = 0.f, dot = 0.f;
#pragma unroll
  for (int i = 0; i < QR; i++) {
    const int c = tid + i * QT;
    v[i] = load_chunk_or_zero(xr, c, nvec);
    const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
    for (int j = 0; j < 4; j++) m = fmaxf(m, fmaxf(fabsf(lo16(w[j])), fabsf(hi16(w[j]))));
    if constexpr (GATE) {
      // chunks past the row are zero on both sides: their +0 terms leave the bf16 logit and its sigmoid as they are
      const uint4 gw = load_chunk_or_zero(reinterpret_cast<const uint4*>(wg), c, nvec);
      const uint32_t u[4] = {gw.x, gw.y, gw.z, gw.w};
#pragma unroll
      for (int j = 0; j < 4; j++) dot += lo16(w[j]) * lo16(u[j]) + hi16(w[j]) * hi16(u[j]);
    }
  }
  const float rmax = block_max<QT>(m, sh);
  if constexpr (GATE) {
    dot = wave_sum(dot);
    if (tid % WAVE == 0) shd[tid / WAVE] = dot;
    __syncthreads();
    if (tid == 0) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < QT / WAVE; i++) d += shd[i];
      const float logit = bf2f(f2bf(d));                       // the router-style bf16 GEMM output
      g[row] = bf2f(f2bf(1.f / (1.f + expf(-logit))));           // bf16 sigmoid
    }
  }
  const float amax = fmaxf(rmax, 1e-12f);
  const float inv = 448.f / amax;
  if (tid == 0) s[row] = amax / 448.f;
  uint2* qr = reinterpret_cast<uint2*>(q + (size_t)row * K);
#pragma unroll
  for (int i = 0; i < QR; i++) {
    const int c = tid + i * QT;
    if (c >= nvec) break;
    qr[c] = pack8_bf16_e4m3(v[i], inv);
  }
}

// Two-pass fallback for any K / ld / alignment: max pass, then a quantise pass that re-reads the row.
template <bool GATE>
__global__ void __launch_bounds__(QT) quant_rows_scalar_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ q,
                                                               float* __restrict__ s, int K, long ld,
                                                               const uint16_t* __restrict__ wg, float* __restrict__ g) {
  __shared__ float sh[QT / WAVE];
  __shared__ float shd[QT / WAVE];
  const int row = blockIdx.x, tid = threadIdx.x;
  const uint16_t* xr = x + (size_t)row * ld;
  float m = 0.f, dot = 0.f;
  for (int k = tid; k < K; k += QT) {
    const float v = bf2f(xr[k]);
    m = fmaxf(m, fabsf(v));
    if constexpr (GATE) dot += v * bf2f(wg[k]);
  }
  const float rmax = block_max<QT>(m, sh);
  if constexpr (GATE) {
    dot = wave_sum(dot);
    if (tid % WAVE == 0) shd[tid / WAVE] = dot;
    __syncthreads();
    if (tid == 0) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < QT / WAVE; i++) d += shd[i];
      const float logit = bf2f(f2bf(d));
      g[row] = bf2f(f2bf(1.f / (1.f + expf(-logit))));
    }
  }
  const float amax = fmaxf(rmax, 1e-12f);
  const float inv = 448.f / amax;
  if (tid == 0) s[row] = amax / 448.f;
  uint8_t* qr = q + (size_t)row * K;
  for (int k = tid; k < K; k += QT) qr[k] = (uint8_t)f32_to_e4m3(bf2f(xr[k]) * inv);
}


// One wave per row, R 16-byte chunks of gate and of up per lane (I <= 512 * R), activations kept in registers.
// NT: non-temporal row loads (the host sets it for prefill-sized inputs).
template <int R, bool NT>
__global__ void __launch_bounds__(WR * WAVE) silu_mul_quant_wave_kernel(const uint16_t* __restrict__ gu,
                                                                        uint8_t* __restrict__ q,
                                                                        float* __restrict__ s, int M, int I) {
  const int row = blockIdx.x * WR + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  if (row >= M) return;
  const float sc = silu_quant_row_wave<R, NT>(gu + (size_t)row * 2 * I, I, q + (size_t)row * I, lane);
  if (lane == 0) s[row] = sc;
}

// One row per workgroup; each thread keeps its activations (I <= QT * 8 * QR) in registers between the max pass
// and the store pass. Larger I recomputes the activation in the store pass.
__global__ void __launch_bounds__(QT) silu_mul_quant_kernel(const uint16_t* __restrict__ gu, uint8_t* __restrict__ q,
                                                            float* __restrict__ s, int I, int vec) {
  __shared__ float sh[QT / WAVE];
  const int row = blockIdx.x, tid = threadIdx.x;
  const uint16_t* gr = gu + (size_t)row * 2 * I;
  const uint16_t* ur = gr + I;
  float m = 0.f;
  float a[QR][8];
  if (vec) {
    const int nvec = I / 8;
#pragma unroll
    for (int i = 0; i < QR; i++) {
      const int c = tid + i * QT;
#pragma unroll
      for (int j = 0; j < 8; j++) a[i][j] = 0.f;
      if (c < nvec) {
        const uint4 gv = reinterpret_cast<const uint4*>(gr)[c];
        const uint4 uv = reinterpret_cast<const uint4*>(ur)[c];
        const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          a[i][2 * j] = silu_mul(lo16(gw[j]), lo16(uw[j]));
          a[i][2 * j + 1] = silu_mul(hi16(gw[j]), hi16(uw[j]));
        }
#pragma unroll
        for (int j = 0; j < 8; j++) m = fmaxf(m, fabsf(a[i][j]));
      }
    }
  } else {
    for (int k = tid; k < I; k += QT) m = fmaxf(m, fabsf(silu_mul(bf2f(gr[k]), bf2f(ur[k]))));
  }
  const float amax = fmaxf(block_max<QT>(m, sh), 1e-12f);
  const float inv = 448.f / amax;
  if (tid == 0) s[row] = amax / 448.f;
  uint8_t* qr = q + (size_t)row * I;
  if (vec) {
    const int nvec = I / 8;
#pragma unroll
    for (int i = 0; i < QR; i++) {
      const int c = tid + i * QT;
      if (c >= nvec) break;
      reinterpret_cast<uint2*>(qr)[c] = pack8_e4m3(a[i], inv);
    }
  } else {
    for (int k = tid; k < I; k += QT) qr[k] = (uint8_t)f32_to_e4m3(silu_mul(bf2f(gr[k]), bf2f(ur[k])) * inv);
  }
}

bool vec_ok(long x, long q, int K, long ld) {
  return K % 8 == 0 && ld % 8 == 0 && (x & 15) == 0 && (q & 7) == 0 && K <= QT * 8 * QR;
}

// 16-byte chunks per lane of the wave-per-row kernels for a row of n elements (0: row too long).
int wave_chunks(int n) {
  const int c = (n / 8 + WAVE - 1) / WAVE;
  return c <= 1 ? 1 : c <= 2 ? 2 : c <= 4 ? 4 : c <= 8 ? 8 : 0;
}

template <bool GATE>
bool launch_wave(long x, long q, long s, long wg, long g, int M, int K, int ld, hipStream_t st) {
  const dim3 grid((M + WR - 1) / WR), blk(WR * WAVE);
  switch (wave_chunks(K)) {
#define QW(RV)                                                                                                  \
  case RV:                                                                                                      \
    hipLaunchKernelGGL((quant_rows_wave_kernel<GATE, RV>), grid, blk, 0, st, (const uint16_t*)x, (uint8_t*)q,   \
                       (float*)s, M, K, (long)ld, (const uint16_t*)wg, (float*)g);                             \
    return true;
    QW(1) QW(2) QW(4) QW(8)
#undef QW
    default: return false;
  }
}

}  // namespace

// Reference: kernels/r9k_moe_mxfp4a8.hip:1745-1757 (r9k_quant_rows_fp8). 0 on success, -3 bad shape, -6 launch error.
extern "C" int r9k_quant_rows_fp8(long x, long q, long s, int M, int K, int ld, long stream) {
  if (M <= 0) return 0;
  if (K <= 0 || ld < K || !x || !q || !s) return -3;
  const hipStream_t st = (hipStream_t)stream;
  if (vec_ok(x, q, K, ld) && launch_wave<false>(x, q, s, 0, 0, M, K, ld, st)) {
  } else if (vec_ok(x, q, K, ld))
    hipLaunchKernelGGL(quant_rows_vec_kernel<false>, dim3(M), dim3(QT), 0, st, (const uint16_t*)x, (uint8_t*)q,
                       (float*)s, K, (long)ld, (const uint16_t*)nullptr, (float*)nullptr);
  else
    hipLaunchKernelGGL(quant_rows_scalar_kernel<false>, dim3(M), dim3(QT), 0, st, (const uint16_t*)x, (uint8_t*)q,
                       (float*)s, K, (long)ld, (const uint16_t*)nullptr, (float*)nullptr);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

// Reference: kernels/r9k_moe_mxfp4a8.hip:1770-1781. The fragment-tiled store (tiled != 0) belongs to the gfx12
// A-tiled prefill kernel, which this library does not carry: tiled != 0 returns -3.
extern "C" int r9k_quant_rows_fp8_gate(long x, long q, long s, long wg, long g, int M, int K, int ld, int tiled,
                                       long stream) {
  if (M <= 0) return 0;
  if (tiled || K <= 0 || ld < K || !x || !q || !s || !wg || !g) return -3;
  const hipStream_t st = (hipStream_t)stream;
  if (vec_ok(x, q, K, ld) && (wg & 15) == 0 && launch_wave<true>(x, q, s, wg, g, M, K, ld, st)) {
  } else if (vec_ok(x, q, K, ld) && (wg & 15) == 0)
    hipLaunchKernelGGL(quant_rows_vec_kernel<true>, dim3(M), dim3(QT), 0, st, (const uint16_t*)x, (uint8_t*)q,
                       (float*)s, K, (long)ld, (const uint16_t*)wg, (float*)g);
  else
    hipLaunchKernelGGL(quant_rows_scalar_kernel<true>, dim3(M), dim3(QT), 0, st, (const uint16_t*)x, (uint8_t*)q,
                       (float*)s, K, (long)ld, (const uint16_t*)wg, (float*)g);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

// Reference: kernels/r9k_moe_mxfp4a8.hip:550-555. gu contiguous [M, 2I] bf16.
extern "C" int r9k_silu_mul_quant_fp8(long gu, long q, long s, int M, int I, long stream) {
  if (M <= 0) return 0;
  if (I <= 0 || !gu || !q || !s) return -3;
  const int vec = (gu & 15) == 0 && (q & 7) == 0 && I % 8 == 0 && I <= QT * 8 * QR;
  const int R = vec ? wave_chunks(I) : 0;
  const dim3 wgrid((M + WR - 1) / WR), wblk(WR * WAVE);
  const hipStream_t st = (hipStream_t)stream;
  // non-temporal loads once the input is far larger than the L2s (config 3's 134 MB); decode widths keep plain loads
  const bool nt = (size_t)M * (size_t)I * 4u >= NT_STREAM_BYTES;
#define SW(RV)                                                                                                      \
  if (nt) hipLaunchKernelGGL((silu_mul_quant_wave_kernel<RV, true>), wgrid, wblk, 0, st, (const uint16_t*)gu,      \
                             (uint8_t*)q, (float*)s, M, I);                                                         \
  else hipLaunchKernelGGL((silu_mul_quant_wave_kernel<RV, false>), wgrid, wblk, 0, st, (const uint16_t*)gu,        \
                          (uint8_t*)q, (float*)s, M, I)
  if (R == 1) SW(1);
  else if (R == 2) SW(2);
  else if (R == 4) SW(4);
  else if (R == 8) SW(8);
#undef SW
  else hipLaunchKernelGGL(silu_mul_quant_kernel, dim3(M), dim3(QT), 0, (hipStream_t)stream, (const uint16_t*)gu,
                     (uint8_t*)q, (float*)s, I, vec);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}
