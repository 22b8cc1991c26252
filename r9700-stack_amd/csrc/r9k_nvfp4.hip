// r9k_nvfp4.hip -- load-time NVFP4 -> MXFP4 conversion with MSE-searched block exponents, on gfx950.
//
// Per 32-element block of a row (reference: r9700_vllm/quant/nvfp4.py:39-90):
//   1. exact dequant  x_i = (E2M1[c_i] * float(s16[i / 16])) / row_div      (fp32 multiply, then fp32 division)
//   2. amax = max(max_i |x_i|, 2^-126);  e0 = ceil(log2(amax / 6)) clamped to [-126, 127]
//   3. for d in (0, -1):  e = clamp(e0 + d, -127, 127);  c_i = nearest E2M1 of x_i / 2^e with ties to the smaller
//      magnitude (torch.bucketize(right=False) on the thresholds 0.25 .. 5.0; > 5 saturates to 6), sign bit set
//      for x_i / 2^e < 0 (so -0.0 encodes as 0, a negative value rounding to zero as 8);
//      err = sum_i (E2M1[c_i] * 2^e - x_i)^2;   the d = -1 candidate wins only if its err is strictly lower
//   4. e8m0 byte = e + 127; codes packed two a byte, element 2i in the low nibble.
// Two places where the reference's torch arithmetic is implementation-defined are computed exactly here:
//   * e0 is the smallest integer e with amax <= 6 * 2^e (frexp), where the reference takes ceil of an fp32 log2;
//     the two differ only when amax / 6 lies within ~2^-20 (relative) above a power of two, which no block with
//     <= 23 significant bits of mantissa above bit 1 reaches -- never for NVFP4-derived values (<= 6 bits);
//   * err is summed in fp64 in ascending i (each term exact in fp64 for fp32 inputs), where torch sums fp32 in an
//     unspecified order; they can only disagree when the two candidates' errors tie within fp32 rounding.
// One thread converts one block: it reads 16 bytes of codes and 2 scale bytes and writes 16 + 1 bytes, so a wave
// streams 1 KB of codes contiguously.
#include "r9k_common.h"

namespace {

using namespace r9k;

__device__ __forceinline__ float e2m1_val(uint32_t c) {
  const float mag[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
  const float m = mag[c & 7u];
  return (c & 8u) ? -m : m;
}

__device__ __forceinline__ uint32_t e2m1_encode(float v) {
  const float a = fabsf(v);
  uint32_t c = (a > 0.25f) + (a > 0.75f) + (a > 1.25f) + (a > 1.75f) + (a > 2.5f) + (a > 3.5f) + (a > 5.0f);
  return c | (v < 0.f ? 8u : 0u);
}

// smallest integer e with a <= 6 * 2^e, for a normal positive fp32 a
__device__ __forceinline__ int exp_no_clip(float a) {
  int p;
  const float m = frexpf(a, &p);          // a = m * 2^p, m in [0.5, 1)
  return p - 3 + (m > 0.75f ? 1 : 0);     // 6 * 2^e = 0.75 * 2^(e + 3)
}

// MSE-searched MXFP4 encode of one 32-element fp32 block: packed codes (4 dwords) and the e8m0 byte.
__device__ __forceinline__ uint32_t search_block(const float (&x)[32], uint32_t (&best_w)[4]) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
  amax = fmaxf(amax, 0x1p-126f);
  int e0 = exp_no_clip(amax);
  e0 = e0 < -126 ? -126 : (e0 > 127 ? 127 : e0);
  int best_e = 0;
  double best_err = 0.0;
#pragma unroll
  for (int d = 0; d >= -1; d--) {
    int e = e0 + d;
    e = e < -127 ? -127 : (e > 127 ? 127 : e);
    uint32_t cw[4] = {0u, 0u, 0u, 0u};
    double err = 0.0;
#pragma unroll
    for (int i = 0; i < 32; i++) {
      const uint32_t c = e2m1_encode(ldexpf(x[i], -e));
      cw[i >> 3] |= c << (4 * (i & 7));
      const double dv = (double)ldexpf(e2m1_val(c), e) - (double)x[i];
      err += dv * dv;
    }
    if (d == 0 || err < best_err) {
      best_err = err;
      best_e = e;
#pragma unroll
      for (int q = 0; q < 4; q++) best_w[q] = cw[q];
    }
  }
  return (uint32_t)(best_e + 127);
}

__global__ void __launch_bounds__(256) nvfp4_to_mxfp4_kernel(const uint8_t* __restrict__ packed,
                                                             const uint8_t* __restrict__ s16,
                                                             const float* __restrict__ row_div,
                                                             uint8_t* __restrict__ out_p, uint8_t* __restrict__ out_e,
                                                             long nblk, int bpr) {
  const long b = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblk) return;
  const long row = b / bpr;
  const uint4 pk = *reinterpret_cast<const uint4*>(packed + b * 16);
  const uint32_t sc = *reinterpret_cast<const uint16_t*>(s16 + b * 2);
  const float rd = row_div[row];
  const float s0 = e4m3_to_f32(sc & 0xffu), s1 = e4m3_to_f32(sc >> 8);
  const uint32_t w[4] = {pk.x, pk.y, pk.z, pk.w};
  float x[32];
#pragma unroll
  for (int i = 0; i < 32; i++) {
    const uint32_t c = (w[i >> 3] >> (4 * (i & 7))) & 0xfu;
    x[i] = (e2m1_val(c) * (i < 16 ? s0 : s1)) / rd;
  }
  uint32_t bw[4];
  const uint32_t eb = search_block(x, bw);
  *reinterpret_cast<uint4*>(out_p + b * 16) = make_uint4(bw[0], bw[1], bw[2], bw[3]);
  out_e[b] = (uint8_t)eb;
}

// fp32 weights [N, K] (row stride ld floats) -> MXFP4 by the same search (quantize_mxfp4_search on any weight).
__global__ void __launch_bounds__(256) mxfp4_search_kernel(const float* __restrict__ w, long ld,
                                                           uint8_t* __restrict__ out_p, uint8_t* __restrict__ out_e,
                                                           long nblk, int bpr) {
  const long b = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblk) return;
  const long row = b / bpr, col = (b - row * bpr) * 32;
  const float4* src = reinterpret_cast<const float4*>(w + row * ld + col);
  float x[32];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float4 v = src[i];
    x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
  }
  uint32_t bw[4];
  const uint32_t eb = search_block(x, bw);
  *reinterpret_cast<uint4*>(out_p + b * 16) = make_uint4(bw[0], bw[1], bw[2], bw[3]);
  out_e[b] = (uint8_t)eb;
}

}  // namespace

// New entry point (no reference C symbol: the reference converts with torch, r9700_vllm/quant/nvfp4.py:78-90).
// packed [N, K/2] u8, s16 [N, K/16] e4m3 bytes, row_div [N] fp32 -> out_packed [N, K/2] u8, out_e8m0 [N, K/32] u8,
// all contiguous, 16-byte aligned codes. 0 / -2 K % 32 / -3 bad pointer / -6 launch error.
extern "C" int r9k_nvfp4_to_mxfp4(long packed, long s16, long row_div, long out_packed, long out_e8m0, int N, int K,
                                  long stream) {
  if (N <= 0) return 0;
  if (K <= 0 || K % 32) return -2;
  if (!packed || !s16 || !row_div || !out_packed || !out_e8m0 || (packed & 15) || (out_packed & 15) || (s16 & 1))
    return -3;
  const int bpr = K / 32;
  const long nblk = (long)N * bpr;
  const long grid = (nblk + 255) / 256;
  if (grid > 0x7fffffffL) return -3;
  hipLaunchKernelGGL(nvfp4_to_mxfp4_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)packed, (const uint8_t*)s16, (const float*)row_div, (uint8_t*)out_packed,
                     (uint8_t*)out_e8m0, nblk, bpr);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

// fp32 [N, K] (row stride ld floats, 16-byte aligned rows) -> out_packed [N, K/2] u8, out_e8m0 [N, K/32] u8 with the
// same MSE search (reference: r9700_vllm/quant/nvfp4.py:54-75 on an arbitrary fp32 weight). 0 / -2 / -3 / -6.
extern "C" int r9k_quantize_mxfp4_search(long w, long out_packed, long out_e8m0, int N, int K, long stream) {
  if (N <= 0) return 0;
  if (K <= 0 || K % 32) return -2;
  if (!w || !out_packed || !out_e8m0 || (w & 15) || (out_packed & 15)) return -3;
  const int bpr = K / 32;
  const long nblk = (long)N * bpr;
  const long grid = (nblk + 255) / 256;
  if (grid > 0x7fffffffL) return -3;
  hipLaunchKernelGGL(mxfp4_search_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, (const float*)w,
                     (long)K, (uint8_t*)out_packed, (uint8_t*)out_e8m0, nblk, bpr);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}
