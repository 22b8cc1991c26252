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

// (E2M1[c] * s) / rd for the 16 codes of one group, with IEEE division semantics, from two divisions: every E2M1
// magnitude is 2^j or 1.5 * 2^j, and scaling a correctly rounded quotient by 2^j is exact while it stays normal, so
// RN(1.5^b * 2^j * s / rd) = 2^j * RN(1.5^b * s / rd). Groups whose quotients could leave the normal range (or a
// non-finite / non-positive divisor) divide per element.
__device__ __forceinline__ void e2m1_decode8(uint32_t w, float (&v)[8]);

__device__ __forceinline__ void dequant_group(const uint32_t w0, const uint32_t w1, float s, float rd, float* x) {
  const float q1 = s / rd, q3 = (1.5f * s) / rd;
  const float aq1 = fabsf(q1), aq3 = fabsf(q3);
  const bool fast = (aq1 >= 0x1p-125f || aq1 == 0.f) && aq3 <= 0x1p125f && rd > 0.f && rd <= 3.0e38f;
  float v[16];
  e2m1_decode8(w0, *reinterpret_cast<float(*)[8]>(v));
  e2m1_decode8(w1, *reinterpret_cast<float(*)[8]>(v + 8));
  if (fast) {
    // V = E2M1[c] = +-2^j (mantissa bit clear) or +-1.5 * 2^j (set): x = (V with its mantissa cleared) * (q1 or q3)
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const uint32_t vb = __float_as_uint(v[i]);
      x[i] = __uint_as_float(vb & 0xff800000u) * ((vb & 0x00400000u) ? q3 : q1);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; i++) x[i] = (v[i] * s) / rd;
  }
}

// The 8 E2M1 codes of one dword (low nibble first) as fp32 values, exact.
__device__ __forceinline__ void e2m1_decode8(uint32_t w, float (&v)[8]) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  const f2 a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
  const f2 b = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
  const f2 c = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
  const f2 d = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
  v[0] = a[0]; v[1] = a[1]; v[2] = b[0]; v[3] = b[1]; v[4] = c[0]; v[5] = c[1]; v[6] = d[0]; v[7] = d[1];
}

// smallest integer e with a <= 6 * 2^e, for a normal positive fp32 a; past the clamp (128) for +inf, as the
// reference's ceil(log2(inf / 6)) is
__device__ __forceinline__ int exp_no_clip(float a) {
  if (a > 0x1.fffffep127f) return 128;
  int p;
  const float m = frexpf(a, &p);          // a = m * 2^p, m in [0.5, 1)
  return p - 3 + (m > 0.75f ? 1 : 0);     // 6 * 2^e = 0.75 * 2^(e + 3)
}

// The 8 codes of x[0..8) / 2^e, packed low nibble first: for each v = x / 2^e the nearest E2M1 code with ties to the
// smaller magnitude (the reference's bucketize on 0.25 .. 5.0, > 5 saturating to 6), sign bit for v < 0.
// V_CVT_SCALEF32_PK_FP4_F32 (scale 1) converts two values into a byte (four conversions chain the dword); it rounds to
// nearest even and saturates (measured on gfx950 against this rule over 1M values), so it differs exactly at the ties
// whose lower neighbour is odd (|v| = 0.75, 1.75, 3.5, where it takes the even code above) and at -0.0 / NaN (sign or
// code kept; the rule gives 0). One mask subtracts 1 from every tied nibble (its magnitude is >= 2: no borrow), another
// clears every -0.0 / NaN nibble.
__device__ __forceinline__ uint32_t e2m1_encode8(const float* x, int e) {
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; j++) v[j] = ldexpf(x[j], -e);
  uint32_t w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, v[0], v[1], 1.0f, 0);
  w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, v[2], v[3], 1.0f, 1);
  w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, v[4], v[5], 1.0f, 2);
  w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, v[6], v[7], 1.0f, 3);
  uint32_t tie = 0u, zero = 0u;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint32_t b = __float_as_uint(v[j]), t = b & 0x7fffffffu;
    const uint32_t tb = (uint32_t)(t == 0x3f400000u) | (uint32_t)(t == 0x3fe00000u) | (uint32_t)(t == 0x40600000u);
    const uint32_t zb = (uint32_t)(b == 0x80000000u) | (uint32_t)(t > 0x7f800000u);
    tie |= tb << (4 * j);
    zero |= (zb * 0xfu) << (4 * j);
  }
  return (w - tie) & ~zero;
}

// fp32 sum of the squared errors of codes cw at exponent e against the block, each term an fma in ascending order.
// It is within 34 * 2^-24 (relative) of the exact sum whenever it is finite and no term underflows past 2^-100.
__device__ __forceinline__ float block_err32(const float (&x)[32], const uint32_t (&cw)[4], int e) {
  float err = 0.f;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    float v[8];
    e2m1_decode8(cw[q], v);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float dv = ldexpf(v[j], e) - x[8 * q + j];
      err = fmaf(dv, dv, err);
    }
  }
  return err;
}

// The reference's comparison sum: fp64 terms added in ascending i (each term's difference exact in fp64).
__device__ __forceinline__ double block_err64(const float (&x)[32], const uint32_t (&cw)[4], int e) {
  double err = 0.0;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    float v[8];
    e2m1_decode8(cw[q], v);                              // the codes' values (exact), back at the block scale
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const double dv = (double)ldexpf(v[j], e) - (double)x[8 * q + j];
      err += dv * dv;
    }
  }
  return err;
}

// MSE-searched MXFP4 encode of one 32-element fp32 block: packed codes (4 dwords) and the e8m0 byte. The e0 - 1
// candidate wins when its fp64 error sum (block_err64) is strictly lower. The fp32 sums decide first: each is within
// DELTA (relative) of the exact error and the fp64 sums within ~2^-47, so when the fp32 sums are apart by more than
// that margin the fp64 comparison agrees with them; ties, near-ties and sums outside fp32's safe range fall back to
// the fp64 sums, so the byte and the codes are the same as from the fp64 comparison alone.
__device__ __forceinline__ uint32_t search_block(const float (&x)[32], uint32_t (&best_w)[4]) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
  amax = fmaxf(amax, 0x1p-126f);
  int e0 = exp_no_clip(amax);
  e0 = e0 < -126 ? -126 : (e0 > 127 ? 127 : e0);
  const int e1 = e0 - 1;                                  // >= -127: no clamp needed
  uint32_t c0[4], c1[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    c0[q] = e2m1_encode8(x + 8 * q, e0);
    c1[q] = e2m1_encode8(x + 8 * q, e1);
  }
  const float a = block_err32(x, c0, e0), b = block_err32(x, c1, e1);
  constexpr float DELTA = 1e-5f;                          // > 34 * 2^-24 plus the rounding of these products
  bool take1;
  if (a >= 0x1p-100f && b >= 0x1p-100f && a <= 0x1p120f && b <= 0x1p120f &&
      (b * (1.f + DELTA) < a * (1.f - DELTA) || b * (1.f - DELTA) > a * (1.f + DELTA))) {
    take1 = b < a;
  } else {
    take1 = block_err64(x, c1, e1) < block_err64(x, c0, e0);
  }
#pragma unroll
  for (int q = 0; q < 4; q++) best_w[q] = take1 ? c1[q] : c0[q];
  return (uint32_t)((take1 ? e1 : e0) + 127);
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
  float x[32];
  dequant_group(pk.x, pk.y, s0, rd, x);
  dequant_group(pk.z, pk.w, s1, rd, x + 16);
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
