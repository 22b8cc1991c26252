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
// Streaming passes (top-k sum, SiLU + quant) switch to non-temporal loads from this many input bytes: prefill-sized
// inputs (config 3's 134-268 MB) stream past the L2s, decode-sized ones (a few MB) keep plain loads.
constexpr size_t NT_STREAM_BYTES = size_t(64) << 20;

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
// Both roundings are computed and the result selected (no divergent branches in a vector of conversions).
__device__ __forceinline__ uint32_t f32_to_e4m3(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  const uint32_t rn = ((a + 0x7ffffu + ((a >> 20) & 1u)) >> 20) - ((127u - 7u) << 3);     // normal, |f| >= 2^-6
  const uint32_t rs = (uint32_t)__builtin_rintf(fminf(__uint_as_float(a), 0x1p-6f) * 512.0f);  // subnormal grid
  uint32_t r = a < 0x3c800000u ? rs : rn;
  r = a > 0x43e80000u ? 0x7fu : r;       // > 464 (or inf / NaN): rounds past 448
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

// Wave-uniform unsigned max: DPP within 16-lane rows (quad swaps, row rotates by 4 and 8: every lane of a row then
// holds the row's max), row_bcast:15 and row_bcast:31 carry the row maxima up to row 3, and lane 63's value is read
// out. Lanes of the rows a broadcast does not write get 0, the identity of the unsigned max.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#define R9K_DPP_MAX(ctrl, rows) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, ctrl, rows, 0xF, false))
  R9K_DPP_MAX(0xB1, 0xF);    // quad_perm [1,0,3,2]
  R9K_DPP_MAX(0x4E, 0xF);    // quad_perm [2,3,0,1]
  R9K_DPP_MAX(0x124, 0xF);   // row_ror:4
  R9K_DPP_MAX(0x128, 0xF);   // row_ror:8
  R9K_DPP_MAX(0x142, 0xA);   // row_bcast:15 -> rows 1, 3
  R9K_DPP_MAX(0x143, 0xC);   // row_bcast:31 -> rows 2, 3
#undef R9K_DPP_MAX
  return __builtin_amdgcn_readlane(v, 63);
}

// Running max of the bf16 magnitudes of the two halves of w (sign bits cleared, compared as unsigned 16-bit
// integers, two at a time). For bf16 magnitudes the integer order is the value order, and the inf / NaN patterns lie
// above every finite one.
typedef unsigned short r9k_u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t max_mag_bf16x2(uint32_t acc, uint32_t w) {
  const r9k_u16x2 a = __builtin_bit_cast(r9k_u16x2, acc), b = __builtin_bit_cast(r9k_u16x2, w & 0x7fff7fffu);
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(a, b));
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

// Chunk c of a row of nvec 16-byte chunks (nvec >= 1), zero past the row. The load always goes out, to an in-range
// chunk, and the zero is a select after it: a load under a branch is waited for inside that branch, which would
// serialise a lane's chunk loads instead of keeping them in flight together.
// NT: a non-temporal load, for passes that stream far more than the L2 holds and never read the row again.
template <bool NT = false>
__device__ __forceinline__ uint4 load_chunk_or_zero(const uint4* __restrict__ row, int c, int nvec) {
  const uint4* p = row + (c < nvec ? c : nvec - 1);
  uint4 t;
  if constexpr (NT) {
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    const u4v w = __builtin_nontemporal_load(reinterpret_cast<const u4v*>(p));
    t = make_uint4(w.x, w.y, w.z, w.w);
  } else {
    t = *p;
  }
  return c < nvec ? t : make_uint4(0u, 0u, 0u, 0u);
}

// bf16 halves of a packed 32-bit word as fp32.
__device__ __forceinline__ float lo16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Eight fp32 values times `inv` to e4m3 bytes (v[0] in the low byte of .x), f32_to_e4m3's bytes for each.
// V_CVT_PK_FP8_F32 (OCP e4m3 on gfx950, round to nearest even) gives them for every |x| <= 464, signed zeros and the
// subnormal grid included, and converts all eight; a product that is NaN or larger in magnitude (code sign | 0x7f,
// which the hardware need not produce) then has its byte replaced, in one short block shared by the eight (kept
// small because several kernels inline this routine once per row).
__device__ __forceinline__ uint2 pack8_e4m3(const float (&v)[8], float inv) {
  float x[8];
  bool ok = true;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    x[j] = v[j] * inv;
    ok = ok && fabsf(x[j]) <= 464.f;
  }
  uint32_t w[2];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int r = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * h], x[4 * h + 1], 0, false);
    w[h] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x[4 * h + 2], x[4 * h + 3], r, true);
  }
  if (__builtin_expect(!ok, 0)) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
      if (!(fabsf(x[j]) <= 464.f)) {
        const uint32_t code = ((__float_as_uint(x[j]) >> 24) & 0x80u) | 0x7fu;
        const int sh = 8 * (j & 3);
        w[j >> 2] = (w[j >> 2] & ~(0xffu << sh)) | (code << sh);
      }
    }
  }
  return make_uint2(w[0], w[1]);
}

// Eight packed bf16 values (one 16-byte chunk) times `inv` to e4m3 bytes.
__device__ __forceinline__ uint2 pack8_bf16_e4m3(uint4 v, float inv) {
  const float f[8] = {lo16(v.x), hi16(v.x), lo16(v.y), hi16(v.y), lo16(v.z), hi16(v.z), lo16(v.w), hi16(v.w)};
  return pack8_e4m3(f, inv);
}

// pack8_bf16_e4m3 for a chunk of a row whose largest magnitude amax is finite and inv = 448 / max(amax, 1e-12):
// every product then has |x * inv| <= 448 (1 + 2^-23) < 464, the range where V_CVT_PK_FP8_F32 alone gives
// f32_to_e4m3's bytes, so the out-of-range check is left out (same bytes as pack8_bf16_e4m3).
__device__ __forceinline__ uint2 pack8_bf16_e4m3_finite(uint4 v, float inv) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint32_t out[2];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int r = __builtin_amdgcn_cvt_pk_fp8_f32(lo16(w[2 * h]) * inv, hi16(w[2 * h]) * inv, 0, false);
    out[h] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(lo16(w[2 * h + 1]) * inv, hi16(w[2 * h + 1]) * inv, r, true);
  }
  return make_uint2(out[0], out[1]);
}

// silu(g) * u with g, u the stored bf16 values, evaluated as (g / (1 + exp(-g))) * u in fp32 with the hardware
// exponential (__expf, as the reference: kernels/r9k_moe_mxfp4a8.hip:526) and a reciprocal-multiply division
// (V_RCP_F32, 1 ulp; within 2 ulp of the reference's IEEE division, whose sequence is 10 instructions an element in a
// VALU-bound kernel). A code can move one step where the product sits within a few ulp of an e4m3 rounding point.
// The standalone SiLU kernel and the gate_up GEMM's fused epilogue both use this one definition.
__device__ __forceinline__ float silu_mul(float gv, float uv) {
  return gv * __builtin_amdgcn_rcpf(1.f + __expf(-gv)) * uv;
}

// One wave quantises one row of K bf16 values (K % 8 == 0, K <= 512 * RMAX, the row 16-byte aligned, the code row
// 8-byte aligned) to OCP e4m3 with a per-row scale:
//   amax = max(max_k |x_k|, 1e-12);  inv = 448 / amax;  q_k = e4m3_rne(x_k * inv);  s = amax / 448.
// Each lane keeps its 16-byte chunks (lane + 64 i) in registers, so the row is read once. The row maximum is taken
// on the bf16 magnitude bits (two values an instruction); a finite maximum is the float one exactly and lets every
// code skip the range check. A row holding inf or NaN takes the float maximum, which passes over NaN, and the checked
// conversion. quant_row_load / quant_row_finish are the two halves, for callers that issue the row's loads early.
template <int RMAX>
__device__ __forceinline__ void quant_row_load(const uint16_t* __restrict__ xrow, int K, int lane, uint4 (&v)[RMAX]) {
  const uint4* xr = reinterpret_cast<const uint4*>(xrow);
#pragma unroll
  for (int i = 0; i < RMAX; i++) v[i] = load_chunk_or_zero(xr, lane + i * WAVE, K / 8);
}

template <int RMAX>
__device__ __forceinline__ void quant_row_finish(const uint4 (&v)[RMAX], int K, uint8_t* __restrict__ qrow,
                                                 float* __restrict__ s_out, int lane) {
  const int nvec = K / 8;
  uint32_t mm = 0u;
#pragma unroll
  for (int i = 0; i < RMAX; i++) {
    mm = max_mag_bf16x2(mm, v[i].x);
    mm = max_mag_bf16x2(mm, v[i].y);
    mm = max_mag_bf16x2(mm, v[i].z);
    mm = max_mag_bf16x2(mm, v[i].w);
  }
  const uint32_t mb = wave_max_u32(max(mm & 0xffffu, mm >> 16));
  uint2* qr = reinterpret_cast<uint2*>(qrow);
  if (mb < 0x7f80u) {                                            // finite row (wave-uniform)
    const float amax = fmaxf(__uint_as_float(mb << 16), 1e-12f);
    const float inv = 448.f / amax;
    if (lane == 0) *s_out = amax / 448.f;
#pragma unroll
    for (int i = 0; i < RMAX; i++) {
      const int c = lane + i * WAVE;
      if (c < nvec) qr[c] = pack8_bf16_e4m3_finite(v[i], inv);
    }
    return;
  }
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < RMAX; i++) {
    const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
    for (int j = 0; j < 4; j++) m = fmaxf(m, fmaxf(fabsf(lo16(w[j])), fabsf(hi16(w[j]))));
  }
  const float amax = fmaxf(wave_max(m), 1e-12f);
  const float inv = 448.f / amax;
  if (lane == 0) *s_out = amax / 448.f;
#pragma unroll
  for (int i = 0; i < RMAX; i++) {
    const int c = lane + i * WAVE;
    if (c < nvec) qr[c] = pack8_bf16_e4m3(v[i], inv);
  }
}

// quant_row_load then quant_row_finish: the row's chunks, all in flight together, then the quant.
template <int RMAX>
__device__ __forceinline__ void quant_row_wave(const uint16_t* __restrict__ xrow, int K, uint8_t* __restrict__ qrow,
                                               float* __restrict__ s_out, int lane) {
  uint4 v[RMAX];
  quant_row_load<RMAX>(xrow, K, lane, v);
  quant_row_finish<RMAX>(v, K, qrow, s_out, lane);
}

// The two halves of silu_quant_chunks, for callers that convert several rows at once and interleave their wave
// reductions: silu_chunk_values gives a lane's products a[i][0..7] (chunk lane + 64 i) and their running max |a|;
// quant_chunks_write takes the row's reduced max and writes the codes, returning the row scale.
template <int R>
__device__ __forceinline__ float silu_chunk_values(const uint4 (&gv)[R], const uint4 (&uv)[R], float (&a)[R][8]) {
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < R; i++) {
    const uint32_t gw[4] = {gv[i].x, gv[i].y, gv[i].z, gv[i].w}, uw[4] = {uv[i].x, uv[i].y, uv[i].z, uv[i].w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      a[i][2 * j] = silu_mul(lo16(gw[j]), lo16(uw[j]));
      a[i][2 * j + 1] = silu_mul(hi16(gw[j]), hi16(uw[j]));
    }
#pragma unroll
    for (int j = 0; j < 8; j++) m = fmaxf(m, fabsf(a[i][j]));      // zero padding lanes give silu(0) * 0 = 0
  }
  return m;
}

template <int R>
__device__ __forceinline__ float quant_chunks_write(const float (&a)[R][8], float row_max, int nvec, uint8_t* qrow,
                                                    int lane) {
  const float amax = fmaxf(row_max, 1e-12f);
  const float inv = 448.f / amax;
  uint2* qr = reinterpret_cast<uint2*>(qrow);
#pragma unroll
  for (int i = 0; i < R; i++) {
    const int c = lane + i * WAVE;
    if (c < nvec) qr[c] = pack8_e4m3(a[i], inv);
  }
  return amax / 448.f;
}

// silu(gate) * up of one gate_up row held in registers (lane chunks c = lane + 64 i of 8 values: gv = gate, uv =
// up, zero past the row's nvec chunks) quantised to OCP e4m3 with a per-row scale, the rule of the per-token quant:
// amax = max(max |h|, 1e-12), inv = 448 / amax, q = e4m3(h * inv) written as 8-byte pieces at qrow + 8 c,
// s = amax / 448 returned to every lane. Every consumer of the gate_up output goes through these routines (the
// standalone SiLU kernel, the decode tail and the prefill down kernel), so their codes are the same bytes.
template <int R>
__device__ __forceinline__ float silu_quant_chunks(const uint4 (&gv)[R], const uint4 (&uv)[R], int nvec,
                                                   uint8_t* qrow, int lane) {
  float a[R][8];
  const float m = silu_chunk_values<R>(gv, uv, a);
  return quant_chunks_write<R>(a, wave_max(m), nvec, qrow, lane);
}

// Loads the lane chunks of one gate_up row for silu_quant_chunks (gate = the first I bf16 values, up = the next I;
// I % 8 == 0, I <= 512 * R, the row 16-byte aligned).
template <int R, bool NT = false>
__device__ __forceinline__ void load_gate_up_row(const uint16_t* __restrict__ grow, int I, int lane, uint4 (&gv)[R],
                                                 uint4 (&uv)[R]) {
  const int nvec = I / 8;
  const uint4* gr = reinterpret_cast<const uint4*>(grow);
  const uint4* ur = reinterpret_cast<const uint4*>(grow + I);
#pragma unroll
  for (int i = 0; i < R; i++) {
    const int c = lane + i * WAVE;
    gv[i] = load_chunk_or_zero<NT>(gr, c, nvec);
    uv[i] = load_chunk_or_zero<NT>(ur, c, nvec);
  }
}

// One wave turns one gate_up row into e4m3 codes (the code row 8-byte aligned) and returns its scale.
template <int R, bool NT = false>
__device__ __forceinline__ float silu_quant_row_wave(const uint16_t* __restrict__ grow, int I, uint8_t* qrow,
                                                     int lane) {
  uint4 gv[R], uv[R];
  load_gate_up_row<R, NT>(grow, I, lane, gv, uv);
  return silu_quant_chunks<R>(gv, uv, I / 8, qrow, lane);
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
