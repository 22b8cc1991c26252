// r9k_moe_decode.hip -- the tail of a decode-width MoE layer in one launch: SiLU-gating + fp8 re-quant of every
// routed row, the grouped down GEMM (MXFP4 x fp8, router weight in the epilogue) and the weighted top-k sum.
//
//   out[t, n] = bf16( sum_{j ascending} bf16( (sum_k aq[t*topk + j, k] * W2_e(t,j)[n, k]) * (as[t*topk+j] * tw[..]) )
//                     (+ shared[t, n]) )
//   aq, as    = per-row e4m3 quant of silu(gate) * up of the gate_up output row (silu_quant_row_wave)
//
// The reference runs this as three launches (r9k_silu_mul_quant_fp8, the down r9k_moe_mxfp4a8 and r9k_moe_sum:
// kernels/r9k_moe_mxfp4a8.hip:517-548, :469-482, kernels/r9k_moe_sum.hip:32-56); each of them is a few microseconds
// of launch and memory latency at decode widths, more than its work. Here the work is token-major: a workgroup owns
// one token and NC 16-column tiles of the output, with one wave per top-k slot j. Wave j
//   1. loads its routed row's expert id and router weight together with the row's gate_up values,
//   2. issues every weight load of its expert's NC column tiles over all of K (one memory round trip),
//   3. meanwhile turns its gate_up row into e4m3 codes in LDS (silu_quant_row_wave: the standalone SiLU kernel's
//      bytes),
//   4. runs the 16x16x128 scaled MFMAs (codes as the fp8 A operand, e2m1 weights as B with their e8m0 block exponent
//      as the B scale; every A row holds the same codes, row 0 of the result is used),
//   5. writes bf16(acc * (as * tw)) of its 16 NC columns to LDS,
// and after one barrier the workgroup sums the top-k values per column in slot order into one bf16 output.
// Nothing goes through HBM between the three steps, and no routing tables are read: the expert of each routed row
// comes from the router's ids. Rows of one expert shared by several tokens re-read that expert's weights (the
// workgroups of different tokens are independent), so the host uses this path only at small token counts.
//
// Numerics: step 3 is the standalone SiLU kernel's routine, the MFMA chain over K-tiles in ascending order is the
// single-wave down GEMM's (SK = 1, its launch shape for K < 1024), the epilogue is its bf16(acc * (As * tw)) and the
// sum is r9k_moe_sum's fp32 accumulation in slot order, so for K2 < 1024 the output equals the three-launch chain
// bit for bit. For longer K2 the down GEMM splits K over waves and sums partials, so the two agree to fp32 rounding.
#include "r9k_common.h"

#include <cstdlib>

namespace {

using namespace r9k;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int KT = 128;           // K per MFMA
constexpr int E8M0_ONE = 127;     // scale byte of 2^0
constexpr int MAX_TOPK = 16;      // waves of a workgroup (1024 threads)

// NC column tiles per workgroup, NKT K-tiles of 128 (K2 = I = 128 * NKT, all loads in flight at once), one wave per
// top-k slot, at most MW slots (the register budget: 8 slots leave 256 VGPRs a lane). LDS: codes [topk][I] then bf16
// down values [topk][NC * 16].
template <int NC, int NKT, int MW>
__global__ void __launch_bounds__(MW * WAVE) moe_down_sum_kernel(
    const uint16_t* __restrict__ gu, const int* __restrict__ ids, const float* __restrict__ tw,
    const uint8_t* __restrict__ Wq, const uint8_t* __restrict__ Ws, long wq_estride, long ws_estride,
    const uint16_t* __restrict__ shared, long ld_shared, uint16_t* __restrict__ out, long ld_out, int topk, int E,
    int N) {
  constexpr int I = NKT * KT;
  constexpr int R = I / (8 * WAVE);                          // 16-byte gate (and up) chunks per lane
  static_assert(I % (8 * WAVE) == 0, "whole lane chunks");
  extern __shared__ uint8_t lds[];
  const int t = blockIdx.y;
  const int j = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  const int g = lane >> 4, c = lane & 15;
  const int NT = N / 16;
  const int nt0 = blockIdx.x * NC;
  const size_t row = (size_t)t * topk + j;
  uint8_t* aq = lds + (size_t)j * I;
  uint16_t* dn = reinterpret_cast<uint16_t*>(lds + (size_t)topk * I);

  // one routed row a wave: the expert id is wave-uniform (readfirstlane makes that known, so a branch on it never
  // splits a wave and the MFMAs below always run under a full exec mask)
  const int e = __builtin_amdgcn_readfirstlane(ids[row]);
  const float w = tw[row];
  const bool live = e >= 0 && e < E;
  const uint8_t* __restrict__ We = Wq + (size_t)(live ? e : 0) * wq_estride;
  const uint8_t* __restrict__ Se = Ws + (size_t)(live ? e : 0) * ws_estride;
  u32x4 bf[NC][NKT];
  uint32_t sb[NC][NKT];
#pragma unroll
  for (int q = 0; q < NC; q++) {
    const int nt = min(nt0 + q, NT - 1);                     // a tile past N computes a copy, never stored
    const uint8_t* wt = We + (size_t)nt * (8 * I) + lane * 16;
    const uint8_t* st = Se + (size_t)nt * (16 * (I / 32)) + lane;
#pragma unroll
    for (int k = 0; k < NKT; k++) {
      bf[q][k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wt + k * 1024));
      sb[q][k] = __builtin_nontemporal_load(st + k * 64);
    }
  }
  const float as = silu_quant_row_wave<R>(gu + row * (2 * I), I, aq, lane);
  const float sc = as * w;                                    // the down GEMM's row scale, in its order
  // the codes were stored as 8-byte pieces by other lanes and are read below as 16-byte pieces: the barrier orders
  // the two for the compiler (different access types) and completes the stores
  __syncthreads();

  v4f acc[NC];
#pragma unroll
  for (int q = 0; q < NC; q++) acc[q] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < NKT; k++) {
    const uint4 lo = *reinterpret_cast<const uint4*>(aq + k * KT + 16 * g);
    const uint4 hi = *reinterpret_cast<const uint4*>(aq + k * KT + 64 + 16 * g);
    const v8i a = (v8i){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
#pragma unroll
    for (int q = 0; q < NC; q++) {
      const v8i b = (v8i){(int)bf[q][k].x, (int)bf[q][k].y, (int)bf[q][k].z, (int)bf[q][k].w, 0, 0, 0, 0};
      acc[q] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc[q], 0, 4, 0, E8M0_ONE, 0, (int)sb[q][k]);
    }
  }
  // C layout: lane holds column lane % 16, rows 4g .. 4g + 3. Every A row holds the same codes, so every row of C
  // is the same and all four lanes of a column store the same value: no branch, so the MFMAs can never be moved
  // under a partial exec mask
#pragma unroll
  for (int q = 0; q < NC; q++) dn[j * (NC * 16) + q * 16 + c] = live ? f2bf(acc[q][0] * sc) : (uint16_t)0;
  __syncthreads();
  const int tid = threadIdx.x;
  if (tid < NC * 16 && nt0 + tid / 16 < NT) {
    const int n = nt0 * 16 + tid;
    float v = 0.f;
    for (int jj = 0; jj < topk; jj++) v += bf2f(dn[jj * (NC * 16) + tid]);
    if (shared) v += bf2f(shared[(size_t)t * ld_shared + n]);
    out[(size_t)t * ld_out + n] = f2bf(v);
  }
}

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}

// Column tiles per workgroup: enough workgroups to spread one token's weight stream over the CUs at T = 1, fewer
// repeats of each token's SiLU prologue as T grows (every column workgroup of a token redoes it).
int pick_nc(int T, int NT, int NKT) {
  int nc = T <= 2 ? 1 : (T <= 8 ? 2 : 4);
  nc = env_int("R9K_DOWNSUM_NC", nc);
  if (NKT > 8) nc = 1;
  else if (NKT > 4 && nc > 2) nc = 2;
  while (nc > 1 && NT % nc) nc >>= 1;
  return nc;
}

}  // namespace

// No reference counterpart as one entry: the reference's r9k_silu_mul_quant_fp8 + down r9k_moe_mxfp4a8 (a_row_div 1,
// topk_w) + r9k_moe_sum (kernels/r9k_moe_mxfp4a8.hip:550, :631-638; kernels/r9k_moe_sum.hip:62) in one launch, for
// decode widths. gu bf16 [T * topk][2I] (the gate_up output, rows t * topk + j); ids int32 [T * topk] (the router's
// expert per routed row; ids outside [0, E) contribute 0); tw fp32 [T * topk]; wq / ws the down weights in the
// r9k_moe_mxfp4a8 layout (ws_estride bytes per expert); shared bf16 [T][N] with row stride ld_shared, or 0; out bf16
// [T][N] with row stride ld_out. Served: I % 128 == 0 and I <= 2048, N % 16 == 0, 1 <= topk <= 16; returns 2 (nothing
// launched) for other shapes, 0 on success, -3 bad argument, -6 launch error.
extern "C" int r9k_moe_down_sum(long gu, long ids, long tw, long wq, long ws, long ws_estride, long shared,
                                long ld_shared, long out, long ld_out, int T, int topk, int E, int I, int N,
                                long stream) {
  if (T <= 0) return 0;
  if (!gu || !ids || !tw || !wq || !ws || !out || E < 1 || N < 16) return -3;
  if (topk < 1 || topk > MAX_TOPK || I % KT || I < KT || I > 16 * KT || N % 16) return 2;
  if ((gu & 15) || (wq & 15)) return 2;
  if (T > 65535) return 2;
  const int NKT = I / KT, NT = N / 16;
  if (NKT != 4 && NKT != 8 && NKT != 16) return 2;
  int nc = pick_nc(T, NT, NKT);
  if (topk > 8 && NKT > 8) return 2;                         // 16 slots x 16 K-tiles: past the register budget
  if (topk > 8 && NKT > 4) nc = 1;
  const dim3 grid((NT + nc - 1) / nc, T), block(topk * WAVE);
  const size_t smem = (size_t)topk * I + (size_t)topk * nc * 16 * 2;
  const hipStream_t st = (hipStream_t)stream;
  const long wq_estride = (long)N * I / 2;
#define DS(NCV, NKTV, MWV)                                                                                         \
  if (nc == NCV && NKT == NKTV && topk <= MWV) {                                                                   \
    hipLaunchKernelGGL((moe_down_sum_kernel<NCV, NKTV, MWV>), grid, block, smem, st, (const uint16_t*)gu,          \
                       (const int*)ids, (const float*)tw, (const uint8_t*)wq, (const uint8_t*)ws, wq_estride,      \
                       ws_estride, (const uint16_t*)shared, ld_shared, (uint16_t*)out, ld_out, topk, E, N);        \
    return hipGetLastError() == hipSuccess ? 0 : -6;                                                               \
  }
  DS(1, 4, 8) DS(2, 4, 8) DS(4, 4, 8) DS(1, 8, 8) DS(2, 8, 8) DS(1, 16, 8)
  DS(1, 4, 16) DS(2, 4, 16) DS(4, 4, 16) DS(1, 8, 16)
#undef DS
  return 2;
}
