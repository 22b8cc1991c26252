// r9k_dense.hip -- the dense MXFP4 weight-only linear at decode widths (M <= 4 rows) in one launch: the per-token
// fp8 (e4m3) quant of the bf16 activations and the MXFP4 x fp8 GEMM.
//
//   out[m, n] = bf16( (sum_k q[m, k] * W[n, k]) * s[m] ),   q, s = the per-row quant of x (quant_row_wave)
//
// The reference runs it as r9k_quant_rows_fp8 then r9k_moe_mxfp4a8 over identity routing tables
// (r9700_vllm/ops.py:89-117; kernels/r9k_moe_mxfp4a8.hip:1683-1743 and :187-485). At decode widths the quant launch
// costs about as much as a third of the GEMM (its launch and memory latency), so here every workgroup quantises the
// M activation rows itself into LDS (each row read once from L2 per workgroup, M * K * 2 bytes, spread over all of
// its threads and issued ahead of its weight loads, which then overlap the quant), then runs the weight stream
// against the LDS codes.
//
// Work split: a workgroup owns NPW 16-column tiles (1 KB of codes + 64 exponent bytes per 128-K tile, the
// r9k_moe_mxfp4a8 weight layout), SK waves split the K-tiles in contiguous ranges, each wave issues the loads of up
// to U K-tiles at once (all of its range when it fits) and runs the 16x16x128 scaled MFMAs: activations as the fp8 A
// operand (rows m < M live, the other rows zero), weights as the fp4 B operand with their e8m0 exponent as the B
// scale. The SK partial tiles meet in LDS and are summed in wave order. With the entry's SK rule (the decode GEMM's:
// 4 waves from 8 K-tiles) the result equals the two-launch path's bit for bit.
#include "r9k_common.h"
#include "r9k_rowquant.h"

#include <cstdlib>

namespace {

using namespace r9k;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int KT = 128;
constexpr int E8M0_ONE = 127;
constexpr int MAXM = 16;          // activation rows: one MFMA M-tile
constexpr int MAXM_QA = 4;        // rows the one-launch entry serves (the quant holds them all in registers)
constexpr int APAD = 16;          // bytes of padding per LDS code row (row stride K + 16: no bank aliasing of rows)

// LDS: codes [M][K + APAD] (fp8), row scales [MAXM] fp32, partial tiles [SK][NPW][256] fp32 (sized by M, so small M
// leaves room for several workgroups a CU).
// DB: a wave's K range is exactly two batches of U K-tiles, and the second batch is issued right after the row
// quant (into a second register set) instead of after the first batch is consumed, so the wave's whole weight range
// is requested within the prologue, as a plain streaming read would request it. The MFMAs run in the same order.
template <int NPW, int SK, int U, int MG, bool DB = false>
__global__ void __launch_bounds__(WAVE * SK) dense_mxfp4_qa_kernel(
    const uint16_t* __restrict__ x, long ldx, const uint8_t* __restrict__ Wq, const uint8_t* __restrict__ Ws,
    uint16_t* __restrict__ out, long ldo, int M, int N, int K) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int lda = K + APAD;
  uint8_t* A = lds;
  float* s_row = reinterpret_cast<float*>(lds + (size_t)M * lda);
  float* red = s_row + MAXM;
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int g = lane >> 4, r = lane & 15;
  const int NT = N / 16, nkt = K / KT, KB = K / 32;

  const uint8_t* wtile[NPW];
  const uint8_t* stile[NPW];
#pragma unroll
  for (int j = 0; j < NPW; j++) {
    const int nt = min((int)blockIdx.x * NPW + j, NT - 1);     // a tile past N computes a copy, never stored
    wtile[j] = Wq + (size_t)nt * (size_t)(8 * K) + lane * 16;
    stile[j] = Ws + (size_t)nt * (size_t)(16 * KB) + lane;
  }
  const int kt0 = wave * nkt / SK, kt1 = (wave + 1) * nkt / SK;

  u32x4 bf[U][NPW], bf2[DB ? U : 1][NPW];
  uint32_t sb[U][NPW], sb2[DB ? U : 1][NPW];
  auto issue = [&](int kb, auto& bq, auto& sq) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = min(kb + u, kt1 - 1);
#pragma unroll
      for (int j = 0; j < NPW; j++) {
        bq[u][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wtile[j] + (size_t)k * 1024));
        sq[u][j] = __builtin_nontemporal_load(stile[j] + k * 64);
      }
    }
  };
  // the activation rows' reads (M <= MG), then the first batch of weight loads, then the rows' quant (whose latency
  // the weight loads overlap); with DB the second batch follows the quant
  {
    constexpr int T = WAVE * SK, XC = row_chunks<T>();
    const int nvec = K / 8;
    uint4 xv[MG][XC];
    load_row_group<T, MG, XC>(x, ldx, 0, M, nvec, tid, xv);
    issue(kt0, bf, sb);
    quant_row_group<T, MG, XC>(xv, 0, M, nvec, A, lda, s_row, red, tid);
  }
  if constexpr (DB) issue(kt0 + U, bf2, sb2);

  v4f acc[NPW];
#pragma unroll
  for (int j = 0; j < NPW; j++) acc[j] = (v4f){0.f, 0.f, 0.f, 0.f};
  const bool arow = r < M;
  const uint8_t* ar = A + (size_t)(arow ? r : 0) * lda + 16 * g;
  auto consume = [&](int kb, const auto& bq, const auto& sq) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = kb + u;
      if (k < kt1) {                                         // wave-uniform
        uint4 lo = *reinterpret_cast<const uint4*>(ar + k * KT);
        uint4 hi = *reinterpret_cast<const uint4*>(ar + k * KT + 64);
        if (!arow) lo = hi = make_uint4(0u, 0u, 0u, 0u);
        const v8i a = (v8i){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
#pragma unroll
        for (int j = 0; j < NPW; j++) {
          const v8i b = (v8i){(int)bq[u][j].x, (int)bq[u][j].y, (int)bq[u][j].z, (int)bq[u][j].w, 0, 0, 0, 0};
          acc[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc[j], 0, 4, 0, E8M0_ONE, 0, (int)sq[u][j]);
        }
      }
    }
  };
  if constexpr (DB) {
    consume(kt0, bf, sb);
    consume(kt0 + U, bf2, sb2);
  } else {
    for (int kb = kt0; kb < kt1; kb += U) {
      if (kb != kt0) issue(kb, bf, sb);
      consume(kb, bf, sb);
    }
  }

  // C layout: lane holds column r, rows 4g .. 4g + 3. The partial tiles always go through LDS (no branch on the
  // MFMA results, so the compiler cannot move the MFMAs under a partial exec mask), then are summed in wave order.
#pragma unroll
  for (int j = 0; j < NPW; j++) {
    float* t = red + (size_t)(wave * NPW + j) * 256;
#pragma unroll
    for (int q = 0; q < 4; q++) t[(4 * g + q) * 16 + r] = acc[j][q];
  }
  __syncthreads();
  constexpr int TOT = NPW * 256;
  for (int idx = tid; idx < TOT; idx += WAVE * SK) {
    const int col = idx & 15, m = (idx >> 4) & 15, j = idx >> 8;
    const int n = (blockIdx.x * NPW + j) * 16 + col;
    if (m >= M || n >= N) continue;
    float v = 0.f;
#pragma unroll
    for (int s = 0; s < SK; s++) v += red[(size_t)s * TOT + idx];
    out[(size_t)m * ldo + n] = f2bf(v * s_row[m]);
  }
}

// The same weight stream, K split over waves and partial-tile sum as dense_mxfp4_qa_kernel, from activations already
// quantised (r9k_quant_rows_fp8's codes q [M][K] and row scales s [M]; optional row weights tw [M], applied as the
// decode GEMM's epilogue does: v * (s * tw)) for up to 16 rows: no quant and no rows in registers, so the LDS holds
// only the partial tiles. Each wave loads its A fragments (row r = lane % 16, 2 x 16
// bytes a K-tile; M * K bytes in all, L2-resident) in the same batches as its weight tiles.
template <int NPW, int SK, int U>
__global__ void __launch_bounds__(WAVE * SK) dense_mxfp4_a8_kernel(
    const uint8_t* __restrict__ q, long ldq, const float* __restrict__ s, const float* __restrict__ tw,
    const uint8_t* __restrict__ Wq, const uint8_t* __restrict__ Ws, uint16_t* __restrict__ out, long ldo, int M, int N,
    int K) {
  __shared__ float red[SK * NPW * 256];
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int g = lane >> 4, r = lane & 15;
  const int NT = N / 16, nkt = K / KT, KB = K / 32;

  const uint8_t* wtile[NPW];
  const uint8_t* stile[NPW];
#pragma unroll
  for (int j = 0; j < NPW; j++) {
    const int nt = min((int)blockIdx.x * NPW + j, NT - 1);     // a tile past N computes a copy, never stored
    wtile[j] = Wq + (size_t)nt * (size_t)(8 * K) + lane * 16;
    stile[j] = Ws + (size_t)nt * (size_t)(16 * KB) + lane;
  }
  const int kt0 = wave * nkt / SK, kt1 = (wave + 1) * nkt / SK;
  const bool arow = r < M;
  const uint8_t* ar = q + (size_t)(arow ? r : 0) * ldq + 16 * g;

  u32x4 bf[U][NPW];
  uint32_t sb[U][NPW];
  uint4 alo[U], ahi[U];
  auto issue = [&](int kb) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = min(kb + u, kt1 - 1);
#pragma unroll
      for (int j = 0; j < NPW; j++) {
        bf[u][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wtile[j] + (size_t)k * 1024));
        sb[u][j] = __builtin_nontemporal_load(stile[j] + k * 64);
      }
      alo[u] = *reinterpret_cast<const uint4*>(ar + k * KT);
      ahi[u] = *reinterpret_cast<const uint4*>(ar + k * KT + 64);
    }
  };

  v4f acc[NPW];
#pragma unroll
  for (int j = 0; j < NPW; j++) acc[j] = (v4f){0.f, 0.f, 0.f, 0.f};
  for (int kb = kt0; kb < kt1; kb += U) {
    issue(kb);
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = kb + u;
      if (k < kt1) {                                         // wave-uniform
        uint4 lo = alo[u], hi = ahi[u];
        if (!arow) lo = hi = make_uint4(0u, 0u, 0u, 0u);
        const v8i a = (v8i){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
#pragma unroll
        for (int j = 0; j < NPW; j++) {
          const v8i b = (v8i){(int)bf[u][j].x, (int)bf[u][j].y, (int)bf[u][j].z, (int)bf[u][j].w, 0, 0, 0, 0};
          acc[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc[j], 0, 4, 0, E8M0_ONE, 0, (int)sb[u][j]);
        }
      }
    }
  }

  // the partial tiles through LDS, summed in wave order (as dense_mxfp4_qa_kernel)
#pragma unroll
  for (int j = 0; j < NPW; j++) {
    float* t = red + (size_t)(wave * NPW + j) * 256;
#pragma unroll
    for (int qq = 0; qq < 4; qq++) t[(4 * g + qq) * 16 + r] = acc[j][qq];
  }
  __syncthreads();
  constexpr int TOT = NPW * 256;
  for (int idx = tid; idx < TOT; idx += WAVE * SK) {
    const int col = idx & 15, m = (idx >> 4) & 15, j = idx >> 8;
    const int n = (blockIdx.x * NPW + j) * 16 + col;
    if (m >= M || n >= N) continue;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < SK; w++) v += red[(size_t)w * TOT + idx];
    float sc = s[m];
    if (tw) sc *= tw[m];
    out[(size_t)m * ldo + n] = f2bf(v * sc);
  }
}

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}

}  // namespace

// No counterpart as one entry in the reference: r9k_quant_rows_fp8 + r9k_moe_mxfp4a8 over identity tables
// (r9700_vllm/ops.py:89-117 calls them back to back) in one launch, for M <= 4 rows. x bf16 [M][K] (row stride
// ldx elements, rows 16-byte aligned); wq / ws one expert's weights in the r9k_moe_mxfp4a8 layout (N columns, K);
// out bf16 [M][N] (row stride ldo). Served: 1 <= M <= 4, K % 128 == 0, K <= 8192, N % 16 == 0; 2 (nothing launched)
// otherwise. 0, -3 bad argument, -6 launch error. The K split (SK waves) follows the decode GEMM's rule, so the
// output equals r9k_quant_rows_fp8 + r9k_moe_mxfp4a8's bit for bit.
extern "C" int r9k_dense_mxfp4_qa(long x, long ldx, long wq, long ws, long out, long ldo, int M, int N, int K,
                                  long stream) {
  if (M <= 0) return 0;
  if (!x || !wq || !ws || !out || N <= 0 || K <= 0) return -3;
  if (M > MAXM_QA || K % KT || K > 8192 || N % 16 || (x & 15) || (ldx & 7) || (wq & 15)) return 2;
  const int nkt = K / KT, NT = N / 16;
  // one 16-column tile a workgroup at M = 1 (every workgroup of config 4 resident at once), two from M = 2
  // (measured at config 4: M = 1 12.2 us with two tiles, 10.7 us with one; M = 2 13.8 us with one, 12.9 us with two)
  const int NPW = env_int("R9K_DENSE_NPW", (NT >= 2 && M >= 2) ? 2 : 1);
  const int SK = env_int("R9K_DENSE_SK", nkt >= 8 ? 4 : 1);
  if (SK != 1 && SK != 4) return 2;
  if (K / 8 > (SK == 4 ? row_chunks<256>() * 256 : row_chunks<64>() * 64)) return 2;   // chunks a thread holds
  const int per = (nkt + SK - 1) / SK;
  // loads in flight a wave: its whole K range up to 5 K-tiles, else two batches (all of a 10-tile range at once
  // needs ~165 VGPRs, two waves a SIMD, and 544 workgroups of config 4 no longer fit the chip in one round:
  // measured 20.2 us against 14.2 us in two batches of 5)
  const int U = env_int("R9K_DENSE_U", per <= 4 ? 4 : (per <= 5 ? 5 : (per <= 8 ? 4 : (per <= 10 ? 5 : 8))));
  const int MG = M == 1 ? 1 : (M == 2 ? 2 : 4);
  // both batches of a two-batch K range issued in the prologue (R9K_DENSE_DB=0: one batch after the other)
  static const bool db_on = env_int("R9K_DENSE_DB", 1) != 0;
  const bool DB = db_on && per == 2 * U && SK == 4 && U == 5 && ((NPW == 1 && MG == 1) || (NPW == 2 && MG == 2));
  const size_t smem = (size_t)M * (K + APAD) + MAXM * sizeof(float) + (size_t)SK * NPW * 256 * sizeof(float);
  const dim3 grid((NT + NPW - 1) / NPW), block(WAVE * SK);
  const hipStream_t st = (hipStream_t)stream;
#define DQB(NPWv, MGv)                                                                                             \
  if (DB && NPW == NPWv && MG == MGv) {                                                                            \
    static const hipError_t a = hipFuncSetAttribute(                                                               \
        reinterpret_cast<const void*>(dense_mxfp4_qa_kernel<NPWv, 4, 5, MGv, true>),                               \
        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);                                                    \
    if (a != hipSuccess) return -6;                                                                                \
    hipLaunchKernelGGL((dense_mxfp4_qa_kernel<NPWv, 4, 5, MGv, true>), grid, block, smem, st, (const uint16_t*)x,  \
                       ldx, (const uint8_t*)wq, (const uint8_t*)ws, (uint16_t*)out, ldo, M, N, K);                 \
    return hipGetLastError() == hipSuccess ? 0 : -6;                                                               \
  }
  DQB(1, 1) DQB(2, 2)
#undef DQB
#define DQ(NPWv, SKv, Uv, MGv)                                                                                     \
  if (NPW == NPWv && SK == SKv && U == Uv && MG == MGv) {                                                          \
    static const hipError_t a = hipFuncSetAttribute(                                                               \
        reinterpret_cast<const void*>(dense_mxfp4_qa_kernel<NPWv, SKv, Uv, MGv>),                                  \
        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);                                                    \
    if (a != hipSuccess) return -6;                                                                                \
    hipLaunchKernelGGL((dense_mxfp4_qa_kernel<NPWv, SKv, Uv, MGv>), grid, block, smem, st, (const uint16_t*)x,     \
                       ldx, (const uint8_t*)wq, (const uint8_t*)ws, (uint16_t*)out, ldo, M, N, K);                 \
    return hipGetLastError() == hipSuccess ? 0 : -6;                                                               \
  }
#define DQM(NPWv, SKv, Uv) DQ(NPWv, SKv, Uv, 1) DQ(NPWv, SKv, Uv, 2) DQ(NPWv, SKv, Uv, 4)
#define DQU(NPWv, SKv) DQM(NPWv, SKv, 4) DQM(NPWv, SKv, 5) DQM(NPWv, SKv, 8) DQM(NPWv, SKv, 10)
  DQU(1, 1) DQU(2, 1) DQU(1, 4) DQU(2, 4)
#undef DQU
#undef DQM
#undef DQ
  return 2;
}

// No counterpart as one entry in the reference: the GEMM half of r9k_quant_rows_fp8 + r9k_moe_mxfp4a8 over identity
// tables (r9700_vllm/ops.py:89-117) for 1 <= M <= 16 pre-quantised rows, on the dense kernel's weight stream. q fp8
// [M][K] (row stride ldq bytes, rows 16-byte aligned), s fp32 [M], tw fp32 [M] row weights or 0 (the decode GEMM's
// topk_w); wq / ws one expert in the r9k_moe_mxfp4a8 layout; out bf16 [M][N] (row stride ldo). Served: 1 <= M <= 16, K % 128 == 0, N % 16 == 0; 2 (nothing launched) otherwise.
// 0, -3 bad argument, -6 launch error. Same K split as r9k_dense_mxfp4_qa, so the same bits as r9k_moe_mxfp4a8.
extern "C" int r9k_dense_mxfp4_a8(long q, long ldq, long s, long tw, long wq, long ws, long out, long ldo, int M,
                                  int N, int K, long stream) {
  if (M <= 0) return 0;
  if (!q || !s || !wq || !ws || !out || N <= 0 || K <= 0) return -3;
  if (M > MAXM || K % KT || N % 16 || (q & 15) || (ldq & 15) || (wq & 15)) return 2;
  const int nkt = K / KT, NT = N / 16;
  // one 16-column tile a workgroup up to 8 rows, two above (each workgroup reads all M rows' codes from L2, so more
  // rows favour more columns a workgroup). Config 4 GEMM (quant launch excluded): M = 4 12.1 us (NPW 1) / 13.2 (2),
  // M = 8 13.6 / 13.6, M = 16 18.3 / 16.7; 5 K-tiles a batch beat 4, 8 and 10 at every M.
  const int NPW = env_int("R9K_DENSE_A8_NPW", M > 8 ? 2 : 1);
  const int SK = nkt >= 8 ? 4 : 1;
  const int per = (nkt + SK - 1) / SK;
  const int U = env_int("R9K_DENSE_A8_U", per <= 4 ? 4 : (per <= 5 ? 5 : (per <= 8 ? 4 : (per <= 10 ? 5 : 8))));
  const dim3 grid((NT + NPW - 1) / NPW), block(WAVE * SK);
  const hipStream_t st = (hipStream_t)stream;
#define DA(NPWv, SKv, Uv)                                                                                          \
  if (NPW == NPWv && SK == SKv && U == Uv) {                                                                       \
    hipLaunchKernelGGL((dense_mxfp4_a8_kernel<NPWv, SKv, Uv>), grid, block, 0, st, (const uint8_t*)q, ldq,         \
                       (const float*)s, (const float*)tw, (const uint8_t*)wq, (const uint8_t*)ws, (uint16_t*)out,  \
                       ldo, M, N, K);                                                                              \
    return hipGetLastError() == hipSuccess ? 0 : -6;                                                               \
  }
#define DAU(NPWv, SKv) DA(NPWv, SKv, 4) DA(NPWv, SKv, 5) DA(NPWv, SKv, 8) DA(NPWv, SKv, 10)
  DAU(1, 1) DAU(2, 1) DAU(1, 4) DAU(2, 4)
#undef DAU
#undef DA
  return 2;
}
