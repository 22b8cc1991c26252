// r9k_moe_nvfp4.hip -- grouped (MoE) native-NVFP4-weight x fp8-activation GEMM for gfx950, routed through the
// moe_align_block_size tables (decode family: 16 * MT-row blocks).
//
//   out[r, n] = bf16( (sum_k A_q[r / a_row_div, k] * e2m1[n, k] * s16[n, k / 16]) * (Wg[n] * As[r / a_row_div]
//                     (* topk_w[r])) )
//
// with s16 the e4m3 scale of each 16-element group and Wg the fp32 per-row global multiplier: the checkpoint's NVFP4
// weight, exact, accumulated in fp32. Reference: kernels/r9k_moe_mxfp4a8.hip:89-96 and 300-340 (NVFP4 weight math),
// :469-482 (epilogue order), :641-647 (entry).
//
// The scaled MFMA applies only power-of-two (e8m0) block scales, and the fp4 -> fp16 / bf16 conversions apply only
// the exponent of their scale operand (both measured on gfx950), so an e4m3 scale rides on neither alone. Here each
// group's scale s16 = 2^E * m (m in [1, 2), the e4m3 mantissa) is applied in two exact steps while the weights are
// widened: V_CVT_SCALEF32_PK_F16_FP4 with s16 as its scale gives e2m1 * 2^E, and one packed fp16 multiply by m gives
// e2m1 * s16 (at most 6 significant bits and within [2^-10, 2688]: exact in fp16). The fp8 activations widen to fp16
// exactly (V_CVT_SCALEF32_PK_F16_FP8, scale 1), and V_MFMA_F32_16X16X32_F16 accumulates the exact products in fp32
// -- no per-group rescaling of partial sums. A zero scale takes conversion scale 1 and m = 0.
// Operand layout of the instruction: A lane l holds row l % 16 and 8 K values, B lane l column l % 16 and the same 8
// K values, lane group g = l / 16 taking instruction K 8g .. 8g + 7; C lane l holds column l % 16, rows 4g .. 4g + 3.
// Step s (0..3) of a 128-wide K-tile gives lane group g the K values 32g + 8s .. + 7, so over the tile lane group g
// covers the 32 contiguous K values 32g .. 32g + 31 (groups 2g and 2g + 1): two 16-byte activation loads a row.
//
// Weight layout (per expert, produced by kernels/moe.py prepare_nvfp4_weights), nkt = ceil(K / 128):
//   codes  : N/16 column tiles of nkt K-tiles of 1 KB. Lane l = g * 16 + c of K-tile kt holds the 16 checkpoint bytes
//            W[16 nt + c, kt * 64 + 16 g .. + 16] at l * 16 (the MXFP4 fragment order), dword s feeding step s.
//   scales : N/16 column tiles of nkt K-tiles of 128 bytes. Lane l's 2 bytes at l * 2 are the e4m3 scales of groups
//            kt * 8 + 2g and kt * 8 + 2g + 1 of column c.
//   A partial last K-tile (K % 128 = 16 G) is stored whole, codes and scales zero past group G.
//   Wg     : fp32 [N] (wg_estride floats per expert).
#include "r9k_common.h"
#include "r9k_dma.h"
#include "r9k_rowquant.h"

namespace {

using namespace r9k;

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int NV_KT = 128;          // K per tile (8 groups)
constexpr int NV_G = 16;            // NVFP4 group

__device__ __forceinline__ u32x4 ld16_nt(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ uint32_t ld2_nt(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(p));
}

// The two ways one e4m3 group scale enters the widening: the conversion scale (only its exponent is used) and the
// packed fp16 mantissa factor.
struct GroupScale {
  float cvt;
  h2 m;
};
__device__ __forceinline__ GroupScale group_scale(uint32_t byte) {
  const float sf = __builtin_amdgcn_cvt_f32_fp8((int)byte, 0);
  const float m = __uint_as_float((__float_as_uint(sf) & 0x807fffffu) | 0x3f800000u);
  const bool z = sf == 0.f;
  const float mz = z ? 0.f : m;
  return {z ? 1.f : sf, (h2){(_Float16)mz, (_Float16)mz}};
}

// 8 e2m1 codes (one dword, low nibble first) -> e2m1 * s16 as 8 fp16, exact
__device__ __forceinline__ h8 e2m1x8_f16(uint32_t w, GroupScale gs) {
  const h2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, gs.cvt, 0) * gs.m;
  const h2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, gs.cvt, 1) * gs.m;
  const h2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, gs.cvt, 2) * gs.m;
  const h2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, gs.cvt, 3) * gs.m;
  return (h8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// 8 e4m3 codes (two dwords) -> 8 fp16, exact
__device__ __forceinline__ h8 e4m3x8_f16(uint32_t lo, uint32_t hi) {
  const h2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)lo, 1.0f, false);
  const h2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)lo, 1.0f, true);
  const h2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)hi, 1.0f, false);
  const h2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)hi, 1.0f, true);
  return (h8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// One workgroup: 16 * MT routed rows x NPW column tiles; SK waves split the K-tiles (SK > 1: partial tiles summed
// through LDS in wave order). Each wave walks its K range in batches of U K-tiles, all loads of a batch issued
// before its MFMAs; addresses past K are clamped and their groups skipped (uniform per tile).
template <int MT, int NPW, int SK, int U>
__global__ void __launch_bounds__(WAVE * SK) moe_nvfp4_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint8_t* __restrict__ Ws, const float* __restrict__ Wg, uint16_t* __restrict__ C,
    const int* __restrict__ sorted_ids, const int* __restrict__ expert_ids, const int* __restrict__ ntpp,
    const float* __restrict__ topk_w, long wq_estride, long ws_estride, long wg_estride, int numel, int a_row_div,
    int K, int N, int blk, int subs) {
  constexpr int BLK = 16 * MT;
  extern __shared__ float red[];

  const int rb = blockIdx.y / subs, sub = blockIdx.y - rb * subs;
  const int row0 = rb * blk + sub * BLK;
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int g = lane >> 4, c = lane & 15;
  const int np = ntpp[0];
  const int e = expert_ids[rb];
  const int first = sorted_ids[rb * blk];
  int fr_in[MT];
#pragma unroll
  for (int i = 0; i < MT; i++) fr_in[i] = sorted_ids[row0 + i * 16 + c];
  if (rb * blk >= np || e < 0) return;
  if (first < 0 || first >= numel || __shfl(fr_in[0], 0, WAVE) >= numel) return;   // padding: end of a block
  const int NT = N / 16;
  const int nkt = (K + NV_KT - 1) / NV_KT;
  const int kvalid_g = K - 32 * g;                          // K values of lane group g's run in tile kt: minus kt*128

  size_t arow[MT];
  float ras[MT], rtw[MT];                                  // row r of M-tile i (lane c's row): As, topk weight
#pragma unroll
  for (int i = 0; i < MT; i++) {
    int fr = fr_in[i];
    if (fr >= numel || fr < 0) fr = first;
    arow[i] = (size_t)(fr / a_row_div) * K;
    ras[i] = As[fr / a_row_div];
    rtw[i] = topk_w ? topk_w[fr] : 1.f;
  }
  const uint8_t* __restrict__ We = Wq + (size_t)e * wq_estride;
  const uint8_t* __restrict__ Se = Ws + (size_t)e * ws_estride;
  const float* __restrict__ Ge = Wg + (size_t)e * wg_estride;
  const uint8_t* wtile[NPW];
  const uint8_t* stile[NPW];
#pragma unroll
  for (int j = 0; j < NPW; j++) {
    int nt = (int)blockIdx.x * NPW + j;
    nt = nt < NT ? nt : NT - 1;                            // out-of-range tiles compute a copy, never stored
    wtile[j] = We + (size_t)nt * nkt * 1024;
    stile[j] = Se + (size_t)nt * nkt * 128;
  }

  v4f acc[NPW][MT];
#pragma unroll
  for (int j = 0; j < NPW; j++)
#pragma unroll
    for (int i = 0; i < MT; i++) acc[j][i] = (v4f){0.f, 0.f, 0.f, 0.f};

  const int kt0 = wave * nkt / SK, kt1 = (wave + 1) * nkt / SK;
  for (int kt = kt0; kt < kt1; kt += U) {
    u32x4 bw[U][NPW];
    uint32_t sw[U][NPW];
    uint4 alo[U][MT], ahi[U][MT];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = min(kt + u, kt1 - 1);
      // lane group g's 32 K values of this tile: 32, 16 (K % 32 == 16 at the end) or none; a missing half loads a
      // valid address and is zeroed below
      const int kv = kvalid_g - k * NV_KT;
      const int olo = kv >= 16 ? k * NV_KT + 32 * g : 0, ohi = kv >= 32 ? k * NV_KT + 32 * g + 16 : 0;
#pragma unroll
      for (int j = 0; j < NPW; j++) {
        bw[u][j] = ld16_nt(wtile[j] + (size_t)k * 1024 + lane * 16);
        sw[u][j] = ld2_nt(stile[j] + (size_t)k * 128 + lane * 2);
      }
#pragma unroll
      for (int i = 0; i < MT; i++) {
        alo[u][i] = *reinterpret_cast<const uint4*>(A + arow[i] + olo);
        ahi[u][i] = *reinterpret_cast<const uint4*>(A + arow[i] + ohi);
      }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = kt + u;
      if (k < kt1) {
        const int kv = kvalid_g - k * NV_KT;
        const bool lo_ok = kv >= 16, hi_ok = kv >= 32;
        h8 a[MT][4];
#pragma unroll
        for (int i = 0; i < MT; i++) {
          const uint4 l = lo_ok ? alo[u][i] : make_uint4(0u, 0u, 0u, 0u);
          const uint4 h = hi_ok ? ahi[u][i] : make_uint4(0u, 0u, 0u, 0u);
          a[i][0] = e4m3x8_f16(l.x, l.y);
          a[i][1] = e4m3x8_f16(l.z, l.w);
          a[i][2] = e4m3x8_f16(h.x, h.y);
          a[i][3] = e4m3x8_f16(h.z, h.w);
        }
#pragma unroll
        for (int j = 0; j < NPW; j++) {
          const GroupScale s0 = group_scale(sw[u][j] & 0xffu), s1 = group_scale((sw[u][j] >> 8) & 0xffu);
#pragma unroll
          for (int st = 0; st < 4; st++) {
            const h8 b = e2m1x8_f16(bw[u][j][st], st < 2 ? s0 : s1);
#pragma unroll
            for (int i = 0; i < MT; i++) acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i][st], b, acc[j][i], 0, 0, 0);
          }
        }
      }
    }
  }

  if constexpr (SK == 1) {
    // lane holds column c of each tile, rows 4g .. 4g + 3; row factors come from the lanes that loaded them
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int fr = __shfl(fr_in[i], 4 * g + q, WAVE);
        const float as_ = __shfl(ras[i], 4 * g + q, WAVE), tw = __shfl(rtw[i], 4 * g + q, WAVE);
        if (fr < 0 || fr >= numel) continue;
#pragma unroll
        for (int j = 0; j < NPW; j++) {
          const int n = (blockIdx.x * NPW + j) * 16 + c;
          if (n < N) {
            float sc = Ge[n] * as_;
            if (topk_w) sc *= tw;
            C[(size_t)fr * N + n] = f2bf(acc[j][i][q] * sc);
          }
        }
      }
  } else {
    __shared__ int s_fr[MT * 16];
    __shared__ float s_as[MT * 16], s_tw[MT * 16];
    if (wave == 0 && g == 0) {
#pragma unroll
      for (int i = 0; i < MT; i++) {
        s_fr[i * 16 + c] = fr_in[i];
        s_as[i * 16 + c] = ras[i];
        s_tw[i * 16 + c] = rtw[i];
      }
    }
#pragma unroll
    for (int j = 0; j < NPW; j++)
#pragma unroll
      for (int i = 0; i < MT; i++) {
        float* t = red + (size_t)((wave * NPW + j) * MT + i) * 256;
#pragma unroll
        for (int q = 0; q < 4; q++) t[(4 * g + q) * 16 + c] = acc[j][i][q];
      }
    __syncthreads();
    constexpr int TOT = NPW * MT * 256;
    for (int idx = tid; idx < TOT; idx += WAVE * SK) {
      const int col = idx & 15, row = (idx >> 4) & 15, ti = idx >> 8;   // ti = j * MT + i
      const int j = ti / MT, i = ti - j * MT;
      const int n = (blockIdx.x * NPW + j) * 16 + col;
      if (n >= N) continue;
      const int fr = s_fr[i * 16 + row];
      if (fr < 0 || fr >= numel) continue;
      float v = 0.f;
#pragma unroll
      for (int s = 0; s < SK; s++) v += red[(size_t)s * TOT + idx];
      float sc = Ge[n] * s_as[i * 16 + row];
      if (topk_w) sc *= s_tw[i * 16 + row];
      C[(size_t)fr * N + n] = f2bf(v * sc);
    }
  }
}

struct NvPick { int NPW, SK, U; };

// Launch shape from the host-known shape: two column tiles a workgroup (one for a dense linear of up to 8 rows); K
// split over SK waves for long K; each wave issues its K range in as few load batches as 4 K-tiles a batch allow (5
// for a dense linear of more than 8 rows).
NvPick nv_pick(int N, int K, int max_blocks, int rows) {
  const int nkt = (K + NV_KT - 1) / NV_KT;
  const int NT = N / 16;
  const int NPW = NT >= 2 ? 2 : 1;
  const long tiles = (long)max_blocks * ((NT + NPW - 1) / NPW);
  const int SK = nkt >= 8 ? (tiles >= 12288 ? 2 : 4) : 1;
  const int per = (nkt + SK - 1) / SK;
  int U = per >= 4 ? 4 : (per >= 2 ? 2 : 1);
  int npw = NPW;
  if (max_blocks <= 2 && SK == 4 && per >= 5) {
    // at most two routing blocks (a dense linear at decode widths: moe_gemm sizes the grid at ceil(numel / 16) +
    // min(numel, E) blocks): one column tile a workgroup up to 8 rows, two and 5-tile
    // batches above (config 4, [17408, 5120], quant + GEMM: M = 1 19.6 -> 18.4 us, M = 4 19.5 -> 18.8, M = 16
    // 23.6 -> 22.8; the K split is unchanged, so the bits are too)
    npw = rows > 8 ? 2 : 1;
    U = rows > 8 ? 5 : 4;
  }
  return {npw, SK, U};
}

template <int MT, int NPW, int SK, int U>
void nv_launch(dim3 grid, hipStream_t st, long a, long as, long wq, long ws, long wg, long c, long sorted_ids,
               long expert_ids, long ntpp, long topk_w, long wq_estride, long ws_estride, long wg_estride, int numel,
               int a_row_div, int K, int N, int blk, int subs) {
  const size_t smem = SK > 1 ? (size_t)SK * NPW * MT * 256 * sizeof(float) : 0;
  hipLaunchKernelGGL((moe_nvfp4_kernel<MT, NPW, SK, U>), grid, dim3(WAVE * SK), smem, st, (const uint8_t*)a,
                     (const float*)as, (const uint8_t*)wq, (const uint8_t*)ws, (const float*)wg, (uint16_t*)c,
                     (const int*)sorted_ids, (const int*)expert_ids, (const int*)ntpp, (const float*)topk_w,
                     wq_estride, ws_estride, wg_estride, numel, a_row_div, K, N, blk, subs);
}

// ------------------------------------------------------------------------------------------ prefill (tiles of 128)
// Routed rows in blocks of 128 (a routing block of 128 or 256 rows covered by 1 or 2 workgroups along grid.y) x 128
// output columns per workgroup; 4 waves in 2 x 2, each 64 rows x 64 columns = 4 x 4 tiles of the fp16 MFMA above.
// K runs in 128-wide tiles through a ring of three LDS stages (activations 16 KB, codes 8 KB, scales 1 KB) filled by
// direct global -> LDS DMA two K-tiles ahead of the MFMAs (every wave issues the same 7 DMA instructions a stage, so
// the waits are fixed vmcnt counts; no compiler-tracked load sits in the loop). Each wave widens its 4 column tiles'
// weights once per K-tile (codes and scales from LDS, as in the decode kernel) and reuses them over its 4 row tiles;
// the activation rows are widened per row tile. Activation row pieces sit XOR-swizzled (16-byte piece p of row r at
// position p ^ (r & 7)) so the 16 rows a fragment read touches land in different banks: the DMA lane that fills
// position p of row r fetches piece p ^ (r & 7). Past K (a partial last K-tile) an activation piece is fetched from
// the row's last valid piece; the weights' codes and scales there are zero, so those products are exact zeros.
constexpr int PV_BM = 128, PV_BN = 128, PV_THREADS = 256;
constexpr int PV_NS = 3;           // LDS stages
constexpr int PV_DMA = 7;          // DMA instructions per wave and stage: 4 activation, 2 code, 1 scale

struct PvStage {
  uint8_t a[PV_BM * NV_KT];        // fp8 activations, row-major, swizzled 16-byte pieces
  uint8_t b[8 * 1024];             // codes of the 8 column tiles, the global layout's K-tile
  uint8_t s[8 * 128];              // their scales
};
constexpr size_t PV_SMEM = PV_NS * sizeof(PvStage) + PV_BM * (sizeof(int) + 2 * sizeof(float));

__global__ void __launch_bounds__(PV_THREADS, 2) nvfp4_prefill_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint8_t* __restrict__ Ws, const float* __restrict__ Wg, uint16_t* __restrict__ C,
    const int* __restrict__ sorted_ids, const int* __restrict__ expert_ids, const int* __restrict__ ntpp,
    const float* __restrict__ topk_w, long wq_estride, long ws_estride, long wg_estride, int numel, int a_row_div,
    int K, int N, int blk, int subs) {
  extern __shared__ __align__(16) uint8_t pv_smem[];
  PvStage* st = reinterpret_cast<PvStage*>(pv_smem);
  int* s_fr = reinterpret_cast<int*>(pv_smem + PV_NS * sizeof(PvStage));
  float* s_as = reinterpret_cast<float*>(s_fr + PV_BM);         // As of each tile row (read once, before the loop)
  float* s_tw = s_as + PV_BM;                                  // topk_w of each tile row
  const int rb = blockIdx.y / subs, sub = blockIdx.y - rb * subs;
  const int row0 = rb * blk + sub * PV_BM;
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int g = lane >> 4, c = lane & 15, wm = wave >> 1, wn = wave & 1;
  const int np = ntpp[0];
  const int e = expert_ids[rb];
  const int first = sorted_ids[row0];
  if (rb * blk >= np || e < 0 || first < 0 || first >= numel) return;     // uniform: a dead block or padding
  if (tid < PV_BM) {
    const int fr = sorted_ids[row0 + tid];
    s_fr[tid] = fr;
    const bool live = fr >= 0 && fr < numel;
    s_as[tid] = live ? As[fr / a_row_div] : 0.f;
    s_tw[tid] = live && topk_w ? topk_w[fr] : 1.f;
  }
  __syncthreads();
  const int NT = N / 16, nkt = (K + NV_KT - 1) / NV_KT;
  const int nt0 = blockIdx.x * (PV_BN / 16);
  const uint8_t* We = uniform_ptr(Wq + (size_t)e * wq_estride);
  const uint8_t* Se = uniform_ptr(Ws + (size_t)e * ws_estride);
  const float* __restrict__ Ge = Wg + (size_t)e * wg_estride;

  // DMA sources (32-bit offsets from uniform bases; the host keeps A and one expert's codes below 4 GiB).
  // Activations: instruction i of wave w fills LDS pieces q = (4 i + w) * 64 + lane, i.e. row r = 32 i + 8 w + lane / 8
  // at position lane % 8, which holds the row's piece (lane % 8) ^ (r & 7) = (lane % 8) ^ (lane / 8).
  const int gp16 = ((lane & 7) ^ (lane >> 3)) * 16;
  uint32_t arow[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    int f = s_fr[32 * i + 8 * wave + (lane >> 3)];
    f = (f < 0 || f >= numel) ? first : f;                     // padding rows load a valid row, never stored
    arow[i] = (uint32_t)(f / a_row_div) * (uint32_t)K;
  }
  // codes: instruction i of wave w fills column tile t = 4 i + w (1 KB); scales: wave w's dword lanes fill tiles
  // 2 w and 2 w + 1 (128 bytes each)
  uint32_t boff[2];
#pragma unroll
  for (int i = 0; i < 2; i++) boff[i] = (uint32_t)min(nt0 + 4 * i + wave, NT - 1) * (uint32_t)(nkt * 1024) + lane * 16;
  const uint32_t soff = (uint32_t)min(nt0 + (tid >> 5), NT - 1) * (uint32_t)(nkt * 128) + (tid & 31) * 4;
  const uint32_t la0 = lds_addr(&st[0].a[wave * 1024]);
  const uint32_t lb0 = lds_addr(&st[0].b[wave * 1024]);
  const uint32_t ls0 = lds_addr(&st[0].s[wave * 256]);
  auto issue = [&](int kt, int sg) {
    const uint32_t so = (uint32_t)(sg * (int)sizeof(PvStage));
    const uint32_t ka = (uint32_t)min(kt * NV_KT + gp16, K - 16);
#pragma unroll
    for (int i = 0; i < 4; i++) dma16s(A, arow[i] + ka, la0 + so + i * 4096);
#pragma unroll
    for (int i = 0; i < 2; i++) dma16s(We, boff[i] + (uint32_t)kt * 1024u, lb0 + so + i * 4096);
    dma4s(Se, soff + (uint32_t)kt * 128u, ls0 + so);
  };

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

  issue(0, 0);
  if (nkt > 1) issue(1, 1);
  int sidx = 0;
  for (int kt = 0; kt < nkt; kt++) {
    // K-tile kt is in once only the next one's DMA (when issued) is outstanding
    if (kt + 1 < nkt) asm volatile("s_waitcnt vmcnt(7)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // K-tile kt + 2 into the stage every wave finished reading in the previous iteration
    if (kt + 2 < nkt) issue(kt + 2, sidx == 0 ? PV_NS - 1 : sidx - 1);
    const PvStage& S = st[sidx];
    h8 b[4][4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int ntl = wn * 4 + j;
      const u32x4 bw = *reinterpret_cast<const u32x4*>(S.b + ntl * 1024 + lane * 16);
      const uint32_t sw = *reinterpret_cast<const uint16_t*>(S.s + ntl * 128 + lane * 2);
      const GroupScale s0 = group_scale(sw & 0xffu), s1 = group_scale((sw >> 8) & 0xffu);
#pragma unroll
      for (int t = 0; t < 4; t++) b[j][t] = e2m1x8_f16(bw[t], t < 2 ? s0 : s1);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = (wm * 4 + i) * 16 + c;
      const uint4 l = *reinterpret_cast<const uint4*>(S.a + r * NV_KT + (((2 * g) ^ (r & 7)) * 16));
      const uint4 h = *reinterpret_cast<const uint4*>(S.a + r * NV_KT + (((2 * g + 1) ^ (r & 7)) * 16));
      const h8 a0 = e4m3x8_f16(l.x, l.y), a1 = e4m3x8_f16(l.z, l.w), a2 = e4m3x8_f16(h.x, h.y),
               a3 = e4m3x8_f16(h.z, h.w);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b[j][0], acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b[j][1], acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, b[j][2], acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a3, b[j][3], acc[i][j], 0, 0, 0);
      }
    }
    sidx = sidx == PV_NS - 1 ? 0 : sidx + 1;
  }

  // epilogue: lane holds column c of each column tile, rows 4g .. 4g + 3 of each row tile; out = bf16(v * ((Wg[n] *
  // As[row]) * topk_w[row])), the row factors from LDS and the lane's 4 column multipliers loaded together. Branch-free:
  // every lane issues its 64 two-byte stores through a raw buffer of numel * N * 2 bytes (the host keeps it below
  // 2 GiB), a padding row or a column past N going to offset `cbytes`, which the range check drops -- no store waits
  // behind another.
  float wgv[4];
#pragma unroll
  for (int j = 0; j < 4; j++) wgv[j] = Ge[min((nt0 + wn * 4 + j) * 16 + c, N - 1)];
  const uint32_t cbytes = (uint32_t)numel * (uint32_t)N * 2u;
  const auto crs = __builtin_amdgcn_make_buffer_rsrc(C, (short)0, (int)cbytes, 0x00020000);
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int row = (wm * 4 + i) * 16 + 4 * g + q;
      const int fr = s_fr[row];
      const bool live = fr >= 0 && fr < numel;
      const float ras = s_as[row], rtw = s_tw[row];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int n = (nt0 + wn * 4 + j) * 16 + c;
        float sc = wgv[j] * ras;
        if (topk_w) sc *= rtw;
        const uint16_t v = (uint16_t)(pack_bf16x2(acc[i][j][q] * sc, 0.f) & 0xffffu);
        const uint32_t off = (live && n < N) ? ((uint32_t)fr * (uint32_t)N + (uint32_t)n) * 2u : cbytes;
        __builtin_amdgcn_raw_buffer_store_b16(v, crs, (int)off, 0, 0);
      }
    }
}

// ------------------------------------------------------------------- dense linear at decode widths, one launch
// The native NVFP4 dense linear for M <= 2 rows with the per-row fp8 activation quant inside the GEMM launch: every
// workgroup quantises the rows into LDS (r9k_rowquant.h: quant_rows_fp8's bytes), then runs moe_nvfp4_kernel's
// weight stream for one routing block of identity rows -- its widening, MFMA order, K split over SK waves and partial-
// tile sum -- so the output equals r9k_quant_rows_fp8 + r9k_moe_nvfp4a8 over identity tables bit for bit. The weight
// loads of the wave's first batch go out before the quant, whose latency they overlap.
constexpr int NQ_APAD = 16;       // bytes of padding per LDS code row

template <int NPW, int SK, int U, int MG>
__global__ void __launch_bounds__(WAVE * SK) dense_nvfp4_qa_kernel(
    const uint16_t* __restrict__ x, long ldx, const uint8_t* __restrict__ Wq, const uint8_t* __restrict__ Ws,
    const float* __restrict__ Wg, uint16_t* __restrict__ out, long ldo, int M, int N, int K) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int lda = K + NQ_APAD;
  uint8_t* A = lds;
  float* s_row = reinterpret_cast<float*>(lds + (size_t)M * lda);
  float* red = s_row + 16;
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int g = lane >> 4, c = lane & 15;
  const int NT = N / 16, nkt = K / NV_KT;

  const uint8_t* wtile[NPW];
  const uint8_t* stile[NPW];
#pragma unroll
  for (int j = 0; j < NPW; j++) {
    const int nt = min((int)blockIdx.x * NPW + j, NT - 1);     // a tile past N computes a copy, never stored
    wtile[j] = Wq + (size_t)nt * nkt * 1024 + lane * 16;
    stile[j] = Ws + (size_t)nt * nkt * 128 + lane * 2;
  }
  const int kt0 = wave * nkt / SK, kt1 = (wave + 1) * nkt / SK;

  u32x4 bw[U][NPW];
  uint32_t sw[U][NPW];
  auto issue = [&](int kt) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = min(kt + u, kt1 - 1);
#pragma unroll
      for (int j = 0; j < NPW; j++) {
        bw[u][j] = ld16_nt(wtile[j] + (size_t)k * 1024);
        sw[u][j] = ld2_nt(stile[j] + (size_t)k * 128);
      }
    }
  };
  {
    constexpr int T = WAVE * SK, XC = row_chunks<T>();
    const int nvec = K / 8;
    uint4 xv[MG][XC];
    load_row_group<T, MG, XC>(x, ldx, 0, M, nvec, tid, xv);
    issue(kt0);
    quant_row_group<T, MG, XC>(xv, 0, M, nvec, A, lda, s_row, red, tid);
  }

  v4f acc[NPW];
#pragma unroll
  for (int j = 0; j < NPW; j++) acc[j] = (v4f){0.f, 0.f, 0.f, 0.f};
  const bool arow = c < M;
  const uint8_t* ar = A + (size_t)(arow ? c : 0) * lda + 32 * g;   // lane group g: K values 32 g .. + 31 of a tile
  for (int kt = kt0; kt < kt1; kt += U) {
    if (kt != kt0) issue(kt);
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = kt + u;
      if (k < kt1) {                                         // wave-uniform
        uint4 l = *reinterpret_cast<const uint4*>(ar + k * NV_KT);
        uint4 h = *reinterpret_cast<const uint4*>(ar + k * NV_KT + 16);
        if (!arow) l = h = make_uint4(0u, 0u, 0u, 0u);
        const h8 a[4] = {e4m3x8_f16(l.x, l.y), e4m3x8_f16(l.z, l.w), e4m3x8_f16(h.x, h.y), e4m3x8_f16(h.z, h.w)};
#pragma unroll
        for (int j = 0; j < NPW; j++) {
          const GroupScale s0 = group_scale(sw[u][j] & 0xffu), s1 = group_scale((sw[u][j] >> 8) & 0xffu);
#pragma unroll
          for (int st = 0; st < 4; st++) {
            const h8 b = e2m1x8_f16(bw[u][j][st], st < 2 ? s0 : s1);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[st], b, acc[j], 0, 0, 0);
          }
        }
      }
    }
  }

  // partial tiles through LDS (the quant's scratch is free again after its closing barrier), summed in wave order;
  // out = bf16(v * (Wg[n] * s[m])), moe_nvfp4_kernel's epilogue
#pragma unroll
  for (int j = 0; j < NPW; j++) {
    float* t = red + (size_t)(wave * NPW + j) * 256;
#pragma unroll
    for (int q = 0; q < 4; q++) t[(4 * g + q) * 16 + c] = acc[j][q];
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
    const float sc = Wg[n] * s_row[m];
    out[(size_t)m * ldo + n] = f2bf(v * sc);
  }
}

}  // namespace

// The prefill entry's native-NVFP4 case (r9k_moe_4bit_prefill with nv = 1; reference kernels/r9k_moe_mxfp4a8.hip:
// 1205-1230): routing blocks of blk = 128 or 256 rows, weights as r9k_moe_nvfp4a8 takes them. 0 / -7 blk / -3 / -6.
int r9k_nvfp4_prefill_launch(long a, long as, long wq, long ws, long wg, long c, long sorted_ids, long expert_ids,
                             long ntpp, long topk_w, long ws_estride, long wg_estride, int max_blocks, int numel,
                             int a_row_div, int K, int N, int blk, long stream) {
  if (blk != PV_BM && blk != 2 * PV_BM) return -7;
  if (max_blocks <= 0 || numel <= 0) return 0;
  if (!a || !as || !wq || !ws || !wg || !c || !sorted_ids || !expert_ids || !ntpp || a_row_div < 1) return -3;
  const int subs = blk / PV_BM;
  const long ny = (long)max_blocks * subs;
  if (ny > 0x7fffffffL) return -3;
  const dim3 grid((N + PV_BN - 1) / PV_BN, (unsigned)ny);
  const long wq_estride = (long)N * ((K + NV_KT - 1) / NV_KT) * 64;
  // the DMA addresses activations and one expert's codes through 32-bit offsets
  if ((long)((numel + a_row_div - 1) / a_row_div) * K >= (1L << 32) || wq_estride >= (1L << 32)) return -3;
  if ((long)numel * N * 2 >= (1L << 31)) return -3;             // the epilogue's raw output buffer
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(nvfp4_prefill_kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)PV_SMEM);
  if (attr != hipSuccess) return -6;
  hipLaunchKernelGGL(nvfp4_prefill_kernel, grid, dim3(PV_THREADS), PV_SMEM, (hipStream_t)stream, (const uint8_t*)a,
                     (const float*)as, (const uint8_t*)wq, (const uint8_t*)ws, (const float*)wg, (uint16_t*)c,
                     (const int*)sorted_ids, (const int*)expert_ids, (const int*)ntpp, (const float*)topk_w,
                     wq_estride, ws_estride, wg_estride, numel, a_row_div, K, N, blk, subs);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

// Reference: kernels/r9k_moe_mxfp4a8.hip:641-647 (r9k_moe_nvfp4a8): same arguments and routing contract. ws / wg as
// the layout above (ws_estride bytes, wg_estride floats per expert); the code stride is N * ceil(K / 128) * 64 bytes
// (N * K / 2 when K % 128 == 0). WV and NPW are the reference's gfx1201 knobs and are not used; SK must divide K / 16
// as there (K % (16 SK) == 0). MT 1 / 2 / 4 rows tiles of 16 (the reference's bit 3 LDS-A flag is ignored).
// 0, or -1 N % 16, -2 K % (16 SK) or K % 16, -3 bad pointer / argument, -7 MT, -6 launch error.
extern "C" int r9k_moe_nvfp4a8(long a, long as, long wq, long ws, long wg, long c, long sorted_ids, long expert_ids,
                               long ntpp, long topk_w, long ws_estride, long wg_estride, int max_blocks, int numel,
                               int a_row_div, int K, int N, int WV, int SK, int NPW, int MT, long stream) {
  (void)WV;
  (void)NPW;
  MT &= 7;
  if (N % 16 || N <= 0) return -1;
  if (K % NV_G || K <= 0 || SK < 1 || K % (NV_G * SK)) return -2;
  if (MT != 1 && MT != 2 && MT != 4) return -7;
  if (a_row_div < 1) return -3;
  if (max_blocks <= 0 || numel <= 0) return 0;
  if (!a || !as || !wq || !ws || !wg || !c || !sorted_ids || !expert_ids || !ntpp) return -3;
  const int blk = 16 * MT;
  const NvPick p = nv_pick(N, K, max_blocks, numel);
  const dim3 grid((N / 16 + p.NPW - 1) / p.NPW, (unsigned)max_blocks);
  const long wq_estride = (long)N * ((K + NV_KT - 1) / NV_KT) * 64;
  const hipStream_t st = (hipStream_t)stream;
#define NVL(MTv, NPWv, SKv, Uv)                                                                                   \
  if (MT == MTv && p.NPW == NPWv && p.SK == SKv && p.U == Uv) {                                                 \
    nv_launch<MTv, NPWv, SKv, Uv>(grid, st, a, as, wq, ws, wg, c, sorted_ids, expert_ids, ntpp, topk_w,          \
                                  wq_estride, ws_estride, wg_estride, numel, a_row_div, K, N, blk, 1);           \
    return hipGetLastError() == hipSuccess ? 0 : -6;                                                            \
  }
#define NVU(MTv, NPWv, SKv) NVL(MTv, NPWv, SKv, 1) NVL(MTv, NPWv, SKv, 2) NVL(MTv, NPWv, SKv, 4)
#define NVS(MTv, NPWv) NVU(MTv, NPWv, 1) NVU(MTv, NPWv, 2) NVU(MTv, NPWv, 4)
  NVS(1, 1) NVS(1, 2) NVS(2, 1) NVS(2, 2) NVS(4, 1) NVS(4, 2)
  NVL(1, 2, 4, 5)
#undef NVS
#undef NVU
#undef NVL
  return -3;
}

// No counterpart as one entry in the reference: r9k_quant_rows_fp8 + r9k_moe_nvfp4a8 over identity tables (the native
// NVFP4 dense linear, r9700_vllm/ops.py:66-83) in one launch, for M <= 2 rows. x bf16 [M][K] (row stride ldx
// elements, rows 16-byte aligned); wq / ws / wg one expert in this kernel's layout (prepare_nvfp4_weights); out bf16
// [M][N] (row stride ldo). Served: 1 <= M <= 2, K % 128 == 0, K <= 8192, N % 16 == 0; 2 (nothing launched) otherwise.
// 0, -3 bad argument, -6 launch error. Bit-equal to the two launches (the decode kernel's launch shape for one block).
extern "C" int r9k_dense_nvfp4_qa(long x, long ldx, long wq, long ws, long wg, long out, long ldo, int M, int N, int K,
                                  long stream) {
  if (M <= 0) return 0;
  if (!x || !wq || !ws || !wg || !out || N <= 0 || K <= 0) return -3;
  if (M > 2 || K % NV_KT || K > 8192 || N % 16 || (x & 15) || (ldx & 7) || (wq & 15)) return 2;
  const NvPick p = nv_pick(N, K, 1, M);
  if (p.SK != 1 && p.SK != 4) return 2;
  const int T = WAVE * p.SK;
  if (K / 8 > (p.SK == 4 ? row_chunks<256>() : row_chunks<64>()) * T) return 2;
  // LDS: codes, 16 row scales, then the partial tiles (which also hold the quant's SK x M row maxima before them)
  const size_t smem = (size_t)M * (K + NQ_APAD) + 16 * sizeof(float) + (size_t)p.SK * p.NPW * 256 * sizeof(float);
  const dim3 grid((N / 16 + p.NPW - 1) / p.NPW), block(T);
  const hipStream_t st = (hipStream_t)stream;
  const int MG = M;
#define NQ(NPWv, SKv, Uv, MGv)                                                                                     \
  if (p.NPW == NPWv && p.SK == SKv && p.U == Uv && MG == MGv) {                                                    \
    hipLaunchKernelGGL((dense_nvfp4_qa_kernel<NPWv, SKv, Uv, MGv>), grid, block, smem, st, (const uint16_t*)x, ldx, \
                       (const uint8_t*)wq, (const uint8_t*)ws, (const float*)wg, (uint16_t*)out, ldo, M, N, K);      \
    return hipGetLastError() == hipSuccess ? 0 : -6;                                                               \
  }
#define NQM(NPWv, SKv, Uv) NQ(NPWv, SKv, Uv, 1) NQ(NPWv, SKv, Uv, 2)
#define NQU(NPWv, SKv) NQM(NPWv, SKv, 1) NQM(NPWv, SKv, 2) NQM(NPWv, SKv, 4)
  NQU(1, 1) NQU(2, 1) NQU(1, 4) NQU(2, 4)
#undef NQU
#undef NQM
#undef NQ
  return 2;
}
