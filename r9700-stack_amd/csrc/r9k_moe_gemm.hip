// r9k_moe_gemm.hip -- grouped (MoE) MXFP4-weight x fp8-activation GEMM for gfx950 (CDNA4), routed through the
// moe_align_block_size tables.
//
//   out[r, n] = bf16( (sum_k A_q[r / a_row_div, k] * W_e[n, k]) * (As[r / a_row_div] (* topk_w[r])) )
//
// for every routed flat row r (token * topk + j) of expert e = expert_ids[block of r], where W_e is the MXFP4
// weight (e2m1 codes times 2^(e8m0 - 127) per 32-element block). Reference: kernels/r9k_moe_mxfp4a8.hip:24-46
// (addressing contract), :469-482 (epilogue: v * (As * topk_w), one bf16 rounding).
//
// The product runs on V_MFMA_SCALE_F32_16X16X128_F8F6F4 with A = e4m3 activations (scale byte 127 = 2^0) and
// B = e2m1 weights with their e8m0 block exponent fed as the B scale: the hardware applies the MXFP4 block scale
// exactly, so there is no per-group fp32 rescaling in the inner loop (the reference's gfx1201 kernel needs one)
// and no exponent folding. The per-token fp32 scale As (and the router weight) are applied in the epilogue.
// Operand layout of that instruction (measured on gfx950): output row r = lane % 16 of A, column c = lane % 16 of
// B, g = lane / 16. The fp4 B operand holds K = 32g .. 32g+31 of column c in nibbles 0..31 (low nibble first), and
// lane's scale byte scales that 32-block. The fp8 A operand splits K in halves: bytes 0..15 hold K = 16g .. 16g+15,
// bytes 16..31 hold K = 64 + 16g .. +15 of row r. C: lane holds column lane % 16, rows 4g .. 4g+3.
//
// Weight layout (per expert, produced by kernels/moe.py permute_fragments / pack_scales):
//   codes  : N/16 column tiles of 16 rows x K/2 bytes (8K bytes each). Within a column tile, K-tile kt (128 K) is
//            1 KB at kt * 1024: lane l = g * 16 + r holds row r, K elements kt*128 + g*32 .. +32 as 16 bytes at
//            l * 16 -- exactly the B operand of one 16x16x128 MFMA, so a wave loads it as one contiguous 1 KB
//            (global_load_dwordx4). A last partial K-tile (K % 128 = 32 * G) holds only lanes l < 16 * G.
//   scales : N/16 column tiles of 16 * K/32 bytes. Full super-steps of 4 K-tiles are 256 bytes each: lane l's
//            dword holds the exponents of its (row, group) for the 4 K-tiles, byte j = K-tile 4q + j. The K-tiles
//            after the last full super-step are 64 bytes each (lane l's byte at l; a partial tile 16 * G bytes).
// One 16-row x 16-column MFMA tile therefore reads 1 KB of codes and 64 bytes of exponents, all coalesced.
//
// Work split: a workgroup owns 16*MT routed rows (MT M-tiles sharing every weight fragment) x NPW column tiles,
// with SK waves splitting K; the SK partial tiles are summed through LDS in the epilogue. A routing block of `blk`
// rows (blk = 16 * MT at decode, the prefill cfg's BM) is covered by blk / (16 * MT) workgroups along grid.y.
// Blocks at or past ntpp, blocks with expert -1, and sub-blocks that are all padding exit at once; padding rows
// are clamped to the block's first row for the loads and dropped at the store.
#include "r9k_common.h"

namespace {

using namespace r9k;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int KT = 128;           // K per MFMA
constexpr int GROUP = 32;         // MXFP4 block
constexpr int E8M0_ONE = 127;     // 2^0

template <bool NTL>
__device__ __forceinline__ u32x4 ld16(const uint8_t* p) {
  if constexpr (NTL) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  else return *reinterpret_cast<const u32x4*>(p);
}
template <bool NTL>
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) {
  if constexpr (NTL) return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
  else return *reinterpret_cast<const uint32_t*>(p);
}

template <int MT, int NPW, int SK>
__global__ void __launch_bounds__(WAVE * SK) moe_mxfp4_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint8_t* __restrict__ Ws, uint16_t* __restrict__ C, const int* __restrict__ sorted_ids,
    const int* __restrict__ expert_ids, const int* __restrict__ ntpp, const float* __restrict__ topk_w,
    long wq_estride, long ws_estride, int numel, int a_row_div, int K, int N, int blk, int subs) {
  constexpr int BLK = 16 * MT;
  constexpr int U = MT == 1 ? 4 : (MT == 2 ? 2 : 1);      // K-tiles whose loads are issued together
  constexpr bool NTL = MT == 1;                            // decode: every weight byte is read once
  extern __shared__ float red[];

  const int rb = blockIdx.y / subs, sub = blockIdx.y - rb * subs;
  if (rb * blk >= ntpp[0]) return;
  const int e = expert_ids[rb];
  if (e < 0) return;
  const int first = sorted_ids[rb * blk];
  if (first < 0 || first >= numel) return;
  const int row0 = rb * blk + sub * BLK;
  if (sorted_ids[row0] >= numel) return;                   // padding sits at the end of a block

  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int g = lane >> 4, r = lane & 15;
  const int NT = N / 16;
  const int nkt = (K + KT - 1) / KT, nkt_full = K / KT, tail_groups = (K % KT) / GROUP;
  const int KB = K / GROUP, nq = KB / 16;

  // A row byte offsets of this lane's row in each M tile (+ its 16-byte K chunk of the low half)
  size_t aoff[MT];
#pragma unroll
  for (int i = 0; i < MT; i++) {
    int fr = sorted_ids[row0 + i * 16 + r];
    if (fr >= numel || fr < 0) fr = first;
    aoff[i] = (size_t)(fr / a_row_div) * K + g * 16;
  }
  // a partial last K-tile (K % 128 = 32 * G) holds K < 32G: the A halves at 16g and 64 + 16g are live below it
  const bool a_lo_tail = g < 2 * tail_groups, a_hi_tail = g < 2 * tail_groups - 4;
  const uint8_t* __restrict__ We = Wq + (size_t)e * wq_estride;
  const uint8_t* __restrict__ Se = Ws + (size_t)e * ws_estride;
  const uint8_t* wbase[NPW];
  const uint8_t* sbase[NPW];
#pragma unroll
  for (int j = 0; j < NPW; j++) {
    int nt = blockIdx.x * NPW + j;
    nt = nt < NT ? nt : NT - 1;                            // out-of-range tiles compute a copy, never stored
    wbase[j] = We + (size_t)nt * (size_t)(8 * K) + lane * 16;
    sbase[j] = Se + (size_t)nt * (size_t)(16 * KB);
  }

  v4f acc[NPW][MT];
#pragma unroll
  for (int j = 0; j < NPW; j++)
#pragma unroll
    for (int i = 0; i < MT; i++) acc[j][i] = (v4f){0.f, 0.f, 0.f, 0.f};

  const int kt0 = wave * nkt / SK, kt1 = (wave + 1) * nkt / SK;
  for (int kt = kt0; kt < kt1; kt += U) {
    v8i af[U][MT];
    u32x4 bf[U][NPW];
    uint32_t sb[U][NPW];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = kt + u;
      const bool live = k < kt1;
      const bool lane_ok = live && (k < nkt_full || g < tail_groups);
#pragma unroll
      for (int j = 0; j < NPW; j++) {
        if (lane_ok) {
          bf[u][j] = ld16<NTL>(wbase[j] + (size_t)k * 1024);
          if (k < 4 * nq) {
            sb[u][j] = (ld4<NTL>(sbase[j] + (k >> 2) * 256 + lane * 4) >> (8 * (k & 3))) & 0xffu;
          } else {
            sb[u][j] = sbase[j][nq * 256 + (k - 4 * nq) * 64 + lane];
          }
        } else {
          bf[u][j] = (u32x4){0u, 0u, 0u, 0u};
          sb[u][j] = E8M0_ONE;
        }
      }
      const bool full = k < nkt_full;
      const bool lo_ok = live && (full || a_lo_tail), hi_ok = live && (full || a_hi_tail);
#pragma unroll
      for (int i = 0; i < MT; i++) {
        const uint8_t* ap = A + aoff[i] + (size_t)k * KT;
        const uint4 a0 = lo_ok ? *reinterpret_cast<const uint4*>(ap) : make_uint4(0u, 0u, 0u, 0u);
        const uint4 a1 = hi_ok ? *reinterpret_cast<const uint4*>(ap + 64) : make_uint4(0u, 0u, 0u, 0u);
        af[u][i] = (v8i){(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
      }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      if (kt + u < kt1) {
#pragma unroll
        for (int j = 0; j < NPW; j++) {
          const v8i b = (v8i){(int)bf[u][j].x, (int)bf[u][j].y, (int)bf[u][j].z, (int)bf[u][j].w, 0, 0, 0, 0};
#pragma unroll
          for (int i = 0; i < MT; i++)
            acc[j][i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[u][i], b, acc[j][i], 0, 4, 0, E8M0_ONE,
                                                                          0, (int)sb[u][j]);
        }
      }
    }
  }

  // C layout of a 16x16 tile: lane l holds column l % 16, rows 4 * (l / 16) + q. Partials to LDS as [row][col].
#pragma unroll
  for (int j = 0; j < NPW; j++)
#pragma unroll
    for (int i = 0; i < MT; i++) {
      float* t = red + (size_t)((wave * NPW + j) * MT + i) * 256;
#pragma unroll
      for (int q = 0; q < 4; q++) t[(4 * g + q) * 16 + r] = acc[j][i][q];
    }
  __syncthreads();
  constexpr int TOT = NPW * MT * 256;
  for (int idx = tid; idx < TOT; idx += WAVE * SK) {
    const int col = idx & 15, row = (idx >> 4) & 15, ti = idx >> 8;   // ti = j * MT + i
    const int j = ti / MT, i = ti - j * MT;
    const int n = (blockIdx.x * NPW + j) * 16 + col;
    if (n >= N) continue;
    const int fr = sorted_ids[row0 + i * 16 + row];
    if (fr < 0 || fr >= numel) continue;
    float v = 0.f;
#pragma unroll
    for (int s = 0; s < SK; s++) v += red[(size_t)s * TOT + idx];
    float sc = As[fr / a_row_div];
    if (topk_w) sc *= topk_w[fr];
    C[(size_t)fr * N + n] = f2bf(v * sc);
  }
}

struct Pick { int MT, NPW, SK; };

// Launch shape for the decode-family kernel: SK waves split K (up to 4 K-tiles a wave at long K), NPW column tiles
// a wave. Chosen from the host-known shape only, so a call stays graph-capturable.
Pick pick(int MT, int N, int K, int max_blocks) {
  const int nkt = (K + KT - 1) / KT;
  const int NT = N / 16;
  int SK = nkt >= 8 ? 4 : (nkt >= 2 ? 2 : 1);
  int NPW = NT >= 4 ? 4 : 2;
  if (MT >= 4) NPW = 2;
  // few live blocks (single-token decode): more, smaller workgroups
  if (max_blocks * ((NT + NPW - 1) / NPW) < 512 && NPW > 2) NPW = 2;
  (void)N;
  return {MT, NPW, SK};
}

template <int MT, int NPW, int SK>
int launch_one(dim3 grid, hipStream_t st, long a, long as, long wq, long ws, long c, long sorted_ids,
               long expert_ids, long ntpp, long topk_w, long wq_estride, long ws_estride, int numel, int a_row_div,
               int K, int N, int blk, int subs) {
  const size_t smem = (size_t)SK * NPW * MT * 256 * sizeof(float);
  hipLaunchKernelGGL((moe_mxfp4_kernel<MT, NPW, SK>), grid, dim3(WAVE * SK), smem, st, (const uint8_t*)a,
                     (const float*)as, (const uint8_t*)wq, (const uint8_t*)ws, (uint16_t*)c, (const int*)sorted_ids,
                     (const int*)expert_ids, (const int*)ntpp, (const float*)topk_w, wq_estride, ws_estride, numel,
                     a_row_div, K, N, blk, subs);
  return 0;
}

// Host dispatch shared by the decode (blk = 16 * MT) and prefill (blk = cfg BM) entries.
// ws_estride: bytes per expert of the packed scale tensor; the code stride is N * K / 2 bytes.
int moe_dispatch(long a, long as, long wq, long ws, long c, long sorted_ids, long expert_ids, long ntpp, long topk_w,
                 long ws_estride, int max_blocks, int numel, int a_row_div, int K, int N, int MT, int blk,
                 long stream) {
  if (N % 16 || N <= 0) return -1;
  if (K % GROUP || K <= 0) return -2;
  if (MT != 1 && MT != 2 && MT != 4) return -7;
  if (blk % (16 * MT)) return -7;
  if (a_row_div < 1) return -3;
  if (max_blocks <= 0 || numel <= 0) return 0;
  if (!a || !as || !wq || !ws || !c || !sorted_ids || !expert_ids || !ntpp) return -3;
  const Pick p = pick(MT, N, K, max_blocks);
  const int subs = blk / (16 * MT);
  const long ny = (long)max_blocks * subs;
  if (ny > 0x7fffffffL) return -3;
  const dim3 grid((N / 16 + p.NPW - 1) / p.NPW, (unsigned)ny);
  const long wq_estride = (long)N * K / 2;
  const hipStream_t st = (hipStream_t)stream;
#define L(MTv, NPWv, SKv)                                                                                   \
  if (p.MT == MTv && p.NPW == NPWv && p.SK == SKv)                                                          \
    return launch_one<MTv, NPWv, SKv>(grid, st, a, as, wq, ws, c, sorted_ids, expert_ids, ntpp, topk_w,     \
                                      wq_estride, ws_estride, numel, a_row_div, K, N, blk, subs);
#define LS(MTv, NPWv) L(MTv, NPWv, 1) L(MTv, NPWv, 2) L(MTv, NPWv, 4)
  LS(1, 2) LS(1, 4) LS(2, 2) LS(2, 4) LS(4, 2)
#undef LS
#undef L
  return -5;
}

// Prefill tile table: cfg -> (BM rows per routing block, BN, BK). BM is what the routing tables are built with
// (r9k_moe_prefill_bm) and keeps the reference's values per cfg index (kernels/r9k_moe_mxfp4a8.hip:1170-1194), so
// a caller's cfg choice maps to the same block size. BK = 32: any K % 32 == 0 is accepted.
struct PfCfg { int BM, BN, BK; };
const PfCfg kPf[] = {
    {256, 64, 32}, {256, 128, 32}, {128, 128, 32}, {128, 64, 32}, {128, 64, 32}, {256, 32, 32}, {64, 64, 32},
    {256, 128, 32}, {256, 128, 32}, {256, 128, 32}, {128, 128, 32}, {64, 64, 32}, {256, 128, 32}, {128, 128, 32},
    {64, 64, 32}, {64, 128, 32}, {256, 128, 32}, {64, 128, 32}, {64, 64, 32}, {64, 128, 32},
};
constexpr int NPF = sizeof(kPf) / sizeof(kPf[0]);

}  // namespace

// Reference: kernels/r9k_moe_mxfp4a8.hip:625-638 (r9k_moe_mxfp4a8). `wref`, WV, SK, NPW and the MT bits 3 (LDS-A)
// and 4 (fold) are gfx1201 tuning / layout knobs with no meaning here and are ignored; MT & 7 in {1, 2, 4} sets the
// routing block (16 * MT rows). ws_estride: bytes per expert of the scale tensor. 0 / negative error code.
extern "C" int r9k_moe_mxfp4a8(long a, long as, long wq, long ws, long wref, long c, long sorted_ids, long expert_ids,
                               long ntpp, long topk_w, long ws_estride, long wref_estride, int max_blocks, int numel,
                               int a_row_div, int K, int N, int WV, int SK, int NPW, int MT, long stream) {
  (void)wref; (void)wref_estride; (void)WV; (void)SK; (void)NPW;
  const int mt = MT & 7;
  const int rc = moe_dispatch(a, as, wq, ws, c, sorted_ids, expert_ids, ntpp, topk_w, ws_estride, max_blocks, numel,
                              a_row_div, K, N, mt, 16 * mt, stream);
  if (rc) return rc;
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

// Reference: kernels/r9k_moe_mxfp4a8.hip:1227-1268. nv: 0 MXFP4, 2 MXFP4 with folded exponents (same data here:
// the block exponents are applied exactly either way), 1 NVFP4 and 3 fp8 weights are not served (-8).
extern "C" int r9k_moe_4bit_prefill(int nv, long a, long as, long wq, long ws, long wref, long c, long sorted_ids,
                                    long expert_ids, long ntpp, long topk_w, long ws_estride, long wref_estride,
                                    int max_blocks, int numel, int a_row_div, int K, int N, int cfg, long stream) {
  (void)wref; (void)wref_estride;
  if (N % 16) return -1;
  if (cfg < 0 || cfg >= NPF) return -7;
  if (K % kPf[cfg].BK) return -2;
  if (nv != 0 && nv != 2) return -8;
  const int rc = moe_dispatch(a, as, wq, ws, c, sorted_ids, expert_ids, ntpp, topk_w, ws_estride, max_blocks, numel,
                              a_row_div, K, N, 4, kPf[cfg].BM, stream);
  if (rc) return rc;
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

extern "C" int r9k_moe_prefill_bm(int cfg) { return (cfg < 0 || cfg >= NPF) ? -1 : kPf[cfg].BM; }
extern "C" int r9k_moe_prefill_bk(int cfg) { return (cfg < 0 || cfg >= NPF) ? -1 : kPf[cfg].BK; }
extern "C" int r9k_moe_block(void) { return 16; }
// Exponent folding is a gfx1201 device for a WMMA without block scales; the scaled MFMA needs none.
extern "C" int r9k_fold_supported(void) { return 0; }
