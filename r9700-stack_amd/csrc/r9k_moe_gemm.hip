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
//   scales : N/16 column tiles of 16 * K/32 bytes. K-tile kt is 64 bytes at kt * 64: lane l's byte at l is the
//            exponent of its (row r, group g) -- the MFMA's B scale operand (a partial last tile 16 * G bytes).
// One 16-row x 16-column MFMA tile therefore reads 1 KB of codes and 64 bytes of exponents, all coalesced.
//
// Work split: a workgroup owns 16*MT routed rows (MT M-tiles sharing every weight fragment) x NPW column tiles,
// with SK waves splitting K; the SK partial tiles are summed through LDS in the epilogue. A routing block of `blk`
// rows (blk = 16 * MT at decode, the prefill cfg's BM) is covered by blk / (16 * MT) workgroups along grid.y.
// Blocks at or past ntpp, blocks with expert -1, and sub-blocks that are all padding exit at once; padding rows
// are clamped to the block's first row for the loads and dropped at the store.
#include "r9k_common.h"

#include <cstdlib>

namespace {

using namespace r9k;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int KT = 128;           // K per MFMA
constexpr int GROUP = 32;         // MXFP4 block
constexpr int E8M0_ONE = 127;     // 2^0
constexpr long MAX_WG = 16384;    // workgroups of one launch at most (64 for each of the 256 CUs); more tile rows
                                  // are walked grid-stride

template <bool NTL>
__device__ __forceinline__ u32x4 ld16(const uint8_t* p) {
  if constexpr (NTL) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  else return *reinterpret_cast<const u32x4*>(p);
}
template <bool NTL>
__device__ __forceinline__ uint32_t ld1(const uint8_t* p) {
  if constexpr (NTL) return __builtin_nontemporal_load(p);
  else return *p;
}

// One workgroup: 16*MT routed rows x NPW column tiles; SK waves split the K-tiles (SK > 1: partial tiles summed
// through LDS). Each wave walks its K range in batches of U K-tiles: all loads of a batch (U*NPW weight tiles,
// U*NPW scale bytes, U*MT*2 activation chunks) are issued back to back with no branch or use in between, then the
// U*NPW*MT MFMAs run. Addresses are clamped instead of branched around (a lane past a partial K-tile, or a batch
// slot past the wave's range, re-reads a valid location and its operand is zeroed by select), so the compiler
// never has to drain the memory queue inside a batch.
//
// FUSE (the reference's r9k_moe_mxfp4a8_f, kernels/r9k_moe_mxfp4a8.hip:236-250, 358-368, 452-467; MT = 1):
//   1: gate_up with the activation in the epilogue. The workgroup's two column tiles are gate tile x and the up
//      tile N/32 further (NPW = 2), and it writes h = silu(bf16(g)) * bf16(u) as fp32 [numel, N/2] -- g and u
//      rounded exactly as the unfused kernel stores them, the activation the standalone SiLU kernel's.
//   2: down with fp32 A rows [numel, K] (h) quantised on load: each lane group of a row first takes the row's
//      absmax over all K, then every A chunk is encoded as e4m3(h * (448 / amax)) and the row scale amax / 448
//      replaces As -- the per-row quant of the standalone SiLU kernel, so fused and unfused results are identical.
//
// One call of moe_tile computes the tile of grid row `by` (routing block by / subs, sub-block by % subs). It returns
// false when that block lies at or past ntpp -- and so does every later one, blocks being in order -- true
// otherwise (a tile done, or an expert-map hole / all-padding sub-block skipped).
template <int MT, int NPW, int SK, int U, int FUSE>
__device__ __forceinline__ bool moe_tile(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint8_t* __restrict__ Ws, uint16_t* __restrict__ C, const int* __restrict__ sorted_ids,
    const int* __restrict__ expert_ids, const int* __restrict__ ntpp, const float* __restrict__ topk_w,
    long wq_estride, long ws_estride, int numel, int a_row_div, int K, int N, int blk, int subs, int by) {
  constexpr int BLK = 16 * MT;
  constexpr bool NTL = MT == 1;                            // decode: every weight byte is read once
  static_assert(FUSE == 0 || (MT == 1 && (FUSE == 2 || NPW == 2)), "fused variants: MT = 1; gate_up NPW = 2");
  extern __shared__ float red[];

  const int rb = by / subs, sub = by - rb * subs;
  const int row0 = rb * blk + sub * BLK;
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int g = lane >> 4, r = lane & 15;
  // the table reads are independent (every block index below the launch's max_blocks is inside the tables), so
  // they go out together and the block is checked once they are back: one memory round trip, not three
  const int np = ntpp[0];
  const int e = expert_ids[rb];
  const int first = sorted_ids[rb * blk];
  int fr_in[MT];
#pragma unroll
  for (int i = 0; i < MT; i++) fr_in[i] = sorted_ids[row0 + i * 16 + r];
  if (rb * blk >= np) return false;
  if (e < 0) return true;
  if (first < 0 || first >= numel || __shfl(fr_in[0], 0, WAVE) >= numel) return true;   // padding: end of a block
  const int NT = N / 16;
  const int nkt = (K + KT - 1) / KT, nkt_full = K / KT, tg = (K % KT) / GROUP;
  const int KB = K / GROUP;

  // per-lane operand offsets that stay valid on a partial last K-tile (only lanes/halves below K are live there)
  const int lane_b_tail = g < tg ? lane : r;                          // B lanes of the partial tile: lanes < 16 * tg
  const int a_lo_tail = g < 2 * tg ? 16 * g : 0;                     // A low half  (K 16g .. 16g + 15)
  const int a_hi_tail = g < 2 * tg - 4 ? 64 + 16 * g : 0;            // A high half (K 64 + 16g ..)
  const bool b_live_tail = g < tg, lo_live_tail = g < 2 * tg, hi_live_tail = g < 2 * tg - 4;

  size_t arow[MT];
  float rsc[MT];                                           // output scale of row r of M-tile i (lane r's row)
  float a_inv[MT];                                         // FUSE 2: 448 / row absmax
#pragma unroll
  for (int i = 0; i < MT; i++) {
    int fr = fr_in[i];
    if (fr >= numel || fr < 0) fr = first;
    arow[i] = (size_t)(fr / a_row_div) * K;
    if constexpr (FUSE == 2) {
      // lanes r, r + 16, r + 32, r + 48 each take a quarter of row r (K % 32 == 0), 8 loads in flight at a time
      const float4* q4 = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(A) + arow[i] + g * (K / 4));
      const int n4 = K / 16;
      float m = 0.f;
      for (int k0 = 0; k0 < n4; k0 += 8) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = q4[min(k0 + u, n4 - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++)
          m = fmaxf(m, fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
      }
      m = fmaxf(m, __shfl_xor(m, 16, WAVE));
      m = fmaxf(m, __shfl_xor(m, 32, WAVE));
      const float amax = fmaxf(m, 1e-12f);
      a_inv[i] = 448.f / amax;
      float sc = amax / 448.f;
      if (topk_w) sc *= topk_w[fr];
      rsc[i] = sc;
    } else {
      a_inv[i] = 0.f;
      float sc = As[fr / a_row_div];                       // loaded with the operands, used in the epilogue
      if (topk_w) sc *= topk_w[fr];
      rsc[i] = sc;
    }
  }
  const uint8_t* __restrict__ We = Wq + (size_t)e * wq_estride;
  const uint8_t* __restrict__ Se = Ws + (size_t)e * ws_estride;
  const uint8_t* wtile[NPW];
  const uint8_t* stile[NPW];
#pragma unroll
  for (int j = 0; j < NPW; j++) {
    int nt = FUSE == 1 ? (int)blockIdx.x + j * (NT / 2) : (int)blockIdx.x * NPW + j;
    nt = nt < NT ? nt : NT - 1;                            // out-of-range tiles compute a copy, never stored
    wtile[j] = We + (size_t)nt * (size_t)(8 * K);
    stile[j] = Se + (size_t)nt * (size_t)(16 * KB);
  }

  v4f acc[NPW][MT];
#pragma unroll
  for (int j = 0; j < NPW; j++)
#pragma unroll
    for (int i = 0; i < MT; i++) acc[j][i] = (v4f){0.f, 0.f, 0.f, 0.f};

  const int kt0 = wave * nkt / SK, kt1 = (wave + 1) * nkt / SK;
  for (int kt = kt0; kt < kt1; kt += U) {
    u32x4 bf[U][NPW];
    uint32_t sb[U][NPW];
    uint4 alo[U][MT], ahi[U][MT];
    float4 flo[FUSE == 2 ? U : 1][MT][4], fhi[FUSE == 2 ? U : 1][MT][4];   // FUSE 2: the fp32 A chunks
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = min(kt + u, kt1 - 1);
      const bool full = k < nkt_full;
      const int bl = full ? lane : lane_b_tail;
      const int soff = k * 64 + bl;
#pragma unroll
      for (int j = 0; j < NPW; j++) {
        bf[u][j] = ld16<NTL>(wtile[j] + (size_t)k * 1024 + bl * 16);
        sb[u][j] = ld1<NTL>(stile[j] + soff);
      }
      const int olo = full ? 16 * g : a_lo_tail, ohi = full ? 64 + 16 * g : a_hi_tail;
#pragma unroll
      for (int i = 0; i < MT; i++) {
        if constexpr (FUSE == 2) {
          const float* ap = reinterpret_cast<const float*>(A) + arow[i] + (size_t)k * KT;
#pragma unroll
          for (int v = 0; v < 4; v++) {
            flo[u][i][v] = reinterpret_cast<const float4*>(ap + olo)[v];
            fhi[u][i][v] = reinterpret_cast<const float4*>(ap + ohi)[v];
          }
        } else {
          const uint8_t* ap = A + arow[i] + (size_t)k * KT;
          alo[u][i] = *reinterpret_cast<const uint4*>(ap + olo);
          ahi[u][i] = *reinterpret_cast<const uint4*>(ap + ohi);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = kt + u;
      if constexpr (FUSE == 2) {
        // the fp32 chunks to e4m3 codes (16 bytes each half), as the standalone per-row quant encodes them
#pragma unroll
        for (int i = 0; i < MT; i++) {
          const float s = a_inv[i];
          uint32_t wl[4], wh[4];
#pragma unroll
          for (int v = 0; v < 4; v++) {
            const float4 a = flo[u][i][v], b = fhi[u][i][v];
            const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            const uint2 w = pack8_e4m3(f, s);
            wl[v] = w.x;
            wh[v] = w.y;
          }
          alo[u][i] = make_uint4(wl[0], wl[1], wl[2], wl[3]);
          ahi[u][i] = make_uint4(wh[0], wh[1], wh[2], wh[3]);
        }
      }
      if (k < kt1) {
        const bool full = k < nkt_full;
        const bool bl = full || b_live_tail, lo = full || lo_live_tail, hi = full || hi_live_tail;
#pragma unroll
        for (int j = 0; j < NPW; j++) {
          const v8i b = bl ? (v8i){(int)bf[u][j].x, (int)bf[u][j].y, (int)bf[u][j].z, (int)bf[u][j].w, 0, 0, 0, 0}
                           : (v8i){0, 0, 0, 0, 0, 0, 0, 0};
          const int sc = bl ? (int)sb[u][j] : E8M0_ONE;
#pragma unroll
          for (int i = 0; i < MT; i++) {
            const uint4 l = lo ? alo[u][i] : make_uint4(0u, 0u, 0u, 0u);
            const uint4 h = hi ? ahi[u][i] : make_uint4(0u, 0u, 0u, 0u);
            const v8i a = (v8i){(int)l.x, (int)l.y, (int)l.z, (int)l.w, (int)h.x, (int)h.y, (int)h.z, (int)h.w};
            acc[j][i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc[j][i], 0, 4, 0, E8M0_ONE, 0, sc);
          }
        }
      }
    }
  }

  if constexpr (SK == 1) {
    // C layout of a 16x16 tile: lane holds column lane % 16, rows 4g .. 4g + 3: store straight from registers; the
    // row ids and scales come from the lanes that loaded them (lane 4g + q holds row 4g + q)
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int fr = __shfl(fr_in[i], 4 * g + q, WAVE);
        const float sc = __shfl(rsc[i], 4 * g + q, WAVE);
        if (fr < 0 || fr >= numel) continue;
        if constexpr (FUSE == 1) {
          const int n = blockIdx.x * 16 + r, Nh = N / 2;
          if (n < Nh)
            reinterpret_cast<float*>(C)[(size_t)fr * Nh + n] =
                silu_mul(bf2f(f2bf(acc[0][i][q] * sc)), bf2f(f2bf(acc[1][i][q] * sc)));
        } else {
#pragma unroll
          for (int j = 0; j < NPW; j++) {
            const int n = (blockIdx.x * NPW + j) * 16 + r;
            if (n < N) C[(size_t)fr * N + n] = f2bf(acc[j][i][q] * sc);
          }
        }
      }
  } else {
    __shared__ int s_fr[MT * 16];
    __shared__ float s_sc[MT * 16];
    if (wave == 0 && g == 0) {
#pragma unroll
      for (int i = 0; i < MT; i++) {
        s_fr[i * 16 + r] = fr_in[i];
        s_sc[i * 16 + r] = rsc[i];
      }
    }
    // partial tiles to LDS as [row][col], then each thread sums SK partials of some outputs
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
    if constexpr (FUSE == 1) {
      // gate (tile 0) and up (tile 1) partials of the same row and column, summed in the unfused kernel's order
      const int Nh = N / 2;
      for (int idx = tid; idx < MT * 256; idx += WAVE * SK) {
        const int col = idx & 15, row = (idx >> 4) & 15, i = idx >> 8;
        const int n = blockIdx.x * 16 + col;
        if (n >= Nh) continue;
        const int fr = s_fr[i * 16 + row];
        if (fr < 0 || fr >= numel) continue;
        float vg = 0.f, vu = 0.f;
#pragma unroll
        for (int s = 0; s < SK; s++) {
          vg += red[(size_t)s * TOT + idx];
          vu += red[(size_t)s * TOT + MT * 256 + idx];
        }
        const float sc = s_sc[i * 16 + row];
        reinterpret_cast<float*>(C)[(size_t)fr * Nh + n] = silu_mul(bf2f(f2bf(vg * sc)), bf2f(f2bf(vu * sc)));
      }
      __syncthreads();                                     // LDS reused by the workgroup's next tile
      return true;
    }
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
      C[(size_t)fr * N + n] = f2bf(v * s_sc[i * 16 + row]);
    }
    __syncthreads();                                       // LDS reused by the workgroup's next tile
  }
  return true;
}

// The grid's rows walk the launch's ny = max_blocks * subs tile rows grid-stride (the host caps the grid at
// MAX_WG workgroups), in ascending order, and a workgroup stops at the first row past ntpp: a launch over a layout
// whose blocks all lie past ntpp (the table layout the device did not keep) ends after one table read a workgroup.
template <int MT, int NPW, int SK, int U, int FUSE>
__global__ void __launch_bounds__(WAVE * SK) moe_mxfp4_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint8_t* __restrict__ Ws, uint16_t* __restrict__ C, const int* __restrict__ sorted_ids,
    const int* __restrict__ expert_ids, const int* __restrict__ ntpp, const float* __restrict__ topk_w,
    long wq_estride, long ws_estride, int numel, int a_row_div, int K, int N, int blk, int subs, int ny) {
  for (int by = blockIdx.y; by < ny; by += gridDim.y)
    if (!moe_tile<MT, NPW, SK, U, FUSE>(A, As, Wq, Ws, C, sorted_ids, expert_ids, ntpp, topk_w, wq_estride,
                                        ws_estride, numel, a_row_div, K, N, blk, subs, by))
      break;
}

struct Pick { int MT, NPW, SK, U; };

// 1 when the environment variable is set to "0" (a switch turned off), else 0.
int getenv_flag_off(const char* name) {
  const char* v = getenv(name);
  return v && v[0] == '0' ? 1 : 0;
}

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}

// Launch shape for the decode-family kernel, from the host-known shape only (graph-capturable). Two column tiles a
// wave. Long K (>= 8 K-tiles) splits over SK waves so that fewer dependent load batches sit on one wave: 4 while the
// grid is small, 2 once it holds >= 12K waves' worth of tiles, in 4-tile load batches below 4K tiles (config 2 at
// T <= 8: one memory round trip a wave) and 2-tile batches above; short K stays in one wave (no LDS reduction), with
// 4-tile load batches while the grid is small. Measured on MI355X over config-2 decode widths (T = 1..64).
// A caller's shape (req: U, SK, NPW all > 0, from the tuned table) replaces this choice. R9K_GEMM_SK / R9K_GEMM_NPW /
// R9K_GEMM_U override both (tuning sweeps).
Pick pick(int MT, int N, int K, int max_blocks, const Pick* req = nullptr) {
  const int nkt = (K + KT - 1) / KT;
  const int NT = N / 16;
  int NPW = NT >= 2 ? 2 : 1;
  const long tiles = (long)max_blocks * ((NT + NPW - 1) / NPW);
  int SK, U;
  if (nkt >= 8) {
    SK = tiles >= 12288 ? 2 : 4;
    U = tiles < 4096 ? 4 : 2;                              // small grids: a wave's K range in one load batch
  } else {
    SK = 1;
    U = tiles >= 8192 ? 1 : 4;
  }
  if (MT >= 4) U = U > 2 ? 2 : U;
  if (req) {
    U = req->U;
    SK = req->SK;
    NPW = req->NPW;
  }
  SK = env_int("R9K_GEMM_SK", SK);
  NPW = env_int("R9K_GEMM_NPW", NPW);
  U = env_int("R9K_GEMM_U", U);
  return {MT, NPW, SK, U};
}

template <int MT, int NPW, int SK, int U, int FUSE = 0>
int launch_one(dim3 grid, hipStream_t st, long a, long as, long wq, long ws, long c, long sorted_ids,
               long expert_ids, long ntpp, long topk_w, long wq_estride, long ws_estride, int numel, int a_row_div,
               int K, int N, int blk, int subs, int ny) {
  const size_t smem = SK > 1 ? (size_t)SK * NPW * MT * 256 * sizeof(float) : 0;
  hipLaunchKernelGGL((moe_mxfp4_kernel<MT, NPW, SK, U, FUSE>), grid, dim3(WAVE * SK), smem, st, (const uint8_t*)a,
                     (const float*)as, (const uint8_t*)wq, (const uint8_t*)ws, (uint16_t*)c, (const int*)sorted_ids,
                     (const int*)expert_ids, (const int*)ntpp, (const float*)topk_w, wq_estride, ws_estride, numel,
                     a_row_div, K, N, blk, subs, ny);
  return 0;
}

// Host dispatch shared by the decode (blk = 16 * MT) and prefill (blk = cfg BM) entries, and the fused decode
// variants (fuse 1 / 2, MT = 1; see moe_mxfp4_kernel).
// ws_estride: bytes per expert of the packed scale tensor; the code stride is N * K / 2 bytes.
int moe_dispatch(long a, long as, long wq, long ws, long c, long sorted_ids, long expert_ids, long ntpp, long topk_w,
                 long ws_estride, int max_blocks, int numel, int a_row_div, int K, int N, int MT, int blk,
                 long stream, int fuse = 0, const Pick* req = nullptr) {
  if (N % 16 || N <= 0) return -1;
  if (K % GROUP || K <= 0) return -2;
  if (MT != 1 && MT != 2 && MT != 4) return -7;
  if (blk % (16 * MT)) return -7;
  if (a_row_div < 1) return -3;
  if (fuse < 0 || fuse > 2) return -8;
  if (fuse && MT != 1) return -7;
  if (fuse == 1 && N % 32) return -1;                       // gate and up halves of whole 16-column tiles
  if (max_blocks <= 0 || numel <= 0) return 0;
  if (!a || (!as && fuse != 2) || !wq || !ws || !c || !sorted_ids || !expert_ids || !ntpp) return -3;
  Pick p = pick(MT, N, K, max_blocks, req);
  if (fuse == 1) p.NPW = 2;
  const int subs = blk / (16 * MT);
  const long ny = (long)max_blocks * subs;
  if (ny > 0x7fffffffL || p.NPW < 1) return -3;
  const unsigned gx = fuse == 1 ? N / 32 : (N / 16 + p.NPW - 1) / p.NPW;
  const long cap_y = MAX_WG / (long)gx > 0 ? MAX_WG / (long)gx : 1;
  const dim3 grid(gx, (unsigned)(ny < cap_y ? ny : cap_y));
  const long wq_estride = (long)N * K / 2;
  const hipStream_t st = (hipStream_t)stream;
  if (fuse) {
#define F(FV, NPWv, SKv, Uv)                                                                                      \
  if (fuse == FV && p.NPW == NPWv && p.SK == SKv && p.U == Uv)                                                    \
    return launch_one<1, NPWv, SKv, Uv, FV>(grid, st, a, as, wq, ws, c, sorted_ids, expert_ids, ntpp, topk_w,     \
                                            wq_estride, ws_estride, numel, a_row_div, K, N, blk, subs, (int)ny);
#define FU(FV, NPWv, SKv) F(FV, NPWv, SKv, 1) F(FV, NPWv, SKv, 2) F(FV, NPWv, SKv, 4)
#define FS(FV, NPWv) FU(FV, NPWv, 1) FU(FV, NPWv, 2) FU(FV, NPWv, 4)
    FS(1, 2) FS(2, 1) FS(2, 2) FS(2, 4)
#undef FS
#undef FU
#undef F
    return -5;
  }
#define L(MTv, NPWv, SKv, Uv)                                                                               \
  if (p.MT == MTv && p.NPW == NPWv && p.SK == SKv && p.U == Uv)                                             \
    return launch_one<MTv, NPWv, SKv, Uv>(grid, st, a, as, wq, ws, c, sorted_ids, expert_ids, ntpp, topk_w, \
                                          wq_estride, ws_estride, numel, a_row_div, K, N, blk, subs, (int)ny);
#define LU(MTv, NPWv, SKv) L(MTv, NPWv, SKv, 1) L(MTv, NPWv, SKv, 2) L(MTv, NPWv, SKv, 4)
#define LS(MTv, NPWv) LU(MTv, NPWv, 1) LU(MTv, NPWv, 2) LU(MTv, NPWv, 4)
  LS(1, 1) LS(1, 2) LS(1, 4) LS(2, 1) LS(2, 2) LS(2, 4) LS(4, 1) LS(4, 2)
#undef LS
#undef LU
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

int r9k_prefill_launch(long a, long as, long wq, long ws, long c, long sorted_ids, long expert_ids, long ntpp,
                       long topk_w, long ws_estride, int max_blocks, int numel, int a_row_div, int K, int N,
                       long stream);
int r9k_prefill_block_rows();
int r9k_nvfp4_prefill_launch(long a, long as, long wq, long ws, long wg, long c, long sorted_ids, long expert_ids,
                             long ntpp, long topk_w, long ws_estride, long wg_estride, int max_blocks, int numel,
                             int a_row_div, int K, int N, int blk, long stream);

// MT bit 5: (WV, SK, NPW) carry this library's launch shape. The reference never sets it and passes its gfx1201 tile
// knobs in those arguments, which then mean nothing here.
constexpr int MT_SHAPE = 32;

// Reference: kernels/r9k_moe_mxfp4a8.hip:625-638 (r9k_moe_mxfp4a8). With MT & MT_SHAPE, (WV, SK, NPW) is the launch
// shape with gfx950 meanings: WV = K-tiles per load batch, SK = waves splitting K, NPW = 16-column tiles per wave,
// each 1, 2 or 4 (the built shapes; another value returns -5; a shape changes only the fp32 summation order of
// SK > 1). Without it the kernel picks the shape and (WV, SK, NPW) are ignored, as are `wref` and the MT bits 3
// (LDS-A) and 4 (fold): the reference's gfx1201 knobs. MT & 7 in {1, 2, 4} sets the routing block (16 * MT rows).
// ws_estride: bytes per expert of the scale tensor. 0 / negative error code.
extern "C" int r9k_moe_mxfp4a8(long a, long as, long wq, long ws, long wref, long c, long sorted_ids, long expert_ids,
                               long ntpp, long topk_w, long ws_estride, long wref_estride, int max_blocks, int numel,
                               int a_row_div, int K, int N, int WV, int SK, int NPW, int MT, long stream) {
  (void)wref; (void)wref_estride;
  const int mt = MT & 7;
  const Pick req{mt, NPW, SK, WV};
  const bool given = (MT & MT_SHAPE) != 0;
  if (given && !(WV > 0 && SK > 0 && NPW > 0)) return -5;
  const int rc = moe_dispatch(a, as, wq, ws, c, sorted_ids, expert_ids, ntpp, topk_w, ws_estride, max_blocks, numel,
                              a_row_div, K, N, mt, 16 * mt, stream, 0, given ? &req : nullptr);
  if (rc) return rc;
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

// Reference: kernels/r9k_moe_mxfp4a8.hip:618-626 (r9k_moe_mxfp4a8_f). fuse 1: gate_up with silu(g) * u in the
// epilogue, c = fp32 [numel, N / 2]; fuse 2: down with fp32 A rows [numel, K] quantised per row on load (as
// ignored). Decode routing blocks only (MT & 7 == 1); the tile knobs are ignored as in r9k_moe_mxfp4a8. -8 for
// another fuse value.
extern "C" int r9k_moe_mxfp4a8_f(int fuse, long a, long as, long wq, long ws, long wref, long c, long sorted_ids,
                                 long expert_ids, long ntpp, long topk_w, long ws_estride, long wref_estride,
                                 int max_blocks, int numel, int a_row_div, int K, int N, int WV, int SK, int NPW,
                                 int MT, long stream) {
  (void)wref; (void)wref_estride; (void)WV; (void)SK; (void)NPW;
  if (fuse < 1 || fuse > 2) return -8;
  if ((MT & 7) != 1) return -7;
  const int rc = moe_dispatch(a, as, wq, ws, c, sorted_ids, expert_ids, ntpp, topk_w, ws_estride, max_blocks, numel,
                              a_row_div, K, N, 1, 16, stream, fuse);
  if (rc) return rc;
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

// Reference: kernels/r9k_moe_mxfp4a8.hip:1227-1268. nv: 0 MXFP4, 2 MXFP4 with folded exponents (same data here:
// the block exponents are applied exactly either way), 1 NVFP4 and 3 fp8 weights are not served (-8).
extern "C" int r9k_moe_4bit_prefill(int nv, long a, long as, long wq, long ws, long wref, long c, long sorted_ids,
                                    long expert_ids, long ntpp, long topk_w, long ws_estride, long wref_estride,
                                    int max_blocks, int numel, int a_row_div, int K, int N, int cfg, long stream) {
  if (N % 16) return -1;
  if (cfg < 0 || cfg >= NPF) return -7;
  if (K % kPf[cfg].BK) return -2;
  // native NVFP4 (ws = its scales, wref = the per-row fp32 multipliers): the fp16-MFMA tile kernel, 128- or 256-row
  // routing blocks (r9k_moe_nvfp4.hip)
  if (nv == 1)
    return r9k_nvfp4_prefill_launch(a, as, wq, ws, wref, c, sorted_ids, expert_ids, ntpp, topk_w, ws_estride,
                                    wref_estride, max_blocks, numel, a_row_div, K, N, kPf[cfg].BM, stream);
  if (nv != 0 && nv != 2) return -8;
  // 256-row blocks with K a multiple of 128: the LDS-tiled 32x32x64 kernel (r9k_moe_prefill.hip)
  if (kPf[cfg].BM == r9k_prefill_block_rows() && K % 128 == 0 && getenv_flag_off("R9K_PREFILL_LDS") == 0)
    return r9k_prefill_launch(a, as, wq, ws, c, sorted_ids, expert_ids, ntpp, topk_w, ws_estride, max_blocks, numel,
                              a_row_div, K, N, stream);
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
