// r9k_moe_stream.hip -- the grouped MXFP4 x fp8 decode GEMMs as block streams: one workgroup walks one 16-row routing
// block's expert (or a column slice of it) from end to end, a long read of HBM with one table lookup at its start.
//
//   plain   (r9k_moe_stream epi 0): out[r, n] = bf16((sum_k A_q[r / a_row_div, k] * W_e[n, k]) * (As[.] (* topk_w[r])))
//   gate_up (r9k_moe_stream epi 1): g, u = bf16 of the plain product's gate column n and up column n + N/2
//                                   aq, as = per-row e4m3 quant of h = silu(g) * u (amax = max(max |h|, 1e-12),
//                                   aq = e4m3(h * (448 / amax)), as = amax / 448: the standalone SiLU + quant rule)
//   layer   (r9k_moe_stream_layer): gate_up + SiLU + quant, then the down product of the same block's rows with the
//                                   router weight, down[r, n] = bf16((sum_k aq[r, k] * W2_e[n, k]) * (as[r] * tw[r]))
//
// Why: a decode step touches most experts with one or two rows each (config 2 at T = 64: 241 of 288 experts, 512
// routed rows), so its GEMMs are weight streams. gate_up and down walk the same routing tables, so block b's down
// rows need only block b's gate_up rows: one workgroup can run both GEMMs of a block with the SiLU-quantised rows
// handed over in LDS, with no launch, no grid-wide wait and no HBM round trip in between.
//
// Structure of a workgroup (16 waves):
//   * the block's 16 activation rows are gathered once into LDS (rows padded by 16 bytes against bank conflicts);
//   * units of TG column tiles are claimed from an LDS counter. Measured on MI355X, the waves of one workgroup are
//     served very unevenly by the memory system (their finish times spread over ~20 us of a ~35 us stream, also in a
//     bare read kernel), so statically owned tiles leave the CU's share of HBM idle while the slowest wave finishes;
//     claimed units keep the block's bytes in flight to its last tile. The values do not depend on which wave runs a
//     unit;
//   * a unit streams its tiles' 1 KB fragments (the decode kernel's layout) in batches of U K-tiles, and while one
//     batch's MFMAs (V_MFMA_SCALE_F32_16X16X128_F8F6F4, e8m0 exponent as the B scale, A fragments from LDS) run, the
//     next batch's loads are in flight. Each tile's K-tiles go into one accumulator in ascending order: the decode
//     kernel's single-wave MFMA chain, so the plain product equals r9k_moe_mxfp4a8's SK = 1 launch bit for bit;
//   * gate_up keeps bf16(acc * As) of every tile in LDS (the values the plain kernel would store), then forms
//     h = silu(g) * u, the row maxima (LDS atomic max on the bit patterns of |h|, which is fmaxf's rule: NaN passes
//     over) and the codes.
#include "r9k_common.h"

#include <cstdlib>
#include <type_traits>

namespace {

using namespace r9k;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int NW = 16;             // waves a workgroup
constexpr int KT = 128;            // K per MFMA
constexpr int BLK = 16;            // rows per routing block
constexpr int E8M0_ONE = 127;      // scale byte of 2^0
constexpr int APAD = 16;           // LDS row padding of staged rows
constexpr int ACH = 4;             // activation staging chunks a thread at most: K <= ACH * NW * 64
constexpr int HCH = 2;             // 8-value activation chunks a thread at most: I <= HCH * NW * 64 * 8 / 16
constexpr long MAX_WG = 16384;     // workgroups of one launch at most; more blocks are walked grid-stride
constexpr int LDS_MAX = 96 * 1024;

// The block's 16 rows of activation codes (K bytes each) into LDS at `dst` (row stride K + APAD), in two halves so
// the caller can put other loads between them: stage_load issues every load of a thread (padding rows read the
// block's first row), stage_store writes them. Chunks past the rows clamp to the last chunk, whose own bytes those
// threads store again, so no load or store sits under a branch (a load under a branch is waited for inside it).
struct Staged {
  uint4 av[ACH];
  int at[ACH];
};
__device__ __forceinline__ void stage_load(Staged& sg, const uint8_t* __restrict__ A, int fr_l, int first, int numel,
                                           int a_row_div, int K, int tid) {
  const int cpr = K / 16, astride = K + APAD;
#pragma unroll
  for (int it = 0; it < ACH; it++) {
    const int c = min(tid + it * NW * WAVE, BLK * cpr - 1);
    const int i = c / cpr, q = c - i * cpr;
    int fr = __shfl(fr_l, i, WAVE);
    if (fr < 0 || fr >= numel) fr = first;
    sg.av[it] = reinterpret_cast<const uint4*>(A + (size_t)(fr / a_row_div) * K)[q];
    sg.at[it] = i * astride + q * 16;
  }
}
__device__ __forceinline__ void stage_store(const Staged& sg, uint8_t* dst) {
#pragma unroll
  for (int it = 0; it < ACH; it++) *reinterpret_cast<uint4*>(dst + sg.at[it]) = sg.av[it];
}

// Per-row factors of the block for the lanes r < 16 of every wave (loaded unconditionally, from the block's first
// row for padding rows): the token's activation scale and, with topk_w, the router weight.
__device__ __forceinline__ void row_factors(const float* __restrict__ As, const float* __restrict__ topk_w, int fr_l,
                                            int first, int numel, int a_row_div, float& as, float& tw) {
  const bool live = fr_l >= 0 && fr_l < numel;
  const int fr = live ? fr_l : first;
  as = As[fr / a_row_div];
  tw = topk_w ? topk_w[fr] : 1.f;
}

// Unit claim: lane 0 takes the next unit index from the workgroup's counter; the value is wave-uniform.
__device__ __forceinline__ int claim(int* counter, int lane) {
  int v = 0;
  if (lane == 0) v = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  return __builtin_amdgcn_readfirstlane(__shfl(v, 0, WAVE));
}

// Register sets of a unit stream: two batches of U K-tiles x TG column tiles (codes + exponent bytes).
template <int TG, int U>
struct Batches {
  u32x4 bf[2][U][TG];
  uint32_t sb[2][U][TG];
};

// An expert's codes and exponents as buffer resources (num_records = their bytes): a load names its 32-bit offset
// only, and one at or past the range returns zeros without touching memory.
struct ExpertRsrc {
  __amdgpu_buffer_rsrc_t w, s;
  uint32_t wbytes, sbytes;
};
__device__ __forceinline__ ExpertRsrc expert_rsrc(const uint8_t* Wq, const uint8_t* Ws, long wq_estride,
                                                  long ws_estride, int e) {
  ExpertRsrc x;
  x.wbytes = (uint32_t)wq_estride;
  x.sbytes = (uint32_t)ws_estride;
  x.w = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(Wq + (size_t)e * wq_estride), (short)0,
                                          (int)x.wbytes, 0x00020000);
  x.s = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(Ws + (size_t)e * ws_estride), (short)0,
                                          (int)x.sbytes, 0x00020000);
  return x;
}

// The loads of batch b (K-tiles b * U .. + U - 1) of unit `un` (column tiles tile0 + un * TG + j) into set P,
// non-temporal. A unit at or past `units` loads at the end of the expert's range instead, which returns zeros with
// no memory access: every batch issues the same loads, so the compiler's waits stay exact counts. The offset is
// integer arithmetic with a mask (all ones for a real unit), since a select there is turned into a branch around
// every load, which then waits inside it.
template <int P, int TG, int U>
__device__ __forceinline__ void load_batch(Batches<TG, U>& bs, int un, int b, int units, int tile0,
                                           const ExpertRsrc& x, uint32_t kbytes, uint32_t sbytes, int lane) {
  const uint32_t m = 0u - (uint32_t)(un < units);
  const uint32_t woff = (uint32_t)lane * 16u;
#pragma unroll
  for (int u = 0; u < U; u++)
#pragma unroll
    for (int j = 0; j < TG; j++) {
      const uint32_t k = (uint32_t)(b * U + u);
      const uint32_t nt = (uint32_t)(tile0 + un * TG + j);
      const uint32_t wo = ((nt * kbytes + k * 1024u) & m) | (x.wbytes & ~m);
      const uint32_t so = ((nt * sbytes + k * 64u) & m) | (x.sbytes & ~m);
      bs.bf[P][u][j] = __builtin_amdgcn_raw_buffer_load_b128(x.w, (int)(wo + woff), 0, 2);
      bs.sb[P][u][j] = __builtin_amdgcn_raw_buffer_load_b8(x.s, (int)(so + (uint32_t)lane), 0, 2);
    }
}

// One wave's part of a block's units. Units 0 .. NW-1 go to waves 0 .. NW-1 before any claim, and with nb == 1
// batch a unit also units NW .. 2 NW - 1 (first_units); further units are claimed from the counter, which the caller
// set to first_units(...). On entry the wave's first two batches are in flight (issue_first: set 0 = batch 0 of unit
// `wave`, set 1 = its successor), so a barrier the caller puts between issue_first and this call does not empty the
// wave's queue. Unit `un` covers column tiles tile0 + un * TG .. + TG - 1 over nkt K-tiles (nkt % U == 0) in batches
// of U; A fragments from the LDS rows at `arow` (lane r's row, 16 g bytes in). The two sets alternate, so while one
// batch's MFMAs run the next batch's loads are in flight. done(un, acc) runs after a unit's last batch.
__device__ __forceinline__ int first_units(int nkt, int U) { return nkt / U == 1 ? 2 * NW : NW; }

template <int TG, int U>
__device__ __forceinline__ void issue_first(Batches<TG, U>& bs, int wave, int units, int tile0, int nkt,
                                            const ExpertRsrc& x, uint32_t kbytes, uint32_t sbytes, int lane) {
  load_batch<0>(bs, wave, 0, units, tile0, x, kbytes, sbytes, lane);
  if (nkt / U > 1) load_batch<1>(bs, wave, 1, units, tile0, x, kbytes, sbytes, lane);
  else load_batch<1>(bs, wave + NW, 0, units, tile0, x, kbytes, sbytes, lane);
}

template <int TG, int U, class Done>
__device__ __forceinline__ void stream_units(Batches<TG, U>& bs, int wave, int* counter, int units, int tile0,
                                             int nkt, const ExpertRsrc& x, uint32_t kbytes, uint32_t sbytes,
                                             const uint8_t* arow, int lane, Done&& done) {
  const int nb = nkt / U;
  v4f acc[TG];
  auto compute = [&](auto pc, int b) {
    constexpr int P = decltype(pc)::value;
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = b * U + u;
      const uint4 lo = *reinterpret_cast<const uint4*>(arow + k * KT);
      const uint4 hi = *reinterpret_cast<const uint4*>(arow + k * KT + 64);
      const v8i a = (v8i){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
#pragma unroll
      for (int j = 0; j < TG; j++) {
        const v8i bv = (v8i){(int)bs.bf[P][u][j].x, (int)bs.bf[P][u][j].y, (int)bs.bf[P][u][j].z,
                             (int)bs.bf[P][u][j].w, 0, 0, 0, 0};
        acc[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, bv, acc[j], 0, 4, 0, E8M0_ONE, 0,
                                                                  (int)bs.sb[P][u][j]);
      }
    }
  };
  auto reset = [&]() {
#pragma unroll
    for (int j = 0; j < TG; j++) acc[j] = (v4f){0.f, 0.f, 0.f, 0.f};
  };
  // (un, b): the batch in the set about to be computed; (un2, b2): the one after it
  int un = wave, b = 0;
  int un2 = nb > 1 ? wave : wave + NW, b2 = nb > 1 ? 1 : 0;
  auto advance = [&]() {
    if (b2 + 1 < nb) {
      b2++;
    } else {
      un2 = claim(counter, lane);
      b2 = 0;
    }
  };
  if (un >= units) return;
  reset();
  // set 0 holds (un, b), set 1 holds (un2, b2)
  for (;;) {
    compute(std::integral_constant<int, 0>{}, b);
    if (b == nb - 1) {
      done(un, acc);
      reset();
    }
    if (un2 >= units) break;
    un = un2;
    b = b2;
    advance();
    load_batch<0>(bs, un2, b2, units, tile0, x, kbytes, sbytes, lane);
    compute(std::integral_constant<int, 1>{}, b);
    if (b == nb - 1) {
      done(un, acc);
      reset();
    }
    if (un2 >= units) break;
    un = un2;
    b = b2;
    advance();
    load_batch<1>(bs, un2, b2, units, tile0, x, kbytes, sbytes, lane);
  }
}

// The SiLU + quant of a block held in LDS as bf16 gate_up rows gu [16][N] (gate = columns 0 .. I-1, up = I .. N-1):
// h = silu(g) * u, each row's max |h| (LDS atomic max on the bit patterns of the non-negative |h|, fmaxf's rule:
// a NaN is passed over), amax = max(rowmax, 1e-12), codes e4m3(h * (448 / amax)) as 8-byte pieces through
// put(row, chunk, uint2) and the scale through put_scale(row, amax / 448), for live rows only. s_max[16] at 0 on
// entry; the caller's barrier precedes (gu complete) and follows (s_max reused).
template <class Put, class PutScale>
__device__ __forceinline__ void silu_quant_block(const uint16_t* gu, int N, uint32_t* s_max, const int* s_fr, int tid,
                                                 Put&& put, PutScale&& put_scale) {
  const int I = N / 2, cpr = I / 8;
  float h[HCH][8];
#pragma unroll
  for (int it = 0; it < HCH; it++) {
    const int c = tid + it * NW * WAVE;
    if (c < BLK * cpr) {
      const int i = c / cpr, q = c - i * cpr;
      const uint4 gv = *reinterpret_cast<const uint4*>(gu + i * N + 8 * q);
      const uint4 uv = *reinterpret_cast<const uint4*>(gu + i * N + I + 8 * q);
      const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        h[it][2 * j] = silu_mul(lo16(gw[j]), lo16(uw[j]));
        h[it][2 * j + 1] = silu_mul(hi16(gw[j]), hi16(uw[j]));
      }
      float m = 0.f;
#pragma unroll
      for (int j = 0; j < 8; j++) m = fmaxf(m, fabsf(h[it][j]));
      __hip_atomic_fetch_max(&s_max[i], __float_as_uint(m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < HCH; it++) {
    const int c = tid + it * NW * WAVE;
    if (c < BLK * cpr) {
      const int i = c / cpr, q = c - i * cpr;
      if (s_fr[i] >= 0) {
        const float amax = fmaxf(__uint_as_float(s_max[i]), 1e-12f);
        put(i, q, pack8_e4m3(h[it], 448.f / amax));
        if (q == 0) put_scale(i, amax / 448.f);
      }
    }
  }
}

// Table reads of block rb. Returns 0 past ntpp (every later block too), 1 for a block to skip (expert-map hole, all
// padding), 2 for a block to run; fr_l (lane r's row id) / first (the block's first row id) / e (its expert) are set
// for the caller.
__device__ __forceinline__ int block_head(int rb, const int* __restrict__ sorted_ids, const int* __restrict__ expert_ids,
                                          const int* __restrict__ ntpp, int numel, int r, int& fr_l, int& first, int& e) {
  const int np = ntpp[0];
  e = expert_ids[rb];
  fr_l = sorted_ids[rb * BLK + r];
  first = __shfl(fr_l, 0, WAVE);
  if (rb * BLK >= np) return 0;
  if (e < 0 || first < 0 || first >= numel) return 1;
  return 2;
}

template <int TG, int U, int EPI>
__global__ void __launch_bounds__(NW * WAVE) moe_stream_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint8_t* __restrict__ Ws, void* __restrict__ Cout, float* __restrict__ Cs, const int* __restrict__ sorted_ids,
    const int* __restrict__ expert_ids, const int* __restrict__ ntpp, const float* __restrict__ topk_w,
    long wq_estride, long ws_estride, int numel, int a_row_div, int K, int N, int units, int ny) {
  static_assert(EPI == 0 || TG == 1, "gate_up: one column tile a unit");
  extern __shared__ __align__(16) uint8_t lds[];           // [16][K + APAD] activation codes, then (epi 1) bf16 [16][N]
  __shared__ int s_fr[BLK];
  __shared__ float s_sc[BLK];
  __shared__ uint32_t s_max[BLK];
  __shared__ int s_next;

  const int tid = threadIdx.x, lane = tid % WAVE;
  const int g = lane >> 4, r = lane & 15;
  const int astride = K + APAD;
  const int tile0 = blockIdx.x * units * TG;                // first column tile of this workgroup's slice
  uint16_t* gu = reinterpret_cast<uint16_t*>(lds + BLK * astride);
  // plain output through a buffer resource: a padding row stores at the end of the range, which the hardware drops,
  // so every unit issues the same stores (no branch for the waits to merge over)
  const uint32_t cbytes = (uint32_t)((size_t)numel * N * 2);
  const auto crs = __builtin_amdgcn_make_buffer_rsrc(Cout, (short)0, (int)cbytes, 0x00020000);

  const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
  if (tid == 0) s_next = first_units(K / KT, U);            // the units each wave owns before any claim
  Batches<TG, U> bs;

  for (int rb = blockIdx.y; rb < ny; rb += gridDim.y) {
    int fr_l, first, e;
    const int hd = block_head(rb, sorted_ids, expert_ids, ntpp, numel, r, fr_l, first, e);
    if (hd == 0) break;
    if (hd == 1) continue;
    const ExpertRsrc x = expert_rsrc(Wq, Ws, wq_estride, ws_estride, e);
    // the rows' loads first, then this wave's first unit: the staging waits only for its own loads (vmcnt counts in
    // issue order) while the weight bytes arrive behind them
    Staged sg;
    stage_load(sg, A, fr_l, first, numel, a_row_div, K, tid);
    float ras, rtw;
    row_factors(As, EPI == 0 ? topk_w : nullptr, fr_l, first, numel, a_row_div, ras, rtw);
    issue_first(bs, wave, units, tile0, K / KT, x, 8u * K, K / 2, lane);
    stage_store(sg, lds);
    if (tid < BLK) {
      s_fr[tid] = fr_l >= 0 && fr_l < numel ? fr_l : -1;
      s_sc[tid] = ras * rtw;
      s_max[tid] = 0u;
    }
    __syncthreads();

    stream_units<TG, U>(bs, wave, &s_next, units, tile0, K / KT, x, 8u * K, K / 2, lds + r * astride + 16 * g, lane,
                        [&](int un, const v4f (&acc)[TG]) {
      // C layout: lane holds column lane % 16 of rows 4g .. 4g + 3
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int row = 4 * g + q;
        const float sc = s_sc[row];
        if constexpr (EPI == 0) {
          const int fr = s_fr[row];
#pragma unroll
          for (int j = 0; j < TG; j++) {
            const uint32_t off = fr >= 0 ? ((uint32_t)fr * N + (tile0 + un * TG + j) * 16 + r) * 2u : cbytes;
            __builtin_amdgcn_raw_buffer_store_b16(f2bf(acc[j][q] * sc), crs, (int)off, 0, 0);
          }
        } else {
          gu[row * N + (tile0 + un) * 16 + r] = f2bf(acc[0][q] * sc);
        }
      }
    });

    if constexpr (EPI == 1) {
      __syncthreads();
      uint8_t* Q = reinterpret_cast<uint8_t*>(Cout);
      const int I = N / 2;
      silu_quant_block(gu, N, s_max, s_fr, tid,
                       [&](int i, int q, uint2 v) { reinterpret_cast<uint2*>(Q + (size_t)s_fr[i] * I)[q] = v; },
                       [&](int i, float s) { Cs[s_fr[i]] = s; });
    }
    __syncthreads();                                        // every claim and LDS read of this block done
    if (tid == 0) s_next = first_units(K / KT, U);          // for the next block (its staging barrier follows)
  }
}

// gate_up (U1 K-tiles a batch, one tile a unit) -> SiLU + quant into LDS -> down (TG2 tiles a unit, U2 K-tiles a
// batch) for one routing block per workgroup. LDS: the gathered x rows [16][K1 + APAD], the bf16 gate_up tile
// [16][N1], the codes [16][I + APAD].
template <int U1, int TG2, int U2>
__global__ void __launch_bounds__(NW * WAVE) moe_stream_layer_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ W1q,
    const uint8_t* __restrict__ W1s, const uint8_t* __restrict__ W2q, const uint8_t* __restrict__ W2s,
    uint16_t* __restrict__ C, const int* __restrict__ sorted_ids, const int* __restrict__ expert_ids,
    const int* __restrict__ ntpp, const float* __restrict__ topk_w, long w1q_estride, long w1s_estride,
    long w2q_estride, long w2s_estride, int numel, int a_row_div, int K1, int N1, int N2, int ny) {
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ int s_fr[BLK];
  __shared__ float s_sc[BLK];                               // gate_up: As of the row's token
  __shared__ float s_sc2[BLK];                              // down: as * topk_w
  __shared__ float s_tw[BLK];
  __shared__ uint32_t s_max[BLK];
  __shared__ int s_next[2];

  const int tid = threadIdx.x, lane = tid % WAVE;
  const int g = lane >> 4, r = lane & 15;
  const int I = N1 / 2;
  const int a1stride = K1 + APAD, a2stride = I + APAD;
  uint16_t* gu = reinterpret_cast<uint16_t*>(lds + BLK * a1stride);
  uint8_t* aq = lds + BLK * a1stride + BLK * N1 * 2;
  const uint32_t cbytes = (uint32_t)((size_t)numel * N2 * 2);
  const auto crs = __builtin_amdgcn_make_buffer_rsrc(C, (short)0, (int)cbytes, 0x00020000);

  const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
  // the units each wave owns before any claim, per GEMM
  if (tid < 2) s_next[tid] = tid == 0 ? first_units(K1 / KT, U1) : first_units(N1 / 2 / KT, U2);
  Batches<1, U1> b1;
  Batches<TG2, U2> b2;
  const int units1 = N1 / 16, units2 = N2 / (16 * TG2);

  for (int rb = blockIdx.y; rb < ny; rb += gridDim.y) {
    int fr_l, first, e;
    const int hd = block_head(rb, sorted_ids, expert_ids, ntpp, numel, r, fr_l, first, e);
    if (hd == 0) break;
    if (hd == 1) continue;
    const ExpertRsrc x1 = expert_rsrc(W1q, W1s, w1q_estride, w1s_estride, e);
    const ExpertRsrc x2 = expert_rsrc(W2q, W2s, w2q_estride, w2s_estride, e);
    // the rows' loads first, then this wave's first gate_up unit: the staging waits only for its own loads (vmcnt
    // counts in issue order) while the weight bytes arrive behind them
    Staged sg;
    stage_load(sg, A, fr_l, first, numel, a_row_div, K1, tid);
    float ras, rtw;
    row_factors(As, topk_w, fr_l, first, numel, a_row_div, ras, rtw);
    issue_first(b1, wave, units1, 0, K1 / KT, x1, 8u * K1, K1 / 2, lane);
    stage_store(sg, lds);
    if (tid < BLK) {
      s_sc[tid] = ras;
      s_tw[tid] = rtw;
      s_fr[tid] = fr_l >= 0 && fr_l < numel ? fr_l : -1;
      s_max[tid] = 0u;
    }
    __syncthreads();

    // gate_up
    stream_units<1, U1>(b1, wave, &s_next[0], units1, 0, K1 / KT, x1, 8u * K1, K1 / 2, lds + r * a1stride + 16 * g,
                        lane, [&](int un, const v4f (&acc)[1]) {
#pragma unroll
      for (int q = 0; q < 4; q++) gu[(4 * g + q) * N1 + un * 16 + r] = f2bf(acc[0][q] * s_sc[4 * g + q]);
    });
    // this wave's first down batches go out before the SiLU: their bytes arrive during the barriers and the activation
    issue_first(b2, wave, units2, 0, I / KT, x2, 8u * I, I / 2, lane);
    __syncthreads();

    // SiLU + quant into LDS; padding rows' codes are never read for a stored output
    silu_quant_block(gu, N1, s_max, s_fr, tid,
                     [&](int i, int q, uint2 v) { *reinterpret_cast<uint2*>(aq + i * a2stride + 8 * q) = v; },
                     [&](int i, float s) { s_sc2[i] = s * s_tw[i]; });
    __syncthreads();

    // down: the row scale is the quant scale times the router weight, the down GEMM's order (As * topk_w)
    stream_units<TG2, U2>(b2, wave, &s_next[1], units2, 0, I / KT, x2, 8u * I, I / 2, aq + r * a2stride + 16 * g,
                          lane, [&](int un, const v4f (&acc)[TG2]) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int row = 4 * g + q;
        const int fr = s_fr[row];
        const float sc = s_sc2[row];
#pragma unroll
        for (int j = 0; j < TG2; j++) {
          const uint32_t off = fr >= 0 ? ((uint32_t)fr * N2 + (un * TG2 + j) * 16 + r) * 2u : cbytes;
          __builtin_amdgcn_raw_buffer_store_b16(f2bf(acc[j][q] * sc), crs, (int)off, 0, 0);
        }
      }
    });
    __syncthreads();                                        // every claim and LDS read of this block done
    if (tid < 2) s_next[tid] = tid == 0 ? first_units(K1 / KT, U1) : first_units(I / KT, U2);   // for the next block
  }
}

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}

// K-tiles a load batch: a power of two dividing nkt, at most `cap` (TG * U = 4 fragments a batch: one batch computed
// while the next is in flight fits 128 VGPRs, 4 waves a SIMD).
int batch_of(int nkt, int cap) {
  int u = cap;
  while (u > 1 && nkt % u) u /= 2;
  return u;
}

struct Shape { int TG, U, slices; };

// Launch shape of r9k_moe_stream: gate_up (epi 1) takes whole rows, one tile a unit; the plain product takes units
// of up to 4 fragments a batch and splits the columns into slices only while the expected blocks (min(E, numel))
// would leave CUs idle. R9K_STREAM_TG / _U / _SLICES override (sweeps).
Shape pick_shape(int epi, int N, int K, int blocks_hint) {
  const int NT = N / 16, nkt = K / KT;
  Shape s{1, 8, 1};
  if (epi == 0) {
    s.TG = nkt >= 8 ? 1 : (nkt >= 4 ? 2 : 4);
    while (s.slices < 4 && (long)blocks_hint * s.slices < 256 && NT % (2 * s.slices * s.TG) == 0) s.slices *= 2;
  }
  s.U = batch_of(nkt, 4 / s.TG > 0 ? 4 / s.TG : 1);
  s.TG = env_int("R9K_STREAM_TG", s.TG);
  s.U = env_int("R9K_STREAM_U", s.U);
  s.slices = env_int("R9K_STREAM_SLICES", s.slices);
  return s;
}

template <class Kern>
bool lds_ok(Kern* k) {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, LDS_MAX) ==
         hipSuccess;
}

template <int TG, int U, int EPI>
int launch(dim3 grid, hipStream_t st, long a, long as, long wq, long ws, long c, long cs, long sid, long eid,
           long ntpp, long tw, long wq_estride, long ws_estride, int numel, int a_row_div, int K, int N, int units,
           int ny) {
  const size_t smem = (size_t)BLK * (K + APAD) + (EPI == 1 ? (size_t)BLK * N * 2 : 0);
  static const bool ok = lds_ok(moe_stream_kernel<TG, U, EPI>);
  if (!ok || smem > (size_t)LDS_MAX) return 2;
  hipLaunchKernelGGL((moe_stream_kernel<TG, U, EPI>), grid, dim3(NW * WAVE), smem, st, (const uint8_t*)a,
                     (const float*)as, (const uint8_t*)wq, (const uint8_t*)ws, (void*)c, (float*)cs,
                     (const int*)sid, (const int*)eid, (const int*)ntpp, (const float*)tw, wq_estride, ws_estride,
                     numel, a_row_div, K, N, units, ny);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

}  // namespace

// No reference counterpart as one entry. epi 0: the r9k_moe_mxfp4a8 product over 16-row routing blocks (MT = 1;
// kernels/r9k_moe_mxfp4a8.hip:631-638 contract), c = bf16 [numel, N], topk_w optional, cs unused. epi 1: the gate_up
// product with SiLU-gating and the per-row fp8 quant in its epilogue (the reference's gate_up GEMM + r9k_silu_mul_quant_fp8,
// :631-638 and :550, in one launch), c = e4m3 codes [numel, N / 2], cs = fp32 row scales [numel], topk_w must be 0.
// Tables: moe_align_block_size format with 16-row blocks. Served: K % 128 == 0, K <= 4096, N % 16 == 0 with the
// column tiles dividing into the launch shape, the LDS (16 activation rows, and for epi 1 the bf16 gate_up tile of
// the block) within 96 KB, numel * N * 2 < 2^31; returns 2 (nothing launched) for other shapes so the caller takes
// the tile kernel, 0 on success, -3 bad argument, -6 launch error. blocks_hint: the caller's estimate of live blocks
// (min(E, numel)), which sets the column slices of epi 0.
extern "C" int r9k_moe_stream(int epi, long a, long as, long wq, long ws, long c, long cs, long sorted_ids,
                              long expert_ids, long ntpp, long topk_w, long ws_estride, int max_blocks, int numel,
                              int a_row_div, int K, int N, int blocks_hint, long stream) {
  if (max_blocks <= 0 || numel <= 0) return 0;
  if (epi != 0 && epi != 1) return -3;
  if (!a || !as || !wq || !ws || !c || !sorted_ids || !expert_ids || !ntpp || a_row_div < 1) return -3;
  if (epi == 1 && (!cs || topk_w)) return -3;
  if (K % KT || K <= 0 || K > ACH * NW * WAVE || N % 16 || N <= 0) return 2;
  if (epi == 1 && (N % 32 || N / 2 > HCH * NW * WAVE * 8 / BLK)) return 2;
  if ((a & 15) || (wq & 15) || (long)numel * N * 2 >= (1L << 31)) return 2;
  const Shape s = pick_shape(epi, N, K, blocks_hint > 0 ? blocks_hint : max_blocks);
  const int NT = N / 16, nkt = K / KT;
  if (s.TG < 1 || s.U < 1 || s.slices < 1 || nkt % s.U || NT % (s.slices * s.TG)) return 2;
  if (epi == 1 && (s.TG != 1 || s.slices != 1)) return 2;
  const int units = NT / (s.slices * s.TG);
  const long ny = max_blocks;
  const long cap_y = MAX_WG / (long)s.slices > 0 ? MAX_WG / (long)s.slices : 1;
  const dim3 grid(s.slices, (unsigned)(ny < cap_y ? ny : cap_y));
  const long wq_estride = (long)N * K / 2;
  const hipStream_t st = (hipStream_t)stream;
#define S(E, TGv, Uv)                                                                                              \
  if (epi == E && s.TG == TGv && s.U == Uv)                                                                       \
    return launch<TGv, Uv, E>(grid, st, a, as, wq, ws, c, cs, sorted_ids, expert_ids, ntpp, topk_w, wq_estride,   \
                              ws_estride, numel, a_row_div, K, N, units, (int)ny);
  S(0, 1, 1) S(0, 1, 2) S(0, 1, 4) S(0, 2, 1) S(0, 2, 2) S(0, 4, 1)
  S(1, 1, 1) S(1, 1, 2) S(1, 1, 4)
#undef S
  return 2;
}

// No reference counterpart as one entry: the reference's gate_up r9k_moe_mxfp4a8 + r9k_silu_mul_quant_fp8 + down
// r9k_moe_mxfp4a8 with topk_w (kernels/r9k_moe_mxfp4a8.hip:631-638, :550) in one launch over 16-row routing blocks,
// one block a workgroup: a = e4m3 x [T][K1] with as fp32 [T] (a_row_div = topk), w1 / w2 the gate_up (N1 = 2I, K1)
// and down (N2, K2 = I) weights in the r9k_moe_mxfp4a8 layout (w?s_estride bytes per expert of the scale tensors),
// c = bf16 [numel][N2] down rows (each equal to the three launches' value bit for bit when those run their
// single-wave split), then r9k_moe_sum. Served: K1 % 128 == 0, K1 <= 4096, I % 128 == 0, N2 % 32 == 0, the LDS within
// 96 KB, numel * N2 * 2 < 2^31; else 2 with nothing launched. 0, -3 bad argument, -6 launch error.
extern "C" int r9k_moe_stream_layer(long a, long as, long w1q, long w1s, long w2q, long w2s, long c, long sorted_ids,
                                    long expert_ids, long ntpp, long topk_w, long w1s_estride, long w2s_estride,
                                    int max_blocks, int numel, int a_row_div, int K1, int N1, int N2, long stream) {
  if (max_blocks <= 0 || numel <= 0) return 0;
  if (!a || !as || !w1q || !w1s || !w2q || !w2s || !c || !sorted_ids || !expert_ids || !ntpp || a_row_div < 1)
    return -3;
  const int I = N1 / 2;
  if (K1 % KT || K1 <= 0 || K1 > ACH * NW * WAVE || N1 % 32 || I % KT || N2 % 32 || N2 <= 0) return 2;
  if (I > HCH * NW * WAVE * 8 / BLK || (a & 15) || (w1q & 15) || (w2q & 15)) return 2;
  if ((long)numel * N2 * 2 >= (1L << 31)) return 2;
  const size_t smem = (size_t)BLK * (K1 + APAD) + (size_t)BLK * N1 * 2 + (size_t)BLK * (I + APAD);
  if (smem > (size_t)LDS_MAX) return 2;
  const int U1 = env_int("R9K_STREAM_U", batch_of(K1 / KT, 4));
  const int TG2 = env_int("R9K_STREAM_TG", 1), U2 = env_int("R9K_STREAM_U2", batch_of(I / KT, 2));
  if ((K1 / KT) % U1 || (I / KT) % U2 || (N2 / 16) % TG2) return 2;
  const long ny = max_blocks < MAX_WG ? max_blocks : MAX_WG;
  const hipStream_t st = (hipStream_t)stream;
#define L(U1v, TG2v, U2v)                                                                                          \
  if (U1 == U1v && TG2 == TG2v && U2 == U2v) {                                                                    \
    static const bool ok = lds_ok(moe_stream_layer_kernel<U1v, TG2v, U2v>);                                       \
    if (!ok) return 2;                                                                                            \
    hipLaunchKernelGGL((moe_stream_layer_kernel<U1v, TG2v, U2v>), dim3(1, (unsigned)ny), dim3(NW * WAVE), smem, st, \
                       (const uint8_t*)a, (const float*)as, (const uint8_t*)w1q, (const uint8_t*)w1s,            \
                       (const uint8_t*)w2q, (const uint8_t*)w2s, (uint16_t*)c, (const int*)sorted_ids,           \
                       (const int*)expert_ids, (const int*)ntpp, (const float*)topk_w, (long)N1 * K1 / 2,        \
                       w1s_estride, (long)N2 * I / 2, w2s_estride, numel, a_row_div, K1, N1, N2, (int)ny);       \
    return hipGetLastError() == hipSuccess ? 0 : -6;                                                               \
  }
  L(4, 1, 2) L(4, 1, 1) L(4, 2, 1) L(2, 1, 2) L(2, 1, 1) L(2, 2, 1) L(1, 1, 2) L(1, 1, 1) L(1, 2, 1)
#undef L
  return 2;
}
