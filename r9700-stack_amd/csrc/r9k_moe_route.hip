// r9k_moe_route.hip -- MoE routing and token-to-expert compaction on gfx950 (wave64).
//
// Routing (one wave per token row): fp32 softmax over the bf16 router logits, top-k, optional renormalisation of
// the selected weights (reference: kernels/r9k_moe_route.hip:22-25, 67-124).
//   * order: by the logit value, ties to the LOWER expert index. Softmax is monotone in the logit, so this is the
//     probability order of the reference (and of torch.softmax(...).topk), without the ties that fp32 exp rounding
//     can create between distinct logits; equal logits tie exactly as there.
//   * an entry whose probability is not a finite positive number counts as probability 0 ("dead": NaN logits, a
//     +inf row, entries more than 87 below the row max): dead entries rank after every live one, among
//     themselves by index, and get weight 0 -- the reference's rule for degenerate rows (:81-95).
//   * weights: p = exp(x - max) / sum_row exp(x - max); renorm: w_k = p_k / sum_j p_j over the selection.
// Keys pack (valid, live, order-preserving bf16 logit, ~index) into 32 bits, so one DPP wave max per selected
// slot is the whole argmax, ties included.
//
// Compaction (the moe_align_block_size tables, reference contract kernels/r9k_moe_route.hip:27-31 and
// r9700_vllm/kernels/moe.py:574-592): each expert's routed flat rows (token * topk + j) padded to a multiple of blk,
// experts ascending, padding value numel; expert_ids[b] = expert of block b or -1 past the end; ntpp[0] = padded
// total. Unlike the reference kernel (atomics: row order within an expert unspecified) the scatter here is STABLE:
// rows ascend within each expert, which is exactly align_block_size_ref's canonical order, so the tables are
// bit-exact against it. At decode widths (route_small_kernel) the stable order comes from a 64-bit token mask per
// expert; elsewhere the ids sit in LDS and, after an LDS histogram and a scan of the block-padded counts, rows are
// placed in rounds of one row per thread: a row's rank among equal ids of its wave comes from a branch-free compare
// against all 64 lanes (v_readlane), earlier waves' rows from per-wave counts in LDS. The whole capacity
// (sorted_ids [cap], expert_ids [cap / blk], cap = ceil((numel + E * (blk - 1)) / blk) * blk) is written, the tail
// with numel / -1. Barriers between phases wait for LDS traffic only; global stores are never waited for inside a
// kernel unless another workgroup reads them back.
//
// Entry points:
//   r9k_moe_route        the reference's one-launch routing + tables (M <= 64: route_small_kernel; numel <= 4096:
//                        one wave per row over ceil(M / 8) workgroups, the last to arrive builds the tables; larger
//                        numel as a top-k launch plus a single-workgroup table launch)
//   r9k_moe_route_quant  the same at decode widths with the experts' per-token fp8 input quant in the launch
//   r9k_moe_topk         routing only (the stock top-k router's role)
//   r9k_moe_align        tables only from given ids (vLLM's moe_align_block_size role); large numel runs as a
//                        per-chunk histogram launch plus a scatter launch (bases from the histograms), caller scratch.
#include "r9k_common.h"
#include "r9k_tables.h"

#include <mutex>

namespace {

using namespace r9k;

constexpr int MAX_E = TAB_MAX_E;  // experts
constexpr int MAX_K = 16;         // top-k
constexpr int AT = 1024;          // threads of an align / fused workgroup (16 waves)
constexpr int AW = AT / WAVE;
constexpr int SMALL_MAX = TAB_SMALL_MAX;   // routed rows whose tables one workgroup builds
constexpr int CH = 2048;          // routed rows per chunk in the multi-workgroup align
constexpr int RW = 8;             // waves (rows) per block of the top-k kernel
constexpr int FT = 512;           // threads of a fused routing workgroup (8 waves, one token row each)
constexpr int FW = FT / WAVE;

#define R9K_DPP(v, ctrl) (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(v), ctrl, 0xF, 0xF, false)

// Wave-uniform max of a 32-bit key (wave_max_u32).
__device__ __forceinline__ uint32_t wave_max_key(uint32_t v) { return wave_max_u32(v); }

// Wave-uniform fmaxf of a float, the same pattern (-inf for the lanes a broadcast does not write). The maximum does
// not depend on the order of the steps.
__device__ __forceinline__ float wave_max_dpp(float v) {
  constexpr int NEG_INF = (int)0xff800000u;
  v = fmaxf(v, __uint_as_float(R9K_DPP(__float_as_uint(v), 0xB1)));
  v = fmaxf(v, __uint_as_float(R9K_DPP(__float_as_uint(v), 0x4E)));
  v = fmaxf(v, __uint_as_float(R9K_DPP(__float_as_uint(v), 0x124)));
  v = fmaxf(v, __uint_as_float(R9K_DPP(__float_as_uint(v), 0x128)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(NEG_INF, __float_as_int(v), 0x142, 0xA, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(NEG_INF, __float_as_int(v), 0x143, 0xC, 0xF, false)));
  return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 63));
}
// Wave-uniform sum of a float in a fixed order (deterministic): the row sums through the same DPP steps, then the
// four rows' lane-0 values as (row0 + row1) + (row2 + row3).
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += __uint_as_float(R9K_DPP(__float_as_uint(v), 0xB1));
  v += __uint_as_float(R9K_DPP(__float_as_uint(v), 0x4E));
  v += __uint_as_float(R9K_DPP(__float_as_uint(v), 0x124));
  v += __uint_as_float(R9K_DPP(__float_as_uint(v), 0x128));
  const float a = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0));
  const float b = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 16));
  const float c = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 32));
  const float d = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 48));
  return (a + b) + (c + d);
}

// Selection key of an expert entry (0 = not selectable: taken, or past E):
//   bit 27 valid | bit 26 live | bits 10..25 the bf16 logit made order-preserving (-0 folded onto +0) | 1023 - e
// so the unsigned maximum is the live entry with the largest logit, ties to the lower index, then dead entries by
// index. E <= 1024.
__device__ __forceinline__ uint32_t route_key(uint16_t h, bool live, int e) {
  uint32_t b = h == 0x8000u ? 0u : h;
  const uint32_t ord = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
  return (1u << 27) | (live ? (1u << 26) | (ord << 10) : 0u) | (uint32_t)(1023 - e);
}

// Logits of one row for this lane: entry lane + 64 i, -inf past E.
template <int EPL>
__device__ __forceinline__ void load_row(const uint16_t* __restrict__ row, int E, int lane, uint16_t* h) {
#pragma unroll
  for (int i = 0; i < EPL; i++) {
    const int e = lane + WAVE * i;
    h[i] = e < E ? row[e] : (uint16_t)0xff80u;
  }
}

// The bf16 logit a live selection key holds (route_key's order-preserving bits inverted; -0 comes back as +0, which
// gives the same softmax numerator).
__device__ __forceinline__ uint16_t key_logit(uint32_t key) {
  const uint32_t ord = (key >> 10) & 0xffffu;
  return (uint16_t)((ord & 0x8000u) ? (ord & 0x7fffu) : (~ord & 0xffffu));
}

// One wave routes one row from its preloaded logits: softmax over the row (max, then exp(l - max) summed in the fixed
// order of wave_sum_dpp), then topk rounds of a wave-wide key maximum, each taking the largest live logit left (ties
// to the lower index) and clearing it. Lane k keeps round k's key; after the rounds it rebuilds the selection's
// numerator from the key's logit bits (the same expression as the first pass, so the same value), divides by the sum
// once, and the probabilities are added in round order for the renormalisation. Lane k < topk ends holding
// selection k; writes w / ids (global) and, when given, the ids to LDS.
template <int EPL>
__device__ __forceinline__ void topk_core(const uint16_t* h, int E, int topk, bool renorm, float* __restrict__ w_out,
                                          int* __restrict__ id_out, short* lds_ids, int lane, bool agent = false) {
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < EPL; i++) mx = fmaxf(mx, bf2f(h[i]));
  mx = wave_max_dpp(mx);
  uint32_t key[EPL];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; i++) {
    const int e = lane + WAVE * i;
    const float d = bf2f(h[i]) - mx;
    const bool live = d >= -87.f;                        // false for NaN (NaN logit, or a +inf row)
    s += (e < E && live) ? expf(d) : 0.f;
    key[i] = e < E ? route_key(h[i], live, e) : 0u;
  }
  s = wave_sum_dpp(s);
  uint32_t won = 0u;                                     // lane k: the key taken in round k
  for (int k = 0; k < topk; k++) {
    uint32_t b = key[0];
#pragma unroll
    for (int i = 1; i < EPL; i++) b = max(b, key[i]);
    b = wave_max_key(b);
    const int idx = 1023 - (int)(b & 1023u);
    const int owner = idx & (WAVE - 1), slot = idx / WAVE;
#pragma unroll
    for (int i = 0; i < EPL; i++)
      if (i == slot && lane == owner) key[i] = 0u;
    if (lane == k) won = b;
  }
  float p = 0.f;
  if (won & (1u << 26)) p = expf(bf2f(key_logit(won)) - mx);   // the first pass's numerator of this entry
  p = s > 0.f ? p / s : 0.f;
  if (renorm) {
    float tot = 0.f;
    for (int k = 0; k < topk; k++) tot += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(p), k));
    p = tot > 0.f ? p / tot : 0.f;
  }
  int isel = 1023 - (int)(won & 1023u);
  if (isel < 0 || isel >= E) isel = 0;               // unreachable (topk <= E); keeps every table write in range
  if (lane < topk) {
    w_out[lane] = p;
    if (agent) __hip_atomic_store(id_out + lane, isel, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // read by
    else id_out[lane] = isel;                                                                        // another CU
    if (lds_ids) lds_ids[lane] = (short)isel;
  }
}

// Optional outputs of the fused routing launch beyond the reference's: the per-token fp8 quant of the layer input
// (x bf16 rows of stride ldx, H values -> xq e4m3 [M, H], xs fp32 [M], quant_row_wave's bytes; x == nullptr: none)
// and a second table layout of the same ids in blocks of big_blk rows (sorted_big == nullptr: none), of which the
// device keeps one: the big layout when its nbig blocks hold numel >= min_rows * nbig rows (pick_blocks_kernel's
// rule), the other's ntpp then 0 and its entries left as they were. The big layout is written live-only (entries up
// to its ntpp), the small one over its whole capacity.
struct RouteExtras {
  const uint16_t* x;
  long ldx;
  int H;
  uint8_t* xq;
  float* xs;
  int big_blk;
  int min_rows;
  int* sorted_big;
  int* expert_big;
  int* ntpp_big;
};

// Fused routing + tables (reference: r9k_moe_route_kernel, kernels/r9k_moe_route.hip:67-210), numel <= SMALL_MAX:
// one wave per token row over ceil(M / 8) workgroups of 8 waves (the rows' latency chains spread over CUs). Each
// workgroup stores its ids as agent-scope atomics, waits for them (vmcnt) and counts itself in `arrive` (zero at
// entry, left zero); the last to arrive reads every id back with agent-scope loads, 8 in flight a thread, into LDS
// and builds the tables. With one workgroup the ids go straight to LDS. With R > 0 each wave then quantises its
// rows of x (after the arrival, so the table build does not wait for it; R chunks of 8 values a lane).
template <int EPL, int R>
__global__ void __launch_bounds__(FT) route_fused_kernel(const uint16_t* __restrict__ logits, int ldl,
                                                         float* __restrict__ weights, int* __restrict__ ids,
                                                         int* __restrict__ sorted_ids, int* __restrict__ expert_ids,
                                                         int* __restrict__ ntpp, int* __restrict__ arrive, int M,
                                                         int E, int topk, int renorm, int blk, RouteExtras ex) {
  __shared__ TabLds<FT> sh;
  __shared__ short lids[SMALL_MAX];
  __shared__ int s_last;
  __shared__ int s_nbig[FW];
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  const int numel = M * topk;
  const bool single = gridDim.x == 1;
  // the input quant of this workgroup's rows; `pre`: the first row's chunks are already in xpre
  uint4 xpre[R > 0 ? R : 1];
  auto quant_rows = [&](bool pre) {
    if constexpr (R > 0) {
      int r = blockIdx.x * FW + wave;
      if (pre && r < M) {
        quant_row_finish<R>(xpre, ex.H, ex.xq + (size_t)r * ex.H, ex.xs + r, lane);
        r += gridDim.x * FW;
      }
      for (; r < M; r += gridDim.x * FW)
        quant_row_wave<R>(ex.x + (size_t)r * ex.ldx, ex.H, ex.xq + (size_t)r * ex.H, ex.xs + r, lane);
    }
  };
  zero_counts(sh, E);
  for (int r = blockIdx.x * FW + wave; r < M; r += gridDim.x * FW) {
    uint16_t h[EPL];
    load_row<EPL>(logits + (size_t)r * ldl, E, lane, h);
    topk_core<EPL>(h, E, topk, renorm != 0, weights + (size_t)r * topk, ids + (size_t)r * topk,
                   single ? lids + r * topk : nullptr, lane, !single);
  }
  if (!single) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");           // this wave's id stores have completed
    lds_barrier();
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add(arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (int)gridDim.x - 1;
    lds_barrier();
    if (!s_last) {
      quant_rows(false);
      return;
    }
    if (threadIdx.x == 0) __hip_atomic_store(arrive, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (R > 0) {                                      // this workgroup's first rows: loads out before the build
      if (blockIdx.x * FW + wave < M) quant_row_load<R>(ex.x + (size_t)(blockIdx.x * FW + wave) * ex.ldx, ex.H, lane, xpre);
    }
    for (int t0 = 0; t0 < numel; t0 += 8 * FT) {                // other workgroups' ids, past this CU's caches
      int v[8];
#pragma unroll
      for (int u = 0; u < 8; u++)
        v[u] = __hip_atomic_load(ids + min(t0 + u * FT + (int)threadIdx.x, numel - 1), __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int t = t0 + u * FT + threadIdx.x;
        if (t < numel) lids[t] = (short)v[u];
      }
    }
  }
  lds_barrier();
  count_ids(sh, lids, numel);
  bool big = false;
  if (ex.sorted_big) {
    // the pick from the per-expert counts (the big layout's block count), then only the kept layout is built; the
    // other's ntpp is 0 (its GEMMs exit before reading its stale entries)
    int nb = 0;
    for (int e = threadIdx.x; e < E; e += FT) nb += (sh.cnt[e] + ex.big_blk - 1) / ex.big_blk;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) nb += __shfl_xor(nb, o, WAVE);
    if (lane == 0) s_nbig[wave] = nb;
    lds_barrier();
    int nbig = 0;
#pragma unroll
    for (int w = 0; w < FW; w++) nbig += s_nbig[w];
    big = nbig > 0 && (long)numel >= (long)ex.min_rows * nbig;
    if (threadIdx.x == 0) (big ? ntpp : ex.ntpp_big)[0] = 0;
  }
  if (big) build_from_counts(sh, lids, numel, E, ex.big_blk, ex.sorted_big, ex.expert_big, ex.ntpp_big, false);
  else build_from_counts(sh, lids, numel, E, blk, sorted_ids, expert_ids, ntpp);
  quant_rows(!single);
}

// ------------------------------------------------------------------ small batches: M <= 64 rows in one workgroup
constexpr int ST = 1024;          // threads of the small-batch routing workgroup (16 waves)
constexpr int SW = ST / WAVE;
constexpr int SMALL_ROWS = 64;    // token rows it routes: one bit each in the per-expert token masks
constexpr int SMALL_E = 512;      // experts (EPL <= 8)
constexpr int SMALL_CAP = 16384;  // table capacity kept in LDS
constexpr int QRMAX = 8;          // 16-byte chunks per lane of the fused activation quant: hidden <= 4096
constexpr int QPW = 4;            // activation rows per quant workgroup: one wave per SIMD (the quant is VALU-bound)

// Wave-inclusive prefix sum of an int: Hillis-Steele over 16-lane rows (DPP row_shr 1, 2, 4, 8; lanes shifted past
// the row start read 0), then the totals of the lower rows through v_readlane.
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
  v += (int)R9K_DPP(v, 0x111);
  v += (int)R9K_DPP(v, 0x112);
  v += (int)R9K_DPP(v, 0x114);
  v += (int)R9K_DPP(v, 0x118);
  const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31);
  const int r2 = __builtin_amdgcn_readlane(v, 47);
  const int row = lane >> 4;
  return v + (row > 0 ? r0 : 0) + (row > 1 ? r1 : 0) + (row > 2 ? r2 : 0);
}

// The table build of the small routing kernels, after every thread t < numel holds e = the expert of flat row t
// and the LDS layout is set up (mask zeroed, tab = numel, eids = -1): LDS mask[e] |= 1 << row, block-padded counts
// scanned over the experts (one per thread), rows placed at offs[e] + the number of earlier rows of e, then the
// tables written out. Every thread of the ST-thread workgroup calls it.
__device__ __forceinline__ void small_tables(int e, int numel, int topk, int E, int blk, int cap,
                                             unsigned long long* mask, int* offs, int* scan, int* tab, int* eids,
                                             int* __restrict__ sorted_ids, int* __restrict__ expert_ids,
                                             int* __restrict__ ntpp) {
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int nblk = cap / blk;
  const int trow = tid < numel ? tid / topk : 0;
  if (tid < numel) atomicOr(&mask[e], 1ull << trow);
  lds_barrier();

  // block-padded counts, scanned over the experts (one per thread)
  const int c = tid < E ? __popcll(mask[tid]) : 0;
  const int n = (c + blk - 1) & ~(blk - 1);
  const int incl = wave_incl_scan(n, lane);
  if (lane == WAVE - 1) scan[wave] = incl;
  lds_barrier();
  int wbase = 0, total = 0;
#pragma unroll
  for (int w = 0; w < SW; w++) {
    const int t = scan[w];
    wbase += w < wave ? t : 0;
    total += t;
  }
  if (tid < E) {
    const int o = wbase + incl - n;
    offs[tid] = o;
    for (int b = o / blk; b < (o + n) / blk; b++) eids[b] = tid;
  }
  if (tid == 0) ntpp[0] = total;
  lds_barrier();
  if (tid < numel) tab[offs[e] + __popcll(mask[e] & ((1ull << trow) - 1ull))] = tid;
  lds_barrier();

  // write-out: 16-byte stores where the destination allows, the rest one int at a time
  int done = 0;
  if ((reinterpret_cast<uintptr_t>(sorted_ids) & 15) == 0) {
    const int n4 = cap / 4;
    for (int i = tid; i < n4; i += ST) reinterpret_cast<int4*>(sorted_ids)[i] = reinterpret_cast<const int4*>(tab)[i];
    done = n4 * 4;
  }
  for (int i = done + tid; i < cap; i += ST) sorted_ids[i] = tab[i];
  for (int b = tid; b < nblk; b += ST) expert_ids[b] = eids[b];
}

// Top-k of NR rows per wave, interleaved so that their reduction chains overlap (same order and numerics as
// topk_core). The selection loop only finds keys; lane k then rebuilds its entry's exp from the key (the key holds
// the bf16 logit) and forms p_k = e_k / sum, and the selected sum is accumulated in k order as before. Returns,
// on lane k < topk, the expert id and the (renormalised) weight of selection k of each row.
template <int EPL, int NR>
__device__ __forceinline__ void topk_rows(const uint16_t (&h)[NR][EPL], int E, int topk, bool renorm, int lane,
                                          int (&id)[NR], float (&w)[NR]) {
  float mx[NR], s[NR];
  uint32_t key[NR][EPL];
#pragma unroll
  for (int r = 0; r < NR; r++) {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < EPL; i++) m = fmaxf(m, bf2f(h[r][i]));
    mx[r] = wave_max_dpp(m);
  }
#pragma unroll
  for (int r = 0; r < NR; r++) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; i++) {
      const int e = lane + WAVE * i;
      const float d = bf2f(h[r][i]) - mx[r];
      const bool live = d >= -87.f;
      acc += (e < E && live) ? expf(d) : 0.f;
      key[r][i] = e < E ? route_key(h[r][i], live, e) : 0u;
    }
    s[r] = wave_sum_dpp(acc);
  }
  uint32_t sel[NR];
#pragma unroll
  for (int r = 0; r < NR; r++) sel[r] = 0u;
  for (int k = 0; k < topk; k++) {
#pragma unroll
    for (int r = 0; r < NR; r++) {
      uint32_t b = key[r][0];
#pragma unroll
      for (int i = 1; i < EPL; i++) b = max(b, key[r][i]);
      b = wave_max_key(b);                          // nonzero: an unselected e < E is left while k < topk <= E
#pragma unroll
      for (int i = 0; i < EPL; i++) key[r][i] = key[r][i] == b ? 0u : key[r][i];   // keys are unique
      sel[r] = lane == k ? b : sel[r];
    }
  }
#pragma unroll
  for (int r = 0; r < NR; r++) {
    const uint32_t b = sel[r];
    const float eb = ((b >> 26) & 1u) ? expf(bf2f(key_logit(b)) - mx[r]) : 0.f;
    float p = s[r] > 0.f ? eb / s[r] : 0.f;
    float tot = 0.f;
    for (int k = 0; k < topk; k++) tot += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(p), k));
    if (renorm) p = tot > 0.f ? p / tot : 0.f;
    const int idx = 1023 - (int)(b & 1023u);
    id[r] = (idx < 0 || idx >= E) ? 0 : idx;        // lanes >= topk only
    w[r] = p;
  }
}

// Routing + tables + (optionally) the per-token fp8 quant of the activations for M <= 64 rows, one launch.
// Routing workgroups g < nrt = ceil(M / rpw) take rows g * rpw + wave (wave < rpw, one row a wave; waves without a
// row skip the top-k, which is VALU-bound at 4 cycles an instruction). With one routing workgroup (rpw = 8,
// M <= 8) the ids stay on chip; with several (rpw = 4: one row per SIMD) each stores its ids as agent-scope
// atomics, waits for them to complete (vmcnt) and then counts itself in `arrive`; the last to arrive reads every id
// back with agent-scope atomic loads and builds the tables, resetting `arrive` to zero. (Agent-scope atomic
// accesses are coherent across the XCDs' L2s on their own, so no whole-L2 writeback / invalidate fence is needed.)
// Table build, one thread per flat row t = row * topk + k with expert e: LDS mask[e] |= 1 << row (an expert's
// routed rows are its set bits: count = popcount; t goes to offs[e] + popcount(mask[e] & bits below row), which is
// the stable ascending order). The tables are assembled in LDS (padding = numel, expert_ids = -1 past the end) and
// written out with 16-byte stores. Workgroups nrt.. quantise 4 activation rows each (quant_row_wave, one wave per
// SIMD). Dynamic LDS: mask u64 [Ep], offs [Ep], scan [64], tab [cap], eids [cap / blk], lids [numel] (Ep = E
// rounded up to 16).
template <int EPL>
__global__ void __launch_bounds__(ST) route_small_kernel(
    const uint16_t* __restrict__ logits, int ldl, float* __restrict__ weights, int* __restrict__ ids,
    int* __restrict__ sorted_ids, int* __restrict__ expert_ids, int* __restrict__ ntpp, int* __restrict__ arrive,
    int M, int E, int topk, int renorm, int blk, int cap, int rpw, const uint16_t* __restrict__ x, long ldx, int H,
    uint8_t* __restrict__ xq, float* __restrict__ xs) {
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int nrt = (M + rpw - 1) / rpw;
  if ((int)blockIdx.x >= nrt) {
    const int row = ((int)blockIdx.x - nrt) * QPW + wave;
    if (wave < QPW && row < M) quant_row_wave<QRMAX>(x + (size_t)row * ldx, H, xq + (size_t)row * H, xs + row, lane);
    return;
  }
  extern __shared__ __align__(16) uint8_t smem[];
  const int Ep = (E + 15) & ~15;
  unsigned long long* mask = reinterpret_cast<unsigned long long*>(smem);
  int* offs = reinterpret_cast<int*>(mask + Ep);
  int* scan = offs + Ep;                                       // [0, SW): per-wave totals; [SW]: last-arrival flag
  int* tab = scan + 64;
  int* eids = tab + cap;
  int* lids = eids + cap / blk;
  const int numel = M * topk, nblk = cap / blk;
  const int row = (int)blockIdx.x * rpw + wave;
  const bool has_row = wave < rpw && row < M;

  uint16_t h[1][EPL];
  if (has_row) load_row<EPL>(logits + (size_t)row * ldl, E, lane, h[0]);
  // LDS set-up under the logit loads
  for (int e = tid; e < E; e += ST) mask[e] = 0ull;
  for (int i = tid; i < cap; i += ST) tab[i] = numel;
  for (int b = tid; b < nblk; b += ST) eids[b] = -1;

  if (has_row) {
    int id[1];
    float wt[1];
    topk_rows<EPL, 1>(h, E, topk, renorm != 0, lane, id, wt);
    if (lane < topk) {
      weights[(size_t)row * topk + lane] = wt[0];
      if (nrt == 1) {
        ids[(size_t)row * topk + lane] = id[0];
        lids[row * topk + lane] = id[0];
      } else {
        __hip_atomic_store(ids + (size_t)row * topk + lane, id[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  int e = 0;
  if (nrt > 1) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");           // this wave's id stores have completed
    lds_barrier();
    if (tid == 0) scan[SW] = __hip_atomic_fetch_add(arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nrt - 1;
    lds_barrier();
    if (!scan[SW]) return;
    if (tid == 0) __hip_atomic_store(arrive, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid < numel) e = __hip_atomic_load(ids + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    lds_barrier();
    if (tid < numel) e = lids[tid];
  }
  small_tables(e, numel, topk, E, blk, cap, mask, offs, scan, tab, eids, sorted_ids, expert_ids, ntpp);
}

// Device-side choice between the two table layouts of one routed step, built side by side: 16 * MT-row decode
// blocks (ntpp_small) and big_blk-row prefill blocks (ntpp_big). The big layout's block count estimates the touched
// experts (one block each up to big_blk rows); min_rows or more routed rows per such block keeps the big layout,
// else the small one. The layout not kept gets ntpp = 0, so every GEMM launched over it exits at once.
__global__ void __launch_bounds__(64) pick_blocks_kernel(int* __restrict__ ntpp_small, int* __restrict__ ntpp_big,
                                                         int numel, int big_blk, int min_rows) {
  if (threadIdx.x) return;
  const int nbig = ntpp_big[0] / big_blk;
  const bool big = nbig > 0 && (long)numel >= (long)min_rows * nbig;
  if (big) ntpp_small[0] = 0;
  else ntpp_big[0] = 0;
}

template <int EPL>
__global__ void __launch_bounds__(RW * WAVE) topk_kernel(const uint16_t* __restrict__ logits, int ldl,
                                                         float* __restrict__ weights, int* __restrict__ ids, int M,
                                                         int E, int topk, int renorm) {
  const int r = blockIdx.x * RW + threadIdx.x / WAVE;
  if (r >= M) return;
  uint16_t h[EPL];
  load_row<EPL>(logits + (size_t)r * ldl, E, threadIdx.x % WAVE, h);
  topk_core<EPL>(h, E, topk, renorm != 0, weights + (size_t)r * topk, ids + (size_t)r * topk, nullptr,
                 threadIdx.x % WAVE);
}

// Top-k routing plus the per-token fp8 quant of the layer's activations in one launch (any M): even blocks route RW
// rows each (one row a wave, VALU-bound), odd blocks quantise RW rows of x each (quant_row_wave, HBM-bound), so every
// CU runs both kinds at once instead of one launch after the other. Outputs are topk_kernel's and
// r9k_quant_rows_fp8's.
template <int EPL, int R>
__global__ void __launch_bounds__(RW * WAVE) topk_quant_kernel(const uint16_t* __restrict__ logits, int ldl,
                                                               float* __restrict__ weights, int* __restrict__ ids,
                                                               int M, int E, int topk, int renorm,
                                                               const uint16_t* __restrict__ x, long ldx, int H,
                                                               uint8_t* __restrict__ xq, float* __restrict__ xs) {
  const int lane = threadIdx.x % WAVE;
  const int r = (int)(blockIdx.x >> 1) * RW + (int)threadIdx.x / WAVE;
  if (r >= M) return;
  if ((blockIdx.x & 1) == 0) {
    uint16_t h[EPL];
    load_row<EPL>(logits + (size_t)r * ldl, E, lane, h);
    topk_core<EPL>(h, E, topk, renorm != 0, weights + (size_t)r * topk, ids + (size_t)r * topk, nullptr, lane);
  } else {
    quant_row_wave<R>(x + (size_t)r * ldx, H, xq + (size_t)r * H, xs + r, lane);
  }
}

// Reductions over the 16 lanes of a DPP row, the result in every lane of the row. The sum pairs lanes by xor
// butterflies (quad swaps, then half-row and row mirrors): each step adds two partial sums in either order, so all
// 16 lanes hold the same bits.
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
  v = max(v, R9K_DPP(v, 0xB1));
  v = max(v, R9K_DPP(v, 0x4E));
  v = max(v, R9K_DPP(v, 0x124));   // row_ror:4
  v = max(v, R9K_DPP(v, 0x128));   // row_ror:8
  return v;
}
__device__ __forceinline__ float row16_max_f(float v) {
  v = fmaxf(v, __uint_as_float(R9K_DPP(__float_as_uint(v), 0xB1)));
  v = fmaxf(v, __uint_as_float(R9K_DPP(__float_as_uint(v), 0x4E)));
  v = fmaxf(v, __uint_as_float(R9K_DPP(__float_as_uint(v), 0x124)));
  v = fmaxf(v, __uint_as_float(R9K_DPP(__float_as_uint(v), 0x128)));
  return v;
}
__device__ __forceinline__ float row16_sum_f(float v) {
  v += __uint_as_float(R9K_DPP(__float_as_uint(v), 0xB1));    // quad_perm [1,0,3,2]
  v += __uint_as_float(R9K_DPP(__float_as_uint(v), 0x4E));    // quad_perm [2,3,0,1]
  v += __uint_as_float(R9K_DPP(__float_as_uint(v), 0x141));   // row_half_mirror
  v += __uint_as_float(R9K_DPP(__float_as_uint(v), 0x140));   // row_mirror
  return v;
}

// Top-k of one row on the 16 lanes of a DPP row (four rows a wave), for the wide launches: NP dwords of logits a
// lane (entries 2d and 2d + 1 of dword d = l16 + 16 i; E even), the same keys, selection rounds and numerator rebuild
// as topk_core with row-wide reductions and no cross-row readlanes, about half of topk_core's VALU work a row. The
// softmax sum is taken in this layout's order (lane sums, then the butterflies above). Lane l16 < topk of the row
// stores selection l16 when `store`.
template <int NP>
__device__ __forceinline__ void topk_row16(const uint16_t* __restrict__ row, int E, int topk, bool renorm,
                                           float* __restrict__ w_out, int* __restrict__ id_out, bool store,
                                           int lane) {
  const int l16 = lane & 15;
  const uint32_t* rp = reinterpret_cast<const uint32_t*>(row);
  uint32_t hv[NP];
#pragma unroll
  for (int i = 0; i < NP; i++) {
    const int d = l16 + 16 * i;
    hv[i] = 2 * d < E ? rp[d] : 0xff80ff80u;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < NP; i++) mx = fmaxf(mx, fmaxf(lo16(hv[i]), hi16(hv[i])));
  mx = row16_max_f(mx);
  uint32_t key[2 * NP];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NP; i++) {
#pragma unroll
    for (int t = 0; t < 2; t++) {
      const int e = 2 * (l16 + 16 * i) + t;
      const uint16_t h = (uint16_t)(t ? hv[i] >> 16 : hv[i] & 0xffffu);
      const float d = bf2f(h) - mx;
      const bool live = d >= -87.f;
      s += (e < E && live) ? expf(d) : 0.f;
      key[2 * i + t] = e < E ? route_key(h, live, e) : 0u;
    }
  }
  s = row16_sum_f(s);
  uint32_t won = 0u;
  for (int k = 0; k < topk; k++) {
    uint32_t b = key[0];
#pragma unroll
    for (int j = 1; j < 2 * NP; j++) b = max(b, key[j]);
    b = row16_max_u32(b);
#pragma unroll
    for (int j = 0; j < 2 * NP; j++) key[j] = key[j] == b ? 0u : key[j];   // keys are unique within a row
    if (l16 == k) won = b;
  }
  float p = 0.f;
  if (won & (1u << 26)) p = expf(bf2f(key_logit(won)) - mx);
  p = s > 0.f ? p / s : 0.f;
  if (renorm) {
    float tot = 0.f;
    for (int k = 0; k < topk; k++) tot += __shfl(p, (lane & ~15) + k, WAVE);
    p = tot > 0.f ? p / tot : 0.f;
  }
  int isel = 1023 - (int)(won & 1023u);
  if (isel < 0 || isel >= E) isel = 0;
  if (store && l16 < topk) {
    w_out[l16] = p;
    id_out[l16] = isel;
  }
}

constexpr int R16 = 4 * RW;        // rows a workgroup of the 16-lane top-k routes

// The 16-lane top-k over the rows: R16 rows a workgroup, rows past M clamp their loads and store nothing.
template <int NP>
__global__ void __launch_bounds__(RW * WAVE) topk16_kernel(const uint16_t* __restrict__ logits, int ldl,
                                                           float* __restrict__ weights, int* __restrict__ ids, int M,
                                                           int E, int topk, int renorm) {
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const int r0 = (int)blockIdx.x * R16 + wave * 4;
  if (r0 >= M) return;
  const int r = r0 + (lane >> 4), rc = r < M ? r : M - 1;
  topk_row16<NP>(logits + (size_t)rc * ldl, E, topk, renorm != 0, weights + (size_t)rc * topk,
                 ids + (size_t)rc * topk, r < M, lane);
}

// topk16_kernel and the per-token fp8 quant in one launch: the first ceil(M / R16) workgroups route R16 rows each
// (four rows a wave), the rest quantise eight rows each (one a wave, quant_row_wave). The long VALU-bound routing
// workgroups are dispatched first, one or so a CU, and the HBM-bound quant workgroups fill the CUs around them.
template <int NP, int R>
__global__ void __launch_bounds__(RW * WAVE) topk16_quant_kernel(const uint16_t* __restrict__ logits, int ldl,
                                                                 float* __restrict__ weights, int* __restrict__ ids,
                                                                 int M, int E, int topk, int renorm,
                                                                 const uint16_t* __restrict__ x, long ldx, int H,
                                                                 uint8_t* __restrict__ xq, float* __restrict__ xs) {
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const int nroute = (M + R16 - 1) / R16;
  if ((int)blockIdx.x < nroute) {
    const int r0 = (int)blockIdx.x * R16 + wave * 4;
    if (r0 >= M) return;
    const int r = r0 + (lane >> 4), rc = r < M ? r : M - 1;
    topk_row16<NP>(logits + (size_t)rc * ldl, E, topk, renorm != 0, weights + (size_t)rc * topk,
                   ids + (size_t)rc * topk, r < M, lane);
  } else {
    const int r = ((int)blockIdx.x - nroute) * RW + wave;
    if (r >= M) return;
    quant_row_wave<R>(x + (size_t)r * ldx, H, xq + (size_t)r * H, xs + r, lane);
  }
}

// Tables from ids in global memory, one workgroup, numel <= SMALL_MAX.
__global__ void __launch_bounds__(AT) align_single_kernel(const int* __restrict__ ids, int numel, int E, int blk,
                                                          int* __restrict__ sorted_ids, int* __restrict__ expert_ids,
                                                          int* __restrict__ ntpp, int tail) {
  __shared__ TabLds<AT> sh;
  __shared__ short lids[SMALL_MAX];
  zero_counts(sh, E);
  for (int t = threadIdx.x; t < numel; t += AT) {
    const int e = ids[t];
    lids[t] = (short)(e >= 0 && e < E ? e : -1);
  }
  lds_barrier();
  build_tables(sh, lids, numel, E, blk, sorted_ids, expert_ids, ntpp, tail != 0);
}

// The split tables of launch_align_split in one workgroup (numel <= SMALL_MAX): one count of every id, then the big
// experts' table (their rows only) and the small experts' table (the ids read again, the other rows left out).
__global__ void __launch_bounds__(AT) align_split_single_kernel(
    const int* __restrict__ ids, int numel, int E, int thr, int blk_big, int* __restrict__ sorted_big,
    int* __restrict__ expert_big, int* __restrict__ ntpp_big, int blk_small, int* __restrict__ sorted_small,
    int* __restrict__ expert_small, int* __restrict__ ntpp_small) {
  __shared__ TabLds<AT> sh;
  __shared__ short lids[SMALL_MAX];
  __shared__ int full[TAB_MAX_E];
  zero_counts(sh, E);
  for (int t = threadIdx.x; t < numel; t += AT) {
    const int e = ids[t];
    lids[t] = (short)(e >= 0 && e < E ? e : -1);
  }
  lds_barrier();
  count_ids(sh, lids, numel);
  for (int e = threadIdx.x; e < E; e += AT) {
    const int c = sh.cnt[e];
    full[e] = c;
    sh.cnt[e] = c > thr ? c : 0;
  }
  lds_barrier();
  for (int t = threadIdx.x; t < numel; t += AT) {
    const int e = lids[t];
    if (e >= 0 && sh.cnt[e] == 0) lids[t] = -1;
  }
  build_from_counts(sh, lids, numel, E, blk_big, sorted_big, expert_big, ntpp_big, false);
  for (int e = threadIdx.x; e < E; e += AT) sh.cnt[e] = full[e] <= thr ? full[e] : 0;
  lds_barrier();
  for (int t = threadIdx.x; t < numel; t += AT) {
    const int e = ids[t];
    lids[t] = (short)(e >= 0 && e < E && sh.cnt[e] > 0 ? e : -1);
  }
  build_from_counts(sh, lids, numel, E, blk_small, sorted_small, expert_small, ntpp_small, false);
}

// Tables from ids in global memory for any numel in one workgroup without scratch (the reference route entry's
// large-M path): count every id, scan, layout, then place chunk by chunk with each expert's cursor in a register.
__global__ void __launch_bounds__(AT) align_big_single_kernel(const int* __restrict__ ids, int numel, int E, int blk,
                                                              int* __restrict__ sorted_ids,
                                                              int* __restrict__ expert_ids, int* __restrict__ ntpp) {
  __shared__ TabLds<AT> sh;
  __shared__ short lids[SMALL_MAX];
  const int tid = threadIdx.x;
  zero_counts(sh, E);
  lds_barrier();
  for (int t0 = 0; t0 < numel; t0 += 4 * AT) {
    int v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) v[u] = t0 + tid + u * AT < numel ? ids[t0 + tid + u * AT] : -1;
#pragma unroll
    for (int u = 0; u < 4; u++)
      if (v[u] >= 0 && v[u] < E) atomicAdd(&sh.cnt[v[u]], 1);
  }
  lds_barrier();
  const int total = padded_scan(sh, E, blk);
  if (tid == 0) ntpp[0] = total;
  write_layout(sh, E, blk, numel, total, 0, 0, 1, sorted_ids, expert_ids);
  for (int c0 = 0; c0 < numel; c0 += SMALL_MAX) {
    const int n = min(SMALL_MAX, numel - c0);
    for (int t = tid; t < n; t += AT) {
      const int e = ids[c0 + t];
      lids[t] = (short)(e >= 0 && e < E ? e : -1);
    }
    lds_barrier();
    for (int base = 0; base < n; base += AT) stable_round(sh, lids, base, n, c0, E, sorted_ids);
  }
}

// Scratch of the multi-block align (int32): from ALIGN_HIST on, nch rows of E: each chunk's per-expert histogram
// (the first ALIGN_HIST ints are not used and stay as the caller left them, zero).
constexpr int ALIGN_HIST = 16;

// Multi-block align, pass 1 (one workgroup per chunk of CH routed rows): the chunk's per-expert histogram, stored as
// row c of the scratch. The next launch reads every row (a launch boundary orders them).
__global__ void __launch_bounds__(AT) align_count_kernel(const int* __restrict__ ids, int numel, int E,
                                                         int* __restrict__ scratch) {
  __shared__ TabLds<AT> sh;
  int* __restrict__ hist = scratch + ALIGN_HIST;
  const int tid = threadIdx.x, c = blockIdx.x;
  for (int e = tid; e < E; e += AT) sh.cnt[e] = 0;
  const int t0 = c * CH, t1 = min(numel, t0 + CH);
  int v[CH / AT];
#pragma unroll
  for (int u = 0; u < CH / AT; u++) v[u] = t0 + tid + u * AT < t1 ? ids[t0 + tid + u * AT] : -1;
  lds_barrier();
#pragma unroll
  for (int u = 0; u < CH / AT; u++)
    if (v[u] >= 0 && v[u] < E) atomicAdd(&sh.cnt[v[u]], 1);
  lds_barrier();
  for (int e = tid; e < E; e += AT) hist[(size_t)c * E + e] = sh.cnt[e];
}

// Multi-block align, pass 2 (one workgroup per chunk): every chunk's histogram (16 loads in flight a thread, one
// expert a thread) gives this chunk's base within each expert (the rows of earlier chunks), each expert's count, and
// by the padded scan each expert's first slot and the padded total (workgroup 0 writes ntpp). Then this chunk's share
// of the layout writes (expert blocks of experts e = c, c + nch, ...; the capacity tail split by chunk) and the
// stable placement of its rows.
// cls selects the experts this table holds by their total row count: 0 every expert, 1 those with more than thr rows,
// 2 those with 1..thr rows (the rows of the others are left out, as ids outside [0, E)).
__global__ void __launch_bounds__(AT) align_scatter_kernel(const int* __restrict__ ids, int numel, int E, int blk,
                                                           int* __restrict__ sorted_ids, int* __restrict__ expert_ids,
                                                           int* __restrict__ ntpp, const int* __restrict__ scratch,
                                                           int tail, int cls, int thr) {
  __shared__ TabLds<AT> sh;
  __shared__ short lids[CH];
  const int* __restrict__ hist = scratch + ALIGN_HIST;
  const int tid = threadIdx.x, c = blockIdx.x, nch = gridDim.x;
  const int t0 = c * CH, t1 = min(numel, t0 + CH), n = t1 - t0;
  zero_counts(sh, E);
  for (int t = tid; t < n; t += AT) {
    const int e = ids[t0 + t];
    lids[t] = (short)(e >= 0 && e < E ? e : -1);
  }
  int pre = 0, tot = 0;
  if (tid < E) {                                               // E <= AT: one expert a thread
    for (int c0 = 0; c0 < nch; c0 += 16) {
      int h[16];
#pragma unroll
      for (int u = 0; u < 16; u++) h[u] = hist[(size_t)min(c0 + u, nch - 1) * E + tid];
#pragma unroll
      for (int u = 0; u < 16; u++)
        if (c0 + u < nch) {
          pre += c0 + u < c ? h[u] : 0;
          tot += h[u];
        }
    }
  }
  lds_barrier();                                               // zero_counts is done before the counts go in
  if (tid < E) {
    const bool keep = cls == 0 || (cls == 1 ? tot > thr : tot <= thr);
    sh.cnt[tid] = keep ? tot : 0;
    pre = keep ? pre : 0;
  }
  lds_barrier();
  if (cls != 0)                                                // rows of experts of the other class are not placed
    for (int t = tid; t < n; t += AT) {
      const int e = lids[t];
      if (e >= 0 && sh.cnt[e] == 0) lids[t] = -1;
    }
  const int total = padded_scan(sh, E, blk);                   // (write_layout's closing barrier orders lids)
  if (c == 0 && tid == 0) ntpp[0] = total;
  write_layout(sh, E, blk, numel, total, pre, c, nch, sorted_ids, expert_ids, tail != 0);
  for (int base = 0; base < n; base += AT) stable_round(sh, lids, base, n, t0, E, sorted_ids);
}

int epl_for(int E) {
  const int need = (E + WAVE - 1) / WAVE;
  for (int v : {2, 4, 6, 8, 12, 16})
    if (need <= v) return v;
  return -1;
}

// Dwords of logits a lane of the 16-lane top-k holds for E experts (E even, at most 512; 0 = not served: the
// one-row-a-wave kernels run instead).
int np16_for(const void* logits, int ldl, int E) {
  if (E % 2 || E > 512 || (reinterpret_cast<uintptr_t>(logits) & 3) || (ldl & 1)) return 0;
  const int need = (E + 31) / 32;
  for (int v : {2, 4, 8, 9, 12, 16})
    if (need <= v) return v;
  return 0;
}

int launch_topk(const uint16_t* logits, int ldl, float* w, int* ids, int M, int E, int topk, int renorm,
                hipStream_t st) {
  if (const int np = np16_for(logits, ldl, E)) {
    const dim3 grid16((M + R16 - 1) / R16), block16(RW * WAVE);
#define TK16(NPV) hipLaunchKernelGGL(topk16_kernel<NPV>, grid16, block16, 0, st, logits, ldl, w, ids, M, E, topk, renorm)
    switch (np) {
      case 2: TK16(2); break;
      case 4: TK16(4); break;
      case 8: TK16(8); break;
      case 9: TK16(9); break;
      case 12: TK16(12); break;
      default: TK16(16); break;
    }
#undef TK16
    return 0;
  }
  const dim3 grid((M + RW - 1) / RW), block(RW * WAVE);
#define TK(EPLV) hipLaunchKernelGGL(topk_kernel<EPLV>, grid, block, 0, st, logits, ldl, w, ids, M, E, topk, renorm)
  switch (epl_for(E)) {
    case 2: TK(2); break;
    case 4: TK(4); break;
    case 6: TK(6); break;
    case 8: TK(8); break;
    case 12: TK(12); break;
    case 16: TK(16); break;
    default: return 1;
  }
#undef TK
  return 0;
}

// Tables for numel routed rows from ids in global memory (any numel): one workgroup up to SMALL_MAX, else the
// histogram + placement launches over CH-row chunks (scratch: align_scratch_ints(numel, E) int32 for the chunk
// histograms, which the count launch overwrites).
long align_scratch_ints(int numel, int E) {
  return numel <= SMALL_MAX ? 1 : ALIGN_HIST + (long)((numel + CH - 1) / CH) * E;
}

int launch_align(const int* ids, int numel, int E, int blk, int* sorted_ids, int* expert_ids, int* ntpp,
                 int* scratch, hipStream_t st, int tail = 1) {
  if (numel <= SMALL_MAX) {
    hipLaunchKernelGGL(align_single_kernel, dim3(1), dim3(AT), 0, st, ids, numel, E, blk, sorted_ids, expert_ids,
                       ntpp, tail);
    return 0;
  }
  if (!scratch) return 1;
  const int nch = (numel + CH - 1) / CH;
  hipLaunchKernelGGL(align_count_kernel, dim3(nch), dim3(AT), 0, st, ids, numel, E, scratch);
  hipLaunchKernelGGL(align_scatter_kernel, dim3(nch), dim3(AT), 0, st, ids, numel, E, blk, sorted_ids, expert_ids,
                     ntpp, (const int*)scratch, tail, 0, 0);
  return 0;
}

// Two live-only tables of one routed step split by expert size: experts with more than thr rows in blk_big-row
// blocks, the others in blk_small-row blocks. One workgroup (two builds from one count) up to SMALL_MAX rows, else
// the count launch and one scatter launch per table.
int launch_align_split(const int* ids, int numel, int E, int thr, int blk_big, int* sorted_big, int* expert_big,
                       int* ntpp_big, int blk_small, int* sorted_small, int* expert_small, int* ntpp_small,
                       int* scratch, hipStream_t st) {
  if (numel <= SMALL_MAX) {
    hipLaunchKernelGGL(align_split_single_kernel, dim3(1), dim3(AT), 0, st, ids, numel, E, thr, blk_big, sorted_big,
                       expert_big, ntpp_big, blk_small, sorted_small, expert_small, ntpp_small);
    return 0;
  }
  if (!scratch) return 1;
  const int nch = (numel + CH - 1) / CH;
  hipLaunchKernelGGL(align_count_kernel, dim3(nch), dim3(AT), 0, st, ids, numel, E, scratch);
  hipLaunchKernelGGL(align_scatter_kernel, dim3(nch), dim3(AT), 0, st, ids, numel, E, blk_big, sorted_big,
                     expert_big, ntpp_big, (const int*)scratch, 0, 1, thr);
  hipLaunchKernelGGL(align_scatter_kernel, dim3(nch), dim3(AT), 0, st, ids, numel, E, blk_small, sorted_small,
                     expert_small, ntpp_small, (const int*)scratch, 0, 2, thr);
  return 0;
}

bool route_args_ok(int M, int E, int topk, int blk) {
  return M >= 1 && E >= 1 && E <= MAX_E && topk >= 1 && topk <= MAX_K && topk <= E && blk >= 1 &&
         (blk & (blk - 1)) == 0;
}

long table_capacity(long numel, int E, int blk) { return (numel + (long)E * (blk - 1) + blk - 1) / blk * blk; }

template <int EPL>
hipError_t launch_small_inst(dim3 grid, size_t lds, hipStream_t st, const uint16_t* logits, int ldl, float* w,
                             int* ids, int* sorted_ids, int* expert_ids, int* ntpp, int* arrive, int M, int E,
                             int topk, int renorm, int blk, int cap, int rpw, const uint16_t* x, long ldx, int H,
                             uint8_t* xq, float* xs) {
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(route_small_kernel<EPL>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(route_small_kernel<EPL>, grid, dim3(ST), lds, st, logits, ldl, w, ids, sorted_ids, expert_ids,
                     ntpp, arrive, M, E, topk, renorm, blk, cap, rpw, x, ldx, H, xq, xs);
  return hipGetLastError();
}

// Routing rows per workgroup of route_small_kernel: all M in one workgroup up to this many rows (no cross-workgroup
// hand-off), else SMALL_RPW rows each (one row per SIMD) and the last workgroup to arrive builds the tables. Up to 8
// rows the one workgroup holds at most two rows a SIMD; at 9-16 rows (three or four a SIMD, the top-k VALU-bound)
// the hand-off is faster: config 2 T = 16 41.0 against 41.9 us a layer on MI355X, T <= 12 unchanged.
constexpr int SMALL_ONE_WG = 8;
constexpr int SMALL_RPW = 4;
int small_rpw(int M) { return M <= SMALL_ONE_WG ? SMALL_ONE_WG : SMALL_RPW; }

// Whether route_small_kernel takes this call (and, with x, the activation quant): M <= 64 rows, E <= 512, a table
// that fits LDS, an arrival counter when several workgroups route, and x rows the wave quant reads as 16-byte chunks.
bool small_fits(int M, int E, int topk, int blk, const void* arrive, const void* x, long ldx, int H, const void* xq,
                const void* xs) {
  if (M > SMALL_ROWS || E > SMALL_E || table_capacity((long)M * topk, E, blk) > SMALL_CAP) return false;
  if (M > SMALL_ONE_WG && !arrive) return false;
  if (!x) return true;
  return xq && xs && H >= 8 && H % 8 == 0 && H <= 512 * QRMAX && ldx >= H && ldx % 8 == 0 &&
         (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(xq) & 7) == 0;
}

// One launch: the routing workgroups, then (with x) ceil(M / 4) quant workgroups.
hipError_t launch_small(const uint16_t* logits, int ldl, float* w, int* ids, int* sorted_ids, int* expert_ids,
                        int* ntpp, int* arrive, int M, int E, int topk, int renorm, int blk, const uint16_t* x,
                        long ldx, int H, uint8_t* xq, float* xs, hipStream_t st) {
  const int cap = (int)table_capacity((long)M * topk, E, blk);
  const int Ep = (E + 15) & ~15;
  const size_t lds = (size_t)Ep * 12 + 64 * 4 + (size_t)cap * 4 + (size_t)(cap / blk) * 4 + (size_t)M * topk * 4;
  const int rpw = small_rpw(M);
  const dim3 grid((M + rpw - 1) / rpw + (x ? (M + QPW - 1) / QPW : 0));
#define RS(EPLV)                                                                                                   \
  return launch_small_inst<EPLV>(grid, lds, st, logits, ldl, w, ids, sorted_ids, expert_ids, ntpp, arrive, M, E, \
                                 topk, renorm, blk, cap, rpw, x, ldx, H, xq, xs)
  switch (epl_for(E)) {
    case 2: RS(2);
    case 4: RS(4);
    case 6: RS(6);
    case 8: RS(8);
    default: return hipErrorInvalidValue;
  }
#undef RS
}

// Chunks of 8 values a lane for quant_row_wave over H values (0: the rows do not suit the wave quant).
int quant_chunks_for(int H, long ldx, const void* x, const void* xq) {
  if (H < 8 || H % 8 || H > 512 * QRMAX || ldx < H || ldx % 8 || (reinterpret_cast<uintptr_t>(x) & 15) ||
      (reinterpret_cast<uintptr_t>(xq) & 7))
    return 0;
  const int nv = (H / 8 + WAVE - 1) / WAVE;
  return nv <= 1 ? 1 : nv <= 2 ? 2 : nv <= 4 ? 4 : 8;
}

// The one-wave-per-row routing launch (numel <= SMALL_MAX), with the extras R (quant chunks, 0 = none) and ex.
int launch_fused(const uint16_t* logits, int ldl, float* w, int* ids, int* sorted_ids, int* expert_ids, int* ntpp,
                 int* arrive, int M, int E, int topk, int renorm, int blk, int R, const RouteExtras& ex,
                 hipStream_t st) {
  const int nblk = (M + FW - 1) / FW;
  if (nblk > 1 && !arrive) return 1;
#define RF(EPLV, RV)                                                                                              \
  hipLaunchKernelGGL((route_fused_kernel<EPLV, RV>), dim3(nblk), dim3(FT), 0, st, logits, ldl, w, ids,           \
                     sorted_ids, expert_ids, ntpp, arrive, M, E, topk, renorm, blk, ex)
#define RFR(EPLV)                    \
  switch (R) {                       \
    case 0: RF(EPLV, 0); break;      \
    case 1: RF(EPLV, 1); break;      \
    case 2: RF(EPLV, 2); break;      \
    case 4: RF(EPLV, 4); break;      \
    case 8: RF(EPLV, 8); break;      \
    default: return 1;               \
  }
  switch (epl_for(E)) {
    case 2: RFR(2); break;
    case 4: RFR(4); break;
    case 6: RFR(6); break;
    case 8: RFR(8); break;
    case 12: RFR(12); break;
    case 16: RFR(16); break;
    default: return 1;
  }
#undef RFR
#undef RF
  return (int)hipGetLastError();
}

}  // namespace

// Reference: kernels/r9k_moe_route.hip:217-233. logits [M, E] bf16 (row stride ldl) -> weights fp32 [M, topk],
// ids int32 [M, topk], and the align tables (first capacity(M * topk) entries). scratch (2E+1 int32, zeroed once by
// the caller, as in the reference contract): its first int is the workgroups' arrival counter, left zero; calls
// that share one scratch must not overlap. numel > 4096 takes the top-k launch plus the single-workgroup table
// launch. Returns 0, 1 for an unsupported shape, else the HIP error code.
extern "C" int r9k_moe_route(long logits, int ldl, long weights, long ids, long sorted_ids, long expert_ids,
                             long ntpp, long scratch, int M, int E, int topk, int renorm, int blk, long stream) {
  if (!route_args_ok(M, E, topk, blk) || ldl < E) return 1;
  const hipStream_t st = (hipStream_t)stream;
  const long numel = (long)M * topk;
  if (small_fits(M, E, topk, blk, (const void*)scratch, nullptr, 0, 0, nullptr, nullptr))
    return (int)launch_small((const uint16_t*)logits, ldl, (float*)weights, (int*)ids, (int*)sorted_ids,
                             (int*)expert_ids, (int*)ntpp, (int*)scratch, M, E, topk, renorm, blk, nullptr, 0, 0,
                             nullptr, nullptr, st);
  if (numel <= SMALL_MAX) {
    const RouteExtras none{};
    return launch_fused((const uint16_t*)logits, ldl, (float*)weights, (int*)ids, (int*)sorted_ids, (int*)expert_ids,
                        (int*)ntpp, (int*)scratch, M, E, topk, renorm, blk, 0, none, st);
  } else {
    if (numel > 0x7fffffffL) return 1;
    if (launch_topk((const uint16_t*)logits, ldl, (float*)weights, (int*)ids, M, E, topk, renorm, st)) return 1;
    hipLaunchKernelGGL(align_big_single_kernel, dim3(1), dim3(AT), 0, st, (const int*)ids, (int)numel, E, blk,
                       (int*)sorted_ids, (int*)expert_ids, (int*)ntpp);
  }
  return (int)hipGetLastError();
}

// r9k_moe_route plus the per-token fp8 quant of the layer's activations in the same launch (the quant of
// r9k_quant_rows_fp8, same bytes): x bf16 [M, H] (row stride ldx) -> xq e4m3 [M, H], xs fp32 [M]. scratch as for
// r9k_moe_route. Served while the routing is one launch (numel <= 4096) for rows that suit the wave quant (H % 8 ==
// 0, H <= 4096, ldx % 8 == 0, x 16-byte and xq 8-byte aligned); returns 2 for any other shape, with nothing
// launched, so the caller runs r9k_moe_route and r9k_quant_rows_fp8. 1 bad arguments, else the HIP error.
extern "C" int r9k_moe_route_quant(long logits, int ldl, long weights, long ids, long sorted_ids, long expert_ids,
                                   long ntpp, long scratch, int M, int E, int topk, int renorm, int blk, long x,
                                   long ldx, int H, long xq, long xs, long stream) {
  if (!route_args_ok(M, E, topk, blk) || ldl < E || !x) return 1;
  if (small_fits(M, E, topk, blk, (const void*)scratch, (const void*)x, ldx, H, (const void*)xq, (const void*)xs))
    return (int)launch_small((const uint16_t*)logits, ldl, (float*)weights, (int*)ids, (int*)sorted_ids,
                             (int*)expert_ids, (int*)ntpp, (int*)scratch, M, E, topk, renorm, blk,
                             (const uint16_t*)x, ldx, H, (uint8_t*)xq, (float*)xs, (hipStream_t)stream);
  const int R = quant_chunks_for(H, ldx, (const void*)x, (const void*)xq);
  if ((long)M * topk > SMALL_MAX || !R || !xs) return 2;
  RouteExtras ex{};
  ex.x = (const uint16_t*)x;
  ex.ldx = ldx;
  ex.H = H;
  ex.xq = (uint8_t*)xq;
  ex.xs = (float*)xs;
  return launch_fused((const uint16_t*)logits, ldl, (float*)weights, (int*)ids, (int*)sorted_ids, (int*)expert_ids,
                      (int*)ntpp, (int*)scratch, M, E, topk, renorm, blk, R, ex, (hipStream_t)stream);
}

// r9k_moe_route(_quant) with the tables in two layouts, of which the device keeps one (no reference counterpart:
// the reference picks its block size on the host from the row count; here a skewed step the host cannot see may
// take the big blocks): blocks of blk rows into sorted_ids / expert_ids / ntpp (the whole capacity) or of big_blk
// rows into sorted_big / expert_big / ntpp_big (live entries only): the big layout is kept when its nbig blocks
// hold numel >= min_rows * nbig rows (r9k_moe_pick_blocks' rule), only the kept layout is written, and the other's
// ntpp is set to 0 (its entries are left as they were). x = 0:
// no activation quant. Served for numel <= 4096 (one-wave-per-row launch) and, with x, rows that suit the wave
// quant (as r9k_moe_route_quant); 2 otherwise (nothing launched). 1 bad arguments, else the HIP error.
extern "C" int r9k_moe_route_dual(long logits, int ldl, long weights, long ids, long sorted_ids, long expert_ids,
                                  long ntpp, long scratch, int M, int E, int topk, int renorm, int blk, long x,
                                  long ldx, int H, long xq, long xs, int big_blk, long sorted_big, long expert_big,
                                  long ntpp_big, int min_rows, long stream) {
  if (!route_args_ok(M, E, topk, blk) || ldl < E || big_blk < 1 || (big_blk & (big_blk - 1)) || min_rows < 0 ||
      !sorted_big || !expert_big || !ntpp_big)
    return 1;
  if ((long)M * topk > SMALL_MAX) return 2;
  int R = 0;
  RouteExtras ex{};
  if (x) {
    R = quant_chunks_for(H, ldx, (const void*)x, (const void*)xq);
    if (!R || !xs) return 2;
    ex.x = (const uint16_t*)x;
    ex.ldx = ldx;
    ex.H = H;
    ex.xq = (uint8_t*)xq;
    ex.xs = (float*)xs;
  }
  ex.big_blk = big_blk;
  ex.min_rows = min_rows;
  ex.sorted_big = (int*)sorted_big;
  ex.expert_big = (int*)expert_big;
  ex.ntpp_big = (int*)ntpp_big;
  return launch_fused((const uint16_t*)logits, ldl, (float*)weights, (int*)ids, (int*)sorted_ids, (int*)expert_ids,
                      (int*)ntpp, (int*)scratch, M, E, topk, renorm, blk, R, ex, (hipStream_t)stream);
}

extern "C" int r9k_moe_route_max_experts(void) { return MAX_E; }
extern "C" int r9k_moe_route_max_topk(void) { return MAX_K; }

// r9k_moe_topk plus r9k_quant_rows_fp8 of the layer's activations in one launch, any M: x bf16 [M, H] (row stride
// ldx) -> xq e4m3 [M, H], xs fp32 [M], the bytes of r9k_quant_rows_fp8. Rows the wave quant does not take (H % 8,
// H > 4096, x not 16-byte or xq not 8-byte aligned, ldx % 8) return 2 with nothing launched, so the caller runs the
// two calls. 1 bad arguments, else the HIP error.
extern "C" int r9k_moe_topk_quant(long logits, int ldl, long weights, long ids, int M, int E, int topk, int renorm,
                                  long x, long ldx, int H, long xq, long xs, long stream) {
  if (!route_args_ok(M, E, topk, 1) || ldl < E || !x || !xq || !xs) return 1;
  if (H < 8 || H % 8 || H > 512 * QRMAX || ldx < H || ldx % 8 || (x & 15) || (xq & 7)) return 2;
  const int nv = (H / 8 + WAVE - 1) / WAVE;
  const int R = nv <= 1 ? 1 : nv <= 2 ? 2 : nv <= 4 ? 4 : 8;
  const dim3 grid(2 * ((M + RW - 1) / RW)), block(RW * WAVE);
  const hipStream_t st = (hipStream_t)stream;
  if (const int np = np16_for((const void*)logits, ldl, E)) {
    const dim3 grid16((M + R16 - 1) / R16 + (M + RW - 1) / RW);
#define TQ16(NPV, RV)                                                                                              \
  hipLaunchKernelGGL((topk16_quant_kernel<NPV, RV>), grid16, block, 0, st, (const uint16_t*)logits, ldl,          \
                     (float*)weights, (int*)ids, M, E, topk, renorm, (const uint16_t*)x, ldx, H, (uint8_t*)xq,      \
                     (float*)xs)
#define TQ16R(NPV)                  \
  switch (R) {                      \
    case 1: TQ16(NPV, 1); break;    \
    case 2: TQ16(NPV, 2); break;    \
    case 4: TQ16(NPV, 4); break;    \
    default: TQ16(NPV, 8); break;   \
  }
    switch (np) {
      case 2: TQ16R(2); break;
      case 4: TQ16R(4); break;
      case 8: TQ16R(8); break;
      case 9: TQ16R(9); break;
      case 12: TQ16R(12); break;
      default: TQ16R(16); break;
    }
#undef TQ16R
#undef TQ16
    return (int)hipGetLastError();
  }
#define TQ(EPLV, RV)                                                                                              \
  hipLaunchKernelGGL((topk_quant_kernel<EPLV, RV>), grid, block, 0, st, (const uint16_t*)logits, ldl,            \
                     (float*)weights, (int*)ids, M, E, topk, renorm, (const uint16_t*)x, ldx, H, (uint8_t*)xq,      \
                     (float*)xs)
#define TQR(EPLV)                 \
  switch (R) {                    \
    case 1: TQ(EPLV, 1); break;   \
    case 2: TQ(EPLV, 2); break;   \
    case 4: TQ(EPLV, 4); break;   \
    default: TQ(EPLV, 8); break;  \
  }
  switch (epl_for(E)) {
    case 2: TQR(2); break;
    case 4: TQR(4); break;
    case 6: TQR(6); break;
    case 8: TQR(8); break;
    case 12: TQR(12); break;
    case 16: TQR(16); break;
    default: return 1;
  }
#undef TQR
#undef TQ
  return (int)hipGetLastError();
}

// Routing only: the stock top-k softmax router's outputs (no tables). 0 / 1 unsupported / HIP error.
extern "C" int r9k_moe_topk(long logits, int ldl, long weights, long ids, int M, int E, int topk, int renorm,
                            long stream) {
  if (!route_args_ok(M, E, topk, 1) || ldl < E) return 1;
  if (launch_topk((const uint16_t*)logits, ldl, (float*)weights, (int*)ids, M, E, topk, renorm,
                  (hipStream_t)stream))
    return 1;
  return (int)hipGetLastError();
}

// int32 count of the scratch r9k_moe_align needs for `numel` routed rows over E experts (the per-chunk histograms
// of the multi-workgroup path, rewritten by every call).
extern "C" long r9k_moe_align_scratch_ints(int numel, int E) { return align_scratch_ints(numel, E); }

// Tables only, from ids int32 [numel] (the stock moe_align_block_size role; ids outside [0, E) are skipped).
// scratch: r9k_moe_align_scratch_ints(numel, E) int32 (the chunk histograms of the two-launch path, overwritten by
// every call; calls sharing one scratch must not overlap). 0 / 1 bad args / HIP
// error.
extern "C" int r9k_moe_align(long ids, int numel, int E, int blk, long sorted_ids, long expert_ids, long ntpp,
                             long scratch, long scratch_ints, long stream) {
  if (numel < 1 || E < 1 || E > MAX_E || blk < 1 || (blk & (blk - 1))) return 1;
  if (numel > SMALL_MAX && (!scratch || scratch_ints < r9k_moe_align_scratch_ints(numel, E))) return 1;
  if (launch_align((const int*)ids, numel, E, blk, (int*)sorted_ids, (int*)expert_ids, (int*)ntpp, (int*)scratch,
                   (hipStream_t)stream))
    return 1;
  return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------- align without allocation
// r9k_moe_align's multi-workgroup path needs scratch (the per-chunk histograms). Callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc) use r9k_moe_align_noalloc, whose scratch is this file-scope device array: 1 MiB per GPU, held by every
// GPU the library runs on until the process ends. The histograms are fully written before they are read within a
// call. All
// calls on one GPU share the array and keep the last call's contents: calls that overlap on one GPU (other streams,
// concurrent graph replays) race on it.
namespace {

constexpr long NOALLOC_SCRATCH_INTS = 1L << 18;
static __device__ __align__(256) int scratch[NOALLOC_SCRATCH_INTS];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
int* g_scratch_ptr[MAX_DEVICES] = {};

// The device address of `scratch` on the current device, looked up once per device (with that device current) by
// hipGetSymbolAddress: in host code the array's name is only a host-side stand-in. nullptr on failure.
int* noalloc_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    g_scratch_ptr[dev] = static_cast<int*>(p);
  }
  return g_scratch_ptr[dev];
}

}  // namespace

// No counterpart in the reference: r9k_moe_align writing only the live part of the tables -- the expert blocks up to
// ntpp with their padding entries -- and leaving the capacity past ntpp as it was, for consumers that read no
// further than ntpp (this library's GEMMs do not). A capacity-sized layout whose tail dominates (256-row blocks over
// many experts at decode widths: numel + E * 255 entries) costs a fraction to build. Arguments and codes as
// r9k_moe_align.
extern "C" int r9k_moe_align_live(long ids, int numel, int E, int blk, long sorted_ids, long expert_ids, long ntpp,
                                  long scratch, long scratch_ints, long stream) {
  if (numel < 1 || E < 1 || E > MAX_E || blk < 1 || (blk & (blk - 1))) return 1;
  if (numel > SMALL_MAX && (!scratch || scratch_ints < r9k_moe_align_scratch_ints(numel, E))) return 1;
  if (launch_align((const int*)ids, numel, E, blk, (int*)sorted_ids, (int*)expert_ids, (int*)ntpp, (int*)scratch,
                   (hipStream_t)stream, 0))
    return 1;
  return (int)hipGetLastError();
}

// No counterpart in the reference: r9k_moe_align for callers that cannot allocate (graph capture, tight serving
// loops, allocation-free harnesses). The scratch is the library's own 1 MiB device array per GPU (see above), so
// the caller passes only ids and the three tables; overlapping calls on one GPU race. Tables as r9k_moe_align's, bit
// for bit. 0; 1 bad arguments or a HIP error (as r9k_moe_align); -9 when the step needs more scratch than the array
// holds (r9k_moe_align_scratch_ints(numel, E) > r9k_moe_align_noalloc_max_ints()); -6 the array's address could not
// be had.
extern "C" long r9k_moe_align_noalloc_max_ints(void) { return NOALLOC_SCRATCH_INTS; }

extern "C" int r9k_moe_align_noalloc(long ids, int numel, int E, int blk, long sorted_ids, long expert_ids,
                                     long ntpp, long stream) {
  if (numel < 1 || E < 1 || E > MAX_E || blk < 1 || (blk & (blk - 1))) return 1;
  if (align_scratch_ints(numel, E) > NOALLOC_SCRATCH_INTS) return -9;
  int* sp = nullptr;
  if (numel > SMALL_MAX && !(sp = noalloc_scratch())) return -6;
  if (launch_align((const int*)ids, numel, E, blk, (int*)sorted_ids, (int*)expert_ids, (int*)ntpp, sp,
                   (hipStream_t)stream))
    return 1;
  return (int)hipGetLastError();
}

// No counterpart in the reference (it routes every expert through one block size picked on the host): the tables of
// one routed step split by expert size on the device. Experts with more than thr rows get blk_big-row blocks in
// (sorted_big, expert_big, ntpp_big), the others blk_small-row blocks in the small tables; each table holds only its
// experts' rows (ascending within each expert, as r9k_moe_align) and is written up to its ntpp only (live, as
// r9k_moe_align_live). Capacities as r9k_moe_align's for each block size; scratch as r9k_moe_align's. 0 / 1 bad
// arguments or HIP error.
extern "C" int r9k_moe_align_split(long ids, int numel, int E, int thr, int blk_big, long sorted_big, long expert_big,
                                   long ntpp_big, int blk_small, long sorted_small, long expert_small,
                                   long ntpp_small, long scratch, long scratch_ints, long stream) {
  if (numel < 1 || E < 1 || E > MAX_E || thr < 0) return 1;
  for (int b : {blk_big, blk_small})
    if (b < 1 || (b & (b - 1))) return 1;
  if (!sorted_big || !expert_big || !ntpp_big || !sorted_small || !expert_small || !ntpp_small) return 1;
  if (numel > SMALL_MAX && (!scratch || scratch_ints < r9k_moe_align_scratch_ints(numel, E))) return 1;
  if (launch_align_split((const int*)ids, numel, E, thr, blk_big, (int*)sorted_big, (int*)expert_big,
                         (int*)ntpp_big, blk_small, (int*)sorted_small, (int*)expert_small, (int*)ntpp_small,
                         (int*)scratch, (hipStream_t)stream))
    return 1;
  return (int)hipGetLastError();
}

// Keep one of two table layouts of a routed step on the device (pick_blocks_kernel): no reference counterpart (the
// reference picks its block size on the host from the row count). 0, -1 bad arguments, -6 launch error.
extern "C" int r9k_moe_pick_blocks(long ntpp_small, long ntpp_big, int numel, int big_blk, int min_rows,
                                   long stream) {
  if (!ntpp_small || !ntpp_big || numel < 0 || big_blk <= 0 || min_rows < 0) return -1;
  hipLaunchKernelGGL(pick_blocks_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, (int*)ntpp_small,
                     (int*)ntpp_big, numel, big_blk, min_rows);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}
