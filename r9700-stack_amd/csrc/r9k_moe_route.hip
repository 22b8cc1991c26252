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
// bit-exact against it. Stable ranks come from a wave64 match loop (ballot per distinct expert in the wave) plus
// per-wave counts in LDS. The whole capacity (sorted_ids [cap], expert_ids [cap / blk], cap =
// ceil((numel + E * (blk - 1)) / blk) * blk) is written, the tail with numel / -1.
//
// Entry points:
//   r9k_moe_route   the reference's one-launch routing + tables (any M; numel <= 4096 in one workgroup and one
//                   launch, larger as a top-k launch plus one single-workgroup table launch)
//   r9k_moe_topk    routing only (the stock top-k router's role)
//   r9k_moe_align   tables only from given ids (vLLM's moe_align_block_size role); large numel runs as a count
//                   launch (the last block to arrive scans) plus a scatter launch, with caller scratch.
#include "r9k_common.h"

namespace {

using namespace r9k;

constexpr int MAX_E = 1024;       // experts
constexpr int MAX_K = 16;         // top-k
constexpr int AT = 1024;          // threads of an align / fused workgroup (16 waves)
constexpr int AW = AT / WAVE;
constexpr int SMALL_MAX = 4096;   // routed rows handled by one workgroup (ids kept in LDS)
constexpr int CH = 2048;          // routed rows per chunk in the multi-workgroup align
constexpr int RW = 8;             // waves (rows) per block of the top-k kernel

// Max of a 32-bit key over the wave, returned as a wave-uniform (scalar) value: DPP within 16-lane rows (quad
// swaps, row rotates by 4 and 8), then the four row results through v_readlane and a scalar max.
__device__ __forceinline__ uint32_t wave_max_key(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));    // quad_perm [1,0,3,2]
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));    // quad_perm [2,3,0,1]
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xF, 0xF, false));   // row_ror:4
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false));   // row_ror:8
  const uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
  const uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
  return max(max(a, b), max(c, d));
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

// One wave routes one row. Lane k < topk ends holding selection k. Writes w/ids (global) and optionally LDS ids.
template <int EPL>
__device__ __forceinline__ void topk_row(const uint16_t* __restrict__ row, int E, int topk, bool renorm,
                                         float* __restrict__ w_out, int* __restrict__ id_out, short* lds_ids,
                                         int lane) {
  uint16_t h[EPL];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < EPL; i++) {
    const int e = lane + WAVE * i;
    h[i] = e < E ? row[e] : (uint16_t)0xff80u;          // -inf for lanes past E
    mx = fmaxf(mx, bf2f(h[i]));
  }
  mx = wave_max(mx);
  float ex[EPL];
  uint32_t key[EPL];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; i++) {
    const int e = lane + WAVE * i;
    const float d = bf2f(h[i]) - mx;
    const bool live = d >= -87.f;                        // false for NaN (NaN logit, or a +inf row)
    ex[i] = (e < E && live) ? expf(d) : 0.f;
    s += ex[i];
    key[i] = e < E ? route_key(h[i], live, e) : 0u;
  }
  s = wave_sum(s);
  float wsel = 0.f, tot = 0.f;
  int isel = 0;
  for (int k = 0; k < topk; k++) {
    uint32_t b = key[0];
#pragma unroll
    for (int i = 1; i < EPL; i++) b = max(b, key[i]);
    b = wave_max_key(b);
    const int idx = 1023 - (int)(b & 1023u);
    const int owner = idx & (WAVE - 1), slot = idx / WAVE;
    float eb = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; i++)
      if (i == slot) eb = ex[i];
    eb = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(eb), owner));
#pragma unroll
    for (int i = 0; i < EPL; i++)
      if (i == slot && lane == owner) key[i] = 0u;
    const float p = s > 0.f ? eb / s : 0.f;
    tot += p;
    if (lane == k) { wsel = p; isel = idx; }
  }
  float p = wsel;
  if (renorm) p = tot > 0.f ? p / tot : 0.f;
  if (isel < 0 || isel >= E) isel = 0;               // unreachable (topk <= E); keeps every table write in range
  if (lane < topk) {
    w_out[lane] = p;
    id_out[lane] = isel;
    if (lds_ids) lds_ids[lane] = (short)isel;
  }
}

struct AlignLds {
  int cnt[MAX_E];              // counts, then the running scatter cursor
  int offs[MAX_E];             // first padded position of each expert
  uint8_t wcnt[AW][MAX_E];     // rows per (wave, expert) in the current 1024-row sub-chunk
  int scan[AW];
};

// Exclusive scan of the block-padded counts (one expert per thread, E <= AT): offs[], returns the padded total.
__device__ __forceinline__ int padded_scan(AlignLds& sh, int E, int blk) {
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int c = tid < E ? sh.cnt[tid] : 0;
  const int n = ((c + blk - 1) / blk) * blk;
  int x = n;
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) {
    const int y = __shfl_up(x, o, WAVE);
    if (lane >= o) x += y;
  }
  if (lane == WAVE - 1) sh.scan[wave] = x;
  __syncthreads();
  int wbase = 0, total = 0;
#pragma unroll
  for (int w = 0; w < AW; w++) {
    if (w < wave) wbase += sh.scan[w];
    total += sh.scan[w];
  }
  if (tid < E) sh.offs[tid] = wbase + x - n;
  __syncthreads();
  return total;
}

// expert_ids / padding entries of every expert with rows, ntpp, and the capacity tail.
__device__ __forceinline__ void write_layout(const int* cnt, const int* offs, int total, int numel, int E, int blk,
                                             int* __restrict__ sorted_ids, int* __restrict__ expert_ids,
                                             int* __restrict__ ntpp) {
  const int tid = threadIdx.x;
  if (tid == 0) ntpp[0] = total;
  if (tid < E) {
    const int c = cnt[tid];
    if (c > 0) {
      const int o = offs[tid], n = ((c + blk - 1) / blk) * blk;
      for (int b = o / blk; b < (o + n) / blk; b++) expert_ids[b] = tid;
      for (int i = o + c; i < o + n; i++) sorted_ids[i] = numel;
    }
  }
  const long cap = ((long)numel + (long)E * (blk - 1) + blk - 1) / blk * blk;
  for (long i = total + tid; i < cap; i += AT) sorted_ids[i] = numel;
  for (long b = total / blk + tid; b < cap / blk; b += AT) expert_ids[b] = -1;
}

// Stable placement of rows [base, min(base + AT, end)) given the per-expert cursor in sh.cnt (advanced here).
// ids_at(t) returns the expert of flat row t. Rows with an expert outside [0, E) are not placed.
template <typename IdsAt>
__device__ __forceinline__ void stable_subchunk(AlignLds& sh, int base, int end, int E, int* __restrict__ sorted_ids,
                                                IdsAt ids_at) {
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int t = base + tid;
  const int e = t < end ? ids_at(t) : -1;
  const bool valid = e >= 0 && e < E;
  uint64_t pending = __ballot(valid);
  int rank = 0;
  while (pending) {
    const int leader = __ffsll((unsigned long long)pending) - 1;
    const int e0 = __shfl(e, leader, WAVE);
    const uint64_t m = __ballot(valid && e == e0);
    if (valid && e == e0) rank = __popcll(m & __lanemask_lt());
    if (lane == leader) sh.wcnt[wave][e0] = (uint8_t)__popcll(m);
    pending &= ~m;
  }
  __syncthreads();
  if (valid) {
    int pre = 0;
    for (int w = 0; w < wave; w++) pre += sh.wcnt[w][e];
    sorted_ids[sh.cnt[e] + pre + rank] = t;
  }
  __syncthreads();
  if (tid < E) {
    int tot = 0;
#pragma unroll
    for (int w = 0; w < AW; w++) { tot += sh.wcnt[w][tid]; sh.wcnt[w][tid] = 0; }
    sh.cnt[tid] += tot;
  }
  __syncthreads();
}

__device__ __forceinline__ void zero_wcnt(AlignLds& sh) {
  uint32_t* p = reinterpret_cast<uint32_t*>(&sh.wcnt[0][0]);
  for (int i = threadIdx.x; i < AW * MAX_E / 4; i += AT) p[i] = 0u;
}

// The whole table build in one workgroup: count, scan, layout, stable scatter (cursor starts at offs).
template <typename IdsAt>
__device__ void align_one_block(AlignLds& sh, int numel, int E, int blk, int* __restrict__ sorted_ids,
                                int* __restrict__ expert_ids, int* __restrict__ ntpp, IdsAt ids_at) {
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += AT) sh.cnt[e] = 0;
  zero_wcnt(sh);
  __syncthreads();
  for (int t = tid; t < numel; t += AT) {
    const int e = ids_at(t);
    if (e >= 0 && e < E) atomicAdd(&sh.cnt[e], 1);
  }
  __syncthreads();
  const int total = padded_scan(sh, E, blk);
  write_layout(sh.cnt, sh.offs, total, numel, E, blk, sorted_ids, expert_ids, ntpp);
  __syncthreads();
  if (tid < E) sh.cnt[tid] = sh.offs[tid];
  __syncthreads();
  for (int base = 0; base < numel; base += AT) stable_subchunk(sh, base, numel, E, sorted_ids, ids_at);
}

// Fused routing + tables, one workgroup, numel <= SMALL_MAX (reference: r9k_moe_route_kernel, single-block path).
template <int EPL>
__global__ void __launch_bounds__(AT) route_fused_kernel(const uint16_t* __restrict__ logits, int ldl,
                                                         float* __restrict__ weights, int* __restrict__ ids,
                                                         int* __restrict__ sorted_ids, int* __restrict__ expert_ids,
                                                         int* __restrict__ ntpp, int M, int E, int topk, int renorm,
                                                         int blk) {
  __shared__ AlignLds sh;
  __shared__ short lids[SMALL_MAX];
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  for (int r = wave; r < M; r += AW)
    topk_row<EPL>(logits + (size_t)r * ldl, E, topk, renorm != 0, weights + (size_t)r * topk,
                  ids + (size_t)r * topk, lids + r * topk, lane);
  __syncthreads();
  align_one_block(sh, M * topk, E, blk, sorted_ids, expert_ids, ntpp, [&](int t) { return (int)lids[t]; });
}

template <int EPL>
__global__ void __launch_bounds__(RW * WAVE) topk_kernel(const uint16_t* __restrict__ logits, int ldl,
                                                         float* __restrict__ weights, int* __restrict__ ids, int M,
                                                         int E, int topk, int renorm) {
  const int r = blockIdx.x * RW + threadIdx.x / WAVE;
  if (r >= M) return;
  topk_row<EPL>(logits + (size_t)r * ldl, E, topk, renorm != 0, weights + (size_t)r * topk, ids + (size_t)r * topk,
                nullptr, threadIdx.x % WAVE);
}

// Tables from ids in global memory, one workgroup (any numel; the multi-block path is faster above SMALL_MAX).
__global__ void __launch_bounds__(AT) align_single_kernel(const int* __restrict__ ids, int numel, int E, int blk,
                                                          int* __restrict__ sorted_ids, int* __restrict__ expert_ids,
                                                          int* __restrict__ ntpp) {
  __shared__ AlignLds sh;
  align_one_block(sh, numel, E, blk, sorted_ids, expert_ids, ntpp, [&](int t) { return ids[t]; });
}

// Multi-block align, pass 1: per-chunk histogram into scratch; the last chunk to arrive turns the histograms into
// per-(chunk, expert) scatter bases and writes the layout. scratch = [arrive][nchunks x E]; arrive is zero at entry
// and left zero.
__global__ void __launch_bounds__(AT) align_count_kernel(const int* __restrict__ ids, int numel, int E, int blk,
                                                         int* __restrict__ sorted_ids, int* __restrict__ expert_ids,
                                                         int* __restrict__ ntpp, int* __restrict__ scratch) {
  __shared__ AlignLds sh;
  __shared__ int s_last;
  const int tid = threadIdx.x, c = blockIdx.x, nch = gridDim.x;
  int* const arrive = scratch;
  int* const hist = scratch + 1;
  for (int e = tid; e < E; e += AT) sh.cnt[e] = 0;
  __syncthreads();
  const int t0 = c * CH, t1 = min(numel, t0 + CH);
  for (int t = t0 + tid; t < t1; t += AT) {
    const int e = ids[t];
    if (e >= 0 && e < E) atomicAdd(&sh.cnt[e], 1);
  }
  __syncthreads();
  for (int e = tid; e < E; e += AT) hist[(size_t)c * E + e] = sh.cnt[e];
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = (atomicAdd(arrive, 1) == nch - 1) ? 1 : 0;
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  // last block: totals, padded scan, per-chunk bases (in place), layout
  int tot = 0;
  if (tid < E)
    for (int cc = 0; cc < nch; cc++)
      tot += __hip_atomic_load(hist + (size_t)cc * E + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (tid < E) sh.cnt[tid] = tot;
  __syncthreads();
  const int total = padded_scan(sh, E, blk);
  write_layout(sh.cnt, sh.offs, total, numel, E, blk, sorted_ids, expert_ids, ntpp);
  if (tid < E) {
    int run = sh.offs[tid];
    for (int cc = 0; cc < nch; cc++) {
      int* h = hist + (size_t)cc * E + tid;
      const int v = __hip_atomic_load(h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *h = run;
      run += v;
    }
  }
  if (tid == 0) *arrive = 0;
}

// Multi-block align, pass 2: stable scatter of one chunk from its bases.
__global__ void __launch_bounds__(AT) align_scatter_kernel(const int* __restrict__ ids, int numel, int E,
                                                           int* __restrict__ sorted_ids,
                                                           const int* __restrict__ scratch) {
  __shared__ AlignLds sh;
  const int tid = threadIdx.x, c = blockIdx.x;
  const int* base = scratch + 1 + (size_t)c * E;
  for (int e = tid; e < E; e += AT) sh.cnt[e] = base[e];
  zero_wcnt(sh);
  __syncthreads();
  const int t0 = c * CH, t1 = min(numel, t0 + CH);
  for (int b = t0; b < t1; b += AT) stable_subchunk(sh, b, t1, E, sorted_ids, [&](int t) { return ids[t]; });
}

int epl_for(int E) {
  const int need = (E + WAVE - 1) / WAVE;
  for (int v : {2, 4, 6, 8, 12, 16})
    if (need <= v) return v;
  return -1;
}

int launch_topk(const uint16_t* logits, int ldl, float* w, int* ids, int M, int E, int topk, int renorm,
                hipStream_t st) {
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

bool route_args_ok(int M, int E, int topk, int blk) {
  return M >= 1 && E >= 1 && E <= MAX_E && topk >= 1 && topk <= MAX_K && topk <= E && blk >= 1 &&
         (blk & (blk - 1)) == 0;
}

}  // namespace

// Reference: kernels/r9k_moe_route.hip:217-233. logits [M, E] bf16 (row stride ldl) -> weights fp32 [M, topk],
// ids int32 [M, topk], and the align tables (first capacity(M * topk) entries). scratch (2E+1 int32) is part of the
// reference contract; this implementation keeps its state in LDS and never touches it. Returns 0, 1 for an
// unsupported shape, else the HIP error code.
extern "C" int r9k_moe_route(long logits, int ldl, long weights, long ids, long sorted_ids, long expert_ids,
                             long ntpp, long scratch, int M, int E, int topk, int renorm, int blk, long stream) {
  (void)scratch;
  if (!route_args_ok(M, E, topk, blk) || ldl < E) return 1;
  const hipStream_t st = (hipStream_t)stream;
  const long numel = (long)M * topk;
  if (numel <= SMALL_MAX) {
#define RF(EPLV)                                                                                                    \
  hipLaunchKernelGGL(route_fused_kernel<EPLV>, dim3(1), dim3(AT), 0, st, (const uint16_t*)logits, ldl,             \
                     (float*)weights, (int*)ids, (int*)sorted_ids, (int*)expert_ids, (int*)ntpp, M, E, topk, renorm, \
                     blk)
    switch (epl_for(E)) {
      case 2: RF(2); break;
      case 4: RF(4); break;
      case 6: RF(6); break;
      case 8: RF(8); break;
      case 12: RF(12); break;
      case 16: RF(16); break;
      default: return 1;
    }
#undef RF
  } else {
    if (numel > 0x7fffffffL) return 1;
    if (launch_topk((const uint16_t*)logits, ldl, (float*)weights, (int*)ids, M, E, topk, renorm, st)) return 1;
    hipLaunchKernelGGL(align_single_kernel, dim3(1), dim3(AT), 0, st, (const int*)ids, (int)numel, E, blk,
                       (int*)sorted_ids, (int*)expert_ids, (int*)ntpp);
  }
  return (int)hipGetLastError();
}

extern "C" int r9k_moe_route_max_experts(void) { return MAX_E; }
extern "C" int r9k_moe_route_max_topk(void) { return MAX_K; }

// Routing only: the stock top-k softmax router's outputs (no tables). 0 / 1 unsupported / HIP error.
extern "C" int r9k_moe_topk(long logits, int ldl, long weights, long ids, int M, int E, int topk, int renorm,
                            long stream) {
  if (!route_args_ok(M, E, topk, 1) || ldl < E) return 1;
  if (launch_topk((const uint16_t*)logits, ldl, (float*)weights, (int*)ids, M, E, topk, renorm,
                  (hipStream_t)stream))
    return 1;
  return (int)hipGetLastError();
}

// int32 count of the scratch r9k_moe_align needs for `numel` routed rows over E experts (zero it once; the kernels
// leave it zero).
extern "C" long r9k_moe_align_scratch_ints(int numel, int E) {
  if (numel <= SMALL_MAX) return 1;
  return 1 + (long)((numel + CH - 1) / CH) * E;
}

// Tables only, from ids int32 [numel] (the stock moe_align_block_size role; ids outside [0, E) are skipped).
// scratch: r9k_moe_align_scratch_ints(numel, E) int32, zero at the first call. 0 / 1 bad args / HIP error.
extern "C" int r9k_moe_align(long ids, int numel, int E, int blk, long sorted_ids, long expert_ids, long ntpp,
                             long scratch, long scratch_ints, long stream) {
  if (numel < 1 || E < 1 || E > MAX_E || blk < 1 || (blk & (blk - 1))) return 1;
  const hipStream_t st = (hipStream_t)stream;
  if (numel <= SMALL_MAX) {
    hipLaunchKernelGGL(align_single_kernel, dim3(1), dim3(AT), 0, st, (const int*)ids, numel, E, blk,
                       (int*)sorted_ids, (int*)expert_ids, (int*)ntpp);
  } else {
    if (!scratch || scratch_ints < r9k_moe_align_scratch_ints(numel, E)) return 1;
    const int nch = (numel + CH - 1) / CH;
    hipLaunchKernelGGL(align_count_kernel, dim3(nch), dim3(AT), 0, st, (const int*)ids, numel, E, blk,
                       (int*)sorted_ids, (int*)expert_ids, (int*)ntpp, (int*)scratch);
    hipLaunchKernelGGL(align_scatter_kernel, dim3(nch), dim3(AT), 0, st, (const int*)ids, numel, E,
                       (int*)sorted_ids, (const int*)scratch);
  }
  return (int)hipGetLastError();
}
