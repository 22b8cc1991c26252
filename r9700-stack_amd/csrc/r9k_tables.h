// r9k_tables.h -- the moe_align_block_size table build of one workgroup (LDS histogram, scan of the block-padded
// counts, block layout and a stable placement: rows ascend within each expert), shared by the routing kernels and
// the expert cache's one-launch manage + tables (reference contract: kernels/r9k_moe_route.hip:27-31,
// r9700_vllm/kernels/moe.py:574-592).
#pragma once
#include "r9k_common.h"

namespace r9k {

constexpr int TAB_MAX_E = 1024;      // experts (ids) one workgroup's tables cover
constexpr int TAB_SMALL_MAX = 4096;  // routed rows whose tables one workgroup builds from LDS

// Workgroup barrier that orders LDS traffic only (global stores stay in flight).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int NT>
struct TabLds {
  static constexpr int NW = NT / WAVE;
  int cnt[TAB_MAX_E];              // rows per expert
  int offs[TAB_MAX_E];             // first padded position of each expert
  int cursor[TAB_MAX_E];           // next slot of each expert during the placement
  uint16_t wcnt[NW][TAB_MAX_E];    // rows per (wave, expert) in the current round of NT rows; zero between rounds
  int scan[NW];
};

template <int NT>
__device__ __forceinline__ void zero_counts(TabLds<NT>& sh, int E) {
  for (int e = threadIdx.x; e < E; e += NT) sh.cnt[e] = 0;
  uint32_t* p = reinterpret_cast<uint32_t*>(&sh.wcnt[0][0]);
  for (int i = threadIdx.x; i < TabLds<NT>::NW * TAB_MAX_E / 2; i += NT) p[i] = 0u;
}

// Block arithmetic of the table builders: rows rounded up to whole blocks and positions in blocks, by shifts and
// masks for the powers of two every routing entry requires (P2), by integer division for the other block sizes the
// expert cache's entries accept. The builders dispatch once on the block size (wave-uniform).
template <bool P2>
struct Blocks {
  int blk, lb;
  __device__ __forceinline__ explicit Blocks(int b) : blk(b), lb(P2 ? __builtin_ctz((unsigned)b) : 0) {}
  __device__ __forceinline__ int up(int v) const { return P2 ? (v + blk - 1) & -blk : (v + blk - 1) / blk * blk; }
  __device__ __forceinline__ int div(int v) const { return P2 ? v >> lb : v / blk; }
};

// Exclusive scan of the block-padded counts: offs[], returns the padded total. Thread t covers the experts
// [t * ept, t * ept + ept), ept = ceil(E / NT) (one expert a thread while E <= NT), so offsets ascend with the expert.
template <int NT, bool P2>
__device__ __forceinline__ int padded_scan_impl(TabLds<NT>& sh, int E, const Blocks<P2> bk) {
  constexpr int NW = NT / WAVE;
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int ept = (E + NT - 1) / NT;
  const int e0 = min(tid * ept, E), e1 = min(e0 + ept, E);
  int n = 0;
  for (int e = e0; e < e1; e++) n += bk.up(sh.cnt[e]);
  int x = n;
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) {
    const int y = __shfl_up(x, o, WAVE);
    if (lane >= o) x += y;
  }
  if (lane == WAVE - 1) sh.scan[wave] = x;
  lds_barrier();
  int wbase = 0, total = 0;
#pragma unroll
  for (int w = 0; w < NW; w++) {
    if (w < wave) wbase += sh.scan[w];
    total += sh.scan[w];
  }
  int o = wbase + x - n;
  for (int e = e0; e < e1; e++) {
    sh.offs[e] = o;
    o += bk.up(sh.cnt[e]);
  }
  lds_barrier();
  return total;
}

template <int NT>
__device__ __forceinline__ int padded_scan(TabLds<NT>& sh, int E, int blk) {
  if ((blk & (blk - 1)) == 0) return padded_scan_impl<NT, true>(sh, E, Blocks<true>(blk));
  return padded_scan_impl<NT, false>(sh, E, Blocks<false>(blk));
}

// Expert blocks and padding entries of the experts e < E with e % nshare == share, every expert's cursor at its
// first slot plus `pre` (the calling thread's expert's rows in earlier chunks), and this share's part of the
// capacity tail: sorted_ids up to `cap` entries, expert_ids up to `cap_blocks` (cap < 0: this library's capacity,
// ceil((numel + E (blk - 1)) / blk) * blk entries and cap / blk blocks). Ends with an LDS barrier.
template <int NT, bool P2>
__device__ __forceinline__ void write_layout_impl(TabLds<NT>& sh, int E, const Blocks<P2> bk, int numel, int total,
                                                  int pre, int share, int nshare, int* __restrict__ sorted_ids,
                                                  int* __restrict__ expert_ids, bool write_tail, long cap,
                                                  long cap_blocks) {
  constexpr int NW = NT / WAVE;
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  for (int e = tid; e < E; e += NT) sh.cursor[e] = sh.offs[e] + (e == tid ? pre : 0);   // pre: callers with E <= NT
  // a wave per expert of the share: its block ids and its padding entries (up to blk - 1) written by the wave's lanes.
  // The wave's experts are e_j = share + (wave + NW j) nshare; lane j % 64 fetches e_j's count and offset for a pass
  // of 64 of them, so the loop over the experts waits on no LDS read.
  const int stride = NW * nshare;
  for (int e0 = share + wave * nshare; e0 < E; e0 += WAVE * stride) {
    const int el = e0 + lane * stride;
    const int cl = el < E ? sh.cnt[el] : 0, ol = el < E ? sh.offs[el] : 0;
    for (int j = 0; j < WAVE && e0 + j * stride < E; j++) {
      const int e = e0 + j * stride;
      const int c = __builtin_amdgcn_readlane(cl, j), o = __builtin_amdgcn_readlane(ol, j);
      if (c > 0) {
        const int n = bk.up(c);
        for (int b = bk.div(o) + lane; b < bk.div(o + n); b += WAVE) expert_ids[b] = e;
        for (int i = o + c + lane; i < o + n; i += WAVE) sorted_ids[i] = numel;
      }
    }
  }
  if (!write_tail) {                            // live entries only: the capacity past ntpp is left as it was
    lds_barrier();
    return;
  }
  if (cap < 0) {
    const long raw = (long)numel + (long)E * (bk.blk - 1) + bk.blk - 1;
    cap = P2 ? raw & ~(long)(bk.blk - 1) : raw / bk.blk * bk.blk;
    cap_blocks = P2 ? cap >> bk.lb : cap / bk.blk;
  }
  const long tail = cap - total, per = nshare == 1 ? tail : (tail + nshare - 1) / nshare;
  const long i1 = min(cap, total + (long)(share + 1) * per);
  for (long i = total + (long)share * per + tid; i < i1; i += NT) sorted_ids[i] = numel;
  const long b0 = bk.div(total), btail = cap_blocks - b0, bper = nshare == 1 ? btail : (btail + nshare - 1) / nshare;
  const long b1 = min(cap_blocks, b0 + (long)(share + 1) * bper);
  for (long b = b0 + (long)share * bper + tid; b < b1; b += NT) expert_ids[b] = -1;
  lds_barrier();
}

template <int NT>
__device__ __forceinline__ void write_layout(TabLds<NT>& sh, int E, int blk, int numel, int total, int pre,
                                             int share, int nshare, int* __restrict__ sorted_ids,
                                             int* __restrict__ expert_ids, bool write_tail = true, long cap = -1,
                                             long cap_blocks = -1) {
  if ((blk & (blk - 1)) == 0)
    write_layout_impl<NT, true>(sh, E, Blocks<true>(blk), numel, total, pre, share, nshare, sorted_ids, expert_ids,
                                write_tail, cap, cap_blocks);
  else
    write_layout_impl<NT, false>(sh, E, Blocks<false>(blk), numel, total, pre, share, nshare, sorted_ids,
                                 expert_ids, write_tail, cap, cap_blocks);
}

// The lanes of this wave whose id equals this lane's (ids in [0, 2^nbits), -1 = none): the valid lanes ANDed with,
// per id bit, the ballot of that bit or its complement -- nbits + 1 ballots instead of a compare against every lane.
__device__ __forceinline__ uint64_t same_id_lanes(int e, int nbits) {
  uint64_t m = __ballot(e >= 0);
  for (int b = 0; b < nbits; b++) {
    const int bit = (e >> b) & 1;
    const uint64_t B = __ballot(bit);
    m &= bit ? B : ~B;
  }
  return m;
}

__device__ __forceinline__ int id_bits(int E) { return E <= 1 ? 0 : 32 - __builtin_clz((unsigned)(E - 1)); }

// Stable placement of ids[base, base + NT) (LDS; -1 = not placed) at their experts' cursors: a lane's rank among
// the equal ids of lower lanes in its wave is the count of same-id lanes below it (same_id_lanes), the rows of
// earlier waves come from the per-wave counts. Advances the cursors; leaves wcnt zero.
template <int NT>
__device__ __forceinline__ void stable_round(TabLds<NT>& sh, const short* ids, int base, int n, int row0, int E,
                                             int* __restrict__ sorted_ids) {
  constexpr int NW = NT / WAVE;
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int t = base + tid;
  const int e = t < n ? ids[t] : -1;
  int rank = 0, cw = 0;
  if (base + wave * WAVE < n) {                                     // waves past the rows skip the ballots
    const uint64_t m = same_id_lanes(e, id_bits(E));
    rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    cw = __popcll(m);
  }
  if (e >= 0 && rank == cw - 1) sh.wcnt[wave][e] = (uint16_t)cw;     // the last of its expert in this wave
  lds_barrier();
  if (e >= 0) {
    // the rows of earlier waves: every wave's count read at once (independent LDS reads), those below this wave added
    int pos = sh.cursor[e] + rank;
    int c[NW];
#pragma unroll
    for (int w = 0; w < NW - 1; w++) c[w] = sh.wcnt[w][e];
#pragma unroll
    for (int w = 0; w < NW - 1; w++) pos += w < wave ? c[w] : 0;
    sorted_ids[pos] = row0 + t;
  }
  lds_barrier();
  for (int ex = tid; ex < E; ex += NT) {
    int add = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) {
      add += sh.wcnt[w][ex];
      sh.wcnt[w][ex] = 0;
    }
    sh.cursor[ex] += add;
  }
  lds_barrier();
}

// The table layout and stable placement from per-expert counts already in sh.cnt (a barrier after the counting;
// wcnt zero): scan, layout and the rounds. The counts stay in sh.cnt, so a second layout of the same rows (another
// block size) can follow with no recount.
template <int NT>
__device__ __forceinline__ void build_from_counts(TabLds<NT>& sh, const short* ids, int numel, int E, int blk,
                                                  int* __restrict__ sorted_ids, int* __restrict__ expert_ids,
                                                  int* __restrict__ ntpp, bool tail = true, long cap = -1,
                                                  long cap_blocks = -1) {
  const int total = padded_scan(sh, E, blk);
  if (threadIdx.x == 0) ntpp[0] = total;
  write_layout(sh, E, blk, numel, total, 0, 0, 1, sorted_ids, expert_ids, tail, cap, cap_blocks);
  for (int base = 0; base < numel; base += NT) stable_round(sh, ids, base, numel, 0, E, sorted_ids);
}

// Per-id row counts into sh.cnt (zero_counts and a barrier done by the caller); ends with a barrier.
template <int NT>
__device__ __forceinline__ void count_ids(TabLds<NT>& sh, const short* ids, int numel) {
  for (int t = threadIdx.x; t < numel; t += NT) {
    const int e = ids[t];
    if (e >= 0) atomicAdd(&sh.cnt[e], 1);
  }
  lds_barrier();
}

// The whole table build in one workgroup from ids in LDS (numel <= TAB_SMALL_MAX, -1 = skipped; zero_counts and a
// barrier done by the caller): histogram, scan, layout and the stable placement.
template <int NT>
__device__ __forceinline__ void build_tables(TabLds<NT>& sh, const short* ids, int numel, int E, int blk,
                                             int* __restrict__ sorted_ids, int* __restrict__ expert_ids,
                                             int* __restrict__ ntpp, bool tail = true, long cap = -1,
                                             long cap_blocks = -1) {
  count_ids(sh, ids, numel);
  build_from_counts(sh, ids, numel, E, blk, sorted_ids, expert_ids, ntpp, tail, cap, cap_blocks);
}

}  // namespace r9k
