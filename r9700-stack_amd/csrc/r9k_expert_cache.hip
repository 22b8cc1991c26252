// Device-side LRU expert cache for host-offloaded experts (MI355X, gfx950).
//
// Reference behaviour (moe/cache.py:1-20, 182-395; kernels/third_party/davetha/r4d_lru.hip:187-274 manage,
// :276-303 gather): every expert of a layer lives in mapped pinned host memory (the backing store); a VRAM arena of
// S slots holds a subset. Per forward, before the GEMMs:
//   manage  marks the experts routed this step; when more than max_distinct are routed it changes nothing else (the
//           step reads every non-resident expert through from host); otherwise it refreshes the stamps of the
//           resident routed experts, lists the non-resident routed experts in expert-id order (at most max_inserts),
//           and gives the r-th of them the slot with the r-th smallest key (stamp << 20 | slot) among the slots
//           whose expert is NOT routed this step, so nothing this step needs is evicted. table (expert -> slot or -1),
//           map_cold (expert -> itself when not resident, else -1), slot_expert and slot_stamp are rewritten in
//           place, and the (expert, slot) miss list is what gather copies host -> slot.
//   gather  copies up to six per-expert slabs of each listed expert from the host store into its slot.
// Both are device work with fixed pointers (no host sync), so a captured graph replays them.
//
// gfx950 design: manage is ONE workgroup of 16 waves. Routed flags, the slot mirror (expert, stamp, key) and the
// victim ranks sit in LDS (E <= 8192, S <= 1024: 8 KB + 20 KB). Victims are chosen by ranking each evictable slot's
// key against all S keys (each lane reads the keys as LDS broadcasts, 8 in flight), which equals taking the argmin
// nins times in a row: installing an expert makes its slot non-evictable and changes no other key. Nothing uses
// atomics, so the evolution is deterministic (identical on every rank that sees the same routing). gather reads the
// host store over PCIe with 16-byte loads; it is link-bound.
#include "r9k_common.h"
#include "r9k_tables.h"

#include <climits>

namespace {

using namespace r9k;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int MT_THREADS = 1024;            // manage: one workgroup, 16 waves
constexpr int MAX_E = 8192;                 // routed flags in LDS
constexpr int MAX_S = 1024;                 // slot mirror in LDS (and the slot index fits the key's low 20 bits)
constexpr int SLOT_BITS = 20;
constexpr int NWAVE = MT_THREADS / WAVE;

// exclusive prefix sum of one int per thread over the workgroup; *total = the sum of all
__device__ __forceinline__ int block_exscan(int v, int* sh, int* total) {
  const int t = threadIdx.x, lane = t % WAVE, w = t / WAVE;
  int x = v;
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) {
    const int y = __shfl_up(x, o, WAVE);
    if (lane >= o) x += y;
  }
  if (lane == WAVE - 1) sh[w] = x;
  __syncthreads();
  if (w == 0) {
    int s = lane < NWAVE ? sh[lane] : 0;
#pragma unroll
    for (int o = 1; o < NWAVE; o <<= 1) {
      const int y = __shfl_up(s, o, WAVE);
      if (lane >= o) s += y;
    }
    if (lane < NWAVE) sh[NWAVE + lane] = s;        // inclusive wave-total prefix
  }
  __syncthreads();
  const int before = w ? sh[NWAVE + w - 1] : 0;
  *total = sh[2 * NWAVE - 1];
  __syncthreads();                                  // sh is reused by the next call
  return before + x - v;
}

// LDS of one manage step: routed flags, the slot mirror (expert, stamp, eviction key), victims, misses, scan space.
struct ManageLds {
  long long st[MAX_S];
  long long key[MAX_S];
  int se[MAX_S];
  int vic[MAX_S];
  int miss[MAX_S];
  int sh[2 * NWAVE];
  uint8_t routed[MAX_E];
};

// One manage step by the whole (MT_THREADS) workgroup; with hot_ids / cold_ids given it also writes the two passes'
// routing ids (ids through the updated table / map_cold).
__device__ __forceinline__ void manage_step(
    ManageLds& L, const int* __restrict__ ids, int mk, int E, int S, int max_distinct, int max_inserts,
    int* __restrict__ table, int* __restrict__ map_cold, int* __restrict__ slot_expert,
    long long* __restrict__ slot_stamp, uint8_t* __restrict__ routed_out, long long* __restrict__ step,
    int* __restrict__ miss, int* __restrict__ n_miss, int* __restrict__ hot_ids, int* __restrict__ cold_ids) {
  uint8_t* s_routed = L.routed;
  int* s_se = L.se;
  long long* s_st = L.st;
  long long* s_key = L.key;
  int* s_vic = L.vic;
  int* s_miss = L.miss;
  int* sh = L.sh;
  const int t = threadIdx.x;

  const long long st = step[0] + 1;                 // every lane reads before lane 0 writes (barrier below)
  for (int e = t; e < E; e += MT_THREADS) s_routed[e] = 0;
  __syncthreads();
  if (t == 0) step[0] = st;
  for (int i = t; i < mk; i += MT_THREADS) {
    const int e = ids[i];
    if (e >= 0 && e < E) s_routed[e] = 1;           // same value from every writer
  }
  __syncthreads();

  // distinct routed experts; experts are taken in contiguous runs so the miss order below is expert-id order
  const int C = (E + MT_THREADS - 1) / MT_THREADS;
  const int lo = min(t * C, E), hi = min(lo + C, E);
  int cnt = 0;
  for (int e = lo; e < hi; e++) cnt += s_routed[e];
  int distinct = 0;
  block_exscan(cnt, sh, &distinct);

  int nact = 0;
  if (distinct <= max_distinct) {                   // else: a wide step reads through; nothing else changes
    for (int i = t; i < S; i += MT_THREADS) {
      s_se[i] = slot_expert[i];
      s_st[i] = slot_stamp[i];
    }
    __syncthreads();
    int local = 0;
    for (int e = lo; e < hi; e++) {
      if (!s_routed[e]) continue;
      const int s = table[e];
      if (s >= 0) s_st[s] = st;                      // a hit: distinct experts hold distinct slots
      else local++;
    }
    int total = 0;
    const int base = block_exscan(local, sh, &total);   // (its barriers also order the stamp refresh)
    const int nins = min(total, max_inserts);
    if (nins > 0) {
      int j = base;
      for (int e = lo; e < hi && j < nins; e++) {
        if (!s_routed[e] || table[e] >= 0) continue;
        s_miss[j++] = e;
      }
      int evictable = 0;
      for (int i = t; i < S; i += MT_THREADS) {
        const int se = s_se[i];
        const bool keep = se >= 0 && se < E && s_routed[se];
        s_key[i] = keep ? LLONG_MAX : (long long)(((unsigned long long)s_st[i] << SLOT_BITS) | (unsigned)i);
        evictable += !keep;
      }
      for (int r = t; r < nins; r += MT_THREADS) s_vic[r] = -1;
      int nev = 0;
      block_exscan(evictable, sh, &nev);            // barrier: keys and misses are in LDS
      nact = min(nins, nev);
      // rank of each evictable key among all keys (keys are unique: the slot index is in the low bits)
      for (int i = t; i < S; i += MT_THREADS) {
        const long long ki = s_key[i];
        if (ki == LLONG_MAX) continue;
        int rank = 0, jj = 0;
        for (; jj + 8 <= S; jj += 8) {
          long long k8[8];
#pragma unroll
          for (int u = 0; u < 8; u++) k8[u] = s_key[jj + u];
#pragma unroll
          for (int u = 0; u < 8; u++) rank += k8[u] < ki;
        }
        for (; jj < S; jj++) rank += s_key[jj] < ki;
        if (rank < nact) s_vic[rank] = i;
      }
      __syncthreads();
      // installs are independent: distinct victim slots, distinct (routed) new experts, evicted experts unrouted
      for (int r = t; r < nact; r += MT_THREADS) {
        const int e = s_miss[r], sl = s_vic[r];
        const int old = s_se[sl];
        if (old >= 0 && old < E) {
          table[old] = -1;
          map_cold[old] = old;
        }
        s_se[sl] = e;
        s_st[sl] = st;
        table[e] = sl;
        map_cold[e] = -1;
        miss[2 * r] = e;
        miss[2 * r + 1] = sl;
      }
      __syncthreads();
    }
    for (int i = t; i < S; i += MT_THREADS) {
      slot_expert[i] = s_se[i];
      slot_stamp[i] = s_st[i];
    }
  }
  for (int e = t; e < E; e += MT_THREADS) routed_out[e] = s_routed[e];
  if (t == 0) n_miss[0] = nact;
  if (hot_ids) {
    // the two passes' routing ids from the updated maps (the installs' global writes are ordered by the barrier)
    __syncthreads();
    for (int i = t; i < mk; i += MT_THREADS) {
      const int e = ids[i];
      const bool ok = e >= 0 && e < E;
      hot_ids[i] = ok ? table[e] : -1;
      cold_ids[i] = ok ? map_cold[e] : -1;
    }
  }
}

__global__ void __launch_bounds__(MT_THREADS) lru_manage_kernel(
    const int* __restrict__ ids, int mk, int E, int S, int max_distinct, int max_inserts, int* __restrict__ table,
    int* __restrict__ map_cold, int* __restrict__ slot_expert, long long* __restrict__ slot_stamp,
    uint8_t* __restrict__ routed_out, long long* __restrict__ step, int* __restrict__ miss, int* __restrict__ n_miss,
    int* __restrict__ hot_ids, int* __restrict__ cold_ids) {
  __shared__ ManageLds L;
  manage_step(L, ids, mk, E, S, max_distinct, max_inserts, table, map_cold, slot_expert, slot_stamp, routed_out, step,
              miss, n_miss, hot_ids, cold_ids);
}

// Manage, then the two passes' moe_align_block_size tables in the same workgroup (E <= TAB_MAX_E, mk <=
// TAB_SMALL_MAX): the routing ids mapped through the updated table (resident pass, ids = slots) and map_cold (host
// pass, ids = experts) go to LDS, and each table set is built by the routing kernels' single-workgroup builder (the
// canonical order, so the tables equal r9k_moe_align's over the same mapped ids). The manage LDS and the builder's
// share one union (the build starts after the last manage read). sorted_c = 0 skips the host pass's tables.
// cap < 0: this library's capacity; else sorted_ids hold cap entries and expert_ids cap_blocks.
__global__ void __launch_bounds__(MT_THREADS) lru_manage_tables_kernel(
    const int* __restrict__ ids, int mk, int E, int S, int max_distinct, int max_inserts, int* __restrict__ table,
    int* __restrict__ map_cold, int* __restrict__ slot_expert, long long* __restrict__ slot_stamp,
    uint8_t* __restrict__ routed_out, long long* __restrict__ step, int* __restrict__ miss, int* __restrict__ n_miss,
    int blk, long cap, long cap_blocks, int* __restrict__ sorted_h, int* __restrict__ eids_h,
    int* __restrict__ ntpp_h, int* __restrict__ sorted_c, int* __restrict__ eids_c, int* __restrict__ ntpp_c,
    int* __restrict__ hot_ids) {
  __shared__ union {
    ManageLds m;
    TabLds<MT_THREADS> t;
  } u;
  __shared__ short lids_h[TAB_SMALL_MAX], lids_c[TAB_SMALL_MAX];
  manage_step(u.m, ids, mk, E, S, max_distinct, max_inserts, table, map_cold, slot_expert, slot_stamp, routed_out,
              step, miss, n_miss, nullptr, nullptr);
  __syncthreads();                                   // the installs' global writes are ordered before the reads
  for (int i = threadIdx.x; i < mk; i += MT_THREADS) {
    const int e = ids[i];
    const bool ok = e >= 0 && e < E;
    const int h = ok ? table[e] : -1;
    lids_h[i] = (short)h;
    lids_c[i] = (short)(ok ? map_cold[e] : -1);
    if (hot_ids) hot_ids[i] = h;                      // the resident pass's slot ids, for token-major consumers
  }
  __syncthreads();                                   // every manage LDS read is done: the union turns over
  zero_counts(u.t, E);
  lds_barrier();
  build_tables(u.t, lids_h, mk, E, blk, sorted_h, eids_h, ntpp_h, true, cap, cap_blocks);
  if (sorted_c) {
    zero_counts(u.t, E);
    lds_barrier();
    build_tables(u.t, lids_c, mk, E, blk, sorted_c, eids_c, ntpp_c, true, cap, cap_blocks);
  }
}

struct Slabs {
  u32x4* d[6];
  const u32x4* s[6];
  long v[6];                                         // 16-byte units per expert
};

// grid (chunks, lanes): block (c, j) copies misses j, j + lanes, ...; each slab is split over the chunks' threads
__global__ void __launch_bounds__(256) lru_gather_kernel(Slabs sl, const int* __restrict__ miss,
                                                         const int* __restrict__ n_miss) {
  const int nm = n_miss[0];
  const long stride = (long)gridDim.x * blockDim.x, start = (long)blockIdx.x * blockDim.x + threadIdx.x;
  for (int j = blockIdx.y; j < nm; j += gridDim.y) {
    const long e = miss[2 * j], slot = miss[2 * j + 1];
#pragma unroll
    for (int b = 0; b < 6; b++) {
      const long v = sl.v[b];
      const u32x4* __restrict__ p = sl.s[b] + e * v;
      u32x4* __restrict__ q = sl.d[b] + slot * v;
      long i = start;
      for (; i + 3 * stride < v; i += 4 * stride) {  // four 16-byte host reads in flight per lane
        const u32x4 a0 = p[i], a1 = p[i + stride], a2 = p[i + 2 * stride], a3 = p[i + 3 * stride];
        q[i] = a0;
        q[i + stride] = a1;
        q[i + 2 * stride] = a2;
        q[i + 3 * stride] = a3;
      }
      for (; i < v; i += stride) q[i] = p[i];
    }
  }
}

// hot[i] = table[ids[i]], cold[i] = map_cold[ids[i]] (-1 for ids outside [0, E)): the two passes' routing ids
__global__ void __launch_bounds__(256) lru_map_ids_kernel(const int* __restrict__ ids, int mk, int E,
                                                          const int* __restrict__ table,
                                                          const int* __restrict__ map_cold, int* __restrict__ hot,
                                                          int* __restrict__ cold) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= mk) return;
  const int e = ids[i];
  const bool ok = e >= 0 && e < E;
  hot[i] = ok ? table[e] : -1;
  cold[i] = ok ? map_cold[e] : -1;
}

// Cold staging map (one workgroup): the experts routed this step that are not resident, numbered in ascending expert
// order -- stage_map[e] = that number (-1 for every other expert), the miss list (e, number) the gather copies host ->
// staging area, and their count. The numbering is a prefix sum of the cold flags, chunk by chunk over the experts
// (a wave-inclusive scan, then the waves' totals), so it is deterministic.
__global__ void __launch_bounds__(MT_THREADS) lru_stage_map_kernel(const int* __restrict__ ids, int mk, int E,
                                                                   const int* __restrict__ table, int cap,
                                                                   int* __restrict__ stage_map,
                                                                   int* __restrict__ miss, int* __restrict__ n_miss) {
  __shared__ uint8_t routed[MAX_E];
  __shared__ int wsum[NWAVE];
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  for (int e = tid; e < E; e += MT_THREADS) routed[e] = 0;
  __syncthreads();
  for (int i = tid; i < mk; i += MT_THREADS) {
    const int e = ids[i];
    if (e >= 0 && e < E) routed[e] = 1;                       // plain stores of the same value: no atomics needed
  }
  __syncthreads();
  int base = 0;
  for (int e0 = 0; e0 < E; e0 += MT_THREADS) {
    const int e = e0 + tid;
    const int cold = (e < E && routed[e] && table[e] < 0) ? 1 : 0;
    int x = cold;
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
      const int y = __shfl_up(x, o, WAVE);
      if (lane >= o) x += y;
    }
    if (lane == WAVE - 1) wsum[wave] = x;
    __syncthreads();
    int wb = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < NWAVE; w++) {
      wb += w < wave ? wsum[w] : 0;
      tot += wsum[w];
    }
    if (e < E) {
      const int idx = base + wb + x - cold;                   // exclusive rank among the cold experts
      const bool staged = cold && idx < cap;
      stage_map[e] = staged ? idx : -1;
      if (staged) {
        miss[2 * idx] = e;
        miss[2 * idx + 1] = idx;
      }
    }
    base += tot;
    __syncthreads();
  }
  if (tid == 0) n_miss[0] = base < cap ? base : cap;
}

}  // namespace

extern "C" int r9k_lru_manage_map(long ids, int mk, int E, int S, int max_distinct, int max_inserts, long table,
                                  long map_cold, long slot_expert, long slot_stamp, long routed, long step, long miss,
                                  long n_miss, long hot, long cold, long stream) {
  if (E <= 0 || E > MAX_E || S <= 0 || S > MAX_S || S > E || mk < 0) return -1;
  if (max_inserts < 0 || max_inserts > S) return -2;
  if ((mk && !ids) || !table || !map_cold || !slot_expert || !slot_stamp || !routed || !step || !miss || !n_miss)
    return -3;
  if ((slot_stamp | step) & 7) return -4;
  if ((hot != 0) != (cold != 0)) return -3;
  hipLaunchKernelGGL(lru_manage_kernel, dim3(1), dim3(MT_THREADS), 0, (hipStream_t)stream, (const int*)ids, mk, E,
                     S, max_distinct, max_inserts, (int*)table, (int*)map_cold, (int*)slot_expert,
                     (long long*)slot_stamp, (uint8_t*)routed, (long long*)step, (int*)miss, (int*)n_miss,
                     (int*)hot, (int*)cold);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

namespace {

int manage_tables_launch(long ids, int mk, int E, int S, int max_distinct, int max_inserts, long table, long map_cold,
                         long slot_expert, long slot_stamp, long routed, long step, long miss, long n_miss, int blk,
                         long cap, long cap_blocks, long sorted_h, long eids_h, long ntpp_h, long sorted_c,
                         long eids_c, long ntpp_c, long hot_ids, long stream) {
  if (E <= 0 || E > MAX_E || S <= 0 || S > MAX_S || S > E || mk < 0 || blk <= 0) return -1;
  if (max_inserts < 0 || max_inserts > S) return -2;
  if ((mk && !ids) || !table || !map_cold || !slot_expert || !slot_stamp || !routed || !step || !miss || !n_miss ||
      !sorted_h || !eids_h || !ntpp_h || (sorted_c && (!eids_c || !ntpp_c)))
    return -3;
  if ((slot_stamp | step) & 7) return -4;
  if (E > TAB_MAX_E || mk > TAB_SMALL_MAX) return 2;          // one workgroup's tables: the composed path serves it
  hipLaunchKernelGGL(lru_manage_tables_kernel, dim3(1), dim3(MT_THREADS), 0, (hipStream_t)stream, (const int*)ids, mk,
                     E, S, max_distinct, max_inserts, (int*)table, (int*)map_cold, (int*)slot_expert,
                     (long long*)slot_stamp, (uint8_t*)routed, (long long*)step, (int*)miss, (int*)n_miss, blk, cap,
                     cap_blocks, (int*)sorted_h, (int*)eids_h, (int*)ntpp_h, (int*)sorted_c, (int*)eids_c,
                     (int*)ntpp_c, (int*)hot_ids);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

}  // namespace

// The manage step and both passes' routing tables in one launch, tables of this library's capacity (sorted
// capacity(mk, E, blk) entries, expert ids capacity / blk); sorted_c = 0 skips the host pass; hot_ids (int32 [mk],
// 0 = not wanted) receives each routed row's slot (-1 not resident), as r9k_lru_manage_map's `hot`. 2 when not
// served (E > 1024 or mk > 4096; nothing launched: manage_map + two aligns give the same result).
extern "C" int r9k_lru_manage_tables(long ids, int mk, int E, int S, int max_distinct, int max_inserts, long table,
                                     long map_cold, long slot_expert, long slot_stamp, long routed, long step,
                                     long miss, long n_miss, int blk, long sorted_h, long eids_h, long ntpp_h,
                                     long sorted_c, long eids_c, long ntpp_c, long hot_ids, long stream) {
  return manage_tables_launch(ids, mk, E, S, max_distinct, max_inserts, table, map_cold, slot_expert, slot_stamp,
                              routed, step, miss, n_miss, blk, -1, -1, sorted_h, eids_h, ntpp_h, sorted_c, eids_c,
                              ntpp_c, hot_ids, stream);
}

// The reference's one-launch manage + both moe_align_block_size outputs with its buffer lengths: sorted_* hold L
// entries and eids_* NB (L must cover the padded total's bound: min(mk * bs, mk + E (bs - 1)) rows while mk < E,
// else mk + E (bs - 1); NB >= ceil(L / bs)). The tails past the padded totals are written (numel / -1) up to L / NB.
extern "C" int r4d_lru_fused(long ids, int mk, int E, int S, int max_distinct, int max_inserts, long table,
                             long map_cold, long slot_expert, long slot_stamp, long routed, long step, long miss,
                             long n_miss, int bs, int L, int NB, long sorted_hot, long eids_hot, long npad_hot,
                             long sorted_cold, long eids_cold, long npad_cold, long stream) {
  if (bs <= 0 || mk < 0 || L <= 0 || NB <= 0) return -1;
  const long lo = (long)mk + (long)E * (bs - 1);
  const long need = mk < E ? (lo < (long)mk * bs ? lo : (long)mk * bs) : lo;
  if (L < need || (long)NB * bs < L) return -1;
  if (!sorted_cold) return -3;
  return manage_tables_launch(ids, mk, E, S, max_distinct, max_inserts, table, map_cold, slot_expert, slot_stamp,
                              routed, step, miss, n_miss, bs, L, NB, sorted_hot, eids_hot, npad_hot, sorted_cold,
                              eids_cold, npad_cold, 0, stream);
}

extern "C" int r4d_lru_manage(long ids, int mk, int E, int S, int max_distinct, int max_inserts, long table,
                              long map_cold, long slot_expert, long slot_stamp, long routed, long step, long miss,
                              long n_miss, long stream) {
  return r9k_lru_manage_map(ids, mk, E, S, max_distinct, max_inserts, table, map_cold, slot_expert, slot_stamp,
                            routed, step, miss, n_miss, 0, 0, stream);
}

extern "C" int r4d_lru_gather(long d0, long s0, long b0, long d1, long s1, long b1, long d2, long s2, long b2,
                              long d3, long s3, long b3, long d4, long s4, long b4, long d5, long s5, long b5,
                              long miss, long n_miss, int chunks, int lanes, long stream) {
  if (chunks <= 0 || lanes <= 0 || chunks > 65535 || lanes > 65535) return -2;
  if (!miss || !n_miss) return -3;
  const long d[6] = {d0, d1, d2, d3, d4, d5}, s[6] = {s0, s1, s2, s3, s4, s5}, b[6] = {b0, b1, b2, b3, b4, b5};
  Slabs sl;
  for (int i = 0; i < 6; i++) {
    if (b[i] < 0 || (b[i] % 16) || ((d[i] | s[i]) & 15)) return -4;
    if (b[i] && (!d[i] || !s[i])) return -3;
    sl.d[i] = (u32x4*)d[i];
    sl.s[i] = (const u32x4*)s[i];
    sl.v[i] = b[i] / 16;
  }
  hipLaunchKernelGGL(lru_gather_kernel, dim3(chunks, lanes), dim3(256), 0, (hipStream_t)stream, sl,
                     (const int*)miss, (const int*)n_miss);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

extern "C" int r9k_lru_map_ids(long ids, int mk, int E, long table, long map_cold, long hot, long cold,
                               long stream) {
  if (mk < 0 || E <= 0) return -1;
  if (mk == 0) return 0;
  if (!ids || !table || !map_cold || !hot || !cold) return -3;
  hipLaunchKernelGGL(lru_map_ids_kernel, dim3((mk + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     (const int*)ids, mk, E, (const int*)table, (const int*)map_cold, (int*)hot, (int*)cold);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

// No counterpart as one entry in the reference: its opt-in cold staging (R9K_STAGE_COLD=1, moe/cache.py:358-393)
// builds the staging map with torch ops. ids int32 [mk] (this step's routed experts), table int32 [E] (expert ->
// slot, -1 = host) after this step's manage -> stage_map int32 [E] (cold expert -> its staging index in ascending
// expert order, else -1), miss int32 [cap][2] ((expert, staging index) pairs for r4d_lru_gather), n_miss int32 [1]
// (their count, at most cap). A cold expert numbered cap or more is left unstaged (-1): with every slot of the arena
// holding an expert, at most E - S are cold, so cap = E - S stages them all. 0, -1 bad sizes, -3 null, -6 launch.
extern "C" int r9k_lru_stage_map(long ids, int mk, int E, long table, int cap, long stage_map, long miss,
                                 long n_miss, long stream) {
  if (E <= 0 || E > MAX_E || mk < 0 || cap < 0) return -1;
  if ((mk && !ids) || !table || !stage_map || (cap && !miss) || !n_miss) return -3;
  hipLaunchKernelGGL(lru_stage_map_kernel, dim3(1), dim3(MT_THREADS), 0, (hipStream_t)stream, (const int*)ids, mk,
                     E, (const int*)table, cap, (int*)stage_map, (int*)miss, (int*)n_miss);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

// Mapped pinned host memory for the backing store: hipHostMalloc(Mapped | Portable); the device address is the host
// address (checked), so one pointer serves the host-side copies and the kernels. Held until r9k_host_free.
extern "C" long r9k_host_alloc(long bytes) {
  if (bytes <= 0) return 0;
  void* h = nullptr;
  if (hipHostMalloc(&h, (size_t)bytes, hipHostMallocMapped | hipHostMallocPortable) != hipSuccess || !h) return 0;
  void* d = nullptr;
  if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess || d != h) {
    (void)hipHostFree(h);
    return 0;
  }
  return (long)h;
}

extern "C" int r9k_host_free(long p) {
  if (!p) return 0;
  return hipHostFree((void*)p) == hipSuccess ? 0 : -6;
}
