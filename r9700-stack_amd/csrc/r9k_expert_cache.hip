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
// The one-launch manage + tables (E <= 1024) also keeps table and map_cold in LDS: every global value the step reads
// (ids, step, table, map_cold, slot state, the activation rows it quantises) is requested at once at the start, so a
// decode step waits on one memory round trip instead of one per phase, and the tables are built from the LDS copies.
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

// LDS of one manage step: routed flags, the slot mirror (expert, stamp, eviction key), victims, misses, scan space;
// with TAB also the LDS copies of table and map_cold (E <= TAB_MAX_E).
template <bool TAB>
struct ManageLds {
  static constexpr int NE = TAB ? TAB_MAX_E : MAX_E;
  long long st[MAX_S];
  long long key[MAX_S];
  int se[MAX_S];
  int vic[MAX_S];
  int miss[MAX_S];
  int sh[2 * NWAVE];
  int tab[TAB ? TAB_MAX_E : 1];
  int cold[TAB ? TAB_MAX_E : 1];
  uint8_t routed[NE];
};

constexpr int QR = 8;                  // 16-byte chunks a lane of the folded activation quant: hidden <= 4096
constexpr int QUANT_MAX_ROWS = 64;     // activation rows the manage launch quantises (one wave a row, 4 a wave)

// The activation rows a manage + tables launch quantises (x == nullptr: none): quant_row_wave's bytes.
struct RowQuant {
  const uint16_t* x;
  long ldx;
  int H, T;
  uint8_t* xq;
  float* xs;
};

// The first half of a manage step: the step counter, the routed flags and (TAB) the LDS copies. Returns the new step
// stamp; ends with a barrier. TAB (E <= TAB_MAX_E, mk <= TAB_SMALL_MAX): every global read is issued at once --
// ids, table and map_cold (kept in LDS for the rest of the step), the slot mirror and the first activation row of
// wave 1, 2, ... (q.x rows 0, 1, ..., left in xv) -- and s_ids receives the routed ids (-1 outside [0, E)) for the
// caller's tables.
template <bool TAB>
__device__ __forceinline__ long long manage_prologue(
    ManageLds<TAB>& L, const int* __restrict__ ids, int mk, int E, int S, const int* __restrict__ table,
    const int* __restrict__ map_cold, const int* __restrict__ slot_expert, const long long* __restrict__ slot_stamp,
    long long* __restrict__ step, short* __restrict__ s_ids = nullptr, const RowQuant* q = nullptr,
    uint4 (*xv)[QR] = nullptr) {
  uint8_t* s_routed = L.routed;
  const int t = threadIdx.x;
  const long long st = step[0] + 1;                 // every lane reads before lane 0 writes (barrier below)
  if constexpr (TAB) {
    constexpr int IR = TAB_SMALL_MAX / MT_THREADS;
    int idr[IR];
#pragma unroll
    for (int u = 0; u < IR; u++) idr[u] = t + u * MT_THREADS < mk ? ids[t + u * MT_THREADS] : -1;
    const int tv = t < E ? table[t] : -1, cv = t < E ? map_cold[t] : -1;
    const int sev = t < S ? slot_expert[t] : -1;
    const long long stv = t < S ? slot_stamp[t] : 0;
    const int wave = t / WAVE;
    if (q->x && wave >= 1 && wave - 1 < q->T)
      quant_row_load<QR>(q->x + (size_t)(wave - 1) * q->ldx, q->H, t % WAVE, *xv);
    if (t < E) s_routed[t] = 0;
    __syncthreads();
    if (t == 0) step[0] = st;
#pragma unroll
    for (int u = 0; u < IR; u++) {
      const int i = t + u * MT_THREADS, e = idr[u];
      const bool ok = e >= 0 && e < E;
      if (i < mk) s_ids[i] = (short)(ok ? e : -1);
      if (ok) s_routed[e] = 1;                      // same value from every writer
    }
    if (t < E) {
      L.tab[t] = tv;
      L.cold[t] = cv;
    }
    if (t < S) {
      L.se[t] = sev;
      L.st[t] = stv;
    }
  } else {
    for (int e = t; e < E; e += MT_THREADS) s_routed[e] = 0;
    __syncthreads();
    if (t == 0) step[0] = st;
    for (int i = t; i < mk; i += MT_THREADS) {
      const int e = ids[i];
      if (e >= 0 && e < E) s_routed[e] = 1;         // same value from every writer
    }
  }
  __syncthreads();
  return st;
}

// The rest of a manage step by the whole (MT_THREADS) workgroup, after manage_prologue; with hot_ids / cold_ids given
// it also writes the two passes' routing ids (ids through the updated table / map_cold). TAB: table / map_cold are
// read and updated in LDS (installs also write them to global).
template <bool TAB>
__device__ __forceinline__ void manage_body(
    ManageLds<TAB>& L, long long st, int mk, const int* __restrict__ ids, int E, int S, int max_distinct,
    int max_inserts, int* __restrict__ table, int* __restrict__ map_cold, int* __restrict__ slot_expert,
    long long* __restrict__ slot_stamp, uint8_t* __restrict__ routed_out, int* __restrict__ miss,
    int* __restrict__ n_miss, int* __restrict__ hot_ids, int* __restrict__ cold_ids) {
  uint8_t* s_routed = L.routed;
  int* s_se = L.se;
  long long* s_st = L.st;
  long long* s_key = L.key;
  int* s_vic = L.vic;
  int* s_miss = L.miss;
  int* sh = L.sh;
  const int t = threadIdx.x;
  auto tab_of = [&](int e) { return TAB ? L.tab[e] : table[e]; };

  // distinct routed experts; experts are taken in contiguous runs so the miss order below is expert-id order
  const int C = (E + MT_THREADS - 1) / MT_THREADS;
  const int lo = min(t * C, E), hi = min(lo + C, E);
  int cnt = 0;
  for (int e = lo; e < hi; e++) cnt += s_routed[e];
  int distinct = 0;
  block_exscan(cnt, sh, &distinct);

  int nact = 0;
  if (distinct <= max_distinct) {                   // else: a wide step reads through; nothing else changes
    if (!TAB) {                                     // (TAB: the slot mirror came in with the prologue)
      for (int i = t; i < S; i += MT_THREADS) {
        s_se[i] = slot_expert[i];
        s_st[i] = slot_stamp[i];
      }
      __syncthreads();
    }
    int local = 0;
    for (int e = lo; e < hi; e++) {
      if (!s_routed[e]) continue;
      const int s = tab_of(e);
      if (s >= 0) s_st[s] = st;                      // a hit: distinct experts hold distinct slots
      else local++;
    }
    int total = 0;
    const int base = block_exscan(local, sh, &total);   // (its barriers also order the stamp refresh)
    const int nins = min(total, max_inserts);
    if (nins > 0) {
      int j = base;
      for (int e = lo; e < hi && j < nins; e++) {
        if (!s_routed[e] || tab_of(e) >= 0) continue;
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
          if (TAB) {
            L.tab[old] = -1;
            L.cold[old] = old;
          }
        }
        s_se[sl] = e;
        s_st[sl] = st;
        table[e] = sl;
        map_cold[e] = -1;
        if (TAB) {
          L.tab[e] = sl;
          L.cold[e] = -1;
        }
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
  if (!TAB && hot_ids) {
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
  __shared__ ManageLds<false> L;
  const long long st = manage_prologue<false>(L, ids, mk, E, S, table, map_cold, slot_expert, slot_stamp, step);
  manage_body<false>(L, st, mk, ids, E, S, max_distinct, max_inserts, table, map_cold, slot_expert, slot_stamp,
                     routed_out, miss, n_miss, hot_ids, cold_ids);
}

// Table capacity as write_layout's: cap < 0 means this library's, ceil((mk + E (blk - 1)) / blk) * blk entries.
__device__ __forceinline__ void table_capacity(int mk, int E, int blk, long& cap, long& cap_blocks) {
  if (cap < 0) {
    cap = ((long)mk + (long)E * (blk - 1) + blk - 1) / blk * blk;
    cap_blocks = cap / blk;
  }
}

// An entry bound no table of mk routed rows reaches: a pass's padded total is the sum over its distinct ids of their
// rows rounded up to the block, at most mk + min(mk, E) (blk - 1). Entries from `bound` on (and blocks from bound /
// blk on) are capacity tail whatever the routing, so they can be written before the tables are known.
__device__ __forceinline__ long tail_bound(int mk, int E, int blk, long cap) {
  const long b = ((long)mk + (long)min(mk, E) * (blk - 1) + blk - 1) / blk * blk;
  return b < cap ? b : cap;
}

// The capacity tail from `from` on (entries numel, blocks -1), by the threads [t0, t0 + nt) of the workgroup.
__device__ __forceinline__ void write_tail(int* __restrict__ sorted_ids, int* __restrict__ expert_ids, int numel,
                                           int blk, long from, long cap, long cap_blocks, int t0, int nt) {
  const int t = threadIdx.x - t0;
  for (long i = from + t; i < cap; i += nt) sorted_ids[i] = numel;
  for (long b = from / blk + t; b < cap_blocks; b += nt) expert_ids[b] = -1;
}

// One pass's moe_align_block_size tables of up to WAVE routed rows by one wave (lane i holds row i's id, -1 =
// skipped), with ballots instead of the workgroup builder: a lane's rank among the equal ids of lower lanes
// (same_id_lanes) places its row, the expert's first lane its padding entries and block ids, and the expert's offset
// is the sum of the padded counts of the smaller ids present (a scalar walk over the first lanes). The tail is written
// up to `bound` (tail_bound: the rest is the caller's). The same tables as build_tables: experts ascending, rows
// ascending within an expert.
__device__ __forceinline__ void wave_tables(int id, int mk, int E, int blk, int* __restrict__ sorted_ids,
                                            int* __restrict__ expert_ids, int* __restrict__ ntpp, long bound,
                                            long cap_blocks) {
  const int lane = threadIdx.x % WAVE;
  const uint64_t same = same_id_lanes(id, id_bits(E));
  const uint64_t below = same & ((1ull << lane) - 1ull);
  const bool first = id >= 0 && below == 0;
  const int cnt = __popcll(same);
  const int up = first ? (cnt + blk - 1) / blk * blk : 0;
  int total = 0, offs = 0;
  for (uint64_t fm = __ballot(first); fm; fm &= fm - 1ull) {
    const int j = __builtin_ctzll(fm);
    const int idj = __builtin_amdgcn_readlane(id, j), uj = __builtin_amdgcn_readlane(up, j);
    offs += idj < id ? uj : 0;
    total += uj;
  }
  if (id >= 0) sorted_ids[offs + __popcll(below)] = lane;
  if (first) {
    for (int i = offs + cnt; i < offs + up; i++) sorted_ids[i] = mk;
    for (int b = offs / blk; b < (offs + up) / blk; b++) expert_ids[b] = id;
  }
  if (lane == 0) ntpp[0] = total;
  const long bb = bound / blk < cap_blocks ? bound / blk : cap_blocks;
  for (long i = total + lane; i < bound; i += WAVE) sorted_ids[i] = mk;
  for (long b = total / blk + lane; b < bb; b += WAVE) expert_ids[b] = -1;
}

// The all-resident decode step of the manage + tables launch, by wave 0 right after manage_prologue<true>: at most
// WAVE routed rows, every routed expert resident and at most max_distinct of them. Nothing is installed, so the step
// refreshes the routed slots' stamps and writes n_miss = 0, hot_ids and both passes' tables (wave_tables, over the ids
// mapped through the LDS copies of table / map_cold, tails up to tail_bound) -- what manage_body + build_tables write
// (routed_out and the tails past tail_bound are the other waves'). False (nothing written) for any other step.
__device__ __forceinline__ bool all_hit_step(
    const ManageLds<true>& L, const short* __restrict__ s_ids, long long st, int mk, int E, int max_distinct,
    long long* __restrict__ slot_stamp, int* __restrict__ n_miss, int blk, long bound, long cap_blocks,
    int* __restrict__ sorted_h, int* __restrict__ eids_h, int* __restrict__ ntpp_h, int* __restrict__ sorted_c,
    int* __restrict__ eids_c, int* __restrict__ ntpp_c, int* __restrict__ hot_ids) {
  if (mk > WAVE) return false;
  const int lane = threadIdx.x % WAVE;
  const int e = lane < mk ? s_ids[lane] : -1;
  const int h = e >= 0 ? L.tab[e] : -1;
  if (__ballot(e >= 0 && h < 0)) return false;                   // a miss: the full step installs
  const uint64_t same = same_id_lanes(e, id_bits(E));
  const bool first = e >= 0 && (same & ((1ull << lane) - 1ull)) == 0;
  if (__popcll(__ballot(first)) > max_distinct) return false;     // a wide step reads through: the full step
  if (first) slot_stamp[h] = st;                                  // distinct experts hold distinct slots
  if (hot_ids && lane < mk) hot_ids[lane] = h;
  if (lane == 0) n_miss[0] = 0;
  wave_tables(h, mk, E, blk, sorted_h, eids_h, ntpp_h, bound, cap_blocks);
  if (sorted_c) wave_tables(e >= 0 ? L.cold[e] : -1, mk, E, blk, sorted_c, eids_c, ntpp_c, bound, cap_blocks);
  return true;
}

// LDS of the manage + tables launch: the manage step's and the table builder's share one union (the build starts
// after the last manage read).
union TablesLds {
  ManageLds<true> m;
  TabLds<MT_THREADS> t;
};

// The full manage step and both passes' tables (any step manage_tables serves): the routing ids mapped through the
// updated table (resident pass, ids = slots) and map_cold (host pass, ids = experts) go to LDS, and each table set is
// built by the routing kernels' single-workgroup builder (the canonical order, so the tables equal r9k_moe_align's
// over the same mapped ids). s_ids holds the routed ids from manage_prologue<true> and is overwritten.
__device__ __forceinline__ void manage_tables_full(
    TablesLds& u, short* __restrict__ lids_h, short* __restrict__ s_ids, long long st, const int* __restrict__ ids,
    int mk, int E, int S, int max_distinct, int max_inserts, int* __restrict__ table, int* __restrict__ map_cold,
    int* __restrict__ slot_expert, long long* __restrict__ slot_stamp, uint8_t* __restrict__ routed_out,
    int* __restrict__ miss, int* __restrict__ n_miss, int blk, long cap, long cap_blocks, int* __restrict__ sorted_h,
    int* __restrict__ eids_h, int* __restrict__ ntpp_h, int* __restrict__ sorted_c, int* __restrict__ eids_c,
    int* __restrict__ ntpp_c, int* __restrict__ hot_ids) {
  manage_body<true>(u.m, st, mk, ids, E, S, max_distinct, max_inserts, table, map_cold, slot_expert, slot_stamp,
                    routed_out, miss, n_miss, nullptr, nullptr);
  __syncthreads();                                   // the LDS copies hold the updated maps
  for (int i = threadIdx.x; i < mk; i += MT_THREADS) {
    const int e = s_ids[i];                          // the routed id (-1 outside [0, E)), from the prologue
    const int h = e >= 0 ? u.m.tab[e] : -1;
    lids_h[i] = (short)h;
    s_ids[i] = (short)(e >= 0 ? u.m.cold[e] : -1);
    if (hot_ids) hot_ids[i] = h;                      // the resident pass's slot ids, for token-major consumers
  }
  __syncthreads();                                   // every manage LDS read is done: the union turns over
  zero_counts(u.t, E);
  lds_barrier();
  build_tables(u.t, lids_h, mk, E, blk, sorted_h, eids_h, ntpp_h, true, cap, cap_blocks);
  if (sorted_c) {
    zero_counts(u.t, E);
    lds_barrier();
    build_tables(u.t, s_ids, mk, E, blk, sorted_c, eids_c, ntpp_c, true, cap, cap_blocks);
  }
}

// The q.T activation rows of a manage + tables launch (q.x == nullptr: none) on waves 1 .. NWAVE - 1 (wave 0 runs
// the tables meanwhile): each wave's first row from the chunks the prologue loaded into xv, the rest read here, one
// wave a row (quant_row_wave's bytes).
__device__ __forceinline__ void quant_rows(const RowQuant& q, const uint4 (&xv)[QR]) {
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  if (!q.x || wave == 0) return;
  if (wave - 1 < q.T) quant_row_finish<QR>(xv, q.H, q.xq + (size_t)(wave - 1) * q.H, q.xs + wave - 1, lane);
  for (int r = wave - 1 + (NWAVE - 1); r < q.T; r += NWAVE - 1)
    quant_row_wave<QR>(q.x + (size_t)r * q.ldx, q.H, q.xq + (size_t)r * q.H, q.xs + r, lane);
}

// Manage, then the two passes' moe_align_block_size tables in the same workgroup (E <= TAB_MAX_E, mk <=
// TAB_SMALL_MAX). After the prologue, wave 0 runs all_hit_step (the all-resident decode steps) while the other waves
// write what both paths write alike -- routed_out and the table tails past tail_bound -- and quantise the activation
// rows; one barrier publishes wave 0's answer, and every other step runs manage_tables_full (which writes the state
// and tables again, the same values where they overlap). sorted_c = 0 skips the host pass's tables. cap < 0: this
// library's capacity; else sorted_ids hold cap entries and expert_ids cap_blocks. With q.x the workgroup also
// quantises the q.T <= QUANT_MAX_ROWS activation rows (quant_row_wave's bytes): one wave a row, the first row of
// each wave requested with the manage step's reads.
__global__ void __launch_bounds__(MT_THREADS) lru_manage_tables_kernel(
    const int* __restrict__ ids, int mk, int E, int S, int max_distinct, int max_inserts, int* __restrict__ table,
    int* __restrict__ map_cold, int* __restrict__ slot_expert, long long* __restrict__ slot_stamp,
    uint8_t* __restrict__ routed_out, long long* __restrict__ step, int* __restrict__ miss, int* __restrict__ n_miss,
    int blk, long cap, long cap_blocks, int* __restrict__ sorted_h, int* __restrict__ eids_h,
    int* __restrict__ ntpp_h, int* __restrict__ sorted_c, int* __restrict__ eids_c, int* __restrict__ ntpp_c,
    int* __restrict__ hot_ids, RowQuant q) {
  __shared__ TablesLds u;
  __shared__ short lids_h[TAB_SMALL_MAX], lids_c[TAB_SMALL_MAX];
  __shared__ int s_fast;
  uint4 xv[QR];
  const long long st = manage_prologue<true>(u.m, ids, mk, E, S, table, map_cold, slot_expert, slot_stamp, step,
                                             lids_c, &q, &xv);
  table_capacity(mk, E, blk, cap, cap_blocks);
  const long bound = tail_bound(mk, E, blk, cap);
  if (threadIdx.x < WAVE) {
    const bool fast = all_hit_step(u.m, lids_c, st, mk, E, max_distinct, slot_stamp, n_miss, blk, bound, cap_blocks,
                                   sorted_h, eids_h, ntpp_h, sorted_c, eids_c, ntpp_c, hot_ids);
    if (threadIdx.x == 0) s_fast = fast;
  } else {
    for (int e = threadIdx.x - WAVE; e < E; e += MT_THREADS - WAVE) routed_out[e] = u.m.routed[e];
    write_tail(sorted_h, eids_h, mk, blk, bound, cap, cap_blocks, WAVE, MT_THREADS - WAVE);
    if (sorted_c) write_tail(sorted_c, eids_c, mk, blk, bound, cap, cap_blocks, WAVE, MT_THREADS - WAVE);
    quant_rows(q, xv);
  }
  __syncthreads();
  if (!s_fast)
    manage_tables_full(u, lids_h, lids_c, st, ids, mk, E, S, max_distinct, max_inserts, table, map_cold, slot_expert,
                       slot_stamp, routed_out, miss, n_miss, blk, cap, cap_blocks, sorted_h, eids_h, ntpp_h, sorted_c,
                       eids_c, ntpp_c, hot_ids);
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
                         long eids_c, long ntpp_c, long hot_ids, const RowQuant& q, long stream) {
  if (E <= 0 || E > MAX_E || S <= 0 || S > MAX_S || S > E || mk < 0 || blk <= 0) return -1;
  if (max_inserts < 0 || max_inserts > S) return -2;
  if ((mk && !ids) || !table || !map_cold || !slot_expert || !slot_stamp || !routed || !step || !miss || !n_miss ||
      !sorted_h || !eids_h || !ntpp_h || (sorted_c && (!eids_c || !ntpp_c)))
    return -3;
  if ((slot_stamp | step) & 7) return -4;
  if (q.x && (q.T < 1 || q.T > QUANT_MAX_ROWS || q.H < 8 || q.H % 8 || q.H > 512 * QR || q.ldx < q.H || q.ldx % 8 ||
              (reinterpret_cast<uintptr_t>(q.x) & 15) || (reinterpret_cast<uintptr_t>(q.xq) & 7) || !q.xq || !q.xs))
    return -7;
  if (E > TAB_MAX_E || mk > TAB_SMALL_MAX) return 2;          // one workgroup's tables: the composed path serves it
  hipLaunchKernelGGL(lru_manage_tables_kernel, dim3(1), dim3(MT_THREADS), 0, (hipStream_t)stream, (const int*)ids, mk,
                     E, S, max_distinct, max_inserts, (int*)table, (int*)map_cold, (int*)slot_expert,
                     (long long*)slot_stamp, (uint8_t*)routed, (long long*)step, (int*)miss, (int*)n_miss, blk, cap,
                     cap_blocks, (int*)sorted_h, (int*)eids_h, (int*)ntpp_h, (int*)sorted_c, (int*)eids_c,
                     (int*)ntpp_c, (int*)hot_ids, q);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

}  // namespace

// The manage step and both passes' routing tables in one launch, tables of this library's capacity (sorted
// capacity(mk, E, blk) entries, expert ids capacity / blk); sorted_c = 0 skips the host pass; hot_ids (int32 [mk],
// 0 = not wanted) receives each routed row's slot (-1 not resident), as r9k_lru_manage_map's `hot`. x != 0: the
// launch also writes xq e4m3 [T][H] and xs fp32 [T], the per-row fp8 quant of the T <= 64 bf16 rows of x (row stride
// ldx), r9k_quant_rows_fp8's bytes. 2 when not served (E > 1024 or mk > 4096; nothing launched, the rows not
// quantised: manage_map + two aligns give the same tables); -7 quant arguments out of range.
extern "C" int r9k_lru_manage_tables(long ids, int mk, int E, int S, int max_distinct, int max_inserts, long table,
                                     long map_cold, long slot_expert, long slot_stamp, long routed, long step,
                                     long miss, long n_miss, int blk, long sorted_h, long eids_h, long ntpp_h,
                                     long sorted_c, long eids_c, long ntpp_c, long hot_ids, long x, long ldx, int H,
                                     int T, long xq, long xs, long stream) {
  const RowQuant q{(const uint16_t*)x, ldx, H, T, (uint8_t*)xq, (float*)xs};
  return manage_tables_launch(ids, mk, E, S, max_distinct, max_inserts, table, map_cold, slot_expert, slot_stamp,
                              routed, step, miss, n_miss, blk, -1, -1, sorted_h, eids_h, ntpp_h, sorted_c, eids_c,
                              ntpp_c, hot_ids, q, stream);
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
                              eids_cold, npad_cold, 0, RowQuant{}, stream);
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
