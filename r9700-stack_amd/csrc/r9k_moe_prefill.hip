// r9k_moe_prefill.hip -- grouped MXFP4 x fp8 GEMM at prefill widths on gfx950: one workgroup computes a 256-row
// routing block (one expert) x 256 columns on V_MFMA_SCALE_F32_32X32X64_F8F6F4, K in 128-wide chunks that stream
// through a three-stage LDS ring filled by direct global->LDS DMA (global_load_lds_dwordx4).
//
// Same contract as the decode-family kernel (r9k_moe_gemm.hip): routed flat rows through the align tables
// (blocks of BM = 256 rows, experts ascending), out[r, n] = bf16(acc * (As[r / a_row_div] * topk_w[r])), the
// reference's epilogue (kernels/r9k_moe_mxfp4a8.hip:469-482). Weights in the same fragment order (1 KB per 16-row x
// 128-K tile) and exponent layout (64 bytes per tile and K-tile), so both kernels serve the same prepared tensors.
//
// Operands: the weights are the MFMA's A operand (fp4, cbsz = 4, their e8m0 block exponent as the A scale) and the
// activations its B operand (fp8, scale byte 127 = 2^0). The accumulator lane then holds one output row (lane % 32)
// and columns 8 * (q / 4) + 4 * g + q % 4 (g = lane / 32, q = 0..15): four consecutive columns per group, stored as
// one 8-byte write. Operand layout per lane (measured on gfx950): fp4 holds K = 32g .. 32g + 31 of its row and its
// scale byte scales that 32-block; fp8 holds K = 16g .. 16g + 15 in bytes 0..15 and K = 32 + 16g .. in bytes 16..31.
//
// Work split: 8 waves (two per SIMD) in 4 x 2, each a 64-row x 128-column sub-tile = 2 x 4 MFMA tiles of 32 x 32.
// Per chunk every thread issues 7 DMA loads (A: 4 x 16 B gathered through sorted_ids, B: 2 x 16 B, exponents: 4 B),
// two chunks ahead of the one being multiplied; an explicit vmcnt wait plus a barrier publishes a chunk. The A stage
// is XOR-swizzled (row r's 16-byte piece p at slot p ^ (r & 7)) so the fragment reads are bank-conflict free. M tiles
// whose 32 rows are all padding skip their MFMAs. Live tiles are renumbered so that each XCD gets a contiguous range
// (the column blocks of one routing block share an L2) and dead blocks past ntpp never occupy an XCD.
#include "r9k_common.h"
#include "r9k_dma.h"

#include <cstdlib>

namespace {

using namespace r9k;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int BM = 256, BN = 256, KC = 128;   // rows, columns, K per chunk
constexpr int NTH = 512;                       // 8 waves
constexpr int NXCD = 8;
constexpr int NSTAGE = 3;
constexpr int NT16 = BN / 16;                  // 16-row weight tiles per column block
constexpr int E8M0_ONE = 127;

struct __align__(16) Stage {
  uint8_t a[BM * KC];                          // 32 KB, swizzled 16-byte pieces
  uint8_t b[NT16 * 1024];                      // 16 KB, one 1 KB fragment-order tile per 16 columns
  uint8_t s[2 * NT16 * 64];                    // exponents: tile t at t * 64; the second KB is a dummy DMA target
};
constexpr size_t SMEM = sizeof(Stage) * NSTAGE;

// n / d for 32-bit unsigned n by a divisor fixed per launch, as a multiply-high and shifts (Granlund & Montgomery,
// "Division by invariant integers using multiplication", 1994, fig. 4.1): with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1, n / d = (t + ((n - t) >> 1)) >> (l - 1), t = mulhi(n, m); l = 0 means d = 1.
struct DivMagic {
  uint32_t m;
  int l;
};

DivMagic div_magic(uint32_t d) {
  int l = 0;
  while ((1ull << l) < d) l++;
  const uint64_t m = ((1ull << 32) * ((1ull << l) - d)) / d + 1;
  return {(uint32_t)m, l};
}

__device__ __forceinline__ uint32_t div_by(uint32_t n, DivMagic dm) {
  if (dm.l == 0) return n;
  const uint32_t t = __umulhi(n, dm.m);
  return (t + ((n - t) >> 1)) >> (dm.l - 1);
}

// 1 when the environment variable is set to "0" (a switch turned off).
int getenv_flag_off_pf(const char* name) {
  const char* v = getenv(name);
  return v && v[0] == '0' ? 1 : 0;
}


__global__ void __launch_bounds__(NTH) moe_prefill_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint8_t* __restrict__ Ws, uint16_t* __restrict__ C, const int* __restrict__ sorted_ids,
    const int* __restrict__ expert_ids, const int* __restrict__ ntpp, const float* __restrict__ topk_w,
    long wq_estride, long ws_estride, int numel, int a_row_div, int K, int N) {
  extern __shared__ __align__(16) uint8_t smem[];
  Stage* st = reinterpret_cast<Stage*>(smem);

  // live tiles only, each XCD (dispatch order L goes round-robin over them) a contiguous range of logical tiles
  const int nnb = gridDim.x;
  const int L = blockIdx.y * nnb + blockIdx.x;
  const int total = (ntpp[0] / BM) * nnb;
  if (L >= total) return;
  const int q = total / NXCD, rem = total % NXCD, x = L % NXCD;
  const int logical = x * q + min(x, rem) + L / NXCD;
  const int rb = logical / nnb, nb = logical % nnb;
  const int e = expert_ids[rb];
  if (e < 0) return;
  const int* __restrict__ rows = sorted_ids + (size_t)rb * BM;
  const int first = rows[0];
  if (first < 0 || first >= numel) return;

  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  // padding sits at the end of a block: the live rows are a prefix
  int live_here = 0;
  if (tid < BM) {
    const int fr = rows[tid];
    live_here = fr >= 0 && fr < numel;
  }
  const int nlive = __syncthreads_count(live_here);

  const int NTt = N / 16;
  const int KB = K / 32;
  const int nchunk = K / KC;
  const uint8_t* __restrict__ We = Wq + (size_t)e * wq_estride;
  const uint8_t* __restrict__ Se = Ws + (size_t)e * ws_estride;

  // ---- per-thread DMA sources (chunk 0) and wave-uniform LDS destinations (stage 0)
  const uint8_t* ga[4];
#pragma unroll
  for (int p = 0; p < 4; p++) {
    const int row = p * 64 + (tid >> 3);
    int fr = rows[row];
    if (row >= nlive) fr = first;
    const int piece = (tid & 7) ^ ((tid >> 3) & 7) ^ ((tid >> 6) & 1);            // row & 7 == (tid >> 3) & 7
    ga[p] = A + (size_t)(fr / a_row_div) * K + piece * 16;
  }
  const uint8_t* gb[2];
#pragma unroll
  for (int p = 0; p < 2; p++) {
    int nt = nb * NT16 + p * 8 + wave;                         // slot p * 512 + tid -> tile p * 8 + wave
    nt = nt < NTt ? nt : NTt - 1;                              // columns past N compute a copy, never stored
    gb[p] = We + (size_t)nt * (size_t)(8 * K) + lane * 16;
  }
  const uint8_t* gs;
  {
    int nt = nb * NT16 + (wave & 3) * 4 + (lane >> 4);
    nt = nt < NTt ? nt : NTt - 1;
    gs = Se + (size_t)nt * (size_t)(16 * KB) + (lane & 15) * 4;
  }
  const uint32_t la0 = lds_addr(&st[0].a[wave * 64 * 16]);
  const uint32_t lb0 = lds_addr(&st[0].b[wave * 64 * 16]);
  const uint32_t ls0 = lds_addr(&st[0].s[wave < 4 ? wave * 256 : 1024 + (wave - 4) * 256]);

  auto issue = [&](int c, int s) {
    const uint32_t so = (uint32_t)(s * (int)sizeof(Stage));
#pragma unroll
    for (int p = 0; p < 4; p++) dma16(ga[p] + (size_t)c * KC, la0 + so + p * 512 * 16);
#pragma unroll
    for (int p = 0; p < 2; p++) dma16(gb[p] + (size_t)c * 1024, lb0 + so + p * 512 * 16);
    dma4(gs + (size_t)c * 64, ls0 + so);
  };

  const int wm = wave >> 1, wn = wave & 1;                     // wave sub-tile: rows wm*64, columns wn*128
  const int g = lane >> 5, c32 = lane & 31;
  const int nmt = min(2, max(0, (nlive - wm * 64 + 31) / 32));  // live 32-row tiles of this wave (uniform)
  v16f acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = (v16f){};

  // fragment offsets within a stage
  int boff[2][4], soff[2][4];
#pragma unroll
  for (int ks = 0; ks < 2; ks++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int t16 = wn * 8 + 2 * j + (c32 >> 4), l16 = (2 * ks + g) * 16 + (c32 & 15);
      boff[ks][j] = t16 * 1024 + l16 * 16;
      soff[ks][j] = t16 * 64 + l16;
    }
  int aoff_lo[2][2], aoff_hi[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int row = wm * 64 + i * 32 + c32;
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      aoff_lo[i][ks] = (row * 8 + ((4 * ks + g) ^ (row & 7) ^ ((row >> 3) & 1))) * 16;
      aoff_hi[i][ks] = (row * 8 + ((4 * ks + 2 + g) ^ (row & 7) ^ ((row >> 3) & 1))) * 16;
    }
  }

  issue(0, 0);
  if (nchunk > 1) issue(1, 1);
  int s = 0;
  for (int c = 0; c < nchunk; c++) {
    if (c + 1 < nchunk) asm volatile("s_waitcnt vmcnt(7)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
    if (c + 2 < nchunk) issue(c + 2, s == 0 ? 2 : s - 1);       // the stage read in the previous iteration
    const Stage& S = st[s];
    if (nmt > 0) {
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        v8i wf[4];
        int sb[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(&S.b[boff[ks][j]]);
          wf[j] = (v8i){(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
          sb[j] = S.s[soff[ks][j]];
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
          if (i < nmt) {
            const u32x4 lo = *reinterpret_cast<const u32x4*>(&S.a[aoff_lo[i][ks]]);
            const u32x4 hi = *reinterpret_cast<const u32x4*>(&S.a[aoff_hi[i][ks]]);
            const v8i af = (v8i){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z,
                                 (int)hi.w};
#pragma unroll
            for (int j = 0; j < 4; j++)
              acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[j], af, acc[i][j], 4, 0, 0, sb[j], 0,
                                                                           E8M0_ONE);
          }
        }
      }
    }
    s = s == NSTAGE - 1 ? 0 : s + 1;
  }

  // epilogue: lane holds row c32 of each 32 x 32 tile, columns 8 * (q / 4) + 4 * g + q % 4
#pragma unroll
  for (int i = 0; i < 2; i++) {
    if (i >= nmt) continue;
    const int row = wm * 64 + i * 32 + c32;
    if (row >= nlive) continue;
    const int fr = rows[row];
    float sc = As[fr / a_row_div];
    if (topk_w) sc *= topk_w[fr];
    uint16_t* __restrict__ crow = C + (size_t)fr * N;
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
      for (int qb = 0; qb < 4; qb++) {
        const int n = nb * BN + wn * 128 + j * 32 + 8 * qb + 4 * g;
        if (n < N) {
          const uint32_t lo = (uint32_t)f2bf(acc[i][j][4 * qb] * sc) | ((uint32_t)f2bf(acc[i][j][4 * qb + 1] * sc) << 16);
          const uint32_t hi = (uint32_t)f2bf(acc[i][j][4 * qb + 2] * sc) |
                              ((uint32_t)f2bf(acc[i][j][4 * qb + 3] * sc) << 16);
          *reinterpret_cast<uint2*>(crow + n) = make_uint2(lo, hi);
        }
      }
    }
  }
}


// ------------------------------------------------------------------------------------------ persistent variant
// LDS beyond the chunk stages: per-tile metadata that arrives by DMA ahead of the tile's first chunk.
struct __align__(16) Aux {
  int rows[4][BM];     // tile sorted_ids, a ring of 4 tiles
  int eid[4][WAVE];    // tile expert id (64 copies), same ring
  float as[2][BM];     // As[row / a_row_div] of each tile row, two tiles
  float tw[2][BM];     // topk_w[row] of each tile row, two tiles
  int dummy[WAVE];     // target of the loads that keep every group at 9 loads a wave
};
constexpr size_t SMEM_P = sizeof(Stage) * NSTAGE + sizeof(Aux);
static_assert(SMEM_P <= 160 * 1024, "LDS");

// LDS fragment offsets of one wave within a stage. The B fragment of column tile j and K-half ks sits at
// b + j * 2048 + ks * 512 (its exponent byte at s + j * 128 + ks * 32); the A fragment of M tile i at
// a[half][ks] + i * 4096, the swizzle depending only on lane % 32.
struct FragOff {
  int b, s;
  int a[2][2];
};

__device__ __forceinline__ FragOff frag_offsets(int wm, int wn, int lane) {
  const int g = lane >> 5, c32 = lane & 31;
  FragOff f;
  const int t16 = wn * 8 + (c32 >> 4), l16 = g * 16 + (c32 & 15);
  f.b = t16 * 1024 + l16 * 16;
  f.s = t16 * 64 + l16;
  const int row = wm * 64 + c32, sw = (row & 7) ^ ((row >> 3) & 1);
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
    f.a[0][ks] = (row * 8 + ((4 * ks + g) ^ sw)) * 16;
    f.a[1][ks] = (row * 8 + ((4 * ks + 2 + g) ^ sw)) * 16;
  }
  return f;
}

// One wave's fragments for one 64-K half of a chunk: 4 weight fragments (fp4) with their exponent bytes, 2
// activation fragments (fp8, low and high K quarters).
struct KFrag {
  u32x4 w[4];
  int sb[4];
  u32x4 lo[2], hi[2];
};

__device__ __forceinline__ void load_kfrag(const Stage& S, const FragOff& f, int ks, KFrag& F) {
#pragma unroll
  for (int j = 0; j < 4; j++) {
    F.w[j] = *reinterpret_cast<const u32x4*>(&S.b[f.b + j * 2048 + ks * 512]);
    F.sb[j] = S.s[f.s + j * 128 + ks * 32];
  }
#pragma unroll
  for (int i = 0; i < 2; i++) {
    F.lo[i] = *reinterpret_cast<const u32x4*>(&S.a[f.a[0][ks] + i * 4096]);
    F.hi[i] = *reinterpret_cast<const u32x4*>(&S.a[f.a[1][ks] + i * 4096]);
  }
}

__device__ __forceinline__ void mfma_kfrag(v16f (&acc)[2][4], const KFrag& F) {
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const v8i af = (v8i){(int)F.lo[i].x, (int)F.lo[i].y, (int)F.lo[i].z, (int)F.lo[i].w,
                         (int)F.hi[i].x, (int)F.hi[i].y, (int)F.hi[i].z, (int)F.hi[i].w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const v8i wf = (v8i){(int)F.w[j].x, (int)F.w[j].y, (int)F.w[j].z, (int)F.w[j].w, 0, 0, 0, 0};
      acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf, af, acc[i][j], 4, 0, 0, F.sb[j], 0, E8M0_ONE);
    }
  }
}

// The 8 MFMAs of one K half from F (those of M tile i only when bit i of the wave-uniform `live` is set: a tile of
// 32 padding rows is skipped), MFMA k followed by extra(k) and the k-th of 8 groups of LDS reads that fill G from
// half `ks` of stage S. An MFMA holds its wave at issue until the matrix pipe takes it, so reads (or DMA
// issue) placed only after the last MFMA of a half run while the pipe idles; spread one group per MFMA, they run
// under the MFMAs instead. Scheduling barriers keep the order (G is a register set no queued MFMA still reads).
template <typename Extra>
__device__ __forceinline__ void mfma_load_kfrag(v16f (&acc)[2][4], const KFrag& F, const Stage& S,
                                                const FragOff& f, int ks, KFrag& G, int live, Extra extra) {
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const int i = k >> 2, j = k & 3;
    const v8i af = (v8i){(int)F.lo[i].x, (int)F.lo[i].y, (int)F.lo[i].z, (int)F.lo[i].w,
                         (int)F.hi[i].x, (int)F.hi[i].y, (int)F.hi[i].z, (int)F.hi[i].w};
    const v8i wf = (v8i){(int)F.w[j].x, (int)F.w[j].y, (int)F.w[j].z, (int)F.w[j].w, 0, 0, 0, 0};
    if (live & (1 << i))
      acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf, af, acc[i][j], 4, 0, 0, F.sb[j], 0, E8M0_ONE);
    __builtin_amdgcn_sched_barrier(0);
    extra(k);
    if (k < 4) {
      G.w[k] = *reinterpret_cast<const u32x4*>(&S.b[f.b + k * 2048 + ks * 512]);
      G.sb[k] = S.s[f.s + k * 128 + ks * 32];
    } else {
      const int ii = (k - 4) >> 1;
      if ((k & 1) == 0) G.lo[ii] = *reinterpret_cast<const u32x4*>(&S.a[f.a[0][ks] + ii * 4096]);
      else G.hi[ii] = *reinterpret_cast<const u32x4*>(&S.a[f.a[1][ks] + ii * 4096]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The same tiles and numerics as moe_prefill_kernel, but each workgroup (one per CU) walks a list of tiles and the
// K-chunk stream runs on across tile boundaries, with DMA three chunks ahead of the MFMAs. Within a chunk the two
// 64-K halves are software-pipelined: the second half's fragments are read from LDS under the first half's MFMAs,
// and the wait + barrier that publish the next chunk sit between the halves, so the next chunk's first fragments
// load under the current chunk's second-half MFMAs. Group j (chunk j + 3 plus 2 metadata dwords) is issued after
// barrier j, into the stage chunk j was read from. A tile's sorted_ids and expert id arrive 6 chunks before its
// first chunk, its per-row scales (As, topk_w) with its first chunk's DMA; its output is stored after its last
// chunk, staged through the activation region of that chunk's stage so each store writes 64 contiguous bytes of 16
// rows. That region is also where the group issued after the tile's last barrier puts its activation parts, so
// those 4 parts go out after the epilogue (each wave stages in the slots its own parts fill) while the group's
// weight, exponent and metadata parts go out under the MFMAs as usual. Every wave issues exactly 9 loads a group (7
// chunk pieces and 2 metadata or dummy dwords) and 16 stores a tile, so the waits are fixed counts: at barrier i
// chunk i + 1's loads are complete once at most 2 + 9 younger loads are outstanding, 2 + 9 + 16 at a tile's first
// chunk, and 9 at its second (the deferred parts came after the stores). Needs K / 128 >= 4: a metadata slot -- 4
// tiles of sorted_ids, 2 of scales -- is refilled at least one barrier after its tile's last reader, and the
// deferred group's chunk is the next tile's third, so its part 0 sets up no tile.
__global__ void __launch_bounds__(NTH) moe_prefill_persistent_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint8_t* __restrict__ Ws, uint16_t* __restrict__ C, const int* __restrict__ sorted_ids,
    const int* __restrict__ expert_ids, const int* __restrict__ ntpp, const float* __restrict__ topk_w,
    long wq_estride, long ws_estride, int numel, DivMagic rdiv, int K, int N, int nnb, int grp) {
  extern __shared__ __align__(16) uint8_t smem[];
  Stage* st = reinterpret_cast<Stage*>(smem);
  Aux& ax = *reinterpret_cast<Aux*>(smem + NSTAGE * sizeof(Stage));

  // tiles: XCD x (dispatch goes round-robin over the XCDs) owns a contiguous range of the live tiles (the column
  // blocks of a routing block, and the blocks of an expert, share its L2); its workgroups take every S-th tile
  const int G = gridDim.x, w = blockIdx.x, x = w % NXCD, jj = w / NXCD;
  const int S = (G - x + NXCD - 1) / NXCD;
  const int total = (ntpp[0] / BM) * nnb;
  const int q = total / NXCD, rem = total % NXCD;
  const int start = x * q + min(x, rem), cnt = q + (x < rem ? 1 : 0);
  if (jj >= cnt) return;
  const int ntiles = (cnt - jj + S - 1) / S;
  const int nchunk = K / KC, iters = ntiles * nchunk;
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int NTt = N / 16, KB = K / 32;
  // logical tile L -> (routing block, column block): groups of `grp` consecutive blocks, column-major within a group
  // (the group's blocks of one column block run side by side, so a hot expert's weight tile is fetched into the
  // XCD's L2 once for up to `grp` of its blocks)
  const int nblk = ntpp[0] / BM;
  if (grp <= 0) {                                              // chosen here: 4 when experts average 2+ blocks
    __shared__ int s_grp;
    if (wave == 0) {
      int starts = 0;                                          // blocks that begin an expert's run
      for (int b0 = 0; b0 < nblk; b0 += WAVE) {
        const int b = b0 + lane;
        starts += __popcll(__ballot(b < nblk && (b == 0 || expert_ids[b] != expert_ids[b - 1])));
      }
      if (lane == 0) s_grp = nblk >= 2 * starts ? 4 : 1;
    }
    __syncthreads();
    grp = __builtin_amdgcn_readfirstlane(s_grp);
  }
  auto tile_rb = [&](int m) {
    const int L = start + jj + m * S, g = L / (grp * nnb), r = L - g * grp * nnb;
    const int gb = min(grp, nblk - g * grp);
    return g * grp + r % gb;
  };
  auto tile_nb = [&](int m) {
    const int L = start + jj + m * S, g = L / (grp * nnb), r = L - g * grp * nnb;
    const int gb = min(grp, nblk - g * grp);
    return r / gb;
  };

  // metadata of the tiles whose DMA slot would come before the first group: plain loads
  for (int m = 0; m < ntiles && m * nchunk < 3; m++) {
    const int rb = tile_rb(m);
    if (tid < BM) ax.rows[m & 3][tid] = sorted_ids[(size_t)rb * BM + tid];
    if (tid < WAVE) ax.eid[m & 3][tid] = expert_ids[rb];
  }
  __syncthreads();

  auto tile_nlive = [&](int slot) {                            // live rows (a prefix of the block), per wave
    int n = 0;
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int fr = ax.rows[slot][u * WAVE + lane];
      n += __popcll(__ballot(fr >= 0 && fr < numel));
    }
    return n;
  };

  // DMA sources of the tile being issued: uniform bases, 32-bit per-lane offsets (the host keeps A and one expert's
  // codes below 2 GiB)
  uint32_t ga[4], gb[2], gs = 0;
  const uint8_t* wbase = Wq;
  const uint8_t* sbase = Ws;
  int issue_nl = 0, issue_slot = 0;
  auto setup_issue = [&](int m) {
    const int slot = m & 3;
    const int nl = tile_nlive(slot);
    int e = __builtin_amdgcn_readfirstlane(ax.eid[slot][0]);
    e = e < 0 ? 0 : e;
    const int nb = tile_nb(m);
    int first = ax.rows[slot][0];
    first = (first >= 0 && first < numel) ? first : 0;
    const int piece = (tid & 7) ^ ((tid >> 3) & 7) ^ ((tid >> 6) & 1);
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const int row = p * 64 + (tid >> 3);
      const int fr = row < nl ? ax.rows[slot][row] : first;
      ga[p] = div_by((uint32_t)fr, rdiv) * (uint32_t)K + piece * 16;
    }
    wbase = uniform_ptr(Wq + (size_t)e * wq_estride);
    sbase = uniform_ptr(Ws + (size_t)e * ws_estride);
#pragma unroll
    for (int p = 0; p < 2; p++) {
      int nt = nb * NT16 + p * 8 + wave;
      nt = nt < NTt ? nt : NTt - 1;
      gb[p] = (uint32_t)nt * (uint32_t)(8 * K) + lane * 16;
    }
    int nt = nb * NT16 + (wave & 3) * 4 + (lane >> 4);
    nt = nt < NTt ? nt : NTt - 1;
    gs = (uint32_t)nt * (uint32_t)(16 * KB) + (lane & 15) * 4;
    issue_nl = nl;
    issue_slot = slot;
  };

  const uint32_t la0 = lds_addr(&st[0].a[wave * 64 * 16]);
  const uint32_t lb0 = lds_addr(&st[0].b[wave * 64 * 16]);
  const uint32_t ls0 = lds_addr(&st[0].s[wave < 4 ? wave * 256 : 1024 + (wave - 4) * 256]);
  const uint32_t ldum = lds_addr(&ax.dummy[0]);
  const uint32_t doff = lane * 4;                              // dummy loads: sorted_ids[lane], always valid

  // group j (issued after barrier j, j >= -3): chunk j + 3, then the metadata dwords, in 8 parts that the main
  // loop places one behind each MFMA of a K half (part 0: the tile set-up on a tile's first chunk and A piece 0;
  // 1-3: A pieces; 4-5: the weight pieces, 5 also the exponents; 6: sorted_ids / expert id of the tile that starts
  // at chunk j + 6; 7: the per-row scales of a tile, with its first chunk). The positions of chunks j + 3 and j + 6
  // advance per group (no division by the chunk count).
  int g_m = 0, g_c = 0, g_s = 0;                               // tile, chunk within it, stage of chunk j + 3
  int h_m = 3 / nchunk, h_c = 3 % nchunk;                      // tile and chunk within it of chunk j + 6
  auto issue_part = [&](int part) {
    const uint32_t so = (uint32_t)(g_s * (int)sizeof(Stage));
    if (part == 0 && g_c == 0) setup_issue(g_m);
    if (part < 4) dma16s(A, ga[part] + (uint32_t)(g_c * KC), la0 + so + part * 512 * 16);
    if (part == 4 || part == 5)
      dma16s(wbase, gb[part - 4] + (uint32_t)(g_c * 1024), lb0 + so + (part - 4) * 512 * 16);
    if (part == 5) dma4s(sbase, gs + (uint32_t)(g_c * 64), ls0 + so);
    if (part == 6) {
      if (h_c == 0 && h_m < ntiles) {
        const int slot = h_m & 3, rb = tile_rb(h_m);
        if (wave < 4) dma4s(sorted_ids, (uint32_t)(rb * BM + wave * 64 + lane) * 4, lds_addr(&ax.rows[slot][wave * 64]));
        else if (wave == 4) dma4s(expert_ids, (uint32_t)rb * 4, lds_addr(&ax.eid[slot][0]));
        else dma4s(sorted_ids, doff, ldum);
      } else {
        dma4s(sorted_ids, doff, ldum);
      }
    }
    if (part == 7) {
      if (g_c == 0) {
        const int r = (wave & 3) * 64 + lane;
        int fr = r < issue_nl ? ax.rows[issue_slot][r] : ax.rows[issue_slot][0];
        fr = (fr >= 0 && fr < numel) ? fr : 0;
        if (wave < 4) dma4s(As, div_by((uint32_t)fr, rdiv) * 4, lds_addr(&ax.as[g_m & 1][wave * 64]));
        else if (topk_w) dma4s(topk_w, (uint32_t)fr * 4, lds_addr(&ax.tw[g_m & 1][(wave - 4) * 64]));
        else dma4s(sorted_ids, doff, ldum);
      } else {
        dma4s(sorted_ids, doff, ldum);
      }
      if (++g_c == nchunk) g_c = 0, g_m++;
      g_s = g_s == NSTAGE - 1 ? 0 : g_s + 1;
      if (++h_c == nchunk) h_c = 0, h_m++;
    }
  };
  auto issue_group = [&]() {
#pragma unroll
    for (int part = 0; part < 8; part++) issue_part(part);
  };

  const int wm = wave >> 1, wn = wave & 1;
  const int g = lane >> 5, c32 = lane & 31;
  const FragOff fo = frag_offsets(wm, wn, lane);
  // the output as a raw buffer (numel * N * 2 bytes, checked < 2^31 by the host): the epilogue's 16-byte stores go
  // out unconditionally and a padding row or a column past N stores at offset `cbytes`, which the buffer's range
  // check drops. Every wave so issues exactly 16 stores per tile, a fixed count the vmcnt waits below account for.
  const uint32_t cbytes = (uint32_t)numel * (uint32_t)N * 2u;
  const auto crs = __builtin_amdgcn_make_buffer_rsrc(C, (short)0, (int)cbytes, 0x00020000);
  constexpr int EPI_STORES = 16;

  issue_group();                                               // groups -3, -2, -1: chunks 0, 1, 2
  issue_group();
  issue_group();
  asm volatile("s_waitcnt vmcnt(20)" ::: "memory");             // chunk 0 (younger: 2 + 9 + 9)
  asm volatile("s_barrier" ::: "memory");
  KFrag F0, F1;
  load_kfrag(st[0], fo, 0, F0);
  int sidx = 0, i = 0;
  for (int m = 0; m < ntiles; m++) {
    v16f acc[2][4];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
      for (int b = 0; b < 4; b++) acc[a][b] = (v16f){};
    // this wave's M tiles (rows wm * 64 + 32 i ..) that hold a live row (the live rows are a prefix of the block)
    const int nlm = __builtin_amdgcn_readfirstlane(tile_nlive(m & 3));
    const int live = __builtin_amdgcn_readfirstlane((wm * 64 < nlm ? 1 : 0) | (wm * 64 + 32 < nlm ? 2 : 0));
    for (int c = 0; c < nchunk; c++, i++) {
      // F0 holds chunk i's first K half (read under the MFMAs of iteration i - 1); the second half's reads go out
      // between its MFMAs
      mfma_load_kfrag(acc, F0, st[sidx], fo, 1, F1, live, [](int) {});
      __builtin_amdgcn_sched_barrier(0);
      const int nidx = sidx == NSTAGE - 1 ? 0 : sidx + 1;
      if (i + 1 < iters) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");    // this wave's reads of chunk i are done
        // chunk i + 1 (group i - 2) is complete once no more than its 2 metadata dwords, group i - 1 (when issued)
        // and the previous tile's 16 output stores (when they came after group i - 2: c = 0 or 1) are outstanding.
        // Every tile but the last defers its last group's activation parts until after its epilogue's stores, so at
        // c = 1 of the next tile only group i - 1 is younger than chunk i + 1's last part.
        if (c == 1 && m > 0) {
          if (i + 2 < iters) asm volatile("s_waitcnt vmcnt(9)" ::: "memory");
          else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        } else {
          const bool epi = m > 0 && c == 0;
          if (i + 2 < iters) {
            if (epi) asm volatile("s_waitcnt vmcnt(27)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(11)" ::: "memory");
          } else {
            if (epi) asm volatile("s_waitcnt vmcnt(18)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
          }
        }
        asm volatile("s_barrier" ::: "memory");
      }
      __builtin_amdgcn_sched_barrier(0);
      // second-half MFMAs, each followed by a part of the next DMA group (into chunk i's stage, released by the
      // barrier) and reads of chunk i + 1's first half (after the last chunk they read a stale stage, unused)
      const bool defer = c == nchunk - 1 && m + 1 < ntiles;      // uniform; then i + 3 < iters (nchunk >= 4)
      mfma_load_kfrag(acc, F1, st[nidx], fo, 0, F0, live, [&](int k) {
        if (i + 3 < iters && !(defer && k < 4)) issue_part(k);
      });
      __builtin_amdgcn_sched_barrier(0);
      sidx = nidx;
    }
    {
      // tile m's output through 2 KB of LDS a wave in the activation region of its last chunk's stage (free since
      // that chunk's barrier): the 1 KB slots this wave's own activation parts 0 and 1 fill, so only its own deferred
      // DMA, issued after its reads, writes there. For M tile ii and 32-column tile j the wave's 32 rows x 64 B go in
      // (lane (c32, g) writes its 16-byte pieces 2 h + g of row c32, piece q of row r at position q ^ (r & 3) in half
      // r / 16), each lane reads piece lane & 3 of row lane / 4 of both halves,
      // and each store writes 64 contiguous bytes of 16 rows -- a row's pieces in neighbouring lanes, which the write
      // path merges. A wave's LDS operations execute in issue order; the next tile is packed while the reads return.
      // 16 stores a wave, as EPI_STORES; padding rows and columns past N go to the dropped offset.
      const int nl = nlm, nb = tile_nb(m);
      const int fidx = sidx == 0 ? NSTAGE - 1 : sidx - 1;      // the last chunk's stage
      uint8_t* ob = &st[fidx].a[wave * 1024];                 // half hs at + hs * 8192 (part hs's slot)
      const int rr = lane >> 2, qq = lane & 3, rl = c32 & 15;
      uint32_t trow[2][2];
      bool tlv[2][2];
      float scv[2];
#pragma unroll
      for (int ii = 0; ii < 2; ii++) {
        const int orow = wm * 64 + ii * 32 + c32;
        float sc = ax.as[m & 1][orow];
        if (topk_w) sc *= ax.tw[m & 1][orow];
        scv[ii] = sc;
#pragma unroll
        for (int hs = 0; hs < 2; hs++) {
          const int r = wm * 64 + ii * 32 + hs * 16 + rr;
          tlv[ii][hs] = r < nl;
          trow[ii][hs] = tlv[ii][hs] ? (uint32_t)ax.rows[m & 3][r] * (uint32_t)N : 0u;
        }
      }
      auto pack_tile = [&](int t, v4i (&v)[2]) {
        const int ii = t >> 2, j = t & 3;
        uint32_t p[4][2];
#pragma unroll
        for (int qb = 0; qb < 4; qb++) {
          p[qb][0] = pack_bf16x2(acc[ii][j][4 * qb] * scv[ii], acc[ii][j][4 * qb + 1] * scv[ii]);
          p[qb][1] = pack_bf16x2(acc[ii][j][4 * qb + 2] * scv[ii], acc[ii][j][4 * qb + 3] * scv[ii]);
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
          uint32_t got[2];
#pragma unroll
          for (int k = 0; k < 2; k++) {
            const auto r = __builtin_amdgcn_permlane32_swap(p[2 * h][k], p[2 * h + 1][k], false, false);
            got[k] = g == 0 ? r[1] : r[0];
          }
          v[h] = g == 0 ? (v4i){(int)p[2 * h][0], (int)p[2 * h][1], (int)got[0], (int)got[1]}
                        : (v4i){(int)got[0], (int)got[1], (int)p[2 * h + 1][0], (int)p[2 * h + 1][1]};
        }
      };
      v4i vb[2][2];
      pack_tile(0, vb[0]);
#pragma unroll
      for (int t = 0; t < 8; t++) {
        const int ii = t >> 2, j = t & 3;
        {
          uint8_t* ow = ob + (c32 >> 4) * 8192 + rl * 64;
#pragma unroll
          for (int h = 0; h < 2; h++) *reinterpret_cast<v4i*>(ow + (((2 * h + g) ^ (rl & 3)) * 16)) = vb[t & 1][h];
        }
        v4i w[2];
#pragma unroll
        for (int hs = 0; hs < 2; hs++)
          w[hs] = *reinterpret_cast<const v4i*>(ob + hs * 8192 + rr * 64 + ((qq ^ (rr & 3)) * 16));
        if (t + 1 < 8) pack_tile(t + 1, vb[(t + 1) & 1]);
        const int n = nb * BN + wn * 128 + j * 32 + qq * 8;
#pragma unroll
        for (int hs = 0; hs < 2; hs++) {
          const uint32_t off = (tlv[ii][hs] && n < N) ? (trow[ii][hs] + (uint32_t)n) * 2u : cbytes;
          __builtin_amdgcn_raw_buffer_store_b128(w[hs], crs, (int)off, 0, 0);
        }
      }
      if (m + 1 < ntiles) {
        // this wave's staging reads are back (each store waited for its read): the deferred group's activation
        // parts refill its slots, for the chunk before the group counter's (chunk 2 of the next tile, same stage)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const int dc = g_c == 0 ? nchunk - 1 : g_c - 1;
        const uint32_t so = (uint32_t)(fidx * (int)sizeof(Stage));
#pragma unroll
        for (int part = 0; part < 4; part++) dma16s(A, ga[part] + (uint32_t)(dc * KC), la0 + so + part * 512 * 16);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}


// ------------------------------------------------------------------------------ row-resident variant (K = 512)
// For the down GEMM at K = 512 (configs 2 and 3): each wave holds its 32 rows' activation fragments for the whole K
// in registers (64 VGPRs), so a routing block's activations are read once per workgroup instead of once per
// 256-column tile, and the LDS holds only a ring of four 34 KB stages. Work items are (routing block, 128-column
// step) pairs, block-major; XCD x owns a contiguous range of them and each of its workgroups a contiguous sub-range,
// so consecutive items of a workgroup are mostly columns of the same block. The workgroup walks a list of ring
// steps: per block it touches, four activation steps (64 rows x 512 B each, plus their As and topk_w; waves 2c and
// 2c + 1 copy theirs into registers) and then its column steps (the prepared layout's contiguous run of 8 column
// tiles x 4 K-tiles of codes, 32 KB, plus 2 KB of exponents). DMA runs three steps ahead. Every load of the loop is
// a global -> LDS DMA with an explicit wait, none a compiler-tracked load, so no compiler-inserted vmcnt wait drains
// the ring (vmcnt completes in order, and a load issued after the output stores would wait for them). Per column
// step and wave: 8 K-steps x 4 column tiles of the 32x32x64 scaled MFMA (weights as the fp4 A operand with their
// block exponent, activations as the fp8 B operand), then bf16(acc * As * topk_w) staged through 2 KB of LDS a
// wave, so each 16-byte-a-lane buffer store writes 64 contiguous bytes of 16 rows (padding rows and columns past N
// sent to the dropped offset). Every step issues the same DMA count per wave, column steps 8 stores and activation
// steps none, so the vmcnt waits are exact counts.
constexpr int RR_K = 512;
constexpr int RR_KS = RR_K / 64;                 // K-steps of one MFMA
constexpr int RR_NTS = 8;                        // 16-column weight tiles per step (128 columns)
constexpr int RR_NS = 4;                         // weight stages
constexpr int RR_MAXB = 7;                       // routing blocks a workgroup's item range may touch (the LDS
                                                 // beside the ring holds their tables and the output staging)
constexpr int RR_TB = RR_K * 8;                  // code bytes of one 16-column tile over K (4 KB)
constexpr int RR_SB = 16 * (RR_K / 32);          // exponent bytes of one 16-column tile over K (256 B)

struct __align__(16) RRStage {
  uint8_t b[RR_NTS * RR_TB];                     // 32 KB of codes
  uint8_t s[RR_NTS * RR_SB];                     // 2 KB of exponents
};
struct __align__(16) RRMeta {
  int rows[RR_MAXB][BM];                         // sorted_ids of the workgroup's blocks
  int eid[RR_MAXB];
  int nlive[RR_MAXB];                            // live rows (a prefix of the block); 0 for a block with no expert
};
constexpr int RR_OST = 2048;                     // LDS bytes a wave stages its output through (2 x 16 rows x 64 B)
constexpr size_t SMEM_RR = sizeof(RRStage) * RR_NS + sizeof(RRMeta) + (size_t)(NTH / WAVE) * RR_OST;
static_assert(SMEM_RR <= 160 * 1024, "LDS");

constexpr int RR_DMA_OPS = 5;                    // weight DMA instructions per wave and step
constexpr int RR_STORES = 8;                     // output stores per wave and column step
constexpr int RR_ACH = BM / 64;                  // activation steps per block (64 rows x 512 B each)

// s_waitcnt vmcnt(min(v, 40)) (waiting on fewer outstanding operations than there are is always safe).
__device__ __forceinline__ void rr_wait_vm(int v) {
#define RR_W(c)                                          \
  case c:                                                \
    asm volatile("s_waitcnt vmcnt(" #c ")" ::: "memory"); \
    break;
  switch (v < 0 ? 0 : v > 40 ? 40 : v) {
    RR_W(0) RR_W(1) RR_W(2) RR_W(3) RR_W(4) RR_W(5) RR_W(6) RR_W(7) RR_W(8) RR_W(9) RR_W(10) RR_W(11) RR_W(12)
    RR_W(13) RR_W(14) RR_W(15) RR_W(16) RR_W(17) RR_W(18) RR_W(19) RR_W(20) RR_W(21) RR_W(22) RR_W(23) RR_W(24)
    RR_W(25) RR_W(26) RR_W(27) RR_W(28) RR_W(29) RR_W(30) RR_W(31) RR_W(32) RR_W(33) RR_W(34) RR_W(35) RR_W(36)
    RR_W(37) RR_W(38) RR_W(39) RR_W(40)
  }
#undef RR_W
}

__global__ void __launch_bounds__(NTH) moe_prefill_rowres_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint8_t* __restrict__ Ws, uint16_t* __restrict__ C, const int* __restrict__ sorted_ids,
    const int* __restrict__ expert_ids, const int* __restrict__ ntpp, const float* __restrict__ topk_w,
    long wq_estride, long ws_estride, int numel, DivMagic rdiv, int N, int nsteps) {
  extern __shared__ __align__(16) uint8_t smem[];
  RRStage* st = reinterpret_cast<RRStage*>(smem);
  RRMeta& mt = *reinterpret_cast<RRMeta*>(smem + RR_NS * sizeof(RRStage));
  uint8_t* ost = smem + RR_NS * sizeof(RRStage) + sizeof(RRMeta) + (threadIdx.x / WAVE) * RR_OST;

  const int G = gridDim.x, wg = blockIdx.x, x = wg % NXCD, jj = wg / NXCD;
  const int S = (G - x + NXCD - 1) / NXCD;                     // workgroups on XCD x
  const int total = (ntpp[0] / BM) * nsteps;
  const int q = total / NXCD, rem = total % NXCD;
  const int xs = x * q + min(x, rem), xc = q + (x < rem ? 1 : 0);
  const int i0 = xs + (int)((long)xc * jj / S), i1 = xs + (int)((long)xc * (jj + 1) / S);
  if (i1 <= i0) return;
  const int rb0 = i0 / nsteps, nblk = (i1 - 1) / nsteps - rb0 + 1;   // <= RR_MAXB, checked by the host
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int NTt = N / 16;

  {
    // the blocks' tables, all loads in flight together (the kernel's only loads into registers)
    int rv[RR_MAXB];
#pragma unroll
    for (int b = 0; b < RR_MAXB; b++) rv[b] = (b < nblk && tid < BM) ? sorted_ids[(size_t)(rb0 + b) * BM + tid] : 0;
    const int ev = tid < nblk ? expert_ids[rb0 + tid] : 0;
#pragma unroll
    for (int b = 0; b < RR_MAXB; b++)
      if (b < nblk && tid < BM) mt.rows[b][tid] = rv[b];
    if (tid < nblk) mt.eid[tid] = ev;
  }
  __syncthreads();
  if (wave < nblk) {
    int nl = 0;
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int fr = mt.rows[wave][u * WAVE + lane];
      nl += __popcll(__ballot(fr >= 0 && fr < numel));
    }
    if (lane == 0) mt.nlive[wave] = mt.eid[wave] < 0 ? 0 : nl;
  }
  __syncthreads();

  // Steps: per touched block, RR_ACH activation steps (64 rows each, for waves 2c and 2c + 1) then its column steps
  // in this workgroup's range. A cursor walks them in order; items(b) = the block's column steps here.
  auto items = [&](int b) {
    const int lo = max(i0, (rb0 + b) * nsteps), hi = min(i1, (rb0 + b + 1) * nsteps);
    return hi - lo;
  };
  auto first_cs = [&](int b) { return max(i0 - (rb0 + b) * nsteps, 0); };
  int nst = 0;
  for (int b = 0; b < nblk; b++) nst += RR_ACH + items(b);
  struct Cursor {
    int b, off, len;
  };
  auto advance = [&](Cursor& c) {
    if (++c.off == c.len) {
      c.b++;
      c.off = 0;
      c.len = c.b < nblk ? RR_ACH + items(c.b) : 0;
    }
  };

  // DMA of step s into stage sg, RR_DMA_OPS instructions a wave whatever the step: a column step's 32 KB run of codes
  // (tiles past N re-read the last tile; their columns are never stored) and 2 KB of exponents; an activation step's
  // 64 rows x 512 B (16-byte piece p of chunk row r at position p ^ (r & 31), so the fragment reads are conflict-free)
  // and their scales (wave 0: As of each row, wave 1: topk_w, others a dummy dword).
  const uint32_t lb0 = lds_addr(&st[0].b[wave * WAVE * 16]);
  const uint32_t ls0 = lds_addr(&st[0].s[wave * WAVE * 4]);
  const uint32_t doff = (uint32_t)lane * 4;                    // dummy loads read sorted_ids[lane]
  auto issue = [&](const Cursor& c, int sg) {
    const uint32_t so = (uint32_t)(sg * (int)sizeof(RRStage));
    const int b = c.b;
    if (c.off < RR_ACH) {
      const int nl = mt.nlive[b];
      int first = mt.rows[b][0];
      first = (first >= 0 && first < numel) ? first : 0;
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const int r = p * 16 + (tid >> 5), row = c.off * 64 + r;  // row of the block
        const int fr = row < nl ? mt.rows[b][row] : first;
        const int piece = (tid & 31) ^ (r & 31);
        dma16s(A, div_by((uint32_t)fr, rdiv) * (uint32_t)RR_K + (uint32_t)piece * 16, lb0 + so + p * NTH * 16);
      }
      const int row = c.off * 64 + lane;
      const int fr = row < nl ? mt.rows[b][row] : first;
      if (wave == 0) dma4s(As, div_by((uint32_t)fr, rdiv) * 4, ls0 + so);
      else if (wave == 1 && topk_w) dma4s(topk_w, (uint32_t)fr * 4, ls0 + so);
      else dma4s(sorted_ids, doff, ls0 + so);
    } else {
      int e = mt.eid[b];
      e = __builtin_amdgcn_readfirstlane(e < 0 ? 0 : e);
      const int cs = first_cs(b) + c.off - RR_ACH;
      const uint8_t* wb = uniform_ptr(Wq + (size_t)e * wq_estride);
      const uint8_t* sb = uniform_ptr(Ws + (size_t)e * ws_estride);
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const int piece = p * NTH + tid;                       // 16-byte piece of the step's 32 KB run
        const int nt = min(cs * RR_NTS + (piece >> 8), NTt - 1);
        dma16s(wb, (uint32_t)nt * RR_TB + (uint32_t)(piece & 255) * 16, lb0 + so + p * NTH * 16);
      }
      const int nt = min(cs * RR_NTS + (tid >> 6), NTt - 1);
      dma4s(sb, (uint32_t)nt * RR_SB + (uint32_t)(tid & 63) * 4, ls0 + so);
    }
  };

  const int g = lane >> 5, c32 = lane & 31;
  // LDS offsets of this lane's weight fragment (column tile j, K-step t: + j * 8192 + t * 512) and exponent byte
  // (+ j * 512 + t * 32)
  const int fb = (c32 >> 4) * RR_TB + g * 256 + (c32 & 15) * 16;
  const int fs = (c32 >> 4) * RR_SB + g * 16 + (c32 & 15);
  const uint32_t cbytes = (uint32_t)numel * (uint32_t)N * 2u;
  const auto crs = __builtin_amdgcn_make_buffer_rsrc(C, (short)0, (int)cbytes, 0x00020000);

  Cursor ci{0, 0, RR_ACH + items(0)};                         // the step whose DMA goes out next
  for (int s = 0; s < 3 && s < nst; s++) {
    issue(ci, s);
    advance(ci);
  }
  Cursor cc{0, 0, RR_ACH + items(0)};                         // the step being computed
  // stores of the three steps before step s (a column step issues RR_STORES, an activation step none)
  int st1 = 0, st2 = 0, st3 = 0;

  u32x4 alo[RR_KS], ahi[RR_KS];
  float sc = 0.f;
  uint32_t trow[2] = {0u, 0u};                                 // output rows of this lane's stores (x N)
  bool tlive[2] = {false, false}, wlive = false;
  int sidx = 0;
  for (int s = 0; s < nst; s++) {
    // DMA of step s: younger are the stores of steps s - 3 .. s - 1 and the DMA of steps s + 1 and s + 2
    rr_wait_vm(st1 + st2 + st3 + (s + 1 < nst ? RR_DMA_OPS : 0) + (s + 2 < nst ? RR_DMA_OPS : 0));
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const RRStage& Sg = st[sidx];
    const int snext = sidx == 0 ? RR_NS - 1 : sidx - 1;       // stage read in the previous step
    int nstores = 0;
    if (cc.off < RR_ACH) {
      if (s + 3 < nst) {
        issue(ci, snext);
        advance(ci);
      }
      if ((wave >> 1) == cc.off) {
        // this wave's 32 rows of the block: activation fragments for all of K, scale, output row
        const int b = cc.b, nl = mt.nlive[b];
        const int r = (wave & 1) * 32 + c32;
        wlive = wave * 32 < nl;
        // the epilogue stores rows 16 hs + lane / 4 of the wave's 32
#pragma unroll
        for (int hs = 0; hs < 2; hs++) {
          const int orow = cc.off * 64 + (wave & 1) * 32 + 16 * hs + (lane >> 2);
          tlive[hs] = orow < nl;
          trow[hs] = tlive[hs] ? (uint32_t)mt.rows[b][orow] * (uint32_t)N : 0u;
        }
        const uint8_t* ab = &Sg.b[r * RR_K];
#pragma unroll
        for (int t = 0; t < RR_KS; t++) {
          alo[t] = *reinterpret_cast<const u32x4*>(ab + (((4 * t + g) ^ (r & 31)) * 16));
          ahi[t] = *reinterpret_cast<const u32x4*>(ab + (((4 * t + 2 + g) ^ (r & 31)) * 16));
        }
        const float* sf = reinterpret_cast<const float*>(Sg.s);
        sc = sf[r];
        if (topk_w) sc *= sf[WAVE + r];
      }
    } else {
      const int cs = first_cs(cc.b) + cc.off - RR_ACH;
      v16f acc[4];
#pragma unroll
      for (int j = 0; j < 4; j++) acc[j] = (v16f){};
      if (wlive) {
        u32x4 wf[2][4];
        int sbv[2][4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          wf[0][j] = *reinterpret_cast<const u32x4*>(&Sg.b[fb + j * 8192]);
          sbv[0][j] = Sg.s[fs + j * 512];
        }
#pragma unroll
        for (int t = 0; t < RR_KS; t++) {
          const int cb = t & 1, nbuf = cb ^ 1;
          if (t + 1 < RR_KS) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
              wf[nbuf][j] = *reinterpret_cast<const u32x4*>(&Sg.b[fb + j * 8192 + (t + 1) * 512]);
              sbv[nbuf][j] = Sg.s[fs + j * 512 + (t + 1) * 32];
            }
          }
          const v8i af = (v8i){(int)alo[t].x, (int)alo[t].y, (int)alo[t].z, (int)alo[t].w,
                               (int)ahi[t].x, (int)ahi[t].y, (int)ahi[t].z, (int)ahi[t].w};
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const v8i w8 = (v8i){(int)wf[cb][j].x, (int)wf[cb][j].y, (int)wf[cb][j].z, (int)wf[cb][j].w, 0, 0, 0, 0};
            acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w8, af, acc[j], 4, 0, 0, sbv[cb][j], 0,
                                                                      E8M0_ONE);
          }
          if (t == 0) {
            __builtin_amdgcn_sched_barrier(0);
            if (s + 3 < nst) {
              issue(ci, snext);
              advance(ci);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      } else if (s + 3 < nst) {
        issue(ci, snext);
        advance(ci);
      }
      // epilogue: bf16(acc * sc). Lanes l and l + 32 hold row c32; after the permlane32 pairs of the persistent
      // kernel's epilogue, lane (c32, g) holds 16-byte piece 2 h + g of each 32-column tile j. The wave stages the
      // rows through its 1 KB of LDS so that every store writes 64 contiguous bytes of 16 rows instead of 32 bytes of
      // 32 rows. For tile j, half hs (its own 1 KB): the 32 lanes of rows 16 hs .. 16 hs + 15 write their two pieces
      // (piece q of row r at position q ^ (r & 3)) and every lane reads piece lane & 3 of row lane / 4. A wave's LDS
      // operations execute in issue order, so the reads see the writes with no wait between them; tile j + 1 is
      // packed while the reads are in flight, then tile j's two stores go out. RR_STORES = 8 stores a wave and
      // column step, the count the vmcnt waits assume; rows past the live ones and columns past N go to the dropped
      // offset.
      auto pack_tile = [&](int j, v4i (&v)[2]) {
        uint32_t pk[4][2];
#pragma unroll
        for (int qb = 0; qb < 4; qb++) {
          pk[qb][0] = pack_bf16x2(acc[j][4 * qb] * sc, acc[j][4 * qb + 1] * sc);
          pk[qb][1] = pack_bf16x2(acc[j][4 * qb + 2] * sc, acc[j][4 * qb + 3] * sc);
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
          uint32_t got[2];
#pragma unroll
          for (int kk = 0; kk < 2; kk++) {
            const auto pr = __builtin_amdgcn_permlane32_swap(pk[2 * h][kk], pk[2 * h + 1][kk], false, false);
            got[kk] = g == 0 ? pr[1] : pr[0];
          }
          v[h] = g == 0 ? (v4i){(int)pk[2 * h][0], (int)pk[2 * h][1], (int)got[0], (int)got[1]}
                        : (v4i){(int)got[0], (int)got[1], (int)pk[2 * h + 1][0], (int)pk[2 * h + 1][1]};
        }
      };
      const int rr = lane >> 2, qq = lane & 3, rl = c32 & 15;
      v4i vb[2][2];
      pack_tile(0, vb[0]);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        {
          uint8_t* ow = ost + (c32 >> 4) * 1024 + rl * 64;
#pragma unroll
          for (int h = 0; h < 2; h++) *reinterpret_cast<v4i*>(ow + (((2 * h + g) ^ (rl & 3)) * 16)) = vb[j & 1][h];
        }
        v4i w[2];
#pragma unroll
        for (int hs = 0; hs < 2; hs++)
          w[hs] = *reinterpret_cast<const v4i*>(ost + hs * 1024 + rr * 64 + ((qq ^ (rr & 3)) * 16));
        if (j + 1 < 4) pack_tile(j + 1, vb[(j + 1) & 1]);
        const int col = cs * RR_NTS * 16 + j * 32 + qq * 8;
#pragma unroll
        for (int hs = 0; hs < 2; hs++) {
          const uint32_t off = (tlive[hs] && col < N) ? (trow[hs] + (uint32_t)col) * 2u : cbytes;
          __builtin_amdgcn_raw_buffer_store_b128(w[hs], crs, (int)off, 0, 0);
        }
      }
      nstores = RR_STORES;
    }
    st3 = st2;
    st2 = st1;
    st1 = nstores;
    advance(cc);
    sidx = sidx == RR_NS - 1 ? 0 : sidx + 1;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

}  // namespace

// Internal entry used by the prefill dispatch in r9k_moe_gemm.hip: tables with blocks of 256 rows, K % 128 == 0.
// K = 512 runs the row-resident kernel, other K >= 384 the persistent kernel (both one workgroup per CU), K = 128
// and 256 the one-tile-per-workgroup kernel.
int r9k_prefill_launch(long a, long as, long wq, long ws, long c, long sorted_ids, long expert_ids, long ntpp,
                       long topk_w, long ws_estride, int max_blocks, int numel, int a_row_div, int K, int N,
                       long stream) {
  if (N % 16) return -1;
  if (K % KC) return -2;
  if (max_blocks <= 0 || numel <= 0) return 0;
  if (max_blocks > 65535) return -3;
  if ((a & 15) || (wq & 15) || (ws & 3) || (c & 15)) return -3;             // 16-byte DMA sources and stores
  const int nnb = (N / 16 + NT16 - 1) / NT16;
  const long a_rows = ((long)numel + a_row_div - 1) / a_row_div;
  if (a_rows * K >= (1L << 31) || (long)N * K / 2 >= (1L << 31) || (long)numel * 4 >= (1L << 31) ||
      (long)numel * N * 2 >= (1L << 31))
    return -3;
  if (K == RR_K && getenv_flag_off_pf("R9K_PREFILL_ROWRES") == 0) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      return -6;
    const int nsteps = (N + RR_NTS * 16 - 1) / (RR_NTS * 16);
    const long items = (long)max_blocks * nsteps;
    const int grid = (int)(items < cus ? items : cus);
    // a workgroup's item range (at most ceil(ceil(items / 8) / (grid / 8)) items) must touch <= RR_MAXB blocks
    const long wpx = grid / NXCD > 1 ? grid / NXCD : 1;
    const long per_wg = ((items + NXCD - 1) / NXCD + wpx - 1) / wpx;
    if ((per_wg + nsteps - 2) / nsteps + 1 <= RR_MAXB) {
      static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(moe_prefill_rowres_kernel),
                                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)SMEM_RR);
      if (attr != hipSuccess) return -4;
      hipLaunchKernelGGL(moe_prefill_rowres_kernel, dim3(grid), dim3(NTH), SMEM_RR, (hipStream_t)stream,
                         (const uint8_t*)a, (const float*)as, (const uint8_t*)wq, (const uint8_t*)ws, (uint16_t*)c,
                         (const int*)sorted_ids, (const int*)expert_ids, (const int*)ntpp, (const float*)topk_w,
                         (long)N * K / 2, ws_estride, numel, div_magic((uint32_t)a_row_div), N, nsteps);
      return hipGetLastError() == hipSuccess ? 0 : -6;
    }
  }
  if (K / KC >= 4 && getenv_flag_off_pf("R9K_PREFILL_PERSIST") == 0) {
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(moe_prefill_persistent_kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)SMEM_P);
    if (attr != hipSuccess) return -4;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      return -6;
    // routing blocks per tile group (column-major within a group), chosen in the kernel from the table (0): 4 when
    // the experts average two or more blocks, else 1. Measured on MI355X: config 5 T = 4096's 256-row pass (65
    // experts, 169 blocks, the hot experts' blocks sharing each weight tile through L2) down 312 -> 292 us, gate_up
    // 531 -> 526 us with 4; config 3's gate_up (300 blocks, 288 experts) reads 460 MB with 1 and 495 MB with 4
    // (four experts' activation blocks live in L2 at once), 148 -> 152 us. R9K_PREFILL_GROUP forces a size.
    const char* pv = getenv("R9K_PREFILL_GROUP");
    const int grp = pv && atoi(pv) > 0 ? atoi(pv) : 0;
    const long tiles = (long)max_blocks * nnb;
    const int grid = (int)(tiles < cus ? tiles : cus);
    hipLaunchKernelGGL(moe_prefill_persistent_kernel, dim3(grid), dim3(NTH), SMEM_P, (hipStream_t)stream,
                       (const uint8_t*)a, (const float*)as, (const uint8_t*)wq, (const uint8_t*)ws, (uint16_t*)c,
                       (const int*)sorted_ids, (const int*)expert_ids, (const int*)ntpp, (const float*)topk_w,
                       (long)N * K / 2, ws_estride, numel, div_magic((uint32_t)a_row_div), K, N, nnb, grp);
    return hipGetLastError() == hipSuccess ? 0 : -6;
  }
  const dim3 grid(nnb, max_blocks);
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(moe_prefill_kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)SMEM);
  if (attr != hipSuccess) return -4;
  hipLaunchKernelGGL(moe_prefill_kernel, grid, dim3(NTH), SMEM, (hipStream_t)stream, (const uint8_t*)a,
                     (const float*)as, (const uint8_t*)wq, (const uint8_t*)ws, (uint16_t*)c, (const int*)sorted_ids,
                     (const int*)expert_ids, (const int*)ntpp, (const float*)topk_w, (long)N * K / 2, ws_estride,
                     numel, a_row_div, K, N);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

int r9k_prefill_block_rows() { return BM; }
