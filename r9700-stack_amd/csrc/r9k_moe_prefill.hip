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

namespace {

using namespace r9k;

typedef int v8i __attribute__((ext_vector_type(8)));
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

// global -> LDS DMA of 16 (4) bytes per lane: lane l's bytes land at LDS address `lds` + 16 l (4 l). M0 carries the
// wave-uniform LDS base. Completion is tracked by vmcnt; the kernel waits for it explicitly.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
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

}  // namespace

// Internal entry used by the prefill dispatch in r9k_moe_gemm.hip: tables with blocks of 256 rows, K % 128 == 0.
int r9k_prefill_launch(long a, long as, long wq, long ws, long c, long sorted_ids, long expert_ids, long ntpp,
                       long topk_w, long ws_estride, int max_blocks, int numel, int a_row_div, int K, int N,
                       long stream) {
  if (N % 16) return -1;
  if (K % KC) return -2;
  if (max_blocks <= 0 || numel <= 0) return 0;
  if (max_blocks > 65535) return -3;
  if ((a & 15) || (wq & 15) || (ws & 3) || (c & 7)) return -3;              // 16-byte DMA sources, 8-byte stores
  const dim3 grid((N / 16 + NT16 - 1) / NT16, max_blocks);
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
