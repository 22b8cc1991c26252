// r9k_moe_prefill.hip -- grouped MXFP4 x fp8 GEMM at prefill widths on gfx950: one workgroup computes a 256-row
// routing block (one expert) x 256 columns, K in 128-wide chunks staged through LDS, on
// V_MFMA_SCALE_F32_32X32X64_F8F6F4 (fp8 A with scale byte 127, fp4 B with its e8m0 block exponent).
//
// Same contract as the decode-family kernel (r9k_moe_gemm.hip): routed flat rows through the align tables
// (blocks of BM = 256 rows, experts ascending), out[r, n] = bf16(acc * (As[r / a_row_div] * topk_w[r])), the
// reference's epilogue (kernels/r9k_moe_mxfp4a8.hip:469-482). Weights in the same fragment order (1 KB per 16-row x
// 128-K tile) and exponent layout, so both kernels serve the same prepared tensors.
//
// Work split: 8 waves (two per SIMD) in 4 x 2, each wave a 64 x 128 sub-tile = 2 x 4 MFMA tiles of 32 x 32 (128 fp32
// accumulators per lane). Per 128-K chunk the workgroup stages A (256 rows x 128 B, gathered through sorted_ids),
// B (16 column tiles x 1 KB, contiguous) and the chunk's exponents (1 KB) in LDS; the next chunk's global loads are
// in flight in registers while the current chunk's 16 MFMAs per wave run, one barrier per chunk. M tiles whose 32
// rows are all padding skip their MFMAs. K % 128 == 0 (the host routes other K to the decode-family kernel).
// Workgroups are renumbered so the column blocks of one routing block run on the same XCD (one L2 holds its A rows).
//
// 32x32x64 operand layout (measured on gfx950): output row = A lane % 32, column = B lane % 32, g = lane / 32; fp4 B
// holds K = 32g .. 32g + 31 (its scale byte scales that block); fp8 A holds K = 16g .. 16g + 15 in bytes 0..15 and
// K = 32 + 16g .. in bytes 16..31; C lane holds column lane % 32, rows 8 * (j / 4) + 4 * g + j % 4 for j = 0..15.
#include "r9k_common.h"

namespace {

using namespace r9k;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 256, BN = 256, KC = 128;   // rows, columns, K per chunk
constexpr int NTH = 512;                       // 8 waves
constexpr int NXCD = 8;
constexpr int ASTR = KC + 16;                  // LDS row stride of the A stage (conflict-free 16-byte reads)
constexpr int NT16 = BN / 16;                  // 16-row weight tiles per column block
constexpr int E8M0_ONE = 127;

struct __align__(16) Stage {
  uint8_t a[BM * ASTR];                        // 36 KB
  uint8_t b[NT16 * 1024];                      // 16 KB: fragment order, one 1 KB tile per 16 columns
  uint8_t s[NT16 * 64];                        // 1 KB: exponent byte of (tile, lane)
};

struct Shared {
  Stage st[2];
  int aoff[BM];                                // byte offset of each row's A row (padding rows: the block's first)
  int fr[BM];                                  // routed flat row or -1 (padding)
  float sc[BM];                                // As * topk_w
};

__global__ void __launch_bounds__(NTH) moe_prefill_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint8_t* __restrict__ Ws, uint16_t* __restrict__ C, const int* __restrict__ sorted_ids,
    const int* __restrict__ expert_ids, const int* __restrict__ ntpp, const float* __restrict__ topk_w,
    long wq_estride, long ws_estride, int numel, int a_row_div, int K, int N) {
  extern __shared__ __align__(16) uint8_t smem[];
  Shared& sh = *reinterpret_cast<Shared*>(smem);
  // dispatch order L goes round-robin over the XCDs; give each XCD a contiguous range of logical tiles
  const int nnb = gridDim.x, total = nnb * gridDim.y;
  const int L = blockIdx.y * nnb + blockIdx.x;
  const int q = total / NXCD, rem = total % NXCD, x = L % NXCD;
  const int logical = x * q + min(x, rem) + L / NXCD;
  const int rb = logical / nnb, nb = logical % nnb;
  if (rb * BM >= ntpp[0]) return;
  const int e = expert_ids[rb];
  if (e < 0) return;
  const int first = sorted_ids[rb * BM];
  if (first < 0 || first >= numel) return;
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;

  // row metadata; padding sits at the end of the block, so the live rows are a prefix
  if (tid < BM) {
    const int fr = sorted_ids[rb * BM + tid];
    const bool live = fr >= 0 && fr < numel;
    const int src = live ? fr : first;
    sh.aoff[tid] = (src / a_row_div) * K;
    sh.fr[tid] = live ? fr : -1;
    float s = 0.f;
    if (live) {
      s = As[fr / a_row_div];
      if (topk_w) s *= topk_w[fr];
    }
    sh.sc[tid] = s;
  }
  __syncthreads();
  int nlive;
  {
    int lo = 0, hi = BM;                                       // first padding row (prefix property)
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (sh.fr[mid] >= 0) lo = mid + 1; else hi = mid;
    }
    nlive = __builtin_amdgcn_readfirstlane(lo);
  }

  const int NTt = N / 16;
  const int nt0 = nb * NT16;
  const uint8_t* __restrict__ We = Wq + (size_t)e * wq_estride;
  const uint8_t* __restrict__ Se = Ws + (size_t)e * ws_estride;
  const int KB = K / 32, nq = KB / 16;
  const int nchunk = K / KC;

  // ---- global -> register staging of one chunk: A 4 x 16 B, B 2 x 16 B, exponents 4 B (threads 0..255)
  const int a_sub = tid & 7, a_row = tid >> 3;                 // 8 threads per A row, 64 rows per pass
  // 32-bit byte offsets from the wave-uniform bases (the host keeps A and one expert's weights below 2 GiB)
  uint32_t aoff[4];
#pragma unroll
  for (int p = 0; p < 4; p++) {
    const int row = p * 64 + a_row;
    aoff[p] = (uint32_t)sh.aoff[row < nlive ? row : 0] + a_sub * 16;
  }
  uint32_t boff[2];
#pragma unroll
  for (int p = 0; p < 2; p++) {
    const int f = p * NTH + tid;                               // 16-byte piece of the 16 KB B stage
    int nt = nt0 + (f >> 6);
    nt = nt < NTt ? nt : NTt - 1;
    boff[p] = (uint32_t)nt * (uint32_t)(8 * K) + (f & 63) * 16;
  }
  uint32_t soff;
  {
    int nt = nt0 + ((tid & 255) >> 4);
    nt = nt < NTt ? nt : NTt - 1;
    soff = (uint32_t)nt * (uint32_t)(16 * KB);                 // this thread: lanes 4 * (tid % 16) .. + 3
  }
  const int sl4 = (tid & 15) * 4;
  u32x4 ra[4];
  u32x4 rbw[2];
  uint32_t rs = 0;
  auto load_chunk = [&](int kt) {
#pragma unroll
    for (int p = 0; p < 4; p++) ra[p] = *reinterpret_cast<const u32x4*>(A + (aoff[p] + (uint32_t)(kt * KC)));
#pragma unroll
    for (int p = 0; p < 2; p++)
      rbw[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(We + (boff[p] + (uint32_t)(kt * 1024))));
    if (tid < 256) {
      if (kt < 4 * nq) {                                       // 4-chunk super-step: one byte of each lane's dword
        const u32x4 d = *reinterpret_cast<const u32x4*>(Se + (soff + (uint32_t)((kt >> 2) * 256 + sl4 * 4)));
        const int sh8 = 8 * (kt & 3);
        rs = ((d.x >> sh8) & 0xffu) | (((d.y >> sh8) & 0xffu) << 8) | (((d.z >> sh8) & 0xffu) << 16) |
             (((d.w >> sh8) & 0xffu) << 24);
      } else {
        rs = *reinterpret_cast<const uint32_t*>(Se + (soff + (uint32_t)(nq * 256 + (kt - 4 * nq) * 64 + sl4)));
      }
    }
  };
  auto store_chunk = [&](Stage& S) {
#pragma unroll
    for (int p = 0; p < 4; p++) *reinterpret_cast<u32x4*>(&S.a[(p * 64 + a_row) * ASTR + a_sub * 16]) = ra[p];
#pragma unroll
    for (int p = 0; p < 2; p++) *reinterpret_cast<u32x4*>(&S.b[(p * NTH + tid) * 16]) = rbw[p];
    if (tid < 256) *reinterpret_cast<uint32_t*>(&S.s[tid * 4]) = rs;
  };

  const int wm = wave >> 1, wn = wave & 1;                     // wave sub-tile: rows wm*64, columns wn*128
  const int g = lane >> 5, c32 = lane & 31;
  v16f acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = (v16f){};
  const int nmt = min(2, max(0, (nlive - wm * 64 + 31) / 32));  // live 32-row tiles of this wave (uniform)

  load_chunk(0);
  store_chunk(sh.st[0]);
  __syncthreads();
  for (int c = 0; c < nchunk; c++) {
    const bool more = c + 1 < nchunk;
    if (more) load_chunk(c + 1);
    const Stage& S = sh.st[c & 1];
    if (nmt > 0) {
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        v8i bf[4];
        int sb[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int col = wn * 128 + j * 32 + c32;             // column within the block
          const int t16 = col >> 4, r16 = col & 15, l16 = (2 * ks + g) * 16 + r16;
          const u32x4 v = *reinterpret_cast<const u32x4*>(&S.b[(t16 * 64 + l16) * 16]);
          bf[j] = (v8i){(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
          sb[j] = S.s[t16 * 64 + l16];
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
          if (i < nmt) {
            const uint8_t* ar = &S.a[(wm * 64 + i * 32 + c32) * ASTR + ks * 64];
            const u32x4 lo = *reinterpret_cast<const u32x4*>(ar + 16 * g);
            const u32x4 hi = *reinterpret_cast<const u32x4*>(ar + 32 + 16 * g);
            const v8i af = (v8i){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                                 (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
#pragma unroll
            for (int j = 0; j < 4; j++)
              acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af, bf[j], acc[i][j], 0, 4, 0, E8M0_ONE,
                                                                           0, sb[j]);
          }
        }
      }
    }
    if (more) store_chunk(sh.st[(c + 1) & 1]);
    __syncthreads();
  }

  // epilogue: lane holds column c32 of each 32 x 32 tile, rows 8 * (q / 4) + 4 * g + q % 4
#pragma unroll
  for (int i = 0; i < 2; i++) {
    if (i >= nmt) continue;
#pragma unroll
    for (int q = 0; q < 16; q++) {
      const int row = wm * 64 + i * 32 + 8 * (q >> 2) + 4 * g + (q & 3);
      const int fr = sh.fr[row];
      if (fr < 0) continue;
      const float s = sh.sc[row];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int n = nt0 * 16 + wn * 128 + j * 32 + c32;
        if (n < N) C[(size_t)fr * N + n] = f2bf(acc[i][j][q] * s);
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
  const long a_rows = ((long)numel + a_row_div - 1) / a_row_div;
  if (a_rows * K >= (1L << 31) || (long)N * K / 2 >= (1L << 31)) return -3;   // 32-bit in-kernel offsets
  const dim3 grid((N / 16 + NT16 - 1) / NT16, max_blocks);
  const size_t smem = sizeof(Shared);
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(moe_prefill_kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (attr != hipSuccess) return -4;
  hipLaunchKernelGGL(moe_prefill_kernel, grid, dim3(NTH), smem, (hipStream_t)stream, (const uint8_t*)a,
                     (const float*)as, (const uint8_t*)wq, (const uint8_t*)ws, (uint16_t*)c, (const int*)sorted_ids,
                     (const int*)expert_ids, (const int*)ntpp, (const float*)topk_w, (long)N * K / 2, ws_estride,
                     numel, a_row_div, K, N);
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

int r9k_prefill_block_rows() { return BM; }
