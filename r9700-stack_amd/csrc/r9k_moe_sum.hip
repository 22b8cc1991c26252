// r9k_moe_sum.hip -- the MoE layer's output: the weighted top-k sum (router weights already applied by the down
// GEMM's epilogue), plus optionally a shared-expert term, in one launch on gfx950.
//
//   out[m, n] = bf16_rne( sum_{j = 0 .. topk-1} float(down[m, j, n])  (+ float(shared[m, n])) )
//
// fp32 accumulation in ascending j, then the shared term, ONE bf16 rounding (reference:
// kernels/r9k_moe_sum.hip:7-12, 32-56). Each thread owns 8 consecutive columns of one token (16-byte loads of
// every top-k row and one 16-byte store); the grid is (column chunks, tokens), so each wave reads whole 1 KB
// row segments and the per-token rows stream once.
#include "r9k_common.h"

namespace {

using namespace r9k;

constexpr int ST = 256;

typedef uint16_t v8u16 __attribute__((ext_vector_type(8)));

__global__ void __launch_bounds__(ST) moe_sum_kernel(const uint16_t* __restrict__ down,
                                                     const uint16_t* __restrict__ shared, uint16_t* __restrict__ out,
                                                     int M, int topk, int N, long ld_shared, long ld_out) {
  const int m = blockIdx.y;
  const int c = (blockIdx.x * ST + threadIdx.x) * 8;
  if (m >= M || c >= N) return;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; i++) acc[i] = 0.f;
  const uint16_t* row = down + (size_t)m * topk * N + c;
  for (int j = 0; j < topk; j++) {
    const v8u16 v = *reinterpret_cast<const v8u16*>(row + (size_t)j * N);
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] += bf2f(v[i]);
  }
  if (shared != nullptr) {
    const v8u16 sv = *reinterpret_cast<const v8u16*>(shared + (size_t)m * ld_shared + c);
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] += bf2f(sv[i]);
  }
  v8u16 o;
#pragma unroll
  for (int i = 0; i < 8; i++) o[i] = f2bf(acc[i]);
  *reinterpret_cast<v8u16*>(out + (size_t)m * ld_out + c) = o;
}

}  // namespace

// Reference: kernels/r9k_moe_sum.hip:62-69. down [M, topk, N] bf16 contiguous; shared [M, N] with row stride
// ld_shared (0 pointer = none); out [M, N] with row stride ld_out. N % 8 == 0, 16-byte aligned rows.
// Returns 0 on success, 1 for an unsupported shape, else the HIP error code.
extern "C" int r9k_moe_sum(long down, long shared, long out, int M, int topk, int N, long ld_shared, long ld_out,
                           long stream) {
  if (M < 1 || topk < 1 || N < 8 || (N & 7)) return 1;
  if ((down & 15) || (out & 15) || (ld_out & 7) || (shared && ((shared & 15) || (ld_shared & 7)))) return 1;
  const dim3 grid((N / 8 + ST - 1) / ST, M), block(ST);
  hipLaunchKernelGGL(moe_sum_kernel, grid, block, 0, (hipStream_t)stream, (const uint16_t*)down,
                     (const uint16_t*)shared, (uint16_t*)out, M, topk, N, ld_shared, ld_out);
  return (int)hipGetLastError();
}
