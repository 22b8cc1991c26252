// r9k_moe_sum.hip -- the MoE layer's output for the multi-launch path: the top-k sum of the routed rows' down
// outputs (router weights already applied in the down GEMM's epilogue), plus an optional shared-expert term.
//
//   out[m, n] = bf16_rne( sum_{j = 0 .. topk-1} float(down[m, j, n])  (+ float(shared[m, n])) )
//
// The summation order and the single rounding are the contract (reference: kernels/r9k_moe_sum.hip:7-12): fp32
// accumulation with j ascending, the shared term last, one bf16 rounding at the end.
//
// Layout of the work on gfx950: one wave owns a segment of 512 columns (8 per lane, one 16-byte chunk) of one
// token, and waves walk the (token, segment) items grid-stride, so the launch is sized to the chip rather than to
// M. For each item a lane issues the loads of all its top-k chunks (up to 16 at once, larger top-k in batches of 16)
// and the shared chunk before it adds any of them, so one item costs one memory round trip however large topk is;
// the adds then run in slot order.
#include "r9k_common.h"

namespace {

using namespace r9k;

constexpr int SUM_WAVES = 4;      // waves per workgroup
constexpr int SEG = 8 * WAVE;     // columns per item (one 16-byte chunk a lane)
constexpr int BATCH = 16;         // top-k chunks a lane keeps in flight
constexpr long MAX_WG = 16384;    // 64 workgroups for each of MI355X's 256 CUs; larger M walks grid-stride

typedef uint16_t v8u16 __attribute__((ext_vector_type(8)));

template <bool NT>
__global__ void __launch_bounds__(SUM_WAVES * WAVE) moe_sum_kernel(const uint16_t* __restrict__ down,
                                                                   const uint16_t* __restrict__ shared,
                                                                   uint16_t* __restrict__ out, int M, int topk, int N,
                                                                   long ld_shared, long ld_out) {
  const int lane = threadIdx.x % WAVE;
  const long segs = (N + SEG - 1) / SEG;
  const long items = (long)M * segs;
  const long nwaves = (long)gridDim.x * SUM_WAVES;
  for (long it = (long)blockIdx.x * SUM_WAVES + threadIdx.x / WAVE; it < items; it += nwaves) {
    const long m = it / segs;
    const int c = (int)(it - m * segs) * SEG + lane * 8;
    if (c >= N) continue;
    const uint16_t* src = down + (size_t)m * topk * N + c;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; j0 < topk; j0 += BATCH) {
      v8u16 v[BATCH];
#pragma unroll
      for (int u = 0; u < BATCH; u++)
        if (j0 + u < topk) {
          const v8u16* p = reinterpret_cast<const v8u16*>(src + (size_t)(j0 + u) * N);
          if constexpr (NT) v[u] = __builtin_nontemporal_load(p);
          else v[u] = *p;
        }
#pragma unroll
      for (int u = 0; u < BATCH; u++)
        if (j0 + u < topk) {
#pragma unroll
          for (int i = 0; i < 8; i++) acc[i] += bf2f(v[u][i]);
        }
    }
    if (shared) {
      const v8u16 sv = *reinterpret_cast<const v8u16*>(shared + (size_t)m * ld_shared + c);
#pragma unroll
      for (int i = 0; i < 8; i++) acc[i] += bf2f(sv[i]);
    }
    v8u16 o;
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = f2bf(acc[i]);
    *reinterpret_cast<v8u16*>(out + (size_t)m * ld_out + c) = o;
  }
}

}  // namespace

// Reference: kernels/r9k_moe_sum.hip:62-69 (same arguments and meaning). down [M, topk, N] bf16 contiguous; shared
// [M, N] with row stride ld_shared (0 pointer = none); out [M, N] with row stride ld_out. N % 8 == 0, 16-byte
// aligned rows. Returns 0 on success, 1 for an unsupported shape, else the HIP error code.
extern "C" int r9k_moe_sum(long down, long shared, long out, int M, int topk, int N, long ld_shared, long ld_out,
                           long stream) {
  if (M < 1 || topk < 1 || N < 8 || (N & 7)) return 1;
  if ((down & 15) || (out & 15) || (ld_out & 7) || (shared && ((shared & 15) || (ld_shared & 7)))) return 1;
  const long items = (long)M * ((N + SEG - 1) / SEG);
  const long want = (items + SUM_WAVES - 1) / SUM_WAVES;
  const int grid = (int)(want < MAX_WG ? want : MAX_WG);
  // non-temporal loads of the routed rows once they are far larger than the L2s (config 3: 268 MB)
  if ((size_t)M * (size_t)topk * (size_t)N * 2u >= NT_STREAM_BYTES)
    hipLaunchKernelGGL(moe_sum_kernel<true>, dim3(grid), dim3(SUM_WAVES * WAVE), 0, (hipStream_t)stream,
                       (const uint16_t*)down, (const uint16_t*)shared, (uint16_t*)out, M, topk, N, ld_shared, ld_out);
  else
    hipLaunchKernelGGL(moe_sum_kernel<false>, dim3(grid), dim3(SUM_WAVES * WAVE), 0, (hipStream_t)stream,
                       (const uint16_t*)down, (const uint16_t*)shared, (uint16_t*)out, M, topk, N, ld_shared, ld_out);
  return (int)hipGetLastError();
}
