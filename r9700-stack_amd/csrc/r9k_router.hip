// r9k_router.hip -- MoE router (gate) GEMM at decode widths on gfx950:
//   out[m, e] = x[m, :] . w[e, :]  (x bf16 [M, K], w bf16 [E, K]), fp32 accumulation, rounded once to bf16 (the
//   rounding of a bf16 x bf16 -> bf16 GEMM) or stored as fp32; M <= 32.
// Reference: kernels/r9k_router.hip:120-155 (r9k_router_gemm, r9k_router_max_m): same entry, arguments, rules and
// error codes, and the same hyper-connection epilogue; the kernel is a different design for CDNA4.
//
// At M <= 32 tokens the product is a stream of the E x K weight (1-4 MB) against a few KB to 160 KB of activations:
// no matrix-core tile pays, and the launch has to keep many loads in flight over the whole chip. A workgroup owns EPT
// experts x MT tokens over all of K (grid E / EPT x M / MT, 256-4096 workgroups for the gates served); the weight rows
// come from HBM once per token tile and the activations from L2. Lane t takes the 16-byte K chunks t, t + blockDim,
// ... of its EPT weight rows and MT token rows and accumulates the EPT x MT dot products with V_DOT2C_F32_BF16 (exact
// bf16 x bf16 products, fp32 sums). A wave then transposes and sums its partials over its 64 lanes (N - 1 exchanges
// for N values), and the waves' sums meet in LDS in wave order: the summation order is fixed by the launch shape, so
// repeated calls give identical bits. Token rows past M are clamped to the last row for the loads and never stored,
// as are expert rows past E.
// act_cols > 0 applies the hyper-connection epilogue (reference kernels/r9k_router.hip:34-40) to the first act_cols
// columns: s = bf16(v) / hc, out = s / (1 + exp(-s)).
#include "r9k_common.h"
#include "r9k_router_tile.h"

namespace {

using namespace r9k;

constexpr int ROUTER_MAX_M = 32;
constexpr int ROUTER_MAX_WAVES = 8;

template <int EPT, int MT, bool BF>
__global__ void __launch_bounds__(ROUTER_MAX_WAVES * WAVE) router_rows_kernel(const uint16_t* __restrict__ x, long sx,
                                                                              const uint16_t* __restrict__ w, long sw,
                                                                              void* __restrict__ out, long so, int M,
                                                                              int E, int K, int act_cols, float hc) {
  constexpr int N = EPT * MT;
  __shared__ float part[ROUTER_MAX_WAVES][N];
  const int tid = threadIdx.x, nw = blockDim.x / WAVE;
  const int e0 = blockIdx.x * EPT, m0 = blockIdx.y * MT;
  float v = router_tile<EPT, MT>(x, sx, w, sw, M, E, K, e0, m0, nw, part);
  if (tid >= N) return;
  const int e = e0 + tid / MT, m = m0 + tid % MT;
  if (e >= E || m >= M) return;
  if (e < act_cols) {
    const float sv = bf2f(f2bf(v)) / hc;
    v = sv / (1.f + __expf(-sv));
  }
  if constexpr (BF) reinterpret_cast<uint16_t*>(out)[(long)m * so + e] = f2bf(v);
  else reinterpret_cast<float*>(out)[(long)m * so + e] = v;
}

struct RouterArgs {
  const uint16_t* x;
  long sx;
  const uint16_t* w;
  long sw;
  void* out;
  long so;
  int M, E, K, act_cols;
  float hc;
};

template <int EPT, int MT>
void launch_shape(const RouterArgs& a, bool bf, int nw, hipStream_t st) {
  const dim3 grid((a.E + EPT - 1) / EPT, (a.M + MT - 1) / MT), block(nw * WAVE);
  if (bf)
    hipLaunchKernelGGL((router_rows_kernel<EPT, MT, true>), grid, block, 0, st, a.x, a.sx, a.w, a.sw, a.out, a.so,
                       a.M, a.E, a.K, a.act_cols, a.hc);
  else
    hipLaunchKernelGGL((router_rows_kernel<EPT, MT, false>), grid, block, 0, st, a.x, a.sx, a.w, a.sw, a.out, a.so,
                       a.M, a.E, a.K, a.act_cols, a.hc);
}

// Launch with EPT experts and MT tokens a workgroup (grid E / EPT x M / MT) and nw waves (1..8); the shapes
// router_shape picks are the ones instantiated.
int router_launch(const RouterArgs& a, bool bf, int ept, int mt, int nw, hipStream_t st) {
  if (nw < 1 || nw > ROUTER_MAX_WAVES) return -5;
  switch (ept * 100 + mt) {
    case 101: launch_shape<1, 1>(a, bf, nw, st); return 0;
    case 102: launch_shape<1, 2>(a, bf, nw, st); return 0;
    case 202: launch_shape<2, 2>(a, bf, nw, st); return 0;
    case 204: launch_shape<2, 4>(a, bf, nw, st); return 0;
    default: return -5;
  }
}

}  // namespace

// out[M, E] (row stride so elements; bf16 when out_bf16 else fp32) = x[M, K] bf16 (row stride sx elements) .
// w[E, K]^T bf16 (row stride sw). act_cols > 0: the hyper-connection epilogue on the first act_cols columns.
// Rules (the reference's): 1 <= M <= 32, split in {1, 2, 4, 8}, K % (8 * split) == 0, row strides multiples of 8
// elements with x and w 16-byte aligned. `split` (the reference's waves per expert) only gates the K rule here: the
// launch shape is this kernel's own. 0, or -1 M / E / K, -2 split, -3 K % (8 split), -4 strides or alignment,
// -7 act_cols with hc <= 0, -6 launch error.
extern "C" int r9k_router_gemm(long x, long sx, long w, long sw, long out, long so, int M, int E, int K, int split,
                               int out_bf16, int act_cols, float hc, long stream) {
  if (M < 1 || M > ROUTER_MAX_M || E < 1 || K < 8) return -1;
  if (split < 1 || split > 8 || (split & (split - 1))) return -2;
  if (K % (8 * split)) return -3;
  if (((sx | sw) & 7) || ((x | w) & 15)) return -4;
  if (act_cols > 0 && hc <= 0.f) return -7;
  RouterArgs a{(const uint16_t*)x, sx, (const uint16_t*)w, sw, (void*)out, so, M, E, K, act_cols, hc};
  int ept, mt, nw;
  router_shape(M, K, &ept, &mt, &nw);
  if (router_launch(a, out_bf16 != 0, ept, mt, nw, (hipStream_t)stream)) return -6;
  return hipGetLastError() == hipSuccess ? 0 : -6;
}

// Largest M the kernel takes. Replaces kernels/r9k_router.hip:155.
extern "C" int r9k_router_max_m(void) { return ROUTER_MAX_M; }
