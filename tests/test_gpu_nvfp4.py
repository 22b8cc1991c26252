"""GPU parity of the native NVFP4 path (f3): r9k_moe_nvfp4a8 through kernels/moe.moe_gemm, ops.nvfp4_linear and a
whole MoE layer on native NVFP4 experts (R9700Mxfp4Experts with nv multipliers), against the oracle's exact NVFP4
GEMM (e2m1 x e4m3 weights in fp64, the multiplier and row scale in the kernel's epilogue order).

Held to what fp32 accumulation order can explain (rel <= 2e-3, cosine >= 0.99999 per GEMM) and the north-star layer
tolerance (rel <= 1e-2, cosine >= 0.9999); routing ids bit-exact."""
import numpy as np
import pytest
import torch

from helpers import bf16_bits_to_f64, cosine, rel_err
from oracle import oracle as O
from r9700_vllm import ops
from r9700_vllm.kernels import moe as K
from r9700_vllm.moe.experts import R9700Mxfp4Experts

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda", 0)


def make_nv(E, N, Kd, g):
    """Uniform e2m1 codes, s16 = e4m3(|N(0,1)| * 0.05) (subnormal and zero scales included), multipliers in
    [0.5, 2): the config 4 recipe per expert."""
    packed = torch.randint(0, 256, (E, N, Kd // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    s16 = (torch.randn(E, N, Kd // 16, generator=g).abs() * 0.05).to(torch.float8_e4m3fn)
    wg = torch.rand(E, N, generator=g) * 1.5 + 0.5
    return packed, s16, wg


def check(got_bits, ref_bits, tol=2e-3, cos=0.99999):
    a, b = bf16_bits_to_f64(got_bits), bf16_bits_to_f64(ref_bits)
    assert not np.isnan(a.numpy()).any(), "a routed row was not written"
    r, c = rel_err(a, b), cosine(a, b)
    assert r < tol and c > cos, (r, c)
    return r, c


@pytest.mark.parametrize("E,M,topk,N,Kd,MT,down", [
    (8, 4, 2, 64, 256, 1, False), (16, 8, 4, 96, 2064, 1, False), (32, 64, 8, 512, 2048, 1, False),
    (32, 64, 8, 2048, 512, 1, True), (8, 40, 2, 48, 384, 2, False), (8, 100, 2, 128, 784, 4, True),
    (4, 3, 1, 16, 16, 1, False),
])
def test_nvfp4_grouped_gemm(dev, E, M, topk, N, Kd, MT, down):
    print(f"nvfp4 gemm E={E} M={M} topk={topk} N={N} K={Kd} MT={MT} down={down}", flush=True)
    g = torch.Generator().manual_seed(E * 7 + M + N + Kd)
    packed, s16, wg = make_nv(E, N, Kd, g)
    W = K.prepare_nvfp4_weights(packed.to(dev), s16.to(dev), wg.to(dev))
    numel = M * topk
    rows_a = numel if down else M
    x = (torch.randn(rows_a, Kd, generator=g) * 0.5).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:topk] for _ in range(M)]).to(torch.int32)
    tw = torch.rand(numel, generator=g).float() if down else None
    sid, eid, ntpp = (t.to(dev) for t in K.align_block_size_ref(ids, E, 16 * MT))
    xq, xs = K.quant_rows_fp8(x.to(dev))
    out = torch.full((numel, N), float("nan"), dtype=torch.bfloat16, device=dev)
    K.moe_gemm(xq, xs, W, out, sid, eid, ntpp, numel, 1 if down else topk, tw.to(dev) if down else None,
               num_experts=E, MT=MT)
    qo, so = O.quant_rows_fp8(x)
    ref = O.nvfp4_gemm(qo, so, packed.numpy(), s16.view(torch.uint8).numpy(), wg.numpy(),
                       ids.reshape(-1).numpy(), 1 if down else topk, tw.numpy() if down else None)
    r, c = check(O.bf16_bits(out), ref)
    print(f"  rel {r:.2e} cos {c:.7f}", flush=True)


@pytest.mark.parametrize("E,M,topk,N,Kd,cfg,down", [
    (8, 200, 2, 256, 512, 2, False), (16, 300, 4, 384, 2080, 12, False), (32, 512, 8, 2048, 512, 12, True),
    (4, 64, 1, 48, 256, 2, False), (8, 700, 8, 1024, 2048, 12, False),
])
def test_nvfp4_grouped_gemm_prefill(dev, E, M, topk, N, Kd, cfg, down):
    """The prefill entry's native-NVFP4 tile kernel (r9k_moe_4bit_prefill nv = 1) on 128- (cfg 2) and 256-row (cfg 12)
    routing blocks: a K tail (K % 128 = 32), N not a multiple of the 128-column tile, the router-weighted down."""
    print(f"nvfp4 prefill gemm E={E} M={M} topk={topk} N={N} K={Kd} cfg={cfg} down={down}", flush=True)
    g = torch.Generator().manual_seed(E * 11 + M + N + Kd)
    packed, s16, wg = make_nv(E, N, Kd, g)
    W = K.prepare_nvfp4_weights(packed.to(dev), s16.to(dev), wg.to(dev))
    numel = M * topk
    rows_a = numel if down else M
    x = (torch.randn(rows_a, Kd, generator=g) * 0.5).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:topk] for _ in range(M)]).to(torch.int32)
    tw = torch.rand(numel, generator=g).float() if down else None
    sid, eid, ntpp = (t.to(dev) for t in K.align_block_size_ref(ids, E, K.prefill_block(cfg)))
    xq, xs = K.quant_rows_fp8(x.to(dev))
    out = torch.full((numel, N), float("nan"), dtype=torch.bfloat16, device=dev)
    K.moe_gemm(xq, xs, W, out, sid, eid, ntpp, numel, 1 if down else topk, tw.to(dev) if down else None,
               num_experts=E, prefill=cfg)
    qo, so = O.quant_rows_fp8(x)
    ref = O.nvfp4_gemm(qo, so, packed.numpy(), s16.view(torch.uint8).numpy(), wg.numpy(),
                       ids.reshape(-1).numpy(), 1 if down else topk, tw.numpy() if down else None)
    r, c = check(O.bf16_bits(out), ref)
    print(f"  rel {r:.2e} cos {c:.7f}", flush=True)


@pytest.mark.parametrize("M,N,Kd", [(1, 1024, 2048), (16, 512, 5120), (300, 256, 1024), (1, 17408, 5120),
                                    (1000, 512, 1024)])
def test_nvfp4_linear(dev, M, N, Kd):
    print(f"nvfp4 linear M={M} N={N} K={Kd}", flush=True)
    g = torch.Generator().manual_seed(M + N + Kd)
    packed, s16, wg = make_nv(1, N, Kd, g)
    W = K.prepare_nvfp4_weights(packed.to(dev), s16.to(dev), wg.to(dev))
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    out = ops.nvfp4_linear(x.to(dev), W.wq, W.ws, W.wg, N, Kd)
    qo, so = O.quant_rows_fp8(x)
    ref = O.nvfp4_gemm(qo, so, packed.numpy(), s16.view(torch.uint8).numpy(), wg.numpy(),
                       np.zeros(M, dtype=np.int32), 1)
    check(O.bf16_bits(out), ref)


@pytest.mark.parametrize("M,N,Kd", [(1, 17408, 5120), (2, 17408, 5120), (1, 1024, 2048), (2, 48, 1024),
                                    (1, 272, 384), (2, 64, 8192), (1, 16, 896), (2, 2064, 640)])
def test_dense_nvfp4_qa_equals_two_launches(dev, M, N, Kd):
    """r9k_dense_nvfp4_qa (the activation quant inside the native NVFP4 GEMM launch, M <= 2) against quant_rows_fp8 +
    the decode kernel over identity tables: bit for bit, every output written, and within the GEMM tolerance of the
    oracle."""
    print(f"dense nvfp4 qa M={M} N={N} K={Kd}", flush=True)
    g = torch.Generator().manual_seed(20261201 + 4300 + M + N + Kd)
    packed, s16, wg = make_nv(1, N, Kd, g)
    W = K.prepare_nvfp4_weights(packed.to(dev), s16.to(dev), wg.to(dev))
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    xd = x.to(dev)
    one = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    assert K.dense_nvfp4_qa(xd, W, one), "shape not served"
    q, s = K.quant_rows_fp8(xd)
    two = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    tabs = ops.IdentityTables.get(dev, M, K.MOE_BLOCK)
    K.moe_gemm(q, s, W, two, *tabs, M, 1, None, num_experts=1, MT=1)
    torch.cuda.synchronize()
    assert torch.equal(one.view(torch.int16), two.view(torch.int16))
    qo, so = O.quant_rows_fp8(x)
    ref = O.nvfp4_gemm(qo, so, packed.numpy(), s16.view(torch.uint8).numpy(), wg.numpy(),
                       np.zeros(M, dtype=np.int32), 1)
    check(O.bf16_bits(one), ref)


def test_dense_nvfp4_qa_refuses_unserved(dev):
    """M > 2 or K not a multiple of 128: False, nothing launched (ops falls back to the two launches)."""
    g = torch.Generator().manual_seed(7)
    packed, s16, wg = make_nv(1, 64, 256, g)
    W = K.prepare_nvfp4_weights(packed.to(dev), s16.to(dev), wg.to(dev))
    assert not K.dense_nvfp4_qa(torch.zeros(3, 256, dtype=torch.bfloat16, device=dev), W,
                                torch.empty(3, 64, dtype=torch.bfloat16, device=dev))
    packed, s16, wg = make_nv(1, 64, 272, g)
    W2 = K.prepare_nvfp4_weights(packed.to(dev), s16.to(dev), wg.to(dev))
    assert not K.dense_nvfp4_qa(torch.zeros(1, 272, dtype=torch.bfloat16, device=dev), W2,
                                torch.empty(1, 64, dtype=torch.bfloat16, device=dev))


def test_nvfp4_linear_config4_prefill_sampled(dev):
    """BASELINE config 4's shape at M = 4096 on native NVFP4 weights (the 128 x 128 tile kernel), checked on 48
    sampled rows (rows are independent)."""
    M, N, Kd = 4096, 17408, 5120
    print("nvfp4 linear config 4 M=4096", flush=True)
    g = torch.Generator().manual_seed(4097)
    packed, s16, wg = make_nv(1, N, Kd, g)
    W = K.prepare_nvfp4_weights(packed.to(dev), s16.to(dev), wg.to(dev))
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    out = ops.nvfp4_linear(x.to(dev), W.wq, W.ws, W.wg, N, Kd)
    rows = np.sort(np.random.default_rng(1).choice(M, 48, replace=False))
    qo, so = O.quant_rows_fp8(x)
    ref = O.nvfp4_gemm(qo, so, packed.numpy(), s16.view(torch.uint8).numpy(), wg.numpy(),
                       np.zeros(M, dtype=np.int32), 1, rows=rows)
    check(O.bf16_bits(out)[rows], ref)


@pytest.mark.parametrize("T", [1, 16, 64, 300, 1024])
def test_nvfp4_native_layer(dev, T):
    """Config 2's layer shape (E=288, hidden 2048, I 512, top-8) on native NVFP4 experts through
    R9700Mxfp4Experts.apply, against the oracle chain: route -> fp8 quant -> NVFP4 gate_up -> SiLU quant -> NVFP4
    down (router weight folded) -> top-k sum."""
    E, H, I, topk = 288, 2048, 512, 8
    print(f"nvfp4 layer T={T}", flush=True)
    g = torch.Generator().manual_seed(20261201 + 3 + T)
    p13, s13, g13 = make_nv(E, 2 * I, H, g)
    p2, s2, g2 = make_nv(E, H, I, g)
    W13 = K.prepare_nvfp4_weights(p13.to(dev), s13.to(dev), g13.to(dev))
    W2 = K.prepare_nvfp4_weights(p2.to(dev), s2.to(dev), g2.to(dev))
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g).to(torch.bfloat16)
    w, ids = K.moe_topk(logits.to(dev), topk, True)
    ex = R9700Mxfp4Experts.standalone(W13.ws, W2.ws, nv=(W13.wg, W2.wg))
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    ex.apply(out, x.to(dev), W13.wq, W2.wq, w, ids, "silu", E, None, None, None, None, None, None, False)
    torch.cuda.synchronize()
    rw, rids = O.route(logits, topk, True)
    assert np.array_equal(ids.cpu().numpy(), rids), "routing ids"
    flat = rids.reshape(-1)
    xq, xs = O.quant_rows_fp8(x)
    gu = O.nvfp4_gemm(xq, xs, p13.numpy(), s13.view(torch.uint8).numpy(), g13.numpy(), flat, topk)
    aq, a_s, _ = O.silu_mul_quant_fp8(O.bits_to_bf16(gu))
    dn = O.nvfp4_gemm(aq, a_s, p2.numpy(), s2.view(torch.uint8).numpy(), g2.numpy(), flat, 1,
                      rw.reshape(-1).astype(np.float32))
    ref = O.moe_sum(O.bits_to_bf16(dn.reshape(T, topk, H)))
    r, c = check(O.bf16_bits(out), ref, tol=1e-2, cos=0.9999)
    print(f"  rel {r:.2e} cos {c:.7f}", flush=True)
