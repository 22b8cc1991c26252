"""GPU parity of the router (gate) GEMM, r9k_router_gemm through router.router_gemm, against the fp64 product of the
oracle (the reference's own criterion, tests/test_router_r9k.py:50-65: ours within 1.5x of stock's bf16 error and
2x of torch's fp32-out error, bf16 results differing from stock's F.linear only where summation order moves a
rounding).

Exact checks on top: the bf16 output is the fp32 output rounded once (one kernel, one summation order); the fp32
error stays under the worst-case bound of fp32 summation, K * 2^-24 * sum |x_k w_k|; the hc_silu epilogue leaves
columns >= act_cols bit-identical and matches the oracle's epilogue within fp32 exp error on the rest."""
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O
from r9700_vllm import router as R

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def operands(M, E, K, seed, stride_pad=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K + stride_pad, generator=g).to(torch.bfloat16).to(DEV)[:, :K]
    w = (torch.randn(E, K, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    return x, w


def fp32_bound(x, w):
    K = x.shape[1]
    return K * 2.0 ** -24 * (x.abs().double().cpu() @ w.abs().double().cpu().t())


@pytest.mark.parametrize("M,E,K,split,pad", [
    (1, 512, 2560, 2, 0), (8, 512, 2560, 1, 0), (32, 512, 2560, 8, 0), (13, 500, 2560, 4, 0), (3, 512, 2560, 2, 64),
    (5, 288, 2048, 1, 0), (16, 300, 2056, 1, 0), (32, 1, 8, 1, 0), (2, 64, 4096, 2, 8), (7, 33, 24, 1, 0),
    (24, 257, 7168, 1, 0), (31, 256, 7168, 2, 0), (4, 511, 4096, 4, 0), (11, 3, 1032, 1, 0),
])
def test_router_gemm_vs_fp64(M, E, K, split, pad):
    print(f"router M={M} E={E} K={K} split={split} pad={pad}", flush=True)
    x, w = operands(M, E, K, seed=M * 1000 + E, stride_pad=pad)
    assert R._takes(x, w, split, None)
    ref = O.router_gemm(x, w)
    o_bf = R.router_gemm(x, w, True, split=split)
    assert torch.equal(o_bf, R.router_gemm(x, w, True, split=split))     # fixed summation order: same bits
    o_32 = R.router_gemm(x, w, False, split=split)
    stock = F.linear(x, w)
    t_32 = torch.mm(x.float(), w.float().t())
    torch.cuda.synchronize()
    assert o_bf.dtype == torch.bfloat16 and o_32.dtype == torch.float32 and o_bf.shape == (M, E)
    assert torch.equal(o_bf, o_32.to(torch.bfloat16))                   # rounded once from the same fp32 sum
    err32 = (o_32.double().cpu() - ref).abs()
    assert bool((err32 <= fp32_bound(x, w) + 1e-30).all())
    e = dict(o=(o_bf.double().cpu() - ref).abs().max().item(), s=(stock.double().cpu() - ref).abs().max().item(),
             o32=err32.max().item(), t=(t_32.double().cpu() - ref).abs().max().item())
    assert e["o"] <= 1.5 * e["s"] + 1e-6, e
    assert e["o32"] <= 2.0 * e["t"] + 1e-7, e
    flips = (o_bf != stock).sum().item()
    assert flips <= max(2, int(o_bf.numel() * 2e-3)), flips


@pytest.mark.parametrize("M,E,K,act,hc", [(4, 336, 2560, 320, 1.5), (32, 512, 2048, 512, 0.75), (1, 40, 64, 7, 3.0)])
def test_router_gemm_hc_epilogue(M, E, K, act, hc):
    print(f"router hc M={M} E={E} K={K} act={act} hc={hc}", flush=True)
    x, w = operands(M, E, K, seed=7 + M)
    v32 = R.router_gemm(x, w, False)
    plain_bf = R.router_gemm(x, w, True)
    a_bf = R.router_gemm(x, w, True, act_cols=act, hc=hc)
    a_32 = R.router_gemm(x, w, False, act_cols=act, hc=hc)
    torch.cuda.synchronize()
    assert torch.equal(a_bf[:, act:], plain_bf[:, act:]) and torch.equal(a_32[:, act:], v32[:, act:])
    exp = O.hc_silu(v32, act, hc)[:, :act]
    assert torch.allclose(a_32[:, :act].double().cpu(), exp, rtol=1e-5, atol=1e-7)
    # bf16: the rounding of a value within fp32-exp error of the oracle's, so at most one bf16 step away
    got = a_bf[:, :act].double().cpu()
    step = torch.exp2(torch.floor(torch.log2(exp.abs().clamp_min(1e-30)))) * 2.0 ** -7
    assert bool(((got - exp).abs() <= step).all())


def test_router_gemm_fallbacks():
    print("router fallbacks", flush=True)
    x, w = operands(33, 512, 2560, seed=5)
    assert torch.equal(R.router_gemm(x, w, True), F.linear(x, w))       # above the tile height: torch's bf16 GEMM
    assert R.router_gemm(x, w, True, act_cols=8, hc=1.0) is None        # the epilogue is the caller's there
    x1, w1 = operands(4, 64, 72, seed=6)
    assert not R._takes(x1, w1, 2, None)                                 # K % (8 split)
    assert torch.equal(R.router_gemm(x1, w1, True, split=2), F.linear(x1, w1))
    assert R.router_gemm(x1[:2], w1, True, split=1, max_m=1).shape == (2, 64)   # row cap -> torch
