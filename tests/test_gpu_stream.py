"""GPU parity of the block-stream decode GEMMs (r9k_moe_stream, csrc/r9k_moe_stream.hip).

* Plain product (epi 0) against the tile kernel's single-wave launch (r9k_moe_mxfp4a8 at R9K_GEMM_SK=1: the same
  operand layout and the same MFMA chain, K-tiles ascending into one accumulator): bit-equal bf16 outputs, with and
  without the router weight, on config 2's gate_up and down shapes and odd ones.
* gate_up with SiLU + fp8 quant in the epilogue (epi 1) against that product followed by r9k_silu_mul_quant_fp8:
  bit-equal codes and row scales (the SiLU kernel's silu_mul, row maximum and e4m3 encoder).
* Expert-map holes (expert -1 blocks) are skipped, as the tile kernel skips them.
* Every launch shape the dispatcher offers (R9K_STREAM_TG / _U / _SLICES) gives the same bits.
* The layer at config 2 T = 48 / 64 through r9k_moe_stream_layer against the oracle (tolerance), and equal to the
  tile-kernel layer to fp32 rounding.
* r9k_moe_stream_layer (gate_up, SiLU + quant and down of a block in one workgroup) bit-equal to the three single-wave
  launches it replaces."""
import numpy as np
import pytest
import torch

from r9700_vllm.kernels import moe as K
from r9700_vllm.moe.experts import R9700Mxfp4Experts

from test_gpu_gemm_layer import make_layer, run_layer

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda", 0)


def _routed(dev, E, T, H, topk, seed, expert_map=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    logits = torch.randn(T, E, generator=g).to(torch.bfloat16).to(dev)
    w, ids = K.moe_topk(logits, topk, True)
    sid, eid, ntpp = K.moe_align(ids, 16, E, expert_map)
    xq, xs = K.quant_rows_fp8(x)
    return x, w, ids, (sid, eid, ntpp), xq, xs


def _tile_sk1(monkeypatch, *args, **kw):
    monkeypatch.setenv("R9K_GEMM_SK", "1")
    try:
        return K.moe_gemm(*args, **kw)
    finally:
        monkeypatch.delenv("R9K_GEMM_SK")


@pytest.mark.parametrize("E,T,H,I,topk", [(288, 64, 2048, 512, 8), (288, 128, 2048, 512, 8), (288, 24, 2048, 512, 8),
                                          (64, 40, 1024, 256, 6), (32, 9, 512, 512, 4)])
def test_stream_equals_single_wave_tile_kernel(dev, monkeypatch, E, T, H, I, topk):
    seed = 20261201 + 31000 + E + T + H + I
    _, _, W13, W2 = make_layer(dev, E, H, I, seed)
    x, w, ids, (sid, eid, ntpp), xq, xs = _routed(dev, E, T, H, topk, seed + 1)
    numel = T * topk
    tw = w.reshape(-1).float().contiguous()
    # gate_up shape, no router weight
    ref = torch.empty(numel, 2 * I, dtype=torch.bfloat16, device=dev)
    _tile_sk1(monkeypatch, xq, xs, W13, ref, sid, eid, ntpp, numel, topk, None, num_experts=E, MT=1)
    got = torch.full_like(ref, float("nan"))
    assert K.moe_stream(xq, xs, W13, got, sid, eid, ntpp, numel, topk, None, E)
    # down shape with the router weight, on the quantised gate_up rows
    aq, as_ = K.silu_mul_quant_fp8(ref)
    dref = torch.empty(numel, H, dtype=torch.bfloat16, device=dev)
    _tile_sk1(monkeypatch, aq, as_, W2, dref, sid, eid, ntpp, numel, 1, tw, num_experts=E, MT=1)
    dgot = torch.full_like(dref, float("nan"))
    assert K.moe_stream(aq, as_, W2, dgot, sid, eid, ntpp, numel, 1, tw, E)
    torch.cuda.synchronize()
    eq1 = torch.equal(got.view(torch.int16), ref.view(torch.int16))
    eq2 = torch.equal(dgot.view(torch.int16), dref.view(torch.int16))
    print(f"stream E={E} T={T} H={H} I={I} k={topk}: gate_up bit-equal {eq1}, down bit-equal {eq2}", flush=True)
    assert eq1 and eq2


@pytest.mark.parametrize("E,T,H,I,topk", [(288, 64, 2048, 512, 8), (288, 256, 2048, 512, 8), (288, 33, 2048, 512, 8),
                                          (64, 40, 1024, 256, 6), (16, 3, 256, 512, 2)])
def test_stream_gate_up_silu_quant_equals_two_launches(dev, monkeypatch, E, T, H, I, topk):
    seed = 20261201 + 32000 + E + T + H + I
    _, _, W13, _ = make_layer(dev, E, H, I, seed)
    x, w, ids, (sid, eid, ntpp), xq, xs = _routed(dev, E, T, H, topk, seed + 1)
    numel = T * topk
    gu = torch.empty(numel, 2 * I, dtype=torch.bfloat16, device=dev)
    _tile_sk1(monkeypatch, xq, xs, W13, gu, sid, eid, ntpp, numel, topk, None, num_experts=E, MT=1)
    qref, sref = K.silu_mul_quant_fp8(gu)
    q = torch.zeros(numel, I, dtype=torch.float8_e4m3fn, device=dev)
    s = torch.full((numel,), float("nan"), dtype=torch.float32, device=dev)
    assert K.moe_stream(xq, xs, W13, q, sid, eid, ntpp, numel, topk, None, E, out_scale=s)
    torch.cuda.synchronize()
    codes = torch.equal(q.view(torch.uint8), qref.view(torch.uint8))
    scales = torch.equal(s.view(torch.int32), sref.view(torch.int32))
    print(f"stream gate_up+silu E={E} T={T} H={H} I={I}: codes {codes} scales {scales}", flush=True)
    assert codes and scales


def test_stream_skips_expert_map_holes(dev, monkeypatch):
    """Experts mapped to -1 (another rank's) produce no rows; the rest equal the tile kernel."""
    E, T, H, I, topk = 64, 48, 1024, 512, 8
    seed = 20261201 + 33000
    _, _, W13, W2 = make_layer(dev, E, H, I, seed)
    emap = torch.arange(E, dtype=torch.int32, device=dev)
    emap[1::3] = -1
    x, w, ids, (sid, eid, ntpp), xq, xs = _routed(dev, E, T, H, topk, seed + 1, expert_map=emap)
    numel = T * topk
    sentinel = -12345.0
    ref = torch.full((numel, 2 * I), sentinel, dtype=torch.bfloat16, device=dev)
    _tile_sk1(monkeypatch, xq, xs, W13, ref, sid, eid, ntpp, numel, topk, None, num_experts=E, MT=1)
    got = torch.full_like(ref, sentinel)
    assert K.moe_stream(xq, xs, W13, got, sid, eid, ntpp, numel, topk, None, E)
    torch.cuda.synchronize()
    foreign = (emap[ids.reshape(-1).long()] < 0)
    assert foreign.any() and (~foreign).any()
    assert torch.all(got[foreign] == sentinel), "a row of a foreign expert was written"
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("tg,u,slices", [(1, 1, 1), (1, 4, 2), (2, 2, 1), (2, 1, 4), (4, 1, 2), (1, 2, 4)])
def test_stream_launch_shapes_agree(dev, monkeypatch, tg, u, slices):
    """Every plain launch shape the dispatcher offers (column tiles a unit, K-tiles a load batch, column slices)
    gives the same bits (down shape of config 2, T = 64)."""
    E, T, H, I, topk = 288, 64, 2048, 512, 8
    seed = 20261201 + 34000
    _, _, _, W2 = make_layer(dev, E, H, I, seed)
    g = torch.Generator().manual_seed(seed + 2)
    _, w, ids, (sid, eid, ntpp), _, _ = _routed(dev, E, T, H, topk, seed + 1)
    numel = T * topk
    h = (torch.randn(numel, I, generator=g) * 2).to(torch.bfloat16).to(dev)
    aq, as_ = K.quant_rows_fp8(h)
    tw = w.reshape(-1).float().contiguous()
    ref = torch.empty(numel, H, dtype=torch.bfloat16, device=dev)
    assert K.moe_stream(aq, as_, W2, ref, sid, eid, ntpp, numel, 1, tw, E)
    monkeypatch.setenv("R9K_STREAM_TG", str(tg))
    monkeypatch.setenv("R9K_STREAM_U", str(u))
    monkeypatch.setenv("R9K_STREAM_SLICES", str(slices))
    got = torch.full_like(ref, float("nan"))
    assert K.moe_stream(aq, as_, W2, got, sid, eid, ntpp, numel, 1, tw, E)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("T", [48, 64])
def test_layer_through_streams(dev, monkeypatch, T):
    """The config 2 layer at decode widths that take r9k_moe_stream_layer: against the oracle (tolerance), and
    against the same layer on the tile kernels (R9K_STREAM off) to fp32-accumulation-order rounding."""
    assert K.stream_wanted(T * 8, 288, 8) and not K.down_sum_fits(T * 8, 2048, 512)
    run_layer(dev, 288, 2048, 512, T, 8, seed=20261201 + 35000 + T)
    seed = 20261201 + 36000 + T
    _, _, W13, W2 = make_layer(dev, 288, 2048, 512, seed)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(T, 2048, generator=g).to(torch.bfloat16).to(dev)
    logits = torch.randn(T, 288, generator=g).to(torch.bfloat16).to(dev)
    w, ids = K.moe_topk(logits, 8, True)
    ex = R9700Mxfp4Experts.standalone(W13.wsr, W2.wsr)
    outs = []
    for on in (True, False):
        monkeypatch.setattr(K, "STREAM", on)
        o = torch.empty(T, 2048, dtype=torch.bfloat16, device=dev)
        ex.apply(o, x, W13.wq, W2.wq, w, ids, "silu", 288, None, None, None, None, None, None, False)
        outs.append(o.float())
    torch.cuda.synchronize()
    rel = float((outs[0] - outs[1]).norm() / outs[1].norm())
    print(f"layer T={T}: streams vs tile kernels rel {rel:.2e}", flush=True)
    assert rel < 1e-2


@pytest.mark.parametrize("E,T,H,I,topk", [(288, 64, 2048, 512, 8), (288, 40, 2048, 512, 8), (64, 40, 1024, 256, 6),
                                          (16, 3, 256, 512, 2), (32, 17, 512, 1024, 4)])
def test_stream_layer_equals_three_launches(dev, monkeypatch, E, T, H, I, topk):
    """r9k_moe_stream_layer (gate_up, SiLU + quant and down of each block in one workgroup) against the tile
    kernel's single-wave gate_up, r9k_silu_mul_quant_fp8 and the single-wave down with the router weight: bit-equal
    down rows."""
    seed = 20261201 + 37000 + E + T + H + I
    _, _, W13, W2 = make_layer(dev, E, H, I, seed)
    x, w, ids, (sid, eid, ntpp), xq, xs = _routed(dev, E, T, H, topk, seed + 1)
    numel = T * topk
    tw = w.reshape(-1).float().contiguous()
    gu = torch.empty(numel, 2 * I, dtype=torch.bfloat16, device=dev)
    _tile_sk1(monkeypatch, xq, xs, W13, gu, sid, eid, ntpp, numel, topk, None, num_experts=E, MT=1)
    aq, as_ = K.silu_mul_quant_fp8(gu)
    ref = torch.empty(numel, H, dtype=torch.bfloat16, device=dev)
    _tile_sk1(monkeypatch, aq, as_, W2, ref, sid, eid, ntpp, numel, 1, tw, num_experts=E, MT=1)
    got = torch.full_like(ref, float("nan"))
    assert K.moe_stream_layer(xq, xs, W13, W2, got, sid, eid, ntpp, numel, topk, tw, E)
    torch.cuda.synchronize()
    same = torch.equal(got.view(torch.int16), ref.view(torch.int16))
    print(f"stream layer E={E} T={T} H={H} I={I} k={topk}: bit-equal {same}", flush=True)
    assert same
