"""GPU parity of the load path: checkpoint tensors on a dummy layer object go through the same vLLM-free functions
the quant methods call after loading (moe/prep.prepare_layer_mxfp4, quant/nvfp4.convert_moe_layer /
prep_native_moe / convert_dense_layer / prepare_native_dense_layer / mxfp4_linearize, linear/mxfp4.prep_dense), and
the layer they leave is run and checked against the oracle on the original checkpoint bits -- the reference's
dummy-layer tests of process_weights_after_loading (tests/test_nvfp4.py:134-151 there).

In-place preparation is checked as such: the prepared expert codes live in the checkpoint tensor's own storage.
Converted codes and exponents are bit-exact against the oracle converter; layer outputs are held to the north-star
tolerance (norm ratio <= 1e-2, cosine >= 0.9999), dense outputs to the GEMM tolerance (rel <= 2e-3)."""
import numpy as np
import pytest
import torch

from helpers import bf16_bits_to_f64, cosine, make_experts, rel_err
from oracle import oracle as O
from r9700_vllm.kernels import moe as K
from r9700_vllm.linear import mxfp4 as LX
from r9700_vllm.moe import prep
from r9700_vllm.moe.experts import R9700Mxfp4Experts
from r9700_vllm.quant import nvfp4 as NV

pytestmark = pytest.mark.gpu

P = lambda t: torch.nn.Parameter(t, requires_grad=False)


class _Lazy:
    def __init__(self, d):
        self.d = d

    def __getitem__(self, e):
        return self.d[int(e)]


def _nvfp4_ckpt(E, N, Kd, g, shards):
    """NVFP4 checkpoint tensors of E experts [N, Kd]: codes, e4m3 per-16 scales, global divisors per shard."""
    packed = torch.randint(0, 256, (E, N, Kd // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    s16 = (torch.randn(E, N, Kd // 16, generator=g).abs() * 0.05).to(torch.float8_e4m3fn)
    gsc = torch.rand(E, shards, generator=g) * 3 + 0.5
    return packed, s16, gsc


def _run_layer(dev, layer, E, H, I, T, topk, seed, nv=None):
    """Route T tokens, run the prepared layer through R9700Mxfp4Experts (process_weights_after_loading reads the
    layer as vLLM's modular kernel would), return (x, logits, w, ids, out)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g).to(torch.bfloat16)
    w, ids = K.moe_topk(logits.to(dev), topk, True)
    ex = R9700Mxfp4Experts.standalone(layer.w13_weight_scale.data, layer.w2_weight_scale.data)
    ex.process_weights_after_loading(layer)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    ex.apply(out, x.to(dev), layer.w13_weight.data, layer.w2_weight.data, w, ids, "silu", E, None, None, None, None,
             None, None, False)
    torch.cuda.synchronize()
    return x, logits, w, ids, out


def _check(got, ref, tol=1e-2, cos=0.9999):
    a, b = bf16_bits_to_f64(got), bf16_bits_to_f64(ref)
    r, c = rel_err(a, b), cosine(a, b)
    assert r < tol and c >= cos, (r, c)
    return r, c


@pytest.mark.parametrize("chunk_bytes", [None, 300_000])
def test_mxfp4_moe_layer_prep_in_place(dev, chunk_bytes):
    """CT MXFP4 MoE tensors (w13/w2 _weight_packed [E, N, K/2], _weight_scale [E, N, K/32]) -> prepare_layer_mxfp4
    (small chunks force several staging rounds), codes kept in the checkpoint storage, the layer against the
    oracle on the checkpoint bits."""
    E, H, I, T, topk = 24, 1024, 512, 9, 4
    g = torch.Generator().manual_seed(20261201 + 12000 + (chunk_bytes or 0) % 97)
    p13, e13 = make_experts(E, 2 * I, H, g)
    p2, e2 = make_experts(E, H, I, g)
    layer = torch.nn.Module()
    layer.w13_weight_packed, layer.w13_weight_scale = P(p13.to(dev)), P(e13.to(dev))
    layer.w2_weight_packed, layer.w2_weight_scale = P(p2.to(dev)), P(e2.to(dev))
    ptr13, ptr2 = layer.w13_weight_packed.data_ptr(), layer.w2_weight_packed.data_ptr()
    prep.prepare_layer_mxfp4(layer, chunk_bytes=chunk_bytes)
    assert not hasattr(layer, "w13_weight_packed") and layer._r9k_fold == (False, False)
    assert layer.w13_weight.data_ptr() == ptr13 and layer.w2_weight.data_ptr() == ptr2, "prep was not in place"
    assert torch.equal(K.unpermute_fragments(layer.w13_weight.data, 2 * I, H).cpu(), p13)
    assert torch.equal(K.unpack_scales(layer.w2_weight_scale.data).cpu(), e2)
    x, logits, w, ids, out = _run_layer(dev, layer, E, H, I, T, topk, 12001)
    ref = O.moe_layer(x, logits, (p13, e13), (p2, e2), topk, True)
    assert np.array_equal(ids.cpu().numpy(), ref["ids"])
    r, c = _check(O.bf16_bits(out), ref["out"])
    print(f"mxfp4 prep chunk={chunk_bytes}: rel {r:.2e} cos {c:.7f}", flush=True)


def test_nvfp4_moe_layer_convert_then_prep(dev):
    """NVFP4 MoE tensors (e4m3 per-16 scales, w13 global scales per gate / up shard, w2 per expert) ->
    convert_moe_layer (codes converted in place, e8m0 exponents bit-exact against the oracle converter) ->
    prepare_layer_mxfp4 -> the layer against the oracle on the converted MXFP4 weights."""
    E, H, I, T, topk = 16, 512, 256, 7, 4
    g = torch.Generator().manual_seed(20261201 + 12100)
    p13, s13, g13 = _nvfp4_ckpt(E, 2 * I, H, g, 2)
    p2, s2, g2 = _nvfp4_ckpt(E, H, I, g, 1)
    layer = torch.nn.Module()
    layer.w13_weight_packed, layer.w13_weight_scale = P(p13.clone().to(dev)), P(s13.to(dev))
    layer.w13_weight_global_scale = P(g13.to(dev))
    layer.w2_weight_packed, layer.w2_weight_scale = P(p2.clone().to(dev)), P(s2.to(dev))
    layer.w2_weight_global_scale = P(g2.reshape(E).to(dev))
    ptr13 = layer.w13_weight_packed.data_ptr()
    NV.convert_moe_layer(layer)
    assert not hasattr(layer, "w13_weight_global_scale") and layer.w13_weight_packed.data_ptr() == ptr13
    div13 = g13.repeat_interleave(I, dim=1)
    div2 = g2.expand(E, H)
    conv = {}
    for pre, p, s, d in (("w13", p13, s13, div13), ("w2", p2, s2, div2)):
        refs = [O.nvfp4_to_mxfp4(p[e].numpy(), s[e].view(torch.uint8).numpy(), d[e].numpy()) for e in range(E)]
        cp = torch.from_numpy(np.stack([r_[0] for r_ in refs]))
        ce = torch.from_numpy(np.stack([r_[1] for r_ in refs]))
        assert torch.equal(getattr(layer, f"{pre}_weight_packed").data.cpu(), cp), pre
        assert torch.equal(getattr(layer, f"{pre}_weight_scale").data.cpu(), ce), pre
        conv[pre] = (cp, ce)
    prep.prepare_layer_mxfp4(layer)
    x, logits, w, ids, out = _run_layer(dev, layer, E, H, I, T, topk, 12101)
    ref = O.moe_layer(x, logits, conv["w13"], conv["w2"], topk, True)
    r, c = _check(O.bf16_bits(out), ref["out"])
    print(f"nvfp4 -> mxfp4 layer: rel {r:.2e} cos {c:.7f}", flush=True)


def test_nvfp4_moe_layer_native(dev):
    """NVFP4 MoE tensors -> prep_native_moe(moe_row_divisors) -> the native NVFP4 layer against the oracle's exact
    NVFP4 chain (multipliers 1 / divisor)."""
    E, H, I, T, topk = 16, 512, 256, 6, 4
    g = torch.Generator().manual_seed(20261201 + 12200)
    p13, s13, g13 = _nvfp4_ckpt(E, 2 * I, H, g, 2)
    p2, s2, g2 = _nvfp4_ckpt(E, H, I, g, 1)
    layer = torch.nn.Module()
    layer.w13_weight_packed, layer.w13_weight_scale = P(p13.to(dev)), P(s13.to(dev))
    layer.w13_weight_global_scale = P(g13.to(dev))
    layer.w2_weight_packed, layer.w2_weight_scale = P(p2.to(dev)), P(s2.to(dev))
    layer.w2_weight_global_scale = P(g2.reshape(E).to(dev))
    NV.prep_native_moe(layer, *NV.moe_row_divisors(layer))
    assert layer._r9k_nvfp4 and not hasattr(layer, "w13_weight_packed")
    x, logits, w, ids, out = _run_layer(dev, layer, E, H, I, T, topk, 12201)
    rw, rids = O.route(logits, topk, True)
    assert np.array_equal(ids.cpu().numpy(), rids)
    m13 = (1.0 / g13.repeat_interleave(I, dim=1)).float().numpy()
    m2 = (1.0 / g2.expand(E, H)).float().numpy()
    flat = rids.reshape(-1)
    xq, xs = O.quant_rows_fp8(x)
    gu = O.nvfp4_gemm(xq, xs, p13.numpy(), s13.view(torch.uint8).numpy(), m13, flat, topk)
    aq, a_s, _ = O.silu_mul_quant_fp8(O.bits_to_bf16(gu))
    dn = O.nvfp4_gemm(aq, a_s, p2.numpy(), s2.view(torch.uint8).numpy(), m2, flat, 1, rw.reshape(-1).astype(np.float32))
    ref = O.moe_sum(O.bits_to_bf16(dn.reshape(T, topk, H)))
    r, c = _check(O.bf16_bits(out), ref)
    print(f"nvfp4 native layer: rel {r:.2e} cos {c:.7f}", flush=True)


def _dense_nvfp4_layer(dev, N, Kd, g):
    packed, s16, gsc = _nvfp4_ckpt(1, N, Kd, g, 2)
    layer = torch.nn.Module()
    layer.weight_packed, layer.weight_scale = P(packed[0].to(dev)), P(s16[0].to(dev))
    layer.weight_global_scale = P(gsc[0].to(dev))
    layer.input_global_scale = P(torch.ones(2, device=dev))
    layer.logical_widths = [N // 2, N // 2]
    return layer, packed[0], s16[0], gsc[0].repeat_interleave(N // 2)


@pytest.mark.parametrize("M", [1, 5, 300])
def test_dense_nvfp4_convert_and_native(dev, M):
    """Dense NVFP4 linear with two fused shards: (a) convert_dense_layer + prep_dense (the MXFP4 dense kernel),
    converted bits exact against the oracle converter and the output against the oracle GEMM on them; (b)
    prepare_native_dense_layer + native_dense_forward against the oracle's exact NVFP4 GEMM."""
    N, Kd = 512, 1024
    g = torch.Generator().manual_seed(20261201 + 12300 + M)
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    qo, so = O.quant_rows_fp8(x)
    a_layer, packed, s16, div = _dense_nvfp4_layer(dev, N, Kd, g)
    NV.convert_dense_layer(a_layer)
    cp, ce = O.nvfp4_to_mxfp4(packed.numpy(), s16.view(torch.uint8).numpy(), div.numpy())
    assert np.array_equal(a_layer.weight.data.cpu().numpy(), cp) and np.array_equal(a_layer.weight_scale.data.cpu().numpy(), ce)
    LX.prep_dense(a_layer)
    got = LX.apply_dense(a_layer, x.to(dev))
    ref = O.grouped_gemm(qo, so, {0: O.mxfp4_dequant(torch.from_numpy(cp), torch.from_numpy(ce))},
                         np.zeros(M, dtype=np.int32), 1)
    r1, _ = _check(O.bf16_bits(got), ref, 2e-3, 0.99999)
    b_layer, packed, s16, div = _dense_nvfp4_layer(dev, N, Kd, torch.Generator().manual_seed(20261201 + 12300 + M))
    NV.prepare_native_dense_layer(b_layer)
    got = NV.native_dense_forward(b_layer, x.to(dev))
    ref = O.nvfp4_gemm(qo, so, packed.numpy()[None], s16.view(torch.uint8).numpy()[None],
                       (1.0 / div).float().numpy()[None], np.zeros(M, dtype=np.int32), 1)
    r2, _ = _check(O.bf16_bits(got), ref, 2e-3, 0.99999)
    print(f"dense nvfp4 M={M}: converted rel {r1:.2e}, native rel {r2:.2e}", flush=True)


@pytest.mark.parametrize("M", [1, 40])
def test_mxfp4_linearize(dev, M):
    """mxfp4_linearize on an arbitrary dense fp32 weight: exponents and codes bit-exact against the oracle's MSE
    search, the returned kernel's forward against the oracle GEMM on those bits."""
    N, Kd = 384, 1536
    g = torch.Generator().manual_seed(20261201 + 12400 + M)
    W = torch.randn(N, Kd, generator=g) * torch.exp(torch.randn(N, 1, generator=g))
    layer = torch.nn.Module()
    kern = NV.mxfp4_linearize(layer, W.to(dev), rows_per_chunk=100)
    po, eo = O.quantize_mxfp4_search(W.numpy())
    assert torch.equal(K.unpermute_fragments(layer.weight.data, N, Kd)[0].cpu(), torch.from_numpy(po))
    assert torch.equal(K.unpack_scales(layer.weight_scale.data)[0].cpu(), torch.from_numpy(eo))
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    got = kern.apply_weights(layer, x.to(dev))
    qo, so = O.quant_rows_fp8(x)
    ref = O.grouped_gemm(qo, so, {0: O.mxfp4_dequant(torch.from_numpy(po), torch.from_numpy(eo))},
                         np.zeros(M, dtype=np.int32), 1)
    r, c = _check(O.bf16_bits(got), ref, 2e-3, 0.99999)
    print(f"mxfp4_linearize M={M}: rel {r:.2e}", flush=True)


def test_route_step_paths(dev):
    """route.route_step (the R9kTopKRouter body, vLLM-free): decode widths fill the persistent buffers and, up to
    4096 routed rows, quantise the input (bytes of quant_rows_fp8); wide calls return the top-k + quant and no tables; the ids
    equal the oracle's and the hand-off helpers find exactly this call's data."""
    from r9700_vllm.moe import route
    E, H, topk = 288, 2048, 8
    bufs = route.RouteBuffers(dev, E, topk)
    for T in (1, 64, 200, 700):
        g = torch.Generator().manual_seed(20261201 + 12500 + T)
        x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
        logits = torch.randn(T, E, generator=g).to(torch.bfloat16)
        w, ids, tabs = route.route_step(logits.to(dev), x, topk, True, E, bufs, use_ops=False)
        torch.cuda.synchronize()
        assert np.array_equal(ids.cpu().numpy(), O.route(logits, topk, True)[1]), T

        class Layer:
            _r9k_tables = tabs
        numel = T * topk
        blk = K.MOE_BLOCK * K.pick_mt(numel, E)
        got_tabs = route.take(Layer, ids, blk, numel)
        got_q = route.take_quant(Layer, ids, x)
        assert (got_tabs is not None) == (T <= route.MAX_ROWS)
        assert (got_q is not None) == (T * topk <= route.QUANT_MAX_NUMEL or T > route.MAX_ROWS)
        if got_q is not None:
            q, s = K.quant_rows_fp8(x)
            assert torch.equal(got_q[0].view(torch.uint8), q.view(torch.uint8)) and torch.equal(got_q[1], s)
        if got_tabs is not None:
            sid, eid, ntpp = (t.cpu() for t in got_tabs)
            rs, re_, rn = O.align(ids.cpu().numpy(), E, blk)
            n = int(rn[0])
            assert int(ntpp[0]) == n and np.array_equal(sid[:n].numpy(), rs[:n])
            assert np.array_equal(eid[: n // blk].numpy(), re_[: n // blk])
        print(f"route_step T={T}: tables {got_tabs is not None}, quant {got_q is not None}", flush=True)
