"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every stored output (no drift), and the stored bytes pass checks that do not go
through the oracle: torch's float8_e4m3fn cast for the quant, torch.softmax + a stable sort for the routing of the
non-degenerate rows, an argsort restatement plus the reference test's invariants for the tables
(tests/test_moe_route_r9k.py:24-41), a float32 loop for the top-k sum, the fp32 torch restatement of
quantize_mxfp4_search (the reference's own operations, r9700_vllm/quant/nvfp4.py:54-75) for the converter.
GPU: every HIP entry point through the C-ABI against the stored bytes (bit-exact), the GEMM to tolerance."""
import os
import sys

import numpy as np
import pytest
import torch

from helpers import bf16_bits_to_f64, check_tables, cosine, rel_err
from oracle import oracle as O

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
from make_golden import CASES, load  # noqa: E402

from test_oracle_nvfp4 import torch_search  # noqa: E402


def bf(bits: np.ndarray) -> torch.Tensor:
    return O.bits_to_bf16(bits)


# ------------------------------------------------------------------------------------------------ CPU
@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_reproduces_fixture(name):
    fresh = CASES[name]()
    stored = load(name)
    assert sorted(fresh) == sorted(stored)
    for k in stored:
        a, b = np.asarray(fresh[k]), stored[k]
        assert a.dtype == b.dtype and a.shape == b.shape, k
        assert np.array_equal(a.view(np.uint8) if a.dtype.kind == "f" else a,
                              b.view(np.uint8) if b.dtype.kind == "f" else b), f"{name}.{k} drifted"


def test_fixture_quant_matches_torch_cast():
    z = load("quant_rows")
    x = bf(z["x"]).float()
    amax = x.abs().amax(1).clamp_min(1e-12).numpy().astype(np.float32)
    inv = np.float32(448.0) / amax                                     # IEEE fp32 division
    q = (x * torch.from_numpy(inv)[:, None]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(q, z["q"])
    assert np.array_equal((amax / np.float32(448.0)).view(np.uint32), z["s"].view(np.uint32))


def test_fixture_route_matches_torch_on_regular_rows():
    z = load("route")
    x = bf(z["logits"]).float()
    k = int(z["topk"])
    regular = [r for r in range(x.shape[0]) if r not in (3, 4, 5, 6)]        # rows 3-6 are degenerate by design
    p = torch.softmax(x[regular], -1)
    _, idx = torch.sort(-p, dim=-1, stable=True)
    assert np.array_equal(idx[:, :k].numpy(), z["ids"][regular])
    w = p.gather(1, idx[:, :k])
    assert np.abs((w / w.sum(-1, keepdim=True)).numpy() - z["w"][regular]).max() < 2e-6
    assert np.abs(w.numpy() - z["w_norenorm"][regular]).max() < 2e-6
    assert z["ids"][5].tolist() == list(range(k)) and not z["w"][5].any()   # all -inf: dead, by index, weight 0
    assert z["ids"][2].tolist() == list(range(k))                           # all equal: ties to the lower index
    assert z["ids"][1, :4].tolist() == [3, 77, 200, 201]


def _tables_by_argsort(ids: np.ndarray, E: int, blk: int):
    flat = ids.reshape(-1)
    numel = flat.size
    cap = (numel + E * (blk - 1) + blk - 1) // blk * blk
    s = np.full(cap, numel, np.int32)
    e = np.full(cap // blk, -1, np.int32)
    valid = (flat >= 0) & (flat < E)
    order = np.argsort(np.where(valid, flat, E), kind="stable")
    pos = 0
    cnt = np.bincount(flat[valid], minlength=E)
    o = 0
    for ex in range(E):
        c = int(cnt[ex])
        if c:
            s[pos:pos + c] = order[o:o + c]
            n = (c + blk - 1) // blk * blk
            e[pos // blk:(pos + n) // blk] = ex
            pos += n
            o += c
    return s, e, np.array([pos], np.int32)


@pytest.mark.parametrize("name,blks", [("route", (16, 64)), ("align", (16, 256))])
def test_fixture_tables(name, blks):
    z = load(name)
    ids = z["ids"].reshape(-1)
    E = 288 if name == "route" else int(z["E"])
    for blk in blks:
        s, e, n = _tables_by_argsort(ids, E, blk)
        assert np.array_equal(s, z[f"sorted_ids_{blk}"]) and np.array_equal(e, z[f"expert_ids_{blk}"])
        assert n[0] == z[f"ntpp_{blk}"][0]
        if name == "route":
            check_tables(s, e, n, ids, blk, ids.size, E)


def test_fixture_moe_sum_float32_loop():
    z = load("moe_sum")
    d = bf(z["down"]).float().numpy()
    acc = np.zeros(d[:, 0].shape, np.float32)
    for j in range(d.shape[1]):
        acc = (acc + d[:, j]).astype(np.float32)
    assert np.array_equal(O.bf16_bits(torch.from_numpy(acc).to(torch.bfloat16)), z["out"])


def test_fixture_converters_match_torch_restatement():
    z = load("mx_search")
    p, e = torch_search(torch.from_numpy(z["w"]))
    assert np.array_equal(p, z["out_packed"]) and np.array_equal(e, z["out_e8m0"])
    z = load("nvfp4")
    deq = O.dequant_nvfp4(z["packed"], z["s16"], z["row_div"])
    lut = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
                   np.float32)
    codes = np.stack([z["packed"] & 15, z["packed"] >> 4], -1).reshape(z["packed"].shape[0], -1)
    s16 = torch.from_numpy(z["s16"]).view(torch.float8_e4m3fn).float().numpy()
    ref = (lut[codes] * np.repeat(s16, 16, axis=1)).astype(np.float32) / z["row_div"][:, None]
    assert np.array_equal(deq.view(np.uint32), ref.astype(np.float32).view(np.uint32))
    p, e = torch_search(torch.from_numpy(deq))
    assert np.array_equal(p, z["out_packed"]) and np.array_equal(e, z["out_e8m0"])


def test_fixture_gemm_pure_python_spot_check():
    z = load("gemm")
    E, N, Kh = z["packed"].shape
    ids = z["ids"]
    k = ids.shape[1]
    xq, xs = O.quant_rows_fp8(bf(z["x"]))
    e4 = O.e4m3_table()
    lut = O.E2M1
    for r in (0, 3, ids.size - 1):
        ex = int(ids.reshape(-1)[r])
        for n in (0, N // 2, N - 1):
            acc = 0.0
            for kk in range(Kh * 2):
                byte = int(z["packed"][ex, n, kk // 2])
                c = byte & 15 if kk % 2 == 0 else byte >> 4
                acc += e4[xq[r // k, kk]] * lut[c] * 2.0 ** (int(z["e8m0"][ex, n, kk // 32]) - 127)
            v = np.float32(np.float32(acc) * np.float32(xs[r // k]))
            want = O.bf16_bits(torch.tensor([v]).to(torch.bfloat16))[0]
            assert want == z["gate_up"][r, n]


# ------------------------------------------------------------------------------------------------ GPU
@pytest.mark.gpu
def test_gpu_golden_quant(dev):
    from r9700_vllm.kernels import moe as K
    z = load("quant_rows")
    q, s = K.quant_rows_fp8(bf(z["x"]).to(dev))
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), z["q"])
    assert np.array_equal(s.cpu().numpy().view(np.uint32), z["s"].view(np.uint32))


@pytest.mark.gpu
def test_gpu_golden_route_and_tables(dev):
    from r9700_vllm.kernels import moe as K
    from r9700_vllm.moe import route
    z = load("route")
    lg = bf(z["logits"]).to(dev)
    k, E = int(z["topk"]), lg.shape[1]
    w, ids = K.moe_topk(lg, k, True)
    assert np.array_equal(ids.cpu().numpy(), z["ids"]) and np.abs(w.cpu().numpy() - z["w"]).max() < 2e-6
    w0, ids0 = K.moe_topk(lg, k, False)
    assert np.array_equal(ids0.cpu().numpy(), z["ids_norenorm"])
    assert np.abs(w0.cpu().numpy() - z["w_norenorm"]).max() < 2e-6
    for blk in (16, 64):
        cap = route.capacity(ids.numel(), E, blk)
        s_ = torch.empty(cap, dtype=torch.int32, device=dev)
        e_ = torch.empty(cap // blk, dtype=torch.int32, device=dev)
        n_ = torch.zeros(1, dtype=torch.int32, device=dev)
        sc = torch.zeros(route.scratch_ints(E), dtype=torch.int32, device=dev)
        w2, ids2 = route.moe_route(lg, k, True, blk, s_, e_, n_, sc)
        assert np.array_equal(ids2.cpu().numpy(), z["ids"])
        assert np.array_equal(s_.cpu().numpy(), z[f"sorted_ids_{blk}"])
        assert np.array_equal(e_.cpu().numpy(), z[f"expert_ids_{blk}"]) and n_.item() == z[f"ntpp_{blk}"][0]
        s2, e2, n2 = K.moe_align(ids, blk, E)
        assert np.array_equal(s2.cpu().numpy(), z[f"sorted_ids_{blk}"])
        assert np.array_equal(e2.cpu().numpy(), z[f"expert_ids_{blk}"]) and n2.item() == z[f"ntpp_{blk}"][0]


@pytest.mark.gpu
def test_gpu_golden_align_skewed(dev):
    from r9700_vllm.kernels import moe as K
    z = load("align")
    for blk in (16, 256):
        s, e, n = K.moe_align(torch.from_numpy(z["ids"]).to(dev), blk, int(z["E"]))
        assert np.array_equal(s.cpu().numpy(), z[f"sorted_ids_{blk}"])
        assert np.array_equal(e.cpu().numpy(), z[f"expert_ids_{blk}"]) and n.item() == z[f"ntpp_{blk}"][0]


@pytest.mark.gpu
def test_gpu_golden_moe_sum(dev):
    from r9700_vllm.kernels import moe as K
    z = load("moe_sum")
    d = bf(z["down"]).to(dev)
    out = torch.empty(d.shape[0], d.shape[2], dtype=torch.bfloat16, device=dev)
    K.moe_sum(d, None, out)
    assert np.array_equal(O.bf16_bits(out), z["out"])


@pytest.mark.gpu
def test_gpu_golden_converters(dev):
    from r9700_vllm.quant import nvfp4 as NV
    z = load("nvfp4")
    pm, em = NV.nvfp4_to_mxfp4(torch.from_numpy(z["packed"]).to(dev),
                               torch.from_numpy(z["s16"]).view(torch.float8_e4m3fn).to(dev),
                               torch.from_numpy(z["row_div"]).to(dev))
    assert np.array_equal(pm.cpu().numpy(), z["out_packed"]) and np.array_equal(em.cpu().numpy(), z["out_e8m0"])
    z = load("mx_search")
    pm, em = NV.quantize_mxfp4_search(torch.from_numpy(z["w"]).to(dev))
    assert np.array_equal(pm.cpu().numpy(), z["out_packed"]) and np.array_equal(em.cpu().numpy(), z["out_e8m0"])


@pytest.mark.gpu
def test_gpu_golden_gemm(dev):
    from r9700_vllm.kernels import moe as K
    z = load("gemm")
    E, N, Kh = z["packed"].shape
    ids = torch.from_numpy(z["ids"])
    M, k = ids.shape
    W = K.prepare_mxfp4_weights(torch.from_numpy(z["packed"]).to(dev), torch.from_numpy(z["e8m0"]).to(dev))
    sid, eid, ntpp = (t.to(dev) for t in K.align_block_size_ref(ids, E, 16))
    for key, xkey, div, tw in (("gate_up", "x", k, None), ("down", "x_rows", 1, torch.from_numpy(z["topk_w"]))):
        xq, xs = K.quant_rows_fp8(bf(z[xkey]).to(dev))
        out = torch.full((M * k, N), float("nan"), dtype=torch.bfloat16, device=dev)
        K.moe_gemm(xq, xs, W, out, sid, eid, ntpp, M * k, div, tw.to(dev) if tw is not None else None,
                   num_experts=E)
        a, b = bf16_bits_to_f64(O.bf16_bits(out)), bf16_bits_to_f64(z[key])
        assert rel_err(a, b) < 2e-3 and cosine(a, b) > 0.99999, key
