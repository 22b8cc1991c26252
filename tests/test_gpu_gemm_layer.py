"""GPU parity: the grouped MXFP4 x fp8 GEMM (decode and prefill entries), the dense MXFP4 linear, the NVFP4 ->
MXFP4 converter and the whole MoE layer (R9700Mxfp4Experts.apply), through the C-ABI against the CPU oracle.

Float outputs are held to the north-star tolerance (norm ratio <= 1e-2, cosine >= 0.9999) and, tighter, to what
fp32 accumulation order can explain (rel <= 2e-3); converter outputs and routing ids are bit-exact."""
import numpy as np
import pytest
import torch

from helpers import bf16_bits_to_f64, block_edge_tokens, cosine, make_experts, rel_err
from oracle import oracle as O
from r9700_vllm import ops
from r9700_vllm.kernels import moe as K
from r9700_vllm.moe.experts import R9700Mxfp4Experts
from r9700_vllm.quant import nvfp4 as NV

pytestmark = pytest.mark.gpu


def gemm_case(dev, E, M, topk, N, Kd, seed, MT=1, prefill=None, down=False):
    g = torch.Generator().manual_seed(seed)
    packed, e8 = make_experts(E, N, Kd, g)
    W = K.prepare_mxfp4_weights(packed.to(dev), e8.to(dev))
    numel = M * topk
    rows_a = numel if down else M
    x = (torch.randn(rows_a, Kd, generator=g) * 0.5).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:topk] for _ in range(M)]).to(torch.int32)
    tw = torch.rand(numel, generator=g).float() if down else None
    blk = K.prefill_block(prefill) if prefill is not None else 16 * MT
    sid, eid, ntpp = (t.to(dev) for t in K.align_block_size_ref(ids, E, blk))
    xq, xs = K.quant_rows_fp8(x.to(dev))
    out = torch.full((numel, N), float("nan"), dtype=torch.bfloat16, device=dev)
    K.moe_gemm(xq, xs, W, out, sid, eid, ntpp, numel, 1 if down else topk, tw.to(dev) if down else None,
               num_experts=E, MT=MT, prefill=prefill)
    qo, so = O.quant_rows_fp8(x)
    Wd = {e: O.mxfp4_dequant(packed[e], e8[e]) for e in range(E)}
    ref = O.grouped_gemm(qo, so, Wd, ids.reshape(-1).numpy(), 1 if down else topk,
                         tw.numpy() if down else None)
    got = O.bf16_bits(out)
    assert not np.isnan(bf16_bits_to_f64(got).numpy()).any(), "a routed row was not written"
    r, c = rel_err(bf16_bits_to_f64(got), bf16_bits_to_f64(ref)), cosine(bf16_bits_to_f64(got), bf16_bits_to_f64(ref))
    exact = (got == ref).mean()
    print(f"gemm E={E} M={M} k={topk} N={N} K={Kd} MT={MT} pf={prefill} down={down}: rel {r:.2e} cos {c:.7f} "
          f"exact {exact:.4f}", flush=True)
    assert r < 2e-3 and c > 0.99999 and exact > 0.97


@pytest.mark.parametrize("E,M,topk,N,Kd", [(8, 1, 2, 1024, 2048), (32, 4, 8, 1024, 2048), (64, 16, 8, 2048, 512),
                                           (288, 64, 8, 1024, 2048), (8, 3, 2, 48, 1024), (8, 3, 2, 2560, 320),
                                           (8, 5, 3, 320, 160), (4, 6, 2, 64, 544), (4, 2, 2, 32, 32)])
@pytest.mark.parametrize("down", [False, True])
def test_grouped_gemm_decode(dev, E, M, topk, N, Kd, down):
    gemm_case(dev, E, M, topk, N, Kd, seed=E * 100 + M + N, down=down)


@pytest.mark.parametrize("MT", [2, 4])
@pytest.mark.parametrize("N,Kd", [(640, 2560), (2560, 320), (1024, 2048)])
def test_grouped_gemm_multitile(dev, MT, N, Kd):
    gemm_case(dev, 16, 200, 4, N, Kd, seed=MT + N, MT=MT)
    gemm_case(dev, 16, 200, 4, Kd if Kd % 16 == 0 else N, N if N % 32 == 0 else Kd, seed=MT + N + 1, MT=MT, down=True)


@pytest.mark.parametrize("cfg", [17, 10, 12, 6, 1])
def test_grouped_gemm_prefill_entry(dev, cfg):
    gemm_case(dev, 16, 600, 4, 1040, 1024, seed=cfg, prefill=cfg)
    gemm_case(dev, 16, 600, 4, 512, 320, seed=cfg + 50, prefill=cfg, down=True)


@pytest.mark.parametrize("E,M,topk,N,Kd", [(16, 1200, 4, 1024, 2048), (8, 900, 2, 2048, 512), (4, 300, 1, 272, 384),
                                           (32, 2000, 8, 512, 256), (64, 200, 8, 1024, 1024)])
@pytest.mark.parametrize("down", [False, True])
def test_grouped_gemm_prefill_256(dev, E, M, topk, N, Kd, down):
    """256-row blocks with K % 128 == 0: the LDS-tiled 32x32x64 kernel (ragged expert sizes, padded M tiles,
    a column block past N, one and several 256-row blocks per expert, blocks of ~25 live rows whose other 64-row
    pieces are never loaded)."""
    gemm_case(dev, E, M, topk, N, Kd, seed=E + M + N + Kd, prefill=12, down=down)


@pytest.mark.parametrize("down", [False, True])
def test_grouped_gemm_prefill_256_config5_widths(dev, down):
    """The whole output of the 256-row prefill GEMM at config 5's widths (gate_up N = K = 4096, down N = 4096 with
    K = 2048) over 4 experts, against the fp64 oracle."""
    gemm_case(dev, 4, 700, 2, 4096, 2048 if down else 4096, seed=4096 + down, prefill=12, down=down)


@pytest.mark.parametrize("E,M,topk,N,gate_up,zipf", [
    (288, 8192, 8, 2048, False, False),   # config 3's down GEMM (65536 routed rows, 16 column steps a block)
    (8, 900, 2, 2048, False, False),      # several blocks per expert
    (16, 1200, 4, 2000, False, True),     # a partial last column step (N % 128 = 80), skewed expert sizes
    (4, 300, 1, 272, False, False),       # three column steps, the last one mostly past N
    (8, 700, 2, 512, True, False),        # activation rows shared by the top-k rows of a token (row divisor 2)
    (3, 20, 1, 128, False, False),        # fewer work items than XCDs
    (64, 6000, 8, 128, False, False),     # one column step a block: a workgroup's items span two blocks
    (2, 3, 1, 16, False, False),          # one 16-column tile: every step's other tiles past N
    (5, 700, 2, 2064, False, False),      # 17 column steps, the last one 16 columns wide
])
def test_prefill_row_resident_equals_persistent(dev, monkeypatch, E, M, topk, N, gate_up, zipf):
    """K = 512 prefill GEMM (256-row blocks): the row-resident kernel (each wave's rows held in registers across the
    column steps) against the persistent tile kernel, bit for bit, every routed row written."""
    Kd = 512
    g = torch.Generator().manual_seed(E * 7 + M + N)
    packed, e8 = make_experts(E, N, Kd, g)
    W = K.prepare_mxfp4_weights(packed.to(dev), e8.to(dev))
    numel = M * topk
    rows_a = M if gate_up else numel
    x = (torch.randn(rows_a, Kd, generator=g) * 0.5).to(torch.bfloat16)
    if zipf:
        p = 1.0 / torch.arange(1, E + 1, dtype=torch.float64) ** 1.1
        ids = torch.stack([torch.multinomial(p, topk, replacement=False, generator=g) for _ in range(M)])
    else:
        ids = torch.stack([torch.randperm(E, generator=g)[:topk] for _ in range(M)])
    ids = ids.to(torch.int32)
    tw = None if gate_up else torch.rand(numel, generator=g).float().to(dev)
    sid, eid, ntpp = (t.to(dev) for t in K.align_block_size_ref(ids, E, K.prefill_block(12)))
    xq, xs = K.quant_rows_fp8(x.to(dev))
    outs = []
    for flag in (None, "0"):
        if flag is None:
            monkeypatch.delenv("R9K_PREFILL_ROWRES", raising=False)
        else:
            monkeypatch.setenv("R9K_PREFILL_ROWRES", flag)
        out = torch.full((numel, N), float("nan"), dtype=torch.bfloat16, device=dev)
        K.moe_gemm(xq, xs, W, out, sid, eid, ntpp, numel, topk if gate_up else 1, tw, num_experts=E, prefill=12)
        torch.cuda.synchronize()
        outs.append(out)
    rr, ps = outs
    assert not torch.isnan(rr.float()).any(), "a routed row was not written"
    diff = (rr.view(torch.int16) != ps.view(torch.int16)).sum().item()
    print(f"row-resident E={E} M={M} k={topk} N={N} gate_up={gate_up}: {diff} of {rr.numel()} values differ",
          flush=True)
    assert diff == 0


@pytest.mark.parametrize("M,N,Kd", [(16, 1024, 2048), (1, 17408, 5120), (4, 1024, 5120), (300, 512, 1024)])
def test_dense_mxfp4_linear(dev, M, N, Kd):
    """BASELINE config 1 (and small slices of config 4): identity routing tables through ops.mxfp4_linear."""
    g = torch.Generator().manual_seed(M + N)
    packed, e8 = make_experts(1, N, Kd, g)
    W = K.prepare_mxfp4_weights(packed.to(dev), e8.to(dev))
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    out = ops.mxfp4_linear(x.to(dev), W.wq, W.wsr, N, Kd)
    qo, so = O.quant_rows_fp8(x)
    ref = O.grouped_gemm(qo, so, {0: O.mxfp4_dequant(packed[0], e8[0])}, np.zeros(M, dtype=np.int32), 1)
    got = O.bf16_bits(out)
    r = rel_err(bf16_bits_to_f64(got), bf16_bits_to_f64(ref))
    assert r < 2e-3 and cosine(bf16_bits_to_f64(got), bf16_bits_to_f64(ref)) > 0.99999


def test_dense_mxfp4_linear_config4_prefill_sampled(dev):
    """BASELINE config 4 at M = 4096: [4096, 5120] x [17408, 5120]^T through ops.mxfp4_linear (256-row tiles), checked
    on 48 sampled rows (rows are independent)."""
    M, N, Kd = 4096, 17408, 5120
    g = torch.Generator().manual_seed(4096)
    packed, e8 = make_experts(1, N, Kd, g)
    W = K.prepare_mxfp4_weights(packed.to(dev), e8.to(dev))
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    out = ops.mxfp4_linear(x.to(dev), W.wq, W.wsr, N, Kd)
    rows = np.sort(np.random.default_rng(0).choice(M, 48, replace=False))
    qo, so = O.quant_rows_fp8(x)
    Wd = O.mxfp4_dequant(packed[0], e8[0], torch.float32)
    ref = O.grouped_gemm(qo, so, {0: Wd}, np.zeros(M, dtype=np.int32), 1, None, rows, acc_dtype=torch.float32)
    got = O.bf16_bits(out)[rows]
    r = rel_err(bf16_bits_to_f64(got), bf16_bits_to_f64(ref))
    assert r < 2e-3 and cosine(bf16_bits_to_f64(got), bf16_bits_to_f64(ref)) > 0.99999


@pytest.mark.parametrize("kind", ["mxfp4", "nvfp4"])
def test_dense_linear_output_past_2gib(dev, kind):
    """A dense linear whose bf16 output just crosses 2 GiB (config 4's N = 17408, M = 61682 rows, K = 1024): ops runs
    it as two row ranges, each inside the kernels' 32-bit buffer range. Checked on the first and last rows of each
    range and 24 random rows against the oracle."""
    M, N, Kd = 61682, 17408, 1024
    assert M * N * 2 > ops.BUF_LIMIT
    ranges = ops.row_ranges(M, N, Kd)
    assert len(ranges) == 2
    print(f"dense {kind} past 2 GiB: M={M} N={N} K={Kd} ranges={ranges}", flush=True)
    g = torch.Generator().manual_seed(61682 + (kind == "nvfp4"))
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    edge = [r for r0, r1 in ranges for r in (r0, r0 + 1, r1 - 2, r1 - 1)]
    rows = np.unique(np.concatenate([edge, np.random.default_rng(1).choice(M, 24, replace=False)]))
    qo, so = O.quant_rows_fp8(x[torch.from_numpy(rows)])
    zero = np.zeros(rows.size, dtype=np.int32)
    if kind == "mxfp4":
        packed, e8 = make_experts(1, N, Kd, g)
        W = K.prepare_mxfp4_weights(packed.to(dev), e8.to(dev))
        out = ops.mxfp4_linear(x.to(dev), W.wq, W.wsr, N, Kd)
        ref = O.grouped_gemm(qo, so, {0: O.mxfp4_dequant(packed[0], e8[0], torch.float32)}, zero, 1,
                             acc_dtype=torch.float32)
    else:
        packed = torch.randint(0, 256, (1, N, Kd // 2), generator=g, dtype=torch.int32).to(torch.uint8)
        s16 = (torch.randn(1, N, Kd // 16, generator=g).abs() * 0.05).to(torch.float8_e4m3fn)
        wg = torch.rand(1, N, generator=g) * 1.5 + 0.5
        W = K.prepare_nvfp4_weights(packed.to(dev), s16.to(dev), wg.to(dev))
        out = ops.nvfp4_linear(x.to(dev), W.wq, W.ws, W.wg, N, Kd)
        ref = O.nvfp4_gemm(qo, so, packed.numpy(), s16.view(torch.uint8).numpy(), wg.numpy(), zero, 1)
    got = O.bf16_bits(out[torch.from_numpy(rows).to(dev)])
    del out
    a, b = bf16_bits_to_f64(got), bf16_bits_to_f64(ref)
    r, c = rel_err(a, b), cosine(a, b)
    print(f"  rel {r:.2e} cos {c:.7f}", flush=True)
    assert not np.isnan(a.numpy()).any() and r < 2e-3 and c > 0.99999


def test_nvfp4_to_mxfp4_config4_bit_exact(dev):
    """BASELINE config 4 full shape: [17408, 5120] NVFP4 (uniform codes, s16 = e4m3(|N(0,1)| * 0.05), global 1)."""
    g = torch.Generator().manual_seed(20261201 + 4000)
    N, Kd = 17408, 5120
    p16 = torch.randint(0, 256, (N, Kd // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    s16 = (torch.randn(N, Kd // 16, generator=g).abs() * 0.05).to(torch.float8_e4m3fn)
    div = torch.ones(N)
    pm, em = NV.nvfp4_to_mxfp4(p16.to(dev), s16.to(dev), div.to(dev))
    po, eo = O.nvfp4_to_mxfp4(p16.numpy(), s16.view(torch.uint8).numpy(), div.numpy())
    assert np.array_equal(pm.cpu().numpy(), po)
    assert np.array_equal(em.cpu().numpy(), eo)


def test_nvfp4_to_mxfp4_row_divisors_and_host_input(dev):
    """Per-row global divisors (a fused gate_up with two shards) and host-resident input (chunked device copies)."""
    g = torch.Generator().manual_seed(9)
    N, Kd = 512, 2560
    w = torch.randn(N, Kd, generator=g) * 0.02
    gd = torch.where(torch.arange(N) < N // 2, torch.tensor(3000.0), torch.tensor(7000.0))
    x = w.reshape(N, Kd // 16, 16)
    s16 = (x.abs().amax(-1) / 6.0 * gd[:, None]).clamp(min=2 ** -9).to(torch.float8_e4m3fn)
    v = x * gd[:, None, None] / s16.float().unsqueeze(-1)
    code = (torch.bucketize(v.abs(), NV._MID).to(torch.uint8) | ((v < 0).to(torch.uint8) << 3)).reshape(N, Kd)
    p16 = code[:, 0::2] | (code[:, 1::2] << 4)
    pm, em = NV.nvfp4_to_mxfp4(p16, s16, gd, rows_per_chunk=200)          # CPU tensors in, CPU tensors out
    po, eo = O.nvfp4_to_mxfp4(p16.numpy(), s16.view(torch.uint8).numpy(), gd.numpy())
    assert pm.device.type == "cpu" and np.array_equal(pm.numpy(), po) and np.array_equal(em.numpy(), eo)


def test_quantize_mxfp4_search_bit_exact(dev):
    g = torch.Generator().manual_seed(12)
    w = torch.randn(1024, 2048, generator=g) * torch.exp(torch.randn(1024, 1, generator=g))
    w[0, :64] = 0.0
    pm, em = NV.quantize_mxfp4_search(w.to(dev))
    po, eo = O.quantize_mxfp4_search(w.numpy())
    assert np.array_equal(pm.cpu().numpy(), po) and np.array_equal(em.cpu().numpy(), eo)


def test_quantize_mxfp4_search_decision_edges(dev):
    """The search's fp32 error sums decide only when they are apart by more than their error bound; the rest fall back
    to the fp64 sums. Blocks that reach each branch, bit for bit against the oracle: exact candidate ties (one value
    at 3.5 * 2^k, whose two candidates both err by (2^(k-1))^2: the e0 candidate wins), near ties just inside and just
    outside the margin, denormal-only and mixed blocks (sums under 2^-100), blocks near the fp32 maximum (sums past
    2^120), NaN, +-inf and -0.0 entries, across exponents from -130 to 127."""
    rows = []
    for k in (-120, -20, -1, 0, 7, 30, 100):
        for rel in (0.0, 2.0 ** -22, -(2.0 ** -22), 2.0 ** -18, -(2.0 ** -18), 2.0 ** -10):
            blk = np.zeros(32, np.float32)
            blk[3] = np.float32(3.5 * 2.0 ** k * (1 + rel))
            blk[17] = np.float32(-1.25 * 2.0 ** k) if rel < 0 else 0.0
            rows.append(blk)
    rng = np.random.default_rng(31)
    for scale in (1e-44, 1e-40, 1e-38, 3e-36, 2.0 ** 59, 2.0 ** 61, 1e37, 5e37):
        blk = (rng.standard_normal(32) * scale).astype(np.float32)
        rows.append(blk)
    mixed = (rng.standard_normal(32) * 1e-39).astype(np.float32)
    mixed[0] = 1e-30
    rows.append(mixed)
    withnan = rng.standard_normal(32).astype(np.float32)
    withnan[5] = np.nan
    rows.append(withnan)
    negz = np.full(32, -0.0, np.float32)
    negz[9] = 0.75
    rows.append(negz)
    withinf = rng.standard_normal(32).astype(np.float32)
    withinf[2], withinf[30] = np.inf, -np.inf
    rows.append(withinf)
    if len(rows) % 2:
        rows.append(np.zeros(32, np.float32))
    w = np.concatenate(rows).reshape(-1, 64)
    pm, em = NV.quantize_mxfp4_search(torch.from_numpy(w).to(dev))
    po, eo = O.quantize_mxfp4_search(w)
    assert np.array_equal(em.cpu().numpy(), eo), np.argwhere(em.cpu().numpy() != eo)[:8]
    assert np.array_equal(pm.cpu().numpy(), po)


# --------------------------------------------------------------------------------------------------- layer
def make_layer(dev, E, H, I, seed, lo=118, hi=126):
    """MXFP4 layer weights drawn on the GPU (seeded), plus their checkpoint-layout copies for the oracle."""
    g = torch.Generator(device=dev).manual_seed(seed)
    p13 = torch.randint(0, 256, (E, 2 * I, H // 2), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    e13 = torch.randint(lo, hi + 1, (E, 2 * I, H // 32), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    p2 = torch.randint(0, 256, (E, H, I // 2), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    e2 = torch.randint(lo, hi + 1, (E, H, I // 32), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    W13 = K.prepare_mxfp4_weights(p13, e13)
    W2 = K.prepare_mxfp4_weights(p2, e2)
    return (p13, e13), (p2, e2), W13, W2


def run_layer(dev, E, H, I, T, topk, seed, tokens=None, zipf=False, lo=118, hi=126, edges=None, extra=0):
    """The layer through apply() against the oracle on `tokens` (default all), or, with `edges`, on the tokens
    holding the first and last live row of every `edges`-row block plus `extra` random tokens."""
    (p13, e13), (p2, e2), W13, W2 = make_layer(dev, E, H, I, seed, lo, hi)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g)
    if zipf:
        rank = torch.randperm(E, generator=g).float() + 1
        logits = logits - 1.1 * torch.log(rank)[None, :]
    logits = logits.to(torch.bfloat16)
    w, ids = K.moe_topk(logits.to(dev), topk, True)
    ex = R9700Mxfp4Experts.standalone(W13.wsr, W2.wsr)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    ex.apply(out, x.to(dev), W13.wq, W2.wq, w, ids, "silu", E, None, None, None, None, None, None, False)
    torch.cuda.synchronize()
    ro = O.route(logits, topk, True)
    assert np.array_equal(ids.cpu().numpy(), ro[1]), "routing ids"
    if edges:
        rnd = np.random.default_rng(seed).choice(T, extra, replace=False)
        tokens = np.union1d(block_edge_tokens(ro[1], E, edges, topk), rnd)
    need = np.unique(ro[1][tokens] if tokens is not None else ro[1])
    sub = lambda p: {int(e): p[int(e)].cpu() for e in need}                         # only touched experts
    c13 = (_Lazy(sub(p13)), _Lazy(sub(e13)))
    c2 = (_Lazy(sub(p2)), _Lazy(sub(e2)))
    ref = O.moe_layer(x, logits, c13, c2, topk, True, tokens=tokens, route_out=ro)
    got = O.bf16_bits(out)[ref["tokens"]]
    a, b = bf16_bits_to_f64(got), bf16_bits_to_f64(ref["out"])
    r, c = rel_err(a, b), cosine(a, b)
    print(f"layer E={E} H={H} I={I} T={T} sampled={None if tokens is None else len(tokens)}: rel {r:.2e} "
          f"cos {c:.7f}", flush=True)
    assert r < 1e-2 and c >= 0.9999


class _Lazy:
    """Dict-backed stand-in for an [E, ...] tensor: the oracle only indexes touched experts."""

    def __init__(self, d):
        self.d = d

    def __getitem__(self, e):
        return self.d[int(e)]


@pytest.mark.parametrize("T", [1, 8, 16, 64])
def test_layer_config2_decode(dev, T):
    run_layer(dev, 288, 2048, 512, T, 8, seed=20261201 + 2000 + T)


def test_layer_config3_prefill_sampled(dev):
    """Config 3 on the tokens holding every 256-row block's first and last live row, plus 32 random tokens."""
    run_layer(dev, 288, 2048, 512, 8192, 8, seed=20261201 + 3000 + 8192, edges=256, extra=32)


@pytest.mark.parametrize("T", [1, 32])
def test_layer_config5_skewed(dev, T):
    run_layer(dev, 384, 4096, 2048, T, 8, seed=20261201 + 5000 + T, zipf=True, lo=116, hi=126)


def test_layer_config5_skewed_4096_sampled(dev):
    """Config 5 at T = 4096 (Zipf routing: the hot expert spans many 256-row blocks) on the tokens holding every
    256-row block's first and last live row, plus 16 random tokens."""
    run_layer(dev, 384, 4096, 2048, 4096, 8, seed=20261201 + 5000 + 4096, zipf=True, lo=116, hi=126, edges=256,
              extra=16)


@pytest.mark.parametrize("E,H,I,T,topk", [(64, 512, 256, 600, 4), (384, 1024, 512, 512, 8)])
def test_layer_split_tables(dev, monkeypatch, E, H, I, T, topk):
    """A prefill step on split tables (K.moe_align_split: experts with at most SPLIT_THR rows on the block stream,
    the others on the 256-row kernel) under Zipf routing, against the oracle on every token."""
    monkeypatch.setattr(K, "SPLIT_MEAN_MAX", 1 << 20)
    monkeypatch.setattr(K, "SPLIT_DECODE_MIN_BYTES", 0)
    assert K.split_wanted(T * topk, E, H, I)
    run_layer(dev, E, H, I, T, topk, seed=20261201 + 18000 + E + T, zipf=True)


@pytest.mark.parametrize("E,T,H,I,topk", [(288, 1, 2048, 512, 8), (288, 8, 2048, 512, 8), (288, 64, 2048, 512, 8),
                                          (16, 5, 512, 256, 4), (8, 3, 320, 160, 2), (4, 2, 64, 32, 2)])
def test_fused_decode_gemms_equal_unfused(dev, E, T, H, I, topk):
    """r9k_moe_mxfp4a8_f: gate_up + activation (fuse 1), then down with the per-row quant on load (fuse 2), gives
    the unfused chain's (gate_up -> r9k_silu_mul_quant_fp8 -> down) output bit for bit; the fused activation is
    silu(g) * u of the unfused gate_up output (torch's exp and division: within a few fp32 ulp)."""
    seed = 20261201 + 7000 + E + T + H
    (_, _), (_, _), W13, W2 = make_layer(dev, E, H, I, seed)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    logits = torch.randn(T, E, generator=g).to(torch.bfloat16).to(dev)
    w, ids = K.moe_topk(logits, topk, True)
    numel = T * topk
    sid, eid, ntpp = K.moe_align(ids, 16, E)
    xq, xs = K.quant_rows_fp8(x)
    tw = w.reshape(-1).float().contiguous()
    gu = torch.empty(numel, 2 * I, dtype=torch.bfloat16, device=dev)
    K.moe_gemm(xq, xs, W13, gu, sid, eid, ntpp, numel, topk, None, num_experts=E, MT=1)
    aq, as_ = K.silu_mul_quant_fp8(gu)
    d0 = torch.empty(numel, H, dtype=torch.bfloat16, device=dev)
    K.moe_gemm(aq, as_, W2, d0, sid, eid, ntpp, numel, 1, tw, num_experts=E, MT=1)
    h = torch.full((numel, I), float("nan"), dtype=torch.float32, device=dev)
    K.moe_gemm(xq, xs, W13, h, sid, eid, ntpp, numel, topk, None, num_experts=E, MT=1, fuse=1)
    d1 = torch.full((numel, H), float("nan"), dtype=torch.bfloat16, device=dev)
    K.moe_gemm(h, None, W2, d1, sid, eid, ntpp, numel, 1, tw, num_experts=E, MT=1, fuse=2)
    torch.cuda.synchronize()
    gf, uf = gu[:, :I].float(), gu[:, I:].float()
    href = gf / (1 + torch.exp(-gf)) * uf
    assert not torch.isnan(h).any(), "a routed row of the fused activation was not written"
    assert torch.allclose(h, href, rtol=4e-6, atol=1e-30), float(((h - href).abs() / href.abs()).max())
    same = torch.equal(d0.view(torch.int16), d1.view(torch.int16))
    print(f"fused E={E} T={T} H={H} I={I} k={topk}: down bit-equal {same}", flush=True)
    assert same


def test_layer_config2_decode_fused(dev, monkeypatch):
    """The layer with R9K_MOE_FUSE on (no SiLU launch at decode) against the oracle."""
    import r9700_vllm.moe.experts as X
    monkeypatch.setattr(X, "MOE_FUSE", True)
    for T in (1, 64):
        run_layer(dev, 288, 2048, 512, T, 8, seed=20261201 + 2000 + T)


@pytest.mark.parametrize("zipf", [True, False])
def test_device_block_choice(dev, monkeypatch, zipf):
    """From R9K_MOE_DEVICE_BLOCKS_MIN routed rows a step the host would put on decode blocks gets its tables in both
    layouts and r9k_moe_pick_blocks keeps one on the device: 256-row blocks when numel >= DEVICE_MIN_ROWS x the
    256-row layout's block count (skewed routing), else the decode blocks. The output equals, bit for bit, the same layer run on that
    layout alone (forced from the host)."""
    E, H, I, T, topk = 128, 512, 256, 256, 8
    monkeypatch.setattr(K, "SPLIT", False)                    # the device-picked layout pair, not split tables
    print(f"device block choice zipf={zipf}", flush=True)
    (_, _), (_, _), W13, W2 = make_layer(dev, E, H, I, 20261201 + 8000 + zipf)
    g = torch.Generator().manual_seed(8001 + zipf)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    logits = torch.randn(T, E, generator=g)
    if zipf:
        logits += -2.5 * torch.log(torch.arange(1, E + 1).float())
    logits = logits.to(torch.bfloat16).to(dev)
    w, ids = K.moe_topk(logits, topk, True)
    counts = torch.bincount(ids.reshape(-1).long().cpu(), minlength=E)
    nbig = int(((counts + 255) // 256).sum())
    want_big = T * topk >= K.DEVICE_MIN_ROWS * nbig
    assert want_big == zipf, (nbig, int((counts > 0).sum()))
    ex = R9700Mxfp4Experts.standalone(W13.wsr, W2.wsr)

    def run():
        o = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=dev)
        ex.apply(o, x, W13.wq, W2.wq, w, ids, "silu", E, None, None, None, None, None, None, False)
        torch.cuda.synchronize()
        return o

    dual = run()
    monkeypatch.setattr(K, "DEVICE_BLOCKS_MIN", 0)
    small = run()
    monkeypatch.setattr(K, "PREFILL_MOE_ROWS", 1)              # the host picks the 256-row blocks
    big = run()
    ref = big if want_big else small
    same = torch.equal(dual.view(torch.int16), ref.view(torch.int16))
    print(f"  touched {int((counts > 0).sum())}, 256-row blocks {nbig}: kept {'big' if want_big else 'small'}, "
          f"bit-equal {same}", flush=True)
    assert same


def test_fused_entry_rejects_bad_args(dev):
    L = K.lib()
    # fuse values other than 1 / 2 -> -8; multi-tile routing blocks -> -7 (checked before any launch)
    assert L.r9k_moe_mxfp4a8_f(3, *([1] * 12), 1, 16, 1, 64, 64, 2, 4, 2, 1, 0) == -8
    assert L.r9k_moe_mxfp4a8_f(1, *([1] * 12), 1, 16, 1, 64, 64, 2, 4, 2, 2, 0) == -7


@pytest.mark.parametrize("M", [1, 16, 300, 2048])
def test_shared_expert(dev, M):
    """moe/shared.shared_expert (gated shared expert: quant + gate, gate_up, SiLU quant, down with the gate folded into
    the row scale) against the oracle chain on the same gate values: norm ratio <= 1e-2, cosine >= 0.9999."""
    from r9700_vllm.moe import shared
    H, I = 2048, 512
    g = torch.Generator().manual_seed(20261201 + 6000 + M)
    p1, e1 = make_experts(1, 2 * I, H, g)
    p2, e2 = make_experts(1, H, I, g)
    W1 = K.prepare_mxfp4_weights(p1.to(dev), e1.to(dev))
    W2 = K.prepare_mxfp4_weights(p2.to(dev), e2.to(dev))
    x = torch.randn(M, H, generator=g).to(torch.bfloat16)
    wg = (torch.randn(H, generator=g) * 0.02).to(torch.bfloat16)
    out = shared.shared_expert(x.to(dev), W1.wq, W1.wsr, W2.wq, W2.wsr, wg.to(dev), 2 * I, H, H, I, False, False)
    _, _, gate = K.quant_rows_fp8_gate(x.to(dev), wg.to(dev))          # the gate values (own test: bit-level)
    torch.cuda.synchronize()
    qo, so = O.quant_rows_fp8(x)
    zeros = np.zeros(M, dtype=np.int64)
    gu = O.grouped_gemm(qo, so, {0: O.mxfp4_dequant(p1[0], e1[0])}, zeros, 1, acc_dtype=torch.float32)
    aq, as_, _ = O.silu_mul_quant_fp8(O.bits_to_bf16(gu))
    ref = O.grouped_gemm(aq, as_, {0: O.mxfp4_dequant(p2[0], e2[0])}, zeros, 1, gate.cpu().numpy(),
                         acc_dtype=torch.float32)
    a, b = bf16_bits_to_f64(O.bf16_bits(out)), bf16_bits_to_f64(ref)
    r, c = rel_err(a, b), cosine(a, b)
    print(f"shared expert M={M}: rel {r:.2e} cos {c:.7f}", flush=True)
    assert r <= 1e-2 and c >= 0.9999


def test_layer_config5_T256_router_handoff(dev, monkeypatch):
    """BASELINE config 5 at T = 256 (E=384, hidden 4096, intermediate 2048, Zipf(1.1) logits) through the default
    apply() with the router's hand-off: the tables come from route.moe_route on the router's own persistent buffers
    (route.Tables on the layer, as R9kTopKRouter leaves them), so the device-side block choice runs on them (the
    256-row layout built beside them, r9k_moe_pick_blocks keeping one). Checked against the oracle on 32 sampled
    tokens, and bit for bit against the layout the host-side counts say must be kept, run alone."""
    from r9700_vllm.moe import route
    monkeypatch.setattr(K, "SPLIT", False)                    # the device-picked layout pair, not split tables
    E, H, I, T, topk = 384, 4096, 2048, 256, 8
    seed = 20261201 + 5000 + T
    (p13, e13), (p2, e2), W13, W2 = make_layer(dev, E, H, I, seed, 116, 126)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    rank = torch.randperm(E, generator=g).float() + 1
    logits = (torch.randn(T, E, generator=g) - 1.1 * torch.log(rank)[None, :]).to(torch.bfloat16)
    xd, ld = x.to(dev), logits.to(dev)
    numel = T * topk
    blk = K.MOE_BLOCK * K.pick_mt(numel, E)
    assert numel >= K.DEVICE_BLOCKS_MIN and K.pick_moe_prefill_block(numel, E, H, I) is None
    cap = route.capacity(numel, E, blk)
    sid = torch.empty(cap, dtype=torch.int32, device=dev)
    eid = torch.empty(cap // blk, dtype=torch.int32, device=dev)
    ntpp = torch.zeros(1, dtype=torch.int32, device=dev)
    scratch = torch.zeros(route.scratch_ints(E), dtype=torch.int32, device=dev)
    w, ids = route.moe_route(ld, topk, True, blk, sid, eid, ntpp, scratch)

    class Routed:
        _r9k_tables = route.Tables(ids, sid, eid, ntpp, blk, numel)

    ex = R9700Mxfp4Experts.standalone(W13.wsr, W2.wsr)
    ex.r9k_layer = Routed()
    assert route.take(ex.r9k_layer, ids, blk, numel) is not None, "the hand-off must be taken"

    def run(e):
        o = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=dev)
        e.apply(o, xd, W13.wq, W2.wq, w, ids, "silu", E, None, None, None, None, None, None, False)
        torch.cuda.synchronize()
        return o

    out = run(ex)
    counts = torch.bincount(ids.reshape(-1).long().cpu(), minlength=E)
    nbig = int(((counts + 255) // 256).sum())
    want_big = numel >= K.DEVICE_MIN_ROWS * nbig
    plain = R9700Mxfp4Experts.standalone(W13.wsr, W2.wsr)
    if want_big:
        monkeypatch.setattr(K, "PREFILL_MOE_ROWS", 1)
    else:
        monkeypatch.setattr(K, "DEVICE_BLOCKS_MIN", 0)
    alone = run(plain)
    same = torch.equal(out.view(torch.int16), alone.view(torch.int16))
    print(f"cfg5 T=256 hand-off: touched {int((counts > 0).sum())}, 256-row blocks {nbig}, kept "
          f"{'256-row' if want_big else '16-row'} layout, bit-equal to it alone: {same}", flush=True)
    assert same
    tokens = np.arange(T)                                      # every token: the whole output
    ro = O.route(logits, topk, True)
    assert np.array_equal(ids.cpu().numpy(), ro[1]), "routing ids"
    need = np.unique(ro[1][tokens])
    sub = lambda p: {int(e): p[int(e)].cpu() for e in need}
    ref = O.moe_layer(x, logits, (_Lazy(sub(p13)), _Lazy(sub(e13))), (_Lazy(sub(p2)), _Lazy(sub(e2))), topk, True,
                      tokens=tokens, route_out=ro)
    a, b = bf16_bits_to_f64(O.bf16_bits(out)[ref["tokens"]]), bf16_bits_to_f64(ref["out"])
    r, c = rel_err(a, b), cosine(a, b)
    print(f"  vs oracle on {len(tokens)} tokens: rel {r:.2e} cos {c:.7f}", flush=True)
    assert r < 1e-2 and c >= 0.9999


def test_layer_config5_T256_split_handoff(dev):
    """BASELINE config 5 at T = 256 on split tables as a serving step runs it: apply() signals the router
    (route.split_planned), the router takes the wide path (top-k + input quant, no tables; route.route_step), apply()
    splits the tables on the device (experts with at most split_thr rows on the block stream, the rest in 256-row
    blocks) and uses the router's quant. Every token against the oracle."""
    from r9700_vllm.moe import route
    E, H, I, T, topk = 384, 4096, 2048, 256, 8
    seed = 20261201 + 5000 + T + 1
    (p13, e13), (p2, e2), W13, W2 = make_layer(dev, E, H, I, seed, 116, 126)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    rank = torch.randperm(E, generator=g).float() + 1
    logits = (torch.randn(T, E, generator=g) - 1.1 * torch.log(rank)[None, :]).to(torch.bfloat16)
    xd, ld = x.to(dev), logits.to(dev)
    numel = T * topk

    class Routed:
        _r9k_tables = None

    ex = R9700Mxfp4Experts.standalone(W13.wsr, W2.wsr)
    ex.r9k_layer = Routed()
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    bufs = route.RouteBuffers(dev, E, topk)
    for step in range(2):                                      # the first call signals the router
        wide = route.split_planned(ex.r9k_layer, numel, E)
        assert wide == (step == 1)
        w, ids, ex.r9k_layer._r9k_tables = route.route_step(ld, xd, topk, True, E, bufs, use_ops=False, wide=wide,
                                                            dual_blk=route.dual_wanted(ex.r9k_layer, numel, E))
        ex.apply(out, xd, W13.wq, W2.wq, w, ids, "silu", E, None, None, None, None, None, None, False)
    torch.cuda.synchronize()
    assert K.split_wanted(numel, E, H, I)
    ro = O.route(logits, topk, True)
    assert np.array_equal(ids.cpu().numpy(), ro[1]), "routing ids"
    need = np.unique(ro[1])
    sub = lambda p: {int(e): p[int(e)].cpu() for e in need}
    ref = O.moe_layer(x, logits, (_Lazy(sub(p13)), _Lazy(sub(e13))), (_Lazy(sub(p2)), _Lazy(sub(e2))), topk, True,
                      route_out=ro)
    a, b = bf16_bits_to_f64(O.bf16_bits(out)), bf16_bits_to_f64(ref["out"])
    r, c = rel_err(a, b), cosine(a, b)
    print(f"cfg5 T=256 split hand-off: rel {r:.2e} cos {c:.7f}", flush=True)
    assert r < 1e-2 and c >= 0.9999


@pytest.mark.parametrize("E,H,I,T,zipf", [(384, 4096, 2048, 256, True), (384, 4096, 2048, 256, False),
                                        (288, 2048, 512, 128, False), (288, 2048, 512, 256, True)])
def test_layer_router_dual_layout(dev, monkeypatch, E, H, I, T, zipf):
    """The router's one-launch dual layout (route.route_step with dual_blk: routing, input quant, both table
    layouts and the device's pick in r9k_moe_route_dual) through apply(): bit for bit the output of the same call
    whose experts build the second layout themselves (moe_align + r9k_moe_pick_blocks), whichever layout the
    device keeps; apply() signals the router through the layer object (route.dual_wanted). Split tables off (they
    take these steps by default)."""
    from r9700_vllm.moe import route
    monkeypatch.setattr(K, "SPLIT", False)
    topk = 8
    seed = 20261201 + 7000 + E + T + int(zipf)
    (_, _), (_, _), W13, W2 = make_layer(dev, E, H, I, seed, 116, 126)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    logits = torch.randn(T, E, generator=g)
    if zipf:
        rank = torch.randperm(E, generator=g).float() + 1
        logits = logits - 1.1 * torch.log(rank)[None, :]
    logits = logits.to(torch.bfloat16).to(dev)
    numel = T * topk
    assert numel >= K.DEVICE_BLOCKS_MIN and K.pick_moe_prefill_block(numel, E, H, I) is None

    class Routed:
        _r9k_tables = None

    def run(layer_obj, tables):
        layer_obj._r9k_tables = tables
        ex = R9700Mxfp4Experts.standalone(W13.wsr, W2.wsr)
        ex.r9k_layer = layer_obj
        o = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=dev)
        ex.apply(o, x, W13.wq, W2.wq, w, ids, "silu", E, None, None, None, None, None, None, False)
        torch.cuda.synchronize()
        return o

    bufs = route.RouteBuffers(dev, E, topk)
    lay = Routed()
    # first call: apply() has not spoken yet -> single layout from the router, the experts build the second one
    w, ids, t1 = route.route_step(logits, x, topk, True, E, bufs, use_ops=False,
                                  dual_blk=route.dual_wanted(lay, numel, E))
    assert t1.big is None
    o1 = run(lay, t1)
    assert route.dual_wanted(lay, numel, E) == 256, "apply() must ask the router for both layouts"
    w, ids, t2 = route.route_step(logits, x, topk, True, E, bufs, use_ops=False,
                                  dual_blk=route.dual_wanted(lay, numel, E))
    assert t2.big is not None and t2.xq is not None
    kept_big = int(t2.big[2].item()) > 0
    o2 = run(lay, t2)
    same = torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    print(f"router dual E={E} T={T} zipf={zipf}: kept {'256-row' if kept_big else '16-row'} layout, bit-equal {same}",
          flush=True)
    assert same
    assert not bool(torch.isnan(o2.float()).any())


@pytest.mark.parametrize("M", [4, 16])
def test_dense_mxfp4_linear_config4_decode_full(dev, M):
    """BASELINE config 4 decode widths on the full [17408, 5120] weight through ops.mxfp4_linear."""
    N, Kd = 17408, 5120
    g = torch.Generator().manual_seed(20261201 + 4000 + M)
    packed, e8 = make_experts(1, N, Kd, g)
    W = K.prepare_mxfp4_weights(packed.to(dev), e8.to(dev))
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    out = ops.mxfp4_linear(x.to(dev), W.wq, W.wsr, N, Kd)
    qo, so = O.quant_rows_fp8(x)
    ref = O.grouped_gemm(qo, so, {0: O.mxfp4_dequant(packed[0], e8[0], torch.float32)}, np.zeros(M, dtype=np.int32),
                         1, acc_dtype=torch.float32)
    got = O.bf16_bits(out)
    a, b = bf16_bits_to_f64(got), bf16_bits_to_f64(ref)
    r, c = rel_err(a, b), cosine(a, b)
    print(f"dense cfg4 M={M}: rel {r:.2e} cos {c:.7f} exact {(got == ref).mean():.4f}", flush=True)
    assert r < 2e-3 and c > 0.99999


def test_layer_past_the_buffer_limit_chunks(dev):
    """A routed step whose gate_up output would reach 2 GiB (E=8, hidden 256, intermediate 2048, T = 32768, top-8:
    262144 routed rows x 4096 bf16 columns = 2^31 bytes), which one launch of the 256-row prefill GEMM cannot
    address: apply() runs it as token chunks and the output matches the oracle on sampled tokens."""
    from r9700_vllm.moe.experts import chunk_tokens
    E, H, I, T, topk = 8, 256, 2048, 32768, 8
    assert len(chunk_tokens(T, topk, 2 * I, H, H, I)) == 2
    tokens = np.unique(np.concatenate([[0, T // 2 - 1, T // 2, T - 1],       # both chunks' ends
                                       np.random.default_rng(7).choice(T, 24, replace=False)]))
    run_layer(dev, E, H, I, T, topk, seed=20261201 + 32768, tokens=tokens)


@pytest.mark.parametrize("E,T,H,I,topk,shared", [(288, 1, 2048, 512, 8, False), (288, 8, 2048, 512, 8, True),
                                                 (288, 16, 2048, 512, 8, False), (64, 5, 1024, 1024, 6, False),
                                                 (32, 3, 512, 512, 16, True), (16, 2, 256, 512, 1, False),
                                                 (24, 4, 4096, 2048, 8, False), (12, 3, 320, 1024, 12, True)])
def test_down_sum_equals_three_launches(dev, E, T, H, I, topk, shared):
    """r9k_moe_down_sum (SiLU + quant, down GEMM and top-k sum in one token-major launch) against the three launches
    it replaces on the same gate_up output: bit for bit when K2 = I < 1024 (the down GEMM's single-wave K chain),
    else within fp32 accumulation order (the down GEMM splits K over waves); optional shared-expert term."""
    seed = 20261201 + 9100 + E + T + H + I
    (_, _), (_, _), W13, W2 = make_layer(dev, E, H, I, seed)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    logits = torch.randn(T, E, generator=g).to(torch.bfloat16).to(dev)
    sh = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev) if shared else None
    w, ids = K.moe_topk(logits, topk, True)
    numel = T * topk
    sid, eid, ntpp = K.moe_align(ids, 16, E)
    xq, xs = K.quant_rows_fp8(x)
    tw = w.reshape(-1).float().contiguous()
    gu = torch.empty(numel, 2 * I, dtype=torch.bfloat16, device=dev)
    K.moe_gemm(xq, xs, W13, gu, sid, eid, ntpp, numel, topk, None, num_experts=E, MT=1)
    aq, as_ = K.silu_mul_quant_fp8(gu)
    down = torch.empty(numel, H, dtype=torch.bfloat16, device=dev)
    K.moe_gemm(aq, as_, W2, down, sid, eid, ntpp, numel, 1, tw, num_experts=E, MT=1)
    o3 = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    K.moe_sum(down.view(T, topk, H), sh, o3)
    o1 = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=dev)
    assert K.moe_down_sum(gu, ids, tw, W2, o1, sh), "shape not served"
    torch.cuda.synchronize()
    same = torch.equal(o1.view(torch.int16), o3.view(torch.int16))
    a, b = o1.double(), o3.double()
    r = float((a - b).norm() / b.norm())
    print(f"down_sum E={E} T={T} H={H} I={I} k={topk} shared={shared}: bit-equal {same}, rel {r:.2e}", flush=True)
    if I < 1024:
        assert same
    else:
        assert r < 1e-3 and (o1 != o3).float().mean() < 0.05


def test_down_sum_refuses_unserved_shapes(dev):
    """Shapes the token-major tail does not take return False with nothing launched (apply() then runs the three
    launches): K2 not a multiple of 128 or past 2048, more than 16 slots."""
    E, H = 4, 256
    for I, topk in ((320, 2), (4096, 2), (512, 17)):
        W2 = K.Mxfp4Experts(torch.zeros(E, H * I // 8, dtype=torch.int32, device=dev),
                            torch.zeros(E, I // 32 + 1, H, dtype=torch.uint8, device=dev), H, I)
        gu = torch.zeros(topk, 2 * I, dtype=torch.bfloat16, device=dev)
        ids = torch.zeros(1, topk, dtype=torch.int32, device=dev)
        out = torch.zeros(1, H, dtype=torch.bfloat16, device=dev)
        assert not K.moe_down_sum(gu, ids, torch.ones(topk, device=dev), W2, out)


def decode_gemm(q, s, W, out, M, topk_w=None):
    """The decode-family GEMM (r9k_moe_mxfp4a8) over identity tables, 16-row blocks, at the kernel's own launch shape:
    the two-launch dense path's GEMM as the reference runs it (ops.mxfp4_gemm_q itself takes the dense kernel up to 16
    rows). The one-launch dense kernels split K over waves as that shape does; a launch-table shape with another SK
    sums in another order."""
    tabs = ops.IdentityTables.get(q.device, M, K.MOE_BLOCK)
    K.moe_gemm(q, s, W, out, *tabs, M, 1, topk_w, num_experts=1, MT=1)


@pytest.mark.parametrize("M,N,Kd", [(1, 17408, 5120), (2, 17408, 5120), (4, 17408, 5120), (3, 1024, 2048),
                                    (4, 1024, 2048), (3, 48, 1024), (2, 272, 384), (1, 64, 8192), (4, 64, 8192),
                                    (1, 32, 256), (4, 16, 896), (1, 17408, 4992), (2, 2064, 4864)])
def test_dense_qa_equals_two_launches(dev, M, N, Kd):
    """r9k_dense_mxfp4_qa (the activation quant inside the dense GEMM launch, M <= 4) against quant_rows_fp8 + the
    decode GEMM over identity tables: bit for bit (same K split over waves), and within the GEMM tolerance of the
    oracle."""
    g = torch.Generator().manual_seed(20261201 + 4100 + M + N + Kd)
    packed, e8 = make_experts(1, N, Kd, g)
    W = K.prepare_mxfp4_weights(packed.to(dev), e8.to(dev))
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    xd = x.to(dev)
    one = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    assert K.dense_mxfp4_qa(xd, W, one), "shape not served"
    q, s = K.quant_rows_fp8(xd)
    two = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    decode_gemm(q, s, W, two, M)
    torch.cuda.synchronize()
    same = torch.equal(one.view(torch.int16), two.view(torch.int16))
    qo, so = O.quant_rows_fp8(x)
    ref = O.grouped_gemm(qo, so, {0: O.mxfp4_dequant(packed[0], e8[0], torch.float32)}, np.zeros(M, dtype=np.int32),
                         1, acc_dtype=torch.float32)
    a, b = bf16_bits_to_f64(O.bf16_bits(one)), bf16_bits_to_f64(ref)
    r = rel_err(a, b)
    print(f"dense qa M={M} N={N} K={Kd}: bit-equal to two launches {same}, rel {r:.2e}", flush=True)
    assert same and r < 2e-3 and cosine(a, b) > 0.99999


@pytest.mark.parametrize("M,N,Kd,rw", [(1, 17408, 5120, False), (4, 17408, 5120, False), (16, 17408, 5120, False),
                                       (3, 1024, 2048, True), (7, 1024, 2048, False), (16, 48, 1024, True),
                                       (5, 272, 384, False), (9, 64, 8192, False), (16, 32, 256, False),
                                       (12, 16, 896, True), (2, 2064, 640, False), (1, 2048, 512, True)])
def test_dense_a8_equals_decode_gemm(dev, M, N, Kd, rw):
    """r9k_dense_mxfp4_a8 (the dense weight stream on pre-quantised rows, M <= 16; with row weights as the shared
    expert's down GEMM passes its gate) against the decode GEMM over identity tables on the same codes: bit for bit,
    every row written, and within the GEMM tolerance of the oracle."""
    g = torch.Generator().manual_seed(20261201 + 4200 + M + N + Kd)
    packed, e8 = make_experts(1, N, Kd, g)
    W = K.prepare_mxfp4_weights(packed.to(dev), e8.to(dev))
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    tw = torch.rand(M, generator=g).float() if rw else None
    twd = tw.to(dev) if rw else None
    q, s = K.quant_rows_fp8(x.to(dev))
    one = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    assert K.dense_mxfp4_a8(q, s, W, one, twd), "shape not served"
    two = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    decode_gemm(q, s, W, two, M, twd)
    three = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    ops.mxfp4_gemm_q(q, s, W, three, M, K.pick_cfg(N, Kd, M=M, kind="mxfp4"), topk_w=twd)   # dispatches to a8
    torch.cuda.synchronize()
    assert not torch.isnan(one.float()).any(), "an output was not written"
    same = torch.equal(one.view(torch.int16), two.view(torch.int16))
    assert torch.equal(one.view(torch.int16), three.view(torch.int16))
    qo, so = O.quant_rows_fp8(x)
    ref = O.grouped_gemm(qo, so, {0: O.mxfp4_dequant(packed[0], e8[0], torch.float32)}, np.zeros(M, dtype=np.int32),
                         1, tw.numpy() if rw else None, acc_dtype=torch.float32)
    a, b = bf16_bits_to_f64(O.bf16_bits(one)), bf16_bits_to_f64(ref)
    r = rel_err(a, b)
    print(f"dense a8 M={M} N={N} K={Kd} rw={rw}: bit-equal to the decode GEMM {same}, rel {r:.2e}", flush=True)
    assert same and r < 2e-3 and cosine(a, b) > 0.99999


def test_dense_a8_refuses_unserved(dev):
    """M > 16, K not a multiple of 128 or a row stride that is not 16-byte aligned: False, nothing launched."""
    W = K.Mxfp4Experts(torch.zeros(1, 64 * 320 // 8, dtype=torch.int32, device=dev),
                       torch.zeros(1, 320 // 32 + 1, 64, dtype=torch.uint8, device=dev), 64, 320)
    s = torch.ones(17, dtype=torch.float32, device=dev)
    assert not K.dense_mxfp4_a8(torch.zeros(2, 320, dtype=torch.uint8, device=dev), s, W,
                                torch.empty(2, 64, dtype=torch.bfloat16, device=dev))
    W2 = K.Mxfp4Experts(torch.zeros(1, 64 * 256 // 8, dtype=torch.int32, device=dev),
                        torch.zeros(1, 256 // 32 + 1, 64, dtype=torch.uint8, device=dev), 64, 256)
    assert not K.dense_mxfp4_a8(torch.zeros(17, 256, dtype=torch.uint8, device=dev), s, W2,
                                torch.empty(17, 64, dtype=torch.bfloat16, device=dev))
    qs = torch.zeros(2, 264, dtype=torch.uint8, device=dev)[:, :256]          # row stride 264: not 16-byte aligned
    assert not K.dense_mxfp4_a8(qs, s, W2, torch.empty(2, 64, dtype=torch.bfloat16, device=dev))


def test_dense_qa_refuses_unserved(dev):
    """M > 4, K not a multiple of 128 or unaligned activations: False, nothing launched (ops falls back)."""
    W = K.Mxfp4Experts(torch.zeros(1, 64 * 320 // 8, dtype=torch.int32, device=dev),
                       torch.zeros(1, 320 // 32 + 1, 64, dtype=torch.uint8, device=dev), 64, 320)
    assert not K.dense_mxfp4_qa(torch.zeros(2, 320, dtype=torch.bfloat16, device=dev), W,
                                torch.empty(2, 64, dtype=torch.bfloat16, device=dev))
    W2 = K.Mxfp4Experts(torch.zeros(1, 64 * 256 // 8, dtype=torch.int32, device=dev),
                        torch.zeros(1, 256 // 32 + 1, 64, dtype=torch.uint8, device=dev), 64, 256)
    for M in (5, 17):
        assert not K.dense_mxfp4_qa(torch.zeros(M, 256, dtype=torch.bfloat16, device=dev), W2,
                                    torch.empty(M, 64, dtype=torch.bfloat16, device=dev))


@pytest.mark.parametrize("MT", [1, 2, 4])
def test_decode_gemm_every_launch_shape(dev, MT):
    """r9k_moe_mxfp4a8 at every built launch shape (WV K-tiles a load batch, SK waves splitting K, NPW column tiles a
    wave, as the launch table passes them) over MoE routing tables, against the oracle; a shape not built raises."""
    import itertools
    E, M, topk, N, Kd = 8, 100, 2, 320, 1024
    g = torch.Generator().manual_seed(20261201 + 21000 + MT)
    packed, e8 = make_experts(E, N, Kd, g)
    W = K.prepare_mxfp4_weights(packed.to(dev), e8.to(dev))
    x = (torch.randn(M, Kd, generator=g) * 0.5).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:topk] for _ in range(M)]).to(torch.int32)
    sid, eid, ntpp = (t.to(dev) for t in K.align_block_size_ref(ids, E, 16 * MT))
    xq, xs = K.quant_rows_fp8(x.to(dev))
    qo, so = O.quant_rows_fp8(x)
    ref = O.grouped_gemm(qo, so, {e: O.mxfp4_dequant(packed[e], e8[e]) for e in range(E)}, ids.reshape(-1).numpy(),
                         topk)
    shapes = [c for c in itertools.product(K.BUILT_KNOBS, repeat=3) if K.legal_cfg(c, N, Kd, MT=MT) == c]
    assert len(shapes) >= 18
    for cfg in shapes:
        out = torch.full((M * topk, N), float("nan"), dtype=torch.bfloat16, device=dev)
        K.moe_gemm(xq, xs, W, out, sid, eid, ntpp, M * topk, topk, None, *cfg, num_experts=E, MT=MT)
        a, b = bf16_bits_to_f64(O.bf16_bits(out)), bf16_bits_to_f64(ref)
        assert not np.isnan(a.numpy()).any(), cfg
        assert rel_err(a, b) < 2e-3 and cosine(a, b) > 0.99999, cfg
    with pytest.raises(RuntimeError):
        K.moe_gemm(xq, xs, W, torch.empty(M * topk, N, dtype=torch.bfloat16, device=dev), sid, eid, ntpp, M * topk,
                   topk, None, 3, 1, 1, num_experts=E, MT=MT)


@pytest.mark.parametrize("MT", [1, 2])
def test_decode_gemm_reference_knobs_ignored(dev, MT):
    """The reference's ctypes wrapper passes its gfx1201 (WV, SK, NPW) sets to r9k_moe_mxfp4a8 without the launch
    shape bit (MT bit 5): every such call returns 0 and gives the bits of the kernel's own choice (all three 0)."""
    E, M, topk, N, Kd = 8, 64, 2, 320, 2560
    g = torch.Generator().manual_seed(20261201 + 23000 + MT)
    packed, e8 = make_experts(E, N, Kd, g)
    W = K.prepare_mxfp4_weights(packed.to(dev), e8.to(dev))
    x = (torch.randn(M, Kd, generator=g) * 0.5).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:topk] for _ in range(M)]).to(torch.int32)
    sid, eid, ntpp = (t.to(dev) for t in K.align_block_size_ref(ids, E, 16 * MT))
    xq, xs = K.quant_rows_fp8(x.to(dev))
    numel = M * topk
    max_blocks = min(eid.numel(), (numel + 16 * MT - 1) // (16 * MT) + min(numel, E))

    def run(WV, SK, NPW):
        out = torch.full((numel, N), float("nan"), dtype=torch.bfloat16, device=dev)
        rc = K.lib().r9k_moe_mxfp4a8(
            xq.data_ptr(), xs.data_ptr(), W.wq.data_ptr(), W.wsr.data_ptr(), W.wsr.data_ptr() + (Kd // 32) * N,
            out.data_ptr(), sid.data_ptr(), eid.data_ptr(), ntpp.data_ptr(), 0, W.estride, W.estride, max_blocks,
            numel, topk, Kd, N, WV, SK, NPW, MT, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert rc == 0, (WV, SK, NPW, rc)
        return O.bf16_bits(out)

    auto = run(0, 0, 0)
    for knobs in ((2, 4, 2), (4, 2, 1), (2, 5, 2), (4, 1, 1), (8, 10, 3)):
        assert np.array_equal(run(*knobs), auto), knobs


@pytest.mark.parametrize("M,N,Kd", [(17, 1024, 2048), (40, 1024, 2048), (100, 1024, 2048), (48, 17408, 5120)])
def test_dense_linear_tuned_shapes(dev, M, N, Kd):
    """ops.mxfp4_linear between the dense weight stream's 16 rows and the prefill kernel's 128: the decode kernel at
    the launch table's shape (kernels/tuned.json), against the oracle on 24 sampled rows."""
    g = torch.Generator().manual_seed(20261201 + 22000 + M + N)
    packed, e8 = make_experts(1, N, Kd, g)
    W = K.prepare_mxfp4_weights(packed.to(dev), e8.to(dev))
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    print(f"dense tuned M={M} N={N} K={Kd}: cfg {K.pick_cfg(N, Kd, M=M, kind='mxfp4')}", flush=True)
    out = ops.mxfp4_linear(x.to(dev), W.wq, W.wsr, N, Kd)
    rows = np.sort(np.random.default_rng(M).choice(M, min(M, 24), replace=False))
    qo, so = O.quant_rows_fp8(x[torch.from_numpy(rows)])
    ref = O.grouped_gemm(qo, so, {0: O.mxfp4_dequant(packed[0], e8[0], torch.float32)}, np.zeros(rows.size, np.int32),
                         1, acc_dtype=torch.float32)
    a, b = bf16_bits_to_f64(O.bf16_bits(out)[rows]), bf16_bits_to_f64(ref)
    assert rel_err(a, b) < 2e-3 and cosine(a, b) > 0.99999
