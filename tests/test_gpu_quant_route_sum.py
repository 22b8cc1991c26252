"""GPU parity: per-row fp8 quant, SiLU-gating quant, routing + align tables, top-k sum -- through the C-ABI against
the CPU oracle. Integer outputs (fp8 codes and scales, ids, tables, bf16 sums) bit-exact; router weights within
2e-6 (tests/test_moe_route_r9k.py:78 of the reference)."""
import numpy as np
import pytest
import torch

from helpers import check_tables
from oracle import oracle as O
from r9700_vllm.kernels import moe as K
from r9700_vllm.moe import route

pytestmark = pytest.mark.gpu


def u8(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.uint8).cpu().numpy()


@pytest.mark.parametrize("M,Kd,scale", [(1, 2048, 1.0), (64, 2048, 1.0), (8192, 2048, 1.0), (16, 5120, 3.0),
                                        (4, 4096, 1e-4), (5, 96, 1.0), (3, 100, 1.0), (2, 9000, 1.0)])
def test_quant_rows_fp8_bit_exact(dev, M, Kd, scale):
    print(f"quant M={M} K={Kd}", flush=True)
    g = torch.Generator().manual_seed(M + Kd)
    x = (torch.randn(M, Kd, generator=g) * scale).to(torch.bfloat16)
    q, s = K.quant_rows_fp8(x.to(dev))
    qo, so = O.quant_rows_fp8(x)
    assert np.array_equal(u8(q), qo)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))


def test_quant_rows_fp8_strided_and_edge_rows(dev):
    base = torch.zeros(4, 80)
    base[1, 3], base[1, 4] = 3.0e38, -1.0
    base[2] = torch.linspace(-1e-3, 1e-3, 80)
    base[2, 0] = 5.0
    base[3], base[3, 7] = -1e-30, 1.0
    xb = base.to(torch.bfloat16)
    xd = xb.to(dev)[:, :64]                      # row stride 80 > K = 64
    q, s = K.quant_rows_fp8(xd)
    qo, so = O.quant_rows_fp8(xb[:, :64].contiguous())
    assert np.array_equal(u8(q), qo) and np.array_equal(s.cpu().numpy(), so)


@pytest.mark.parametrize("Kd", [64, 2048])
def test_quant_rows_fp8_nonfinite_rows(dev, Kd):
    """Rows holding NaN or +-inf take the checked conversion (the row maximum passes over NaN; an inf maximum gives
    inv = 0, finite values -> +-0 and inf * 0 -> NaN -> sign | 0x7f); finite rows at the bf16 extremes (the largest
    finite value, values under the 1e-12 floor, zeros) take the unchecked one. Codes and scale bits equal the
    oracle's, standalone and in the fused top-k + quant launch."""
    print(f"quant non-finite K={Kd}", flush=True)
    g = torch.Generator().manual_seed(Kd)
    x = torch.randn(12, Kd, generator=g)
    x[0, 5] = float("nan")
    x[1] = float("nan")
    x[2, 9] = float("inf")
    x[3, Kd - 1] = float("-inf")
    x[4] = float("inf")
    x[5, 3], x[5, 4] = float("inf"), float("nan")
    x[6, 0] = 3.3895313892515355e38                     # the largest finite bf16
    x[7] = 1e-30
    x[8] = 0.0
    x[9, ::3] = -0.0
    x[10] = -3.0e38
    xb = x.to(torch.bfloat16)
    qo, so = O.quant_rows_fp8(xb)
    q, s = K.quant_rows_fp8(xb.to(dev))
    assert np.array_equal(u8(q), qo)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    logits = torch.randn(12, 288, generator=g).to(torch.bfloat16).to(dev)
    r = K.moe_topk_quant(logits, 8, True, xb.to(dev))
    assert r is not None
    assert np.array_equal(u8(r[2]), qo)
    assert np.array_equal(r[3].cpu().numpy().view(np.uint32), so.view(np.uint32))


def test_quant_rows_fp8_gate(dev):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(37, 2048, generator=g).to(torch.bfloat16)
    wg = (torch.randn(2048, generator=g) * 0.02).to(torch.bfloat16)
    q, s, gate = K.quant_rows_fp8_gate(x.to(dev), wg.to(dev))
    qo, so = O.quant_rows_fp8(x)
    assert np.array_equal(u8(q), qo) and np.array_equal(s.cpu().numpy(), so)
    ref = torch.sigmoid((x.float() @ wg.float()).to(torch.bfloat16).float()).to(torch.bfloat16).float()
    assert (gate.cpu() - ref).abs().max().item() <= 2 ** -8        # one bf16 ulp of a value in (0, 1)


@pytest.mark.parametrize("M,I", [(65536, 512), (16384, 2048)])
def test_silu_mul_quant_fp8_streaming_size(dev, M, I):
    """From 64 MiB of input (config 3's 134 MB gate_up output, config 5's 268 MB at T = 4096) the launch takes
    non-temporal row loads: its rows equal, bit for bit, the same rows converted from slices small enough for the
    plain loads (which test_silu_mul_quant_fp8 holds against the oracle)."""
    g = torch.Generator(device=dev).manual_seed(M + I)
    gu = (torch.randn(M, 2 * I, generator=g, device=dev) * 2).to(torch.bfloat16)
    assert gu.numel() * 2 >= 64 << 20
    q, s = K.silu_mul_quant_fp8(gu)
    for lo, hi in [(0, 512), (M // 2 - 3, M // 2 + 300), (M - 37, M)]:
        qs, ss = K.silu_mul_quant_fp8(gu[lo:hi].contiguous())
        assert torch.equal(q[lo:hi].view(torch.uint8), qs.view(torch.uint8)), (lo, hi)
        assert torch.equal(s[lo:hi].view(torch.int32), ss.view(torch.int32)), (lo, hi)


@pytest.mark.parametrize("M,I,scale", [(37, 320, 2.0), (512, 512, 1.0), (64, 2048, 1.0), (3, 100, 1.0)])
def test_silu_mul_quant_fp8(dev, M, I, scale):
    g = torch.Generator().manual_seed(M * I)
    gu = (torch.randn(M, 2 * I, generator=g) * scale).to(torch.bfloat16)
    q, s = K.silu_mul_quant_fp8(gu.to(dev))
    qo, so, act = O.silu_mul_quant_fp8(gu)
    # exp() may differ by an fp32 ulp between the device and libm: codes may move by one step at a rounding edge
    qd = u8(q)
    same = (qd == qo).mean()
    assert same >= 0.999, same
    assert np.all(np.abs(O.e4m3_table()[qd] - O.e4m3_table()[qo])[qd != qo] <= np.abs(O.e4m3_table()[qo])[qd != qo] / 8 + 2 ** -9)
    assert np.allclose(s.cpu().numpy(), so, rtol=1e-6, atol=0)
    deq = O.e4m3_table()[qd] * s.cpu().numpy()[:, None]
    gf, uf = gu.float()[:, :I], gu.float()[:, I:]
    ref = (torch.nn.functional.silu(gf) * uf).numpy()
    assert np.linalg.norm(deq - ref) / np.linalg.norm(ref) < 6e-2      # the reference's quant round-trip gate


def test_silu_mul_quant_fp8_special_values(dev):
    """Non-finite products take the encoder's fallback block: a NaN product encodes as sign | 0x7f, a row whose
    maximum is inf quantises with inv = 0 (finite products -> +-0, inf * 0 -> NaN -> sign | 0x7f), a product past
    the fp32 range overflows to inf. The codes of those positions match the oracle's bit routine exactly."""
    g = torch.Generator().manual_seed(77)
    M, I = 8, 512
    gu = torch.randn(M, 2 * I, generator=g)
    gu[0, 3] = float("nan"); gu[0, I + 9] = float("nan")          # NaN gate / NaN up in a finite row
    gu[1, I + 5] = float("inf"); gu[1, I + 6] = float("-inf")     # inf up: the row maximum is inf
    gu[2, 7] = 3e38; gu[2, I + 7] = 3e38                           # silu(3e38) * 3e38 overflows to inf
    gu[3, :I] = float("-inf")                                      # silu(-inf) = -inf / (1 + inf) = NaN
    gu[4, 11] = 200.0; gu[4, I + 11] = 2.0                         # an ordinary large product
    gu = gu.to(torch.bfloat16)
    q, s = K.silu_mul_quant_fp8(gu.to(dev))
    qo, so, _ = O.silu_mul_quant_fp8(gu)
    qd = u8(q)
    # a NaN's sign bit is not specified (the GPU's default NaN is positive, x86's negative): compare NaN codes as
    # 0x7f with either sign, everything else exactly where no exp() rounding can matter (rows with inv = 0 or a
    # NaN-only row)
    special = (qo & 0x7F) == 0x7F
    assert special.sum() >= 4
    assert np.array_equal(qd[special] & 0x7F, qo[special] & 0x7F)
    for r in (1, 2, 3):
        assert np.array_equal(qd[r][~special[r]], qo[r][~special[r]]), r
    assert (qd == qo)[~special].mean() >= 0.99
    sd = s.cpu().numpy()
    assert np.array_equal(np.isnan(sd), np.isnan(so)) and np.array_equal(np.isinf(sd), np.isinf(so))


@pytest.mark.parametrize("M,E,topk,blk", [(1, 288, 8, 16), (8, 288, 8, 16), (16, 288, 8, 16), (64, 288, 8, 16),
                                          (37, 512, 10, 32), (256, 384, 8, 64), (5, 48, 6, 16), (300, 100, 10, 16),
                                          (512, 288, 8, 16), (300, 1024, 8, 16), (100, 700, 16, 32)])
@pytest.mark.parametrize("renorm", [True, False])
def test_moe_route_fused(dev, M, E, topk, blk, renorm):
    print(f"route M={M} E={E} topk={topk} blk={blk} renorm={renorm}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + E)
    logits = torch.randn(M, E, generator=g).to(torch.bfloat16)
    numel = M * topk
    cap = route.capacity(numel, E, blk)
    guard = 64
    s_ = torch.full((cap + guard,), -9, dtype=torch.int32, device=dev)
    e_ = torch.full((cap // blk + guard,), -9, dtype=torch.int32, device=dev)
    n_ = torch.zeros(1, dtype=torch.int32, device=dev)
    scratch = torch.zeros(route.scratch_ints(E), dtype=torch.int32, device=dev)
    w, ids = route.moe_route(logits.to(dev), topk, renorm, blk, s_[:cap], e_[:cap // blk], n_, scratch)
    wo, ido = O.route(logits, topk, renorm)
    assert np.array_equal(ids.cpu().numpy(), ido)
    assert np.abs(w.cpu().numpy() - wo).max() < 2e-6
    so, eo, no = O.align(ido, E, blk)
    s_h, e_h = s_.cpu().numpy(), e_.cpu().numpy()
    assert np.array_equal(s_h[:cap], so) and np.array_equal(e_h[:cap // blk], eo) and n_.item() == no[0]
    assert np.all(s_h[cap:] == -9) and np.all(e_h[cap // blk:] == -9), "wrote past the tables"
    assert not scratch.any()
    check_tables(so, eo, no, ido, blk, numel, E)


@pytest.mark.parametrize("M,E,topk,zipf,quant", [(128, 288, 8, False, True), (256, 384, 8, True, True),
                                                 (256, 384, 8, True, False), (512, 64, 8, False, True),
                                                 (300, 1024, 8, True, True), (130, 288, 8, True, False)])
def test_moe_route_dual(dev, M, E, topk, zipf, quant):
    """r9k_moe_route_dual: routing (bit-exact ids against the oracle), both table layouts and the device's pick
    (r9k_moe_pick_blocks' rule on the oracle's counts), the kept layout's tables bit-exact against the oracle's align
    (the 256-row one over its live entries), the other's ntpp 0, and the activation quant's bytes."""
    print(f"route_dual M={M} E={E} topk={topk} zipf={zipf} quant={quant}", flush=True)
    g = torch.Generator().manual_seed(M * 13 + E)
    logits = torch.randn(M, E, generator=g)
    if zipf:
        rank = torch.randperm(E, generator=g).float() + 1
        logits = logits - 1.1 * torch.log(rank)[None, :]
    logits = logits.to(torch.bfloat16)
    H = 2048
    x = (torch.randn(M, H, generator=g) * 2.0).to(torch.bfloat16).to(dev)
    numel = M * topk
    blk, bb, min_rows = 16, 256, K.DEVICE_MIN_ROWS
    i32 = dict(dtype=torch.int32, device=dev)
    cap, capb = route.capacity(numel, E, blk), route.capacity(numel, E, bb)
    s_, e_, n_ = torch.full((cap,), -9, **i32), torch.full((cap // blk,), -9, **i32), torch.full((1,), -9, **i32)
    sb, eb, nb = torch.full((capb,), -9, **i32), torch.full((capb // bb,), -9, **i32), torch.full((1,), -9, **i32)
    scratch = torch.zeros(route.scratch_ints(E), **i32)
    w, ids, xq, xs = route.moe_route_dual(logits.to(dev), topk, True, blk, s_, e_, n_, scratch, x if quant else None,
                                          bb, sb, eb, nb, min_rows)
    torch.cuda.synchronize()
    wo, ido = O.route(logits, topk, True)
    assert np.array_equal(ids.cpu().numpy(), ido)
    assert np.abs(w.cpu().numpy() - wo).max() < 2e-6
    counts = np.bincount(ido.reshape(-1), minlength=E)
    nbig = int(((counts + bb - 1) // bb).sum())
    want_big = nbig > 0 and numel >= min_rows * nbig
    so, eo, no = O.align(ido, E, blk)
    sbo, ebo, nbo = O.align(ido, E, bb)
    print(f"  nbig {nbig} -> {'256-row' if want_big else '16-row'} layout", flush=True)
    if want_big:
        assert n_.item() == 0 and nb.item() == nbo[0]
        assert np.array_equal(sb.cpu().numpy()[:nbo[0]], sbo[:nbo[0]])
        assert np.array_equal(eb.cpu().numpy()[:nbo[0] // bb], ebo[:nbo[0] // bb])
    else:
        assert nb.item() == 0 and n_.item() == no[0]
        assert np.array_equal(s_.cpu().numpy(), so) and np.array_equal(e_.cpu().numpy(), eo)
    assert not scratch.any()
    if quant:
        q, s2 = K.quant_rows_fp8(x)
        assert torch.equal(xq.view(torch.uint8), q.view(torch.uint8)) and torch.equal(xs, s2)
    else:
        assert xq.numel() == 0 and xs.numel() == 0


@pytest.mark.parametrize("M,E,topk,blk,H,ldx", [(1, 288, 8, 16, 2048, 2048), (64, 288, 8, 16, 2048, 2048),
                                                 (37, 384, 8, 16, 4096, 4096), (13, 100, 6, 32, 520, 528),
                                                 (16, 512, 10, 16, 2048, 2560),
                                                 (100, 288, 8, 16, 2048, 2048),     # M > 64: one wave a row
                                                 (512, 288, 8, 16, 2048, 2048), (300, 384, 8, 32, 4096, 4104),
                                                 (600, 288, 8, 16, 2048, 2048),     # numel > 4096: two launches
                                                 (8, 288, 8, 16, 8192, 8192)])      # H > 4096: two launches
def test_moe_route_quant(dev, M, E, topk, blk, H, ldx):
    """Routing + tables + the activation quant in one launch: every output bit-exact against the oracle, and the
    quant bytes equal to r9k_quant_rows_fp8's."""
    print(f"route_quant M={M} E={E} topk={topk} blk={blk} H={H} ldx={ldx}", flush=True)
    g = torch.Generator().manual_seed(M * 11 + H)
    logits = torch.randn(M, E, generator=g).to(torch.bfloat16)
    xb = (torch.randn(M, ldx, generator=g) * 3.0).to(torch.bfloat16)
    xb[0, :H] = 0.0                                                    # all-zero row: amax clamps to 1e-12
    x = xb.to(dev)[:, :H]
    numel = M * topk
    cap = route.capacity(numel, E, blk)
    s_ = torch.full((cap + 64,), -9, dtype=torch.int32, device=dev)
    e_ = torch.full((cap // blk + 64,), -9, dtype=torch.int32, device=dev)
    n_ = torch.zeros(1, dtype=torch.int32, device=dev)
    scratch = torch.zeros(route.scratch_ints(E), dtype=torch.int32, device=dev)
    for rep in range(2):                                               # a second call on the same buffers
        w, ids, xq, xs = route.moe_route_quant(logits.to(dev), topk, True, blk, s_[:cap], e_[:cap // blk], n_,
                                               scratch, x)
    torch.cuda.synchronize()
    wo, ido = O.route(logits, topk, True)
    assert np.array_equal(ids.cpu().numpy(), ido)
    assert np.abs(w.cpu().numpy() - wo).max() < 2e-6
    so, eo, no = O.align(ido, E, blk)
    assert np.array_equal(s_[:cap].cpu().numpy(), so) and np.array_equal(e_[:cap // blk].cpu().numpy(), eo)
    assert n_.item() == no[0]
    assert bool((s_[cap:] == -9).all()) and bool((e_[cap // blk:] == -9).all()), "wrote past the tables"
    qo, so_ = O.quant_rows_fp8(xb[:, :H])
    assert np.array_equal(u8(xq), qo) and np.array_equal(xs.cpu().numpy().view(np.uint32), so_.view(np.uint32))
    q2, s2 = K.quant_rows_fp8(x)
    assert torch.equal(xq.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(xs, s2)
    w2, ids2 = route.moe_route(logits.to(dev), topk, True, blk, s_[:cap], e_[:cap // blk], n_, scratch)
    assert torch.equal(w, w2) and torch.equal(ids, ids2)
    assert not scratch.any()


def test_moe_route_degenerate_rows(dev):
    """NaN, +-inf, all-equal and -3e38 rows, E not a multiple of 64 (tests/test_moe_route_r9k.py:84-104)."""
    for Ed in (512, 100, 48):
        M, tk = 24, 10
        g = torch.Generator().manual_seed(Ed)
        x = torch.randn(M, Ed, generator=g) * 2
        x[0] = float("nan"); x[1, :5] = float("nan"); x[2] = float("inf"); x[3] = float("-inf"); x[4] = 0.0
        x[5] = 1.0; x[6, ::2] = float("inf"); x[7] = -3e38
        x = x.to(torch.bfloat16)
        blk = 16
        cap = route.capacity(M * tk, Ed, blk)
        s_ = torch.full((cap + 64,), -9, dtype=torch.int32, device=dev)
        e_ = torch.full((cap // blk + 64,), -9, dtype=torch.int32, device=dev)
        n_ = torch.zeros(1, dtype=torch.int32, device=dev)
        sc = torch.zeros(route.scratch_ints(Ed), dtype=torch.int32, device=dev)
        w, ids = route.moe_route(x.to(dev), tk, True, blk, s_[:cap], e_[:cap // blk], n_, sc)
        wo, ido = O.route(x, tk, True)
        assert np.array_equal(ids.cpu().numpy(), ido)
        assert np.isfinite(w.cpu().numpy()).all() and np.abs(w.cpu().numpy() - wo).max() < 2e-6
        assert bool((s_[cap:] == -9).all()) and bool((e_[cap // blk:] == -9).all())
        check_tables(s_[:cap].cpu().numpy(), e_[:cap // blk].cpu().numpy(), n_.cpu().numpy(), ido, blk, M * tk, Ed)


@pytest.mark.parametrize("M,E,topk", [(37, 512, 16), (70, 288, 8), (33, 384, 8), (5, 100, 10), (64, 48, 6),
                                      (40, 256, 8), (19, 160, 4), (9, 7, 2), (11, 1024, 8), (1, 2, 2)])
def test_moe_topk_degenerate_rows(dev, M, E, topk):
    """moe_topk (the wide launches' top-k: four rows a wave for even E <= 512, else one row a wave) and the fused
    top-k + quant on NaN, +-inf, all-equal, zero and -3e38 rows and M not a multiple of the rows a workgroup
    routes: ids equal the oracle's, weights within 2e-6, and the two launches agree bit for bit."""
    print(f"topk degenerate M={M} E={E} topk={topk}", flush=True)
    g = torch.Generator().manual_seed(M * 1000 + E)
    x = torch.randn(M, E, generator=g) * 2
    for r, fill in enumerate([float("nan"), None, float("inf"), float("-inf"), 0.0, 1.0, None, -3e38]):
        if r >= M:
            break
        if r == 1:
            x[1, : min(5, E)] = float("nan")
        elif r == 6:
            x[6, ::2] = float("inf")
        else:
            x[r] = fill
    xb = x.to(torch.bfloat16)
    w, ids = K.moe_topk(xb.to(dev), topk, True)
    wo, ido = O.route(xb, topk, True)
    assert np.array_equal(ids.cpu().numpy(), ido)
    assert np.isfinite(w.cpu().numpy()).all() and np.abs(w.cpu().numpy() - wo).max() < 2e-6
    xa = (torch.randn(M, 256, generator=g)).to(torch.bfloat16).to(dev)
    r = K.moe_topk_quant(xb.to(dev), topk, True, xa)
    assert r is not None
    assert torch.equal(r[1], ids) and torch.equal(r[0], w)
    q, s = K.quant_rows_fp8(xa)
    assert torch.equal(r[2].view(torch.uint8), q.view(torch.uint8)) and torch.equal(r[3], s)


def test_moe_route_large_m_path(dev):
    """numel above the one-workgroup limit: top-k kernel + single-workgroup table launch."""
    M, E, topk, blk = 1024, 288, 8, 64
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(M, E, generator=g).to(torch.bfloat16)
    cap = route.capacity(M * topk, E, blk)
    s_ = torch.empty(cap, dtype=torch.int32, device=dev)
    e_ = torch.empty(cap // blk, dtype=torch.int32, device=dev)
    n_ = torch.zeros(1, dtype=torch.int32, device=dev)
    w, ids = route.moe_route(logits.to(dev), topk, True, blk, s_, e_, n_,
                             torch.zeros(route.scratch_ints(E), dtype=torch.int32, device=dev))
    wo, ido = O.route(logits, topk, True)
    so, eo, no = O.align(ido, E, blk)
    assert np.array_equal(ids.cpu().numpy(), ido) and np.abs(w.cpu().numpy() - wo).max() < 2e-6
    assert np.array_equal(s_.cpu().numpy(), so) and np.array_equal(e_.cpu().numpy(), eo) and n_.item() == no[0]


@pytest.mark.parametrize("T,E,topk,blk,zipf", [(8192, 288, 8, 64, False), (4096, 384, 8, 64, True),
                                               (256, 384, 8, 16, True), (3000, 64, 4, 128, False),
                                               (8192, 288, 8, 256, False), (600, 1024, 16, 256, True),
                                               (2049, 7, 2, 1, False)])
def test_topk_and_align_multiblock(dev, T, E, topk, blk, zipf):
    print(f"topk+align T={T} E={E} blk={blk} zipf={zipf}", flush=True)
    g = torch.Generator().manual_seed(T + E)
    logits = torch.randn(T, E, generator=g)
    if zipf:
        rank = torch.randperm(E, generator=g).float() + 1
        logits = logits - 1.1 * torch.log(rank)[None, :]
    logits = logits.to(torch.bfloat16)
    w, ids = K.moe_topk(logits.to(dev), topk, True)
    wo, ido = O.route(logits, topk, True)
    assert np.array_equal(ids.cpu().numpy(), ido) and np.abs(w.cpu().numpy() - wo).max() < 2e-6
    for rep in range(2):                                  # the second call reuses the histogram scratch
        s_, e_, n_ = K.moe_align(ids, blk, E)
        so, eo, no = O.align(ido, E, blk)
        assert np.array_equal(s_.cpu().numpy(), so) and np.array_equal(e_.cpu().numpy(), eo)
        assert n_.item() == no[0]
    # the multi-workgroup path's arrival counter (first int of the zero-once scratch) is left zero
    assert int(K._align_scratch(torch.device(dev), 1)[0]) == 0


@pytest.mark.parametrize("T", [40, 3000])
def test_align_skips_foreign_experts_wide(dev, T):
    """Expert-map holes at both table builders (one workgroup, and chunked over workgroups above 4096 rows)."""
    g = torch.Generator().manual_seed(T)
    ids = torch.stack([torch.randperm(64, generator=g)[:4] for _ in range(T)]).to(torch.int32)
    emap = torch.tensor([i // 2 if i % 2 == 0 else -1 for i in range(64)], dtype=torch.int32)
    s_, e_, n_ = K.moe_align(ids.to(dev), 64, 32, emap.to(dev))
    mapped = emap[ids.long()].numpy()
    so, eo, no = O.align(mapped, 32, 64)
    assert np.array_equal(s_.cpu().numpy(), so) and np.array_equal(e_.cpu().numpy(), eo) and n_.item() == no[0]


def test_align_skips_foreign_experts(dev):
    """Ids mapped to -1 (an expert map: experts on another rank) are left out of the tables."""
    g = torch.Generator().manual_seed(3)
    ids = torch.stack([torch.randperm(16, generator=g)[:4] for _ in range(40)]).to(torch.int32)
    emap = torch.tensor([i if i < 10 else -1 for i in range(16)], dtype=torch.int32)
    s_, e_, n_ = K.moe_align(ids.to(dev), 16, 10, emap.to(dev))
    mapped = emap[ids.long()].numpy()
    so, eo, no = O.align(mapped, 10, 16)
    assert np.array_equal(s_.cpu().numpy(), so) and np.array_equal(e_.cpu().numpy(), eo) and n_.item() == no[0]


@pytest.mark.parametrize("M,topk,N", [(1, 8, 2048), (64, 8, 2048), (37, 10, 2560), (8192, 8, 2048), (3, 4, 320)])
def test_moe_sum_bit_exact(dev, M, topk, N):
    g = torch.Generator().manual_seed(M + N)
    down = (torch.randn(M, topk, N, generator=g) * 0.5).to(torch.bfloat16)
    shared = (torch.randn(M, N, generator=g) * 0.5).to(torch.bfloat16)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    K.moe_sum(down.to(dev), None, out)
    assert np.array_equal(O.bf16_bits(out), O.moe_sum(down))
    out2 = torch.empty(M, N + 16, dtype=torch.bfloat16, device=dev)[:, :N]          # strided output rows
    K.moe_sum(down.to(dev), shared.to(dev), out2)
    assert np.array_equal(O.bf16_bits(out2), O.moe_sum(down, shared))


@pytest.mark.parametrize("M,E,topk,H", [(8192, 288, 8, 2048), (300, 288, 8, 2048), (4096, 384, 8, 4096),
                                        (257, 64, 4, 512), (33, 1024, 16, 136), (5, 16, 2, 100)])
def test_moe_topk_quant(dev, M, E, topk, H):
    """r9k_moe_topk_quant: the top-k and the activation quant of one launch equal moe_topk's and quant_rows_fp8's
    outputs bit for bit (H % 8 != 0 returns None: nothing launched, the caller runs the two calls)."""
    g = torch.Generator().manual_seed(20261201 + 9000 + M + E + H)
    logits = torch.randn(M, E, generator=g).to(torch.bfloat16).to(dev)
    x = (torch.randn(M, H, generator=g) * 3).to(torch.bfloat16).to(dev)
    r = K.moe_topk_quant(logits, topk, True, x)
    if H % 8:
        assert r is None
        return
    w, ids, xq, xs = r
    w0, ids0 = K.moe_topk(logits, topk, True)
    xq0, xs0 = K.quant_rows_fp8(x)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids0) and torch.equal(w, w0)
    assert torch.equal(xq.view(torch.uint8), xq0.view(torch.uint8)) and torch.equal(xs, xs0)


@pytest.mark.parametrize("T,E,topk,blk", [(256, 384, 8, 256), (1, 288, 8, 256), (700, 64, 6, 16), (4096, 288, 8, 64)])
def test_align_live_only(dev, T, E, topk, blk):
    """r9k_moe_align_live: the tables up to ntpp equal r9k_moe_align's bit for bit, and nothing past ntpp is
    written (the buffers' sentinel survives) -- one workgroup below 4097 routed rows, the multi-workgroup path
    above."""
    g = torch.Generator().manual_seed(20261201 + 13000 + T + E)
    logits = torch.randn(T, E, generator=g).to(torch.bfloat16).to(dev)
    ids = K.moe_topk(logits, topk, True)[1]
    numel = T * topk
    s0, e0, n0 = K.moe_align(ids, blk, E)
    L = K.lib()
    cap = K.capacity(numel, E, blk)
    s1 = torch.full((cap,), -777, dtype=torch.int32, device=dev)
    e1 = torch.full((cap // blk,), -777, dtype=torch.int32, device=dev)
    n1 = torch.zeros(1, dtype=torch.int32, device=dev)
    scratch = K._align_scratch(dev, L.r9k_moe_align_scratch_ints(numel, E))
    assert L.r9k_moe_align_live(ids.data_ptr(), numel, E, blk, s1.data_ptr(), e1.data_ptr(), n1.data_ptr(),
                                scratch.data_ptr(), scratch.numel(), torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    n = int(n0.item())
    print(f"align live T={T} E={E} k={topk} blk={blk}: ntpp {n} of capacity {cap}", flush=True)
    assert int(n1.item()) == n
    assert torch.equal(s1[:n], s0[:n]) and torch.equal(e1[: n // blk], e0[: n // blk])
    assert bool((s1[n:] == -777).all()) and bool((e1[n // blk:] == -777).all())


@pytest.mark.parametrize("E,T,topk,thr,zipf", [(384, 4096, 8, 16, True), (384, 256, 8, 16, True),
                                               (64, 300, 4, 8, False), (288, 1024, 8, 0, False),
                                               (128, 1000, 4, 10000, True), (16, 3, 2, 1, False),
                                               (1024, 600, 16, 3, True)])
def test_align_split_tables(dev, E, T, topk, thr, zipf):
    """r9k_moe_align_split: the big table (experts with more than thr rows, 256-row blocks) and the small table
    (the others, 16-row blocks) each equal the oracle's canonical align over the ids of its own experts (the other
    ids left out) up to ntpp, bit for bit; together they place every routed row once. One workgroup up to 4096
    routed rows, the count + two scatter launches above."""
    g = torch.Generator().manual_seed(20261201 + 17000 + E + T + thr)
    logits = torch.randn(T, E, generator=g)
    if zipf:
        logits = logits - 1.1 * torch.log(torch.randperm(E, generator=g).float() + 1)[None, :]
    ids = K.moe_topk(logits.to(torch.bfloat16).to(dev), topk, True)[1]
    numel = T * topk
    big, small = K.moe_align_split(ids, E, thr, 256, 16)
    torch.cuda.synchronize()
    flat = ids.reshape(-1).cpu().numpy()
    cnt = np.bincount(flat, minlength=E)
    placed = []
    for (s, e, n), blk, keep in ((big, 256, cnt > thr), (small, 16, (cnt > 0) & (cnt <= thr))):
        want = np.where(keep[flat], flat, -1).astype(np.int32)
        so, eo, no = O.align(want, E, blk)
        m = int(n.item())
        assert m == int(no[0]), (blk, m, int(no[0]))
        assert np.array_equal(s[:m].cpu().numpy(), so[:m]) and np.array_equal(e[: m // blk].cpu().numpy(), eo[: m // blk])
        sm = s[:m].cpu().numpy()
        placed.append(sm[sm < numel])
    print(f"align split E={E} T={T} k={topk} thr={thr}: big ntpp {int(big[2].item())}, small ntpp "
          f"{int(small[2].item())} ({int(((cnt > 0) & (cnt <= thr)).sum())} small experts)", flush=True)
    assert np.array_equal(np.sort(np.concatenate(placed)), np.arange(numel))
