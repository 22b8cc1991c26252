"""Host-side logic of the package (CPU only, no kernel launches): the gfx950 weight layouts and their inverses,
table sizing and the tile-selection helpers that mirror the reference's kernels/moe.py."""
import numpy as np
import pytest
import torch

from helpers import make_experts
from r9700_vllm.kernels import moe as K


@pytest.mark.parametrize("N,Kd", [(16, 128), (32, 2048), (48, 320), (64, 160), (16, 32), (32, 544)])
def test_permute_fragments_lane_layout(N, Kd):
    g = torch.Generator().manual_seed(N + Kd)
    packed, _ = make_experts(2, N, Kd, g)
    wq = K.permute_fragments(packed)
    assert wq.dtype == torch.int32 and wq.shape == (2, N * Kd // 8)
    b = wq.view(torch.uint8).reshape(2, -1)
    nkf, G = Kd // 128, (Kd % 128) // 32
    for e in range(2):
        for nt in range(N // 16):
            base = nt * 8 * Kd
            for kt in range(nkf + (1 if G else 0)):
                groups = 4 if kt < nkf else G
                for lane in range(16 * groups):
                    gg, r = lane >> 4, lane & 15
                    got = b[e, base + kt * 1024 + lane * 16: base + kt * 1024 + lane * 16 + 16]
                    want = packed[e, nt * 16 + r, kt * 64 + gg * 16: kt * 64 + gg * 16 + 16]
                    assert torch.equal(got, want)
    assert torch.equal(K.unpermute_fragments(wq, N, Kd), packed)


@pytest.mark.parametrize("N,Kd", [(16, 128), (32, 2048), (48, 320), (64, 160), (16, 32), (32, 544), (16, 512)])
def test_pack_scales_lane_layout(N, Kd):
    g = torch.Generator().manual_seed(N * Kd)
    _, e8 = make_experts(2, N, Kd, g, 0, 255)
    wsr = K.pack_scales(e8)
    KB = Kd // 32
    assert wsr.shape == (2, KB + 1, N)
    body = wsr.reshape(2, -1)
    for e in range(2):
        for nt in range(N // 16):
            base = nt * 16 * KB
            for kb in range(KB):
                kt, gg = kb // 4, kb % 4
                for r in range(16):
                    lane = gg * 16 + r
                    off = kt * 64 + lane
                    assert body[e, base + off] == e8[e, nt * 16 + r, kb]
        assert torch.equal(wsr[e, KB], e8[e].max(dim=1).values)
    assert torch.equal(K.unpack_scales(wsr), e8)


def test_capacity_and_pick_mt():
    assert K.capacity(512, 288, 16) == (512 + 288 * 15 + 15) // 16 * 16
    assert K.pick_mt(8, 288) == 1 and K.pick_mt(65536, 288) == 4 and K.pick_mt(288 * 20, 288) == 2


def test_prefill_cfg_table_from_library():
    for cfg, (bm, _) in K.PREFILL_TILES.items():
        assert K.prefill_block(cfg) == bm
        assert K.prefill_bk(cfg) == 32
    assert K.pick_moe_prefill(4, 512) == 17 and K.pick_moe_prefill(1, 512) is None
    with pytest.raises(ValueError):
        K.prefill_block(99)


def test_align_block_size_ref_canonical():
    ids = torch.tensor([[3, 1], [1, 0], [3, 2]])
    s, e, n = K.align_block_size_ref(ids, 4, 4)
    assert n.item() == 16 and s[:16].tolist() == [3, 6, 6, 6, 1, 2, 6, 6, 5, 6, 6, 6, 0, 4, 6, 6]
    assert e[:4].tolist() == [0, 1, 2, 3] and (e[4:] == -1).all()


def test_nvfp4_layout_places_checkpoint_bytes():
    """prepare_nvfp4_weights: lane l = g*16 + c of K-tile kt holds checkpoint bytes kt*64 + 16g .. +16 of row
    nt*16 + c, its 2 scale bytes are groups kt*8 + 2g, +1 of that row, and a partial last K-tile is zero-padded."""
    import torch
    from r9700_vllm.kernels import moe as K
    E, N, Kd = 2, 32, 272                      # K % 128 = 16: one live group in the last K-tile
    g = torch.Generator().manual_seed(0)
    p = torch.randint(0, 256, (E, N, Kd // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    s8 = torch.randint(0, 0x7f, (E, N, Kd // 16), generator=g, dtype=torch.int32).to(torch.uint8)
    W = K.prepare_nvfp4_weights(p, s8.view(torch.float8_e4m3fn), torch.ones(E, N))
    nkt = 3
    assert W.wq.dtype == torch.int32 and W.ws.shape == (E, nkt * 8, N) and W.ws_estride == N * nkt * 8
    wq = W.wq.view(torch.uint8).reshape(E, N // 16, nkt, 64, 16)               # [e, nt, kt, lane, byte]
    ws = W.ws.reshape(E, N // 16, nkt, 64, 2)                                  # [e, nt, kt, lane, group of 2]
    for e in range(E):
        for n in range(N):
            for kt in range(nkt):
                for gg in range(4):
                    lane = gg * 16 + n % 16
                    for b in range(16):
                        kb = kt * 64 + 16 * gg + b
                        want = int(p[e, n, kb]) if kb < Kd // 2 else 0
                        assert int(wq[e, n // 16, kt, lane, b]) == want, (e, n, kt, gg, b)
                    for h in range(2):
                        gi = kt * 8 + 2 * gg + h
                        want = int(s8[e, n, gi]) if gi < Kd // 16 else 0
                        assert int(ws[e, n // 16, kt, lane, h]) == want, (e, n, kt, gg, h)


@pytest.mark.parametrize("M,topk,N1,K1,N2,K2", [(1, 8, 1024, 2048, 2048, 512), (8192, 8, 1024, 2048, 2048, 512),
                                                 (32768, 8, 4096, 4096, 4096, 2048), (65536, 8, 4096, 4096, 4096, 2048),
                                                 (40000, 16, 8192, 7168, 7168, 4096), (32768, 8, 4096, 256, 256, 2048),
                                                 (3, 1, 1 << 30, 64, 64, 1 << 29), (0, 8, 1024, 2048, 2048, 512)])
def test_chunk_tokens_plan(M, topk, N1, K1, N2, K2):
    """The token chunks of a routed step cover 0..M once, in order, as evenly as possible, with every per-step buffer
    of each chunk within the 32-bit buffer range the 256-row prefill GEMM addresses (< 2 GiB), and as few chunks
    as that allows."""
    from r9700_vllm.moe.experts import BUF_LIMIT, chunk_tokens
    ch = chunk_tokens(M, topk, N1, K1, N2, K2)
    if M == 0:
        assert ch == []
        return
    assert ch[0][0] == 0 and ch[-1][1] == M and all(a[1] == b[0] for a, b in zip(ch, ch[1:]))
    sizes = [t1 - t0 for t0, t1 in ch]
    assert max(sizes) - min(sizes) <= 1 and min(sizes) >= 1
    for t0, t1 in ch:
        rows = t1 - t0
        bufs = [rows * topk * N1 * 2, rows * topk * N2 * 2, rows * K1, rows * topk * K2, rows * topk * 4]
        assert max(bufs) <= BUF_LIMIT or rows == 1
    per_token = max(topk * N1 * 2, topk * N2 * 2, K1, topk * K2, topk * 4)
    assert len(ch) == -(-M // max(1, BUF_LIMIT // per_token))
    if M * per_token <= BUF_LIMIT:
        assert ch == [(0, M)]


def test_align_block_size_ref_matches_oracle_align():
    """The host-side table builder (a vectorised stable sort) equals the oracle's align (C restatement of the
    canonical moe_align_block_size order) on random shapes, block sizes and ids outside [0, E)."""
    from oracle import oracle as O
    rng = np.random.default_rng(0)
    for _ in range(200):
        E, n, blk = int(rng.integers(1, 40)), int(rng.integers(1, 300)), int(2 ** rng.integers(0, 6))
        ids = torch.from_numpy(rng.integers(-2, E + 2, n).astype(np.int32))
        s, e, t = K.align_block_size_ref(ids, E, blk)
        rs, re_, rt = O.align(ids.numpy(), E, blk)
        N = int(t[0])
        assert N == int(rt[0])
        assert np.array_equal(s[:N].numpy(), rs[:N]) and np.array_equal(e[: N // blk].numpy(), re_[: N // blk])
        assert bool((s[N:] == n).all()) and bool((e[N // blk:] == -1).all())


def test_expected_blocks_closed_form():
    """expected_blocks is E (1 - (1 - k/E)^T): checked against a brute-force count of distinct experts over random
    top-k draws (uniform routing), and its limits (one token -> k experts; many tokens -> E)."""
    import numpy as np
    from r9700_vllm.kernels import moe as K
    assert abs(K.expected_blocks(8, 288, 8) - 8.0) < 1e-9
    assert abs(K.expected_blocks(8 * 100000, 288, 8) - 288.0) < 1e-6
    rng = np.random.default_rng(5)
    for T in (16, 64, 100):
        d = np.mean([len(np.unique(np.concatenate([rng.choice(288, 8, replace=False) for _ in range(T)])))
                     for _ in range(200)])
        assert abs(K.expected_blocks(T * 8, 288, 8) - d) < 0.03 * d, (T, d)


def test_dense_row_ranges_stay_in_the_buffer_range():
    """ops.row_ranges: ranges cover 0..M in order without gaps, each range's output (2N bytes a row) and activation
    codes (K bytes a row) within the 2 GiB limit, as few ranges as that allows, balanced to one row."""
    from r9700_vllm import ops
    for M, N, K in ((0, 17408, 5120), (1, 17408, 5120), (61680, 17408, 5120), (61681, 17408, 5120),
                    (200000, 17408, 5120), (10, 8, 1 << 30), (7, 3, 5)):
        rr = ops.row_ranges(M, N, K)
        if M == 0:
            assert rr == []
            continue
        assert rr[0][0] == 0 and rr[-1][1] == M and all(a[1] == b[0] for a, b in zip(rr, rr[1:]))
        per = max(2 * N, K)
        assert all((r1 - r0) * per <= ops.BUF_LIMIT for r0, r1 in rr)
        assert len(rr) == -(-M // (ops.BUF_LIMIT // per))
        sizes = [r1 - r0 for r0, r1 in rr]
        assert max(sizes) - min(sizes) <= 1
    assert len(ops.row_ranges(61680, 17408, 5120)) == 1 and len(ops.row_ranges(61681, 17408, 5120)) == 2


def test_split_plan():
    """Which steps split their tables by expert size, the threshold, and the router's side of the hand-off."""
    from r9700_vllm.kernels import moe as K
    from r9700_vllm.moe import route
    assert K.split_wanted(32768, 384, 4096, 2048)            # config 5 T = 4096
    assert K.split_wanted(2048, 384, 4096, 2048)             # config 5 T = 256
    assert not K.split_wanted(65536, 288, 2048, 512)         # config 3: 227 rows an expert
    assert not K.split_wanted(512, 288, 2048, 512)           # config 2 T = 64: below SPLIT_MIN_NUMEL
    assert not K.split_wanted(2048, 288, 2048, 512)          # config 2 T = 256: 1 MB experts at decode widths
    assert K.split_wanted(8192, 288, 2048, 512)              # config 2 T = 1024: past the router's table width
    assert not K.split_wanted(32768, 384, 5120, 2048)        # K past the block stream's 4096
    assert not K.split_wanted(32768, 384, 4096, 2000)        # K not a multiple of 128
    assert K.split_thr(2048) == 32 and K.split_thr(32768) == 16

    class Layer:
        _r9k_split_k = (4096, 2048)
        _r9k_dual_blk = 256

    assert route.split_planned(Layer, 2048, 384) and route.dual_wanted(Layer, 2048, 384) == 0
    assert not route.split_planned(Layer, 512, 384)
    Layer._r9k_split_k = None
    assert not route.split_planned(Layer, 2048, 384) and not route.split_planned(None, 2048, 384)


def test_tuned_table_lookup(tmp_path, monkeypatch):
    """The gfx950 launch table: nearest measured M at or below, else the smallest; legal_cfg drops shapes the decode
    kernel is not built for; pick_cfg answers (0, 0, 0) for shapes the table does not hold."""
    import json
    from r9700_vllm.kernels import moe as K, tuned
    doc = {"entries": [{"kind": "mxfp4", "N": 1024, "K": 2048, "M": 17, "cfg": [4, 2, 2]},
                       {"kind": "mxfp4", "N": 1024, "K": 2048, "M": 64, "cfg": [2, 1, 2]},
                       {"kind": "mxfp4", "N": 512, "K": 256, "M": 17, "cfg": [4, 4, 4]}]}
    path = tmp_path / "t.json"
    path.write_text(json.dumps(doc))
    monkeypatch.setenv("R9K_TUNED", str(path))
    monkeypatch.setattr(tuned, "_TABLE", None)
    assert tuned.lookup("mxfp4", 1024, 2048, 17) == (4, 2, 2)
    assert tuned.lookup("mxfp4", 1024, 2048, 63) == (4, 2, 2)
    assert tuned.lookup("mxfp4", 1024, 2048, 100) == (2, 1, 2)
    assert tuned.lookup("mxfp4", 1024, 2048, 5) == (4, 2, 2)
    assert tuned.lookup("mxfp4", 999, 2048, 17) is None
    assert K.pick_cfg(1024, 2048, M=40, kind="mxfp4") == (4, 2, 2)
    assert K.pick_cfg(1024, 2048, M=200, kind="mxfp4")[0] == "P"
    assert K.pick_cfg(999, 2048, M=40, kind="mxfp4") == (0, 0, 0)
    assert K.pick_cfg(512, 256, M=17, kind="mxfp4") == (0, 0, 0)   # SK 4 > the 2 K-tiles of K = 256
    assert K.legal_cfg((2, 2, 4), 1024, 2048, MT=4) == (0, 0, 0)   # NPW 4 is not built at MT 4
    assert K.legal_cfg((2, 2, 4), 1024, 2048, MT=2) == (2, 2, 4)
    assert K.legal_cfg((3, 1, 1), 1024, 2048) == (0, 0, 0)
    monkeypatch.setenv("R9K_TUNED", "0")
    monkeypatch.setattr(tuned, "_TABLE", None)
    assert K.pick_cfg(1024, 2048, M=40, kind="mxfp4") == (0, 0, 0)
    monkeypatch.setattr(tuned, "_TABLE", None)
