"""Pins the oracle's routing and align tables (CPU only).

ids: torch.softmax(fp32) + a stable descending sort (the reference test's oracle, tests/test_moe_mxfp4.py:44-45,
with ties to the lower index as kernels/r9k_moe_route.hip:57-65 breaks them); weights within 2e-6
(tests/test_moe_route_r9k.py:78); degenerate rows by the reference kernel's rules (:81-95); tables against an
independent numpy restatement of align_block_size_ref (r9700_vllm/kernels/moe.py:574-592) and the reference test's
invariants (tests/test_moe_route_r9k.py:24-41)."""
import numpy as np
import pytest
import torch

from helpers import check_tables
from oracle import oracle as O


def torch_route(logits: torch.Tensor, topk: int, renorm: bool):
    p = torch.softmax(logits.float(), dim=-1)
    srt, idx = torch.sort(-p, dim=-1, stable=True)
    ids = idx[:, :topk]
    w = p.gather(1, ids)
    if renorm:
        w = w / w.sum(-1, keepdim=True)
    return w.numpy(), ids.numpy().astype(np.int32), p


@pytest.mark.parametrize("M,E,topk,scale", [(64, 288, 8, 1.0), (33, 384, 8, 1.0), (16, 512, 10, 4.0),
                                            (8, 48, 6, 2.0), (5, 100, 16, 1.0), (200, 128, 1, 1.0)])
@pytest.mark.parametrize("renorm", [True, False])
def test_route_matches_torch(M, E, topk, scale, renorm):
    g = torch.Generator().manual_seed(M * 1000 + E)
    logits = (torch.randn(M, E, generator=g) * scale).to(torch.bfloat16)
    w, ids = O.route(logits, topk, renorm)
    wr, idr, p = torch_route(logits, topk, renorm)
    # the orders agree unless two DISTINCT logits round to the same fp32 probability (torch then ties by index):
    # assert such collapses do not occur in this data, then require exact ids
    x = logits.float()
    for r in range(M):
        sel = idr[r]
        for a, b in zip(sel[:-1], sel[1:]):
            assert not (p[r, a] == p[r, b] and x[r, a] != x[r, b]), "fp32 collapse in the test data"
    assert np.array_equal(ids, idr)
    assert np.abs(w - wr).max() < 2e-6


def test_route_ties_go_to_lower_index():
    logits = torch.zeros(3, 64)
    logits[0, [5, 9, 40]] = 1.0          # three-way tie at the top
    logits[1] = 0.5                      # all equal
    logits[2, [63, 1]] = 2.0
    logits = logits.to(torch.bfloat16)
    w, ids = O.route(logits, 4, True)
    assert ids[0].tolist() == [5, 9, 40, 0]
    assert ids[1].tolist() == [0, 1, 2, 3] and np.allclose(w[1], 0.25)
    assert ids[2].tolist() == [1, 63, 0, 2]


def test_route_degenerate_rows():
    """NaN, +-inf, all-equal and huge-negative rows (tests/test_moe_route_r9k.py:84-104): ids valid and distinct,
    weights finite; dead entries (probability not a finite positive number) rank by index with weight 0."""
    E, k = 100, 10
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(8, E, generator=g) * 2)
    x[0] = float("nan")
    x[1, :5] = float("nan")
    x[2] = float("inf")
    x[3] = float("-inf")
    x[4] = 0.0
    x[5, ::2] = float("inf")
    x[6] = -3e38
    x[7, 3] = 200.0                       # every other entry is > 87 below the max: dead
    x = x.to(torch.bfloat16)
    w, ids = O.route(x, k, True)
    assert ids.min() >= 0 and ids.max() < E
    assert all(len(set(r.tolist())) == k for r in ids)
    assert np.isfinite(w).all()
    assert ids[0].tolist() == list(range(k)) and np.all(w[0] == 0)          # all NaN: all dead
    assert ids[2].tolist() == list(range(k)) and np.all(w[2] == 0)          # +inf row: x - max is NaN everywhere
    assert ids[3].tolist() == list(range(k)) and np.all(w[3] == 0)          # -inf row
    assert ids[4].tolist() == list(range(k)) and np.allclose(w[4], 1.0 / k)
    assert not set(ids[1].tolist()) & set(range(5))                         # NaN entries never beat live ones
    assert ids[7, 0] == 3 and w[7, 0] == 1.0 and np.all(w[7, 1:] == 0)
    assert ids[7, 1:].tolist() == [e for e in range(E) if e != 3][: k - 1]


def numpy_align(ids: np.ndarray, E: int, blk: int):
    flat = ids.reshape(-1).astype(np.int64)
    numel = flat.size
    cap = (numel + E * (blk - 1) + blk - 1) // blk * blk
    order = np.argsort(flat, kind="stable")            # experts ascending, rows ascending within an expert
    counts = np.bincount(flat, minlength=E)
    s = np.full(cap, numel, dtype=np.int32)
    e = np.full(cap // blk, -1, dtype=np.int32)
    pos, i = 0, 0
    for ex in range(E):
        c = counts[ex]
        if c == 0:
            continue
        s[pos:pos + c] = order[i:i + c]
        n = -(-c // blk) * blk
        e[pos // blk:(pos + n) // blk] = ex
        pos += n
        i += c
    return s, e, np.array([pos], dtype=np.int32)


@pytest.mark.parametrize("T,E,topk,blk", [(1, 288, 8, 16), (64, 288, 8, 16), (300, 288, 8, 64), (37, 512, 10, 32),
                                          (1000, 384, 8, 64), (5, 7, 3, 256)])
def test_align_matches_restatement(T, E, topk, blk):
    g = torch.Generator().manual_seed(T + E)
    ids = torch.stack([torch.randperm(E, generator=g)[:topk] for _ in range(T)]).numpy().astype(np.int32)
    s, e, n = O.align(ids, E, blk)
    s2, e2, n2 = numpy_align(ids, E, blk)
    assert np.array_equal(s, s2) and np.array_equal(e, e2) and np.array_equal(n, n2)
    check_tables(s, e, n, ids, blk, T * topk, E)
    assert s.size == O.capacity(T * topk, E, blk)
