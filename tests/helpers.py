"""Shared generators and comparisons for the tests (seeded, CPU generators like the reference's
tests/test_moe_mxfp4.py:16-26 and tests/test_nvfp4.py:18-27)."""
from __future__ import annotations

import numpy as np
import torch


def make_experts(E: int, N: int, K: int, g: torch.Generator, lo: int = 118, hi: int = 126):
    """MXFP4 experts in checkpoint layout: uniform-random e2m1 codes packed 2/byte (low nibble = even element) and
    e8m0 exponents uniform in [lo, hi]. Returns (packed [E, N, K/2] u8, e8m0 [E, N, K/32] u8)."""
    packed = torch.randint(0, 256, (E, N, K // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    e8m0 = torch.randint(lo, hi + 1, (E, N, K // 32), generator=g, dtype=torch.int32).to(torch.uint8)
    return packed, e8m0


def rel_err(got, ref) -> float:
    got = torch.as_tensor(got).double()
    ref = torch.as_tensor(ref).double()
    return float((got - ref).norm() / ref.norm().clamp_min(1e-30))


def cosine(got, ref) -> float:
    a = torch.as_tensor(got).double().reshape(-1)
    b = torch.as_tensor(ref).double().reshape(-1)
    return float((a @ b) / (a.norm() * b.norm()).clamp_min(1e-30))


def bf16_bits_to_f64(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy((np.asarray(b).astype(np.uint32) << 16).view(np.float32).astype(np.float64))


def check_tables(sorted_ids, expert_ids, ntpp, ids, blk: int, numel: int, E: int):
    """The reference's table invariants (tests/test_moe_route_r9k.py:24-41): every routed row exactly once, each
    block's rows on its expert, experts ascending, padding = numel, ntpp = sum of block-padded counts."""
    n = int(np.asarray(ntpp).reshape(-1)[0])
    assert n % blk == 0, f"ntpp {n} not a multiple of {blk}"
    s = np.asarray(sorted_ids)[:n].tolist()
    e = np.asarray(expert_ids)[: n // blk].tolist()
    flat = np.asarray(ids).reshape(-1).tolist()
    seen = sorted(x for x in s if x != numel)
    assert seen == list(range(numel)), "not every routed row appears exactly once"
    last = -1
    for b in range(n // blk):
        assert e[b] >= last, "experts not ascending"
        last = e[b]
        for x in s[b * blk:(b + 1) * blk]:
            if x != numel:
                assert flat[x] == e[b], f"row {x} (expert {flat[x]}) in a block of expert {e[b]}"
    cnt = np.bincount(np.asarray(flat, dtype=np.int64), minlength=E)
    assert n == int(sum((c + blk - 1) // blk * blk for c in cnt)), "ntpp != sum of padded counts"


def block_edge_tokens(ids, E: int, blk: int, topk: int) -> np.ndarray:
    """Sorted tokens that hold the first or the last live routed row of some blk-row block of the canonical align
    tables over ids [T, topk] (every block of every expert, the hot expert's included): a check on these tokens
    reads every block's edges."""
    from oracle import oracle as O
    flat = np.asarray(ids).reshape(-1)
    numel = flat.size
    s, _, n = O.align(flat, E, blk)
    s = s[: int(n[0])].reshape(-1, blk)
    live = s < numel
    nl = live.sum(1)
    keep = nl > 0
    first = s[keep, 0]                                      # live rows lead each block, padding follows
    last = s[keep, nl[keep] - 1]
    assert (live[keep, 0]).all() and (s[keep][np.arange(keep.sum()), nl[keep] - 1] < numel).all()
    return np.unique(np.concatenate([first, last]) // topk)
