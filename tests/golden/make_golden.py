"""Writes the committed golden fixtures of the MoE hot path (tests/golden/*.npz).

    python tests/golden/make_golden.py          # rewrites every fixture from its seeded inputs

The reference (bkvargyas/r9700-stack v0.4.3) commits no golden vectors: its tests draw seeded inputs at run time and
compare against torch (tests/test_moe_mxfp4.py:16-72, tests/test_nvfp4.py:18-59, tests/test_moe_route_r9k.py:24-113).
These fixtures freeze small seeded cases of the bit-exact (integer / byte) outputs, produced by the CPU oracle
(oracle/, itself pinned against torch library routines, closed forms and brute force by tests/test_oracle_*.py),
so that the GPU tests check the HIP path against stored bytes and the CPU tests catch any drift of the oracle.
Each case stores its inputs and expected outputs as plain arrays (np.savez, no pickles).

Cases (edge inputs chosen the way the reference's tests choose them):
  quant_rows.npz   per-token fp8 e4m3 quant (a zero row, an overflow-edge row, subnormal-range rows)
  route.npz        softmax top-8 over 288 experts with renorm (ties, NaN / +-inf / all-equal rows), and the
                   align tables of those ids at blk 16 and 64
  align.npz        tables at blk 16 / 256 for a Zipf-skewed id set with ids outside [0, E) (skipped)
  moe_sum.npz      top-k sum (fp32 over j, one bf16 rounding) incl. cancellation and bf16 tie cases
  nvfp4.npz        NVFP4 -> MXFP4 conversion (uniform codes, s16 = e4m3(|N(0,1)| * 0.05), per-row divisors)
  mx_search.npz    MSE-searched MXFP4 of fp32 weights (zero blocks, +-0, wide dynamic range)
  gemm.npz         grouped MXFP4 x fp8 GEMM, gate_up (a_row_div = topk) and down (router weight) bf16 outputs:
                   float outputs, compared to tolerance (they are the oracle's fp64-accumulated values)
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402  (test infrastructure: the checker that writes the fixtures)

SEED = 20261201


def bf16(x: torch.Tensor) -> np.ndarray:
    return O.bf16_bits(x.to(torch.bfloat16))


def quant_rows_case():
    g = torch.Generator().manual_seed(SEED + 1)
    x = torch.randn(8, 320, generator=g)
    x[1] = 0.0                                            # all-zero row: amax clamps to 1e-12
    x[2] *= 1e-6                                          # small magnitudes
    x[3, :] = 448.0                                       # the e4m3 maximum exactly
    x[3, 7] = -448.0
    x[4] *= 1e4                                           # large magnitudes
    x[5, ::3] = 0.0
    x[6] = torch.linspace(-3, 3, 320)                     # dense grid across the rounding points
    xb = x.to(torch.bfloat16)
    q, s = O.quant_rows_fp8(xb)
    return dict(x=bf16(xb), q=q, s=s)


def route_case():
    g = torch.Generator().manual_seed(SEED + 2)
    M, E, k = 24, 288, 8
    lg = torch.randn(M, E, generator=g)
    lg[1, [3, 77, 200, 201]] = 6.0                         # four-way tie at the top
    lg[2] = 0.25                                          # all equal
    lg[3, 17] = float("nan")                              # NaN entry
    lg[4, 5] = float("inf")                               # +inf entry: the row's other entries die
    lg[5, :] = -float("inf")                              # all -inf: every entry dead, ids by index
    lg[6, 100:] = -1e4                                    # far below the max: dead
    lg[7] = lg[7] * 8.0                                   # sharp distribution
    lb = lg.to(torch.bfloat16)
    w, ids = O.route(lb, k, True)
    w0, ids0 = O.route(lb, k, False)
    out = dict(logits=bf16(lb), topk=np.int32(k), w=w, ids=ids, w_norenorm=w0, ids_norenorm=ids0)
    for blk in (16, 64):
        s, e, n = O.align(ids.reshape(-1), E, blk)
        out[f"sorted_ids_{blk}"], out[f"expert_ids_{blk}"], out[f"ntpp_{blk}"] = s, e, n
    return out


def align_case():
    rng = np.random.default_rng(SEED + 3)
    E, numel = 64, 3000
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    ids = rng.choice(E, numel, p=p / p.sum()).astype(np.int32)
    ids[::97] = -1                                        # rows of experts on another rank (expert_map -> -1)
    ids[5::131] = E + 3                                   # out of range: skipped
    out = dict(ids=ids, E=np.int32(E))
    for blk in (16, 256):
        s, e, n = O.align(ids, E, blk)
        out[f"sorted_ids_{blk}"], out[f"expert_ids_{blk}"], out[f"ntpp_{blk}"] = s, e, n
    return out


def moe_sum_case():
    g = torch.Generator().manual_seed(SEED + 4)
    M, k, N = 6, 8, 160
    d = torch.randn(M, k, N, generator=g)
    d[1, :4] = 1.0
    d[1, 4:] = -1.0                                       # exact cancellation to 0
    d[2, 0] = 1.0
    d[2, 1:] = 2.0 ** -9                                  # ties at the bf16 rounding point
    d[3] *= 1e30
    db = d.to(torch.bfloat16)
    return dict(down=bf16(db), out=O.moe_sum(db))


def nvfp4_case():
    g = torch.Generator().manual_seed(SEED + 5)
    N, K = 48, 512
    p16 = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.int32).to(torch.uint8).numpy()
    s16 = (torch.randn(N, K // 16, generator=g).abs() * 0.05).to(torch.float8_e4m3fn)
    s16[0, :4] = 0.0                                      # zero scales: all-zero blocks -> exponent byte 1
    s16b = s16.view(torch.uint8).numpy()
    div = np.ones(N, dtype=np.float32)
    div[N // 2:] = 3000.0                                 # a second shard's global divisor
    po, eo = O.nvfp4_to_mxfp4(p16, s16b, div)
    return dict(packed=p16, s16=s16b, row_div=div, out_packed=po, out_e8m0=eo)


def mx_search_case():
    g = torch.Generator().manual_seed(SEED + 6)
    N, K = 16, 256
    w = torch.randn(N, K, generator=g) * torch.exp(2 * torch.randn(N, 1, generator=g))
    w[0, :32] = 0.0                                       # zero block
    w[0, 32:64] = -0.0                                    # negative zeros encode as +0
    w[1, :32] = 6.0 * 2.0 ** -3                           # amax exactly on 6 * 2^e
    w[2, 5] = 1e-30                                       # tiny value next to normal ones
    w = w.numpy().astype(np.float32)
    po, eo = O.quantize_mxfp4_search(w)
    return dict(w=w, out_packed=po, out_e8m0=eo)


def gemm_case():
    g = torch.Generator().manual_seed(SEED + 7)
    E, M, k, N, Kd = 3, 5, 2, 32, 288
    packed = torch.randint(0, 256, (E, N, Kd // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    e8 = torch.randint(118, 127, (E, N, Kd // 32), generator=g, dtype=torch.int32).to(torch.uint8)
    x = (torch.randn(M, Kd, generator=g) * 0.5).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(M)]).to(torch.int32)
    tw = torch.rand(M * k, generator=g).float()
    xq, xs = O.quant_rows_fp8(x)
    Wd = {e: O.mxfp4_dequant(packed[e], e8[e]) for e in range(E)}
    flat = ids.reshape(-1).numpy()
    gate_up = O.grouped_gemm(xq, xs, Wd, flat, k)
    # down-style call: one A row per routed row (a_row_div = 1) and the router weight in the epilogue
    xr = (torch.randn(M * k, Kd, generator=g) * 0.5).to(torch.bfloat16)
    rq, rs = O.quant_rows_fp8(xr)
    down = O.grouped_gemm(rq, rs, Wd, flat, 1, tw.numpy())
    return dict(packed=packed.numpy(), e8m0=e8.numpy(), x=bf16(x), ids=ids.numpy(), topk_w=tw.numpy(),
                x_rows=bf16(xr), gate_up=gate_up, down=down)


CASES = {"quant_rows": quant_rows_case, "route": route_case, "align": align_case, "moe_sum": moe_sum_case,
         "nvfp4": nvfp4_case, "mx_search": mx_search_case, "gemm": gemm_case}


def load(name: str) -> dict:
    with np.load(os.path.join(HERE, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def main() -> None:
    for name, fn in CASES.items():
        arrs = fn()
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrs)
        print(f"{path}: {os.path.getsize(path)} bytes", flush=True)


if __name__ == "__main__":
    main()
