"""The decode GEMM's launch table for gfx950: (kind, N, K, M) -> (WV, SK, NPW), the launch shape of
r9k_moe_mxfp4a8 that measured fastest on MI355X for a dense [M, K] x [N, K]^T product over identity routing tables
(WV = K-tiles per load batch, SK = waves splitting K, NPW = 16-column tiles per wave). The role of the reference's
r9700_vllm/kernels/tuned.py + tuned.json (a per-shape table of its gfx1201 knobs), rebuilt for this device by
kernels/tune.py:

    python -m r9700_vllm.kernels.tune --out r9700_vllm/kernels/tuned.json

lookup() answers with the entry of the same kind, N and K at the largest measured M <= M (else the smallest), or None
when the table holds no such shape; R9K_TUNED=0 ignores the table, R9K_TUNED=<path> reads another one.
"""
from __future__ import annotations

import json
import os

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tuned.json")
_TABLE: dict | None = None


def table() -> dict:
    """The table file as loaded (keys: device, source, entries), {} when it is absent or switched off."""
    global _TABLE
    if _TABLE is None:
        src = os.environ.get("R9K_TUNED", "")
        if src == "0":
            _TABLE = {}
        else:
            try:
                with open(src or PATH) as f:
                    _TABLE = json.load(f)
            except OSError:
                _TABLE = {}
    return _TABLE


def lookup(kind: str, N: int, K: int, M: int):
    """(WV, SK, NPW) for this product, or None."""
    rows = sorted((e for e in table().get("entries", ()) if e["kind"] == kind and e["N"] == N and e["K"] == K),
                  key=lambda e: e["M"])
    if not rows:
        return None
    best = rows[0]
    for e in rows:
        if e["M"] <= M:
            best = e
    return tuple(best["cfg"])
