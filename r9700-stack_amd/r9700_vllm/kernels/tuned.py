"""Tuned launch configs (a JSON table next to this file): {kind: {"N,K": {"M": [..cfg..]}}}.

A call uses the smallest tuned M bucket >= its M; larger M and untuned shapes keep the defaults. The gfx950 build
ships no table (the kernels size their own split from the shape), so lookup() returns None unless R9K_TUNED points
at one. Same contract as the reference's r9700_vllm/kernels/tuned.py:11-24.
"""
from __future__ import annotations

import json
import os

_T: dict | None = None


def lookup(kind: str, N: int, K: int, M: int):
    global _T
    if _T is None:
        p = os.environ.get("R9K_TUNED") or os.path.join(os.path.dirname(__file__), "tuned.json")
        try:
            with open(p) as f:
                _T = json.load(f)
        except (OSError, ValueError):
            _T = {}
    entry = _T.get(kind, {}).get(f"{N},{K}")
    if not entry:
        return None
    buckets = sorted(int(m) for m in entry)
    b = next((m for m in buckets if m >= M), None)
    return tuple(entry[str(b)]) if b is not None else None
