"""torch.library custom ops over libr9k's ctypes kernels, so the dense linears can sit inside a torch.compile'd
graph (Dynamo cannot trace a ctypes call) and be captured into HIP graphs. The reference's r9700_vllm/ops.py surface
for the 4-bit path:

  torch.ops.r9700.mxfp4_linear(x [M, K] bf16, wq, wsr, N, K, fold) -> [M, N] bf16   MXFP4 weight, per-token fp8 act
  torch.ops.r9700.nvfp4_linear(x [M, K] bf16, wq, ws, wg, N, K) -> [M, N] bf16      native NVFP4 weight (exact bits)

plus `mxfp4_gemm_q` (the GEMM on already-quantised rows, which the shared expert uses). A dense linear is the grouped
MoE GEMM with one expert and identity routing tables (`IdentityTables`); at decode widths the MXFP4 linear is one
launch with the activation quant inside (kernels.moe.dense_mxfp4_qa), and up to 16 rows the GEMM on quantised rows
is the dense kernel's weight stream (kernels.moe.dense_mxfp4_a8). The reference's fp8_linear / fp8_block_linear
(dense fp8 GEMMs) are outside this build.
"""
from __future__ import annotations

import torch

from ._compat import register_custom_op

_LIB = torch.library.Library("r9700", "FRAGMENT")
_registered = False


class IdentityTables:
    """Routing tables that make the grouped GEMM a dense one: rows 0..Mpad-1 in order, every block on expert 0,
    Mpad = M rounded up to the block. Built once per (device, Mpad, block) and reused (graph capture needs fixed
    addresses, and a decode step asks for the same few shapes every time)."""

    _cache: dict = {}

    @classmethod
    def get(cls, device: torch.device, M: int, block: int):
        mpad = -(-M // block) * block
        key = (device.type, device.index, mpad, block)
        t = cls._cache.get(key)
        if t is None:
            i32 = dict(dtype=torch.int32, device=device)
            t = cls._cache[key] = (torch.arange(mpad, **i32), torch.zeros(mpad // block, **i32),
                                   torch.tensor([mpad], **i32))
        return t


def _decode_mt(M: int) -> int:
    """M-tiles per routing block of a dense decode GEMM (kernels.moe.decode_mt)."""
    from .kernels import moe as KM
    return KM.decode_mt(M)


def mxfp4_gemm_q(q: torch.Tensor, s: torch.Tensor, W, out: torch.Tensor, M: int, cfg, topk_w=None) -> None:
    """out [M, W.N] bf16 = dequant(q, s) @ W^T (* topk_w[row]) for one dense MXFP4 weight, on the kernel `cfg` names:
    ("P", prefill cfg) or a decode tuple (WV, SK, NPW[, MT]) whose only meaning here is the optional MT. A decode cfg
    with at most KM.DENSE_A8_MAX_M rows runs on the dense kernel (r9k_dense_mxfp4_a8), the decode GEMM's bits."""
    from .kernels import moe as KM
    if (not KM.is_prefill_cfg(cfg) and M <= KM.DENSE_A8_MAX_M and not W.fold
            and KM.dense_mxfp4_a8(q, s, W, out, topk_w)):
        return
    if KM.is_prefill_cfg(cfg):
        tabs = IdentityTables.get(q.device, M, KM.prefill_block(cfg[1]))
        KM.moe_gemm(q, s, W, out, *tabs, M, 1, topk_w, num_experts=1, prefill=cfg[1])
        return
    MT = cfg[3] if len(cfg) > 3 else _decode_mt(M)
    tabs = IdentityTables.get(q.device, M, KM.MOE_BLOCK * MT)
    KM.moe_gemm(q, s, W, out, *tabs, M, 1, topk_w, *cfg[:3], num_experts=1, MT=MT)


# The prefill GEMMs address their activation rows and their output through 32-bit buffer ranges, so one launch may
# touch at most this many bytes of either; a longer dense linear runs as row ranges (row_ranges), each a launch of its
# own over its own identity tables.
BUF_LIMIT = (1 << 31) - 1


def row_ranges(M: int, N: int, K: int, limit: int = BUF_LIMIT) -> list:
    """[(r0, r1), ...] covering rows 0..M, as few and as even as possible, each range's output [r1 - r0, N] bf16 and
    fp8 activation codes [r1 - r0, K] within `limit` bytes."""
    per_row = max(2 * N, K, 1)
    n = -(-M // max(1, limit // per_row)) if M else 0
    bounds = [M * i // n for i in range(n + 1)] if n else [0]
    return list(zip(bounds[:-1], bounds[1:]))


def _mxfp4_linear_rows(x: torch.Tensor, W, out: torch.Tensor, fold: bool) -> None:
    from .kernels import moe as KM
    M = x.shape[0]
    if M <= KM.DENSE_QA_MAX_M and not fold and KM.dense_mxfp4_qa(x, W, out):   # decode widths: quant in the launch
        return
    q, s = KM.quant_rows_fp8(x)
    mxfp4_gemm_q(q, s, W, out, M, KM.pick_cfg(W.N, W.K, M=M, kind="mxfp4", fold=fold))


def _mxfp4_linear(x: torch.Tensor, wq: torch.Tensor, wsr: torch.Tensor, N: int, K: int, fold: bool = False
                  ) -> torch.Tensor:
    from .kernels import moe as KM
    M = x.shape[0]
    out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    W = KM.Mxfp4Experts(wq, wsr, N, K, fold)
    for r0, r1 in row_ranges(M, N, K):
        _mxfp4_linear_rows(x[r0:r1], W, out[r0:r1], fold)
    return out


def _nvfp4_linear_rows(x: torch.Tensor, W, out: torch.Tensor) -> None:
    from .kernels import moe as KM
    M = x.shape[0]
    if M <= KM.DENSE_NV_QA_MAX_M and KM.dense_nvfp4_qa(x, W, out):   # decode widths: the quant inside the GEMM launch
        return
    q, s = KM.quant_rows_fp8(x)
    if M >= KM.NV_PREFILL_MIN_M and W.K % 32 == 0:
        tabs = IdentityTables.get(x.device, M, KM.prefill_block(KM.NV_PREFILL_CFG))
        KM.moe_gemm(q, s, W, out, *tabs, M, 1, None, num_experts=1, prefill=KM.NV_PREFILL_CFG)
    else:
        MT = _decode_mt(M)
        tabs = IdentityTables.get(x.device, M, KM.MOE_BLOCK * MT)
        KM.moe_gemm(q, s, W, out, *tabs, M, 1, None, num_experts=1, MT=MT)


def _nvfp4_linear(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, wg: torch.Tensor, N: int, K: int
                  ) -> torch.Tensor:
    """Native NVFP4 weights (prepare_nvfp4_weights of one expert) with per-row fp8 activations: one launch with the
    quant inside up to DENSE_NV_QA_MAX_M rows, the decode-family kernel below NV_PREFILL_MIN_M rows, the 128 x 128-tile
    prefill kernel (r9k_moe_4bit_prefill nv = 1) from there; row ranges past the 2 GiB buffer range (row_ranges)."""
    from .kernels import moe as KM
    M = x.shape[0]
    out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    W = KM.Nvfp4Experts(wq, ws, wg, N, K)
    for r0, r1 in row_ranges(M, N, K):
        _nvfp4_linear_rows(x[r0:r1], W, out[r0:r1])
    return out


def _rows_out_fake(x: torch.Tensor, N: int) -> torch.Tensor:
    return torch.empty((x.shape[0], N), dtype=torch.bfloat16, device=x.device)


def _mxfp4_linear_fake(x: torch.Tensor, wq: torch.Tensor, wsr: torch.Tensor, N: int, K: int, fold: bool = False
                       ) -> torch.Tensor:
    return _rows_out_fake(x, N)


def _nvfp4_linear_fake(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, wg: torch.Tensor, N: int, K: int
                       ) -> torch.Tensor:
    return _rows_out_fake(x, N)


_OPS = (("mxfp4_linear", _mxfp4_linear, _mxfp4_linear_fake), ("nvfp4_linear", _nvfp4_linear, _nvfp4_linear_fake))


def register() -> None:
    global _registered
    if not _registered:
        for name, fn, fake in _OPS:
            register_custom_op(_LIB, name, fn, [], fake)
        _registered = True


def _call_on_rows(op, x: torch.Tensor, K: int, N: int) -> torch.Tensor:
    """op over x viewed as contiguous bf16 rows [-1, K], the result shaped back to x's leading dims + [N]."""
    register()
    rows = x.reshape(-1, K)
    if rows.dtype != torch.bfloat16:
        rows = rows.to(torch.bfloat16)
    return op(rows.contiguous()).reshape(*x.shape[:-1], N)


def mxfp4_linear(x: torch.Tensor, wq: torch.Tensor, wsr: torch.Tensor, N: int, K: int, fold: bool = False
                 ) -> torch.Tensor:
    return _call_on_rows(lambda r: torch.ops.r9700.mxfp4_linear(r, wq, wsr, N, K, fold), x, K, N)


def nvfp4_linear(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, wg: torch.Tensor, N: int, K: int
                 ) -> torch.Tensor:
    return _call_on_rows(lambda r: torch.ops.r9700.nvfp4_linear(r, wq, ws, wg, N, K), x, K, N)
