"""torch.library custom ops around libr9k's ctypes kernels, so they can sit inside a torch.compile'd graph and be
captured into HIP graphs (reference: r9700_vllm/ops.py:1-170, MXFP4 path).

  torch.ops.r9700.mxfp4_linear(x[M,K] bf16, wq, wsr, N, K, fold) -> [M,N] bf16   MXFP4 weight x per-token fp8 act
  torch.ops.r9700.nvfp4_linear(x[M,K] bf16, wq, ws, wg, N, K) -> [M,N] bf16      native NVFP4 weight (exact bits)

The reference's fp8_linear / fp8_block_linear (dense fp8 GEMMs) are not part of the gfx950 MoE build.
"""
from __future__ import annotations

import torch

from ._compat import register_custom_op

_LIB = torch.library.Library("r9700", "FRAGMENT")
_DONE = False

_MX_TABLES: dict[tuple, tuple] = {}


def _identity_tables(x, M, MT=None):
    """Routing tables for a dense GEMM: sorted ids 0..Mpad-1, every block on expert 0 (cached per shape)."""
    from .kernels import moe as KM
    if MT is None:
        MT = 4 if M >= 64 else (2 if M >= 32 else 1)
    blk = KM.MOE_BLOCK * MT
    mpad = (M + blk - 1) // blk * blk
    key = (x.device.index, mpad, blk)
    t = _MX_TABLES.get(key)
    if t is None:
        t = (torch.arange(mpad, dtype=torch.int32, device=x.device),
             torch.zeros(mpad // blk, dtype=torch.int32, device=x.device),
             torch.full((1,), mpad, dtype=torch.int32, device=x.device))
        _MX_TABLES[key] = t
    return t, MT


def mxfp4_gemm_q(q: torch.Tensor, s: torch.Tensor, W, out: torch.Tensor, M: int, cfg, topk_w=None) -> None:
    """out [M, W.N] bf16 = dequant(q * s) @ W^T (* topk_w[row]) for a dense MXFP4 weight on the kernel `cfg` names:
    the prefill entry ("P", cfg) or the decode kernel (a (WV, SK, NPW[, MT]) tuple)."""
    from .kernels import moe as KM
    if KM.is_prefill_cfg(cfg):
        t, _ = _identity_tables(q, M, KM.prefill_block(cfg[1]) // KM.MOE_BLOCK)
        KM.moe_gemm(q, s, W, out, *t, M, 1, topk_w, num_experts=1, prefill=cfg[1])
    else:
        t, MT = _identity_tables(q, M, cfg[3] if len(cfg) > 3 else None)
        KM.moe_gemm(q, s, W, out, *t, M, 1, topk_w, *cfg[:3], num_experts=1, MT=MT)


def _mxfp4_linear(x: torch.Tensor, wq: torch.Tensor, wsr: torch.Tensor, N: int, K: int, fold: bool = False
                  ) -> torch.Tensor:
    from .kernels import moe as KM
    M = x.shape[0]
    out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    if M == 0:
        return out
    W = KM.Mxfp4Experts(wq, wsr, N, K, fold)
    if M <= KM.DENSE_QA_MAX_M and KM.dense_mxfp4_qa(x, W, out):   # decode widths: the quant inside the GEMM launch
        return out
    cfg = KM.pick_cfg(N, K, M=M, kind="mxfp4", fold=fold)
    q, s = KM.quant_rows_fp8(x)
    mxfp4_gemm_q(q, s, W, out, M, cfg)
    return out


def _mxfp4_linear_fake(x: torch.Tensor, wq: torch.Tensor, wsr: torch.Tensor, N: int, K: int, fold: bool = False
                       ) -> torch.Tensor:
    return x.new_empty((x.shape[0], N))


def _nvfp4_linear(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, wg: torch.Tensor, N: int, K: int
                  ) -> torch.Tensor:
    """x [M, K] bf16 -> [M, N] bf16 over native NVFP4 weights (prepare_nvfp4_weights of one expert) with per-row fp8
    activations (reference: r9700_vllm/ops.py nvfp4_linear): the decode-family kernel below NV_PREFILL_MIN_M rows,
    the 128 x 128-tile prefill kernel (r9k_moe_4bit_prefill nv = 1) from there."""
    from .kernels import moe as KM
    M = x.shape[0]
    out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    if M == 0:
        return out
    W = KM.Nvfp4Experts(wq, ws, wg, N, K)
    q, s = KM.quant_rows_fp8(x)
    if M >= KM.NV_PREFILL_MIN_M and K % 32 == 0:
        t, _ = _identity_tables(q, M, KM.prefill_block(KM.NV_PREFILL_CFG) // KM.MOE_BLOCK)
        KM.moe_gemm(q, s, W, out, *t, M, 1, None, num_experts=1, prefill=KM.NV_PREFILL_CFG)
    else:
        t, MT = _identity_tables(q, M)
        KM.moe_gemm(q, s, W, out, *t, M, 1, None, num_experts=1, MT=MT)
    return out


def _nvfp4_linear_fake(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, wg: torch.Tensor, N: int, K: int
                       ) -> torch.Tensor:
    return x.new_empty((x.shape[0], N))


def register() -> None:
    global _DONE
    if _DONE:
        return
    register_custom_op(_LIB, "mxfp4_linear", _mxfp4_linear, [], _mxfp4_linear_fake)
    register_custom_op(_LIB, "nvfp4_linear", _nvfp4_linear, [], _nvfp4_linear_fake)
    _DONE = True


def mxfp4_linear(x: torch.Tensor, wq: torch.Tensor, wsr: torch.Tensor, N: int, K: int, fold: bool = False
                 ) -> torch.Tensor:
    register()
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    x2 = (x2 if x2.dtype == torch.bfloat16 else x2.to(torch.bfloat16)).contiguous()
    return torch.ops.r9700.mxfp4_linear(x2, wq, wsr, N, K, fold).reshape(*lead, N)


def nvfp4_linear(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, wg: torch.Tensor, N: int, K: int
                 ) -> torch.Tensor:
    register()
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    x2 = (x2 if x2.dtype == torch.bfloat16 else x2.to(torch.bfloat16)).contiguous()
    return torch.ops.r9700.nvfp4_linear(x2, wq, ws, wg, N, K).reshape(*lead, N)
