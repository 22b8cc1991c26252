"""The MoE block's gated shared expert in four launches (reference: r9700_vllm/moe/shared.py:1-113).

    quant_rows_fp8_gate (row quant + the expert-gate dot + sigmoid)  ->  gate_up GEMM  ->  silu_mul_quant_fp8  ->
    down GEMM with sigmoid(gate) folded into its per-row epilogue (the routed layer's router-weight fold)

on the same libr9k kernels as the dense MXFP4 linear (identity routing tables, E = 1). Numerics as the reference's:
the gate is bf16(sigmoid(bf16(x . wg))) (stock's F.sigmoid(expert_gate(x)) values) and the down output is rounded
once, bf16(acc * (s * g)). `install(model)` binds the fused forward on the gated shared-expert MLPs of a vLLM model
(the reference's model classes call it; R9K_SHARED_EXPERT=stock keeps the stock forward).
"""
from __future__ import annotations

import os
import types

import torch

from .._compat import get_logger, register_custom_op
from ..kernels import moe as KM
from ..ops import _LIB, mxfp4_gemm_q

_DONE = False


def available() -> bool:
    try:
        return hasattr(KM.lib(), "r9k_quant_rows_fp8_gate")
    except OSError:
        return False


def shared_expert(x: torch.Tensor, wq1: torch.Tensor, wsr1: torch.Tensor, wq2: torch.Tensor, wsr2: torch.Tensor,
                  wg: torch.Tensor, N1: int, K1: int, N2: int, K2: int, fold1: bool, fold2: bool) -> torch.Tensor:
    """x [M, K1] bf16 -> [M, N2] bf16 = down(silu(gate) * up) * sigmoid(x . wg), one rounding at the end; wq / wsr as
    the dense MXFP4 linear stores them (prepare_mxfp4_weights of one expert), wg [K1] bf16 (reference: :36-58)."""
    M = x.shape[0]
    out = torch.empty((M, N2), dtype=torch.bfloat16, device=x.device)
    if M == 0:
        return out
    cfg1 = KM.pick_cfg(N1, K1, M=M, kind="mxfp4", fold=fold1)
    cfg2 = KM.pick_cfg(N2, K2, M=M, kind="mxfp4", fold=fold2)
    W1 = KM.Mxfp4Experts(wq1, wsr1, N1, K1, fold1)
    W2 = KM.Mxfp4Experts(wq2, wsr2, N2, K2, fold2)
    q, s, g = KM.quant_rows_fp8_gate(x, wg)
    gate_up = torch.empty((M, N1), dtype=torch.bfloat16, device=x.device)
    mxfp4_gemm_q(q, s, W1, gate_up, M, cfg1)
    aq, as_ = KM.silu_mul_quant_fp8(gate_up)
    mxfp4_gemm_q(aq, as_, W2, out, M, cfg2, topk_w=g)
    return out


def _shared_expert_fake(x: torch.Tensor, wq1: torch.Tensor, wsr1: torch.Tensor, wq2: torch.Tensor,
                        wsr2: torch.Tensor, wg: torch.Tensor, N1: int, K1: int, N2: int, K2: int, fold1: bool,
                        fold2: bool) -> torch.Tensor:
    return x.new_empty((x.shape[0], N2))


def register() -> None:
    """torch.ops.r9700.shared_expert (graph-capturable: host-known shapes, no synchronisation)."""
    global _DONE
    if _DONE:
        return
    register_custom_op(_LIB, "shared_expert", shared_expert, [], _shared_expert_fake)
    _DONE = True


def _forward(self, x: torch.Tensor) -> torch.Tensor:
    gu, dn = self.gate_up_proj, self.down_proj
    if getattr(gu, "_r9k_nk", None) is None or getattr(dn, "_r9k_nk", None) is None or x.dim() != 2 \
            or x.dtype != torch.bfloat16:
        return self._r9k_stock_forward(x)           # not on the MXFP4 kernels (weights not prepared / other format)
    return torch.ops.r9700.shared_expert(x.contiguous(), gu.weight, gu.weight_scale, dn.weight, dn.weight_scale,
                                         self.expert_gate.weight.view(-1), *gu._r9k_nk, *dn._r9k_nk,
                                         bool(getattr(gu, "_r9k_fold", False)), bool(getattr(dn, "_r9k_fold", False)))


def install(model: torch.nn.Module) -> int:
    """Bind the fused forward on every gated shared-expert MLP under `model` whose expert gate is a plain bf16 linear
    without bias (reference: :87-113); the projections are checked at call time, after weight preparation, and fall
    back to the stock forward otherwise. Returns the number of modules bound."""
    if os.environ.get("R9K_SHARED_EXPERT", "r9k") != "r9k" or not available():
        return 0
    register()
    log = get_logger(__name__)
    n = 0
    for name, mod in model.named_modules():
        if type(mod).__name__ not in ("Qwen3NextMLP", "Qwen2MoeMLP") or getattr(mod, "_r9k_shared", False):
            continue
        eg = getattr(mod, "expert_gate", None)
        w = getattr(eg, "weight", None) if eg is not None else None
        if not (isinstance(w, torch.Tensor) and w.dtype == torch.bfloat16 and w.dim() == 2 and w.shape[0] == 1
                and getattr(eg, "bias", None) is None
                and type(getattr(eg, "quant_method", None)).__name__ == "UnquantizedLinearMethod"
                and hasattr(mod, "gate_up_proj") and hasattr(mod, "down_proj")):
            if eg is not None:
                log.warning("r9700: fused shared expert skipped for %s", name)
            continue
        mod._r9k_stock_forward = mod.forward
        mod.forward = types.MethodType(_forward, mod)
        mod._r9k_shared = True
        n += 1
    if n:
        log.info("r9700: fused shared expert (quant+gate, gate_up, silu_mul_quant, down*gate) on %d modules", n)
    return n
