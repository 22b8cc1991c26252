"""The MoE block's gated shared expert on libr9k's MXFP4 kernels (the role of the reference's
r9700_vllm/moe/shared.py: the `torch.ops.r9700.shared_expert` op and the `install` hook).

A gated shared expert computes  y = down(silu(gate) * up)(x) * sigmoid(x . wg)  beside every routed MoE layer. Here
it is four launches on the dense (single-expert) path of the routed kernels:

    r9k_quant_rows_fp8_gate   x -> fp8 rows + scales, and g = bf16(sigmoid(bf16(x . wg))) in the same pass
    gate_up GEMM              (identity routing tables, E = 1)
    r9k_silu_mul_quant_fp8    silu(gate) * up -> fp8 rows + scales
    down GEMM                 with g as the per-row factor of its epilogue: bf16(acc * (s * g)), one rounding

`SharedExpertWeights` holds one module's prepared projections; `run` is the chain; `shared_expert` is the op's
function (the reference's argument list, so model code binds it unchanged). `install(model)` binds the fused forward
on every gated shared-expert MLP whose expert gate is a plain bf16 linear; a bound module whose projections are not
on the MXFP4 kernels (not prepared, another format) keeps its stock forward. R9K_SHARED_EXPERT=stock skips binding.
"""
from __future__ import annotations

import os
import types
from dataclasses import dataclass

import torch

from .._compat import get_logger, register_custom_op
from ..kernels import moe as KM
from ..ops import _LIB, mxfp4_gemm_q

# the module classes whose gated shared expert the reference's model code hands to install (matched by name: vLLM's
# classes are not importable without vLLM)
SHARED_MLP_CLASSES = ("Qwen3NextMLP", "Qwen2MoeMLP")

_registered = False


def available() -> bool:
    """libr9k loads and exports the fused quant + gate kernel."""
    try:
        return hasattr(KM.lib(), "r9k_quant_rows_fp8_gate")
    except OSError:
        return False


@dataclass
class SharedExpertWeights:
    """One shared expert's projections in the kernels' layout (prepare_mxfp4_weights of a single expert each) and its
    expert-gate row wg [K1] bf16."""
    gate_up: KM.Mxfp4Experts
    down: KM.Mxfp4Experts
    wg: torch.Tensor

    @classmethod
    def from_module(cls, mlp) -> "SharedExpertWeights | None":
        """The prepared weights of a gated MLP (its projections carry `_r9k_nk` once the dense MXFP4 prep has run),
        or None when either projection is not on the MXFP4 kernels."""
        gu, dn = mlp.gate_up_proj, mlp.down_proj
        nk1, nk2 = getattr(gu, "_r9k_nk", None), getattr(dn, "_r9k_nk", None)
        if nk1 is None or nk2 is None:
            return None
        fold1, fold2 = bool(getattr(gu, "_r9k_fold", False)), bool(getattr(dn, "_r9k_fold", False))
        return cls(KM.Mxfp4Experts(gu.weight, gu.weight_scale, *nk1, fold1),
                   KM.Mxfp4Experts(dn.weight, dn.weight_scale, *nk2, fold2),
                   mlp.expert_gate.weight.view(-1))

    def run(self, x: torch.Tensor) -> torch.Tensor:
        """x [M, K1] bf16 contiguous -> [M, N2] bf16."""
        M = x.shape[0]
        W1, W2 = self.gate_up, self.down
        y = torch.empty((M, W2.N), dtype=torch.bfloat16, device=x.device)
        if M == 0:
            return y
        q, s, gate = KM.quant_rows_fp8_gate(x, self.wg)
        h = torch.empty((M, W1.N), dtype=torch.bfloat16, device=x.device)
        mxfp4_gemm_q(q, s, W1, h, M, KM.pick_cfg(W1.N, W1.K, M=M, kind="mxfp4", fold=W1.fold))
        hq, hs = KM.silu_mul_quant_fp8(h)
        mxfp4_gemm_q(hq, hs, W2, y, M, KM.pick_cfg(W2.N, W2.K, M=M, kind="mxfp4", fold=W2.fold), topk_w=gate)
        return y


def shared_expert(x: torch.Tensor, wq1: torch.Tensor, wsr1: torch.Tensor, wq2: torch.Tensor, wsr2: torch.Tensor,
                  wg: torch.Tensor, N1: int, K1: int, N2: int, K2: int, fold1: bool, fold2: bool) -> torch.Tensor:
    """x [M, K1] bf16 -> [M, N2] bf16 = down(silu(gate) * up) * sigmoid(x . wg), rounded once; wq / wsr as the dense
    MXFP4 linear stores them, wg [K1] bf16 (the reference's op signature, moe/shared.py:36-58 there)."""
    sw = SharedExpertWeights(KM.Mxfp4Experts(wq1, wsr1, N1, K1, fold1), KM.Mxfp4Experts(wq2, wsr2, N2, K2, fold2), wg)
    return sw.run(x)


def _shared_expert_fake(x: torch.Tensor, wq1: torch.Tensor, wsr1: torch.Tensor, wq2: torch.Tensor,
                        wsr2: torch.Tensor, wg: torch.Tensor, N1: int, K1: int, N2: int, K2: int, fold1: bool,
                        fold2: bool) -> torch.Tensor:
    return torch.empty((x.shape[0], N2), dtype=torch.bfloat16, device=x.device)


def register() -> None:
    """torch.ops.r9700.shared_expert (host-known shapes, no synchronisation: graph-capturable)."""
    global _registered
    if not _registered:
        register_custom_op(_LIB, "shared_expert", shared_expert, [], _shared_expert_fake)
        _registered = True


def _fused_forward(self, x: torch.Tensor) -> torch.Tensor:
    sw = SharedExpertWeights.from_module(self) if x.dim() == 2 and x.dtype == torch.bfloat16 else None
    if sw is None:
        return self._r9k_stock_forward(x)
    W1, W2 = sw.gate_up, sw.down
    return torch.ops.r9700.shared_expert(x.contiguous(), W1.wq, W1.wsr, W2.wq, W2.wsr, sw.wg, W1.N, W1.K, W2.N,
                                         W2.K, W1.fold, W2.fold)


def _not_bindable(mlp) -> str | None:
    """Why a gated-MLP module cannot take the fused forward, or None when it can: it needs gate_up / down projections
    and an expert gate that is a plain (unquantized, bias-free) bf16 [1, hidden] linear."""
    if not (hasattr(mlp, "gate_up_proj") and hasattr(mlp, "down_proj")):
        return "no gate_up / down projections"
    eg = getattr(mlp, "expert_gate", None)
    if eg is None:
        return "no expert gate"
    w = getattr(eg, "weight", None)
    if not isinstance(w, torch.Tensor) or w.dtype != torch.bfloat16 or w.dim() != 2 or w.shape[0] != 1:
        return "expert gate is not a bf16 [1, hidden] weight"
    if getattr(eg, "bias", None) is not None:
        return "expert gate has a bias"
    if type(getattr(eg, "quant_method", None)).__name__ != "UnquantizedLinearMethod":
        return "expert gate is quantized"
    return None


def install(model: torch.nn.Module) -> int:
    """Bind the fused forward on the gated shared-expert MLPs under `model`; returns how many were bound (already
    bound modules are skipped, so calling it again binds nothing)."""
    if os.environ.get("R9K_SHARED_EXPERT", "r9k") != "r9k" or not available():
        return 0
    register()
    log = get_logger(__name__)
    bound = 0
    for name, mod in model.named_modules():
        if type(mod).__name__ not in SHARED_MLP_CLASSES or getattr(mod, "_r9k_shared", False):
            continue
        why = _not_bindable(mod)
        if why is not None:
            if getattr(mod, "expert_gate", None) is not None:
                log.warning("r9700: fused shared expert skipped for %s (%s)", name, why)
            continue
        mod._r9k_stock_forward = mod.forward
        mod.forward = types.MethodType(_fused_forward, mod)
        mod._r9k_shared = True
        bound += 1
    if bound:
        log.info("r9700: fused shared expert on %d modules (quant + gate, gate_up, SiLU quant, down x gate)", bound)
    return bound
