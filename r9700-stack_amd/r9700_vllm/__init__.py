"""r9700_vllm for MI355X (gfx950): the quantized-MoE hot path of r9700-stack behind the same plugin surface.

Entry point (vllm.general_plugins): r9700 = r9700_vllm:register. register() adds the torch custom ops
(r9700::mxfp4_linear, r9700::moe_route) and, when vLLM is installed, the compressed-tensors override for MXFP4 /
NVFP4 MoE and dense layers (quant/ct.py). Only the MoE hot path is in this build: the reference's model classes,
attention backends, collectives and fp8 dense GEMMs are not. R9K_DISABLE=quant turns the quant override off.
"""
import os

__version__ = "0.4.3+gfx950"


def _disabled(name: str) -> bool:
    return name in {s.strip() for s in os.environ.get("R9K_DISABLE", "").split(",") if s.strip()}


def register() -> None:
    from ._compat import get_logger, vllm_available
    log = get_logger("r9700_vllm")
    done = []
    from . import ops
    ops.register()
    from .moe import route
    route.register()
    done.append("ops:mxfp4_linear,moe_route")
    if vllm_available() and not _disabled("quant"):
        from .quant import ct  # noqa: F401  (registers "compressed-tensors")
        done.append("quant:compressed-tensors")
    log.info("r9700_vllm %s registered: %s", __version__, ", ".join(done))
