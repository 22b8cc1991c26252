"""Load-time preparation of an MXFP4 MoE layer for the gfx950 kernels (the names of the reference's
r9700_vllm/moe/prep.py: `permute_in_place`, `pack_scales_gpu`, `as_param`, `maybe_attach_cache`), plus the whole step
as one vLLM-free function, `prepare_layer_mxfp4`, which R9kMxfp4MoEMethod calls after loading.

The fragment-order permute (kernels/moe.py permute_fragments) moves bytes within each expert without changing its
size, so it runs IN PLACE inside the checkpoint tensor's storage (device memory or mapped host memory): experts go
through one staging buffer a chunk at a time (CHUNK_BYTES), so the extra memory is one chunk, never a second copy
of the layer. The e8m0 scales (1/16 of the weight bytes) are repacked into a new [E, K/32 + 1, N] device tensor.
"""
from __future__ import annotations

import re

import torch

from .._compat import get_logger
from ..kernels import moe as KM

CHUNK_BYTES = 256 << 20
_log = get_logger(__name__)


def _experts_per_chunk(per_expert_bytes: int, chunk_bytes: int | None) -> int:
    return max(1, (chunk_bytes or CHUNK_BYTES) // max(1, per_expert_bytes))


def permute_in_place(packed: torch.Tensor, chunk_bytes: int | None = None) -> torch.Tensor:
    """packed [E, N, K/2] uint8 checkpoint codes -> the same storage viewed as [E, N*K/8] int32 in fragment order.
    Each chunk of experts is permuted into a staging buffer on the device (one allocation for the whole call) and
    copied back over itself."""
    E, N, Kh = packed.shape
    step = _experts_per_chunk(N * Kh, chunk_bytes)
    dev = packed.device if packed.is_cuda else torch.device("cuda", torch.cuda.current_device())
    stage = torch.empty((min(step, E), N * Kh // 4), dtype=torch.int32, device=dev)
    for e0 in range(0, E, step):
        n = min(step, E - e0)
        src = packed[e0:e0 + n]
        KM.permute_fragments(src.to(dev), out=stage[:n])
        src.view(n, -1).copy_(stage[:n].view(torch.uint8).view(n, -1))
    return packed.view(E, -1).view(torch.int32)


def pack_scales_gpu(scale: torch.Tensor, device, chunk_bytes: int | None = None) -> torch.Tensor:
    """[E, N, K/32] e8m0 (any device) -> the pack_scales layout [E, K/32 + 1, N] on `device`, chunk by chunk of
    experts straight into the result."""
    E, N, KB = scale.shape
    out = torch.empty((E, KB + 1, N), dtype=torch.uint8, device=device)
    step = _experts_per_chunk(N * KB, chunk_bytes)
    for e0 in range(0, E, step):
        n = min(step, E - e0)
        KM.pack_scales(scale[e0:e0 + n].to(device), out=out[e0:e0 + n])
    return out


def as_param(t: torch.Tensor, like: torch.nn.Parameter) -> torch.nn.Parameter:
    """t as a frozen Parameter that keeps `like`'s host-offload mark (vLLM's `_vllm_is_uva_offloaded`)."""
    p = torch.nn.Parameter(t, requires_grad=False)
    if getattr(like, "_vllm_is_uva_offloaded", False):
        p._vllm_is_uva_offloaded = True
    return p


def prepare_layer_mxfp4(layer, device=None, chunk_bytes: int | None = None) -> None:
    """Compressed-tensors MXFP4 MoE checkpoint tensors on `layer` (w13 / w2 `_weight_packed` [E, N, K/2] u8 and
    `_weight_scale` [E, N, K/32] e8m0) -> the kernels' layout, in place: `w13_weight` / `w2_weight` (int32 fragment
    order over the same storage), `_weight_scale` repacked [E, K/32 + 1, N] on `device`, `_r9k_fold` = (False,
    False); the `_weight_packed` attributes are removed."""
    dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
    for pre in ("w13", "w2"):
        packed = getattr(layer, f"{pre}_weight_packed")
        scales = pack_scales_gpu(getattr(layer, f"{pre}_weight_scale").data, dev, chunk_bytes)
        codes = permute_in_place(packed.data, chunk_bytes)
        setattr(layer, f"{pre}_weight", as_param(codes, packed))
        delattr(layer, f"{pre}_weight_packed")
        setattr(layer, f"{pre}_weight_scale", torch.nn.Parameter(scales, requires_grad=False))
    layer._r9k_fold = (False, False)


def _layer_index(layer) -> int:
    m = re.search(r"layers\.(\d+)\.", getattr(layer, "layer_name", "") or "")
    return int(m.group(1)) if m else 0


def cache_plan(layer):
    """(slots, (N1, K1, N2, K2), bytes per expert) for host-offloading `layer`'s experts behind a VRAM cache, or None
    when no cache is asked for (R9K_EXPERT_CACHE_GB / R9K_EXPERT_CACHE_SLOTS unset) or the layer is device-resident
    and only host-offloaded layers are cached (R9K_EXPERT_CACHE_HOST_ONLY=1, the default)."""
    from . import cache as C
    s13, s2 = layer.w13_weight_scale, layer.w2_weight_scale
    dims = (s13.shape[2], (s13.shape[1] - 1) * KM.GROUP, s2.shape[2], (s2.shape[1] - 1) * KM.GROUP)
    per_expert = sum(t[0].numel() * t.element_size() for t in (layer.w13_weight, layer.w2_weight, s13, s2))
    slots = C.slots_per_layer(per_expert)
    if slots <= 0:
        return None
    if C.host_only() and not (C.is_host(layer.w13_weight) and C.is_host(layer.w2_weight)):
        return None
    return slots, dims, per_expert


def maybe_attach_cache(method, layer) -> None:
    """Host-offloaded experts with a per-layer VRAM LRU cache (moe/cache.py) when cache_plan asks for one: the
    layer's weights move to mapped host memory (unless already there), the scales' host copies back the cold pass,
    and the experts object (method.moe_kernel.fused_experts, when present) gets `r9k_cache`. Off by default: 288 GB
    of HBM holds every expert of the configurations this build targets."""
    from . import cache as C
    plan = cache_plan(layer)
    if plan is None:
        return
    slots, (N1, K1, N2, K2), per_expert = plan
    for name in ("w13_weight", "w2_weight"):
        p = getattr(layer, name)
        if not C.is_host(p):
            setattr(layer, name, as_param(C.to_host(p.data), p))
    cache = C.LayerCache(_layer_index(layer), layer.w13_weight.data, layer.w2_weight.data,
                         layer.w13_weight_scale.data, layer.w2_weight_scale.data, N1, K1, N2, K2, slots)
    layer.w13_weight_scale = torch.nn.Parameter(cache.h_s13, requires_grad=False)
    layer.w2_weight_scale = torch.nn.Parameter(cache.h_s2, requires_grad=False)
    experts = getattr(getattr(method, "moe_kernel", None), "fused_experts", None)
    if experts is not None:
        try:
            from vllm.model_executor.layers.fused_moe.config import mxfp4_w4a16_moe_quant_config
            method.moe_quant_config = mxfp4_w4a16_moe_quant_config(w1_scale=layer.w13_weight_scale,
                                                                   w2_scale=layer.w2_weight_scale)
            experts.quant_config = method.moe_quant_config
        except ImportError:
            pass
        experts.w1_scale, experts.w2_scale = cache.h_s13, cache.h_s2
        experts.r9k_cache = cache
    layer.r9k_cache = cache
    torch.cuda.empty_cache()
    _log.info("r9700: expert cache for layer %d: %d slots (%.2f MiB an expert)", cache.layer_idx, cache.S,
              per_expert / 2**20)
