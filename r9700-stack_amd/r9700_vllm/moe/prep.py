"""Weight preparation for R9kMxfp4MoEMethod (quant/ct.py): same names and contract as the reference's
r9700_vllm/moe/prep.py:19-61.

The fragment-order permute (kernels/moe.py permute_fragments) moves bytes within each expert without changing its
size, so it runs IN PLACE, chunk by chunk, inside the checkpoint tensor's own storage (device or pinned host
memory). The E8M0 scales are repacked on the device into a new [E, K/32 + 1, N] tensor (~1/16 of the weights).
"""
from __future__ import annotations

import torch

_CHUNK_BYTES = 256 << 20


def permute_in_place(packed: torch.Tensor) -> torch.Tensor:
    """packed [E, N, K/2] uint8 -> the same storage viewed as [E, N*K/8] int32 in fragment order."""
    from ..kernels.moe import permute_fragments
    E, N, Kh = packed.shape
    per = N * Kh
    step = max(1, _CHUNK_BYTES // per)
    for e0 in range(0, E, step):
        e1 = min(E, e0 + step)
        tmp = permute_fragments(packed[e0:e1])
        packed[e0:e1].view(e1 - e0, -1).copy_(tmp.view(torch.uint8).view(e1 - e0, -1))
        del tmp
    return packed.view(E, -1).view(torch.int32)


def pack_scales_gpu(scale: torch.Tensor, device) -> torch.Tensor:
    """[E, N, K/32] E8M0 (any device) -> pack_scales layout [E, K/32 + 1, N] on `device`, chunked by expert."""
    from ..kernels.moe import pack_scales
    E = scale.shape[0]
    per = scale[0].numel()
    step = max(1, _CHUNK_BYTES // per)
    out = torch.empty((E, scale.shape[2] + 1, scale.shape[1]), dtype=torch.uint8, device=device)
    for e0 in range(0, E, step):
        e1 = min(E, e0 + step)
        out[e0:e1].copy_(pack_scales(scale[e0:e1].to(device)))
    return out


def as_param(t: torch.Tensor, like: torch.nn.Parameter) -> torch.nn.Parameter:
    p = torch.nn.Parameter(t, requires_grad=False)
    if getattr(like, "_vllm_is_uva_offloaded", False):
        p._vllm_is_uva_offloaded = True
    return p


def maybe_attach_cache(method, layer) -> None:
    """Host-offloaded experts with a per-layer VRAM LRU cache (moe/cache.py), when R9K_EXPERT_CACHE_GB or
    R9K_EXPERT_CACHE_SLOTS asks for one (reference moe/prep.py:64-101): the layer's weights move to mapped host
    memory (unless already there), the scales' host copies back the cold pass, and the experts object gets
    `r9k_cache`. Off by default: 288 GB of HBM holds every expert of the BASELINE models."""
    import re
    from . import cache as C
    from ..kernels.moe import GROUP
    s13, s2 = layer.w13_weight_scale, layer.w2_weight_scale
    N1, K1 = s13.shape[2], (s13.shape[1] - 1) * GROUP
    N2, K2 = s2.shape[2], (s2.shape[1] - 1) * GROUP
    per_expert = (layer.w13_weight[0].numel() * 4 + layer.w2_weight[0].numel() * 4 + s13[0].numel() + s2[0].numel())
    slots = C.slots_per_layer(per_expert)
    if slots <= 0:
        return
    if C.host_only() and not (C.is_host(layer.w13_weight) and C.is_host(layer.w2_weight)):
        return                                   # the layer is device-resident already: nothing to cache
    name = getattr(layer, "layer_name", "") or ""
    m = re.search(r"layers\.(\d+)\.", name)
    idx = int(m.group(1)) if m else 0
    w13, w2 = layer.w13_weight.data, layer.w2_weight.data
    if not C.is_host(w13):
        w13 = C.to_host(w13)
        layer.w13_weight = as_param(w13, layer.w13_weight)
    if not C.is_host(w2):
        w2 = C.to_host(w2)
        layer.w2_weight = as_param(w2, layer.w2_weight)
    cache = C.LayerCache(idx, w13, w2, s13.data, s2.data, N1, K1, N2, K2, slots)
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
            experts.w1_scale, experts.w2_scale = cache.h_s13, cache.h_s2
        experts.r9k_cache = cache
    layer.r9k_cache = cache
    torch.cuda.empty_cache()
