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
    """The reference's host-offloaded expert cache is not part of the gfx950 build (288 GB of HBM holds the
    experts); weights stay device-resident."""
    return None
