"""NVFP4 checkpoints on gfx950: served natively (the checkpoint's exact bits) or converted to MXFP4 while loading;
and dense MXFP4 re-quantisation of arbitrary weights. The names, modes and argument meanings of the reference's
r9700_vllm/quant/nvfp4.py (`dequant_nvfp4`, `quantize_mxfp4_search`, `nvfp4_to_mxfp4`, `mxfp4_linearize`,
`prep_native_moe`, `make_dense_scheme_cls`, `make_native_dense_scheme_cls`, `make_moe_method_cls`).

NVFP4 = E2M1 codes with an FP8-E4M3 scale per 16 values and an FP32 global scale, which compressed-tensors stores as
a divisor. Conversion per 32-block (r9k_nvfp4_to_mxfp4, one kernel launch per chunk of rows):

  exact dequant   w = e2m1 * s16 / global                       (fp32)
  requant         e = ceil(log2(amax / 6)) (no clipping) or e - 1 (clips the top value(s), finer grid for the rest),
                  values rounded to the nearest E2M1 (ties to the smaller magnitude), the candidate with the lower
                  squared error kept.

Modes, as the reference's: dense linears NATIVE by default (R9K_NVFP4=native: r9k_moe_nvfp4a8 over the
checkpoint's codes and scales, the global scale as a per-row fp32 multiplier; R9K_NVFP4=mxfp4 converts); MoE layers
CONVERT by default (R9K_NVFP4_MOE=native serves them natively).

The load-time work is in plain functions over a layer object (`convert_dense_layer`, `prepare_native_dense_layer`,
`convert_moe_layer`, `prep_native_moe`, `moe_row_divisors`), so it runs, and is tested, without vLLM; the vLLM scheme
and method classes built by the make_* factories only call them. Everything but `dequant_nvfp4` (a torch expression,
the exact reference dequant used in checks) runs on the GPU: there is no CPU path.
"""
from __future__ import annotations

import os

import torch

from .._compat import get_logger
from ..kernels import moe as KM

logger = get_logger(__name__)

_E2M1_MAG = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
_E2M1 = torch.cat([_E2M1_MAG, -_E2M1_MAG])                          # code c: sign bit 3, magnitude bits 0-2
_MID = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])       # E2M1 decision thresholds on |x|
_NV_ATTRS = ("weight_packed", "weight_global_scale", "input_global_scale")


def dequant_nvfp4(packed: torch.Tensor, scale16: torch.Tensor, row_div: torch.Tensor) -> torch.Tensor:
    """packed [N, K/2] u8 (low nibble = even element), scale16 [N, K/16] e4m3, row_div [N] fp32 -> fp32 [N, K] =
    e2m1(code) * float(scale16) / row_div, the multiply then the division in fp32 (exact up to the division)."""
    N = packed.shape[0]
    codes = torch.stack((packed & 0xF, packed >> 4), dim=-1).reshape(N, -1, 16).long()
    mag = _E2M1_MAG.to(packed.device)[codes & 7]
    val = torch.where(codes >= 8, -mag, mag) * scale16.float().unsqueeze(-1)
    return val.reshape(N, -1) / row_div.float().reshape(N, 1)


def _gpu() -> torch.device:
    return torch.device("cuda", torch.cuda.current_device())


def quantize_mxfp4_search(w: torch.Tensor, candidates=(0, -1)):
    """fp32 [N, K] (K % 32 == 0) -> (packed [N, K/2] u8, e8m0 [N, K/32] u8) on w's device: per 32-block the better of
    the exponents e and e - 1 (r9k_quantize_mxfp4_search; a CPU `w` is sent to the GPU and the result brought back)."""
    if tuple(candidates) != (0, -1):
        raise ValueError("the libr9k search evaluates the candidates (0, -1)")
    N, K = w.shape
    dev = w.device if w.is_cuda else _gpu()
    src = w.to(dev, torch.float32).contiguous()
    packed = torch.empty((N, K // 2), dtype=torch.uint8, device=dev)
    e8 = torch.empty((N, K // 32), dtype=torch.uint8, device=dev)
    rc = KM.lib().r9k_quantize_mxfp4_search(src.data_ptr(), packed.data_ptr(), e8.data_ptr(), N, K, KM._stream())
    if rc:
        raise RuntimeError(f"r9k_quantize_mxfp4_search failed ({rc}) N={N} K={K}")
    return packed.to(w.device), e8.to(w.device)


def nvfp4_to_mxfp4(packed, scale16, row_div, rows_per_chunk: int = 2048):
    """NVFP4 [N, K/2] codes + [N, K/16] e4m3 scales + [N] divisors -> (MXFP4 codes [N, K/2] u8, e8m0 [N, K/32] u8) on
    packed's device, converted on the GPU `rows_per_chunk` rows at a time (host-resident inputs are copied over a
    chunk at a time)."""
    N, Kh = packed.shape
    K = 2 * Kh
    dev = _gpu()
    out_p = torch.empty_like(packed)
    out_e = torch.empty((N, K // 32), dtype=torch.uint8, device=packed.device)
    on_gpu = out_p.is_cuda
    for r0 in range(0, N, rows_per_chunk):
        r1 = min(N, r0 + rows_per_chunk)
        p = packed[r0:r1].to(dev).contiguous()
        s = scale16[r0:r1].to(dev).contiguous().view(torch.uint8)
        d = row_div[r0:r1].to(dev, torch.float32).contiguous()
        dst_p = out_p[r0:r1] if on_gpu else torch.empty_like(p)
        dst_e = out_e[r0:r1] if on_gpu else torch.empty((r1 - r0, K // 32), dtype=torch.uint8, device=dev)
        rc = KM.lib().r9k_nvfp4_to_mxfp4(p.data_ptr(), s.data_ptr(), d.data_ptr(), dst_p.data_ptr(),
                                         dst_e.data_ptr(), r1 - r0, K, KM._stream())
        if rc:
            raise RuntimeError(f"r9k_nvfp4_to_mxfp4 failed ({rc}) rows={r1 - r0} K={K}")
        if not on_gpu:
            out_p[r0:r1].copy_(dst_p)
            out_e[r0:r1].copy_(dst_e)
    return out_p, out_e


def global_row_divisors(global_scale: torch.Tensor, widths) -> torch.Tensor:
    """fp32 [sum(widths)]: each output row's NVFP4 global divisor (one per fused shard of `widths` rows, or one for
    all rows)."""
    g = global_scale.detach().float().reshape(-1)
    n = int(sum(widths))
    if g.numel() == 1:
        return g.expand(n).contiguous()
    return torch.cat([g[i].expand(int(w)) for i, w in enumerate(widths)])


_row_div = global_row_divisors


def _drop(layer, names) -> None:
    for n in names:
        if hasattr(layer, n):
            delattr(layer, n)


def _param(t: torch.Tensor) -> torch.nn.Parameter:
    return torch.nn.Parameter(t, requires_grad=False)


# ------------------------------------------------------------------------------------------------ dense
def convert_dense_layer(layer) -> None:
    """NVFP4 dense linear (weight_packed [N, K/2], weight_scale [N, K/16] e4m3, weight_global_scale, logical_widths)
    -> MXFP4 checkpoint layout in place: weight [N, K/2] u8 codes and weight_scale [N, K/32] e8m0 (the dense MXFP4
    kernel's prep then lays them out)."""
    div = global_row_divisors(layer.weight_global_scale.data, list(layer.logical_widths))
    codes, e8 = nvfp4_to_mxfp4(layer.weight_packed.data, layer.weight_scale.data, div)
    _drop(layer, _NV_ATTRS)
    layer.weight = _param(codes)
    layer.weight_scale = _param(e8)


def prepare_native_dense_layer(layer) -> None:
    """NVFP4 dense linear -> the native kernel's layout in place (codes and e4m3 scales re-laid out, bits kept; the
    global divisor as a per-row fp32 multiplier): weight, weight_scale, weight_row_mult and `_r9k_nk` = (N, K)."""
    packed, s16 = layer.weight_packed.data, layer.weight_scale.data
    N, Kh = packed.shape
    if N % 16 or (2 * Kh) % 16:
        raise ValueError(f"r9700 native NVFP4: unsupported shape N={N} K={2 * Kh}")
    mult = 1.0 / global_row_divisors(layer.weight_global_scale.data, list(layer.logical_widths))
    W = KM.prepare_nvfp4_weights(packed.unsqueeze(0), s16.unsqueeze(0), mult.to(packed.device).unsqueeze(0))
    _drop(layer, _NV_ATTRS + ("weight_scale",))
    layer.weight, layer.weight_scale, layer.weight_row_mult = _param(W.wq), _param(W.ws), _param(W.wg)
    layer._r9k_nk = (N, 2 * Kh)


def native_dense_forward(layer, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    from .. import ops
    N, K = layer._r9k_nk
    y = ops.nvfp4_linear(x, layer.weight, layer.weight_scale, layer.weight_row_mult, N, K).to(x.dtype)
    return y if bias is None else y + bias


def mxfp4_linearize(layer, W: torch.Tensor, rows_per_chunk: int = 4096):
    """Serve `layer` from a dense weight W [N, K] (fp32 / bf16) as MXFP4: MSE-searched e8m0 exponents per 32-block
    (quantize_mxfp4_search, `rows_per_chunk` rows per launch), then the dense MXFP4 kernel's prep. Returns the kernel
    object whose apply_weights(layer, x, bias) is the forward (vLLM's R9700Mxfp4LinearKernel when vLLM is installed,
    else linear.mxfp4.DenseMxfp4Kernel)."""
    from ..linear import mxfp4 as LX
    N, K = W.shape
    codes = torch.empty((N, K // 2), dtype=torch.uint8, device=W.device)
    e8 = torch.empty((N, K // 32), dtype=torch.uint8, device=W.device)
    for r0 in range(0, N, rows_per_chunk):
        c, e = quantize_mxfp4_search(W[r0:r0 + rows_per_chunk].float())
        codes[r0:r0 + c.shape[0]].copy_(c)
        e8[r0:r0 + c.shape[0]].copy_(e)
    layer.weight, layer.weight_scale = _param(codes), _param(e8)
    kern = LX.dense_kernel()
    kern.process_weights_after_loading(layer)
    return kern


def make_dense_scheme_cls(base):
    """vLLM's CompressedTensorsW4A4Fp4 with the checkpoint converted to MXFP4 after loading and served by the dense
    MXFP4 kernel (R9K_NVFP4=mxfp4)."""

    class R9kNvfp4AsMxfp4(base):

        def process_weights_after_loading(self, layer) -> None:
            convert_dense_layer(layer)
            logger.info("r9700: NVFP4 linears converted to MXFP4 at load -> libr9k (fp8 activations)")
            self.kernel.process_weights_after_loading(layer)

        def apply_weights(self, layer, x, bias=None):
            return self.kernel.apply_weights(layer, x, bias)

    return R9kNvfp4AsMxfp4


def make_native_dense_scheme_cls(base):
    """vLLM's CompressedTensorsW4A4Fp4 served by libr9k's native NVFP4 kernel (R9K_NVFP4=native, the default): the
    checkpoint's bits kept, the activations as per-row fp8 (the checkpoint's NVFP4 activation quant is not used)."""

    class R9kNvfp4Native(base):

        def process_weights_after_loading(self, layer) -> None:
            prepare_native_dense_layer(layer)
            logger.info("r9700: NVFP4 linears on libr9k's native NVFP4 kernel (exact weights, fp8 activations)")

        def apply_weights(self, layer, x, bias=None):
            return native_dense_forward(layer, x, bias)

    return R9kNvfp4Native


# -------------------------------------------------------------------------------------------------- MoE
MOE_MODE = (os.environ.get("R9K_NVFP4_MOE", "") or "mxfp4").lower()
_MOE_NV_ATTRS = ("w13_weight_global_scale", "w2_weight_global_scale", "w13_input_global_scale",
                 "w2_input_global_scale")


def moe_row_divisors(layer) -> tuple[torch.Tensor, torch.Tensor]:
    """The per-row global divisors of an NVFP4 MoE layer: (w13 [E, 2I], w2 [E, hidden]). w13 carries one divisor per
    fused shard (gate, up), w2 one per expert."""
    g13 = layer.w13_weight_global_scale.data.float().reshape(layer.w13_weight_packed.shape[0], -1)
    rows13 = layer.w13_weight_packed.shape[1]
    div13 = g13.repeat_interleave(rows13 // g13.shape[1], dim=1)
    g2 = layer.w2_weight_global_scale.data.float().reshape(-1, 1)
    div2 = g2.expand(-1, layer.w2_weight_packed.shape[1])
    return div13, div2


def convert_moe_layer(layer) -> None:
    """NVFP4 MoE layer (w13 / w2 _weight_packed [E, N, K/2], _weight_scale [E, N, K/16] e4m3, _weight_global_scale)
    -> MXFP4 checkpoint layout IN PLACE: the codes overwrite the packed tensors expert by expert (same size), the
    scales become [E, N, K/32] e8m0, the global scales are dropped. moe.prep.prepare_layer_mxfp4 then lays them out."""
    div13, div2 = moe_row_divisors(layer)
    for pre, div in (("w13", div13), ("w2", div2)):
        packed = getattr(layer, f"{pre}_weight_packed").data
        s16 = getattr(layer, f"{pre}_weight_scale").data
        E, N, Kh = packed.shape
        e8 = torch.empty((E, N, 2 * Kh // 32), dtype=torch.uint8, device=s16.device)
        for e in range(E):
            codes, ex = nvfp4_to_mxfp4(packed[e], s16[e], div[e])
            packed[e].copy_(codes)
            e8[e].copy_(ex)
        setattr(layer, f"{pre}_weight_scale", _param(e8))
    _drop(layer, _MOE_NV_ATTRS)


def prep_native_moe(layer, div13: torch.Tensor, div2: torch.Tensor) -> None:
    """Serve an NVFP4 MoE layer's experts exactly: codes and e4m3 scales re-laid out for r9k_moe_nvfp4a8
    (prepare_nvfp4_weights), the per-row divisors (div13 [E, 2I], div2 [E, hidden]) as fp32 multipliers. Leaves
    w13_weight / w2_weight (int32), *_weight_scale (u8), *_weight_row_mult (fp32) and `_r9k_nvfp4` on the layer and
    drops *_weight_packed."""
    for pre, div in (("w13", div13), ("w2", div2)):
        packed = getattr(layer, f"{pre}_weight_packed").data
        s16 = getattr(layer, f"{pre}_weight_scale").data
        E, N, Kh = packed.shape
        if s16.shape != (E, N, 2 * Kh // 16) or tuple(div.shape) != (E, N):
            raise ValueError(f"prep_native_moe {pre}: scales {tuple(s16.shape)}, divisors {tuple(div.shape)} for "
                             f"codes {tuple(packed.shape)}")
        W = KM.prepare_nvfp4_weights(packed, s16, (1.0 / div.float()).to(packed.device))
        _drop(layer, (f"{pre}_weight_packed",))
        setattr(layer, f"{pre}_weight", _param(W.wq))
        setattr(layer, f"{pre}_weight_scale", _param(W.ws))
        setattr(layer, f"{pre}_weight_row_mult", _param(W.wg))
    layer._r9k_fold = (False, False)
    layer._r9k_nvfp4 = True


def make_moe_method_cls(mxfp4_method_cls):
    """An MoE method that creates vLLM's NVFP4 checkpoint parameters (CompressedTensorsW4A4Nvfp4MoEMethod's
    create_weights) and, after loading, either converts them to MXFP4 in place and continues as `mxfp4_method_cls`
    (default), or serves them natively (R9K_NVFP4_MOE=native)."""
    from vllm.model_executor.layers.quantization.compressed_tensors.compressed_tensors_moe.compressed_tensors_moe_w4a4_nvfp4 import (  # noqa: E501
        CompressedTensorsW4A4Nvfp4MoEMethod as NvMethod,
    )

    class R9kNvfp4MoEMethod(mxfp4_method_cls):

        def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition, params_dtype,
                           **extra_weight_attrs):
            # the NVFP4 method's parameter set wants group_size 16 while it creates them; restore ours after
            had = "group_size" in self.__dict__
            prev = self.__dict__.get("group_size")
            self.group_size = 16
            try:
                NvMethod.create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition,
                                        params_dtype, **extra_weight_attrs)
            finally:
                if had:
                    self.group_size = prev
                else:
                    del self.__dict__["group_size"]

        def process_weights_after_loading(self, layer) -> None:
            if MOE_MODE == "native":
                prep_native_moe(layer, *moe_row_divisors(layer))
                _drop(layer, _MOE_NV_ATTRS)
                logger.info("r9700: NVFP4 MoE experts served natively by libr9k (exact checkpoint bits)")
                self._install_kernel(layer)
                return
            convert_moe_layer(layer)
            logger.info("r9700: NVFP4 MoE experts converted to MXFP4 at load -> libr9k")
            super().process_weights_after_loading(layer)

    return R9kNvfp4MoEMethod
