"""NVFP4 checkpoints on gfx950: served natively (exact checkpoint bits) or converted to MXFP4 while loading.

Mirrors the reference's r9700_vllm/quant/nvfp4.py (names, argument meaning, modes). NVFP4 = E2M1 values with an
FP8-E4M3 scale per 16 values and an FP32 global scale (stored by compressed-tensors as a divisor).

Modes, as the reference's: dense linears default to NATIVE (R9K_NVFP4=native: libr9k's r9k_moe_nvfp4a8 over the
checkpoint's codes and scales, the global scale as a per-row fp32 multiplier; R9K_NVFP4=mxfp4 converts); MoE layers
CONVERT by default (R9K_NVFP4_MOE=native serves them natively, on the decode-family kernel at every width).

Conversion per 32-group (reference nvfp4.py:39-90), done by one libr9k kernel (r9k_nvfp4_to_mxfp4) per chunk:

  exact dequant   w = e2m1 * s16_e4m3 / global      (fp32)
  requant         E8M0 exponent e = ceil(log2(amax/6)) (no clipping) vs e-1 (clips the top value(s), finer grid for
                  the rest), round-to-nearest E2M1 (ties to the smaller magnitude), keeping the candidate with the
                  lower squared error for that group.

quantize_mxfp4_search runs the same search on an arbitrary fp32 weight (r9k_quantize_mxfp4_search). Both need a
GPU: there is no CPU path. dequant_nvfp4 stays a torch expression (it is the exact reference dequant the tests
compare against, and is not on the serving path).
"""
from __future__ import annotations

import os

import torch

from .._compat import get_logger
from ..kernels import moe as KM

logger = get_logger(__name__)

_E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])
_MID = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])      # E2M1 decision thresholds on |x|


def dequant_nvfp4(packed: torch.Tensor, scale16: torch.Tensor, row_div: torch.Tensor) -> torch.Tensor:
    """packed [N, K/2] u8 (low nibble = even element), scale16 [N, K/16] e4m3, row_div [N] fp32 -> fp32 [N, K]."""
    N, Kh = packed.shape
    lut = _E2M1.to(packed.device)
    codes = torch.stack((packed & 0x0F, packed >> 4), dim=-1).reshape(N, Kh * 2).long()
    v = lut[codes].reshape(N, -1, 16) * scale16.float().unsqueeze(-1)
    return v.reshape(N, Kh * 2) / row_div.float().unsqueeze(-1)


def _device() -> torch.device:
    return torch.device("cuda", torch.cuda.current_device())


def quantize_mxfp4_search(w: torch.Tensor, candidates=(0, -1)):
    """fp32 [N, K] (K % 32 == 0) -> (packed [N, K/2] u8, e8m0 [N, K/32] u8) on w.device, per-group best of {e, e-1}.
    Runs on the GPU (a CPU `w` is copied over and the result copied back)."""
    if tuple(candidates) != (0, -1):
        raise ValueError("the libr9k search evaluates the candidates (0, -1)")
    N, K = w.shape
    dev = w.device if w.is_cuda else _device()
    wd = w.to(dev, torch.float32).contiguous()
    p = torch.empty((N, K // 2), dtype=torch.uint8, device=dev)
    e = torch.empty((N, K // 32), dtype=torch.uint8, device=dev)
    rc = KM.lib().r9k_quantize_mxfp4_search(wd.data_ptr(), p.data_ptr(), e.data_ptr(), N, K, KM._stream())
    if rc:
        raise RuntimeError(f"r9k_quantize_mxfp4_search failed ({rc}) N={N} K={K}")
    return p.to(w.device), e.to(w.device)


def nvfp4_to_mxfp4(packed, scale16, row_div, rows_per_chunk: int = 2048):
    """Chunked on the GPU. Returns (packed [N, K/2] u8 on packed.device, e8m0 [N, K/32] u8 on packed.device)."""
    dev = _device()
    N, Kh = packed.shape
    out_p = torch.empty_like(packed)
    out_s = torch.empty((N, Kh * 2 // 32), dtype=torch.uint8, device=packed.device)
    L = KM.lib()
    for r0 in range(0, N, rows_per_chunk):
        r1 = min(N, r0 + rows_per_chunk)
        p = packed[r0:r1].to(dev).contiguous()
        s = scale16[r0:r1].to(dev).contiguous().view(torch.uint8)
        d = row_div[r0:r1].to(dev, torch.float32).contiguous()
        po = out_p[r0:r1] if out_p.is_cuda else torch.empty_like(p)
        so = out_s[r0:r1] if out_s.is_cuda else torch.empty((r1 - r0, Kh * 2 // 32), dtype=torch.uint8, device=dev)
        rc = L.r9k_nvfp4_to_mxfp4(p.data_ptr(), s.data_ptr(), d.data_ptr(), po.data_ptr(), so.data_ptr(), r1 - r0,
                                  Kh * 2, KM._stream())
        if rc:
            raise RuntimeError(f"r9k_nvfp4_to_mxfp4 failed ({rc}) rows={r1 - r0} K={Kh * 2}")
        if not out_p.is_cuda:
            out_p[r0:r1].copy_(po)
            out_s[r0:r1].copy_(so)
    return out_p, out_s


def _row_div(global_scale: torch.Tensor, widths) -> torch.Tensor:
    g = global_scale.detach().float().reshape(-1)
    if g.numel() == 1:
        return g.expand(sum(widths)).contiguous()
    return torch.repeat_interleave(g, torch.tensor(widths, device=g.device))


# ------------------------------------------------------------------------------------------------ dense
def make_dense_scheme_cls(base):
    """Subclass of vLLM's CompressedTensorsW4A4Fp4: stock create_weights (the checkpoint loads as-is), MXFP4
    conversion + the libr9k dense MXFP4 kernel after loading."""

    class R9kNvfp4AsMxfp4(base):

        def process_weights_after_loading(self, layer) -> None:
            from torch.nn.parameter import Parameter
            widths = list(layer.logical_widths)
            div = _row_div(layer.weight_global_scale.data, widths)
            p, s = nvfp4_to_mxfp4(layer.weight_packed.data, layer.weight_scale.data, div)
            del layer.weight_packed
            del layer.weight_global_scale
            if hasattr(layer, "input_global_scale"):
                del layer.input_global_scale
            layer.weight = Parameter(p, requires_grad=False)
            layer.weight_scale = Parameter(s, requires_grad=False)
            logger.info("r9700: NVFP4 linears converted to MXFP4 at load -> libr9k (fp8 activations)")
            self.kernel.process_weights_after_loading(layer)

        def apply_weights(self, layer, x, bias=None):
            return self.kernel.apply_weights(layer, x, bias)

    return R9kNvfp4AsMxfp4


def make_native_dense_scheme_cls(base):
    """Subclass of vLLM's CompressedTensorsW4A4Fp4 served by libr9k's native NVFP4 kernel (R9K_NVFP4=native, the
    default for dense linears; reference nvfp4.py:145-180): the checkpoint's e2m1 codes and e4m3 per-16 scales are
    kept bit-exact (re-laid out only), the per-partition global scale becomes a per-row fp32 multiplier, and the
    activations run as per-row fp8 (the checkpoint's NVFP4 activation quantisation is dropped)."""

    class R9kNvfp4Native(base):

        def process_weights_after_loading(self, layer) -> None:
            from torch.nn.parameter import Parameter
            w, s16 = layer.weight_packed.data, layer.weight_scale.data
            N, Kh = w.shape
            if N % 16 or (2 * Kh) % 16:
                raise ValueError(f"r9700 native NVFP4: unsupported shape N={N} K={2 * Kh}")
            mult = 1.0 / _row_div(layer.weight_global_scale.data, list(layer.logical_widths))
            W = KM.prepare_nvfp4_weights(w[None], s16[None], mult[None].to(w.device))
            for n in ("weight_packed", "weight_global_scale", "input_global_scale", "weight_scale"):
                if hasattr(layer, n):
                    delattr(layer, n)
            layer.weight = Parameter(W.wq, requires_grad=False)
            layer.weight_scale = Parameter(W.ws, requires_grad=False)
            layer.weight_row_mult = Parameter(W.wg, requires_grad=False)
            layer._r9k_nk = (N, 2 * Kh)
            logger.info("r9700: NVFP4 linears on libr9k's native NVFP4 kernel (exact weights, fp8 activations)")

        def apply_weights(self, layer, x, bias=None):
            from .. import ops
            N, Kd = layer._r9k_nk
            out = ops.nvfp4_linear(x, layer.weight, layer.weight_scale, layer.weight_row_mult, N, Kd).to(x.dtype)
            return out + bias if bias is not None else out

    return R9kNvfp4Native


# -------------------------------------------------------------------------------------------------- MoE
MOE_MODE = (os.environ.get("R9K_NVFP4_MOE", "") or "mxfp4").lower()


def prep_native_moe(layer, div13: torch.Tensor, div2: torch.Tensor) -> None:
    """Serve the layer's NVFP4 experts exactly (reference nvfp4.py:185-206): codes and e4m3 scales re-laid out for
    r9k_moe_nvfp4a8 (prepare_nvfp4_weights), the per-shard global divisors (div13 [E, 2I], div2 [E, N]) as per-row
    fp32 multipliers. Leaves w13_weight / w2_weight (int32), *_weight_scale (uint8), *_weight_row_mult (fp32) on the
    layer and drops *_weight_packed."""
    from torch.nn.parameter import Parameter
    for pre, div in (("w13", div13), ("w2", div2)):
        packed = getattr(layer, f"{pre}_weight_packed")
        scale = getattr(layer, f"{pre}_weight_scale")
        E, N, Kh = packed.shape
        assert scale.shape == (E, N, Kh * 2 // 16), (pre, scale.shape, packed.shape)
        assert div.shape == (E, N), (pre, div.shape, (E, N))
        W = KM.prepare_nvfp4_weights(packed.data, scale.data, (1.0 / div.float()).to(packed.device))
        delattr(layer, f"{pre}_weight_packed")
        setattr(layer, f"{pre}_weight", Parameter(W.wq, requires_grad=False))
        setattr(layer, f"{pre}_weight_scale", Parameter(W.ws, requires_grad=False))
        setattr(layer, f"{pre}_weight_row_mult", Parameter(W.wg, requires_grad=False))
    layer._r9k_fold = (False, False)
    layer._r9k_nvfp4 = True


def make_moe_method_cls(mxfp4_method_cls):
    """NVFP4 checkpoint layout at create time (vLLM's CompressedTensorsW4A4Nvfp4MoEMethod.create_weights),
    converted per expert IN PLACE (MXFP4 codes are the same size) to the MXFP4 layout R9kMxfp4MoEMethod consumes."""
    from vllm.model_executor.layers.quantization.compressed_tensors.compressed_tensors_moe.compressed_tensors_moe_w4a4_nvfp4 import (  # noqa: E501
        CompressedTensorsW4A4Nvfp4MoEMethod as _Nv,
    )

    class R9kNvfp4MoEMethod(mxfp4_method_cls):

        def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition, params_dtype,
                           **extra_weight_attrs):
            saved = self.__dict__.get("group_size", None)
            self.group_size = 16
            try:
                _Nv.create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition,
                                   params_dtype, **extra_weight_attrs)
            finally:
                if saved is None:
                    self.__dict__.pop("group_size", None)
                else:
                    self.group_size = saved

        @staticmethod
        def _convert(packed_p, scale_p, row_div):
            E = packed_p.shape[0]
            s_out = torch.empty((E, packed_p.shape[1], packed_p.shape[2] * 2 // 32), dtype=torch.uint8,
                                device=scale_p.device)
            for e in range(E):
                p, s = nvfp4_to_mxfp4(packed_p.data[e], scale_p.data[e], row_div[e])
                packed_p.data[e].copy_(p)
                s_out[e].copy_(s)
            return s_out

        def process_weights_after_loading(self, layer) -> None:
            from torch.nn.parameter import Parameter
            I2 = layer.w13_weight_packed.shape[1]
            g13 = layer.w13_weight_global_scale.data.float()                  # [E, shards]
            div13 = g13.repeat_interleave(I2 // g13.shape[1], dim=1)          # [E, 2I]
            g2 = layer.w2_weight_global_scale.data.float()                    # [E]
            div2 = g2[:, None].expand(-1, layer.w2_weight_packed.shape[1])
            if MOE_MODE == "native":
                prep_native_moe(layer, div13, div2)
                for n in ("w13_weight_global_scale", "w2_weight_global_scale", "w13_input_global_scale",
                          "w2_input_global_scale"):
                    if hasattr(layer, n):
                        delattr(layer, n)
                logger.info("r9700: NVFP4 MoE experts served natively by libr9k (exact checkpoint bits)")
                self._install_kernel(layer)
                return
            s13 = self._convert(layer.w13_weight_packed, layer.w13_weight_scale, div13)
            s2 = self._convert(layer.w2_weight_packed, layer.w2_weight_scale, div2)
            layer.w13_weight_scale = Parameter(s13, requires_grad=False)
            layer.w2_weight_scale = Parameter(s2, requires_grad=False)
            for n in ("w13_weight_global_scale", "w2_weight_global_scale", "w13_input_global_scale",
                      "w2_input_global_scale"):
                if hasattr(layer, n):
                    delattr(layer, n)
            logger.info("r9700: NVFP4 MoE experts converted to MXFP4 at load -> libr9k")
            super().process_weights_after_loading(layer)

    return R9kNvfp4MoEMethod
