"""Python bindings for libr9k's grouped MXFP4 x FP8 MoE GEMM and its companion kernels (gfx950 / CDNA4).

Mirrors r9700_vllm/kernels/moe.py of the reference (same names, argument meaning and RuntimeError on a negative
return code). Weights come from a compressed-tensors ``mxfp4-pack-quantized`` checkpoint: per expert
``weight_packed [N, K/2] uint8`` (element 2i in the low nibble, 2i+1 in the high nibble, e2m1 codes) and
``weight_scale [N, K/32] uint8`` (E8M0). ``prepare_mxfp4_weights`` converts them once at load to the layout the
gfx950 kernels read (see ``permute_fragments`` / ``pack_scales``): one 16x16x128 scaled-MFMA B operand per 1 KB,
plus its 64 exponent bytes. Everything here launches on torch's current stream and never synchronises.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import torch

GROUP = 32
MOE_BLOCK = 16
KTILE = 128          # K per scaled MFMA (16x16x128): one fragment-order weight tile is 16 rows x 128 K = 1 KB

_LIB = None


def _lib_path() -> str:
    return os.environ.get("R9K_LIB") or os.path.join(os.path.dirname(__file__), "libr9k.so")


def lib() -> ctypes.CDLL:
    """The kernel library (lazy, process-global). Raises OSError when libr9k.so is missing: there is no fallback."""
    global _LIB
    if _LIB is None:
        L = ctypes.CDLL(_lib_path())
        i, l = ctypes.c_int, ctypes.c_long
        L.r9k_moe_mxfp4a8.restype = i
        L.r9k_moe_mxfp4a8.argtypes = [l] * 12 + [i] * 9 + [l]
        L.r9k_moe_mxfp4a8_f.restype = i
        L.r9k_moe_mxfp4a8_f.argtypes = [i] + [l] * 12 + [i] * 9 + [l]
        L.r9k_moe_nvfp4a8.restype = i
        L.r9k_moe_nvfp4a8.argtypes = [l] * 12 + [i] * 9 + [l]
        L.r9k_moe_4bit_prefill.restype = i
        L.r9k_moe_4bit_prefill.argtypes = [i] + [l] * 12 + [i] * 6 + [l]
        L.r9k_moe_prefill_bm.restype = i
        L.r9k_moe_prefill_bm.argtypes = [i]
        L.r9k_moe_prefill_bk.restype = i
        L.r9k_moe_prefill_bk.argtypes = [i]
        L.r9k_quant_rows_fp8.restype = i
        L.r9k_quant_rows_fp8.argtypes = [l] * 3 + [i] * 3 + [l]
        L.r9k_silu_mul_quant_fp8.restype = i
        L.r9k_silu_mul_quant_fp8.argtypes = [l] * 3 + [i] * 2 + [l]
        L.r9k_quant_rows_fp8_gate.restype = i
        L.r9k_quant_rows_fp8_gate.argtypes = [l] * 5 + [i] * 4 + [l]
        L.r9k_moe_sum.restype = i
        L.r9k_moe_sum.argtypes = [l] * 3 + [i] * 3 + [l] * 3
        L.r9k_moe_topk.restype = i
        L.r9k_moe_topk.argtypes = [l, i, l, l, i, i, i, i, l]
        L.r9k_moe_topk_quant.restype = i
        L.r9k_moe_topk_quant.argtypes = [l, i, l, l, i, i, i, i, l, l, i, l, l, l]
        L.r9k_moe_align.restype = i
        L.r9k_moe_align.argtypes = [l, i, i, i, l, l, l, l, l, l]
        L.r9k_moe_align_live.restype = i
        L.r9k_moe_align_live.argtypes = [l, i, i, i, l, l, l, l, l, l]
        L.r9k_moe_align_split.restype = i
        L.r9k_moe_align_split.argtypes = [l, i, i, i, i, l, l, l, i, l, l, l, l, l, l]
        L.r9k_moe_align_scratch_ints.restype = l
        L.r9k_moe_align_noalloc.restype = i
        L.r9k_moe_align_noalloc.argtypes = [l, i, i, i, l, l, l, l]
        L.r9k_moe_align_noalloc_max_ints.restype = l
        L.r9k_moe_align_noalloc_max_ints.argtypes = []
        L.r9k_moe_pick_blocks.restype = i
        L.r9k_moe_pick_blocks.argtypes = [l, l, i, i, i, l]
        L.r9k_moe_align_scratch_ints.argtypes = [i, i]
        L.r9k_nvfp4_to_mxfp4.restype = i
        L.r9k_nvfp4_to_mxfp4.argtypes = [l] * 5 + [i] * 2 + [l]
        L.r9k_quantize_mxfp4_search.restype = i
        L.r9k_quantize_mxfp4_search.argtypes = [l] * 3 + [i] * 2 + [l]
        L.r9k_fold_supported.restype = i
        L.r9k_moe_down_sum.restype = i
        L.r9k_dense_mxfp4_qa.restype = i
        L.r9k_dense_mxfp4_qa.argtypes = [l] * 6 + [i] * 3 + [l]
        L.r9k_dense_mxfp4_a8.restype = i
        L.r9k_dense_nvfp4_qa.restype = i
        L.r9k_dense_nvfp4_qa.argtypes = [l] * 7 + [i] * 3 + [l]
        L.r9k_dense_mxfp4_a8.argtypes = [l] * 8 + [i] * 3 + [l]
        L.r9k_moe_down_sum.argtypes = [l] * 10 + [i] * 5 + [l]
        L.r9k_moe_stream.restype = i
        L.r9k_moe_stream.argtypes = [i] + [l] * 11 + [i] * 6 + [l]
        L.r9k_moe_stream_layer.restype = i
        L.r9k_moe_stream_layer.argtypes = [l] * 13 + [i] * 6 + [l]
        assert L.r9k_moe_block() == MOE_BLOCK
        _LIB = L
    return _LIB


def fold_supported() -> bool:
    L = lib()
    return hasattr(L, "r9k_fold_supported") and bool(L.r9k_fold_supported())


def atiled_supported() -> bool:
    """The gfx1201 fragment-tiled-activation prefill kernel has no gfx950 counterpart here."""
    return hasattr(lib(), "r9k_moe_4bit_prefill_at")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _check(rc: int, what: str) -> None:
    if rc:
        raise RuntimeError(f"{what} failed ({rc})")


@dataclass
class Mxfp4Experts:
    wq: torch.Tensor    # [E, N/16 * K/16 * 32] int32: fragment order (permute_fragments)
    wsr: torch.Tensor   # [E, K/32 + 1, N] uint8: exponents in fragment order (pack_scales), last row = per-row max
    N: int
    K: int
    fold: bool = False  # folded-exponent kernels: not used on gfx950 (the scaled MFMA applies the exponents)

    @property
    def estride(self) -> int:
        return (self.K // GROUP + 1) * self.N


NV_KT = 128            # K per NVFP4 weight tile (8 groups of 16)


@dataclass
class Nvfp4Experts:
    """Native NVFP4 experts (e2m1 codes, e4m3 scale per 16, fp32 multiplier per row) in the gfx950 kernel layout
    (prepare_nvfp4_weights): wq int32 [E, N * ceil(K/128) * 16], ws uint8 [E, ceil(K/128) * 8, N] (the reference's
    [E, K/16, N] size when K % 128 == 0; the bytes are in the kernel's order), wg fp32 [E, N]."""
    wq: torch.Tensor
    ws: torch.Tensor
    wg: torch.Tensor
    N: int
    K: int

    @property
    def ws_estride(self) -> int:
        return self.N * ((self.K + NV_KT - 1) // NV_KT) * 8


def prepare_nvfp4_weights(packed: torch.Tensor, scale16: torch.Tensor, row_mult: torch.Tensor) -> Nvfp4Experts:
    """packed [E, N, K/2] u8, scale16 [E, N, K/16] e4m3, row_mult [E, N] fp32 -> Nvfp4Experts, the checkpoint bits
    kept (reference: kernels/moe.py:86-104; the layout is this kernel's, csrc/r9k_moe_nvfp4.hip).

    Codes: the MXFP4 fragment order over K-tiles of 128 -- column tile nt (16 rows) holds ceil(K/128) K-tiles of 1 KB,
    lane l = g*16 + c holding the 16 checkpoint bytes W[nt*16 + c, kt*64 + 16g .. +16] at l*16. Scales: per column
    tile and K-tile 128 bytes, lane l's 2 bytes at l*2 the scales of groups kt*8 + 2g, kt*8 + 2g + 1 of row nt*16 + c.
    A partial last K-tile is zero-padded (codes and scales)."""
    E, N, Kh = packed.shape
    K = Kh * 2
    assert N % 16 == 0 and K % 16 == 0, (N, K)
    assert scale16.shape == (E, N, K // 16), (scale16.shape, (E, N, K // 16))
    nkt = (K + NV_KT - 1) // NV_KT
    p = packed.view(torch.uint8)
    sc = scale16.view(torch.uint8)
    if nkt * 64 != Kh:
        p = torch.nn.functional.pad(p, (0, nkt * 64 - Kh))
        sc = torch.nn.functional.pad(sc, (0, nkt * 8 - K // 16))
    NT = N // 16
    wq = p.reshape(E, NT, 16, nkt, 4, 16).permute(0, 1, 3, 4, 2, 5).contiguous().reshape(E, -1)
    ws = sc.reshape(E, NT, 16, nkt, 4, 2).permute(0, 1, 3, 4, 2, 5).contiguous().reshape(E, nkt * 8, N)
    return Nvfp4Experts(wq.view(torch.int32), ws, row_mult.float().reshape(E, N).contiguous(), N, K)


def permute_fragments(packed: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """[E, N, K/2] uint8 checkpoint order -> [E, N*K/8] int32 fragment order (same bytes, same size); written into
    `out` (any tensor of E * N * K/2 bytes, not overlapping `packed`) when given.

    Column tile nt (16 rows) occupies 8*K bytes. Its K-tile kt (128 K) is 1 KB at kt*1024: lane l = g*16 + r of the
    V_MFMA_SCALE_F32_16X16X128_F8F6F4 B operand holds row nt*16 + r, K elements kt*128 + g*32 .. +32, i.e. the 16
    checkpoint bytes W[nt*16 + r, kt*64 + g*16 .. +16], at l*16. A last partial K-tile (K % 128 = 32*G) keeps only
    its G groups (lanes l < 16*G), 256*G bytes."""
    E, N, Kh = packed.shape
    K = Kh * 2
    assert N % 16 == 0 and K % GROUP == 0, (N, K)
    nt, nkf, G = N // 16, K // KTILE, (K % KTILE) // GROUP
    if out is None:
        out = torch.empty((E, N * Kh // 4), dtype=torch.int32, device=packed.device)
    dst = out.view(torch.uint8).reshape(E, nt, 8 * K)
    w = packed.reshape(E, nt, 16, Kh)
    if nkf:
        f = w[..., : nkf * 64].reshape(E, nt, 16, nkf, 4, 16).permute(0, 1, 3, 4, 2, 5)   # [E, nt, kt, g, r, 16]
        dst[..., : nkf * 1024].view(E, nt, nkf, 4, 16, 16).copy_(f)
    if G:
        t = w[..., nkf * 64:].reshape(E, nt, 16, G, 16).permute(0, 1, 3, 2, 4)              # [E, nt, g, r, 16]
        dst[..., nkf * 1024:].view(E, nt, G, 16, 16).copy_(t)
    return out.view(torch.uint8).reshape(E, -1).view(torch.int32)


def unpermute_fragments(wq: torch.Tensor, N: int, K: int) -> torch.Tensor:
    """Inverse of permute_fragments: [E, N*K/8] int32 -> [E, N, K/2] uint8."""
    E = wq.shape[0]
    nt, nkf, G = N // 16, K // KTILE, (K % KTILE) // GROUP
    b = wq.contiguous().view(torch.uint8).reshape(E, nt, 8 * K)
    parts = []
    if nkf:
        f = b[..., : nkf * 1024].reshape(E, nt, nkf, 4, 16, 16).permute(0, 1, 4, 2, 3, 5)  # [E, nt, r, kt, g, 16]
        parts.append(f.reshape(E, nt, 16, nkf * 64))
    if G:
        t = b[..., nkf * 1024:].reshape(E, nt, G, 16, 16).permute(0, 1, 3, 2, 4)            # [E, nt, r, g, 16]
        parts.append(t.reshape(E, nt, 16, G * 16))
    out = parts[0] if len(parts) == 1 else torch.cat(parts, dim=3)
    return out.reshape(E, N, K // 2).contiguous()


def prepare_mxfp4_weights(packed: torch.Tensor, scale: torch.Tensor) -> Mxfp4Experts:
    E, N, Kh = packed.shape
    K = Kh * 2
    assert N % 16 == 0 and K % GROUP == 0, (N, K)
    assert scale.shape == (E, N, K // GROUP), (scale.shape, (E, N, K // GROUP))
    return Mxfp4Experts(permute_fragments(packed.view(torch.uint8)), pack_scales(scale), N, K)


def pack_scales(scale: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """[E, N, K/32] E8M0 -> [E, K/32 + 1, N] uint8 (into `out` when given): the first (K/32)*N bytes of each expert
    are the exponents in the kernels' fragment order, the last N bytes the per-row maximum exponent.

    Column tile nt owns 16*K/32 bytes at nt*16*K/32. K-tile kt (128 K, four 32-blocks) is 64 bytes at kt*64: lane
    l = g*16 + r has the exponent of row r, block 4*kt + g at byte l -- the scale operand of one MFMA tile, one byte
    a lane. A partial last K-tile (K % 128 = 32*G) keeps its 16*G bytes."""
    scale = scale.view(torch.uint8)
    E, N, KB = scale.shape
    nt, nkf, G = N // 16, KB // 4, KB % 4
    if out is None:
        out = torch.empty((E, KB + 1, N), dtype=torch.uint8, device=scale.device)
    body = out.view(E, -1)[:, : KB * N].view(E, nt, 16 * KB)
    s = scale.reshape(E, nt, 16, KB)                                                     # [E, nt, r, kb]
    if nkf:
        body[..., : nkf * 64].view(E, nt, nkf, 4, 16).copy_(
            s[..., : nkf * 4].reshape(E, nt, 16, nkf, 4).permute(0, 1, 3, 4, 2))         # [E, nt, kt, g, r]
    if G:
        body[..., nkf * 64:].view(E, nt, G, 16).copy_(s[..., nkf * 4:].permute(0, 1, 3, 2))   # [E, nt, g, r]
    out[:, KB] = scale.max(dim=2).values
    return out


def unpack_scales(wsr: torch.Tensor) -> torch.Tensor:
    """Inverse of pack_scales: [E, K/32 + 1, N] -> [E, N, K/32] uint8 exponents."""
    E, KB1, N = wsr.shape
    KB = KB1 - 1
    nt, nkf, G = N // 16, KB // 4, KB % 4
    body = wsr.reshape(E, -1)[:, : KB * N].reshape(E, nt, 16 * KB)
    parts = []
    if nkf:
        q = body[..., : nkf * 64].reshape(E, nt, nkf, 4, 16).permute(0, 1, 4, 2, 3)         # [E, nt, r, kt, g]
        parts.append(q.reshape(E, nt, 16, nkf * 4))
    if G:
        parts.append(body[..., nkf * 64:].reshape(E, nt, G, 16).permute(0, 1, 3, 2))        # [E, nt, r, g]
    out = parts[0] if len(parts) == 1 else torch.cat(parts, dim=3)
    return out.reshape(E, N, KB).contiguous()


# ------------------------------------------------------------------------------------------ activations
def quant_rows_fp8(x: torch.Tensor, tiled: bool = False):
    """bf16 [M, K] -> (e4m3fn [M, K], fp32 [M]) with a per-row dynamic scale (amax / 448)."""
    assert x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1
    if tiled:
        raise RuntimeError("quant_rows_fp8(tiled=True): the fragment-tiled layout is a gfx1201 A-tiled-kernel format")
    M, K = x.shape
    s = torch.empty((M,), dtype=torch.float32, device=x.device)
    q = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=x.device)
    if M == 0:
        return q, s
    rc = lib().r9k_quant_rows_fp8(x.data_ptr(), q.data_ptr(), s.data_ptr(), M, K, x.stride(0), _stream())
    if rc:
        raise RuntimeError(f"r9k_quant_rows_fp8 failed ({rc}) M={M} K={K}")
    return q, s


def quant_rows_fp8_gate(x: torch.Tensor, wg: torch.Tensor, tiled: bool = False):
    """quant_rows_fp8 plus the shared expert's gate in the same launch: (q, s, g) with g [M] fp32 =
    bf16(sigmoid(bf16(x @ wg)))."""
    assert x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1
    assert wg.dtype == torch.bfloat16 and wg.is_contiguous() and wg.numel() == x.shape[1]
    if tiled:
        raise RuntimeError("quant_rows_fp8_gate(tiled=True): not available on gfx950")
    M, K = x.shape
    s = torch.empty((M,), dtype=torch.float32, device=x.device)
    g = torch.empty((M,), dtype=torch.float32, device=x.device)
    q = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=x.device)
    if M == 0:
        return q, s, g
    rc = lib().r9k_quant_rows_fp8_gate(x.data_ptr(), q.data_ptr(), s.data_ptr(), wg.data_ptr(), g.data_ptr(), M, K,
                                       x.stride(0), 0, _stream())
    if rc:
        raise RuntimeError(f"r9k_quant_rows_fp8_gate failed ({rc}) M={M} K={K}")
    return q, s, g


def silu_mul_quant_fp8(gu: torch.Tensor):
    """bf16 [M, 2I] (gate | up) -> (e4m3fn [M, I], fp32 [M]): silu(gate) * up with a per-row dynamic scale."""
    assert gu.dtype == torch.bfloat16 and gu.is_contiguous() and gu.shape[1] % 2 == 0
    M, I2 = gu.shape
    q = torch.empty((M, I2 // 2), dtype=torch.float8_e4m3fn, device=gu.device)
    s = torch.empty((M,), dtype=torch.float32, device=gu.device)
    if M == 0:
        return q, s
    rc = lib().r9k_silu_mul_quant_fp8(gu.data_ptr(), q.data_ptr(), s.data_ptr(), M, I2 // 2, _stream())
    if rc:
        raise RuntimeError(f"r9k_silu_mul_quant_fp8 failed ({rc})")
    return q, s


# ------------------------------------------------------------------------------------------------ GEMMs
# Prefill tile table: cfg -> (rows per routing block BM, columns BN). The kernel is the source of truth for BM
# (prefill_block() asks it); the cfg indices keep the reference's BM per index.
PREFILL_TILES = {0: (256, 64), 1: (256, 128), 2: (128, 128), 3: (128, 64), 4: (128, 64), 5: (256, 32),
                 6: (64, 64), 7: (256, 128), 8: (256, 128), 9: (256, 128), 10: (128, 128), 11: (64, 64),
                 12: (256, 128), 13: (128, 128), 14: (64, 64), 15: (64, 128), 16: (256, 128), 17: (64, 128),
                 18: (64, 64), 19: (64, 128)}
PREFILL_MIN_M = int(os.environ.get("R9K_PREFILL_MIN_M", "128"))
PREFILL_DEFAULT = int(os.environ.get("R9K_PREFILL_CFG", "12"))
PREFILL_DEFAULT_SMALL = int(os.environ.get("R9K_PREFILL_CFG_SMALL", "10"))


def prefill_block(cfg: int) -> int:
    """Rows per routing block (moe_align_block_size block) of prefill tile `cfg`."""
    bm = lib().r9k_moe_prefill_bm(cfg)
    if bm <= 0:
        raise ValueError(f"unknown prefill cfg {cfg}")
    return bm


def prefill_bk(cfg: int) -> int:
    """K granularity of prefill tile `cfg`: the kernel needs K % BK == 0."""
    bk = lib().r9k_moe_prefill_bk(cfg)
    if bk <= 0:
        raise ValueError(f"unknown prefill cfg {cfg}")
    return bk


def is_prefill_cfg(cfg) -> bool:
    return bool(cfg) and cfg[0] == "P"


def is_atiled_cfg(cfg) -> bool:
    return bool(cfg) and cfg[0] == "A"


def pick_atiled(N: int, K: int, M: int, fold: bool = True):
    """The gfx1201 A-tiled kernel is not part of the gfx950 library: never selected."""
    return None


def moe_gemm(a_q: torch.Tensor, a_s: torch.Tensor, w: Mxfp4Experts, out: torch.Tensor,
             sorted_ids: torch.Tensor, expert_ids: torch.Tensor, ntpp: torch.Tensor, numel: int,
             a_row_div: int, topk_w: torch.Tensor | None = None, WV: int = 0, SK: int = 0, NPW: int = 0,
             num_experts: int | None = None, MT: int = 1, ldsa: bool = False, prefill: int | None = None,
             a_tiled: bool = False, fuse: int = 0):
    """out[r, :] = dequant(a_q[r // a_row_div]) @ W[expert(r)]^T (* topk_w[r]) for every routed flat row r.

    sorted_ids/expert_ids must come from an align with block_size 16*MT (or prefill_block(prefill)). WV/SK/NPW: the
    decode kernel's gfx950 launch shape (K-tiles per load batch, waves splitting K, column tiles per wave: pick_cfg's
    tuned values, passed with MT_SHAPE set), all 0 for the kernel's own choice; ldsa is a gfx1201 knob, accepted and
    not used.
    The grid covers at most ceil(numel/BLK) + min(numel, E) blocks -- the most an align can fill with numel routed
    rows over E experts -- so the launch stays graph-capturable."""
    E = num_experts if num_experts is not None else w.wq.shape[0]
    if fuse:
        # fuse 1: gate_up with silu(g)*u in the epilogue -> out fp32 [numel, N/2]; fuse 2: down with the fp32 A rows
        # quantised per row on load (a_s unused). Decode routing blocks (MT == 1), MXFP4 experts
        # (reference contract: kernels/moe.py:416-434).
        if fuse not in (1, 2):
            raise RuntimeError(f"moe_gemm: fuse={fuse} is not a fused variant (1 gate_up+act, 2 down+quant)")
        assert isinstance(w, Mxfp4Experts) and MT == 1 and prefill is None and not a_tiled
        assert a_q.shape[1] == w.K and a_q.is_contiguous() and out.is_contiguous()
        assert (out.dtype == torch.float32 and out.shape[1] == w.N // 2 if fuse == 1
                else out.dtype == torch.bfloat16 and out.shape[1] == w.N)
        if fuse == 2:
            assert a_q.dtype == torch.float32 and a_row_div == 1
        else:
            assert a_s is not None and a_s.dtype == torch.float32
        if topk_w is not None:
            assert topk_w.dtype == torch.float32 and topk_w.is_contiguous()
        max_blocks = min(expert_ids.numel(), (numel + MOE_BLOCK - 1) // MOE_BLOCK + min(numel, E))
        rc = lib().r9k_moe_mxfp4a8_f(
            fuse, a_q.data_ptr(), a_s.data_ptr() if a_s is not None else 0, w.wq.data_ptr(), w.wsr.data_ptr(),
            w.wsr.data_ptr() + (w.K // GROUP) * w.N, out.data_ptr(), sorted_ids.data_ptr(), expert_ids.data_ptr(),
            ntpp.data_ptr(), topk_w.data_ptr() if topk_w is not None else 0, w.estride, w.estride, max_blocks,
            numel, a_row_div, w.K, w.N, WV, SK, NPW, 1 | (16 if w.fold else 0), _stream())
        if rc:
            raise RuntimeError(f"r9k_moe_mxfp4a8_f failed ({rc}) fuse={fuse} N={w.N} K={w.K}")
        return out
    if a_tiled:
        raise RuntimeError("moe_gemm(a_tiled=True) is a gfx1201 kernel format")
    if isinstance(w, Nvfp4Experts):
        # decode family (16*MT-row blocks; reference entry kernels/r9k_moe_mxfp4a8.hip:641-647) or the prefill entry's
        # nv = 1 tile kernel (prefill_block(prefill) = 128 or 256 rows; :1205-1230)
        assert out.dtype == torch.bfloat16 and out.shape[1] == w.N and a_q.shape[1] == w.K and out.is_contiguous()
        assert a_q.is_contiguous() and a_s.dtype == torch.float32
        if topk_w is not None:
            assert topk_w.dtype == torch.float32 and topk_w.is_contiguous()
        if prefill is not None:
            blk = prefill_block(prefill)
            max_blocks = min(expert_ids.numel(), (numel + blk - 1) // blk + min(numel, E))
            rc = lib().r9k_moe_4bit_prefill(
                1, a_q.data_ptr(), a_s.data_ptr(), w.wq.data_ptr(), w.ws.data_ptr(), w.wg.data_ptr(), out.data_ptr(),
                sorted_ids.data_ptr(), expert_ids.data_ptr(), ntpp.data_ptr(),
                topk_w.data_ptr() if topk_w is not None else 0, w.ws_estride, w.N, max_blocks, numel, a_row_div,
                w.K, w.N, prefill, _stream())
            if rc:
                raise RuntimeError(f"r9k_moe_4bit_prefill(nv=1) failed ({rc}) N={w.N} K={w.K} cfg={prefill}")
            return out
        blk = MOE_BLOCK * MT
        max_blocks = min(expert_ids.numel(), (numel + blk - 1) // blk + min(numel, E))
        rc = lib().r9k_moe_nvfp4a8(
            a_q.data_ptr(), a_s.data_ptr(), w.wq.data_ptr(), w.ws.data_ptr(), w.wg.data_ptr(), out.data_ptr(),
            sorted_ids.data_ptr(), expert_ids.data_ptr(), ntpp.data_ptr(),
            topk_w.data_ptr() if topk_w is not None else 0, w.ws_estride, w.N, max_blocks, numel, a_row_div, w.K,
            w.N, WV, 1, NPW, MT, _stream())
        if rc:
            raise RuntimeError(f"r9k_moe_nvfp4a8 failed ({rc}) N={w.N} K={w.K} MT={MT}")
        return out
    assert out.dtype == torch.bfloat16 and out.shape[1] == w.N and a_q.shape[1] == w.K and out.is_contiguous()
    assert a_q.is_contiguous() and a_s.dtype == torch.float32
    if topk_w is not None:
        assert topk_w.dtype == torch.float32 and topk_w.is_contiguous()
    tw = topk_w.data_ptr() if topk_w is not None else 0
    wsr = w.wsr
    if prefill is not None:
        blk = prefill_block(prefill)
        max_blocks = min(expert_ids.numel(), (numel + blk - 1) // blk + min(numel, E))
        rc = lib().r9k_moe_4bit_prefill(
            2 if w.fold else 0, a_q.data_ptr(), a_s.data_ptr(), w.wq.data_ptr(), wsr.data_ptr(),
            wsr.data_ptr() + (w.K // GROUP) * w.N, out.data_ptr(), sorted_ids.data_ptr(), expert_ids.data_ptr(),
            ntpp.data_ptr(), tw, w.estride, w.estride, max_blocks, numel, a_row_div, w.K, w.N, prefill, _stream())
        if rc:
            raise RuntimeError(f"r9k_moe_4bit_prefill failed ({rc}) N={w.N} K={w.K} cfg={prefill}")
        return out
    blk = MOE_BLOCK * MT
    max_blocks = min(expert_ids.numel(), (numel + blk - 1) // blk + min(numel, E))
    rc = lib().r9k_moe_mxfp4a8(
        a_q.data_ptr(), a_s.data_ptr(), w.wq.data_ptr(), wsr.data_ptr(), wsr.data_ptr() + (w.K // GROUP) * w.N,
        out.data_ptr(), sorted_ids.data_ptr(), expert_ids.data_ptr(), ntpp.data_ptr(), tw,
        w.estride, w.estride, max_blocks, numel, a_row_div, w.K, w.N, WV, SK, NPW,
        MT | (8 if ldsa and MT > 1 else 0) | (MT_SHAPE if (WV or SK or NPW) else 0), _stream())
    if rc:
        raise RuntimeError(f"r9k_moe_mxfp4a8 failed ({rc}) N={w.N} K={w.K} MT={MT}")
    return out


def pick_cfg(N: int, K: int, group: int = GROUP, M: int | None = None, kind: str | None = None,
             fold: bool = False) -> tuple:
    """("P", cfg) for the prefill entry at M >= PREFILL_MIN_M, else the decode kernel's (WV, SK, NPW) launch shape on
    this device for a dense [M, K] x [N, K]^T product: the gfx950 table's entry (kernels/tuned.json, written by
    kernels/tune.py's sweep; WV = K-tiles per load batch, SK = waves splitting K, NPW = column tiles per wave) for the
    nearest measured M, or (0, 0, 0) -- the kernel's own choice -- for a shape the table does not hold.
    R9K_TUNED=0 ignores the table."""
    if kind and M:
        if M >= PREFILL_MIN_M and K % prefill_bk(PREFILL_DEFAULT) == 0:
            return ("P", PREFILL_DEFAULT if M >= 512 else PREFILL_DEFAULT_SMALL)
    from . import tuned
    cfg = tuned.lookup(kind or "mxfp4", N, K, M or 1)
    return legal_cfg(cfg, N, K, group, decode_mt(M or 1)) if cfg else (0, 0, 0)


def decode_mt(M: int) -> int:
    """M tiles per routing block of a dense decode GEMM over identity tables (ops.mxfp4_gemm_q): 16-row blocks up to
    31 rows, 32 up to 63, then 64."""
    return 4 if M >= 64 else (2 if M >= 32 else 1)


# r9k_moe_mxfp4a8's MT bit that marks (WV, SK, NPW) as this library's launch shape; without it the kernel picks the
# shape and the three are ignored, as the reference's gfx1201 knobs are.
MT_SHAPE = 32

# Launch shapes the decode kernel is built for (r9k_moe_gemm.hip): each of WV (K-tiles per load batch), SK (waves
# splitting K) and NPW (column tiles per wave) in {1, 2, 4}.
BUILT_KNOBS = (1, 2, 4)


def legal_cfg(cfg: tuple, N: int, K: int, group: int = GROUP, MT: int = 1) -> tuple:
    """cfg's (WV, SK, NPW) when the decode kernel is built for it at MT M-tiles a block (NPW 4 only below MT 4) and
    the shape can use it (SK waves each hold at least one of the K / 128 K-tiles, NPW column tiles fit in N / 16),
    else (0, 0, 0): the kernel's own choice."""
    WV, SK, NPW = (int(v) for v in cfg[:3])
    nkt, nt = -(-K // 128), N // 16
    if (all(v in BUILT_KNOBS for v in (WV, SK, NPW)) and SK <= nkt and NPW <= max(1, nt) and K % group == 0
            and not (MT >= 4 and NPW > 2)):
        return WV, SK, NPW
    return 0, 0, 0


MOE_MT = int(os.environ.get("R9K_MOE_MT", "0"))


def pick_mt(numel: int, num_experts: int) -> int:
    """M tiles per routing block from the host-known row count: rows per touched expert >= 32 -> 4, >= 16 -> 2
    (R9K_MOE_MT = 1, 2 or 4 fixes it)."""
    if MOE_MT in (1, 2, 4):
        return MOE_MT
    per = numel / max(1, min(num_experts, numel))
    return 4 if per >= 32 else (2 if per >= 16 else 1)


MOE_PREFILL_CFG = int(os.environ.get("R9K_MOE_PREFILL_CFG", "17"))
MOE_PREFILL_CFG_GATE_UP = int(os.environ.get("R9K_MOE_PREFILL_CFG1", "17"))


# 256-row blocks win from ~24 average rows per expert on MI355X (measured at E = 288 / 384, hidden 2048 / 4096,
# uniform and Zipf(1.1) routing: 2.1x at 114 rows, even at 28-43; 6% behind at 21 uniform, ahead from 8 under Zipf)
PREFILL_MOE_ROWS = int(os.environ.get("R9K_PREFILL_MOE_ROWS", "24"))
# native NVFP4 dense linears: 128-row tiles of the nv = 1 prefill kernel from this many rows (cfg 2: 128-row blocks)
NV_PREFILL_MIN_M = int(os.environ.get("R9K_NVFP4_PREFILL_MIN_M", "128"))
NV_PREFILL_CFG = 2
MOE_PREFILL_CFG_BIG = int(os.environ.get("R9K_MOE_PREFILL_CFG_BIG", "12"))


def pick_moe_prefill_block(numel: int, num_experts: int, K1: int, K2: int):
    """(cfg, rows per routing block) for a routed layer whose touched experts average >= PREFILL_MOE_ROWS rows: the
    256-row LDS-tiled kernel on the 32x32x64 scaled MFMA (both GEMMs' K multiples of 128), one block ~ one expert so
    each weight tile streams from HBM once. None keeps the 16*MT-row decode-family blocks."""
    per = numel / max(1, min(num_experts, numel))
    if MOE_PREFILL_CFG_BIG < 0 or per < PREFILL_MOE_ROWS or K1 % 128 or K2 % 128:
        return None
    return MOE_PREFILL_CFG_BIG, prefill_block(MOE_PREFILL_CFG_BIG)


# From this many routed rows, a step the host would run on decode blocks gets its tables in both layouts and the
# device keeps the 256-row one when the touched experts average >= DEVICE_MIN_ROWS rows (skewed routing: the host
# only sees the average over all experts). 0 turns it off. The per-touched-expert threshold sits below the host's
# all-expert one: config 5 under Zipf(1.1) at T = 256 (23.8 rows per touched expert) runs 17% faster on 256-row
# blocks, uniform routing at ~21 rows 6% slower.
DEVICE_BLOCKS_MIN = int(os.environ.get("R9K_MOE_DEVICE_BLOCKS_MIN", "1024"))
DEVICE_MIN_ROWS = int(os.environ.get("R9K_MOE_DEVICE_MIN_ROWS", "22"))


def big_block_cfg(K1: int, K2: int):
    """(cfg, rows per block) of the 256-row prefill layout when both GEMMs can take it, else None."""
    if MOE_PREFILL_CFG_BIG < 0 or K1 % 128 or K2 % 128:
        return None
    return MOE_PREFILL_CFG_BIG, prefill_block(MOE_PREFILL_CFG_BIG)


def pick_blocks(ntpp_small: torch.Tensor, ntpp_big: torch.Tensor, numel: int, big_blk: int,
                min_rows: int | None = None) -> None:
    """Keep one of the two table layouts on the device (r9k_moe_pick_blocks): the other's ntpp becomes 0."""
    rc = lib().r9k_moe_pick_blocks(ntpp_small.data_ptr(), ntpp_big.data_ptr(), numel, big_blk,
                                   DEVICE_MIN_ROWS if min_rows is None else min_rows, _stream())
    if rc:
        raise RuntimeError(f"r9k_moe_pick_blocks failed ({rc})")


def pick_moe_prefill(MT: int, K_down: int, gate_up: bool = False) -> int | None:
    """Prefill tile for the routed-MoE GEMMs of a step whose routing block is 16*MT rows (None: the decode kernel).
    Both GEMMs must share the block size, so one align table serves both."""
    cfg = MOE_PREFILL_CFG_GATE_UP if gate_up else MOE_PREFILL_CFG
    if cfg < 0 or 16 * MT != prefill_block(cfg) or K_down % prefill_bk(cfg):
        return None
    return cfg


# At decode widths the SiLU + re-quant, the down GEMM and the top-k sum run as one token-major launch
# (r9k_moe_down_sum), which saves two launches but reads an expert's down weights once per routed row instead of
# once per routing block. It is used while the routed rows' down weight bytes (numel * N2 * K2 / 2, re-reads
# included) stay within DOWN_SUM_MAX_BYTES. Measured on MI355X: config 2 (E=288, 0.5 MB of down weights an expert)
# T = 1 / 8 / 16 / 32: 21.2 -> 14.4, 35.3 -> 27.8, 47.4 -> 40.5, 62.0 -> 59.5 us a layer, T = 64 81.0 -> 90.6 (not
# taken); config 5 (4 MB an expert, Zipf routing) T = 1 / 2: 36.7 -> 30.0, 43.7 -> 39.5, T = 4 even, T = 8 68.9 ->
# 84.3 (not taken).
DOWN_SUM_MAX_BYTES = int(os.environ.get("R9K_MOE_DOWN_SUM_MAX_BYTES", str(128 << 20)))


def down_sum_fits(numel: int, N2: int, K2: int) -> bool:
    """Whether a decode step of `numel` routed rows takes the token-major tail (r9k_moe_down_sum)."""
    return numel * N2 * K2 // 2 <= DOWN_SUM_MAX_BYTES


def moe_down_sum(gate_up: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor, w: Mxfp4Experts,
                 out: torch.Tensor, shared: torch.Tensor | None = None) -> bool:
    """out[t] = sum_j bf16(silu-quant(gate_up[t*k+j]) @ W2[ids[t, j]]^T * (as * topk_w[t*k+j])) (+ shared[t]) in one
    launch (r9k_moe_down_sum): the three-launch tail's values (bit for bit when K2 < 1024). gate_up bf16 [T*k, 2*K2]
    contiguous; topk_ids int32 [T, k]; topk_w fp32 [T*k]. False when the shape is not served (nothing launched:
    run silu_mul_quant_fp8, the down moe_gemm and moe_sum)."""
    T, k = topk_ids.shape
    assert gate_up.is_contiguous() and gate_up.dtype == torch.bfloat16 and gate_up.shape == (T * k, 2 * w.K)
    assert topk_ids.dtype == torch.int32 and topk_ids.is_contiguous()
    assert topk_w.dtype == torch.float32 and topk_w.is_contiguous() and topk_w.numel() == T * k
    assert out.dtype == torch.bfloat16 and out.shape == (T, w.N) and out.stride(1) == 1
    if shared is not None:
        assert shared.dtype == torch.bfloat16 and shared.shape == (T, w.N) and shared.stride(1) == 1
    rc = lib().r9k_moe_down_sum(gate_up.data_ptr(), topk_ids.data_ptr(), topk_w.data_ptr(), w.wq.data_ptr(),
                                w.wsr.data_ptr(), w.estride, shared.data_ptr() if shared is not None else 0,
                                shared.stride(0) if shared is not None else 0, out.data_ptr(), out.stride(0), T, k,
                                w.wq.shape[0], w.K, w.N, _stream())
    if rc == 2:
        return False
    if rc:
        raise RuntimeError(f"r9k_moe_down_sum failed ({rc}) T={T} topk={k} N={w.N} K={w.K}")
    return True


# Decode steps whose routing touches at least STREAM_MIN_BLOCKS experts and at most one 16-row block per CU
# (expected_blocks) run gate_up, the SiLU + fp8 quant and down of each routing block in one workgroup
# (r9k_moe_stream_layer); with fewer blocks a block stream would leave CUs idle, with more some CUs would run two
# blocks while the rest wait. R9K_STREAM=0 turns it off.
STREAM_MIN_BLOCKS = int(os.environ.get("R9K_STREAM_MIN_BLOCKS", "160"))
STREAM = os.environ.get("R9K_STREAM", "1") == "1"
_CUS: dict = {}


def device_cus(device=None) -> int:
    """Compute units of the current (or given) device."""
    idx = torch.cuda.current_device() if device is None else torch.device(device).index
    if idx not in _CUS:
        _CUS[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _CUS[idx]


def expected_blocks(numel: int, num_experts: int, topk: int) -> float:
    """Expected 16-row routing blocks of a step of numel / topk tokens under uniform routing: the expected number of
    distinct experts, E * (1 - (1 - topk / E)^T) (each expert's ~numel / E rows fit one block at decode widths)."""
    T = numel / max(1, topk)
    return num_experts * (1.0 - (1.0 - min(topk, num_experts) / num_experts) ** T)


def moe_stream(a_q: torch.Tensor, a_s: torch.Tensor, w: Mxfp4Experts, out: torch.Tensor, sorted_ids: torch.Tensor,
               expert_ids: torch.Tensor, ntpp: torch.Tensor, numel: int, a_row_div: int,
               topk_w: torch.Tensor | None = None, num_experts: int | None = None,
               out_scale: torch.Tensor | None = None, blocks_hint: int | None = None) -> bool:
    """The grouped GEMM over 16-row routing blocks as a block stream (r9k_moe_stream). out_scale None: out bf16
    [numel, N] = moe_gemm's values (its single-wave launch, bit for bit). out_scale given: the gate_up product with
    SiLU-gating and the per-row fp8 quant in the epilogue, out e4m3 codes [numel, N/2] and out_scale fp32 [numel] =
    silu_mul_quant_fp8 of moe_gemm's bf16 output, bit for bit. blocks_hint: the live blocks expected (sets how many
    workgroups split a block's columns; default min(E, numel)). False when the shape is not served (nothing
    launched)."""
    E = num_experts if num_experts is not None else w.wq.shape[0]
    epi = 1 if out_scale is not None else 0
    assert a_q.is_contiguous() and a_q.shape[1] == w.K and a_s.dtype == torch.float32 and out.is_contiguous()
    if epi:
        assert topk_w is None and out.dtype == torch.float8_e4m3fn and out.shape == (numel, w.N // 2)
        assert out_scale.dtype == torch.float32 and out_scale.numel() >= numel
    else:
        assert out.dtype == torch.bfloat16 and out.shape[1] == w.N
        if topk_w is not None:
            assert topk_w.dtype == torch.float32 and topk_w.is_contiguous()
    max_blocks = min(expert_ids.numel(), (numel + MOE_BLOCK - 1) // MOE_BLOCK + min(numel, E))
    rc = lib().r9k_moe_stream(epi, a_q.data_ptr(), a_s.data_ptr(), w.wq.data_ptr(), w.wsr.data_ptr(),
                              out.data_ptr(), out_scale.data_ptr() if epi else 0, sorted_ids.data_ptr(),
                              expert_ids.data_ptr(), ntpp.data_ptr(), topk_w.data_ptr() if topk_w is not None else 0,
                              w.estride, max_blocks, numel, a_row_div, w.K, w.N,
                              blocks_hint if blocks_hint else min(E, numel), _stream())
    if rc == 2:
        return False
    if rc:
        raise RuntimeError(f"r9k_moe_stream failed ({rc}) epi={epi} N={w.N} K={w.K}")
    return True


def moe_stream_layer(a_q: torch.Tensor, a_s: torch.Tensor, w1: Mxfp4Experts, w2: Mxfp4Experts, down: torch.Tensor,
                     sorted_ids: torch.Tensor, expert_ids: torch.Tensor, ntpp: torch.Tensor, numel: int, topk: int,
                     topk_w: torch.Tensor, num_experts: int | None = None) -> bool:
    """gate_up, SiLU + per-row fp8 quant and the down GEMM (router weight in its epilogue) of every 16-row routing block
    in one workgroup (r9k_moe_stream_layer): down bf16 [numel, N2] = the down moe_gemm's rows over the quantised
    activation of the gate_up output (bit for bit against the single-wave launches). False when the shape is not
    served (nothing launched)."""
    E = num_experts if num_experts is not None else w1.wq.shape[0]
    assert a_q.is_contiguous() and a_q.shape[1] == w1.K and a_s.dtype == torch.float32
    assert w2.K == w1.N // 2 and down.dtype == torch.bfloat16 and down.shape == (numel, w2.N) and down.is_contiguous()
    assert topk_w.dtype == torch.float32 and topk_w.is_contiguous() and topk_w.numel() == numel
    max_blocks = min(expert_ids.numel(), (numel + MOE_BLOCK - 1) // MOE_BLOCK + min(numel, E))
    rc = lib().r9k_moe_stream_layer(a_q.data_ptr(), a_s.data_ptr(), w1.wq.data_ptr(), w1.wsr.data_ptr(),
                                    w2.wq.data_ptr(), w2.wsr.data_ptr(), down.data_ptr(), sorted_ids.data_ptr(),
                                    expert_ids.data_ptr(), ntpp.data_ptr(), topk_w.data_ptr(), w1.estride, w2.estride,
                                    max_blocks, numel, topk, w1.K, w1.N, w2.N, _stream())
    if rc == 2:
        return False
    if rc:
        raise RuntimeError(f"r9k_moe_stream_layer failed ({rc}) N1={w1.N} K1={w1.K} N2={w2.N}")
    return True


def stream_wanted(numel: int, num_experts: int, topk: int) -> bool:
    """Whether a decode step of `numel` routed rows over `num_experts` experts takes r9k_moe_stream_layer."""
    if not STREAM:
        return False
    b = expected_blocks(numel, num_experts, topk)
    return STREAM_MIN_BLOCKS <= b <= device_cus()


# Steps whose routing may leave many experts with a handful of rows (config 5's Zipf skew: at T = 4096, 104 of 169
# touched experts hold at most 16 rows) split their tables on the device (moe_align_split): experts with more than
# split_thr(numel) rows go to 256-row blocks on the prefill kernel, the others to 16-row blocks on the block stream,
# which reads their weights at the streaming rate instead of paying a 256-row tile's DMA for a few rows. Measured on
# MI355X at config 5, each GEMM alone at T = 4096 (169 touched experts): gate_up 840 us in one 256-row layout, 537
# (65 experts over 16 rows, 256-row kernel) + 144 us (104 experts, block stream) split; down 439 against 315 + 76 us.
# The layer: T = 4096 1312 -> 1181 us (threshold 16; 32 / 64 / 128: 1298 / 1287 / 1382 us), T = 256 363 us on the
# device-picked layout pair -> 318 us split at threshold 32 (16 / 64 / 128: 358 / 350 / 378 us: at 2048 routed rows
# the 256-row kernel has too few tiles to fill the CUs, so more experts stay on the stream). Taken from
# SPLIT_MIN_NUMEL routed rows while the mean rows per expert is at most SPLIT_MEAN_MAX (a uniform config 3 step, 227
# rows an expert, never has experts that small). Up to the router's table-building width (4096 routed rows) only
# for experts of at least SPLIT_DECODE_MIN_BYTES of gate_up codes: config 2's 1 MB experts run T = 128 / 256 faster
# on the router's tables and decode blocks (110 / 127 us against 135 / 142 us split; T = 512: 193 against 170 us).
# The stream's column split is sized for SPLIT_HINT live blocks. R9K_SPLIT=0 turns it off.
SPLIT = os.environ.get("R9K_SPLIT", "1") == "1"
SPLIT_MIN_NUMEL = int(os.environ.get("R9K_SPLIT_MIN_NUMEL", "1024"))
SPLIT_MEAN_MAX = int(os.environ.get("R9K_SPLIT_MEAN_MAX", "128"))
SPLIT_DECODE_MIN_BYTES = int(os.environ.get("R9K_SPLIT_DECODE_MIN_BYTES", str(4 << 20)))
SPLIT_HINT = int(os.environ.get("R9K_SPLIT_HINT", "128"))
_SPLIT_THR = os.environ.get("R9K_SPLIT_THR")


def split_wanted(numel: int, num_experts: int, K1: int, K2: int) -> bool:
    """Whether a step of `numel` routed rows over `num_experts` experts (gate_up K1 x 2 K2, down K2) splits its
    tables by expert size: the block stream and the 256-row kernel serve K % 128 == 0, the stream up to 4096."""
    if not (SPLIT and SPLIT_MIN_NUMEL <= numel <= SPLIT_MEAN_MAX * num_experts
            and all(k % 128 == 0 and 0 < k <= 4096 for k in (K1, K2)) and big_block_cfg(K1, K2) is not None):
        return False
    return numel > 4096 or K1 * K2 >= SPLIT_DECODE_MIN_BYTES          # gate_up codes: K1 * 2 K2 / 2 bytes


def split_thr(numel: int) -> int:
    """Rows up to which an expert of a split step goes to the block stream."""
    return int(_SPLIT_THR) if _SPLIT_THR else (32 if numel <= 4096 else 16)


# ops.mxfp4_linear runs the one-launch dense path (r9k_dense_mxfp4_qa, M <= 4) up to this many rows. Measured on
# MI355X at config 4 ([17408, 5120]), one launch against the two (quant + GEMM): M = 1 10.7 vs 16.3 us, M = 2 13.2
# vs 16.4 us, M = 3 17.8 vs 16.5 us, M = 4 19.6 vs 16.6 us (from three rows the activation chunks the workgroup holds
# in registers, 228 VGPRs at M = 4, leave two waves a SIMD), so M > 2 keeps two launches.
DENSE_QA_MAX_M = int(os.environ.get("R9K_DENSE_QA_MAX_M", "2"))


def dense_mxfp4_qa(x: torch.Tensor, w: Mxfp4Experts, out: torch.Tensor) -> bool:
    """out [M, N] = bf16(quant_rows_fp8(x) @ W^T) for one dense MXFP4 weight (w.wq / w.wsr of a single expert) in ONE
    launch (r9k_dense_mxfp4_qa: every workgroup quantises the <= 4 activation rows into LDS itself), the values of
    quant_rows_fp8 + moe_gemm over identity tables bit for bit. False when not served (nothing launched)."""
    M = x.shape[0]
    assert x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1 and x.shape[1] == w.K
    assert out.dtype == torch.bfloat16 and out.shape == (M, w.N) and out.stride(1) == 1
    rc = lib().r9k_dense_mxfp4_qa(x.data_ptr(), x.stride(0), w.wq.data_ptr(), w.wsr.data_ptr(), out.data_ptr(),
                                  out.stride(0), M, w.N, w.K, _stream())
    if rc == 2:
        return False
    if rc:
        raise RuntimeError(f"r9k_dense_mxfp4_qa failed ({rc}) M={M} N={w.N} K={w.K}")
    return True


# ops.mxfp4_gemm_q (the dense GEMM on quantised rows: the MXFP4 linear from DENSE_QA_MAX_M + 1 rows, the shared
# expert) runs the dense kernel (r9k_dense_mxfp4_a8) up to this many rows (the kernel serves up to 16); above it the
# decode-family GEMM. Measured at config 4 ([17408, 5120]), quant + GEMM against quant + decode GEMM: M = 4 15.0 vs
# 16.7 us, M = 8 16.6 vs 18.1, M = 16 19.9 vs 21.1.
DENSE_A8_MAX_M = int(os.environ.get("R9K_DENSE_A8_MAX_M", "16"))


def dense_mxfp4_a8(q: torch.Tensor, s: torch.Tensor, w: Mxfp4Experts, out: torch.Tensor,
                   topk_w: torch.Tensor | None = None) -> bool:
    """out [M, N] = bf16(dequant(q, s) @ W^T (* topk_w[row])) for one dense MXFP4 weight and M <= 16 rows already
    quantised (quant_rows_fp8's codes and scales), on the dense kernel's weight stream (r9k_dense_mxfp4_a8): the values
    of moe_gemm over identity tables bit for bit. False when not served (nothing launched)."""
    M = q.shape[0]
    assert q.dtype in (torch.uint8, torch.float8_e4m3fn) and q.dim() == 2 and q.stride(1) == 1 and q.shape[1] == w.K
    assert s.dtype == torch.float32 and s.is_contiguous() and s.numel() >= M
    assert out.dtype == torch.bfloat16 and out.shape == (M, w.N) and out.stride(1) == 1
    if topk_w is not None:
        assert topk_w.dtype == torch.float32 and topk_w.is_contiguous() and topk_w.numel() >= M
    rc = lib().r9k_dense_mxfp4_a8(q.data_ptr(), q.stride(0), s.data_ptr(),
                                  topk_w.data_ptr() if topk_w is not None else 0, w.wq.data_ptr(), w.wsr.data_ptr(),
                                  out.data_ptr(), out.stride(0), M, w.N, w.K, _stream())
    if rc == 2:
        return False
    if rc:
        raise RuntimeError(f"r9k_dense_mxfp4_a8 failed ({rc}) M={M} N={w.N} K={w.K}")
    return True


# ops.nvfp4_linear runs the one-launch native NVFP4 path (r9k_dense_nvfp4_qa: the activation quant inside the GEMM
# launch) up to this many rows (the kernel serves up to 2). Measured at config 4 ([17408, 5120]), one launch against
# quant + GEMM: M = 1 15.2 vs 19.7 us, M = 2 18.7 vs 18.7 us.
DENSE_NV_QA_MAX_M = int(os.environ.get("R9K_DENSE_NV_QA_MAX_M", "1"))


def dense_nvfp4_qa(x: torch.Tensor, w: Nvfp4Experts, out: torch.Tensor) -> bool:
    """out [M, N] = bf16(quant_rows_fp8(x) @ W^T) for one native NVFP4 weight (w.wq / w.ws / w.wg of a single expert)
    in ONE launch (r9k_dense_nvfp4_qa: every workgroup quantises the <= 2 activation rows into LDS itself), the values
    of quant_rows_fp8 + moe_gemm over identity tables bit for bit. False when not served (nothing launched)."""
    M = x.shape[0]
    assert x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1 and x.shape[1] == w.K
    assert out.dtype == torch.bfloat16 and out.shape == (M, w.N) and out.stride(1) == 1
    rc = lib().r9k_dense_nvfp4_qa(x.data_ptr(), x.stride(0), w.wq.data_ptr(), w.ws.data_ptr(), w.wg.data_ptr(),
                                  out.data_ptr(), out.stride(0), M, w.N, w.K, _stream())
    if rc == 2:
        return False
    if rc:
        raise RuntimeError(f"r9k_dense_nvfp4_qa failed ({rc}) M={M} N={w.N} K={w.K}")
    return True


# ------------------------------------------------------------------------------------- routing and sum
def moe_sum(down: torch.Tensor, shared: torch.Tensor | None, out: torch.Tensor) -> torch.Tensor:
    """out[M, N] = sum over top-k of down[M, topk, N] (+ shared[M, N]) in fp32, one bf16 rounding."""
    M, topk, N = down.shape
    assert down.is_contiguous() and out.shape == (M, N) and out.dtype == torch.bfloat16 and out.stride(1) == 1
    rc = lib().r9k_moe_sum(down.data_ptr(), shared.data_ptr() if shared is not None else 0, out.data_ptr(), M, topk,
                           N, shared.stride(0) if shared is not None else 0, out.stride(0), _stream())
    if rc:
        raise RuntimeError(f"r9k_moe_sum failed ({rc}) M={M} topk={topk} N={N}")
    return out


def capacity(numel: int, num_experts: int, blk: int) -> int:
    """sorted_ids length for `numel` routed rows (moe_align_block_size's sizing)."""
    cap = numel + num_experts * (blk - 1)
    return (cap + blk - 1) // blk * blk


_ALIGN_SCRATCH: dict = {}


def _align_scratch(device: torch.device, n: int) -> torch.Tensor:
    key = (device.type, device.index)
    t = _ALIGN_SCRATCH.get(key)
    if t is None or t.numel() < n:
        # the multi-workgroup align's per-chunk histograms (every call rewrites what it reads)
        t = torch.zeros(max(n, 1 << 16), dtype=torch.int32, device=device)
        _ALIGN_SCRATCH[key] = t
    return t


def moe_align(topk_ids: torch.Tensor, block: int, num_experts: int, expert_map: torch.Tensor | None = None,
              live_only: bool = False):
    """GPU moe_align_block_size: (sorted_ids [cap], expert_ids [cap/block], ntpp [1]) int32, rows ascending within
    each expert (align_block_size_ref's canonical order). expert_map (global -> local id, -1 = not here) is
    applied first; rows of experts outside [0, num_experts) are left out of the tables. live_only writes the entries
    up to ntpp only (r9k_moe_align_live; the rest of the capacity is left unset), enough for this library's GEMMs."""
    ids = topk_ids.reshape(-1)
    if expert_map is not None:
        ids = expert_map[ids.long()]
    ids = ids.to(torch.int32).contiguous()
    numel = ids.numel()
    dev = ids.device
    cap = capacity(numel, num_experts, block)
    sorted_ids = torch.empty(cap, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(cap // block, dtype=torch.int32, device=dev)
    ntpp = torch.empty(1, dtype=torch.int32, device=dev)
    L = lib()
    n = L.r9k_moe_align_scratch_ints(numel, num_experts)
    scratch = _align_scratch(dev, n)
    fn = L.r9k_moe_align_live if live_only else L.r9k_moe_align
    rc = fn(ids.data_ptr(), numel, num_experts, block, sorted_ids.data_ptr(), expert_ids.data_ptr(), ntpp.data_ptr(),
            scratch.data_ptr(), scratch.numel(), _stream())
    if rc:
        raise RuntimeError(f"r9k_moe_align failed ({rc}) numel={numel} E={num_experts} block={block}")
    return sorted_ids, expert_ids, ntpp


def moe_align_split(topk_ids: torch.Tensor, num_experts: int, thr: int, big_block: int, small_block: int):
    """Tables of one routed step split by expert size on the device (r9k_moe_align_split): (big, small), each
    (sorted_ids, expert_ids, ntpp) int32 written up to its ntpp. big holds the experts with more than thr rows in
    big_block-row blocks, small the others in small_block-row blocks. small's expert_ids is cut to the most blocks
    its experts can fill (at most min(E, numel) experts of at most thr rows), so a kernel gridded on its length
    launches no more workgroups than that."""
    ids = topk_ids.reshape(-1).to(torch.int32).contiguous()
    numel, E, dev = ids.numel(), num_experts, ids.device
    i32 = dict(dtype=torch.int32, device=dev)
    capb = capacity(numel, E, big_block)
    nbs = min(E, numel) * -(-max(thr, 1) // small_block)
    big = (torch.empty(capb, **i32), torch.empty(capb // big_block, **i32), torch.empty(1, **i32))
    small = (torch.empty(max(capacity(numel, E, small_block), nbs * small_block), **i32),
             torch.empty(capacity(numel, E, small_block) // small_block, **i32), torch.empty(1, **i32))
    L = lib()
    n = L.r9k_moe_align_scratch_ints(numel, E)
    scratch = _align_scratch(dev, n)
    rc = L.r9k_moe_align_split(ids.data_ptr(), numel, E, thr, big_block, *(t.data_ptr() for t in big), small_block,
                               *(t.data_ptr() for t in small), scratch.data_ptr(), scratch.numel(), _stream())
    if rc:
        raise RuntimeError(f"r9k_moe_align_split failed ({rc}) numel={numel} E={E} thr={thr}")
    return big, (small[0], small[1][:nbs], small[2])


def moe_align_noalloc(topk_ids: torch.Tensor, block: int, num_experts: int, out=None):
    """moe_align's tables from r9k_moe_align_noalloc, which allocates nothing on the device (its scratch is the
    library's own fixed 1 MiB array per GPU; overlapping calls on one GPU race on it). `out` = (sorted_ids,
    expert_ids, ntpp) int32 buffers of at least capacity(numel, num_experts, block), that / block and 1 entries, or
    None to allocate them here. Raises RuntimeError when the step needs more scratch than the array holds."""
    ids = topk_ids.reshape(-1)
    assert ids.dtype == torch.int32 and ids.is_contiguous()
    numel = ids.numel()
    cap = capacity(numel, num_experts, block)
    if out is None:
        out = (torch.empty(cap, dtype=torch.int32, device=ids.device),
               torch.empty(cap // block, dtype=torch.int32, device=ids.device),
               torch.empty(1, dtype=torch.int32, device=ids.device))
    sorted_ids, expert_ids, ntpp = out
    assert sorted_ids.numel() >= cap and expert_ids.numel() >= cap // block and ntpp.numel() >= 1
    L = lib()
    rc = L.r9k_moe_align_noalloc(ids.data_ptr(), numel, num_experts, block, sorted_ids.data_ptr(),
                                 expert_ids.data_ptr(), ntpp.data_ptr(), _stream())
    if rc == -9:
        raise RuntimeError(f"r9k_moe_align_noalloc: numel={numel} E={num_experts} needs "
                           f"{L.r9k_moe_align_scratch_ints(numel, num_experts)} scratch ints, more than the "
                           f"{L.r9k_moe_align_noalloc_max_ints()} it holds")
    if rc:
        raise RuntimeError(f"r9k_moe_align_noalloc failed ({rc}) numel={numel} E={num_experts} block={block}")
    return sorted_ids, expert_ids, ntpp


def moe_topk(logits: torch.Tensor, topk: int, renorm: bool):
    """Softmax top-k routing (stock FusedTopKRouter's outputs): logits [M, E] bf16 -> (w fp32 [M, topk],
    ids int32 [M, topk]), descending probability, ties to the lower expert index."""
    assert logits.dtype == torch.bfloat16 and logits.dim() == 2 and logits.stride(1) == 1
    M, E = logits.shape
    w = torch.empty((M, topk), dtype=torch.float32, device=logits.device)
    ids = torch.empty((M, topk), dtype=torch.int32, device=logits.device)
    if M == 0:
        return w, ids
    rc = lib().r9k_moe_topk(logits.data_ptr(), logits.stride(0), w.data_ptr(), ids.data_ptr(), M, E, topk,
                            1 if renorm else 0, _stream())
    if rc:
        raise RuntimeError(f"r9k_moe_topk failed ({rc}) M={M} E={E} topk={topk}")
    return w, ids


def moe_topk_quant(logits: torch.Tensor, topk: int, renorm: bool, x: torch.Tensor):
    """moe_topk and quant_rows_fp8(x) in one launch (r9k_moe_topk_quant; the two kernels' work interleaved over the
    CUs): (w, ids, xq e4m3fn [M, H], xs fp32 [M]), the same values as the two calls. None when x's shape or
    alignment does not suit the fused launch (then nothing ran: call the two functions)."""
    assert logits.dtype == torch.bfloat16 and logits.dim() == 2 and logits.stride(1) == 1
    M, E = logits.shape
    if not (x.dim() == 2 and x.dtype == torch.bfloat16 and x.shape[0] == M and x.stride(1) == 1) or M == 0:
        return None
    dev = logits.device
    H = x.shape[1]
    w = torch.empty((M, topk), dtype=torch.float32, device=dev)
    ids = torch.empty((M, topk), dtype=torch.int32, device=dev)
    xq = torch.empty((M, H), dtype=torch.float8_e4m3fn, device=dev)
    xs = torch.empty((M,), dtype=torch.float32, device=dev)
    rc = lib().r9k_moe_topk_quant(logits.data_ptr(), logits.stride(0), w.data_ptr(), ids.data_ptr(), M, E, topk,
                                  1 if renorm else 0, x.data_ptr(), x.stride(0), H, xq.data_ptr(), xs.data_ptr(),
                                  _stream())
    if rc == 2:
        return None
    if rc:
        raise RuntimeError(f"r9k_moe_topk_quant failed ({rc}) M={M} E={E} topk={topk} H={H}")
    return w, ids, xq, xs


def align_block_size_ref(topk_ids: torch.Tensor, num_experts: int, block: int = MOE_BLOCK):
    """Host-side moe_align_block_size in the canonical order (tests and host table builds): a stable sort of the
    routed rows by expert, each expert's run padded to a multiple of `block` with the pad value numel, expert_ids
    -1 past the used blocks; ids outside [0, num_experts) are left out. Returns (sorted_ids, expert_ids, ntpp) int32,
    sized to capacity()."""
    flat = topk_ids.flatten().to(torch.int64).cpu()
    numel = flat.numel()
    cap = capacity(numel, num_experts, block)
    keep = (flat >= 0) & (flat < num_experts)
    order = torch.argsort(torch.where(keep, flat, num_experts), stable=True)[: int(keep.sum())]
    counts = torch.bincount(flat[keep], minlength=num_experts)
    padded = (counts + block - 1) // block * block
    start = torch.cumsum(padded, 0) - padded                     # first slot of each expert
    first_row = torch.cumsum(counts, 0) - counts                 # its first entry in `order`
    e_of = flat[order]
    slot = start[e_of] + (torch.arange(order.numel()) - first_row[e_of])
    sorted_ids = torch.full((cap,), numel, dtype=torch.int32)
    sorted_ids[slot] = order.to(torch.int32)
    total = int(padded.sum())
    expert_ids = torch.full((cap // block,), -1, dtype=torch.int32)
    expert_ids[: total // block] = torch.repeat_interleave(torch.arange(num_experts, dtype=torch.int32),
                                                          padded // block)
    return sorted_ids, expert_ids, torch.tensor([total], dtype=torch.int32)
