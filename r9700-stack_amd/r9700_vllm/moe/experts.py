"""R9700Mxfp4Experts: the fused-MoE experts backed by libr9k's grouped MXFP4 x FP8 GEMM on gfx950.

Mirrors the reference's r9700_vllm/moe/experts.py (class name, apply() signature, in-place output). With vLLM
installed it is a vLLM modular fused-MoE experts class; without it, the same class works standalone
(``R9700Mxfp4Experts.standalone(w13_scale, w2_scale)``), which is how the tests and bench.py drive it.

Layer weights (set by weight prep, quant/ct.py or kernels/moe.prepare_mxfp4_weights):
  w13_weight        [E, N1*K1/8] int32   fragment order (N1 = 2*I, K1 = hidden)
  w2_weight         [E, N2*K2/8] int32                  (N2 = hidden, K2 = I)
  w13_weight_scale  [E, K1/32 + 1, N1]  uint8  exponents in fragment order + per-row max (last row)
  w2_weight_scale   [E, K2/32 + 1, N2]  uint8
Flow per call (reference experts.py:149-251): align tables (from the router, else the GPU align) -> per-token fp8
quant -> grouped gate_up GEMM -> silu(g)*u + per-row fp8 quant -> grouped down GEMM with the router weight in the
epilogue -> top-k sum into `output`, all on torch's current stream with no host synchronisation, so a call can be
captured in a HIP graph. Decode widths fuse launches: up to ~128 MiB of routed down weights the SiLU, down and sum
run as one token-major launch (r9k_moe_down_sum); wider steps that touch most experts run gate_up, the SiLU + quant
and down of each routing block in one workgroup (r9k_moe_stream_layer), then the top-k sum.
"""
from __future__ import annotations

import os

import torch

from .._compat import vllm_available
from ..kernels import moe as K
from . import route

ZERO_DOWN = os.environ.get("R9K_MOE_ZERO_DOWN", "0") == "1"
# R9K_MOE_FUSE=1: at decode (MT == 1) the activation runs in the gate_up GEMM's epilogue and the per-row fp8 quant in
# the down GEMM's A-load (r9k_moe_mxfp4a8_f), so there is no SiLU launch; results equal the unfused chain's
# (reference switch: moe/experts.py:55-58).
MOE_FUSE = os.environ.get("R9K_MOE_FUSE", "0") == "1"


# A launch of the 256-row prefill GEMM addresses its activations, one expert's codes and its output through 32-bit
# buffer ranges, so no buffer one launch touches may reach 2 GiB. A step whose routed rows would cross that runs as
# token chunks (each a complete layer step over its own tables), planned by chunk_tokens.
BUF_LIMIT = (1 << 31) - 1


def chunk_tokens(M: int, topk: int, N1: int, K1: int, N2: int, K2: int, limit: int = BUF_LIMIT) -> list:
    """Token ranges [(t0, t1), ...] covering 0..M, as few and as even as possible, such that in each range every
    per-step buffer stays <= `limit` bytes: the gate_up output [rows*topk, N1] and the down output [rows*topk, N2]
    (bf16), the fp8 activations of both GEMMs ([rows, K1] and [rows*topk, K2]) and the fp32 row scales."""
    per_token = max(topk * N1 * 2, topk * N2 * 2, K1, topk * K2, topk * 4)
    n = -(-M // max(1, limit // per_token))
    if n == 0:
        return []
    bounds = [M * i // n for i in range(n + 1)]
    return list(zip(bounds[:-1], bounds[1:]))


# A pass whose GEMMs run on the block stream (r9k_moe_stream over 16-row blocks): the small-expert table of a split
# prefill step (kernels.moe.split_wanted).
STREAM_PASS = 0


def _stream_pass(a, a_s, W, out, sid, eid, ntpp, numel: int, a_row_div: int, tw, E: int) -> None:
    if not K.moe_stream(a, a_s, W, out, sid, eid, ntpp, numel, a_row_div, tw, num_experts=E,
                        blocks_hint=K.SPLIT_HINT):
        raise RuntimeError(f"r9k MoE: the block stream does not serve N={W.N} K={W.K} (split tables need it)")


def r9k_available() -> bool:
    """ROCm torch with a gfx950 device and the kernel library loadable."""
    try:
        if not torch.cuda.is_available() or torch.version.hip is None:
            return False
        arch = torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName
        if not arch.startswith("gfx950"):
            return False
        K.lib()
        return True
    except Exception:
        return False


def _experts_base():
    if vllm_available():
        try:
            import vllm.model_executor.layers.fused_moe.modular_kernel as mk
            return mk.FusedMoEExpertsModular
        except Exception:
            pass

    class _StandaloneExperts:
        """Base used when vLLM is not installed: holds the two scale tensors the modular kernel would supply."""

        def __init__(self, moe_config=None, quant_config=None, max_num_tokens=None, num_dispatchers=None):
            self.moe_config = moe_config
            self.quant_config = quant_config
            self.w1_scale = getattr(quant_config, "w1_scale", None)
            self.w2_scale = getattr(quant_config, "w2_scale", None)

    return _StandaloneExperts


class R9700Mxfp4Experts(_experts_base()):

    @classmethod
    def standalone(cls, w1_scale: torch.Tensor, w2_scale: torch.Tensor, nv=None) -> "R9700Mxfp4Experts":
        """An experts object outside vLLM over pack_scales-layout scale tensors, or, with nv = (w13 row multipliers,
        w2 row multipliers), over native NVFP4 scale tensors (prepare_nvfp4_weights)."""
        obj = cls.__new__(cls)
        obj.w1_scale = w1_scale
        obj.w2_scale = w2_scale
        obj.nv = nv
        return obj

    @staticmethod
    def activation_format():
        import vllm.model_executor.layers.fused_moe.modular_kernel as mk
        return mk.FusedMoEActivationFormat.Standard

    def finalize_weight_and_reduce_impl(self):
        from vllm.model_executor.layers.fused_moe.topk_weight_and_reduce import TopKWeightAndReduceNoOP
        return TopKWeightAndReduceNoOP()

    @staticmethod
    def _supports_current_device() -> bool:
        return r9k_available()

    @staticmethod
    def _supports_no_act_and_mul() -> bool:
        return False

    @staticmethod
    def _supports_quant_scheme(weight_key, activation_key) -> bool:
        return activation_key is None

    @staticmethod
    def _supports_activation(activation) -> bool:
        return str(getattr(activation, "name", activation)).lower() == "silu"

    @staticmethod
    def _supports_parallel_config(moe_parallel_config) -> bool:
        return not (getattr(moe_parallel_config, "use_fi_nvl_two_sided_kernels", False)
                    or getattr(moe_parallel_config, "use_fi_nvl_one_sided_kernels", False))

    fold = (False, False)
    # native NVFP4 experts (quant/nvfp4.py prep_native_moe): (w13, w2) per-row fp32 multipliers [E, N]; the scale
    # tensors then hold prepare_nvfp4_weights' layout and both GEMMs run r9k_moe_nvfp4a8 on decode-family blocks
    # (reference: moe/experts.py:118-145)
    nv: tuple[torch.Tensor, torch.Tensor] | None = None

    def _dims(self, ws: torch.Tensor) -> tuple[int, int]:
        """(N, K) of one GEMM from its pack_scales tensor [E, K/32 + 1, N]."""
        return ws.shape[2], (ws.shape[1] - 1) * K.GROUP

    def _gemm_dims(self, hidden: int) -> tuple[int, int, int, int]:
        """(N1, K1, N2, K2): from the scale tensors for MXFP4, from the row multipliers and the input for NVFP4."""
        if self.nv is not None:
            N1, N2 = self.nv[0].shape[1], self.nv[1].shape[1]
            return N1, hidden, N2, N1 // 2
        return (*self._dims(self.w1_scale), *self._dims(self.w2_scale))

    def process_weights_after_loading(self, layer) -> None:
        sup = getattr(super(), "process_weights_after_loading", None)
        if sup is not None:
            sup(layer)
        self.fold = (False, False)
        self.nv = ((layer.w13_weight_row_mult, layer.w2_weight_row_mult)
                   if getattr(layer, "_r9k_nvfp4", False) else None)

    def moe_problem_size(self, a1, w1, w2, topk_ids):
        N1 = self._gemm_dims(a1.size(-1))[0]
        return w1.size(0), a1.size(0), N1 // 2, a1.size(-1), topk_ids.size(1)

    def workspace_shapes(self, M, N, K_, topk, global_num_experts, local_num_experts, expert_tokens_meta,
                         activation):
        # only the output buffer comes from the modular kernel's workspace; intermediates are allocated per call
        return ((M, K_), (1,), (M, K_))

    def apply(self, output, hidden_states, w1, w2, topk_weights, topk_ids, activation, global_num_experts,
              expert_map, a1q_scale, a2_scale, workspace13, workspace2, expert_tokens_meta,
              apply_router_weight_on_input):
        assert not apply_router_weight_on_input, "R9700Mxfp4Experts: router weight on input not supported"
        assert hidden_states.dtype == torch.bfloat16 and hidden_states.is_contiguous()
        N1, K1, N2, K2 = self._gemm_dims(hidden_states.shape[1])
        M, topk = hidden_states.shape[0], topk_ids.shape[1]
        E = w1.shape[0]
        if global_num_experts == -1:
            global_num_experts = E
        numel = M * topk
        dev = hidden_states.device
        if M == 0:
            return

        chunks = chunk_tokens(M, topk, N1, K1, N2, K2)
        if len(chunks) > 1:
            for t0, t1 in chunks:
                self.apply(output[t0:t1], hidden_states[t0:t1], w1, w2, topk_weights[t0:t1], topk_ids[t0:t1],
                           activation, global_num_experts, expert_map, a1q_scale, a2_scale, workspace13, workspace2,
                           expert_tokens_meta, apply_router_weight_on_input)
            return output

        nv = self.nv
        MT = K.pick_mt(numel, global_num_experts)
        big = K.pick_moe_prefill_block(numel, global_num_experts, K1, K2)
        if big is not None:                                  # prefill widths: one 256-row block ~ one expert
            pf_gate = pf_down = big[0]
            blk = big[1]
        else:
            blk = K.MOE_BLOCK * MT
            pf_down = None if nv is not None else K.pick_moe_prefill(MT, K2)
            pf_gate = None if nv is not None else K.pick_moe_prefill(MT, K1, gate_up=True)
        cache = getattr(self, "r9k_cache", None)
        slot_ids = cache_q = None
        if cache is not None:
            # host-offloaded experts (moe/cache.py): LRU manage + gather, then a pass over the VRAM slots (ids
            # through table) and, unless provably empty, one over the host store (ids through map_cold); every
            # routed row belongs to exactly one pass (reference moe/experts.py:167-199)
            if expert_map is not None or nv is not None:
                raise RuntimeError("r9k expert cache: MXFP4 experts without an expert map only")
            (h1, h2), (c1, c2) = cache.hot(), cache.cold()
            need_cold = numel > cache.no_cold_limit
            staged = need_cold and cache.stage is not None
            if cache.fused:
                # with staging the cold pass gets its tables from the stage map below, not from the host map; the
                # same launch quantises the input unless the router already did
                rq = route.take_quant(getattr(self, "r9k_layer", None), topk_ids, hidden_states)
                hot_al, cold_al = cache.update_fused(topk_ids, blk, need_cold and not staged,
                                                     x=hidden_states if rq is None else None)
                cache_q = cache.x_quant
                if not need_cold:
                    slot_ids = cache.hot_ids.view(M, topk)   # every routed expert resident: each row's slot
            else:
                cache.update(topk_ids)
                hot_al = K.moe_align(topk_ids, blk, E, cache.table)
                cold_al = K.moe_align(topk_ids, blk, E, cache.map_cold) if need_cold and not staged else None
            if staged:
                # R9K_STAGE_COLD=1: the cold experts copied into VRAM in one gather, the cold pass over that copy
                c1, c2, stage_map = cache.stage_cold(topk_ids)
                cold_al = K.moe_align(topk_ids, blk, E, stage_map)
            passes = [(h1, h2, hot_al, (MT, pf_gate, pf_down))]
            if need_cold:
                passes.append((c1, c2, cold_al, (MT, pf_gate, pf_down)))
        else:
            layer = getattr(self, "r9k_layer", None)
            bc = K.big_block_cfg(K1, K2)
            plain = nv is None and expert_map is None and not MOE_FUSE
            dual_ok = plain and bc is not None and K.DEVICE_BLOCKS_MIN > 0
            if layer is not None:
                # tells the router which of this layer's steps need no tables from it (route.split_planned: the
                # experts split theirs) and for which it should build both layouts (route.dual_wanted)
                layer._r9k_split_k = (K1, K2) if plain else None
                layer._r9k_dual_blk = bc[1] if dual_ok else 0
            split = plain and K.split_wanted(numel, E, K1, K2)
            tabs = route.take(layer, topk_ids, blk, numel) if expert_map is None and not split else None
            tabs_big = route.take_big(layer, topk_ids, blk, numel) if tabs is not None else None
            tabs_small = None
            if split:
                # experts with a handful of rows on the block stream, the rest in the 256-row layout (split on the
                # device: the host cannot see the counts)
                MT, (pf_gate, blk) = 1, bc
                pf_down = pf_gate
                tabs, tabs_small = K.moe_align_split(topk_ids, E, K.split_thr(numel), blk, K.MOE_BLOCK)
            elif tabs is None:
                tabs = K.moe_align(topk_ids, blk, E, expert_map)
            if nv is not None:
                W1 = K.Nvfp4Experts(w1, self.w1_scale, nv[0], N1, K1)
                W2 = K.Nvfp4Experts(w2, self.w2_scale, nv[1], N2, K2)
            else:
                W1 = K.Mxfp4Experts(w1, self.w1_scale, N1, K1)
                W2 = K.Mxfp4Experts(w2, self.w2_scale, N2, K2)
            passes = [(W1, W2, tabs, (MT, pf_gate, pf_down))]
            if tabs_small is not None:
                passes.append((W1, W2, tabs_small, (STREAM_PASS, None, None)))
            if tabs_big is not None:
                # the router built both layouts and the device kept one: both passes run (the other's GEMMs exit)
                if big is not None or not dual_ok or tabs_big[3] != bc[1]:
                    raise RuntimeError("r9k MoE: the router's second table layout does not fit this layer's pass")
                passes.append((W1, W2, tabs_big[:3], (1, bc[0], bc[0])))
            elif big is None and dual_ok and not split and numel >= K.DEVICE_BLOCKS_MIN:
                # skew the host cannot see: the 256-row layout too, the device keeps one (the other's GEMMs exit)
                tabs_big = K.moe_align(topk_ids, bc[1], E, live_only=True)
                K.pick_blocks(tabs[2], tabs_big[2], numel, bc[1])
                passes.append((W1, W2, tabs_big, (1, bc[0], bc[0])))

        # the router's fp8 quant of this input, when it made one (with its tables at decode, alone at prefill)
        q = route.take_quant(getattr(self, "r9k_layer", None), topk_ids, hidden_states) if expert_map is None else None
        if q is None:
            q = cache_q                                      # the expert cache's manage launch made it
        xq, xs = q if q is not None else K.quant_rows_fp8(hidden_states)
        fused = MOE_FUSE and nv is None and MT == 1 and pf_gate is None and pf_down is None
        # wide decode steps (most experts touched, one 16-row block each, about one block a CU): gate_up, the SiLU +
        # fp8 quant and down of each routing block in one workgroup (r9k_moe_stream_layer), the quantised rows handed
        # over in LDS: no SiLU launch and no gate_up intermediate in HBM
        if (not fused and cache is None and nv is None and expert_map is None and not ZERO_DOWN and len(passes) == 1
                and MT == 1 and pf_gate is None and pf_down is None and K.stream_wanted(numel, E, topk)
                and not K.down_sum_fits(numel, N2, K2)):
            W1, W2, (sid, eid, ntpp), _ = passes[0]
            down = torch.empty((numel, N2), dtype=torch.bfloat16, device=dev)
            tw = topk_weights.reshape(-1).to(torch.float32).contiguous()
            if K.moe_stream_layer(xq, xs, W1, W2, down, sid, eid, ntpp, numel, topk, tw, E):
                K.moe_sum(down.view(M, topk, N2), None, output)
                return output
        if fused:
            aq = torch.empty((numel, N1 // 2), dtype=torch.float32, device=dev)
            for W1, _, (sid, eid, ntpp), _ in passes:
                K.moe_gemm(xq, xs, W1, aq, sid, eid, ntpp, numel, topk, None, num_experts=E, MT=1, fuse=1)
            as_ = None
        else:
            gate_up = torch.empty((numel, N1), dtype=torch.bfloat16, device=dev)
            for W1, _, (sid, eid, ntpp), (mt, pfg, _) in passes:
                if mt == STREAM_PASS:
                    _stream_pass(xq, xs, W1, gate_up, sid, eid, ntpp, numel, topk, None, E)
                else:
                    K.moe_gemm(xq, xs, W1, gate_up, sid, eid, ntpp, numel, topk, None, num_experts=E, MT=mt,
                               prefill=pfg)
            # the token-major tail's expert ids: the routing ids, or each row's slot when every routed expert is
            # resident (the cache's one-launch manage wrote them; the host pass is provably empty)
            ds_ids = topk_ids.to(torch.int32).contiguous() if cache is None else slot_ids
            if (ds_ids is not None and len(passes) == 1 and nv is None and expert_map is None and MT == 1
                    and pf_gate is None and K.down_sum_fits(numel, N2, K2) and not ZERO_DOWN):
                # decode widths: SiLU + quant, down and the top-k sum in one token-major launch
                tw = topk_weights.reshape(-1).to(torch.float32).contiguous()
                if K.moe_down_sum(gate_up, ds_ids, tw, passes[0][1], output):
                    return output
            aq, as_ = K.silu_mul_quant_fp8(gate_up)
        # Rows no table places (experts on other ranks under an expert map) must not feed moe_sum garbage.
        if expert_map is not None or ZERO_DOWN:
            down = torch.zeros((numel, N2), dtype=torch.bfloat16, device=dev)
        else:
            down = torch.empty((numel, N2), dtype=torch.bfloat16, device=dev)
        tw = topk_weights.reshape(-1).to(torch.float32).contiguous()
        for _, W2, (sid, eid, ntpp), (mt, _, pfd) in passes:
            if mt == STREAM_PASS:
                _stream_pass(aq, as_, W2, down, sid, eid, ntpp, numel, 1, tw, E)
            else:
                K.moe_gemm(aq, as_, W2, down, sid, eid, ntpp, numel, 1, tw, num_experts=E, MT=mt, prefill=pfd,
                           fuse=2 if fused else 0)
        K.moe_sum(down.view(M, topk, N2), None, output)
        return output
