"""MoE routing in one launch at decode widths (libr9k r9k_moe_route): softmax top-k, renormalisation and the
moe_align_block_size tables together. Mirrors the reference's r9700_vllm/moe/route.py (same names and contract).

The router (``R9kTopKRouter``, a ``FusedTopKRouter`` whose ``_compute_routing`` runs ``torch.ops.r9700.moe_route``)
leaves the tables on the ``RoutedExperts`` object it shares with ``R9700Mxfp4Experts``, whose apply() then skips its
own align. Rows above ``MAX_ROWS`` take the top-k kernel plus the multi-workgroup align instead.

Numerics: fp32 softmax; ids ordered by logit (the probability order), ties to the lower expert index; weights
p / sum (renorm over the selection). The tables are in canonical order (rows ascending within each expert).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import torch

from .._compat import get_logger, register_custom_op
from ..kernels import moe as KM

logger = get_logger(__name__)

MAX_ROWS = int(os.environ.get("R9K_MOE_ROUTE_MAX_ROWS", "256"))
_L = None
_DONE = False
_LIB = torch.library.Library("r9700", "FRAGMENT")


def lib():
    global _L
    if _L is None:
        L = KM.lib()
        if not hasattr(L, "r9k_moe_route"):
            raise RuntimeError("libr9k.so has no r9k_moe_route (rebuild r9700-stack_amd)")
        L.r9k_moe_route.restype = ctypes.c_int
        L.r9k_moe_route.argtypes = [ctypes.c_long, ctypes.c_int] + [ctypes.c_long] * 6 + [ctypes.c_int] * 5 \
            + [ctypes.c_long]
        L.r9k_moe_route_quant.restype = ctypes.c_int
        L.r9k_moe_route_quant.argtypes = [ctypes.c_long, ctypes.c_int] + [ctypes.c_long] * 6 + [ctypes.c_int] * 5 \
            + [ctypes.c_long, ctypes.c_long, ctypes.c_int, ctypes.c_long, ctypes.c_long, ctypes.c_long]
        L.r9k_moe_route_max_experts.restype = ctypes.c_int
        L.r9k_moe_route_max_topk.restype = ctypes.c_int
        _L = L
    return _L


def available() -> bool:
    try:
        lib()
        return True
    except Exception:
        return False


def capacity(numel: int, num_experts: int, blk: int) -> int:
    """sorted_ids length for `numel` routed rows, as moe_align_block_size sizes it."""
    return KM.capacity(numel, num_experts, blk)


def scratch_ints(E: int) -> int:
    """int32 count of the routing scratch of the reference contract (counts[E], cursor[E], arrive), zeroed once by
    the caller. The gfx950 kernel keeps counts and cursors in LDS and uses only the first int, the workgroups'
    arrival counter, which it leaves zero; the size is kept so callers allocate as before."""
    return 2 * E + 1


def moe_route(logits: torch.Tensor, topk: int, renorm: bool, blk: int, sorted_ids: torch.Tensor,
              expert_ids: torch.Tensor, ntpp: torch.Tensor, scratch: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """logits [M, E] bf16 -> (weights fp32 [M, topk], ids int32 [M, topk]); fills the first capacity(M*topk)
    entries of sorted_ids / expert_ids and ntpp[0]."""
    M, E = logits.shape
    w = torch.empty((M, topk), dtype=torch.float32, device=logits.device)
    ids = torch.empty((M, topk), dtype=torch.int32, device=logits.device)
    rc = lib().r9k_moe_route(logits.data_ptr(), logits.stride(0), w.data_ptr(), ids.data_ptr(),
                             sorted_ids.data_ptr(), expert_ids.data_ptr(), ntpp.data_ptr(), scratch.data_ptr(),
                             M, E, topk, 1 if renorm else 0, blk, torch.cuda.current_stream().cuda_stream)
    if rc:
        raise RuntimeError(f"r9k_moe_route failed ({rc}) M={M} E={E} topk={topk} blk={blk}")
    return w, ids


def _moe_route_fake(logits: torch.Tensor, topk: int, renorm: bool, blk: int, sorted_ids: torch.Tensor,
                    expert_ids: torch.Tensor, ntpp: torch.Tensor, scratch: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    M = logits.shape[0]
    return (logits.new_empty((M, topk), dtype=torch.float32), logits.new_empty((M, topk), dtype=torch.int32))


def moe_route_quant(logits: torch.Tensor, topk: int, renorm: bool, blk: int, sorted_ids: torch.Tensor,
                    expert_ids: torch.Tensor, ntpp: torch.Tensor, scratch: torch.Tensor,
                    x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """moe_route plus the per-token fp8 quant of the layer input x bf16 [M, H] (the bytes of quant_rows_fp8):
    (weights, ids, xq e4m3fn [M, H], xs fp32 [M]). One launch (r9k_moe_route_quant) at decode widths; other shapes
    run moe_route and quant_rows_fp8."""
    M, E = logits.shape
    if not (x.dim() == 2 and x.dtype == torch.bfloat16 and x.stride(1) == 1 and x.shape[0] == M):
        raise ValueError("moe_route_quant: x must be bf16 [M, H] with unit column stride")
    H = x.shape[1]
    w = torch.empty((M, topk), dtype=torch.float32, device=logits.device)
    ids = torch.empty((M, topk), dtype=torch.int32, device=logits.device)
    xq = torch.empty((M, H), dtype=torch.float8_e4m3fn, device=x.device)
    xs = torch.empty((M,), dtype=torch.float32, device=x.device)
    rc = lib().r9k_moe_route_quant(logits.data_ptr(), logits.stride(0), w.data_ptr(), ids.data_ptr(),
                                   sorted_ids.data_ptr(), expert_ids.data_ptr(), ntpp.data_ptr(),
                                   scratch.data_ptr(), M, E, topk,
                                   1 if renorm else 0, blk, x.data_ptr(), x.stride(0), H, xq.data_ptr(),
                                   xs.data_ptr(), torch.cuda.current_stream().cuda_stream)
    if rc == 2:
        w, ids = moe_route(logits, topk, renorm, blk, sorted_ids, expert_ids, ntpp, scratch)
        xq, xs = KM.quant_rows_fp8(x)
        return w, ids, xq, xs
    if rc:
        raise RuntimeError(f"r9k_moe_route_quant failed ({rc}) M={M} E={E} topk={topk} blk={blk} H={H}")
    return w, ids, xq, xs


def _moe_route_quant_fake(logits: torch.Tensor, topk: int, renorm: bool, blk: int, sorted_ids: torch.Tensor,
                          expert_ids: torch.Tensor, ntpp: torch.Tensor, scratch: torch.Tensor,
                          x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    M = logits.shape[0]
    return (logits.new_empty((M, topk), dtype=torch.float32), logits.new_empty((M, topk), dtype=torch.int32),
            x.new_empty(x.shape, dtype=torch.float8_e4m3fn), x.new_empty((M,), dtype=torch.float32))


def register() -> None:
    global _DONE
    if _DONE:
        return
    register_custom_op(_LIB, "moe_route", moe_route, ["sorted_ids", "expert_ids", "ntpp", "scratch"],
                       _moe_route_fake)
    register_custom_op(_LIB, "moe_route_quant", moe_route_quant, ["sorted_ids", "expert_ids", "ntpp", "scratch"],
                       _moe_route_quant_fake)
    _DONE = True


@dataclass
class Tables:
    """Routing tables for one call, keyed by the topk_ids tensor the router returned with them (at prefill widths
    only the activation quant: sorted_ids / expert_ids / ntpp None, and the experts build the tables)."""
    ids: torch.Tensor
    sorted_ids: torch.Tensor | None
    expert_ids: torch.Tensor | None
    ntpp: torch.Tensor | None
    blk: int
    numel: int
    x: torch.Tensor | None = None          # the layer input the router quantised, with its version at that time
    x_version: int = -1
    xq: torch.Tensor | None = None
    xs: torch.Tensor | None = None

    def matches(self, topk_ids: torch.Tensor, blk: int, numel: int) -> bool:
        return (self.sorted_ids is not None and self.ids.data_ptr() == topk_ids.data_ptr()
                and self.ids.shape == topk_ids.shape and self.blk == blk and self.numel == numel)

    def quant_for(self, x: torch.Tensor):
        """(xq, xs) when the router quantised this very tensor, unmodified since; else None."""
        if self.xq is None or self.x is not x or x._version != self.x_version:
            return None
        return self.xq, self.xs


def _fits(logits: torch.Tensor, topk: int, E: int) -> bool:
    L = lib()
    return (logits.dim() == 2 and logits.dtype == torch.bfloat16 and logits.stride(1) == 1
            and 1 <= logits.shape[0] <= MAX_ROWS and logits.shape[1] == E and E <= L.r9k_moe_route_max_experts()
            and 1 <= topk <= min(E, L.r9k_moe_route_max_topk()))


def _fits_wide(logits: torch.Tensor, topk: int, E: int, x) -> bool:
    """Rows above MAX_ROWS whose top-k and activation quant can share one launch (r9k_moe_topk_quant)."""
    L = lib()
    return (logits.dim() == 2 and logits.dtype == torch.bfloat16 and logits.stride(1) == 1
            and logits.shape[0] > MAX_ROWS and logits.shape[1] == E and E <= L.r9k_moe_route_max_experts()
            and 1 <= topk <= min(E, L.r9k_moe_route_max_topk()) and isinstance(x, torch.Tensor)
            and x.dim() == 2 and x.shape[0] == logits.shape[0])


def make_router(stock, routed_experts):
    """An R9kTopKRouter standing in for a stock FusedTopKRouter (softmax scoring, no EPLB). Needs vLLM."""
    from vllm.model_executor.layers.fused_moe.router.fused_topk_router import FusedTopKRouter

    class R9kTopKRouter(FusedTopKRouter):
        def __init__(self):
            super().__init__(top_k=stock.top_k, global_num_experts=stock.global_num_experts,
                             scoring_func=stock.scoring_func, renormalize=stock.renormalize,
                             eplb_state=stock.eplb_state)
            self.capture_fn = getattr(stock, "capture_fn", None)
            self._routing_replay_out = getattr(stock, "_routing_replay_out", None)
            self.routed_experts = routed_experts
            self._bufs: dict = {}
            # allocate at construction, outside any graph-capture memory-profiling pass
            if torch.cuda.is_available():
                self._buffers(torch.device("cuda", torch.cuda.current_device()), stock.global_num_experts)

        def _buffers(self, device: torch.device, E: int):
            b = self._bufs.get(device)
            if b is None:
                cap = max(capacity(m * self.top_k, E, 16 * KM.pick_mt(m * self.top_k, E))
                          for m in range(1, MAX_ROWS + 1))
                b = (torch.empty(cap, dtype=torch.int32, device=device),
                     torch.empty(cap // 16, dtype=torch.int32, device=device),
                     torch.zeros(1, dtype=torch.int32, device=device),
                     torch.zeros(scratch_ints(E), dtype=torch.int32, device=device))
                self._bufs[device] = b
            return b

        def _compute_routing(self, hidden_states, router_logits, indices_type, *, input_ids=None):
            E = self.global_num_experts
            if indices_type in (None, torch.int32) and _fits_wide(router_logits, self.top_k, E, hidden_states):
                # prefill widths: top-k and the experts' fp8 input quant in one launch; the experts build the
                # tables (multi-workgroup align) and take the quant from here (Tables.quant_for)
                r = KM.moe_topk_quant(router_logits, self.top_k, self.renormalize, hidden_states)
                if r is not None:
                    w, ids, xq, xs = r
                    self.routed_experts._r9k_tables = Tables(ids, None, None, None, -1, ids.numel(), hidden_states,
                                                             hidden_states._version, xq, xs)
                    return w, ids
            if indices_type not in (None, torch.int32) or not _fits(router_logits, self.top_k, E):
                self.routed_experts._r9k_tables = None
                return super()._compute_routing(hidden_states, router_logits, indices_type, input_ids=input_ids)
            M = router_logits.shape[0]
            numel = M * self.top_k
            blk = KM.MOE_BLOCK * KM.pick_mt(numel, E)
            sorted_ids, expert_ids, ntpp, scratch = self._buffers(router_logits.device, E)
            if _quantisable(hidden_states, M):
                # the experts' fp8 input quant rides along in the routing launch (Tables.quant_for hands it over)
                w, ids, xq, xs = torch.ops.r9700.moe_route_quant(router_logits, self.top_k, self.renormalize, blk,
                                                                 sorted_ids, expert_ids, ntpp, scratch,
                                                                 hidden_states)
                self.routed_experts._r9k_tables = Tables(ids, sorted_ids, expert_ids, ntpp, blk, numel,
                                                         hidden_states, hidden_states._version, xq, xs)
                return w, ids
            w, ids = torch.ops.r9700.moe_route(router_logits, self.top_k, self.renormalize, blk, sorted_ids,
                                               expert_ids, ntpp, scratch)
            self.routed_experts._r9k_tables = Tables(ids, sorted_ids, expert_ids, ntpp, blk, numel)
            return w, ids

    return R9kTopKRouter()


def take(layer, topk_ids: torch.Tensor, blk: int, numel: int):
    """The tables the router left for this call on the RoutedExperts `layer`, or None."""
    t = getattr(layer, "_r9k_tables", None)
    if t is None or not t.matches(topk_ids, blk, numel):
        return None
    return t.sorted_ids, t.expert_ids, t.ntpp


def take_quant(layer, topk_ids: torch.Tensor, x: torch.Tensor):
    """The (xq, xs) fp8 quant of `x` the router produced with this call's tables, or None."""
    t = getattr(layer, "_r9k_tables", None)
    if t is None or t.ids.data_ptr() != topk_ids.data_ptr():
        return None
    return t.quant_for(x)


def _quantisable(x, M: int) -> bool:
    """A layer input the routing launch can quantise (decode widths; the kernel checks the rest)."""
    return (isinstance(x, torch.Tensor) and x.dim() == 2 and x.dtype == torch.bfloat16 and x.shape[0] == M
            and x.is_contiguous() and M <= 64)


def install(model: torch.nn.Module) -> int:
    """Replace the router of every MoE runner under `model` that routes by plain softmax top-k.
    R9K_MOE_ROUTE=stock skips."""
    if os.environ.get("R9K_MOE_ROUTE", "stock") != "r9k" or not available():
        return 0
    register()
    n = 0
    for name, mod in model.named_modules():
        router = getattr(mod, "router", None)
        re_ = getattr(mod, "routed_experts", None)
        if router is None or re_ is None or type(router).__name__ != "FusedTopKRouter":
            continue
        if getattr(router, "scoring_func", None) != "softmax" or getattr(router, "eplb_state", None) is not None:
            logger.warning("r9700: fused MoE routing skipped for %s", name)
            continue
        mod.router = make_router(router, re_)
        n += 1
    if n:
        logger.info("r9700: fused MoE routing (softmax top-k + align in one launch, <= %d rows) on %d runners",
                    MAX_ROWS, n)
    return n
