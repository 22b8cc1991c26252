"""MoE routing on libr9k at decode widths: softmax top-k, renormalisation and the moe_align_block_size tables (and,
up to 64 rows, the experts' fp8 input quant) in one launch, handed to the experts' apply() through the layer
object router and experts share. The role and names of the reference's r9700_vllm/moe/route.py (`moe_route`, the
`R9kTopKRouter` made by `make_router`, `install`, `capacity`, `scratch_ints`).

How a call is routed (`plan_route`, then `route_step`, both vLLM-free):
  * "decode"  1..MAX_ROWS rows: r9k_moe_route (or r9k_moe_route_quant, which also quantises the layer input) on the
              router's persistent table buffers (`RouteBuffers`), so the experts skip their align;
  * "wide"    more rows, or any step whose experts split their tables by expert size themselves (`split_planned`):
              r9k_moe_topk_quant (top-k and the input quant in one launch); the experts build the tables;
  * "stock"   anything the kernels do not take (other index dtypes, too many experts or top-k): vLLM's router.
The hand-off is a `Tables` record on the layer, keyed by the ids tensor the router returned, so apply() uses it
only for the very call it was made for (`take`, `take_quant`).

Numerics: fp32 softmax; ids in probability order (the bf16 logit order), ties to the lower expert index; weights
p / sum over the selection. Tables in canonical order (experts ascending, rows ascending within an expert).
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
QUANT_MAX_NUMEL = 4096              # routed rows (M * topk) r9k_moe_route_quant and _dual take in one launch
_LIB = torch.library.Library("r9700", "FRAGMENT")
_bound = None
_registered = False


def lib() -> ctypes.CDLL:
    """libr9k with the routing entries' signatures set (RuntimeError when the library lacks them)."""
    global _bound
    if _bound is None:
        L = KM.lib()
        if not hasattr(L, "r9k_moe_route"):
            raise RuntimeError("libr9k.so has no r9k_moe_route (rebuild r9700-stack_amd)")
        i, l = ctypes.c_int, ctypes.c_long
        common = [l, i] + [l] * 6 + [i] * 5          # logits, ldl, w, ids, sorted, expert_ids, ntpp, scratch, M..blk
        L.r9k_moe_route.argtypes, L.r9k_moe_route.restype = common + [l], i
        L.r9k_moe_route_quant.argtypes = common + [l, l, i, l, l, l]
        L.r9k_moe_route_quant.restype = i
        L.r9k_moe_route_dual.argtypes = common + [l, l, i, l, l, i, l, l, l, i, l]
        L.r9k_moe_route_dual.restype = i
        L.r9k_moe_route_max_experts.restype = i
        L.r9k_moe_route_max_topk.restype = i
        _bound = L
    return _bound


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
    """int32 count of the routing scratch a caller allocates (zeroed once) -- the reference contract's size
    (counts[E], cursor[E], arrival). The gfx950 kernel keeps counts and cursors in LDS and uses the first int, its
    workgroups' arrival counter, which every call leaves zero."""
    return 2 * E + 1


def _launch(quant_x, logits, topk, renorm, blk, sorted_ids, expert_ids, ntpp, scratch):
    """One routing launch; with quant_x also the fp8 quant of that input. Returns (rc, w, ids, xq, xs)."""
    M, E = logits.shape
    dev = logits.device
    w = torch.empty((M, topk), dtype=torch.float32, device=dev)
    ids = torch.empty((M, topk), dtype=torch.int32, device=dev)
    head = (logits.data_ptr(), logits.stride(0), w.data_ptr(), ids.data_ptr(), sorted_ids.data_ptr(),
            expert_ids.data_ptr(), ntpp.data_ptr(), scratch.data_ptr(), M, E, topk, int(bool(renorm)), blk)
    st = torch.cuda.current_stream().cuda_stream
    if quant_x is None:
        return lib().r9k_moe_route(*head, st), w, ids, None, None
    H = quant_x.shape[1]
    xq = torch.empty((M, H), dtype=torch.float8_e4m3fn, device=dev)
    xs = torch.empty((M,), dtype=torch.float32, device=dev)
    rc = lib().r9k_moe_route_quant(*head, quant_x.data_ptr(), quant_x.stride(0), H, xq.data_ptr(), xs.data_ptr(), st)
    return rc, w, ids, xq, xs


def moe_route(logits: torch.Tensor, topk: int, renorm: bool, blk: int, sorted_ids: torch.Tensor,
              expert_ids: torch.Tensor, ntpp: torch.Tensor, scratch: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """logits [M, E] bf16 -> (weights fp32 [M, topk], ids int32 [M, topk]); fills the first capacity(M * topk) entries
    of sorted_ids / expert_ids and ntpp[0] (blocks of `blk` rows)."""
    rc, w, ids, _, _ = _launch(None, logits, topk, renorm, blk, sorted_ids, expert_ids, ntpp, scratch)
    if rc:
        raise RuntimeError(f"r9k_moe_route failed ({rc}) M={logits.shape[0]} E={logits.shape[1]} topk={topk} "
                           f"blk={blk}")
    return w, ids


def moe_route_quant(logits: torch.Tensor, topk: int, renorm: bool, blk: int, sorted_ids: torch.Tensor,
                    expert_ids: torch.Tensor, ntpp: torch.Tensor, scratch: torch.Tensor,
                    x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """moe_route plus the per-token fp8 quant of the layer input x bf16 [M, H] (quant_rows_fp8's bytes): (weights,
    ids, xq e4m3fn [M, H], xs fp32 [M]). One launch at decode widths; other shapes run moe_route + quant_rows_fp8."""
    M = logits.shape[0]
    if not (x.dim() == 2 and x.dtype == torch.bfloat16 and x.stride(1) == 1 and x.shape[0] == M):
        raise ValueError("moe_route_quant: x must be bf16 [M, H] with unit column stride")
    rc, w, ids, xq, xs = _launch(x, logits, topk, renorm, blk, sorted_ids, expert_ids, ntpp, scratch)
    if rc == 2:                                       # a shape the one-launch kernel does not take: nothing ran
        w, ids = moe_route(logits, topk, renorm, blk, sorted_ids, expert_ids, ntpp, scratch)
        xq, xs = KM.quant_rows_fp8(x)
    elif rc:
        raise RuntimeError(f"r9k_moe_route_quant failed ({rc}) M={M} E={logits.shape[1]} topk={topk} blk={blk} "
                           f"H={x.shape[1]}")
    return w, ids, xq, xs


def moe_route_dual(logits: torch.Tensor, topk: int, renorm: bool, blk: int, sorted_ids: torch.Tensor,
                   expert_ids: torch.Tensor, ntpp: torch.Tensor, scratch: torch.Tensor, x: torch.Tensor | None,
                   big_blk: int, sorted_big: torch.Tensor, expert_big: torch.Tensor, ntpp_big: torch.Tensor,
                   min_rows: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """moe_route(_quant) with the tables in two layouts -- blocks of blk rows and of big_blk rows (live entries) --
    of which the device keeps one (the big one when its blocks average >= min_rows rows; the other's ntpp is set
    to 0), in one launch (r9k_moe_route_dual). Returns (weights, ids, xq, xs); without x, xq and xs are empty.
    The caller keeps to the served shapes (dual_wanted, quant_suits): anything else raises."""
    M, E = logits.shape
    assert logits.dtype == torch.bfloat16 and logits.stride(1) == 1
    dev = logits.device
    w = torch.empty((M, topk), dtype=torch.float32, device=dev)
    ids = torch.empty((M, topk), dtype=torch.int32, device=dev)
    xq = torch.empty((0,), dtype=torch.float8_e4m3fn, device=dev)
    xs = torch.empty((0,), dtype=torch.float32, device=dev)
    xa = (0, 0, 0, 0, 0)
    if x is not None:
        if not (x.dim() == 2 and x.dtype == torch.bfloat16 and x.stride(1) == 1 and x.shape[0] == M):
            raise ValueError("moe_route_dual: x must be bf16 [M, H] with unit column stride")
        H = x.shape[1]
        xq = torch.empty((M, H), dtype=torch.float8_e4m3fn, device=dev)
        xs = torch.empty((M,), dtype=torch.float32, device=dev)
        xa = (x.data_ptr(), x.stride(0), H, xq.data_ptr(), xs.data_ptr())
    rc = lib().r9k_moe_route_dual(logits.data_ptr(), logits.stride(0), w.data_ptr(), ids.data_ptr(),
                                  sorted_ids.data_ptr(), expert_ids.data_ptr(), ntpp.data_ptr(), scratch.data_ptr(),
                                  M, E, topk, int(renorm), blk, *xa, big_blk, sorted_big.data_ptr(),
                                  expert_big.data_ptr(), ntpp_big.data_ptr(), min_rows,
                                  torch.cuda.current_stream().cuda_stream)
    if rc:
        raise RuntimeError(f"r9k_moe_route_dual failed ({rc}) M={M} E={E} topk={topk} blk={blk} big={big_blk}")
    return w, ids, xq, xs


def quant_suits(x: torch.Tensor) -> bool:
    """Rows the routing launch's wave quant takes: H % 8 == 0, H <= 4096, 16-byte aligned rows."""
    H = x.shape[1]
    return H % 8 == 0 and 8 <= H <= 4096 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0


def _moe_route_dual_fake(logits, topk: int, renorm: bool, blk: int, sorted_ids, expert_ids, ntpp, scratch, x,
                         big_blk: int, sorted_big, expert_big, ntpp_big, min_rows: int):
    M = logits.shape[0]
    dev = logits.device
    w, ids = _moe_route_fake(logits, topk, renorm, blk, sorted_ids, expert_ids, ntpp, scratch)
    if x is None:
        return (w, ids, torch.empty((0,), dtype=torch.float8_e4m3fn, device=dev),
                torch.empty((0,), dtype=torch.float32, device=dev))
    return (w, ids, torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=dev),
            torch.empty((M,), dtype=torch.float32, device=dev))


def _moe_route_fake(logits, topk: int, renorm: bool, blk: int, sorted_ids, expert_ids, ntpp, scratch):
    M = logits.shape[0]
    return (torch.empty((M, topk), dtype=torch.float32, device=logits.device),
            torch.empty((M, topk), dtype=torch.int32, device=logits.device))


def _moe_route_quant_fake(logits, topk: int, renorm: bool, blk: int, sorted_ids, expert_ids, ntpp, scratch, x):
    w, ids = _moe_route_fake(logits, topk, renorm, blk, sorted_ids, expert_ids, ntpp, scratch)
    return (w, ids, torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device),
            torch.empty((x.shape[0],), dtype=torch.float32, device=x.device))


def register() -> None:
    """torch.ops.r9700.moe_route / moe_route_quant (they mutate the table buffers and the scratch)."""
    global _registered
    if _registered:
        return
    mut = ["sorted_ids", "expert_ids", "ntpp", "scratch"]
    register_custom_op(_LIB, "moe_route", moe_route, mut, _moe_route_fake)
    register_custom_op(_LIB, "moe_route_quant", moe_route_quant, mut, _moe_route_quant_fake)
    register_custom_op(_LIB, "moe_route_dual", moe_route_dual, mut + ["sorted_big", "expert_big", "ntpp_big"],
                       _moe_route_dual_fake)
    _registered = True


@dataclass
class Tables:
    """What the router leaves on the layer for one call: its ids tensor (the key), the align tables (None when the
    experts build them: wide calls) and the fp8 quant of the input it routed with (with that tensor's version, so a
    modified input is never taken)."""
    ids: torch.Tensor
    sorted_ids: torch.Tensor | None
    expert_ids: torch.Tensor | None
    ntpp: torch.Tensor | None
    blk: int
    numel: int
    x: torch.Tensor | None = None
    x_version: int = -1
    xq: torch.Tensor | None = None
    xs: torch.Tensor | None = None
    big: tuple | None = None          # (sorted_ids, expert_ids, ntpp, big_blk): the second layout (moe_route_dual)

    def matches(self, topk_ids: torch.Tensor, blk: int, numel: int) -> bool:
        return (self.sorted_ids is not None and self.blk == blk and self.numel == numel
                and self.ids.data_ptr() == topk_ids.data_ptr() and self.ids.shape == topk_ids.shape)

    def quant_for(self, x: torch.Tensor):
        """(xq, xs) when the router quantised this very tensor, unmodified since; else None."""
        if self.xq is not None and self.x is x and x._version == self.x_version:
            return self.xq, self.xs
        return None


def take(layer, topk_ids: torch.Tensor, blk: int, numel: int):
    """The (sorted_ids, expert_ids, ntpp) the router left on `layer` for this call, or None."""
    t = getattr(layer, "_r9k_tables", None)
    return (t.sorted_ids, t.expert_ids, t.ntpp) if t is not None and t.matches(topk_ids, blk, numel) else None


def take_big(layer, topk_ids: torch.Tensor, blk: int, numel: int):
    """The second table layout (sorted_ids, expert_ids, ntpp, big_blk) the router built for this call, of which the
    device kept one (the small layout's tables, take(), carry the other ntpp), or None. A caller that takes the
    small tables of a call with a second layout must run both layouts' GEMMs."""
    t = getattr(layer, "_r9k_tables", None)
    return t.big if t is not None and t.big is not None and t.matches(topk_ids, blk, numel) else None


def split_planned(layer, numel: int, E: int) -> bool:
    """Whether the experts of `layer` split the tables of a call of `numel` routed rows by expert size themselves
    (kernels.moe.split_wanted with the widths they signalled in `_r9k_split_k`): the router then builds no tables
    and takes the wide path (top-k and the input quant in one launch)."""
    ks = getattr(layer, "_r9k_split_k", None) if layer is not None else None
    return ks is not None and KM.split_wanted(numel, E, *ks)


def dual_wanted(layer, numel: int, E: int) -> int:
    """The big block size when the router should build both layouts for a call of `numel` routed rows: the experts
    of `layer` signalled they run the device-picked pair (their `_r9k_dual_blk`) and do not split the step's tables
    (split_planned), the step has at least DEVICE_BLOCKS_MIN rows and the host would keep small blocks (touched
    experts average below PREFILL_MOE_ROWS); else 0."""
    if split_planned(layer, numel, E):
        return 0
    bb = getattr(layer, "_r9k_dual_blk", 0) if layer is not None else 0
    if not bb or KM.DEVICE_BLOCKS_MIN <= 0 or numel < KM.DEVICE_BLOCKS_MIN or numel > QUANT_MAX_NUMEL:
        return 0
    return bb if numel / max(1, min(E, numel)) < KM.PREFILL_MOE_ROWS else 0


def take_quant(layer, topk_ids: torch.Tensor, x: torch.Tensor):
    """The (xq, xs) fp8 quant of `x` the router made with this call's ids, or None."""
    t = getattr(layer, "_r9k_tables", None)
    if t is None or t.ids.data_ptr() != topk_ids.data_ptr():
        return None
    return t.quant_for(x)


class RouteBuffers:
    """The router's persistent table buffers on one device, sized for MAX_ROWS rows at the largest block the
    decode path uses, plus the zero-once routing scratch. Allocated once (outside graph capture) and reused by every
    call, so captured graphs keep valid addresses."""

    def __init__(self, device: torch.device, E: int, topk: int, big_blk: int = 256):
        cap = max(capacity(m * topk, E, KM.MOE_BLOCK * KM.pick_mt(m * topk, E)) for m in range(1, MAX_ROWS + 1))
        i32 = dict(dtype=torch.int32, device=device)
        self.sorted_ids = torch.empty(cap, **i32)
        self.expert_ids = torch.empty(cap // KM.MOE_BLOCK, **i32)
        self.ntpp = torch.zeros(1, **i32)
        self.scratch = torch.zeros(scratch_ints(E), **i32)
        # the second (big-block) layout of moe_route_dual: live entries only, so sized by the routed rows
        capb = capacity(min(MAX_ROWS * topk, QUANT_MAX_NUMEL), E, big_blk)
        self.big_blk = big_blk
        self.sorted_big = torch.empty(capb, **i32)
        self.expert_big = torch.empty(capb // big_blk, **i32)
        self.ntpp_big = torch.zeros(1, **i32)


def plan_route(logits: torch.Tensor, topk: int, E: int, x, indices_type=None) -> str:
    """'decode', 'wide' or 'stock' for one router call (see the module docstring)."""
    if indices_type not in (None, torch.int32):
        return "stock"
    L = lib()
    if not (logits.dim() == 2 and logits.dtype == torch.bfloat16 and logits.stride(1) == 1
            and logits.shape[1] == E and E <= L.r9k_moe_route_max_experts()
            and 1 <= topk <= min(E, L.r9k_moe_route_max_topk())):
        return "stock"
    M = logits.shape[0]
    if 1 <= M <= MAX_ROWS:
        return "decode"
    if M > MAX_ROWS and isinstance(x, torch.Tensor) and x.dim() == 2 and x.shape[0] == M:
        return "wide"
    return "stock"


def _quantisable(x, M: int, topk: int) -> bool:
    """A layer input the decode routing launch can quantise alongside (the kernel checks its alignment)."""
    return (isinstance(x, torch.Tensor) and x.dim() == 2 and x.dtype == torch.bfloat16 and x.shape[0] == M
            and x.is_contiguous() and M * topk <= QUANT_MAX_NUMEL)


def route_step(logits: torch.Tensor, x, topk: int, renorm: bool, E: int, bufs: RouteBuffers | None,
               indices_type=None, use_ops: bool = True, dual_blk: int = 0, wide: bool = False):
    """Route one call: (weights, ids, Tables) on the decode / wide paths, or None when the stock router must run.
    At decode widths `bufs` holds the tables; use_ops routes the launch through the torch.ops.r9700 custom ops
    (the compiled-graph path), else the plain functions. dual_blk (dual_wanted): also the big-block layout, of which
    the device keeps one (moe_route_dual). wide (split_planned): the wide path at any width (no tables)."""
    path = plan_route(logits, topk, E, x, indices_type)
    if path == "stock":
        return None
    if wide:
        path = "wide"
    M = logits.shape[0]
    numel = M * topk
    if path == "wide":
        r = KM.moe_topk_quant(logits, topk, renorm, x)
        if r is None:
            return None
        w, ids, xq, xs = r
        return w, ids, Tables(ids, None, None, None, -1, numel, x, x._version, xq, xs)
    blk = KM.MOE_BLOCK * KM.pick_mt(numel, E)
    args = (logits, topk, renorm, blk, bufs.sorted_ids, bufs.expert_ids, bufs.ntpp, bufs.scratch)
    if use_ops:
        register()
    if dual_blk and dual_blk == bufs.big_blk and numel <= QUANT_MAX_NUMEL:
        xd = x if _quantisable(x, M, topk) and quant_suits(x) else None
        fn = torch.ops.r9700.moe_route_dual if use_ops else moe_route_dual
        w, ids, xq, xs = fn(*args, xd, dual_blk, bufs.sorted_big, bufs.expert_big, bufs.ntpp_big,
                            KM.DEVICE_MIN_ROWS)
        big = (bufs.sorted_big, bufs.expert_big, bufs.ntpp_big, dual_blk)
        if xd is None:
            return w, ids, Tables(ids, bufs.sorted_ids, bufs.expert_ids, bufs.ntpp, blk, numel, big=big)
        return w, ids, Tables(ids, bufs.sorted_ids, bufs.expert_ids, bufs.ntpp, blk, numel, x, x._version, xq, xs,
                              big=big)
    if _quantisable(x, M, topk):
        fn = torch.ops.r9700.moe_route_quant if use_ops else moe_route_quant
        w, ids, xq, xs = fn(*args, x)
        return w, ids, Tables(ids, bufs.sorted_ids, bufs.expert_ids, bufs.ntpp, blk, numel, x, x._version, xq, xs)
    fn = torch.ops.r9700.moe_route if use_ops else moe_route
    w, ids = fn(*args)
    return w, ids, Tables(ids, bufs.sorted_ids, bufs.expert_ids, bufs.ntpp, blk, numel)


def make_router(stock, routed_experts):
    """An R9kTopKRouter in place of a stock FusedTopKRouter (softmax scoring, no EPLB), sharing `routed_experts`
    (the layer apply() reads the hand-off from). Needs vLLM."""
    from vllm.model_executor.layers.fused_moe.router.fused_topk_router import FusedTopKRouter

    class R9kTopKRouter(FusedTopKRouter):
        def __init__(self):
            super().__init__(top_k=stock.top_k, global_num_experts=stock.global_num_experts,
                             scoring_func=stock.scoring_func, renormalize=stock.renormalize,
                             eplb_state=stock.eplb_state)
            for attr in ("capture_fn", "_routing_replay_out"):
                setattr(self, attr, getattr(stock, attr, None))
            self.routed_experts = routed_experts
            self._r9k_bufs: dict = {}
            if torch.cuda.is_available():               # allocate now, outside any capture / profiling pass
                self._bufs_for(torch.device("cuda", torch.cuda.current_device()))

        def _bufs_for(self, device):
            b = self._r9k_bufs.get(device)
            if b is None:
                b = self._r9k_bufs[device] = RouteBuffers(device, self.global_num_experts, self.top_k)
            return b

        def _compute_routing(self, hidden_states, router_logits, indices_type, *, input_ids=None):
            numel = router_logits.shape[0] * self.top_k
            E = self.global_num_experts
            r = route_step(router_logits, hidden_states, self.top_k, self.renormalize, E,
                           self._bufs_for(router_logits.device), indices_type,
                           dual_blk=dual_wanted(self.routed_experts, numel, E),
                           wide=split_planned(self.routed_experts, numel, E))
            if r is None:
                self.routed_experts._r9k_tables = None
                return super()._compute_routing(hidden_states, router_logits, indices_type, input_ids=input_ids)
            w, ids, self.routed_experts._r9k_tables = r
            return w, ids

    return R9kTopKRouter()


def _router_refusal(router) -> str | None:
    if type(router).__name__ != "FusedTopKRouter":
        return "not a FusedTopKRouter"
    if getattr(router, "scoring_func", None) != "softmax":
        return "scoring is not softmax"
    if getattr(router, "eplb_state", None) is not None:
        return "expert load balancing is on"
    return None


def install(model: torch.nn.Module) -> int:
    """Swap in R9kTopKRouter on every MoE runner under `model` (a module with `router` and `routed_experts`) whose
    router is plain softmax top-k; returns how many. Opt-in: R9K_MOE_ROUTE=r9k (the reference's default is stock)."""
    if os.environ.get("R9K_MOE_ROUTE", "stock") != "r9k" or not available():
        return 0
    register()
    swapped = 0
    for name, mod in model.named_modules():
        router, experts = getattr(mod, "router", None), getattr(mod, "routed_experts", None)
        if router is None or experts is None:
            continue
        why = _router_refusal(router)
        if why is not None:
            if type(router).__name__ == "FusedTopKRouter":
                logger.warning("r9700: fused MoE routing skipped for %s (%s)", name, why)
            continue
        mod.router = make_router(router, experts)
        swapped += 1
    if swapped:
        logger.info("r9700: fused MoE routing (top-k + tables in one launch up to %d rows) on %d runners", MAX_ROWS,
                    swapped)
    return swapped
