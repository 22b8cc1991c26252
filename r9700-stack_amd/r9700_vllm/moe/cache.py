"""Per-layer device-side LRU expert cache over mapped pinned host memory (reference r9700_vllm/moe/cache.py:1-414).

Every routed expert of a cached layer lives in mapped pinned host memory (`uva_empty`: hipHostMalloc, the device
address equals the host address): the fragment-order weights w13 / w2 and the packed scales s13 / s2 are the
backing store. A VRAM arena of S slots per layer holds a changing subset. Each forward, before the GEMMs,
`r4d_lru_manage` (csrc/r9k_expert_cache.hip) refreshes the resident experts routed this step, picks victims among
the slots not routed this step (least recently routed first, ties to the lower slot: deterministic, so ranks that
see the same routing agree), rewrites `table` / `map_cold` and emits a miss list, and `r4d_lru_gather` copies the
missed experts host -> slot. The GEMMs then run twice: over the arena with the routing ids mapped through `table`
(expert -> slot) and over the host store with them mapped through `map_cold` (expert -> itself when not resident);
the second pass is empty unless the step read through (more distinct experts than the threshold, or the insert cap
was hit). Everything is device work on fixed addresses, so a captured HIP graph replays it.

Config (per process, the reference's names): R9K_EXPERT_CACHE_GB (0 = off), R9K_EXPERT_CACHE_SLOTS,
R9K_EXPERT_CACHE_LAYERS, R9K_LRU_THRESH (0.99: a step routing to more distinct experts than this share of the slots
inserts nothing and reads every non-resident expert through from host), R9K_LRU_MAX_INSERTS (64),
R9K_LRU_GATHER="chunks,lanes" (64,16), R9K_LRU_FUSED (1), R9K_EXPERT_CACHE_HOST_ONLY (1), R9K_EXPERT_CACHE_STATS.
Warm start: the checkpoint's model-expertprofile.safetensors (expert_routing_counts [layers, experts]) when vLLM
names a model directory holding one, else experts 0..S-1.

On gfx950 the cold pass reads weights over PCIe inside the GEMM (the decode kernels read every weight byte once per
routing block). R9K_STAGE_COLD (the reference's opt-in bulk staging of cold experts, recorded there as without a
measured gain) is not built: `staging_enabled()` is always False.
"""
from __future__ import annotations

import ctypes
import logging
import os

import numpy as np
import torch

from ..kernels import moe as K

logger = logging.getLogger("vllm." + __name__)

_BOUND = False
_PROFILE: torch.Tensor | None = None
_PROFILE_LOADED = False
_HOST_BUFFERS: list = []          # (pointer, bytes) of every mapped host buffer: held until the process ends
HOST_COPY_BYTES = 512 << 20       # largest single device -> host transfer of to_host


def _L():
    global _BOUND
    L = K.lib()
    if not _BOUND:
        i, l = ctypes.c_int, ctypes.c_long
        L.r4d_lru_manage.restype = i
        L.r4d_lru_manage.argtypes = [l, i, i, i, i, i] + [l] * 8 + [l]
        L.r4d_lru_gather.restype = i
        L.r4d_lru_gather.argtypes = [l, l, l] * 6 + [l, l, i, i, l]
        L.r9k_lru_manage_map.restype = i
        L.r9k_lru_manage_map.argtypes = [l, i, i, i, i, i] + [l] * 10 + [l]
        L.r9k_lru_map_ids.restype = i
        L.r9k_lru_map_ids.argtypes = [l, i, i, l, l, l, l, l]
        L.r9k_lru_manage_tables.restype = i
        L.r9k_lru_manage_tables.argtypes = [l, i, i, i, i, i] + [l] * 8 + [i] + [l] * 7 + [l]
        L.r4d_lru_fused.restype = i
        L.r4d_lru_fused.argtypes = [l, i, i, i, i, i] + [l] * 8 + [i, i, i] + [l] * 6 + [l]
        L.r9k_lru_stage_map.restype = i
        L.r9k_lru_stage_map.argtypes = [l, i, i, l, i, l, l, l, l]
        L.r9k_host_alloc.restype = l
        L.r9k_host_alloc.argtypes = [l]
        L.r9k_host_free.restype = i
        L.r9k_host_free.argtypes = [l]
        _BOUND = True
    return L


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def uva_empty(shape, dtype) -> torch.Tensor:
    """A CPU tensor over fresh mapped pinned host memory whose address kernels can read (r9k_host_alloc checks that
    the device address is the host address). Marked `_r9k_host`; held until the process ends."""
    shape = tuple(int(x) for x in shape)
    itemsize = torch.empty((), dtype=dtype).element_size()
    nbytes = max(16, int(np.prod(shape, dtype=np.int64)) * itemsize)
    nbytes = (nbytes + 255) // 256 * 256
    ptr = _L().r9k_host_alloc(nbytes)
    if not ptr:
        raise RuntimeError(f"r9k_host_alloc({nbytes}) failed: no mapped pinned host memory")
    _HOST_BUFFERS.append((ptr, nbytes))
    buf = (ctypes.c_uint8 * nbytes).from_address(ptr)
    n = int(np.prod(shape, dtype=np.int64)) * itemsize
    t = torch.from_numpy(np.frombuffer(buf, dtype=np.uint8, count=n)).view(dtype).view(shape)
    t._r9k_host = ptr
    return t


def is_host(t: torch.Tensor) -> bool:
    """True for a tensor in mapped host memory made by uva_empty (or marked by vLLM's UVA offloader)."""
    return bool(getattr(t, "_vllm_is_uva_offloaded", False) or getattr(t, "_r9k_host", None) is not None)


def to_host(t: torch.Tensor) -> torch.Tensor:
    """A mapped host copy of `t` (uva_empty). The destination is pinned, so each copy is one DMA; a device source is
    copied a slab of whole experts (dim-0 slices) at a time so no single transfer exceeds HOST_COPY_BYTES."""
    h = uva_empty(t.shape, t.dtype)
    per = max(1, t[0].numel() * t.element_size()) if t.dim() and t.shape[0] else 1
    rows = max(1, HOST_COPY_BYTES // per)
    for lo in range(0, t.shape[0] if t.dim() else 1, rows):
        h[lo:lo + rows].copy_(t[lo:lo + rows])
    return h


def budget_gb() -> float:
    return float(os.environ.get("R9K_EXPERT_CACHE_GB", "0") or 0)


def _profile() -> torch.Tensor | None:
    global _PROFILE, _PROFILE_LOADED
    if _PROFILE_LOADED:
        return _PROFILE
    _PROFILE_LOADED = True
    try:
        from vllm.config import get_current_vllm_config
        from safetensors.torch import load_file
        p = os.path.join(get_current_vllm_config().model_config.model, "model-expertprofile.safetensors")
        if os.path.isfile(p):
            _PROFILE = load_file(p)["expert_routing_counts"].float()
            logger.info("r9700: expert routing profile %s %s", p, tuple(_PROFILE.shape))
    except Exception as e:                       # no vLLM config or no profile: cold start from experts 0..S-1
        logger.debug("r9700: no expert routing profile (%s)", e)
    return _PROFILE


def _num_moe_layers() -> int:
    try:
        from vllm.config import get_current_vllm_config
        hf = get_current_vllm_config().model_config.hf_text_config
        return int(getattr(hf, "num_hidden_layers"))
    except Exception:
        return 48


def staging_enabled() -> bool:
    """R9K_STAGE_COLD=1 (opt-in, as in the reference): a step that needs the cold pass first copies every routed
    expert that is not resident into a VRAM staging area with one bulk gather, and the cold pass reads it there
    instead of reading host memory inside the GEMMs (once per routing block)."""
    return os.environ.get("R9K_STAGE_COLD", "0") == "1"


_STAGE_AREAS: dict = {}


def _stage_area(dev: torch.device, cap: int, store) -> tuple:
    """The staging slabs (w13, w2, s13, s2) for `cap` experts, shaped like the host store's, one set per device and
    shape: layers run one after another on one stream, so every cached layer of a model shares it."""
    key = (dev.index, cap) + tuple((tuple(h.shape[1:]), h.dtype) for h in store)
    area = _STAGE_AREAS.get(key)
    if area is None:
        area = _STAGE_AREAS[key] = tuple(torch.empty((cap, *h.shape[1:]), dtype=h.dtype, device=dev) for h in store)
    return area


def stats_enabled() -> bool:
    return os.environ.get("R9K_EXPERT_CACHE_STATS", "0") == "1"


STAT_FIELDS = ("steps", "distinct", "inserts", "read_through", "wide")


class _StatsReporter:
    """Per-layer cache counters (each cached layer's device tensor `stats`, STAT_FIELDS) and one daemon thread that
    logs the change over every R9K_EXPERT_CACHE_STATS_SEC seconds (0 = no thread). A reporter that fails stops
    itself: a diagnostic never takes the worker down."""

    def __init__(self):
        self.layers: list = []
        self.thread = None

    def add(self, cache) -> None:
        self.layers.append(cache)
        period = float(os.environ.get("R9K_EXPERT_CACHE_STATS_SEC", "10") or 0)
        if self.thread is None and period > 0:
            import threading
            self.thread = threading.Thread(target=self._run, args=(period,), name="r9k-cache-stats", daemon=True)
            self.thread.start()

    def snapshot(self) -> torch.Tensor:
        if not self.layers:
            return torch.zeros((0, len(STAT_FIELDS)), dtype=torch.int64)
        return torch.stack([c.stats for c in self.layers]).cpu()

    def _run(self, period: float) -> None:
        import time
        prev = None
        while True:
            time.sleep(period)
            try:
                now = self.snapshot()
                if prev is not None and now.shape == prev.shape and int((now - prev)[:, 0].sum()) > 0:
                    c = self.layers[0]
                    logger.info("r9700: expert cache over %.0f s (S=%d, threshold %d, insert cap %d): %s", period,
                                c.S, c.max_distinct, c.max_inserts, stats_line(now - prev, sum(c.bytes) / 2**20))
                prev = now
            except Exception as e:
                logger.warning("r9700: expert cache stats reporter stopped: %s", e)
                return


_REPORTER = _StatsReporter()


def stats_snapshot() -> torch.Tensor:
    """[layers, 5] int64 on the host: per cached layer, totals since load of STAT_FIELDS."""
    return _REPORTER.snapshot()


def stats_line(delta: torch.Tensor, mib_per_expert: float) -> str:
    """One line for a [layers, 5] difference of two snapshots: per layer-step means over the layers that stepped."""
    steps, distinct, inserts, through, wide = delta.sum(0).tolist()
    n = max(steps, 1)
    return (f"{steps} layer-steps: routed {distinct / n:.1f} distinct experts, {inserts / n:.1f} inserted, "
            f"{through / n:.1f} read through from host ({through / n * mib_per_expert:.0f} MiB), "
            f"{100.0 * wide / n:.0f}% of steps over the insert threshold")


class LayerCache:
    """One MoE layer's cache (reference moe/cache.py:182-395): host store of all E experts, S-slot VRAM arena,
    LRU state, and one persistent set of align buffers (pointer-stable, so captured graphs replay through it)."""

    def __init__(self, layer_idx: int, w13: torch.Tensor, w2: torch.Tensor, s13: torch.Tensor, s2: torch.Tensor,
                 N1: int, K1: int, N2: int, K2: int, slots: int):
        dev = torch.device("cuda", torch.cuda.current_device())
        E = w13.shape[0]
        self.E, self.S, self.layer_idx = E, min(slots, E, 1024), layer_idx
        if self.S < 1:
            raise ValueError("LayerCache: at least one slot")
        if E > 8192:
            raise ValueError(f"LayerCache: {E} experts (the device manager holds at most 8192)")
        self.N1, self.K1, self.N2, self.K2 = N1, K1, N2, K2
        self.fold = (False, False)
        if not (is_host(w13) and is_host(w2)):
            raise ValueError("LayerCache: w13 / w2 must be mapped host tensors (to_host / uva_empty)")
        # host store (the backing copy of every expert) and the VRAM arena of S slots with the same slab shapes
        self.h_w13, self.h_w2 = w13, w2
        self.h_s13, self.h_s2 = (s if is_host(s) else to_host(s.contiguous()) for s in (s13, s2))
        store = (self.h_w13, self.h_w2, self.h_s13, self.h_s2)
        self.a_w13, self.a_w2, self.a_s13, self.a_s2 = (
            torch.empty((self.S, *h.shape[1:]), dtype=h.dtype, device=dev) for h in store)
        self.bytes = [h[0].numel() * h.element_size() for h in store]
        if any(b % 16 for b in self.bytes):
            raise ValueError(f"LayerCache: per-expert slab sizes must be multiples of 16 bytes: {self.bytes}")
        self._init_lru_state(dev)
        self._init_policy()
        self._warm_start()
        if staging_enabled() and self.E > self.S:
            # every slot holds an expert after the warm start and keeps one, so at most E - S routed experts are cold
            cap = self.E - self.S
            self.stage = _stage_area(dev, cap, store)
            self.stage_cap = cap
            self.stage_map = torch.full((self.E,), -1, dtype=torch.int32, device=dev)
            self.stage_miss = torch.full((cap, 2), -1, dtype=torch.int32, device=dev)
            self.stage_n = torch.zeros((1,), dtype=torch.int32, device=dev)
        self.stats = None
        if stats_enabled():
            self.stats = torch.zeros((len(STAT_FIELDS),), dtype=torch.int64, device=dev)
            _REPORTER.add(self)

    def _init_lru_state(self, dev) -> None:
        """table [E] (expert -> slot, -1 = host), map_cold [E] (expert -> itself when not resident, else -1),
        slot_expert [S], slot_stamp [S] (step of last use), routed [E] flags, the step counter."""
        E, S = self.E, self.S
        self.table = torch.full((E,), -1, dtype=torch.int32, device=dev)
        self.map_cold = torch.arange(E, dtype=torch.int32, device=dev)
        self.slot_expert = torch.full((S,), -1, dtype=torch.int32, device=dev)
        self.slot_stamp = torch.zeros((S,), dtype=torch.int64, device=dev)
        self.routed = torch.zeros((E,), dtype=torch.uint8, device=dev)
        self.step = torch.zeros((1,), dtype=torch.int64, device=dev)

    def _init_policy(self) -> None:
        """Insert cap and read-through threshold (R9K_LRU_MAX_INSERTS, R9K_LRU_THRESH), the miss list they size,
        the gather launch shape (R9K_LRU_GATHER = "chunks,lanes") and the fused manage + align switch."""
        S, dev = self.S, self.table.device
        self.max_inserts = min(int(os.environ.get("R9K_LRU_MAX_INSERTS", "64")), S)
        self.max_distinct = int(S * float(os.environ.get("R9K_LRU_THRESH", "0.99")))
        self.miss = torch.full((max(1, self.max_inserts), 2), -1, dtype=torch.int32, device=dev)
        self.n_miss = torch.zeros((1,), dtype=torch.int32, device=dev)
        # a step of at most this many routed rows cannot need the cold pass: its distinct experts fit both limits
        self.no_cold_limit = min(self.max_distinct, self.max_inserts) if S > self.max_distinct else 0
        self.fused = os.environ.get("R9K_LRU_FUSED", "1") == "1"
        chunks, lanes = os.environ.get("R9K_LRU_GATHER", "64,16").split(",")
        self.chunks, self.lanes = int(chunks), int(lanes)
        self._one = None
        self._one_old: list = []
        self.stage = None
        self.hot_ids = None                      # set by update_fused: the last step's slot per routed row

    def _warm_start(self):
        prof = _profile()
        if prof is not None and self.layer_idx < prof.shape[0] and prof.shape[1] == self.E:
            order = torch.argsort(prof[self.layer_idx], descending=True, stable=True)
        else:
            order = torch.arange(self.E)
        init = order[: self.S].to(torch.int32)
        n = init.numel()
        dev = self.table.device
        pairs = torch.stack([init, torch.arange(n, dtype=torch.int32)], dim=1).to(dev)
        for i in range(0, n, max(1, self.max_inserts)):      # the gather kernel, in miss-list-sized batches
            chunk = pairs[i: i + max(1, self.max_inserts)]
            self.miss[: chunk.shape[0]].copy_(chunk)
            self.n_miss.fill_(chunk.shape[0])
            self._gather()
        self.n_miss.zero_()
        self.miss.fill_(-1)
        il = init.long().to(dev)
        self.table[il] = torch.arange(n, dtype=torch.int32, device=dev)
        self.map_cold[il] = -1
        self.slot_expert[:n] = init.to(dev)
        # older stamps for colder warm experts, so the hottest are evicted last
        self.slot_stamp[:n] = torch.arange(n, 0, -1, dtype=torch.int64, device=dev) - n
        torch.cuda.synchronize()

    def _gather(self, dst=None, miss=None, n_miss=None):
        """The listed experts host -> their slots (default: the arena and the manager's miss list)."""
        d13, d2, ds13, ds2 = dst if dst is not None else (self.a_w13, self.a_w2, self.a_s13, self.a_s2)
        miss = self.miss if miss is None else miss
        n_miss = self.n_miss if n_miss is None else n_miss
        b = self.bytes
        rc = _L().r4d_lru_gather(
            d13.data_ptr(), self.h_w13.data_ptr(), b[0], d2.data_ptr(), self.h_w2.data_ptr(), b[1],
            ds13.data_ptr(), self.h_s13.data_ptr(), b[2], ds2.data_ptr(), self.h_s2.data_ptr(), b[3],
            0, 0, 0, 0, 0, 0, miss.data_ptr(), n_miss.data_ptr(), self.chunks, self.lanes, _stream())
        if rc:
            raise RuntimeError(f"r4d_lru_gather failed ({rc})")

    def _manage(self, ids: torch.Tensor, hot: torch.Tensor | None = None, cold: torch.Tensor | None = None) -> None:
        """LRU manage; with hot / cold given, the same launch also writes the two passes' mapped routing ids."""
        rc = _L().r9k_lru_manage_map(ids.data_ptr(), ids.numel(), self.E, self.S, self.max_distinct,
                                     self.max_inserts, self.table.data_ptr(), self.map_cold.data_ptr(),
                                     self.slot_expert.data_ptr(), self.slot_stamp.data_ptr(), self.routed.data_ptr(),
                                     self.step.data_ptr(), self.miss.data_ptr(), self.n_miss.data_ptr(),
                                     hot.data_ptr() if hot is not None else 0,
                                     cold.data_ptr() if cold is not None else 0, _stream())
        if rc:
            raise RuntimeError(f"r4d_lru_manage failed ({rc}) E={self.E} S={self.S}")

    @staticmethod
    def _ids(topk_ids: torch.Tensor) -> torch.Tensor:
        ids = topk_ids.reshape(-1)
        if ids.dtype != torch.int32:
            ids = ids.to(torch.int32)
        return ids.contiguous()

    def update(self, topk_ids: torch.Tensor) -> None:
        """LRU manage + gather of this step's inserts (host -> slots)."""
        self._manage(self._ids(topk_ids))
        self._gather()
        if self.stats is not None:
            self._record()

    def _record(self):
        """After manage + gather: routed marks this step's experts and table already holds the inserted ones, so
        routed-and-not-resident is what the cold pass reads through from host memory."""
        r = self.routed.to(torch.int64)
        d = r.sum()
        cold = (r * (self.table < 0)).sum()
        self.stats.add_(torch.stack([torch.ones_like(d), d, self.n_miss[0].to(torch.int64), cold,
                                     (d > self.max_distinct).to(torch.int64)]))

    def _align_bufs(self, mk: int, bs: int):
        """Align outputs for (mk, bs), sized as moe_align sizes them (capacity()), as views of ONE buffer set per
        layer sized by the largest step seen. A larger step keeps the old set alive (a captured graph may replay
        through it) and takes one at least twice the size, so the total stays under twice the largest."""
        L = K.capacity(mk, self.E, bs)
        NB = L // bs
        o = self._one
        if o is None or o[0] < L or o[1] < mk:
            if o is not None:
                self._one_old.append(o)
            cl = max(L, 2 * o[0]) if o is not None else L
            cm = max(mk, 2 * o[1]) if o is not None else mk
            cn = cl // K.MOE_BLOCK + 1
            i32 = dict(dtype=torch.int32, device=self.table.device)
            o = (cl, cm, torch.empty((cl,), **i32), torch.empty((cn,), **i32), torch.empty((1,), **i32),
                 torch.empty((cl,), **i32), torch.empty((cn,), **i32), torch.empty((1,), **i32),
                 torch.empty((max(1, cm),), **i32), torch.empty((max(1, cm),), **i32))
            self._one = o
        return (L, NB, o[2][:L], o[3][:NB], o[4], o[5][:L], o[6][:NB], o[7], o[8][:mk], o[9][:mk])

    def update_fused(self, topk_ids: torch.Tensor, bs: int, need_cold: bool = True):
        """LRU manage and both align outputs -- the resident one over slot ids (ids through table), the host one
        over expert ids (through map_cold) -- in one launch (r9k_lru_manage_tables; E <= 1024 and mk <= 4096, else
        manage with the mapped ids, then two aligns: the same tables), then the gather. Returns
        ((sorted, eids, ntpp) hot, (sorted, eids, ntpp) cold), views of the layer's persistent buffers. need_cold =
        False skips the host tables (their contents are then stale): for steps of at most no_cold_limit rows, whose
        cold pass is provably empty."""
        ids = self._ids(topk_ids)
        mk = ids.numel()
        L_, NB, sh, eh, nh, sc, ec, nc, hid, cid = self._align_bufs(mk, bs)
        lib, st = _L(), _stream()
        # one launch (manage + both table sets) while one workgroup can build the tables, else manage + two aligns
        rc = lib.r9k_lru_manage_tables(ids.data_ptr(), mk, self.E, self.S, self.max_distinct, self.max_inserts,
                                       self.table.data_ptr(), self.map_cold.data_ptr(), self.slot_expert.data_ptr(),
                                       self.slot_stamp.data_ptr(), self.routed.data_ptr(), self.step.data_ptr(),
                                       self.miss.data_ptr(), self.n_miss.data_ptr(), bs, sh.data_ptr(), eh.data_ptr(),
                                       nh.data_ptr(), sc.data_ptr() if need_cold else 0,
                                       ec.data_ptr() if need_cold else 0, nc.data_ptr() if need_cold else 0,
                                       hid.data_ptr(), st)
        self.hot_ids = hid                       # each routed row's slot (-1 not resident), both paths below
        if rc not in (0, 2):
            raise RuntimeError(f"r9k_lru_manage_tables failed ({rc}) E={self.E} S={self.S} mk={mk}")
        if rc == 0:
            self._gather()
            if self.stats is not None:
                self._record()
            return (sh, eh, nh), (sc, ec, nc)
        self._manage(ids, hid, cid)
        self._gather()
        if self.stats is not None:
            self._record()
        n = lib.r9k_moe_align_scratch_ints(mk, self.E)
        scratch = K._align_scratch(ids.device, n)
        for a, s_, e_, t_ in ((hid, sh, eh, nh), (cid, sc, ec, nc))[: 2 if need_cold else 1]:
            rc = lib.r9k_moe_align(a.data_ptr(), mk, self.E, bs, s_.data_ptr(), e_.data_ptr(), t_.data_ptr(),
                                   scratch.data_ptr(), scratch.numel(), st)
            if rc:
                raise RuntimeError(f"r9k_moe_align failed ({rc}) numel={mk} E={self.E} block={bs}")
        return (sh, eh, nh), (sc, ec, nc)

    def stage_cold(self, topk_ids: torch.Tensor):
        """After this step's manage: number the routed experts that are not resident (r9k_lru_stage_map, ascending
        expert order), copy them host -> staging area with one gather, and return (w13, w2) experts over the staging
        area plus stage_map [E] (expert -> staging index, -1 otherwise) for the cold pass's tables. Device work only
        (no host sync), so a captured graph replays it."""
        if self.stage is None:
            raise RuntimeError("LayerCache.stage_cold: staging is off (R9K_STAGE_COLD=1 turns it on)")
        ids = self._ids(topk_ids)
        rc = _L().r9k_lru_stage_map(ids.data_ptr(), ids.numel(), self.E, self.table.data_ptr(), self.stage_cap,
                                    self.stage_map.data_ptr(), self.stage_miss.data_ptr(), self.stage_n.data_ptr(),
                                    _stream())
        if rc:
            raise RuntimeError(f"r9k_lru_stage_map failed ({rc}) E={self.E}")
        self._gather(self.stage, self.stage_miss, self.stage_n)
        w13, w2, s13, s2 = self.stage
        return (*self._experts(w13, s13, w2, s2), self.stage_map)

    def _experts(self, w13, s13, w2, s2):
        return (K.Mxfp4Experts(w13, s13, self.N1, self.K1, self.fold[0]),
                K.Mxfp4Experts(w2, s2, self.N2, self.K2, self.fold[1]))

    def hot(self):
        """(w13, w2) experts over the VRAM arena: the pass whose ids go through `table`."""
        return self._experts(self.a_w13, self.a_s13, self.a_w2, self.a_s2)

    def cold(self):
        """(w13, w2) experts over the mapped host store: the pass whose ids go through `map_cold`."""
        return self._experts(self.h_w13, self.h_s13, self.h_w2, self.h_s2)


def slots_per_layer(bytes_per_expert: int) -> int:
    """VRAM slots of each cached layer: R9K_EXPERT_CACHE_SLOTS when set; else the R9K_EXPERT_CACHE_GB budget shared
    by the cached layers (R9K_EXPERT_CACHE_LAYERS, default every MoE layer of the model), in whole experts; 0 = off."""
    fixed = int(os.environ.get("R9K_EXPERT_CACHE_SLOTS", "0") or 0)
    if fixed > 0:
        return fixed
    budget = int(budget_gb() * 2**30)
    if budget <= 0:
        return 0
    layers = int(os.environ.get("R9K_EXPERT_CACHE_LAYERS", "0") or 0) or _num_moe_layers()
    return budget // layers // bytes_per_expert


def host_only() -> bool:
    """Cache only layers whose experts are already host-offloaded (R9K_EXPERT_CACHE_HOST_ONLY=1, the default);
    0 moves device-resident layers to host as well."""
    return os.environ.get("R9K_EXPERT_CACHE_HOST_ONLY", "1") == "1"
