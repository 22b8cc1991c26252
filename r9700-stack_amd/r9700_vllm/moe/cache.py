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

Layout of this module's host side (its own design; the names, knobs and LRU policy are the reference's, which
callers and its tests bind):
* `LruPolicy`   -- the knobs, read once per layer from the environment into a frozen record;
* `_StateBlock` -- every LRU array of a layer (table, map_cold, slot_expert, slot_stamp, routed, step, miss list)
  carved from ONE device allocation at 256-byte offsets, so the state has one base address for its whole life and
  the warm start writes it with a single host -> device copy of a host-built image;
* `_Counters`   -- the optional per-layer statistics as rows of one shared device tensor per device, read by one
  `.cpu()` for all layers, and a reporter thread that logs the change over each period.

Config (per process, the reference's names): R9K_EXPERT_CACHE_GB (0 = off), R9K_EXPERT_CACHE_SLOTS,
R9K_EXPERT_CACHE_LAYERS, R9K_LRU_THRESH (0.99: a step routing to more distinct experts than this share of the slots
inserts nothing and reads every non-resident expert through from host), R9K_LRU_MAX_INSERTS (64),
R9K_LRU_GATHER="chunks,lanes" (16,4), R9K_LRU_FUSED (1), R9K_EXPERT_CACHE_HOST_ONLY (1), R9K_EXPERT_CACHE_STATS,
R9K_EXPERT_CACHE_STATS_SEC (10), R9K_STAGE_COLD (0). Warm start: the checkpoint's model-expertprofile.safetensors
(expert_routing_counts [layers, experts]) when vLLM names a model directory holding one, else experts 0..S-1; the
hottest expert gets the newest stamp, so the warm set is evicted coldest first.

On gfx950 the cold pass reads weights over PCIe inside the GEMM (the decode kernels read every weight byte once per
routing block). R9K_STAGE_COLD=1 first copies the step's cold experts into a VRAM staging area shared by the layers.
"""
from __future__ import annotations

import ctypes
import dataclasses
import functools
import logging
import os
import threading

import numpy as np
import torch

from ..kernels import moe as K

logger = logging.getLogger("vllm." + __name__)

_BOUND = False
_HOST_BUFFERS: list = []          # (pointer, bytes) of every mapped host buffer: held until the process ends
HOST_COPY_BYTES = 512 << 20       # largest single device -> host transfer of to_host
WARM_COPY_EXPERTS = 64            # experts per host -> arena copy of the warm start


# Activation rows the manage launch quantises alongside (r9k_lru_manage_tables: one wave a row, 16 waves).
QUANT_MAX_ROWS = 64


def quant_fits(x: torch.Tensor) -> bool:
    """Whether r9k_lru_manage_tables can make the fp8 input quant of x (bf16 [T <= 64, H], unit column stride, 16-byte
    aligned rows, H % 8 == 0, H <= 4096)."""
    return (x.dtype == torch.bfloat16 and x.dim() == 2 and 1 <= x.shape[0] <= QUANT_MAX_ROWS and x.stride(1) == 1
            and 8 <= x.shape[1] <= 4096 and x.shape[1] % 8 == 0 and x.stride(0) >= x.shape[1]
            and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0)


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
        L.r9k_lru_manage_tables.argtypes = [l, i, i, i, i, i] + [l] * 8 + [i] + [l] * 9 + [i, i, l, l, l]
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


def staging_enabled() -> bool:
    """R9K_STAGE_COLD=1 (opt-in, as in the reference): a step that needs the cold pass first copies every routed
    expert that is not resident into a VRAM staging area with one bulk gather, and the cold pass reads it there
    instead of reading host memory inside the GEMMs (once per routing block)."""
    return os.environ.get("R9K_STAGE_COLD", "0") == "1"


def stats_enabled() -> bool:
    return os.environ.get("R9K_EXPERT_CACHE_STATS", "0") == "1"


def host_only() -> bool:
    """Cache only layers whose experts are already host-offloaded (R9K_EXPERT_CACHE_HOST_ONLY=1, the default);
    0 moves device-resident layers to host as well."""
    return os.environ.get("R9K_EXPERT_CACHE_HOST_ONLY", "1") == "1"


# ---------------------------------------------------------------------------------------------------------------
# What vLLM tells us about the model: its directory (for the routing profile) and its layer count (for the budget)

@functools.lru_cache(maxsize=None)
def _model_facts() -> tuple:
    """(model directory or None, hidden layer count or None) from vLLM's current config; (None, None) without one."""
    try:
        from vllm.config import get_current_vllm_config
        mc = get_current_vllm_config().model_config
    except Exception:
        return None, None
    layers = getattr(getattr(mc, "hf_text_config", None), "num_hidden_layers", None)
    return getattr(mc, "model", None), (int(layers) if layers else None)


@functools.lru_cache(maxsize=None)
def routing_profile() -> torch.Tensor | None:
    """expert_routing_counts [layers, experts] (fp32) from <model>/model-expertprofile.safetensors, read once per
    process; None when vLLM names no model directory or it holds no profile."""
    model_dir, _ = _model_facts()
    path = os.path.join(model_dir, "model-expertprofile.safetensors") if model_dir else None
    if not path or not os.path.isfile(path):
        return None
    from safetensors import safe_open
    with safe_open(path, framework="pt") as f:
        counts = f.get_tensor("expert_routing_counts").float()
    logger.info("r9700: warm-starting expert caches from %s, counts %s", path, tuple(counts.shape))
    return counts


def slots_per_layer(bytes_per_expert: int) -> int:
    """VRAM slots of each cached layer: R9K_EXPERT_CACHE_SLOTS when set; else the R9K_EXPERT_CACHE_GB budget shared
    by the cached layers (R9K_EXPERT_CACHE_LAYERS, default every hidden layer of the model, 48 when vLLM does not
    say), in whole experts; 0 = off."""
    fixed = int(os.environ.get("R9K_EXPERT_CACHE_SLOTS", "0") or 0)
    if fixed > 0:
        return fixed
    budget = int(budget_gb() * 2**30)
    if budget <= 0:
        return 0
    layers = int(os.environ.get("R9K_EXPERT_CACHE_LAYERS", "0") or 0) or _model_facts()[1] or 48
    return budget // layers // bytes_per_expert


# ---------------------------------------------------------------------------------------------------------------
# Policy and state

@dataclasses.dataclass(frozen=True)
class LruPolicy:
    """The cache's knobs for one layer of S slots.
    max_inserts   experts copied in per step at most (R9K_LRU_MAX_INSERTS, capped at S);
    max_distinct  a step routing to more distinct experts inserts nothing (int(S * R9K_LRU_THRESH));
    no_cold_limit a step of at most this many routed rows cannot need the cold pass (its distinct experts fit both
                  limits above; 0 when the threshold covers every slot);
    fused         manage and both table sets in one launch (R9K_LRU_FUSED);
    chunks, lanes the gather's launch shape (R9K_LRU_GATHER = "chunks,lanes"). 16 x 4 workgroups keep ~1 MB of host
                  reads in flight, more than PCIe needs: measured on MI355X, 64 experts gathered at 57.0 GB/s against
                  54.3 with 64 x 16, and a step that gathers nothing (its launch still runs) 0.4 us shorter."""
    max_inserts: int
    max_distinct: int
    no_cold_limit: int
    fused: bool
    chunks: int
    lanes: int

    @classmethod
    def from_env(cls, slots: int) -> "LruPolicy":
        env = os.environ.get
        ins = min(int(env("R9K_LRU_MAX_INSERTS", "64")), slots)
        distinct = int(slots * float(env("R9K_LRU_THRESH", "0.99")))
        chunks, lanes = (int(v) for v in env("R9K_LRU_GATHER", "16,4").split(","))
        return cls(max_inserts=ins, max_distinct=distinct,
                   no_cold_limit=min(distinct, ins) if slots > distinct else 0,
                   fused=env("R9K_LRU_FUSED", "1") == "1", chunks=chunks, lanes=lanes)


class _StateBlock:
    """The LRU arrays of one layer as typed views of a single device byte buffer (256-byte aligned fields):

        table       [E]     int32  expert -> slot, -1 = not resident
        map_cold    [E]     int32  expert -> itself when not resident, else -1
        slot_expert [S]     int32  slot -> expert, -1 = empty
        slot_stamp  [S]     int64  step of the slot's last use (victims: smallest stamp, then lowest slot)
        routed      [E]     uint8  this step's routed flags (the manager's scratch)
        step        [1]     int64  step counter
        miss        [I, 2]  int32  (expert, slot) inserts of the step, I = max(1, max_inserts)
        n_miss      [1]     int32  their count

    `image(...)` builds the bytes of a whole state on the host, `load(...)` writes it with one copy."""

    FIELDS = (("table", "E", np.int32), ("map_cold", "E", np.int32), ("slot_expert", "S", np.int32),
              ("slot_stamp", "S", np.int64), ("routed", "E", np.uint8), ("step", 1, np.int64),
              ("miss", "I2", np.int32), ("n_miss", 1, np.int32))

    def __init__(self, dev: torch.device, E: int, S: int, inserts: int):
        sizes = {"E": E, "S": S, "I2": 2 * max(1, inserts), 1: 1}
        self.layout, off = {}, 0
        for name, n, dt in self.FIELDS:
            count = sizes[n]
            self.layout[name] = (off, count, np.dtype(dt))
            off += -(-count * np.dtype(dt).itemsize // 256) * 256
        self.nbytes = off
        self.buf = torch.zeros((off,), dtype=torch.uint8, device=dev)
        tdt = {np.dtype(np.int32): torch.int32, np.dtype(np.int64): torch.int64, np.dtype(np.uint8): torch.uint8}
        for name, (o, count, dt) in self.layout.items():
            v = self.buf[o:o + count * dt.itemsize].view(tdt[dt])
            setattr(self, name, v.view(-1, 2) if name == "miss" else v)

    def image(self, E: int, residents: np.ndarray) -> np.ndarray:
        """The state after installing `residents` (expert ids, hottest first) in slots 0..n-1: each resident's stamp
        is minus its rank, so the coldest warm expert is the first victim."""
        img = np.zeros(self.nbytes, dtype=np.uint8)

        def field(name):
            o, count, dt = self.layout[name]
            return img[o:o + count * dt.itemsize].view(dt)
        n = residents.size
        table, cold = field("table"), field("map_cold")
        table[:] = -1
        table[residents] = np.arange(n, dtype=np.int32)
        cold[:] = np.where(table < 0, np.arange(E, dtype=np.int32), -1)
        slots = field("slot_expert")
        slots[:] = -1
        slots[:n] = residents
        field("slot_stamp")[:n] = -np.arange(n, dtype=np.int64)
        field("miss")[:] = -1
        return img

    def load(self, img: np.ndarray) -> None:
        self.buf.copy_(torch.from_numpy(img))


def _warm_residents(layer_idx: int, E: int, S: int) -> np.ndarray:
    """The S experts a layer starts with, hottest first: by the routing profile's counts for this layer (ties to
    the lower id) when it has a row for a layer of E experts, else 0..S-1."""
    prof = routing_profile()
    if prof is None or layer_idx >= prof.shape[0] or prof.shape[1] != E:
        return np.arange(S, dtype=np.int32)
    counts = prof[layer_idx].double().numpy()
    return np.lexsort((np.arange(E), -counts))[:S].astype(np.int32)


# ---------------------------------------------------------------------------------------------------------------
# Statistics

STAT_FIELDS = ("steps", "distinct", "inserts", "read_through", "wide")


class _Counters:
    """Statistics of every cached layer of the process: one int64 device tensor [rows, len(STAT_FIELDS)] per device,
    a row per layer (grown by whole blocks; a layer keeps its row view), and a reporter thread that logs the change
    of the totals over each R9K_EXPERT_CACHE_STATS_SEC period (0 = no thread). A failing reporter stops itself."""

    BLOCK = 128

    def __init__(self):
        self.blocks: dict = {}          # device index -> list of [BLOCK, fields] tensors
        self.used: dict = {}
        self.owners: list = []          # (cache) in registration order, for the log line's shape
        self.lock = threading.Lock()
        self.stop = threading.Event()
        self.thread = None

    def row(self, cache, dev: torch.device) -> torch.Tensor:
        with self.lock:
            blocks = self.blocks.setdefault(dev.index, [])
            n = self.used.get(dev.index, 0)
            if n == len(blocks) * self.BLOCK:
                blocks.append(torch.zeros((self.BLOCK, len(STAT_FIELDS)), dtype=torch.int64, device=dev))
            self.used[dev.index] = n + 1
            self.owners.append(cache)
            r = blocks[n // self.BLOCK][n % self.BLOCK]
        period = float(os.environ.get("R9K_EXPERT_CACHE_STATS_SEC", "10") or 0)
        if self.thread is None and period > 0:
            self.thread = threading.Thread(target=self._report, args=(period,), name="r9k-cache-stats", daemon=True)
            self.thread.start()
        return r

    def totals(self) -> torch.Tensor:
        with self.lock:
            parts = []
            for d in sorted(self.blocks):
                n = self.used[d]
                parts += [b.cpu() for b in self.blocks[d]]
                parts[-1] = parts[-1][: n - (len(self.blocks[d]) - 1) * self.BLOCK]
        if not parts:
            return torch.zeros((0, len(STAT_FIELDS)), dtype=torch.int64)
        return torch.cat(parts)

    def _report(self, period: float) -> None:
        before = None
        while not self.stop.wait(period):
            try:
                now = self.totals()
                if before is not None and now.shape == before.shape:
                    d = now - before
                    if int(d[:, 0].sum()):
                        c = self.owners[0]
                        logger.info("r9700 expert cache (%d slots a layer, insert cap %d, read-through above %d "
                                    "experts), last %.0f s: %s", c.S, c.max_inserts, c.max_distinct, period,
                                    stats_line(d, sum(c.bytes) / 2**20))
                before = now
            except Exception as exc:
                logger.warning("r9700: expert cache statistics off after an error: %s", exc)
                return


_COUNTERS = _Counters()


def stats_snapshot() -> torch.Tensor:
    """[layers, 5] int64 on the host: per cached layer, totals since load of STAT_FIELDS."""
    return _COUNTERS.totals()


def stats_line(delta: torch.Tensor, mib_per_expert: float) -> str:
    """One line for a [layers, 5] difference of two snapshots: per layer-step means over the layers that stepped."""
    tot = dict(zip(STAT_FIELDS, delta.sum(0).tolist()))
    per = 1.0 / max(tot["steps"], 1)
    host = tot["read_through"] * per
    return (f"{tot['steps']} layer-steps; per layer-step {tot['distinct'] * per:.1f} experts routed, "
            f"{tot['inserts'] * per:.1f} copied into VRAM, {host:.1f} read from host memory "
            f"({host * mib_per_expert:.0f} MiB); {100.0 * tot['wide'] * per:.0f}% of steps read through")


_STAGE_AREAS: dict = {}


def _stage_area(dev: torch.device, cap: int, store) -> tuple:
    """The staging slabs (w13, w2, s13, s2) for `cap` experts, shaped like the host store's, one set per device and
    shape: layers run one after another on one stream, so every cached layer of a model shares it."""
    key = (dev.index, cap) + tuple((tuple(h.shape[1:]), h.dtype) for h in store)
    area = _STAGE_AREAS.get(key)
    if area is None:
        area = _STAGE_AREAS[key] = tuple(torch.empty((cap, *h.shape[1:]), dtype=h.dtype, device=dev) for h in store)
    return area


# ---------------------------------------------------------------------------------------------------------------

class LayerCache:
    """One MoE layer's cache (reference moe/cache.py:182-395): host store of all E experts, S-slot VRAM arena,
    LRU state, and one persistent set of align buffers (pointer-stable, so captured graphs replay through it)."""

    def __init__(self, layer_idx: int, w13: torch.Tensor, w2: torch.Tensor, s13: torch.Tensor, s2: torch.Tensor,
                 N1: int, K1: int, N2: int, K2: int, slots: int):
        if not (is_host(w13) and is_host(w2)):
            raise ValueError("LayerCache: w13 / w2 must be mapped host tensors (to_host / uva_empty)")
        E = w13.shape[0]
        S = min(slots, E, 1024)
        if S < 1:
            raise ValueError("LayerCache: at least one slot")
        if E > 8192:
            raise ValueError(f"LayerCache: {E} experts (the device manager holds at most 8192)")
        dev = torch.device("cuda", torch.cuda.current_device())
        self.layer_idx, self.E, self.S = layer_idx, E, S
        self.N1, self.K1, self.N2, self.K2 = N1, K1, N2, K2
        self.fold = (False, False)
        self.policy = LruPolicy.from_env(S)

        # the backing store (scales copied to host when they are not there) and an arena of S slots shaped alike
        store = (w13, w2) + tuple(s if is_host(s) else to_host(s.contiguous()) for s in (s13, s2))
        self.h_w13, self.h_w2, self.h_s13, self.h_s2 = store
        self.bytes = [h[0].numel() * h.element_size() for h in store]
        if any(b % 16 for b in self.bytes):
            raise ValueError(f"LayerCache: per-expert slab sizes must be multiples of 16 bytes: {self.bytes}")
        arena = tuple(torch.empty((S, *h.shape[1:]), dtype=h.dtype, device=dev) for h in store)
        self.a_w13, self.a_w2, self.a_s13, self.a_s2 = arena

        self.state = _StateBlock(dev, E, S, self.policy.max_inserts)
        residents = _warm_residents(layer_idx, E, S)
        self.state.load(self.state.image(E, residents))
        idx = torch.from_numpy(residents.astype(np.int64))
        for lo in range(0, residents.size, WARM_COPY_EXPERTS):
            sel = idx[lo:lo + WARM_COPY_EXPERTS]
            for dst, src in zip(arena, store):
                dst[lo:lo + sel.numel()].copy_(src.index_select(0, sel))
        torch.cuda.synchronize()

        self._one = None
        self._one_old: list = []
        self.hot_ids = None                      # set by update_fused: the last step's slot per routed row
        self.x_quant = None                      # set by update_fused: its fp8 input quant (xq, xs), or None
        self.stage = None
        if staging_enabled() and E > S:
            # every slot holds an expert after the warm start and keeps one, so at most E - S routed experts are cold
            self.stage_cap = E - S
            self.stage = _stage_area(dev, self.stage_cap, store)
            self.stage_map = torch.full((E,), -1, dtype=torch.int32, device=dev)
            self.stage_miss = torch.full((self.stage_cap, 2), -1, dtype=torch.int32, device=dev)
            self.stage_n = torch.zeros((1,), dtype=torch.int32, device=dev)
        self.stats = _COUNTERS.row(self, dev) if stats_enabled() else None

    # the state arrays and knobs under the names the manager's callers use
    table = property(lambda self: self.state.table)
    map_cold = property(lambda self: self.state.map_cold)
    slot_expert = property(lambda self: self.state.slot_expert)
    slot_stamp = property(lambda self: self.state.slot_stamp)
    routed = property(lambda self: self.state.routed)
    step = property(lambda self: self.state.step)
    miss = property(lambda self: self.state.miss)
    n_miss = property(lambda self: self.state.n_miss)
    max_inserts = property(lambda self: self.policy.max_inserts)
    max_distinct = property(lambda self: self.policy.max_distinct)
    no_cold_limit = property(lambda self: self.policy.no_cold_limit)
    fused = property(lambda self: self.policy.fused)

    def _gather(self, dst=None, miss=None, n_miss=None):
        """The listed experts host -> their slots (default: the arena and the manager's miss list)."""
        d13, d2, ds13, ds2 = dst if dst is not None else (self.a_w13, self.a_w2, self.a_s13, self.a_s2)
        miss = self.miss if miss is None else miss
        n_miss = self.n_miss if n_miss is None else n_miss
        b = self.bytes
        rc = _L().r4d_lru_gather(
            d13.data_ptr(), self.h_w13.data_ptr(), b[0], d2.data_ptr(), self.h_w2.data_ptr(), b[1],
            ds13.data_ptr(), self.h_s13.data_ptr(), b[2], ds2.data_ptr(), self.h_s2.data_ptr(), b[3],
            0, 0, 0, 0, 0, 0, miss.data_ptr(), n_miss.data_ptr(), self.policy.chunks, self.policy.lanes, _stream())
        if rc:
            raise RuntimeError(f"r4d_lru_gather failed ({rc})")

    def _state_ptrs(self) -> list:
        s = self.state
        return [s.table.data_ptr(), s.map_cold.data_ptr(), s.slot_expert.data_ptr(), s.slot_stamp.data_ptr(),
                s.routed.data_ptr(), s.step.data_ptr(), s.miss.data_ptr(), s.n_miss.data_ptr()]

    def _manage(self, ids: torch.Tensor, hot: torch.Tensor | None = None, cold: torch.Tensor | None = None) -> None:
        """LRU manage; with hot / cold given, the same launch also writes the two passes' mapped routing ids."""
        rc = _L().r9k_lru_manage_map(ids.data_ptr(), ids.numel(), self.E, self.S, self.max_distinct,
                                     self.max_inserts, *self._state_ptrs(),
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

    def update_fused(self, topk_ids: torch.Tensor, bs: int, need_cold: bool = True, x: torch.Tensor | None = None):
        """LRU manage and both align outputs -- the resident one over slot ids (ids through table), the host one
        over expert ids (through map_cold) -- in one launch (r9k_lru_manage_tables; E <= 1024 and mk <= 4096, else
        manage with the mapped ids, then two aligns: the same tables), then the gather. Returns
        ((sorted, eids, ntpp) hot, (sorted, eids, ntpp) cold), views of the layer's persistent buffers. need_cold =
        False skips the host tables (their contents are then stale): for steps of at most no_cold_limit rows, whose
        cold pass is provably empty. x (bf16 [T, H], optional): the one launch also makes the experts' fp8 input
        quant (quant_rows_fp8's bytes) when it serves x (quant_fits); x_quant is then (xq, xs), else None."""
        ids = self._ids(topk_ids)
        mk = ids.numel()
        L_, NB, sh, eh, nh, sc, ec, nc, hid, cid = self._align_bufs(mk, bs)
        lib, st = _L(), _stream()
        xq = xs = None
        if x is not None and quant_fits(x):
            T, H = x.shape
            xq = torch.empty((T, H), dtype=torch.float8_e4m3fn, device=x.device)
            xs = torch.empty((T,), dtype=torch.float32, device=x.device)
        # one launch (manage + both table sets) while one workgroup can build the tables, else manage + two aligns
        rc = lib.r9k_lru_manage_tables(ids.data_ptr(), mk, self.E, self.S, self.max_distinct, self.max_inserts,
                                       *self._state_ptrs(), bs, sh.data_ptr(), eh.data_ptr(),
                                       nh.data_ptr(), sc.data_ptr() if need_cold else 0,
                                       ec.data_ptr() if need_cold else 0, nc.data_ptr() if need_cold else 0,
                                       hid.data_ptr(), x.data_ptr() if xq is not None else 0,
                                       x.stride(0) if xq is not None else 0, x.shape[1] if xq is not None else 0,
                                       x.shape[0] if xq is not None else 0, xq.data_ptr() if xq is not None else 0,
                                       xs.data_ptr() if xq is not None else 0, st)
        self.hot_ids = hid                       # each routed row's slot (-1 not resident), both paths below
        self.x_quant = (xq, xs) if rc == 0 and xq is not None else None
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
