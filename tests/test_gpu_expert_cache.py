"""GPU parity of the host-offloaded expert cache (f4; moe/cache.py, csrc/r9k_expert_cache.hip).

* r4d_lru_manage against the oracle's manager (oracle.lru_manage): every state array bit-exact after every step of
  80-step sequences with padding ids, wide (read-through) steps, insert caps, working-set shifts.
* r4d_lru_gather: the listed experts' slabs byte-exact in their slots, other slots untouched.
* The reference's own bar (tests/test_cache_moe.py): the hot pass over the VRAM slots plus the cold pass over the
  mapped host store gives exactly the output of one pass over the full host store, bit for bit, on every step,
  through both update paths, with the cache invariants and the oracle's state checked alongside.
* A config 2 layer (E=288, hidden 2048, intermediate 512, top-8) through R9700Mxfp4Experts.apply with a 64-slot cache
  equals the same layer without one, bit for bit, at T = 1 (inserts) and T = 16 / 64 (read-through steps).
* R9K_STAGE_COLD=1: the staging map against its contract, and the layer with its cold pass over the staged VRAM copy
  equal to the resident layer, bit for bit.
* update_fused captured in a HIP graph and replayed with new routing equals an eager twin on every replay
  (reference tests/test_cache_shapes.py part 2), and its buffers keep one address once the largest step was seen."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from r9700_vllm.kernels import moe as K
from r9700_vllm.moe import cache as C
from r9700_vllm.moe.experts import R9700Mxfp4Experts

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda", 0)


def make_w(dev, E, N, Kd, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    p = torch.randint(0, 256, (E, N, Kd // 2), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    e = torch.randint(118, 127, (E, N, Kd // 32), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    return K.prepare_mxfp4_weights(p, e)


class DevState:
    def __init__(self, dev, E, S, max_ins):
        i32 = dict(dtype=torch.int32, device=dev)
        self.E, self.S = E, S
        self.table = torch.full((E,), -1, **i32)
        self.map_cold = torch.arange(E, **i32)
        self.slot_expert = torch.full((S,), -1, **i32)
        self.slot_stamp = torch.zeros((S,), dtype=torch.int64, device=dev)
        self.routed = torch.zeros((E,), dtype=torch.uint8, device=dev)
        self.step = torch.zeros((1,), dtype=torch.int64, device=dev)
        self.miss = torch.full((max(1, max_ins), 2), -1, **i32)
        self.n_miss = torch.zeros((1,), **i32)

    def manage(self, ids, max_distinct, max_ins, mapped=False):
        """r4d_lru_manage, or with mapped=True r9k_lru_manage_map (returns the hot / cold routing ids)."""
        args = (ids.data_ptr(), ids.numel(), self.E, self.S, max_distinct, max_ins, self.table.data_ptr(),
                self.map_cold.data_ptr(), self.slot_expert.data_ptr(), self.slot_stamp.data_ptr(),
                self.routed.data_ptr(), self.step.data_ptr(), self.miss.data_ptr(), self.n_miss.data_ptr())
        st = torch.cuda.current_stream().cuda_stream
        if not mapped:
            assert C._L().r4d_lru_manage(*args, st) == 0
            return None
        hot = torch.full_like(ids, -9)
        cold = torch.full_like(ids, -9)
        assert C._L().r9k_lru_manage_map(*args, hot.data_ptr(), cold.data_ptr(), st) == 0
        return hot, cold


def same_state(d: DevState, st: O.LruState):
    return (np.array_equal(d.table.cpu().numpy(), st.table) and np.array_equal(d.map_cold.cpu().numpy(), st.map_cold)
            and np.array_equal(d.slot_expert.cpu().numpy(), st.slot_expert)
            and np.array_equal(d.slot_stamp.cpu().numpy(), st.slot_stamp) and int(d.step.item()) == st.step)


@pytest.mark.parametrize("E,S,thresh,max_ins,M,k,seed", [
    (64, 48, 0.5, 48, 4, 6, 1), (288, 64, 0.99, 64, 8, 8, 2), (16, 16, 1.0, 16, 3, 4, 3), (40, 8, 0.99, 2, 2, 4, 4),
    (384, 256, 0.99, 64, 32, 8, 5), (8, 3, 1.0, 3, 1, 2, 6), (2048, 1024, 0.99, 1024, 200, 8, 7),
])
def test_lru_manage_matches_oracle(dev, E, S, thresh, max_ins, M, k, seed):
    print(f"lru manage E={E} S={S} max_ins={max_ins} M={M} k={k}", flush=True)
    rng = np.random.default_rng(seed)
    st = O.LruState(E, S)
    d = DevState(dev, E, S, max_ins)
    max_distinct = int(S * thresh)
    hot = rng.permutation(E)[: max(1, S // 2)]
    for step in range(80):
        if step == 50:
            hot = rng.permutation(E)[: max(1, S // 2)]
        pool = np.arange(E) if step % 7 == 0 else hot
        ids = np.stack([rng.choice(pool, size=min(k, pool.size), replace=False) for _ in range(M)]).reshape(-1)
        if step % 5 == 0:
            ids = np.concatenate([ids, [-1, E, E + 3]])
        routed, misses = O.lru_manage(st, ids, max_distinct, max_ins)
        hc = d.manage(torch.from_numpy(ids.astype(np.int32)).to(dev), max_distinct, max_ins, mapped=step % 2 == 1)
        torch.cuda.synchronize()
        if hc is not None:                                # the ids through the updated maps, -1 outside [0, E)
            ok = (ids >= 0) & (ids < E)
            safe = np.where(ok, ids, 0)
            assert np.array_equal(hc[0].cpu().numpy(), np.where(ok, st.table[safe], -1)), step
            assert np.array_equal(hc[1].cpu().numpy(), np.where(ok, st.map_cold[safe], -1)), step
        n = int(d.n_miss.item())
        got = [tuple(x) for x in d.miss[:n].cpu().tolist()]
        assert got == misses, (step, got, misses)
        assert np.array_equal(d.routed.cpu().numpy(), routed), step
        assert same_state(d, st), step


def _tables_state(d: DevState):
    return [d.table, d.map_cold, d.slot_expert, d.slot_stamp, d.routed, d.step, d.n_miss]


@pytest.mark.parametrize("E,S,thresh,max_ins,M,k,blk,seed", [
    (64, 48, 0.5, 48, 4, 6, 16, 11), (288, 64, 0.99, 64, 8, 8, 16, 12), (384, 256, 0.99, 64, 32, 8, 32, 13),
    (1024, 512, 0.99, 256, 500, 8, 16, 14), (16, 16, 1.0, 16, 3, 4, 64, 15), (96, 64, 0.99, 64, 5, 8, 32, 16),
    (64, 48, 0.1, 48, 4, 6, 16, 17)])
def test_manage_tables_one_launch_equals_composed(dev, E, S, thresh, max_ins, M, k, blk, seed):
    """r9k_lru_manage_tables (manage + both passes' tables in one launch) against r9k_lru_manage_map + two
    r9k_moe_align launches on a twin state: every state array and both table sets (the whole capacity) bit for bit
    after every step, with the host tables skipped on some steps; the state also against the oracle's manager. On
    every other step (M <= 64 rows) the launch also quantises M activation rows: xq / xs bit for bit against
    quant_rows_fp8 (rows of 16 + more waves than rows, a hidden size that leaves lanes idle, a padded row stride).
    Steps of at most 64 routed rows whose experts are all resident take the launch's ballot path (no installs); the
    cases include a 32-row block there and a distinct-expert threshold that sends all-resident steps to the
    read-through branch."""
    print(f"manage+tables E={E} S={S} M={M} k={k} blk={blk}", flush=True)
    rng = np.random.default_rng(seed)
    a, b = DevState(dev, E, S, max_ins), DevState(dev, E, S, max_ins)
    st = O.LruState(E, S)
    max_distinct = int(S * thresh)
    hot = rng.permutation(E)[: max(1, S // 2)]
    L = C._L()
    s_ = torch.cuda.current_stream().cuda_stream
    for step in range(40):
        if step == 25:
            hot = rng.permutation(E)[: max(1, S // 2)]
        pool = np.arange(E) if step % 7 == 0 else hot
        ids_np = np.stack([rng.choice(pool, size=min(k, pool.size), replace=False) for _ in range(M)]).reshape(-1)
        if step % 5 == 0:
            ids_np = np.concatenate([ids_np, [-1, E, E + 3]])
        O.lru_manage(st, ids_np, max_distinct, max_ins)
        ids = torch.from_numpy(ids_np.astype(np.int32)).to(dev)
        mk = ids.numel()
        cap = K.capacity(mk, E, blk)
        need_cold = step % 3 != 2
        i32 = dict(dtype=torch.int32, device=dev)
        ta = [torch.full((cap,), -7, **i32), torch.full((cap // blk,), -7, **i32), torch.full((1,), -7, **i32),
              torch.full((cap,), -7, **i32), torch.full((cap // blk,), -7, **i32), torch.full((1,), -7, **i32)]
        cold_ptrs = [t.data_ptr() for t in ta[3:]] if need_cold else [0, 0, 0]
        hot_out = torch.full((mk,), -7, **i32)
        quant = step % 2 == 0 and M <= C.QUANT_MAX_ROWS
        qa = ()
        if quant:
            H = (2048, 136, 4096)[step % 3]
            xp = (torch.randn(M, H + 8, generator=torch.Generator().manual_seed(seed * 100 + step)) * 3)
            x = xp.to(torch.bfloat16).to(dev)[:, :H]
            xq = torch.full((M, H), 7, dtype=torch.uint8, device=dev)
            xs = torch.full((M,), -1.0, device=dev)
            qa = (x.data_ptr(), x.stride(0), H, M, xq.data_ptr(), xs.data_ptr())
        rc = L.r9k_lru_manage_tables(ids.data_ptr(), mk, E, S, max_distinct, max_ins, a.table.data_ptr(),
                                     a.map_cold.data_ptr(), a.slot_expert.data_ptr(), a.slot_stamp.data_ptr(),
                                     a.routed.data_ptr(), a.step.data_ptr(), a.miss.data_ptr(), a.n_miss.data_ptr(),
                                     blk, ta[0].data_ptr(), ta[1].data_ptr(), ta[2].data_ptr(), *cold_ptrs,
                                     hot_out.data_ptr(), *(qa or (0, 0, 0, 0, 0, 0)), s_)
        assert rc == 0, rc
        if quant:
            rq, rs = K.quant_rows_fp8(x)
            assert torch.equal(xq, rq.view(torch.uint8)) and torch.equal(xs, rs), (step, H)
        hid, cid = b.manage(ids, max_distinct, max_ins, mapped=True)
        hb = K.moe_align(hid, blk, E)
        cb = K.moe_align(cid, blk, E) if need_cold else None
        torch.cuda.synchronize()
        for x, y in zip(_tables_state(a), _tables_state(b)):
            assert torch.equal(x, y), step
        assert torch.equal(hot_out, hid), step
        n = int(a.n_miss.item())
        assert torch.equal(a.miss[:n], b.miss[:n]), step
        assert same_state(a, st), step
        for x, y in zip(ta[:3], hb):
            assert torch.equal(x, y), step
        if need_cold:
            for x, y in zip(ta[3:], cb):
                assert torch.equal(x, y), step
        else:
            assert bool((ta[3] == -7).all()) and bool((ta[5] == -7).all()), step


@pytest.mark.parametrize("blk,M", [(24, 16), (48, 16), (24, 5), (48, 3)])
def test_manage_tables_block_not_power_of_two(dev, blk, M):
    """The one-launch manage + tables at a block size that is not a power of two (the entry accepts any; the routing
    entries require powers of two, so this is the table builders' division path): the resident pass's tables over the
    whole capacity equal the oracle's align of the slot ids the launch wrote, bit for bit, over several steps. With
    M = 5 / 3 rows (40 / 24 routed) the steps after the first route to resident experts only, the launch's ballot
    path."""
    print(f"manage+tables blk={blk} M={M}", flush=True)
    E, S, max_ins, k = 288, 64, 64, 8
    rng = np.random.default_rng(blk + M)
    a = DevState(dev, E, S, max_ins)
    L = C._L()
    s_ = torch.cuda.current_stream().cuda_stream
    i32 = dict(dtype=torch.int32, device=dev)
    pool = rng.permutation(E)[: S // 2] if M * k <= 64 else np.arange(E)
    for step in range(6):
        ids = torch.from_numpy(np.stack([rng.choice(pool, size=k, replace=False) for _ in range(M)])
                               .reshape(-1).astype(np.int32)).to(dev)
        mk = ids.numel()
        cap = K.capacity(mk, E, blk)
        ta = [torch.full((cap,), -7, **i32), torch.full((cap // blk,), -7, **i32), torch.full((1,), -7, **i32)]
        hot_out = torch.full((mk,), -7, **i32)
        rc = L.r9k_lru_manage_tables(ids.data_ptr(), mk, E, S, S, max_ins, a.table.data_ptr(),
                                     a.map_cold.data_ptr(), a.slot_expert.data_ptr(), a.slot_stamp.data_ptr(),
                                     a.routed.data_ptr(), a.step.data_ptr(), a.miss.data_ptr(), a.n_miss.data_ptr(),
                                     blk, ta[0].data_ptr(), ta[1].data_ptr(), ta[2].data_ptr(), 0, 0, 0,
                                     hot_out.data_ptr(), 0, 0, 0, 0, 0, 0, s_)
        assert rc == 0, rc
        torch.cuda.synchronize()
        so, eo, no = O.align(hot_out.cpu().numpy(), E, blk)
        assert so.size == cap, (so.size, cap)
        assert np.array_equal(ta[0].cpu().numpy(), so), step
        assert np.array_equal(ta[1].cpu().numpy(), eo), step
        assert int(ta[2].item()) == int(no[0]), step


def test_r4d_lru_fused_reference_sizing(dev):
    """The reference's entry with vLLM's table lengths (L = min(mk * bs, mk + E (bs - 1)) while mk < E): the tables
    equal this library's over their first L / NB entries and nothing past L / NB is written; E > 1024 is not served
    (2, nothing changes)."""
    E, S, max_ins, bs = 288, 64, 64, 16
    rng = np.random.default_rng(21)
    a, b = DevState(dev, E, S, max_ins), DevState(dev, E, S, max_ins)
    L = C._L()
    s_ = torch.cuda.current_stream().cuda_stream
    for M in (1, 4, 40, 300):
        ids = torch.from_numpy(np.stack([rng.choice(E, 8, replace=False) for _ in range(M)]).reshape(-1)
                               .astype(np.int32)).to(dev)
        mk = ids.numel()
        Lr = min(mk * bs, mk + E * (bs - 1)) if mk < E else mk + E * (bs - 1)
        NB = -(-Lr // bs)
        i32 = dict(dtype=torch.int32, device=dev)
        bufs = [torch.full((Lr + 64,), -7, **i32), torch.full((NB + 8,), -7, **i32), torch.full((1,), -7, **i32),
                torch.full((Lr + 64,), -7, **i32), torch.full((NB + 8,), -7, **i32), torch.full((1,), -7, **i32)]
        rc = L.r4d_lru_fused(ids.data_ptr(), mk, E, S, S, max_ins, a.table.data_ptr(), a.map_cold.data_ptr(),
                             a.slot_expert.data_ptr(), a.slot_stamp.data_ptr(), a.routed.data_ptr(),
                             a.step.data_ptr(), a.miss.data_ptr(), a.n_miss.data_ptr(), bs, Lr, NB,
                             *[t.data_ptr() for t in bufs], s_)
        assert rc == 0, rc
        hid, cid = b.manage(ids, S, max_ins, mapped=True)
        hb, cb = K.moe_align(hid, bs, E), K.moe_align(cid, bs, E)
        torch.cuda.synchronize()
        print(f"  r4d_lru_fused M={M}: L={Lr} NB={NB} npad hot {int(bufs[2].item())} cold {int(bufs[5].item())}",
              flush=True)
        for (so, eo, no), (sr, er, nr) in (((bufs[0], bufs[1], bufs[2]), hb), ((bufs[3], bufs[4], bufs[5]), cb)):
            assert torch.equal(no, nr)
            assert torch.equal(so[:Lr], sr[:Lr]) and bool((so[Lr:] == -7).all())
            assert torch.equal(eo[:NB], er[:NB]) and bool((eo[NB:] == -7).all())
        for x, y in zip(_tables_state(a), _tables_state(b)):
            assert torch.equal(x, y)
    big = DevState(dev, 2048, 64, 64)
    before = [t.clone() for t in _tables_state(big)]
    ids = torch.randint(0, 2048, (64,), dtype=torch.int32, device=dev)
    mk, Lr = 64, 64 * bs
    out = [torch.empty(Lr, dtype=torch.int32, device=dev) for _ in range(6)]
    rc = L.r4d_lru_fused(ids.data_ptr(), mk, 2048, 64, 64, 64, big.table.data_ptr(), big.map_cold.data_ptr(),
                         big.slot_expert.data_ptr(), big.slot_stamp.data_ptr(), big.routed.data_ptr(),
                         big.step.data_ptr(), big.miss.data_ptr(), big.n_miss.data_ptr(), bs, Lr, Lr // bs,
                         *[t.data_ptr() for t in out], s_)
    torch.cuda.synchronize()
    assert rc == 2
    for x, y in zip(_tables_state(big), before):
        assert torch.equal(x, y)


def test_lru_gather_copies_listed_slabs(dev):
    E, S = 12, 5
    print("lru gather", flush=True)
    g = torch.Generator().manual_seed(5)
    host = [C.uva_empty((E, b), torch.uint8) for b in (4096, 1040, 48, 16)]
    for h in host:
        h.copy_(torch.randint(0, 256, h.shape, generator=g, dtype=torch.int32).to(torch.uint8))
    arena = [torch.full((S, h.shape[1]), 7, dtype=torch.uint8, device=dev) for h in host]
    miss = torch.tensor([[9, 3], [0, 0], [11, 4], [5, 1]], dtype=torch.int32, device=dev)
    n_miss = torch.tensor([3], dtype=torch.int32, device=dev)            # the fourth pair is not listed
    args = []
    for a, h in zip(arena, host):
        args += [a.data_ptr(), h.data_ptr(), h.shape[1]]
    args += [0, 0, 0, 0, 0, 0]
    assert C._L().r4d_lru_gather(*args, miss.data_ptr(), n_miss.data_ptr(), 4, 2,
                                 torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    for a, h in zip(arena, host):
        a = a.cpu()
        for e, s in ((9, 3), (0, 0), (11, 4)):
            assert torch.equal(a[s], h[e])
        assert torch.all(a[1] == 7) and torch.all(a[2] == 7)


def test_two_pass_gemms_equal_one_pass_over_host_store(dev, monkeypatch):
    """The reference's test_cache_moe.py sequence: E=64, S=48 (max_distinct 24), 4 tokens x top-6 from a 24-expert
    working set, every 7th step uniform over E, a working-set shift at step 30."""
    monkeypatch.setenv("R9K_LRU_THRESH", "0.5")
    E, S, M, topk = 64, 48, 4, 6
    N1, K1, N2, K2 = 640, 2560, 2560, 320
    w1, w2 = make_w(dev, E, N1, K1, 11), make_w(dev, E, N2, K2, 12)
    hw13, hw2 = C.to_host(w1.wq), C.to_host(w2.wq)
    cache = C.LayerCache(0, hw13, hw2, w1.wsr, w2.wsr, N1, K1, N2, K2, S)
    ref1 = K.Mxfp4Experts(hw13, cache.h_s13, N1, K1)
    ref2 = K.Mxfp4Experts(hw2, cache.h_s2, N2, K2)
    st = O.LruState(E, S)                                 # the warm start: experts 0..S-1 in slots 0..S-1
    st.table[:S] = np.arange(S)
    st.map_cold[:S] = -1
    st.slot_expert[:] = np.arange(S)
    st.slot_stamp[:] = -np.arange(S)
    g = torch.Generator().manual_seed(1)
    hot_pref = torch.randperm(E, generator=g)[:24]
    for step in range(40):
        if step == 30:
            hot_pref = torch.randperm(E, generator=g)[:24]
        pool = hot_pref if step % 7 else torch.arange(E)
        ids = torch.stack([pool[torch.randperm(pool.numel(), generator=g)[:topk]] for _ in range(M)])
        ids = ids.to(torch.int32).to(dev)
        tw = torch.rand(M * topk, generator=g).to(dev)
        x = (torch.randn(M, K1, generator=g) * 0.5).to(torch.bfloat16).to(dev)
        h = (torch.randn(M * topk, K2, generator=g) * 0.5).to(torch.bfloat16).to(dev)
        xq, xs = K.quant_rows_fp8(x)
        hq, hs = K.quant_rows_fp8(h)
        numel = M * topk
        r1 = torch.zeros(numel, N1, dtype=torch.bfloat16, device=dev)
        r2 = torch.zeros(numel, N2, dtype=torch.bfloat16, device=dev)
        sid, eid, ntpp = K.moe_align(ids, K.MOE_BLOCK, E)
        K.moe_gemm(xq, xs, ref1, r1, sid, eid, ntpp, numel, topk, None, num_experts=E)
        K.moe_gemm(hq, hs, ref2, r2, sid, eid, ntpp, numel, 1, tw, num_experts=E)
        (h1, h2), (c1, c2) = cache.hot(), cache.cold()
        o1 = torch.zeros_like(r1)
        o2 = torch.zeros_like(r2)
        if step % 2:
            hot_al, cold_al = cache.update_fused(ids, K.MOE_BLOCK)
        else:
            cache.update(ids)
            hot_al = K.moe_align(ids, K.MOE_BLOCK, E, cache.table)
            cold_al = K.moe_align(ids, K.MOE_BLOCK, E, cache.map_cold)
        for (W1, W2), al in (((h1, h2), hot_al), ((c1, c2), cold_al)):
            K.moe_gemm(xq, xs, W1, o1, *al, numel, topk, None, num_experts=E)
            K.moe_gemm(hq, hs, W2, o2, *al, numel, 1, tw, num_experts=E)
        torch.cuda.synchronize()
        _, misses = O.lru_manage(st, ids.cpu().numpy(), cache.max_distinct, cache.max_inserts)
        same = torch.equal(o1.view(torch.int16), r1.view(torch.int16)) and \
            torch.equal(o2.view(torch.int16), r2.view(torch.int16))
        state = same_state(cache, st)
        nm = int(cache.n_miss.item())
        print(f"  step {step:2d}: inserts {nm:2d} bit-identical {same} state {state}", flush=True)
        assert same and state
        assert [tuple(x) for x in cache.miss[:nm].cpu().tolist()] == misses
        # the arena holds the host bytes of every resident expert
        for s_, e_ in enumerate(cache.slot_expert.cpu().tolist()):
            if e_ >= 0 and step % 10 == 9:
                assert torch.equal(cache.a_w2[s_].cpu(), hw2[e_]) and torch.equal(cache.a_s13[s_].cpu(), cache.h_s13[e_])


@pytest.mark.parametrize("T", [1, 16, 64])
def test_cached_layer_equals_resident_layer(dev, T):
    E, H, I, topk, S = 288, 2048, 512, 8, 64
    print(f"cached layer T={T}", flush=True)
    W13, W2 = make_w(dev, E, 2 * I, H, 21), make_w(dev, E, H, I, 22)
    cache = C.LayerCache(0, C.to_host(W13.wq), C.to_host(W2.wq), W13.wsr, W2.wsr, 2 * I, H, H, I, S)
    plain = R9700Mxfp4Experts.standalone(W13.wsr, W2.wsr)
    cached = R9700Mxfp4Experts.standalone(cache.h_s13, cache.h_s2)
    cached.r9k_cache = cache
    g = torch.Generator().manual_seed(31 + T)
    for step in range(4):
        x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
        logits = torch.randn(T, E, generator=g).to(torch.bfloat16).to(dev)
        w, ids = K.moe_topk(logits, topk, True)
        o0 = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
        o1 = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
        plain.apply(o0, x, W13.wq, W2.wq, w, ids, "silu", E, None, None, None, None, None, None, False)
        cached.apply(o1, x, cache.h_w13, cache.h_w2, w, ids, "silu", E, None, None, None, None, None, None, False)
        torch.cuda.synchronize()
        same = torch.equal(o0.view(torch.int16), o1.view(torch.int16))
        print(f"  step {step}: inserts {int(cache.n_miss.item())} bit-identical {same}", flush=True)
        assert same


def test_stage_map_numbers_routed_cold_experts(dev):
    """r9k_lru_stage_map against a CPU restatement of its contract: the routed experts whose table entry is -1,
    numbered in ascending expert order (stage_map, the (expert, index) miss list, the count), capped at cap."""
    g = torch.Generator().manual_seed(61)
    for E, mk, cap, seed in ((288, 512, 224, 1), (1500, 3000, 1400, 2), (64, 40, 5, 3), (16, 0, 8, 4)):
        table = torch.full((E,), -1, dtype=torch.int32)
        res = torch.randperm(E, generator=g)[: E // 3]
        table[res] = torch.arange(res.numel(), dtype=torch.int32)
        ids = torch.randint(-1, E, (mk,), generator=g, dtype=torch.int32)
        sm = torch.full((E,), -7, dtype=torch.int32, device=dev)
        miss = torch.full((max(cap, 1), 2), -7, dtype=torch.int32, device=dev)
        n = torch.full((1,), -7, dtype=torch.int32, device=dev)
        idd, td = ids.to(dev), table.to(dev)
        rc = C._L().r9k_lru_stage_map(idd.data_ptr(), mk, E, td.data_ptr(), cap, sm.data_ptr(), miss.data_ptr(),
                                      n.data_ptr(), torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        torch.cuda.synchronize()
        routed = np.zeros(E, dtype=bool)
        for e in ids.tolist():
            if 0 <= e < E:
                routed[e] = True
        cold = [e for e in range(E) if routed[e] and int(table[e]) < 0]
        want = np.full(E, -1, dtype=np.int32)
        for k, e in enumerate(cold[:cap]):
            want[e] = k
        print(f"stage map E={E} mk={mk} cap={cap}: {len(cold)} cold", flush=True)
        assert np.array_equal(sm.cpu().numpy(), want)
        assert int(n.item()) == min(len(cold), cap)
        got = miss.cpu().numpy()[: min(len(cold), cap)]
        assert np.array_equal(got[:, 0], np.array(cold[:cap], dtype=np.int32).reshape(-1)) if cold else True
        assert np.array_equal(got[:, 1], np.arange(min(len(cold), cap), dtype=np.int32))


@pytest.mark.parametrize("T", [16, 64])
def test_staged_cold_pass_equals_resident_layer(dev, monkeypatch, T):
    """R9K_STAGE_COLD=1: a config 2 layer whose wide steps stage the cold experts into VRAM (one gather) and run the
    cold pass over that copy equals the same layer without a cache, bit for bit, over several steps."""
    monkeypatch.setenv("R9K_STAGE_COLD", "1")
    E, H, I, topk, S = 288, 2048, 512, 8, 64
    print(f"staged cached layer T={T}", flush=True)
    W13, W2 = make_w(dev, E, 2 * I, H, 71), make_w(dev, E, H, I, 72)
    cache = C.LayerCache(0, C.to_host(W13.wq), C.to_host(W2.wq), W13.wsr, W2.wsr, 2 * I, H, H, I, S)
    assert cache.stage is not None and cache.stage_cap == E - S
    plain = R9700Mxfp4Experts.standalone(W13.wsr, W2.wsr)
    cached = R9700Mxfp4Experts.standalone(cache.h_s13, cache.h_s2)
    cached.r9k_cache = cache
    g = torch.Generator().manual_seed(73 + T)
    for step in range(3):
        x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
        logits = torch.randn(T, E, generator=g).to(torch.bfloat16).to(dev)
        w, ids = K.moe_topk(logits, topk, True)
        o0 = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
        o1 = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
        plain.apply(o0, x, W13.wq, W2.wq, w, ids, "silu", E, None, None, None, None, None, None, False)
        cached.apply(o1, x, cache.h_w13, cache.h_w2, w, ids, "silu", E, None, None, None, None, None, None, False)
        torch.cuda.synchronize()
        routed = set(ids.reshape(-1).tolist())
        cold = sum(1 for e in routed if int(cache.table[e].item()) < 0)
        same = torch.equal(o0.view(torch.int16), o1.view(torch.int16))
        print(f"  step {step}: {cold} cold experts staged ({int(cache.stage_n.item())}), bit-identical {same}",
              flush=True)
        assert int(cache.stage_n.item()) == cold
        assert same


def test_update_fused_graph_replays_equal_eager_twin(dev):
    E, S, topk, M = 64, 48, 6, 8
    N1, K1, N2, K2 = 64, 256, 256, 64
    print("cache graph replay", flush=True)
    caches = []
    for _ in range(2):
        w1, w2 = make_w(dev, E, N1, K1, 41), make_w(dev, E, N2, K2, 42)
        caches.append(C.LayerCache(0, C.to_host(w1.wq), C.to_host(w2.wq), w1.wsr, w2.wsr, N1, K1, N2, K2, S))
    a, b = caches
    g = torch.Generator().manual_seed(43)

    def route(m):
        return torch.stack([torch.randperm(E, generator=g)[:topk] for _ in range(m)]).to(torch.int32).to(dev)

    ids = route(M)
    a.update_fused(ids, K.MOE_BLOCK)
    b.update_fused(ids, K.MOE_BLOCK)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        (sh, eh, nh), (sc, ec, nc) = a.update_fused(ids, K.MOE_BLOCK)
    torch.cuda.synchronize()
    if int(a.step.item()) == int(b.step.item()) + 1:        # the capture also ran the step: keep the twin in step
        b.update_fused(ids, K.MOE_BLOCK)
    assert int(a.step.item()) == int(b.step.item())
    for trial in range(8):
        ids.copy_(route(M))
        graph.replay()
        (rh, reh, rnh), (rc, rec, rnc) = b.update_fused(ids, K.MOE_BLOCK)
        torch.cuda.synchronize()
        same = all(torch.equal(x, y) for x, y in ((sh, rh), (eh, reh), (nh, rnh), (sc, rc), (ec, rec), (nc, rnc)))
        same &= torch.equal(a.table, b.table) and torch.equal(a.slot_expert, b.slot_expert)
        same &= torch.equal(a.a_w13, b.a_w13) and torch.equal(a.slot_stamp, b.slot_stamp)
        print(f"  replay {trial}: equal {same}", flush=True)
        assert same
        r3 = route(3)                                      # eager work of another size between replays
        b.update_fused(r3, K.MOE_BLOCK)
        a.update_fused(r3, K.MOE_BLOCK)
        torch.cuda.synchronize()
    # once the largest step has been seen, the align buffers keep one address
    ptr = a._one[2].data_ptr()
    for m in (1, 5, 8, 3):
        hot, _ = a.update_fused(route(m), K.MOE_BLOCK)
        assert hot[0].data_ptr() == ptr
