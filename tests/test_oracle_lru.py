"""Pins the oracle's LRU expert-cache manager (oracle.lru_manage, the reference's
kernels/third_party/davetha/r4d_lru.hip:187-274) three ways:

* against a serial simulation written here independently: one argmin over the evictable (stamp, slot) pairs per
  insert, the slot taken out of the pool after each install (the form the reference's own comments give for the
  batched ranking, r4d_lru.hip:80-95), over random step sequences with padding, out-of-range ids, wide steps and
  insert caps;
* against a seven-step sequence worked by hand (ties to the lower slot, read-through leaving stamps alone, an
  eviction, an insert cap of two);
* through the cache invariants the reference's test checks (tests/test_cache_moe.py:87-93): table and map_cold
  complementary, slot_expert the inverse of table, no expert routed this step evicted, every inserted expert
  resident."""
import numpy as np
import pytest

from oracle import oracle as O


def serial_manage(table, map_cold, slot_expert, slot_stamp, step, ids, E, S, max_distinct, max_inserts):
    step += 1
    routed = sorted({int(e) for e in ids if 0 <= e < E})
    if len(routed) > max_distinct:
        return step, []
    for e in routed:
        if table[e] >= 0:
            slot_stamp[table[e]] = step
    misses = [e for e in routed if table[e] < 0][:max_inserts]
    pool = [s for s in range(S) if not (slot_expert[s] >= 0 and slot_expert[s] in routed)]
    done = []
    for e in misses:
        if not pool:
            break
        best = min(pool, key=lambda s: (int(slot_stamp[s]), s))
        pool.remove(best)
        old = slot_expert[best]
        if old >= 0:
            table[old] = -1
            map_cold[old] = old
        slot_expert[best], slot_stamp[best] = e, step
        table[e], map_cold[e] = best, -1
        done.append((e, best))
    return step, done


def check_invariants(st, ids, misses):
    E = st.E
    assert np.all((st.table >= 0) ^ (st.map_cold >= 0))
    assert np.all(st.map_cold[st.map_cold >= 0] == np.flatnonzero(st.map_cold >= 0))
    for s, e in enumerate(st.slot_expert):
        if e >= 0:
            assert st.table[e] == s
    assert np.count_nonzero(st.table >= 0) == np.count_nonzero(st.slot_expert >= 0)
    for e, s in misses:
        assert st.table[e] == s and st.slot_expert[s] == e


@pytest.mark.parametrize("E,S,thresh,max_ins,M,k,seed", [
    (64, 48, 0.5, 48, 4, 6, 1), (288, 64, 0.99, 64, 8, 8, 2), (16, 16, 1.0, 16, 3, 4, 3), (40, 8, 0.99, 2, 2, 4, 4),
    (300, 256, 0.99, 64, 32, 8, 5), (8, 3, 1.0, 3, 1, 2, 6),
])
def test_lru_manage_equals_serial_argmin(E, S, thresh, max_ins, M, k, seed):
    rng = np.random.default_rng(seed)
    st = O.LruState(E, S)
    t2, m2 = st.table.copy(), st.map_cold.copy()
    se2, ss2, step2 = st.slot_expert.copy(), st.slot_stamp.copy(), 0
    max_distinct = int(S * thresh)
    hot = rng.permutation(E)[: max(1, S // 2)]
    for step in range(80):
        if step == 50:
            hot = rng.permutation(E)[: max(1, S // 2)]
        pool = np.arange(E) if step % 7 == 0 else hot
        ids = np.stack([rng.choice(pool, size=min(k, pool.size), replace=False) for _ in range(M)]).reshape(-1)
        if step % 5 == 0:
            ids = np.concatenate([ids, [-1, E, E + 3]])           # padding and out-of-range ids are ignored
        routed, misses = O.lru_manage(st, ids, max_distinct, max_ins)
        step2, done = serial_manage(t2, m2, se2, ss2, step2, ids, E, S, max_distinct, max_ins)
        assert misses == done, step
        assert st.step == step2
        assert np.array_equal(st.table, t2) and np.array_equal(st.map_cold, m2)
        assert np.array_equal(st.slot_expert, se2) and np.array_equal(st.slot_stamp, ss2)
        assert np.array_equal(np.flatnonzero(routed), np.unique(ids[(ids >= 0) & (ids < E)]))
        check_invariants(st, ids, misses)
        # nothing routed this step was evicted: every routed expert resident before the step still is
        if len(np.unique(ids[(ids >= 0) & (ids < E)])) <= max_distinct:
            assert all(st.table[e] >= 0 for e, _ in misses)


def test_lru_manage_hand_worked():
    st = O.LruState(6, 2)
    steps = [([3], 2, 1, [(3, 0)], [3, -1], [1, 0]),
             ([1, 3], 2, 1, [(1, 1)], [3, 1], [2, 2]),
             ([5], 2, 1, [(5, 0)], [5, 1], [3, 2]),              # tie on stamp 2: the lower slot goes
             ([0, 2, 4], 2, 1, [], [5, 1], [3, 2]),              # 3 distinct > 2: read through, stamps untouched
             ([0, 1], 2, 1, [(0, 0)], [0, 1], [5, 5]),
             ([2, 4], 2, 2, [(2, 0), (4, 1)], [2, 4], [6, 6]),
             ([-1, 7, 2], 2, 2, [], [2, 4], [7, 6])]
    for i, (ids, md, mi, exp_miss, exp_se, exp_st) in enumerate(steps):
        _, misses = O.lru_manage(st, ids, md, mi)
        assert misses == exp_miss, i
        assert st.slot_expert.tolist() == exp_se and st.slot_stamp.tolist() == exp_st, i
    assert st.step == 7
    assert st.table.tolist() == [-1, -1, 0, -1, 1, -1]
    assert st.map_cold.tolist() == [0, 1, -1, 3, -1, 5]


def test_lru_gather_copies_listed_rows_only():
    store = np.arange(10 * 4).reshape(10, 4)
    arena = np.full((3, 4), -7)
    O.lru_gather(arena, store, [(9, 2), (4, 0)])
    assert arena[2].tolist() == store[9].tolist() and arena[0].tolist() == store[4].tolist()
    assert arena[1].tolist() == [-7] * 4
