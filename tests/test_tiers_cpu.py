"""Three-tier Belady hierarchy (T0 HBM / T1 DRAM / T2 NVMe, README.md:150-154) on the CPU:
the oracle's explicit two-heap hierarchy, pinned against single-level Belady MIN (whose
own pins are in test_oracle.py), and the host bookkeeping of zenyx_amd's planner (slots,
moves, batches) checked by a sequential replay of oracle schedules."""
import numpy as np
import pytest

from oracle import oracle as O
from zenyx_amd.train.belady_tiers import SRC_HIT, SRC_NEW, SRC_T1, SRC_T2, ThreeTierPlan, fifo_slots


def test_tiers_known_answer():
    # worked by hand from the definition: c0 = 2, c1 = 1; keys are next uses, ties among
    # never-again pages go to the smallest id
    t = np.array([0, 1, 2, 0, 3, 1, 4, 0, 2, 3], np.int32)
    src, v0, v1, m = O.belady_tiers(t, 5, 2, 1)
    assert src.tolist() == [3, 3, 3, 0, 3, 1, 3, 0, 2, 1]
    assert v0.tolist() == [-1, -1, 1, -1, 2, 3, 1, -1, 0, 2]
    assert v1.tolist() == [-1, -1, -1, -1, 2, -1, 1, -1, 0, -1]
    assert m == 8


def _traces():
    rng = np.random.default_rng(7)
    out = []
    for n_pages, n in [(6, 60), (30, 400), (200, 3000), (1000, 20000)]:
        out.append((rng.integers(0, n_pages, n).astype(np.int32), n_pages))
        # skewed: a hot set plus a cold tail
        hot = rng.integers(0, max(2, n_pages // 8), n)
        cold = rng.integers(0, n_pages, n)
        out.append((np.where(rng.random(n) < 0.7, hot, cold).astype(np.int32), n_pages))
    out.append((O.ring_trace(3, 4, 8), 3 * 4 * 8))
    out.append((O.ring_trace(5, 8, 16), 5 * 8 * 16))
    return out


@pytest.mark.parametrize("case", range(10))
def test_tiers_equal_nested_min(case):
    """T0 behaves as MIN(c0) and T0 + T1 as MIN(c0 + c1), access by access."""
    trace, n_pages = _traces()[case]
    rng = np.random.default_rng(case)
    for _ in range(3):
        c0 = int(rng.integers(1, max(2, n_pages // 2)))
        c1 = int(rng.integers(0, max(1, n_pages // 2)))
        src, v0, v1, misses = O.belady_tiers(trace, n_pages, c0, c1)
        ep0, eg0, st0, mf0 = O.belady_simulate(trace, n_pages, c0, miss_flags=True)
        ep1, eg1, st1, mf1 = O.belady_simulate(trace, n_pages, c0 + c1, miss_flags=True)
        assert misses == st0["misses"]
        assert np.array_equal(src != SRC_HIT, mf0.astype(bool))
        # union misses: from T2 or new
        assert np.array_equal((src == SRC_T2) | (src == SRC_NEW), mf1.astype(bool))
        # T0 victims are MIN(c0)'s
        pos0 = np.nonzero(v0 >= 0)[0]
        assert np.array_equal(pos0, ep0) and np.array_equal(v0[pos0], eg0)
        # pages leaving T0 + T1 are MIN(c0 + c1)'s victims
        pos1 = np.nonzero(v1 >= 0)[0]
        assert np.array_equal(pos1, ep1) and np.array_equal(v1[pos1], eg1)
        # src 2 vs 3: seen before or not
        seen = np.zeros(n_pages, bool)
        for i, p in enumerate(trace):
            if src[i] in (SRC_T2, SRC_NEW):
                assert (src[i] == SRC_T2) == seen[p]
            seen[p] = True


def test_tiers_without_t1():
    trace, n_pages = _traces()[2]
    src, v0, v1, _ = O.belady_tiers(trace, n_pages, 17, 0)
    ev = v0 >= 0
    assert np.array_equal(v1[ev], v0[ev]) and np.all(v1[~ev] == -1)
    assert not np.any(src == SRC_T1)


def _plan(trace, n_pages, c0, c1, spare):
    src, v0, v1, _ = O.belady_tiers(trace, n_pages, c0, c1)
    nu, pu = O.next_use(trace, n_pages)
    return ThreeTierPlan.from_schedule(trace, n_pages, c0, c1, spare, src, v0, v1, nu, pu)


def _replay_check(plan: ThreeTierPlan):
    """Sequential replay of the plan's slot bookkeeping with explicit owners."""
    n0, n1 = plan.c0 + plan.spare, plan.c1 + plan.spare
    own0, own1 = np.full(n0, -1, np.int64), np.full(n1, -1, np.int64)
    freed0, freed1 = np.full(n0, -(10 ** 9)), np.full(n1, -(10 ** 9))
    where = {}  # page -> (tier, slot)
    tr, src, v0, v1 = plan.trace, plan.src, plan.v0, plan.v1
    for i in range(tr.size):
        p = int(tr[i])
        # departures first
        if src[i] == SRC_T1:
            s = plan.dep1[i]
            assert where[p] == (1, s) and own1[s] == p
            own1[s] = -1
            freed1[s] = i
        if v0[i] >= 0:
            r = int(v0[i])
            s = plan.dep0[i]
            assert where[r] == (0, s) and own0[s] == r
            own0[s] = -1
            freed0[s] = i
            if v1[i] == r:
                where[r] = (2, -1)
            else:
                s1 = plan.adm1[i]
                assert 0 <= s1 < n1 and own1[s1] == -1 and i - freed1[s1] >= plan.spare
                own1[s1] = r
                where[r] = (1, s1)
        if v1[i] >= 0 and v1[i] != v0[i]:
            q = int(v1[i])
            s = plan.dep1[i]
            assert where[q] == (1, s) and own1[s] == q
            own1[s] = -1
            freed1[s] = i
            where[q] = (2, -1)
        if src[i] != SRC_HIT:
            s = plan.adm0[i]
            assert 0 <= s < n0 and own0[s] == -1 and i - freed0[s] >= plan.spare
            if src[i] == SRC_NEW:
                assert p not in where
            elif src[i] == SRC_T2:
                assert where[p] == (2, -1)
            own0[s] = p
            where[p] = (0, s)
        assert where[p] == (0, plan.slot0[i]) and own0[plan.slot0[i]] == p
        assert np.sum(own0 >= 0) <= plan.c0 and np.sum(own1 >= 0) <= plan.c1


@pytest.mark.parametrize("case,c0,c1,spare", [(0, 2, 1, 1), (1, 5, 3, 2), (3, 9, 7, 4), (4, 40, 30, 16),
                                               (8, 20, 16, 8), (9, 100, 60, 32), (5, 50, 0, 8)])
def test_plan_slots_replay(case, c0, c1, spare):
    trace, n_pages = _traces()[case]
    plan = _plan(trace, n_pages, c0, c1, spare)
    _replay_check(plan)


@pytest.mark.parametrize("case,c0,c1,spare", [(4, 40, 30, 16), (9, 100, 60, 32), (6, 300, 200, 64)])
def test_plan_moves_and_batches(case, c0, c1, spare):
    trace, n_pages = _traces()[case]
    plan = _plan(trace, n_pages, c0, c1, spare)
    n = trace.size
    bs = plan.batches(0, n)
    assert bs[0][0] == 0 and bs[-1][1] == n
    assert all(b0[1] == b1[0] for b0, b1 in zip(bs, bs[1:]))
    total = {}
    for a, b in bs:
        assert 0 < b - a <= spare
        m = plan.moves(a, b)
        pages = np.concatenate([m[k][0] for k in m])
        assert len(np.unique(pages)) == len(pages), "a page moves twice in one batch"
        for k in m:
            total[k] = total.get(k, 0) + len(m[k][0])
            assert len(m[k][0]) == len(m[k][1]) == len(m[k][2])
    src, v0, v1 = plan.src, plan.v0, plan.v1
    assert total["t1_t0"] == np.sum(src == SRC_T1)
    assert total["t2_t0"] == np.sum(src == SRC_T2)
    assert total["new"] == np.sum(src == SRC_NEW)
    pos = np.arange(n)
    live0 = plan.last_use[np.maximum(v0, 0)] > pos
    live1 = plan.last_use[np.maximum(v1, 0)] > pos
    assert total["t0_t1"] == np.sum((v0 >= 0) & (v1 != v0) & live0)
    assert total["t0_t2"] == np.sum((v0 >= 0) & (v1 == v0) & live0)
    assert total["t1_t2"] == np.sum((v1 >= 0) & (v1 != v0) & live1)
    # a page read back from T2 was written there (live) earlier
    written = set()
    for a, b in bs:
        m = plan.moves(a, b)
        for p in m["t2_t0"][0]:
            assert int(p) in written
        written.update(int(p) for p in m["t1_t2"][0])
        written.update(int(p) for p in m["t0_t2"][0])


def test_fifo_slots_rejects_bad_sequences():
    with pytest.raises(ValueError):  # departure of a page never admitted
        fifo_slots([0], [1], [1], [2], 4)
    with pytest.raises(ValueError):  # three resident pages in two slots
        fifo_slots([0, 1, 2], [1, 2, 3], [], [], 2)


def test_replay_chunks_respect_cross_direction_order():
    """BeladyKVCacheTieringManager._chunks on random move lists: every chunk waits only for
    a chunk of the other direction issued before it, and every move whose page last moved
    the other way is covered by that wait (or by an earlier chunk of its own stream, which
    waited already), so the two copy streams run in a valid order without a cycle."""
    import numpy as np

    from zenyx_amd.train.belayd_kv_cache_tiering import BeladyKVCacheTieringManager as M

    rng = np.random.default_rng(3)
    for n, pages, cap in [(50, 5, 4), (400, 40, 16), (3000, 300, 64), (3000, 3000, 1024)]:
        page = rng.integers(0, pages, n)
        kind = np.empty(n, np.int8)
        state = {}
        for i, p in enumerate(page):  # alternate per page, as D2H / H2D of one page do
            kind[i] = state.get(int(p), int(rng.integers(0, 2)))
            state[int(p)] = 1 - kind[i]
        chunks = M._chunks(kind, page, cap)
        issued = {0: 0, 1: 0}
        chunk_of = {}  # move index -> (direction, chunk index)
        waited = {0: -1, 1: -1}  # highest chunk of the other direction each stream has waited for
        seen = set()
        for k, idx, wait in chunks:
            assert wait < issued[1 - k], "a chunk waits for one not issued yet"
            waited[k] = max(waited[k], wait)
            assert 0 < len(idx) <= cap and all(kind[i] == k for i in idx)
            for i in idx:
                chunk_of[i] = (k, issued[k])
                seen.add(i)
            issued[k] += 1
            for i in idx:  # this move's page's previous move in the other direction is covered
                prev = [j for j in range(i) if page[j] == page[i]]
                if prev and kind[prev[-1]] != k:
                    pk, pc = chunk_of[prev[-1]]
                    assert pc <= waited[k]
        assert seen == set(range(n))
