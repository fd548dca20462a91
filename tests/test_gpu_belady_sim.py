"""GPU Belady MIN (zx_belady_simulate) against the heap oracle: eviction order (position
and page of every victim), miss/hit counts and per-position miss flags, bit-exact."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from zenyx_amd import kv

pytestmark = pytest.mark.gpu


def run_and_compare(dev, trace, n_pages, capacity, pieces=1):
    sim = kv.BeladyTraceSim(torch.from_numpy(trace).to(dev), n_pages, capacity, record_misses=True)
    cuts = np.linspace(0, len(trace), pieces + 1).astype(int)[1:]
    for c in cuts:
        sim.run(int(c))
    ep, eg, st, mf = O.belady_simulate(trace, n_pages, capacity, miss_flags=True)
    gp, gg = sim.evictions()
    s = sim.stats()
    assert s["evictions"] == st["evictions"]
    assert s["misses"] == st["misses"] and s["hits"] == st["hits"] and s["resident"] == st["resident"]
    np.testing.assert_array_equal(gp.numpy(), ep)
    np.testing.assert_array_equal(gg.numpy(), eg)
    np.testing.assert_array_equal(sim.miss_flags.cpu().numpy(), mf)


def test_reference_known_answer_trace(dev):
    # zenyx/tests/test_streaming.py:14-22 as a page trace: a=0, b=1, c=2
    trace = np.array([0, 1, 2, 0, 2] + [3] * 95 + [1], np.int32)
    sim = kv.BeladyTraceSim(torch.from_numpy(trace).to(dev), 4, 2)
    sim.run()
    pos, page = sim.evictions()
    assert (int(pos[0]), int(page[0])) == (2, 1)
    run_and_compare(dev, trace, 4, 2)


@pytest.mark.parametrize("seed", range(10))
def test_random_traces_small_capacity(dev, seed):
    rng = np.random.default_rng(seed)
    n_pages = int(rng.integers(2, 80))
    cap = int(rng.integers(1, n_pages + 3))
    trace = rng.integers(0, n_pages, int(rng.integers(1, 6000))).astype(np.int32)
    run_and_compare(dev, trace, n_pages, cap, pieces=1 + seed % 3)


@pytest.mark.parametrize("seed", range(3))
def test_random_traces_large(dev, seed):
    rng = np.random.default_rng(50 + seed)
    n_pages = 5000
    # skewed reuse so both hits and misses are common
    trace = (rng.zipf(1.3, 200_000) % n_pages).astype(np.int32)
    for cap in (1, 37, 1200, 4999):
        run_and_compare(dev, trace, n_pages, cap)


# budgets below one layer (0.3, 0.5, 0.75): most windows of the simulator then have victims
# among pages they have just seen (the parking path); (3, 2048, 0.75) is bench.py's
# both-directions tier window: 786,432 accesses, 245,760 evictions
@pytest.mark.parametrize("layers,shard,cap_layers", [(6, 64, 2.5), (10, 256, 3.7), (3, 16, 0.3), (4, 512, 0.5),
                                                     (3, 2048, 0.75)])
def test_ring_schedule_traces(dev, layers, shard, cap_layers):
    ring = 8
    trace = O.ring_trace(layers, ring, shard)
    n_pages = layers * ring * shard
    cap = max(1, int(cap_layers * ring * shard))
    run_and_compare(dev, trace, n_pages, cap, pieces=3)
