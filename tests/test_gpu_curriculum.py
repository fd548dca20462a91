"""Ring curriculum traces on the GPU (zx_ring_curriculum_trace) against the oracle, and
a Belady schedule across a phase change."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from zenyx_amd import kv
from zenyx_amd.train.dynamic_ring_curriculum import CurriculumPhase, RingDegreeScheduler

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


@pytest.mark.parametrize("degrees,ctx,L,stride", [([4], [32], 3, 32), ([3], [7], 2, 7), ([8, 8], [5, 3], 4, 6),
                                                  ([1, 2, 4, 8], [16, 32, 64, 128], 5, 128),
                                                  ([6, 5, 7], [1000, 999, 1001], 3, 1024)])
def test_curriculum_trace_matches_oracle(degrees, ctx, L, stride):
    print(f"curriculum trace {degrees} {ctx} L={L}", flush=True)
    got = kv.ring_curriculum_trace(degrees, ctx, L, stride, device=DEV).cpu().numpy()
    assert np.array_equal(got, O.ring_curriculum_trace(degrees, ctx, L, stride))


def test_curriculum_trace_rejects_bad_arguments():
    with pytest.raises(ValueError):
        kv.ring_curriculum_trace([0], [4], 2, 4, device=DEV)
    with pytest.raises(ValueError):
        kv.ring_curriculum_trace([2], [9], 2, 8, device=DEV)  # pages per layer > layer stride


def test_belady_across_a_phase_change():
    s = RingDegreeScheduler([CurriculumPhase("short", 2, 2048, 1), CurriculumPhase("long", 4, 8192)],
                            num_devices=4)
    L, pt = 6, 64
    trace = s.access_trace([0, 1, 2], L, page_tokens=pt, device=DEV)
    n_pages = L * s.layer_stride(pt)
    want = O.ring_curriculum_trace([2, 4, 4], [32, 128, 128], L, 128)
    assert np.array_equal(trace.cpu().numpy(), want)
    cap = n_pages // 3
    sim = kv.BeladyTraceSim(trace, n_pages, cap)
    sim.run()
    pos, page = sim.evictions()
    ep, eg, st = O.belady_simulate(want, n_pages, cap)
    assert np.array_equal(pos.numpy(), ep) and np.array_equal(page.numpy(), eg)
    assert sim.stats()["misses"] == st["misses"]
