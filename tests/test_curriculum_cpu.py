"""Dynamic ring curriculum (README.md:162-165, 330, 345; behaviour defined by this build):
RingDegreeScheduler's phase / degree / context lookup and loss-driven advance, and the
oracle's curriculum ring trace pinned against the constant-degree ring trace (itself
pinned against build_ring_timeline, kv_tiering.py:69-73) and structural invariants."""
import numpy as np
import pytest

from oracle import oracle as O
from zenyx_amd.train.dynamic_ring_curriculum import CurriculumPhase, RingDegreeScheduler


def test_default_curriculum_doubles_degree():
    s = RingDegreeScheduler(num_devices=8, context_length=1 << 20, total_steps=400)
    assert [p.ring_degree for p in s.phases] == [1, 2, 4, 8]
    assert [p.context_length for p in s.phases] == [1 << 17, 1 << 18, 1 << 19, 1 << 20]
    assert [s.degree_at(t) for t in (0, 99, 100, 199, 200, 299, 300, 10 ** 6)] == [1, 1, 2, 2, 4, 4, 8, 8]
    assert s.layer_stride(64) == (1 << 20) // 64


def test_context_ramp_interpolates():
    s = RingDegreeScheduler([CurriculumPhase("a", 2, 1000, 5), CurriculumPhase("b", 4, 2000, 10, ramp_steps=3)],
                            num_devices=4)
    assert [s.context_at(t) for t in range(5, 10)] == [1250, 1500, 1750, 2000, 2000]
    assert s.degree_at(5) == 4 and s.context_at(4) == 1000
    assert s.pages_per_layer(6, 64) == -(-1500 // 64)


def test_adaptive_advance_on_plateau():
    s = RingDegreeScheduler([CurriculumPhase("a", 1, 100, 50), CurriculumPhase("b", 2, 200, 50),
                             CurriculumPhase("c", 4, 400)], num_devices=4, patience=3, min_delta=0.01)
    losses = [5.0, 4.0, 3.0, 2.99, 2.995, 2.992]  # improvements stop after step 2
    moved = [s.observe_loss(t, x) for t, x in enumerate(losses)]
    assert moved == [False, False, False, False, False, True]
    assert s.phase_start(1) == 6 and s.phase_start(2) == 56
    assert s.degree_at(5) == 1 and s.degree_at(6) == 2 and s.degree_at(56) == 4
    # the next plateau moves phase c up as well
    for t, x in zip(range(6, 12), [3.0, 2.0, 1.0, 1.0, 1.0, 1.0]):
        s.observe_loss(t, x)
    assert s.phase_start(2) == 12 and s.degree_at(12) == 4


def test_scheduler_rejects_bad_phases():
    with pytest.raises(ValueError):
        RingDegreeScheduler([CurriculumPhase("a", 16, 100, 5)], num_devices=8)
    with pytest.raises(ValueError):
        RingDegreeScheduler([CurriculumPhase("a", 2, 100, 0), CurriculumPhase("b", 4, 100, 5)])
    with pytest.raises(ValueError):
        RingDegreeScheduler([CurriculumPhase("a", 2, 100, 5, ramp_steps=9)])
    with pytest.raises(ValueError):
        RingDegreeScheduler()


def test_curriculum_trace_constant_degree_is_the_ring_trace():
    for L, R, S in [(1, 1, 5), (3, 4, 8), (2, 8, 16)]:
        got = O.ring_curriculum_trace([R], [R * S], L, R * S)
        assert np.array_equal(got, O.ring_trace(L, R, S))


@pytest.mark.parametrize("R,P", [(3, 7), (8, 5), (5, 5), (4, 1), (1, 9), (6, 100)])
def test_curriculum_trace_structure(R, P):
    L, stride = 3, 128
    t = O.ring_curriculum_trace([R], [P], L, stride)
    n = 2 * L * R * P
    assert t.size == n
    fwd, bwd = t[:n // 2], t[n // 2:]
    assert np.array_equal(bwd, fwd[::-1])
    for l in range(L):
        seg = fwd[l * R * P:(l + 1) * R * P]
        assert np.all((seg >= l * stride) & (seg < l * stride + P))
        # every page of the layer once per ring step
        for r in range(R):
            assert np.array_equal(np.sort(seg[r * P:(r + 1) * P]), l * stride + np.arange(P))
    # ring step r starts with shard (0 - r) mod R
    seg = fwd[:R * P]
    for r in range(R):
        a = (R - r) % R
        assert seg[r * P] == (a * P // R) % P


def test_curriculum_trace_concatenates_steps():
    t = O.ring_curriculum_trace([2, 4, 4], [6, 12, 9], 2, 12)
    sizes = [2 * 2 * 2 * 6, 2 * 2 * 4 * 12, 2 * 2 * 4 * 9]
    assert t.size == sum(sizes)
    parts = np.split(t, np.cumsum(sizes)[:-1])
    for (R, P), part in zip([(2, 6), (4, 12), (4, 9)], parts):
        assert np.array_equal(part, O.ring_curriculum_trace([R], [P], 2, 12))
