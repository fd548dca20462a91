"""LayerWeightStreamer's residency policy against a line-by-line restatement of the
reference (zenyx/streaming/parameter_streamer.py:32-76), on the CPU device the reference
also supports (no copies involved)."""
from collections import OrderedDict

import numpy as np
import pytest
import torch

from zenyx_amd.streaming import LayerWeightStreamer, ParameterStore


class RefStreamer:
    """parameter_streamer.py:42-76 without the tensors: which layers are resident / pending."""

    def __init__(self, max_resident_layers):
        self.max_resident_layers = max_resident_layers
        self._resident = OrderedDict()
        self._prefetch = {}

    def prefetch(self, lid):
        if lid in self._resident or lid in self._prefetch:
            return
        self._prefetch[lid] = True

    def get(self, lid):
        if lid in self._resident:
            self._resident.move_to_end(lid)
            return
        self._prefetch.pop(lid, None)
        self._resident[lid] = True
        while len(self._resident) > self.max_resident_layers:
            self._resident.popitem(last=False)

    def evict(self, lid):
        self._resident.pop(lid, None)


@pytest.mark.parametrize("seed,cap", [(0, 1), (1, 2), (2, 3), (3, 5)])
def test_residency_matches_reference(seed, cap):
    store = ParameterStore()
    ids = [f"layer{i}" for i in range(7)]
    for i, lid in enumerate(ids):
        store.register(lid, torch.full((3, 4), float(i)))
    s = LayerWeightStreamer(store, torch.device("cpu"), max_resident_layers=cap)
    ref = RefStreamer(cap)
    rng = np.random.default_rng(seed)
    for _ in range(300):
        op, lid = rng.integers(0, 3), ids[rng.integers(0, len(ids))]
        if op == 0:
            s.prefetch(lid), ref.prefetch(lid)
        elif op == 1:
            t = s.get(lid)
            ref.get(lid)
            assert torch.equal(t, store.load(lid))
        else:
            s.evict(lid), ref.evict(lid)
        assert list(s._resident) == list(ref._resident)
        assert set(s._prefetch) == set(ref._prefetch)


def test_unknown_layer_raises_key_error():
    s = LayerWeightStreamer(ParameterStore(), torch.device("cpu"))
    with pytest.raises(KeyError):
        s.get("missing")
    s.prefetch("missing")  # as the reference: the failure surfaces at get()
    with pytest.raises(KeyError):
        s.get("missing")
