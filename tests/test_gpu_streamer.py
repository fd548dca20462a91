"""LayerWeightStreamer on the GPU (parameter_streamer.py:32-87): bytes arrive intact, the
caller's stream waits for prefetched copies, residency follows the reference."""
import numpy as np
import pytest
import torch

from zenyx_amd.streaming import LayerWeightStreamer, ParameterStore
from test_streamer_cpu import RefStreamer

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _store():
    g = torch.Generator().manual_seed(3)
    store, host = ParameterStore(), {}
    shapes = [((1000, 37), torch.bfloat16), ((5 << 20,), torch.float32), ((3, 0), torch.float16),
              ((7, 11, 13), torch.int8), ((1 << 22,), torch.bfloat16), ((1,), torch.float32)]
    for i, (shape, dt) in enumerate(shapes):
        t = (torch.randn(shape, generator=g) * 100).to(dt)
        host[f"l{i}"] = t.clone()
        store.register(f"l{i}", t)
    return store, host


def test_streamed_layers_are_exact():
    store, host = _store()
    s = LayerWeightStreamer(store, DEV, max_resident_layers=2)
    for lid in host:
        assert store.load(lid).is_pinned() or store.load(lid).numel() == 0  # nothing to pin
    for lid in host:
        s.prefetch(lid)
    for lid in host:
        got = s.get(lid).clone()  # a kernel on the current stream, ordered after the copy
        assert got.device.type == "cuda" and got.dtype == host[lid].dtype
        assert torch.equal(got.cpu(), host[lid]), lid


def test_prefetch_pipeline_under_compute():
    """prefetch(i + 1) while layer i is in use, as StreamingExecutionEngine does
    (engine.py:72-78), with large layers so copies and kernels overlap."""
    store = ParameterStore()
    n, numel = 8, 16 << 20
    for i in range(n):
        store.register(f"w{i}", torch.full((numel,), float(i), dtype=torch.float32))
    s = LayerWeightStreamer(store, DEV, max_resident_layers=2)
    sums = []
    for i in range(n):
        if i + 1 < n:
            s.prefetch(f"w{i + 1}")
        w = s.get(f"w{i}")
        sums.append((w * 2.0).sum())
    torch.cuda.synchronize()
    assert [float(x) for x in sums] == [2.0 * i * numel for i in range(n)]


def test_residency_matches_reference_on_gpu():
    store, host = _store()
    s = LayerWeightStreamer(store, DEV, max_resident_layers=3)
    ref = RefStreamer(3)
    rng = np.random.default_rng(1)
    ids = list(host)
    for _ in range(200):
        op, lid = rng.integers(0, 3), ids[rng.integers(0, len(ids))]
        if op == 0:
            s.prefetch(lid), ref.prefetch(lid)
        elif op == 1:
            s.get(lid), ref.get(lid)
        else:
            s.evict(lid), ref.evict(lid)
        assert list(s._resident) == list(ref._resident)
    for lid in list(s._resident):
        assert torch.equal(s.get(lid).cpu(), host[lid])


def test_engine_call_order_and_loss():
    """StreamingExecutionEngine (engine.py:59-103): per layer prefetch(next), get, compute,
    update_future(i + 1), touch, evict(victims); the loss and gradients equal a plain
    forward/backward of the same model."""
    import copy

    from oracle import oracle as O
    from zenyx_amd.streaming import engine as E

    torch.manual_seed(0)
    model = torch.nn.Sequential(torch.nn.Linear(16, 32), torch.nn.ReLU(), torch.nn.Linear(32, 32),
                                torch.nn.Linear(32, 8), torch.nn.Linear(8, 4)).to(DEV)
    twin = copy.deepcopy(model)
    eng = E.StreamingExecutionEngine(model, DEV, E.StreamingConfig(max_hbm_layers=2))
    calls = []
    for obj, names in ((eng.weight_streamer, ("prefetch", "get", "evict")), (eng.cache, ("update_future", "touch"))):
        for nm in names:
            orig = getattr(obj, nm)

            def rec(*a, _orig=orig, _nm=nm):
                r = _orig(*a)
                calls.append((_nm,) + tuple(a) + ((tuple(r),) if _nm == "touch" else ()))
                return r
            setattr(obj, nm, rec)
    x = torch.randn(8, 16, device=DEV)
    y = torch.randn(8, 4, device=DEV)
    loss = eng.run_forward_backward(x, y, torch.nn.functional.mse_loss)
    # the reference's order, with victims from its own linear-scan cache (belady.py:14-55)
    ref_cache = O.RefBeladyApproxCache(2)
    names = [n for n, _ in model.named_children()]
    want = []
    for i, n in enumerate(names):
        if i + 1 < len(names):
            want.append(("prefetch", names[i + 1]))
        want.append(("get", n))
        ref_cache.update_future(n, i + 1)
        want.append(("update_future", n, i + 1))
        ev = ref_cache.touch(n)
        want.append(("touch", n, tuple(ev)))
        want.extend(("evict", v) for v in ev)
    assert calls == want
    ref_loss = torch.nn.functional.mse_loss(twin(x), y)
    ref_loss.backward()
    assert loss == float(ref_loss.item())
    for p, q in zip(model.parameters(), twin.parameters()):
        assert torch.equal(p.grad, q.grad)
    # streamed copies hold each layer's flattened state
    for n, m in model.named_children():
        st = [t.detach().reshape(-1) for t in m.state_dict().values()]
        want_flat = torch.cat(st) if st else torch.zeros(1, device=DEV)
        assert torch.equal(eng.store.load(n).to(DEV), want_flat.to(eng.store.load(n).dtype))
