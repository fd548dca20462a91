"""The drop-in Python layer on the GPU: zenyx_amd.streaming (reference names and contracts of
zenyx/streaming) and zenyx_amd.train (README Phase-7/8 names), checked against the
reference's own tests, the pure-Python restatements and the C oracle."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from zenyx_amd.streaming import (BeladyApproxCache, KVTierManager, build_ring_timeline,
                                 dequantize_for_bf16_compute, quantize_to_fp8_storage)
from zenyx_amd.train.belayd_kv_cache_tiering import BeladyKVCacheTieringManager, RingAttentionAccessSequence
from zenyx_amd.train.fp8_kv_quantization import FP8KVQuantizer, PagedFP8KVCache, QuantizedRingAttention

pytestmark = pytest.mark.gpu


def bits16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------------ precision.py

def test_reference_precision_roundtrip_shape_dtype(dev):
    """zenyx/tests/test_streaming.py:31-36, on CPU tensors as the reference test uses."""
    x = torch.randn(4, 4)
    q, scale = quantize_to_fp8_storage(x)
    y = dequantize_for_bf16_compute(q, scale)
    assert y.shape == x.shape
    assert y.dtype == torch.bfloat16
    assert q.device.type == "cpu" and q.dtype == torch.int8 and scale.dim() == 0


def test_precision_values_match_reference_expressions(dev):
    g = torch.Generator().manual_seed(3)
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        x = (torch.randn(257, 33, generator=g) * 3).to(dt)
        q, s = quantize_to_fp8_storage(x.to(dev))
        # precision.py:10-11 evaluated by torch on the CPU
        s_ref = x.abs().amax().clamp_min(1e-8) / 127.0
        q_ref = torch.clamp((x / s_ref).round(), -127, 127).to(torch.int8)
        assert torch.equal(q.cpu(), q_ref)
        assert s.cpu().float().item() == s_ref.float().item()
        y = dequantize_for_bf16_compute(q, s)
        assert torch.equal(bits_t(y), bits_t((q_ref.float() * s_ref).to(torch.bfloat16)))


def bits_t(t):
    return t.detach().cpu().view(torch.int16)


# ------------------------------------------------------------------ belady.py

def test_reference_belady_known_answer(dev):
    """zenyx/tests/test_streaming.py:14-22."""
    cache = BeladyApproxCache(capacity=2)
    cache.update_future("a", 1)
    cache.update_future("b", 100)
    cache.update_future("c", 2)
    cache.touch("a")
    cache.touch("b")
    evicted = cache.touch("c")
    assert evicted == ["b"]


@pytest.mark.parametrize("seed", range(6))
def test_belady_cache_matches_restatement(dev, seed):
    rng = np.random.default_rng(seed)
    cap = int(rng.integers(0, 5))
    mine, ref = BeladyApproxCache(cap), O.RefBeladyApproxCache(cap)
    ids = [f"t{i}" for i in range(9)]
    for _ in range(150):
        tid = ids[int(rng.integers(0, len(ids)))]
        if rng.random() < 0.5:
            nu = int(rng.choice([-5, -1, 0, 3, 7, 10**18, 10**20]))
            mine.update_future(tid, nu)
            ref.update_future(tid, nu)
        else:
            assert mine.touch(tid) == ref.touch(tid)
        assert mine.resident == ref.resident


def test_belady_cache_large_incremental(dev):
    """A cache of 1,500 ids whose device tables grow while misses evict (3,000 ids seen,
    next uses rewritten as they go): every touch's victim and the resident set equal the
    restatement of belady.py's linear scan, with distinct keys (no ties)."""
    rng = np.random.default_rng(8)
    cap, n_ids = 1500, 3000
    mine, ref = BeladyApproxCache(cap), O.RefBeladyApproxCache(cap)
    keys = rng.permutation(10 * n_ids)
    k = 0
    for step in range(6000):
        tid = int(rng.integers(0, min(n_ids, 200 + step)))
        nu = int(keys[k % len(keys)]) + (10**6 if step % 7 == 0 else 0)
        k += 1
        mine.update_future(tid, nu)
        ref.update_future(tid, nu)
        assert mine.touch(tid) == ref.touch(tid)
    assert mine.resident == ref.resident and len(mine.resident) == cap


def test_belady_cache_quirks(dev):
    c = BeladyApproxCache(capacity=1)
    for t in "abc":
        c.update_future(t, -1)  # next use <= -1 never qualifies as a victim (belady.py:48-50)
    assert c.touch("a") == [] and c.touch("b") == [] and c.touch("c") == []
    assert c.resident == {"a", "b", "c"}
    z = BeladyApproxCache(capacity=0)  # behaves like capacity 1
    assert z.touch("x") == [] and z.touch("y") == ["x"]


# ------------------------------------------------------------------ kv_tiering.py

class RefTiers:
    """Bookkeeping of kv_tiering.py:26-66 (which block sits in which tier, LRU order)."""

    def __init__(self, c0, c1):
        from collections import OrderedDict

        self.t0, self.t1, self.t2 = OrderedDict(), OrderedDict(), {}
        self.c0, self.c1 = c0, c1

    def put(self, b):
        self.t2[b] = True

    def prefetch(self, b):
        if b in self.t0:
            self.t0.move_to_end(b)
            return
        if b in self.t1:
            self.t1.pop(b)
        else:
            self.t2[b]
        self.t0[b] = True
        while len(self.t0) > self.c0:
            o, _ = self.t0.popitem(last=False)
            self.t1[o] = True
            self._t1()

    def evict(self, b):
        if self.t0.pop(b, None) is not None:
            self.t1[b] = True
            self._t1()

    def _t1(self):
        while len(self.t1) > self.c1:
            o, _ = self.t1.popitem(last=False)
            self.t2[o] = True


def test_kv_tier_manager_lru_and_bytes(dev):
    rng = np.random.default_rng(1)
    mgr, ref = KVTierManager(t0_capacity=2, t1_capacity=3), RefTiers(2, 3)
    data = {b: torch.randn(5, 64, generator=torch.Generator().manual_seed(b)).to(torch.bfloat16) for b in range(8)}
    for b, t in data.items():
        mgr.put(b, t.to(dev) if b % 2 else t)
        ref.put(b)
    for _ in range(60):
        b = int(rng.integers(0, 8))
        if rng.random() < 0.7:
            g = mgr.prefetch_to_t0(b, dev)
            ref.prefetch(b)
            assert g.device.type == "cuda" and torch.equal(bits_t(g), bits_t(data[b]))
        else:
            mgr.evict_from_t0(b)
            ref.evict(b)
        assert list(mgr.t0) == list(ref.t0) and list(mgr.t1) == list(ref.t1)
        assert set(mgr.t2) >= set(ref.t2)
        for d in (mgr.t1, mgr.t2):
            for k, v in d.items():
                assert v.device.type == "cpu" and torch.equal(bits_t(v), bits_t(data[k]))
    with pytest.raises(KeyError):
        mgr.prefetch_to_t0(99, dev)
    assert build_ring_timeline(3) == {"forward": [0, 1, 2], "backward": [2, 1, 0]}


def test_kv_tier_manager_synchronize_before_another_stream(dev):
    """After synchronize(), a prefetched block can be read on a stream that was not ordered
    after the copy."""
    mgr = KVTierManager(t0_capacity=4, t1_capacity=4)
    host = torch.randn(1 << 20, generator=torch.Generator().manual_seed(3))
    mgr.put(7, host)
    g = mgr.prefetch_to_t0(7, dev)
    mgr.synchronize(dev)
    other = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(other):
        copy = g.clone()
    other.synchronize()
    assert torch.equal(copy.cpu(), host)
    mgr.synchronize()  # every device used so far


# ------------------------------------------------------------------ fp8_kv_quantization.py

def test_kv_tier_manager_pinned_source_outlives_its_copy(dev):
    """prefetch_to_t0 pops the pinned T1 tensor and drops it while its host-to-device copy
    is still queued behind the caller's kernels.  A pinned block of the same size taken
    and overwritten right after must not be the one the copy still reads."""
    n = 64 << 20
    mgr = KVTierManager(t0_capacity=4, t1_capacity=4)
    want = torch.randint(0, 255, (n,), dtype=torch.uint8, generator=torch.Generator().manual_seed(4))
    mgr.put(0, want.to(dev))
    mgr.prefetch_to_t0(0, dev)
    mgr.evict_from_t0(0)  # T1 now holds a pinned copy made by the tier mover
    assert 0 in mgr.t1 and mgr.t1[0].is_pinned()
    del mgr.t2[0]  # only T1 refers to the block's bytes now
    busy = torch.empty(1 << 28, dtype=torch.float32, device=dev)
    for _ in range(200):  # ~100 ms of work ahead of the copy on the caller's stream
        busy.mul_(1.0001)
    t0 = mgr.prefetch_to_t0(0, dev)  # pops T1; the side stream waits for the kernels above
    other = torch.empty(n, dtype=torch.uint8, pin_memory=True)
    other.fill_(0xA5)
    torch.cuda.synchronize(dev)
    assert torch.equal(t0.cpu(), want)
    mgr.synchronize()


def test_fp8_kv_quantizer_config1_shape(dev):
    """The README toy model's cache shape (12 layers, 12 heads, D = 64) with 256 tokens."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn((12, 2, 1, 12, 256, 64), generator=g).to(torch.bfloat16)
    q = FP8KVQuantizer()
    codes, scales = q.quantize(x)
    wc, ws = O.fp8_quant_heads(bits16(x).reshape(24, 1, 12, 256 * 64))
    np.testing.assert_array_equal(codes.cpu().numpy().reshape(wc.shape), wc)
    np.testing.assert_array_equal(scales.cpu().numpy().reshape(ws.shape).view(np.uint32), ws.view(np.uint32))
    y = q.dequantize(codes, scales)
    np.testing.assert_array_equal(bits16(y).reshape(wc.shape), O.fp8_dequant_heads(wc, ws))


def test_paged_cache_prefill_then_decode(dev):
    L, H, D, P = 2, 4, 128, 16
    cache = PagedFP8KVCache(L, H, D, num_pages=64, page_size=P)
    g = torch.Generator().manual_seed(5)
    lens = [37, 5, 64]
    x0 = torch.randn((L, sum(lens), 2, H, D), generator=g).to(torch.bfloat16)
    cache.append(x0, ["a", "b", "c"], lens)
    steps = [torch.randn((L, 3, 2, H, D), generator=g).to(torch.bfloat16) for _ in range(4)]
    for xs in steps:
        cache.append(xs, ["a", "b", "c"], [1, 1, 1])
    # oracle: one prefill with dynamic scales, then static-scale appends at the same pages
    seqs = ["a", "b", "c"]
    bt = np.full((3, max(len(cache.pages[s]) for s in seqs)), -1, np.int32)
    for i, s in enumerate(seqs):
        bt[i, :len(cache.pages[s])] = cache.pages[s]
    pool = np.zeros((L, 64, 2, H, P, D), np.uint8)
    cu = np.array([0, 37, 42, 106], np.int32)
    sc, err = O.kv_quant_append(bits16(x0), cu, None, bt, pool, P)
    assert err == 0
    over = 0
    for k, xs in enumerate(steps):
        start = np.array([lens[0] + k, lens[1] + k, lens[2] + k], np.int32)
        _, err = O.kv_quant_append(bits16(xs), np.array([0, 1, 2, 3], np.int32), start, bt, pool, P, scales=sc)
        assert err in (0, 8)
        over |= err
    np.testing.assert_array_equal(cache.pool.cpu().numpy(), pool)
    # N(0,1) decode tokens under the prefill's scales: one beyond 464 x its scale is a NaN
    # code, which the cache reports exactly when the oracle does
    if over:
        with pytest.raises(ValueError, match="static FP8 scale"):
            cache.check_errors()
    cache.check_errors()
    k, v = cache.gather(1, seqs)
    wk, wv, _ = O.kv_gather_dequant(pool[1], sc[1], bt, np.array([41, 9, 68], np.int32), 68)
    np.testing.assert_array_equal(bits16(k), wk)
    np.testing.assert_array_equal(bits16(v), wv)
    cache.free("b")
    assert "b" not in cache.pages


# ------------------------------------------------------------------ belayd_kv_cache_tiering.py

@pytest.mark.parametrize("L,R,S", [(1, 1, 5), (3, 8, 4), (2, 4, 7)])
def test_ring_access_sequence_matches_oracle(dev, L, R, S):
    seq = RingAttentionAccessSequence(L, R, S)
    tr = seq.trace(dev)
    assert tr.is_cuda and tr.dtype == torch.int32
    np.testing.assert_array_equal(tr.cpu().numpy(), O.ring_trace(L, R, S))
    assert len(seq) == tr.numel() and seq.n_pages == L * R * S


def test_tiering_manager_plan_matches_oracle(dev):
    m = BeladyKVCacheTieringManager(num_devices=8, context_length=8 * 64 * 32, num_layers=6, num_kv_heads=8,
                                    head_dim=128, page_tokens=64, hbm_budget_bytes=2.5 * 8 * 32 * 128 * 1024)
    assert m.pages_per_shard == 32 and m.capacity == int(2.5 * 8 * 32)
    stats = m.plan()
    trace = O.ring_trace(6, 8, 32)
    np.testing.assert_array_equal(RingAttentionAccessSequence(6, 8, 32).trace("cpu").numpy(), trace)
    ep, eg, st = O.belady_simulate(trace, m.n_pages, m.capacity)
    pos, page = m.eviction_schedule()
    np.testing.assert_array_equal(pos.numpy(), ep)
    np.testing.assert_array_equal(page.numpy(), eg)
    assert stats["misses"] == st["misses"]
    n = len(trace)
    d2h, h2d = m.transfers(n // 2, n)
    assert len(h2d) > 0 and len(d2h) >= 0
    r = m.replay_transfers(n // 2, n, check_bytes=True)
    assert r["h2d_pages"] == len(h2d) and r["d2h_pages"] == len(d2h)


def test_tier_replay_both_directions_round_trip(dev):
    """A budget below one layer's pages: inside a layer's forward window, victims used again
    later are written back (D2H) while pages evicted earlier come back (H2D), on the two
    copy streams at once.  Every page's bytes must be intact on both sides afterwards (a
    copy that ran before the one bringing its page in would leave filler)."""
    m = BeladyKVCacheTieringManager(num_devices=8, context_length=8 * 64 * 32, num_layers=3, num_kv_heads=8,
                                    head_dim=128, page_tokens=64, hbm_budget_bytes=100 * 128 * 1024)
    assert m.capacity == 100 and m.pages_per_shard == 32  # 256 pages per layer
    m.plan()
    per_layer = len(m.sequence) // 2 // 3
    d2h, h2d = m.transfers(per_layer, 2 * per_layer)
    assert len(d2h) > 0 and len(h2d) > 0
    assert len(np.intersect1d(d2h, h2d)) > 0  # pages written back and fetched again in the window
    for max_batch in (16, 1024):  # short chunks (many cross-stream waits) and the default
        r = m.replay_transfers(per_layer, 2 * per_layer, check_bytes=True, max_batch=max_batch)
        assert r["d2h_pages"] == len(d2h) and r["h2d_pages"] == len(h2d) and r["chunks"] > 1


def test_quantized_ring_attention_over_paged_cache(dev):
    """README.md:344's import line, then ring attention and decode over a PagedFP8KVCache
    (appended twice: a prefill and a continuation) against the oracle: ring attention in the
    default precision within 2 bf16 ulps + 2^-10 max|V| and in the exact one within one ulp
    + 2^-17 max|V|, decode within one ulp + 2^-17 max|V|."""
    from test_gpu_attention import assert_within_bound, assert_within_one_ulp
    from zenyx_amd.train.fp8_kv_quantization import FP8KVQuantizer as _Q, QuantizedRingAttention as _R  # noqa: F401

    L, H, D, P, Hq = 2, 4, 128, 16, 16
    cache = PagedFP8KVCache(L, H, D, num_pages=64, page_size=P, device=dev)
    g = torch.Generator().manual_seed(21)
    lens1, lens2 = [70, 33], [20, 31]
    cache.append(torch.randn((L, sum(lens1), 2, H, D), generator=g).to(torch.bfloat16), ["a", "b"], lens1)
    # the continuation reuses the first append's scales: keep it inside their range (no NaN codes)
    cache.append((0.5 * torch.randn((L, sum(lens2), 2, H, D), generator=g)).to(torch.bfloat16), ["a", "b"], lens2)
    att = QuantizedRingAttention(cache, ring_degree=3)
    q = torch.randn((sum(lens2), Hq, D), generator=g).to(torch.bfloat16)
    layer = 1
    out = att(q, layer, ["a", "b"], lens2)
    torch.cuda.synchronize()
    pool = cache.pool[layer].cpu().numpy()
    sc = cache.scales[layer].cpu().numpy()
    bt = cache._tables(["a", "b"]).cpu().numpy()
    tot = np.array([lens1[0] + lens2[0], lens1[1] + lens2[1]], np.int32)
    cu = np.array([0, lens2[0], sum(lens2)], np.int32)
    sm = float(np.float32(1.0 / np.sqrt(D)))
    want, _, err = O.paged_attention_prefill(bits16(q), cu, tot - np.array(lens2, np.int32), pool, sc, bt,
                                             np.zeros(2, np.int32), tot, True, sm)
    assert err == 0
    dec = np.abs(O.e4m3_decode(np.arange(256, dtype=np.uint8)).astype(np.float64))
    assert not np.isnan(dec[pool]).any()
    vmax = float(dec[pool[:, 1]].max() * sc[1].max())
    assert_within_bound(bits16(out), want, np.full(want.shape, vmax), 2.0 ** -10, ulps=2)
    out_x = QuantizedRingAttention(cache, ring_degree=3, precision="exact")(q, layer, ["a", "b"], lens2)
    assert_within_one_ulp(bits16(out_x), want, np.full(want.shape, vmax))
    with pytest.raises(ValueError, match="precision"):
        QuantizedRingAttention(cache, precision="fp8")
    qd = torch.randn((2, Hq, D), generator=g).to(torch.bfloat16)
    od = att.decode(qd, layer, ["a", "b"])
    torch.cuda.synchronize()
    wd, derr = O.paged_attention_decode(bits16(qd), pool, sc, bt, tot, sm)
    assert derr == 0
    assert_within_one_ulp(bits16(od), wd, np.full(wd.shape, vmax))
    with pytest.raises(ValueError):
        att(q, layer, ["a", "b"], [lens2[0], lens2[1] + 1])
