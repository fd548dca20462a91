"""Static-scale FP8 overflow on the GPU: a decode token larger than 464 x the prefill's
scale.  The kernels flag it (ZX_KERR_OVERFLOW) and store the NaN code, or +-448 when
saturating, bit-exact with the oracle (itself pinned to torch's cast and clamp in
tests/test_oracle.py); PagedFP8KVCache raises on it, or saturates and keeps attention
finite."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from zenyx_amd import _native as N
from zenyx_amd import kv
from zenyx_amd.train.fp8_kv_quantization import PagedFP8KVCache, QuantizedRingAttention

pytestmark = pytest.mark.gpu


def bits16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _tables(lens, P, extra, seed):
    rng = np.random.default_rng(seed)
    nb = [(n + P - 1) // P for n in lens]
    n_pages = sum(nb) + extra
    perm = rng.permutation(n_pages).astype(np.int32)
    bt = np.full((len(lens), max(nb)), -1, np.int32)
    k = 0
    for b, m in enumerate(nb):
        bt[b, :m] = perm[k:k + m]
        k += m
    return bt, n_pages


@pytest.mark.parametrize("saturate", [False, True])
@pytest.mark.parametrize("D", [64, 128])
def test_static_append_overflow_matches_oracle(dev, saturate, D):
    L, H, P = 3, 4, 16
    lens = [40, 1, 17, 100]
    bt, n_pages = _tables(lens, P, 3, 7)
    g = torch.Generator().manual_seed(31)
    x = torch.randn((L, sum(lens), 2, H, D), generator=g) * 6
    specials = torch.tensor([float("inf"), -float("inf"), float("nan"), -2.0e4])
    x[1, 3, 0, 2, :4] = specials
    x[0, 5, 1, 1, :4] = specials
    x = x.to(torch.bfloat16)
    x.view(torch.int16)[0, 6, 1, 1, 7] = -63  # 0xFFC1: a NaN with the sign bit set
    # finite scales of both signs (some small enough to overflow), one +inf slab; the two
    # slabs holding +-inf and NaN inputs get one sign each
    sc = (torch.rand((L, 2, H), generator=g) * 0.2 + 0.004) * torch.where(torch.rand((L, 2, H), generator=g) < 0.3,
                                                                         -1.0, 1.0)
    sc[1, 0, 2] = sc[1, 0, 2].abs()
    sc[0, 1, 1] = -sc[0, 1, 1].abs()
    sc[2, 1, 3] = float("inf")
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    want = np.zeros((L, n_pages, 2, H, P, D), np.uint8)
    _, werr = O.kv_quant_append(bits16(x), cu, None, bt, want, P, scales=sc.numpy(), saturate=saturate)
    assert werr == N.ZX_KERR_OVERFLOW
    pool = torch.zeros(want.shape, dtype=torch.uint8, device=dev)
    scd = sc.to(dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    kv.kv_quant_append(x.to(dev), torch.from_numpy(cu).to(dev), torch.from_numpy(bt).to(dev), pool, scales=scd,
                       static_scales=True, saturate=saturate, err=err)
    assert int(err.item()) == werr
    got = pool.cpu().numpy()
    bad = np.argwhere(got != want)
    if bad.size:  # name the elements: input value, slab scale, both codes
        xf = x.float().numpy()
        seq = np.repeat(np.arange(len(lens)), lens)
        pos = np.concatenate([np.arange(n) for n in lens])
        rows = []
        for l, page, kvi, h, slot, d in bad[:8]:
            t = np.nonzero((bt[seq, pos // P] == page) & (pos % P == slot))[0][0]
            rows.append(f"layer {l} token {t} kv {kvi} head {h} d {d}: x={xf[l, t, kvi, h, d]!r} "
                        f"scale={sc[l, kvi, h].item()!r} gpu=0x{got[l, page, kvi, h, slot, d]:02x} "
                        f"oracle=0x{want[l, page, kvi, h, slot, d]:02x}")
        raise AssertionError(f"{len(bad)} codes differ:\n" + "\n".join(rows))
    assert torch.equal(scd.cpu(), sc)
    with pytest.raises(ValueError, match="static FP8 scale"):
        kv.kv_quant_append(x.to(dev), torch.from_numpy(cu).to(dev), torch.from_numpy(bt).to(dev), pool, scales=scd,
                           static_scales=True, saturate=saturate, check=True)


@pytest.mark.parametrize("saturate", [False, True])
def test_static_append_every_input(dev, saturate):
    """Every bf16 bit pattern (zeros of both signs, subnormals, +-inf, NaNs of both signs)
    in each of four slabs, appended under static scales 0.75, -0.75, 2.5e-3 (most finite
    inputs overflow) and -inf: codes and the error word equal the oracle's."""
    H, D, P = 2, 128, 16
    lens = [200, 312]
    bt, n_pages = _tables(lens, P, 2, 11)
    allbf = np.arange(65536, dtype=np.uint16).reshape(512, D)
    x = np.empty((1, 512, 2, H, D), np.uint16)
    for kvi in range(2):
        for h in range(H):
            x[0, :, kvi, h] = allbf
    sc = torch.tensor([[[0.75, -0.75], [2.5e-3, -float("inf")]]], dtype=torch.float32)
    cu = np.array([0, 200, 512], np.int32)
    want = np.zeros((1, n_pages, 2, H, P, D), np.uint8)
    _, werr = O.kv_quant_append(x, cu, None, bt, want, P, scales=sc.numpy(), saturate=saturate)
    pool = torch.zeros(want.shape, dtype=torch.uint8, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    kv.kv_quant_append(xt.to(dev), torch.from_numpy(cu).to(dev), torch.from_numpy(bt).to(dev), pool,
                       scales=sc.to(dev), static_scales=True, saturate=saturate, err=err)
    assert int(err.item()) == werr
    got = pool.cpu().numpy()
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} codes differ, e.g. (layer, page, kv, head, slot, d) {bad[:4].tolist()}: " \
                          f"gpu {[hex(got[tuple(i)]) for i in bad[:4]]} oracle {[hex(want[tuple(i)]) for i in bad[:4]]}"


def test_static_append_without_overflow_sets_no_bit(dev):
    L, H, D, P = 2, 8, 128, 16
    lens = [33, 64]
    bt, n_pages = _tables(lens, P, 0, 8)
    x = torch.randn((L, sum(lens), 2, H, D), generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    sc = torch.full((L, 2, H), 1.0, dtype=torch.float32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pool = torch.zeros((L, n_pages, 2, H, P, D), dtype=torch.uint8, device=dev)
    kv.kv_quant_append(x.to(dev), torch.from_numpy(cu).to(dev), torch.from_numpy(bt).to(dev), pool,
                       scales=sc.to(dev), static_scales=True, check=True)


def _prefill_then_outlier(dev, overflow):
    L, H, D, P = 2, 4, 128, 16
    cache = PagedFP8KVCache(L, H, D, num_pages=32, page_size=P, device=dev, overflow=overflow)
    g = torch.Generator().manual_seed(41)
    lens = [50, 20]
    x0 = torch.randn((L, sum(lens), 2, H, D), generator=g).to(torch.bfloat16)
    cache.append(x0, ["a", "b"], lens, check=True)
    x1 = torch.randn((L, 2, 2, H, D), generator=g)
    x1[1, 0, 1, 2, 5] = 3000.0  # one outlier decode token: V of layer 1, head 2, sequence "a"
    x1 = x1.to(torch.bfloat16)
    return cache, x0, x1, lens


def test_paged_cache_outlier_decode_token_raises(dev):
    cache, x0, x1, lens = _prefill_then_outlier(dev, "raise")
    cache.append(x1, ["a", "b"], [1, 1])  # not checked here: the NaN code is written, the bit recorded
    att = QuantizedRingAttention(cache, ring_degree=2)
    q = torch.randn((2, 16, 128), generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    with pytest.raises(ValueError, match="static FP8 scale"):
        att.decode(q, 1, ["a", "b"])
    cache.check_errors()  # the word was cleared by the raise
    # the codes equal the oracle's: a NaN code at the outlier, nothing else touched
    seqs = ["a", "b"]
    bt = cache._tables(seqs).cpu().numpy()
    pool = np.zeros(tuple(cache.pool.shape), np.uint8)
    cu = np.array([0, lens[0], sum(lens)], np.int32)
    sc, err = O.kv_quant_append(bits16(x0), cu, None, bt, pool, cache.P)
    assert err == 0
    _, err = O.kv_quant_append(bits16(x1), np.array([0, 1, 2], np.int32), np.array(lens, np.int32), bt, pool,
                               cache.P, scales=sc)
    assert err == N.ZX_KERR_OVERFLOW
    np.testing.assert_array_equal(cache.pool.cpu().numpy(), pool)
    page = bt[0, lens[0] // cache.P]
    assert pool[1, page, 1, 2, lens[0] % cache.P, 5] == 0x7F
    with pytest.raises(ValueError, match="static FP8 scale"):
        cache.append(x1, ["a", "b"], [1, 1], check=True)


def test_paged_cache_outlier_decode_token_saturates(dev):
    cache, x0, x1, lens = _prefill_then_outlier(dev, "saturate")
    cache.append(x1, ["a", "b"], [1, 1])
    seqs = ["a", "b"]
    bt = cache._tables(seqs).cpu().numpy()
    pool = np.zeros(tuple(cache.pool.shape), np.uint8)
    cu = np.array([0, lens[0], sum(lens)], np.int32)
    sc, _ = O.kv_quant_append(bits16(x0), cu, None, bt, pool, cache.P)
    _, err = O.kv_quant_append(bits16(x1), np.array([0, 1, 2], np.int32), np.array(lens, np.int32), bt, pool,
                               cache.P, scales=sc, saturate=True)
    assert err == N.ZX_KERR_OVERFLOW
    np.testing.assert_array_equal(cache.pool.cpu().numpy(), pool)
    page = bt[0, lens[0] // cache.P]
    assert pool[1, page, 1, 2, lens[0] % cache.P, 5] == 0x7E
    att = QuantizedRingAttention(cache, ring_degree=2)
    q = torch.randn((2, 16, 128), generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    out = att.decode(q, 1, seqs)
    assert torch.isfinite(out.float()).all()
    assert cache.saturated_appends == 1
    k, v = cache.gather(1, seqs)
    assert torch.isfinite(v.float()).all()


def test_paged_cache_refuses_rescale_and_rolls_back(dev):
    cache, x0, x1, lens = _prefill_then_outlier(dev, "raise")
    with pytest.raises(ValueError, match="re-scale"):
        cache.append(x1, ["a", "b"], [1, 1], dynamic_scales=True)
    free_before, pages_before = list(cache._free), {k: list(v) for k, v in cache.pages.items()}
    bad = torch.zeros((2, 40, 2, 4, 64), dtype=torch.bfloat16)  # wrong head_dim: the kernel call refuses it
    with pytest.raises(ValueError):
        cache.append(bad, ["a", "c"], [20, 20])
    assert cache._free == free_before and cache.pages == pages_before
    assert cache.lengths == {"a": lens[0], "b": lens[1]}
