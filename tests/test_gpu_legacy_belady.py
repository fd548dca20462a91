"""GPU parity of the legacy int8 path (precision.py) and of Belady victim selection /
next-use tables against the CPU oracle."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from zenyx_amd import _native as N
from zenyx_amd import kv

pytestmark = pytest.mark.gpu


def raw(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("mag", [1.0, 1e-3, 3e4, 0.0])
def test_int8_legacy_quant_dequant(dev, dt, mag):
    g = torch.Generator().manual_seed(int(mag * 7) + len(dt))
    x = (torch.randn(4099, generator=g) * mag).to(DTYPES[dt])
    q, s = kv.int8_legacy_quant(x.to(dev))
    wq, ws = O.int8_legacy_quant(raw(x), dt)
    np.testing.assert_array_equal(q.cpu().numpy(), wq)
    assert s.dtype == x.dtype and s.dim() == 0
    assert np.float32(s.float().item()).tobytes() == np.float32(ws).tobytes()
    y = kv.int8_legacy_dequant(q, s)
    assert y.dtype == torch.bfloat16
    got, want = raw(y), O.int8_legacy_dequant(wq, ws)
    # NaN (an f16 input that overflowed to inf gives an inf scale) matches NaN as a class
    g_nan, w_nan = (got & 0x7FFF) > 0x7F80, (want & 0x7FFF) > 0x7F80
    np.testing.assert_array_equal(g_nan, w_nan)
    np.testing.assert_array_equal(got[~g_nan], want[~w_nan])


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("shape", [(2, 1037), (4, 256)])  # unaligned slabs (element path), aligned (16-byte path)
def test_int8_legacy_slabs_match_per_tensor_and_oracle(dev, dt, shape):
    """Per-slab batch (one launch) == the per-tensor functions on every slab == the oracle,
    with slabs of different magnitudes, an all-zero slab (scale from the 1e-8 floor) and a
    slab with one outlier; slab length not a multiple of the block size."""
    g = torch.Generator().manual_seed(3 + len(dt))
    mags = [1.0, 1e-3, 0.0, 3e2, 1.0, 7.5]
    x = torch.stack([torch.randn(*shape, generator=g) * m for m in mags])
    x[4, 1, 5] = 40.0
    x = x.to(DTYPES[dt])
    q, sc = kv.int8_legacy_quant_slabs(x.to(dev))
    y = kv.int8_legacy_dequant_slabs(q, sc)
    assert q.shape == x.shape and sc.shape == (len(mags),) and sc.dtype == x.dtype and y.dtype == torch.bfloat16
    for i in range(len(mags)):
        q1, s1 = kv.int8_legacy_quant(x[i].to(dev))
        assert torch.equal(q[i].cpu(), q1.cpu())
        assert raw(sc[i:i + 1]).tobytes() == raw(s1.reshape(1)).tobytes()
        wq, ws = O.int8_legacy_quant(raw(x[i]), dt)
        np.testing.assert_array_equal(q[i].cpu().numpy(), wq)
        np.testing.assert_array_equal(raw(y[i]), O.int8_legacy_dequant(wq, ws))


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_int8_legacy_every_input_below_amax(dev, dt):
    """The vector path's fast encoder (no NaN or range guard, integer rounding by adding
    1.5 * 2^23) on complete input sets: slab i holds every bit pattern of the format whose
    magnitude is at most the pattern a_i (both signs, so a_i is the slab's amax), zero
    padded.  The a_i cover scales from the 1e-8 floor to the format's largest value, the
    quotients 127 / 127.5 / 128 at the clamp, and (f16) subnormal and zero scales, whose
    slabs take the division path.  Codes, scales and dequantised values equal the oracle's."""
    tops = {"bf16": [0x0001, 0x2F00, 0x3280, 0x3A83, 0x3C00, 0x3F80, 0x42FE, 0x42FF, 0x4300, 0x4480, 0x4700,
                     0x5000, 0x6A00, 0x7F7F],
            "f16": [0x0001, 0x0010, 0x0100, 0x0300, 0x0400, 0x0C00, 0x1400, 0x2000, 0x3C00, 0x57F0, 0x57F8,
                    0x5800, 0x7000, 0x7BFF]}[dt]
    L = 1 << 17
    rows = np.zeros((len(tops), L), np.uint16)
    for i, a in enumerate(tops):
        mags = np.arange(a + 1, dtype=np.uint16)
        v = np.concatenate([mags, mags | np.uint16(0x8000)])
        rows[i, :v.size] = v
    x = torch.from_numpy(rows.view(np.int16)).view(DTYPES[dt])
    q, sc = kv.int8_legacy_quant_slabs(x.to(dev))
    y = kv.int8_legacy_dequant_slabs(q, sc)
    for i in range(len(tops)):
        wq, ws = O.int8_legacy_quant(rows[i], dt)
        np.testing.assert_array_equal(q[i].cpu().numpy(), wq, err_msg=f"amax pattern {tops[i]:#06x}")
        assert np.float32(sc[i].float().item()).tobytes() == np.float32(ws).tobytes()
        np.testing.assert_array_equal(raw(y[i]), O.int8_legacy_dequant(wq, ws))


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_int8_legacy_unaligned_view(dev, dt):
    """A view starting one element in (not 16-byte aligned) takes the element-by-element
    path; results equal the oracle's."""
    g = torch.Generator().manual_seed(9)
    base = (torch.randn(4097, generator=g) * 3).to(DTYPES[dt]).to(dev)
    x = base[1:]  # the Python wrappers require 16-byte alignment: call the C ABI directly
    qb = torch.empty(4097, dtype=torch.int8, device=dev)
    q = qb[1:]
    s = torch.empty((), dtype=x.dtype, device=dev)
    ws = torch.empty(256, dtype=torch.uint8, device=dev)
    lib = N.load()
    N.check(lib.zx_int8_legacy_quant(N.ptr(x), kv._DT[x.dtype], x.numel(), N.ptr(q), N.ptr(s), N.ptr(ws), 256,
                                     N.stream_ptr(dev)), "int8_legacy_quant")
    wq, wsc = O.int8_legacy_quant(raw(x), dt)
    np.testing.assert_array_equal(q.cpu().numpy(), wq)
    yb = torch.empty(4097, dtype=torch.bfloat16, device=dev)
    y = yb[1:]
    N.check(lib.zx_int8_legacy_dequant(N.ptr(q), N.ptr(s), kv._DT[s.dtype], q.numel(), N.ptr(y), N.stream_ptr(dev)),
            "int8_legacy_dequant")
    np.testing.assert_array_equal(raw(y), O.int8_legacy_dequant(wq, wsc))


def test_int8_legacy_empty_raises(dev):
    with pytest.raises(RuntimeError):
        kv.int8_legacy_quant(torch.empty(0, device=dev))


def test_belady_argmax_matches_oracle(dev):
    rng = np.random.default_rng(5)
    for n in (1, 7, 1000, 100_003):
        keys = rng.integers(-3, 50, n).astype(np.int64)  # many ties and many <= -1
        keys[rng.integers(0, n, max(1, n // 10))] = 10**18
        res = (rng.random(n) < 0.6).astype(np.uint8)
        out = kv.belady_argmax(torch.from_numpy(keys).to(dev), torch.from_numpy(res).to(dev)).cpu().tolist()
        assert tuple(out) == O.belady_argmax(keys, res)
        rank = rng.permutation(n).astype(np.int64) // 3  # ranks with ties
        out = kv.belady_argmax(torch.from_numpy(keys).to(dev), None, torch.from_numpy(rank).to(dev)).cpu().tolist()
        assert tuple(out) == O.belady_argmax(keys, None, rank)
    # nothing qualifies: every resident key <= -1 (belady.py:45-51 returns None)
    keys = np.full(10, -1, np.int64)
    out = kv.belady_argmax(torch.from_numpy(keys).to(dev), torch.ones(10, dtype=torch.uint8, device=dev))
    assert out.cpu().tolist() == [-1, -1]


def test_next_use_matches_oracle(dev):
    """The hand-written radix sort behind next_use: 1 to 4 passes of 7-bit digits, lengths
    that end mid-tile, one page accessed everywhere (one digit holds every element), and
    skewed traces."""
    rng = np.random.default_rng(9)
    cases = [(1, 1), (50, 3), (4097, 2), (100_000, 777), (300_000, 1 << 17), (12_345, 1 << 14),
             (70_001, 1 << 21), (5_000, 1 << 25)]
    for n, n_pages in cases:
        trace = rng.integers(0, n_pages, n).astype(np.int32)
        nu, pu = kv.next_use(torch.from_numpy(trace).to(dev), n_pages, check=True)
        wnu, wpu = O.next_use(trace, n_pages)
        np.testing.assert_array_equal(nu.cpu().numpy(), wnu)
        np.testing.assert_array_equal(pu.cpu().numpy(), wpu)
    for trace, n_pages in ((np.full(50_000, 7, np.int32), 9),
                           ((rng.zipf(1.3, 200_000) % 5000).astype(np.int32), 5000)):
        nu, pu = kv.next_use(torch.from_numpy(trace).to(dev), n_pages, check=True)
        wnu, wpu = O.next_use(trace, n_pages)
        np.testing.assert_array_equal(nu.cpu().numpy(), wnu)
        np.testing.assert_array_equal(pu.cpu().numpy(), wpu)
    bad = torch.tensor([0, 3, -1, 2, 3], dtype=torch.int32, device=dev)
    with pytest.raises(ValueError, match="block table entry outside"):
        kv.next_use(bad, 4, check=True)
    ring = O.ring_trace(2, 8, 16)
    nu, pu = kv.next_use(torch.from_numpy(ring).to(dev), 2 * 8 * 16)
    wnu, wpu = O.next_use(ring, 2 * 8 * 16)
    np.testing.assert_array_equal(nu.cpu().numpy(), wnu)
    np.testing.assert_array_equal(pu.cpu().numpy(), wpu)
