"""GPU decode attention from FP8 pages (zx_paged_attention_decode) against the C oracle.

The oracle evaluates softmax(sm_scale q K^T) V in double on the decoded codes times the
per-head scales and rounds once to bf16 (it is pinned bit-exact against torch float64 in
tests/test_oracle.py).  The kernel computes in fp32 with a split online softmax and
exp2, so the tolerance is one bf16 ulp of the exact value plus the fp32 accumulation
error of a weighted mean of the V column (which matters only where the output cancels
to far below the V values):
    |got - want| <= ulp(|want|) + 2^-17 * max_t |V_t[d]|,   ulp(x) = 2^(floor(log2 x) - 7)
(values below 2^-100 take ulp 2^-107; 2^-17 bounds the fp32 error of summing up to 4096
weighted terms in the kernel's order), NaN compared as a class.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from zenyx_amd import kv

pytestmark = pytest.mark.gpu


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def v_colmax(pool, scales, bt, lens, Hq):
    """max_t |V_t[d]| over each sequence's positions with a valid page: [B, Hq, D]."""
    n_pages, _, Hkv, P, D = pool.shape
    dec = np.abs(O.e4m3_decode(np.arange(256, dtype=np.uint8)).astype(np.float64))
    out = np.zeros((len(lens), Hq, D))
    for b, n in enumerate(lens):
        t = np.arange(n)
        pages = bt[b, t // P]
        ok = (pages >= 0) & (pages < n_pages)
        t, pages = t[ok], pages[ok]
        for hq in range(Hq):
            h = hq // (Hq // Hkv)
            if len(t):
                out[b, hq] = np.nanmax(dec[pool[pages, 1, h, t % P, :]], axis=0) * abs(float(scales[1, h]))
    return out


def assert_within_bound(got_bits: np.ndarray, want_bits: np.ndarray, vmax: np.ndarray, e: float, ulps: int = 1):
    """|got - want| <= ``ulps`` bf16 ulps of want + e * max|V| elementwise (NaN as a class)."""
    g, w = bf16_to_f32(got_bits), bf16_to_f32(want_bits)
    g_nan, w_nan = np.isnan(g), np.isnan(w)
    np.testing.assert_array_equal(g_nan, w_nan)
    g, w, vm = g[~g_nan].astype(np.float64), w[~w_nan].astype(np.float64), vmax[~w_nan]
    mag = np.maximum(np.abs(w), 2.0 ** -100)
    tol = ulps * np.exp2(np.floor(np.log2(mag)) - 7) + e * vm
    bad = np.abs(g - w) > tol
    assert not bad.any(), f"{bad.sum()} of {bad.size} beyond tolerance, e.g. got {g[bad][:4]} want {w[bad][:4]}"
    return float(np.max(np.abs(g - w) / np.maximum(vm, 1e-30))) if g.size else 0.0


def assert_within_one_ulp(got_bits: np.ndarray, want_bits: np.ndarray, vmax: np.ndarray):
    """The exact kernels' bound: one bf16 ulp + 2^-17 max|V|."""
    return assert_within_bound(got_bits, want_bits, vmax, 2.0 ** -17)


def make_case(Hq, Hkv, D, P, lens, seed, n_pages=None, nan_codes=False):
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    B = len(lens)
    max_blocks = max(1, (int(lens.max()) + P - 1) // P)
    n_pages = n_pages or B * max_blocks + 5
    pool = rng.integers(0, 256, (n_pages, 2, Hkv, P, D), dtype=np.uint8)
    if not nan_codes:
        pool[(pool & 0x7F) == 0x7F] = 0x3A
    perm = rng.permutation(n_pages)
    bt = perm[:B * max_blocks].reshape(B, max_blocks).astype(np.int32)
    scales = rng.uniform(1e-3, 0.05, (2, Hkv)).astype(np.float32)
    q = torch.from_numpy(rng.standard_normal((B, Hq, D)).astype(np.float32)).to(torch.bfloat16)
    return q, pool, scales, bt, lens


@pytest.mark.parametrize("Hq,Hkv,D,P,lens", [
    (32, 8, 128, 16, [0, 1, 15, 16, 17, 1023, 1024, 1025, 3000]),  # 4 query heads per block
    (8, 8, 64, 16, [5, 64, 2100]),                                  # no grouping, D = 64
    (12, 4, 256, 32, [700, 31, 2049]),                              # groups of 3 (one head per block)
    (16, 8, 128, 5, [1, 333, 1500]),                                # page size 5, pairs of heads
    (8, 8, 128, 32, [40, 1, 2222]),                                 # matrix-core variant, one head
    (16, 8, 128, 16, [17, 4000]),                                   # matrix-core variant, pairs
])
def test_paged_attention_decode_matches_oracle(dev, Hq, Hkv, D, P, lens):
    q, pool, scales, bt, lens = make_case(Hq, Hkv, D, P, lens, seed=Hq + D + P)
    sm = 1.0 / np.sqrt(D)
    want, werr = O.paged_attention_decode(bits16(q), pool, scales, bt, lens, sm)
    assert werr == 0
    got = kv.paged_attention_decode(q.to(dev), torch.from_numpy(pool).to(dev), torch.from_numpy(scales).to(dev),
                                    torch.from_numpy(bt).to(dev), torch.from_numpy(lens).to(dev), check=True)
    assert_within_one_ulp(bits16(got), want, v_colmax(pool, scales, bt, lens, Hq))
    assert not bits16(got)[lens == 0].any()  # empty sequences give zeros


def test_paged_attention_decode_large_scores_and_custom_scale(dev):
    """Large logits (scale 8x sm_scale) stress the running-max rescaling across splits."""
    q, pool, scales, bt, lens = make_case(32, 8, 128, 16, [4096, 2000, 9], seed=5)
    scales[0] *= 20.0
    sm = 8.0 / np.sqrt(128)
    want, _ = O.paged_attention_decode(bits16(q), pool, scales, bt, lens, sm)
    got = kv.paged_attention_decode(q.to(dev), torch.from_numpy(pool).to(dev), torch.from_numpy(scales).to(dev),
                                    torch.from_numpy(bt).to(dev), torch.from_numpy(lens).to(dev), sm_scale=sm)
    assert_within_one_ulp(bits16(got), want, v_colmax(pool, scales, bt, lens, 32))


@pytest.mark.parametrize("Hq,Hkv,D", [(32, 8, 128), (8, 8, 64)])
def test_paged_attention_decode_negative_scales(dev, Hq, Hkv, D):
    """Scales of either sign (a static scale may be negative): K heads 0, 2, .. and V heads
    1, 3, .. negated, so scores and values change sign per head (matrix-core kernel for
    D = 128, VALU kernel for D = 64)."""
    q, pool, scales, bt, lens = make_case(Hq, Hkv, D, 16, [1, 300, 2500], seed=13)
    scales[0, 0::2] *= -1.0
    scales[1, 1::2] *= -1.0
    sm = 1.0 / np.sqrt(D)
    want, werr = O.paged_attention_decode(bits16(q), pool, scales, bt, lens, sm)
    assert werr == 0
    got = kv.paged_attention_decode(q.to(dev), torch.from_numpy(pool).to(dev), torch.from_numpy(scales).to(dev),
                                    torch.from_numpy(bt).to(dev), torch.from_numpy(lens).to(dev), check=True)
    assert_within_one_ulp(bits16(got), want, v_colmax(pool, scales, bt, lens, Hq))


@pytest.mark.parametrize("D", [64, 128])
def test_paged_attention_decode_nan_codes_and_bad_pages(dev, D):
    """NaN codes make the affected heads NaN; an out-of-range page id is skipped and flagged
    (D = 64: VALU kernel, D = 128: matrix-core kernel)."""
    q, pool, scales, bt, lens = make_case(8, 2, D, 16, [100, 200, 50], seed=6)
    pool[bt[1, 3], 0, 1, 4, 7] = 0x7F  # a NaN code in sequence 1, kv head 1
    bt_bad = bt.copy()
    bt_bad[2, 1] = pool.shape[0] + 10
    want, werr = O.paged_attention_decode(bits16(q), pool, scales, bt_bad, lens, 0.125)
    assert werr == 1
    args = (q.to(dev), torch.from_numpy(pool).to(dev), torch.from_numpy(scales).to(dev),
            torch.from_numpy(bt_bad).to(dev), torch.from_numpy(lens).to(dev))
    with pytest.raises(ValueError, match="block table"):
        kv.paged_attention_decode(*args, sm_scale=0.125, check=True)
    got = kv.paged_attention_decode(*args, sm_scale=0.125)
    assert_within_one_ulp(bits16(got), want, v_colmax(pool, scales, bt_bad, lens, 8))
    assert np.isnan(bf16_to_f32(bits16(got)[1, 4:8])).all()
