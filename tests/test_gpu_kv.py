"""GPU parity of the FP8 KV kernels (libzenyx_kv.so) against the CPU oracle.

Codes, scales and gathered bytes must be bit-exact; dequantized bf16 must be bit-exact
as well (stronger than a 1-ulp tolerance), with NaN compared as
a class because torch itself writes different NaN payloads on different paths.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from zenyx_amd import kv

pytestmark = pytest.mark.gpu


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def assert_bf16_equal(got: np.ndarray, want: np.ndarray):
    g_nan = (got & 0x7FFF) > 0x7F80
    w_nan = (want & 0x7FFF) > 0x7F80
    np.testing.assert_array_equal(g_nan, w_nan)
    np.testing.assert_array_equal(got[~g_nan], want[~w_nan])


def e4m3_probe_values() -> np.ndarray:
    """All bf16 values, every e4m3 rounding midpoint +-0..3 ulp, random fp32."""
    allbf = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    grid = O.e4m3_decode(np.arange(256, dtype=np.uint8))
    grid = np.unique(np.abs(grid[np.isfinite(grid)]).astype(np.float64))
    grid = np.concatenate([grid, [480.0]])
    mids = ((grid[:-1] + grid[1:]) / 2).astype(np.float32)
    near = [mids]
    up, dn = mids, mids
    for _ in range(3):
        up = np.nextafter(up, np.float32(np.inf))
        dn = np.nextafter(dn, np.float32(0))
        near += [up, dn]
    rng = np.random.default_rng(7)
    rnd = np.concatenate([
        rng.uniform(-500, 500, 1 << 20).astype(np.float32),
        (rng.choice([-1, 1], 1 << 20) * np.exp2(rng.uniform(-14, 9, 1 << 20))).astype(np.float32),
    ])
    near = np.concatenate(near)
    return np.concatenate([allbf, near, -near, rnd]).astype(np.float32)


def test_e4m3_device_encode_matches_oracle(dev):
    v = e4m3_probe_values()
    got = kv.fp8_encode_f32(torch.from_numpy(v).to(dev)).cpu().numpy()
    want = O.e4m3_encode(v)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} mismatches, e.g. {v[bad[:5]]} -> {got[bad[:5]]} vs {want[bad[:5]]}"


def make_kv_cache(L, B, H, T, D, seed, outlier_heads=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((L, 2, B, H, T, D), generator=g, dtype=torch.float32)
    if outlier_heads:
        for l in range(L):
            hs = torch.randperm(H, generator=g)[:outlier_heads]
            x[l, :, :, hs] *= 50.0
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("mode", ["two", "single"])
def test_fp8_heads_every_input_below_amax(dev, mode):
    """Complete input sets through both quantiser paths: slab (o, h) holds every bf16 bit
    pattern whose magnitude is at most the pattern a (both signs, so a is the slab's
    amax), zero padded; a runs from below the 1e-8 scale floor to the largest finite bf16.
    Codes, scales and dequantised values equal the oracle's."""
    tops = [0x0001, 0x2F00, 0x3280, 0x3A83, 0x3C00, 0x3F80, 0x43E0, 0x43E8, 0x4400, 0x4700, 0x5000, 0x6A00,
            0x7A00, 0x7F7F, 0x3E4C, 0x40A1]
    run = 1 << 17
    rows = np.zeros((len(tops), run), np.uint16)
    for i, a in enumerate(tops):
        mags = np.arange(a + 1, dtype=np.uint16)
        v = np.concatenate([mags, mags | np.uint16(0x8000)])
        rows[i, :v.size] = v
    x = torch.from_numpy(rows.view(np.int16)).view(torch.bfloat16).reshape(2, 1, len(tops) // 2, run)
    codes, scales = kv.fp8_quant_heads(x.to(dev), two_pass=mode == "two", single_pass=mode == "single", check=True)
    wc, ws = O.fp8_quant_heads(bits16(x))
    np.testing.assert_array_equal(scales.cpu().numpy().view(np.uint32), ws.view(np.uint32))
    np.testing.assert_array_equal(codes.cpu().numpy(), wc)
    y = kv.fp8_dequant_heads(codes, scales)
    assert_bf16_equal(bits16(y), O.fp8_dequant_heads(wc, ws))


@pytest.mark.parametrize("shape,seed", [((2, 1, 12, 256, 64), 0), ((3, 2, 4, 48, 128), 1),
                                        ((1, 3, 2, 16, 256), 2)])
def test_fp8_quant_dequant_heads_bit_exact(dev, shape, seed):
    L, B, H, T, D = shape
    x = make_kv_cache(L, B, H, T, D, seed, outlier_heads=1)
    xv = x.reshape(2 * L, B, H, T * D)
    codes, scales = kv.fp8_quant_heads(xv.to(dev))
    wc, ws = O.fp8_quant_heads(bits16(xv))
    np.testing.assert_array_equal(scales.cpu().numpy().view(np.uint32), ws.view(np.uint32))
    np.testing.assert_array_equal(codes.cpu().numpy(), wc)
    y = kv.fp8_dequant_heads(codes, scales)
    assert_bf16_equal(bits16(y), O.fp8_dequant_heads(wc, ws))


@pytest.mark.parametrize("mode", ["single", "two", "auto"])
@pytest.mark.parametrize("shape", [(4, 1, 3, 16), (2, 3, 2, 30720 * 8 + 5 * 16), (3, 7, 3, 4000),
                                   (1, 1, 2, 64), (2, 300, 1, 16), (5, 2, 5, 61440 * 8), (40, 2, 8, 5760 * 8 * 3 + 16)])
def test_fp8_heads_single_and_two_pass(dev, shape, mode):
    """Both quantiser paths against the oracle ("single" forces the single pass below the
    256 MiB where "auto" picks two passes): runs split into several shares with a ragged
    last one, more batches than shares, spare groups (more groups than slabs), a slab
    needing more workgroups than the device has (falls back to two passes), 320 slabs of
    runs whose last share is two vectors long (many steps per group); special values in
    one slab of every shape."""
    two_pass = mode == "two"
    n_outer, B, H, run = shape
    g = torch.Generator().manual_seed(run + B)
    x = (torch.randn((n_outer, B, H, run), generator=g) * torch.rand((n_outer, 1, H, 1), generator=g) * 9)
    x[0, B - 1, H - 1, 3] = float("inf")
    x[n_outer - 1, 0, 0, run - 1] = -3.0e4
    x = x.to(torch.bfloat16)
    err = torch.zeros(1, dtype=torch.int32)
    codes, scales = kv.fp8_quant_heads(x.to(dev), two_pass=two_pass, single_pass=mode == "single", check=True)
    wc, ws = O.fp8_quant_heads(bits16(x))
    np.testing.assert_array_equal(scales.cpu().numpy().view(np.uint32), ws.view(np.uint32))
    np.testing.assert_array_equal(codes.cpu().numpy(), wc)
    del err


def test_fp8_heads_single_pass_at_size(dev):
    """The bench's 1 Gi-element shape [64, 4, 8, 2^19]: single pass equal to the two-pass path
    on every code and scale, and four whole slabs against the oracle."""
    x = torch.randn((64, 4, 8, 1 << 19), device=dev, generator=torch.Generator(device=dev).manual_seed(4))
    x = x.to(torch.bfloat16)
    c1, s1 = kv.fp8_quant_heads(x, check=True)
    c2, s2 = kv.fp8_quant_heads(x, two_pass=True)
    assert torch.equal(s1.view(torch.int32), s2.view(torch.int32))
    assert torch.equal(c1, c2)
    for o, h in ((0, 0), (17, 3), (40, 7), (63, 5)):
        wc, ws = O.fp8_quant_heads(bits16(x[o:o + 1, :, h:h + 1].contiguous()))
        assert s1[o, h].cpu().numpy().view(np.uint32) == ws.view(np.uint32)[0, 0]
        np.testing.assert_array_equal(c1[o:o + 1, :, h:h + 1].cpu().numpy(), wc)
    del x, c1, c2
    torch.cuda.empty_cache()


def test_fp8_heads_special_slabs(dev):
    """Zero slab (scale clamps to 1e-8/448), +-inf slab, NaN slab, subnormal bf16 inputs."""
    x = torch.randn((4, 1, 4, 64), dtype=torch.float32).to(torch.bfloat16)
    x[0, :, 0] = 0.0
    x[1, :, 1, 5] = float("inf")
    x[1, :, 1, 6] = -float("inf")
    x[2, :, 2, 7] = float("nan")
    x[3, :, 3] = torch.tensor([2.0 ** -130], dtype=torch.bfloat16) * torch.arange(64).float().to(torch.bfloat16)
    codes, scales = kv.fp8_quant_heads(x.to(dev))
    wc, ws = O.fp8_quant_heads(bits16(x))
    np.testing.assert_array_equal(scales.cpu().numpy().view(np.uint32), ws.view(np.uint32))
    np.testing.assert_array_equal(codes.cpu().numpy(), wc)
    assert_bf16_equal(bits16(kv.fp8_dequant_heads(codes, scales)), O.fp8_dequant_heads(wc, ws))


def make_append_case(L, H, D, P, lens, seed, extra_pages=7, start=None):
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    pos0 = [0] * B if start is None else list(start)
    ends = [s + n for s, n in zip(pos0, lens)]
    max_blocks = max((e + P - 1) // P for e in ends)
    need = sum((e + P - 1) // P for e in ends)
    n_pages = need + extra_pages
    perm = torch.randperm(n_pages, generator=g).to(torch.int32)
    bt = torch.full((B, max_blocks), -1, dtype=torch.int32)
    k = 0
    for b, e in enumerate(ends):
        nb = (e + P - 1) // P
        bt[b, :nb] = perm[k:k + nb]
        k += nb
    T = sum(lens)
    x = torch.randn((L, T, 2, H, D), generator=g, dtype=torch.float32)
    cu = torch.zeros(B + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    for b in range(B):  # 5%-style outliers: one (layer, head) per sequence x50
        l = int(torch.randint(L, (1,), generator=g))
        h = int(torch.randint(H, (1,), generator=g))
        x[l, cu[b]:cu[b + 1], :, h] *= 50.0
    sp = None if start is None else torch.tensor(pos0, dtype=torch.int32)
    return x.to(torch.bfloat16), cu, bt, n_pages, sp


@pytest.mark.parametrize("two_pass", [False, True])
def test_kv_quant_append_every_input_below_amax(dev, two_pass):
    """Complete input sets through the single-pass and the two-pass append: the slab of
    (kv, head) holds every bf16 bit pattern whose magnitude is at most its pattern a (both
    signs, so a is the slab's amax: -0 included), zero padded, over 1,024 tokens of two
    sequences with pages in random order.  Scales and pool bytes equal the oracle's."""
    H, D, P, T = 8, 128, 16, 1024
    tops = [0x0001, 0x2F00, 0x3280, 0x3A83, 0x3C00, 0x3F80, 0x43E0, 0x43E8, 0x4400, 0x4700, 0x5000, 0x6A00,
            0x7A00, 0x7F7F, 0x3E4C, 0x40A1]
    x = np.zeros((1, T, 2, H, D), np.uint16)
    for i, a in enumerate(tops):
        mags = np.arange(a + 1, dtype=np.uint16)
        v = np.zeros(T * D, np.uint16)
        both = np.concatenate([mags, mags | np.uint16(0x8000)])
        v[:both.size] = both
        x[0, :, i // H, i % H, :] = v.reshape(T, D)
    lens = [400, 624]
    cu = torch.tensor([0, 400, 1024], dtype=torch.int32)
    n_pages = 80
    g = torch.Generator().manual_seed(5)
    perm = torch.randperm(n_pages, generator=g).to(torch.int32)
    bt = torch.full((2, 40), -1, dtype=torch.int32)
    bt[0, :25] = perm[:25]
    bt[1, :39] = perm[25:64]
    pool = torch.zeros((1, n_pages, 2, H, P, D), dtype=torch.uint8)
    wpool = pool.numpy().copy()
    wsc, werr = O.kv_quant_append(x, cu.numpy(), None, bt.numpy(), wpool, P)
    assert werr == 0 and sum(lens) == T
    xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    pool_d = pool.to(dev)
    sc = kv.kv_quant_append(xt.to(dev), cu.to(dev), bt.to(dev), pool_d, check=True, two_pass=two_pass,
                            single_pass=not two_pass)
    np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), wsc.view(np.uint32))
    np.testing.assert_array_equal(pool_d.cpu().numpy(), wpool)
    # and back: every e4m3 code (-0 included) through the paged gather + dequant
    seq_lens = torch.tensor(lens, dtype=torch.int32)
    wk, wv, werr = O.kv_gather_dequant(wpool[0], wsc[0], bt.numpy(), seq_lens.numpy(), 640)
    assert werr == 0
    k, v = kv.kv_gather_dequant(pool_d[0], sc[0], bt.to(dev), seq_lens.to(dev), 640, check=True)
    assert_bf16_equal(bits16(k), wk)
    assert_bf16_equal(bits16(v), wv)


@pytest.mark.parametrize("H,D,P", [(8, 128, 16), (12, 64, 64), (2, 256, 5)])
def test_kv_quant_append_bit_exact(dev, H, D, P):
    L = 3
    lens = [1, 17, 300, 64, 129]
    x, cu, bt, n_pages, _ = make_append_case(L, H, D, P, lens, seed=H + D + P)
    pool = torch.zeros((L, n_pages, 2, H, P, D), dtype=torch.uint8)
    wpool = pool.numpy().copy()
    wsc, werr = O.kv_quant_append(bits16(x), cu.numpy(), None, bt.numpy(), wpool, P)
    assert werr == 0
    pool_d = pool.to(dev)
    sc = kv.kv_quant_append(x.to(dev), cu.to(dev), bt.to(dev), pool_d, check=True)
    np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), wsc.view(np.uint32))
    np.testing.assert_array_equal(pool_d.cpu().numpy(), wpool)
    # scales alone
    np.testing.assert_array_equal(kv.kv_scales(x.to(dev)).cpu().numpy().view(np.uint32), wsc.view(np.uint32))


def test_kv_quant_append_static_scales_decode_positions(dev):
    """Decode-style append at start_pos > 0 with scales fixed by an earlier prefill."""
    L, H, D, P = 2, 4, 128, 16
    lens = [1, 1, 3]
    x, cu, bt, n_pages, sp = make_append_case(L, H, D, P, lens, seed=11, start=[15, 40, 7])
    scales = torch.rand((L, 2, H), dtype=torch.float32, generator=torch.Generator().manual_seed(12)) * 0.05 + 1e-3
    pool = torch.randint(0, 255, (L, n_pages, 2, H, P, D), dtype=torch.uint8)
    wpool = pool.numpy().copy()
    _, werr = O.kv_quant_append(bits16(x), cu.numpy(), sp.numpy(), bt.numpy(), wpool, P,
                                scales=scales.numpy())
    assert werr == 8  # N(0,1) tokens under scales down to 1e-3: some exceed 464 x their scale
    pool_d = pool.to(dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    kv.kv_quant_append(x.to(dev), cu.to(dev), bt.to(dev), pool_d, scales=scales.to(dev),
                       start_pos=sp.to(dev), static_scales=True, err=err)
    assert int(err.item()) == werr
    np.testing.assert_array_equal(pool_d.cpu().numpy(), wpool)


def test_kv_quant_append_rejects_bad_page_ids(dev):
    L, H, D, P = 1, 2, 64, 16
    x, cu, bt, n_pages, _ = make_append_case(L, H, D, P, [20, 5], seed=3)
    bt[1, 0] = n_pages + 3  # out of range: must not be written, must be flagged
    pool = torch.zeros((L, n_pages, 2, H, P, D), dtype=torch.uint8)
    wpool = pool.numpy().copy()
    _, werr = O.kv_quant_append(bits16(x), cu.numpy(), None, bt.numpy(), wpool, P)
    assert werr == 1
    pool_d = pool.to(dev)
    with pytest.raises(ValueError, match="block table"):
        kv.kv_quant_append(x.to(dev), cu.to(dev), bt.to(dev), pool_d, check=True)
    np.testing.assert_array_equal(pool_d.cpu().numpy(), wpool)


@pytest.mark.parametrize("H,D,P,out_len", [(8, 128, 16, 512), (4, 64, 32, 200), (2, 256, 7, 100)])
def test_kv_gather_dequant_bit_exact(dev, H, D, P, out_len):
    g = torch.Generator().manual_seed(H * D + P)
    n_pages = 300
    B = 5
    max_blocks = (out_len + P - 1) // P
    pool = torch.randint(0, 256, (n_pages, 2, H, P, D), dtype=torch.uint8, generator=g)
    pool[pool == 0x7F] = 0x11
    pool[pool == 0xFF] = 0x91
    seq_lens = torch.tensor([out_len, 1, out_len // 2, 0, out_len - 3], dtype=torch.int32)
    bt = torch.stack([torch.randperm(n_pages, generator=g)[:max_blocks] for _ in range(B)]).to(torch.int32)
    scales = (torch.rand((2, H), generator=g) * 0.999 + 1e-3).float()
    wk, wv, werr = O.kv_gather_dequant(pool.numpy(), scales.numpy(), bt.numpy(), seq_lens.numpy(), out_len)
    assert werr == 0
    k, v = kv.kv_gather_dequant(pool.to(dev), scales.to(dev), bt.to(dev), seq_lens.to(dev), out_len, check=True)
    assert_bf16_equal(bits16(k), wk)
    assert_bf16_equal(bits16(v), wv)


def test_kv_gather_dequant_nan_codes_and_bad_pages(dev):
    H, D, P, out_len = 2, 64, 16, 64
    pool = torch.full((10, 2, H, P, D), 0x7F, dtype=torch.uint8)
    pool[:, :, :, :, 1::2] = 0xFF
    bt = torch.tensor([[0, 1, 2, 3], [4, 5, 11, 6]], dtype=torch.int32)
    seq_lens = torch.tensor([64, 64], dtype=torch.int32)
    scales = torch.ones((2, H), dtype=torch.float32)
    wk, wv, werr = O.kv_gather_dequant(pool.numpy(), scales.numpy(), bt.numpy(), seq_lens.numpy(), out_len)
    assert werr == 1
    with pytest.raises(ValueError, match="block table"):
        kv.kv_gather_dequant(pool.to(dev), scales.to(dev), bt.to(dev), seq_lens.to(dev), out_len, check=True)
    k, v = kv.kv_gather_dequant(pool.to(dev), scales.to(dev), bt.to(dev), seq_lens.to(dev), out_len)
    assert_bf16_equal(bits16(k), wk)
    assert_bf16_equal(bits16(v), wv)


@pytest.mark.parametrize("two_pass", [False, True])
@pytest.mark.parametrize("L,H,D,P,lens", [
    (2, 8, 128, 16, [1000, 17, 2048, 511]),   # single pass: every share fits in registers
    (1, 1, 256, 16, [30000, 20001]),          # share beyond the registers: spill path
    (1, 1, 256, 16, [60000, 41000]),          # share beyond twice the registers: two passes
    (3, 4, 64, 32, [3, 1, 2]),                # fewer tokens than workgroups
    (2, 3, 128, 16, [700, 45, 1300]),         # odd head count: K h paired with V h
    (2, 6, 64, 16, [900, 333]),               # even, not a power of two: K h with V h ^ 1
])
def test_kv_quant_append_fused_and_two_pass_bit_exact(dev, two_pass, L, H, D, P, lens):
    x, cu, bt, n_pages, _ = make_append_case(L, H, D, P, lens, seed=L * 1000 + H + D)
    pool = torch.zeros((L, n_pages, 2, H, P, D), dtype=torch.uint8)
    wpool = pool.numpy().copy()
    wsc, werr = O.kv_quant_append(bits16(x), cu.numpy(), None, bt.numpy(), wpool, P)
    assert werr == 0
    pool_d = pool.to(dev)
    sc = kv.kv_quant_append(x.to(dev), cu.to(dev), bt.to(dev), pool_d, check=True, two_pass=two_pass,
                            single_pass=not two_pass)
    np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), wsc.view(np.uint32))
    np.testing.assert_array_equal(pool_d.cpu().numpy(), wpool)


@pytest.mark.parametrize("two_pass", [False, True])
def test_kv_quant_append_special_slabs(dev, two_pass):
    """Slabs whose scale is clamped (all zero), +inf (holds +-inf), NaN (holds NaNs of both
    signs), and subnormal inputs, through the single-pass and the two-pass kernels."""
    L, H, D, P = 3, 4, 128, 16
    lens = [5, 40, 300, 77]
    x, cu, bt, n_pages, _ = make_append_case(L, H, D, P, lens, seed=21)
    x[0, :, 0, 0] = 0.0
    x[1, 7, 1, 1, 3] = float("inf")
    x[1, 100, 1, 1, 9] = -float("inf")
    xi = x.view(torch.int16)
    xi[2, 50, 0, 2, 11] = 0x7FC1
    xi[2, 51, 0, 2, 12] = -63  # 0xFFC1, a negative NaN
    x[2, :, 1, 3] = (torch.arange(x.shape[1] * D, dtype=torch.float32).reshape(-1, D) % 97 - 48) * 2.0 ** -133
    pool = torch.zeros((L, n_pages, 2, H, P, D), dtype=torch.uint8)
    wpool = pool.numpy().copy()
    wsc, werr = O.kv_quant_append(bits16(x), cu.numpy(), None, bt.numpy(), wpool, P)
    assert werr == 0
    assert np.isinf(wsc[1, 1, 1]) and np.isnan(wsc[2, 0, 2])
    pool_d = pool.to(dev)
    sc = kv.kv_quant_append(x.to(dev), cu.to(dev), bt.to(dev), pool_d, check=True, two_pass=two_pass,
                            single_pass=not two_pass)
    np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), wsc.view(np.uint32))
    np.testing.assert_array_equal(pool_d.cpu().numpy(), wpool)


def test_kv_quant_append_static_special_scales(dev):
    """Given scales of both signs, +-inf and NaN (inputs include +-inf)."""
    L, H, D, P = 1, 4, 64, 16
    lens = [33, 64]
    x, cu, bt, n_pages, _ = make_append_case(L, H, D, P, lens, seed=22)
    x[0, 3, 0, 1, 5] = float("inf")
    x[0, 4, 1, 2, 6] = -float("inf")
    scales = torch.tensor([[[0.02, -0.03, float("inf"), float("nan")],
                            [-float("inf"), 0.5, 1e-3, -7.0]]], dtype=torch.float32)
    pool = torch.zeros((L, n_pages, 2, H, P, D), dtype=torch.uint8)
    wpool = pool.numpy().copy()
    _, werr = O.kv_quant_append(bits16(x), cu.numpy(), None, bt.numpy(), wpool, P, scales=scales.numpy())
    assert werr == 8  # the 1e-3 slab overflows; the +-inf and NaN slabs never flag
    pool_d = pool.to(dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    kv.kv_quant_append(x.to(dev), cu.to(dev), bt.to(dev), pool_d, scales=scales.to(dev), static_scales=True,
                       err=err)
    assert int(err.item()) == werr
    np.testing.assert_array_equal(pool_d.cpu().numpy(), wpool)


@pytest.mark.parametrize("two_pass", [False, True])
def test_kv_quant_append_pool_layer_over_2gib(dev, two_pass):
    """A pool layer of 2.3 GB (70,000 pages of 32 KiB): pages past 2 GiB take the 64-bit
    store path.  The oracle runs on a compact pool with the same pages renumbered."""
    L, H, D, P = 1, 8, 128, 16
    lens = [100, 37, 250]
    x, cu, bt_small, n_small, _ = make_append_case(L, H, D, P, lens, seed=23, extra_pages=0)
    n_big = 70_000
    g = torch.Generator().manual_seed(24)
    big_ids = (n_big - 1 - torch.randperm(4000, generator=g)[:n_small]).to(torch.int32)  # > 2 GiB offsets
    bt_big = torch.where(bt_small >= 0, big_ids[bt_small.clamp(min=0).long()], bt_small)
    wpool = np.zeros((L, n_small, 2, H, P, D), np.uint8)
    wsc, werr = O.kv_quant_append(bits16(x), cu.numpy(), None, bt_small.numpy(), wpool, P)
    assert werr == 0
    pool_d = torch.zeros((L, n_big, 2, H, P, D), dtype=torch.uint8, device=dev)
    sc = kv.kv_quant_append(x.to(dev), cu.to(dev), bt_big.to(dev), pool_d, check=True, two_pass=two_pass,
                            single_pass=not two_pass)
    np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), wsc.view(np.uint32))
    got = pool_d[:, big_ids.long().to(dev)].cpu().numpy()
    np.testing.assert_array_equal(got, wpool)
    touched = int(pool_d[:, big_ids.long().to(dev)].sum(dtype=torch.int64))
    assert int(pool_d.sum(dtype=torch.int64)) == touched  # nothing written elsewhere
    del pool_d


def test_kv_quant_append_repeated_calls_reset_state(dev):
    """The single-pass kernel's counters live in the per-call workspace and start at zero:
    two appends in a row (second one smaller) both match the oracle."""
    for lens, seed in (([700, 300], 5), ([40], 6)):
        x, cu, bt, n_pages, _ = make_append_case(2, 8, 128, 16, lens, seed=seed)
        pool = torch.zeros((2, n_pages, 2, 8, 16, 128), dtype=torch.uint8)
        wpool = pool.numpy().copy()
        wsc, _ = O.kv_quant_append(bits16(x), cu.numpy(), None, bt.numpy(), wpool, 16)
        pool_d = pool.to(dev)
        sc = kv.kv_quant_append(x.to(dev), cu.to(dev), bt.to(dev), pool_d, check=True, single_pass=True)
        np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), wsc.view(np.uint32))
        np.testing.assert_array_equal(pool_d.cpu().numpy(), wpool)
