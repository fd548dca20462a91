"""Pins the CPU oracle (oracle/zx_oracle.c) before it is trusted as the GPU checker.

Each check is independent of the oracle's own code: torch's CPU casts to
float8_e4m3fn / bfloat16 / float16 (library routines), torch's evaluation of the
reference's precision.py expressions, the OCP e4m3fn boundary table, closed forms,
brute-force indexing in numpy, and the reference's own Belady test values.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O


def f32_bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def assert_bf16_equal(got, want):
    """Bit-exact, except that any NaN matches any NaN (torch's own bf16 casts write
    0x7FC0 on the scalar path and 0xFFFF on the vectorised one)."""
    g_nan = (got & 0x7FFF) > 0x7F80
    w_nan = (want & 0x7FFF) > 0x7F80
    np.testing.assert_array_equal(g_nan, w_nan)
    np.testing.assert_array_equal(got[~g_nan], want[~w_nan])


# ------------------------------------------------------------------ scalar formats

def test_e4m3_encode_all_bf16_matches_torch():
    v = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    want = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(O.e4m3_encode(v), want)


def test_e4m3_encode_random_fp32_matches_torch():
    rng = np.random.default_rng(1)
    v = np.concatenate([
        rng.uniform(-500, 500, 1 << 20).astype(np.float32),
        (rng.choice([-1, 1], 1 << 20) * np.exp2(rng.uniform(-16, 9, 1 << 20))).astype(np.float32),
        rng.integers(0, 1 << 32, 1 << 18, dtype=np.uint64).astype(np.uint32).view(np.float32),
    ])
    want = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(O.e4m3_encode(v), want)


def test_e4m3_midpoints_match_torch():
    grid = O.e4m3_decode(np.arange(256, dtype=np.uint8))
    grid = np.unique(np.abs(grid[np.isfinite(grid)]).astype(np.float64))
    grid = np.concatenate([grid, [480.0]])
    mids = ((grid[:-1] + grid[1:]) / 2).astype(np.float32)
    vals = [mids]
    up, dn = mids, mids
    for _ in range(3):
        up, dn = np.nextafter(up, np.float32(np.inf)), np.nextafter(dn, np.float32(0))
        vals += [up, dn]
    v = np.concatenate(vals + [-x for x in vals]).astype(np.float32)
    want = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(O.e4m3_encode(v), want)


# OCP OFP8 e4m3fn boundary table (include/zenyx_kv.h numeric contract).
KAT = [(448.0, 0x7E), (464.0, 0x7E), (470.0, 0x7F), (2.0 ** -10, 0x00), (1.5 * 2.0 ** -9, 0x02),
       (2.0 ** -9, 0x01), (1.0625, 0x38), (1.1875, 0x3A), (240.0, 0x77), (248.0, 0x78), (-0.0, 0x80),
       (float("inf"), 0x7F), (-float("inf"), 0xFF), (float("nan"), 0x7F), (-470.0, 0xFF), (2.0 ** -6, 0x08)]


@pytest.mark.parametrize("v,code", KAT)
def test_e4m3_boundary_table(v, code):
    assert int(O.e4m3_encode(np.array([v], np.float32))[0]) == code


def test_e4m3_decode_all_codes_matches_torch():
    c = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(c).view(torch.float8_e4m3fn).float().numpy()
    got = O.e4m3_decode(c)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_array_equal(f32_bits(got[ok]), f32_bits(want[ok]))


def test_e4m3_roundtrip_every_finite_code():
    c = np.arange(256, dtype=np.uint8)
    d = O.e4m3_decode(c)
    fin = ~np.isnan(d)
    np.testing.assert_array_equal(O.e4m3_encode(d[fin]), c[fin])


def test_bf16_and_f16_rounding_match_torch():
    rng = np.random.default_rng(2)
    v = np.concatenate([
        rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32),
        rng.standard_normal(1 << 18).astype(np.float32),
        np.array([0.0, -0.0, 1e-40, -1e-45, 3.4e38, 65504.0, 65520.0, 65519.99, 6e-8, 2.98e-8], np.float32),
    ]).astype(np.float32)
    t = torch.from_numpy(v)
    for mine, dt in ((O.bf16_rne, torch.bfloat16), (O.f16_rne, torch.float16)):
        got = mine(v)
        want = t.to(dt).view(torch.int16).numpy().view(np.uint16)
        nan = np.isnan(v)
        np.testing.assert_array_equal(got[~nan], want[~nan])
        assert np.all(np.isnan(t[nan].to(dt).float().numpy()))


# ------------------------------------------------------------------ FP8 per head

def torch_fp8_heads(x_bf16: torch.Tensor):
    """Independent composition with torch ops: amax per (outer, head), fp32 scale, IEEE
    division in fp32, torch's e4m3fn cast; dequant through torch's decode."""
    xf = x_bf16.float()
    amax = xf.abs().amax(dim=(1, 3))
    scale = amax.clamp_min(1e-8) / 448.0
    q = (xf / scale[:, None, :, None]).to(torch.float8_e4m3fn)
    y = (q.float() * scale[:, None, :, None]).to(torch.bfloat16)
    return q.view(torch.uint8).numpy(), scale.numpy(), y.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("seed", [0, 1])
def test_fp8_heads_oracle_matches_torch_composition(seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((6, 2, 5, 128), generator=g)
    x[1, :, 2] *= 50.0
    x[3, :, 0] *= 1e-30
    x = x.to(torch.bfloat16)
    bits = x.view(torch.int16).numpy().view(np.uint16)
    codes, scales = O.fp8_quant_heads(bits)
    tq, ts, ty = torch_fp8_heads(x)
    np.testing.assert_array_equal(f32_bits(scales), f32_bits(ts))
    np.testing.assert_array_equal(codes, tq)
    np.testing.assert_array_equal(O.fp8_dequant_heads(codes, scales), ty)


def test_fp8_scale_closed_forms():
    assert O.fp8_scale(448.0) == 1.0
    assert O.fp8_scale(0.0) == np.float32(np.float32(1e-8) / np.float32(448.0))
    assert np.isnan(O.fp8_scale(float("nan")))
    assert O.fp8_scale(float("inf")) == float("inf")


def test_fp8_quantized_values_never_exceed_range():
    # |x / scale| <= 448 (1 + eps) for every x of the slab, so no finite input maps to NaN
    g = torch.Generator().manual_seed(3)
    x = (torch.randn((3, 1, 4, 4096), generator=g) * 1e4).to(torch.bfloat16)
    codes, _ = O.fp8_quant_heads(x.view(torch.int16).numpy().view(np.uint16))
    assert not np.any((codes & 0x7F) == 0x7F)
    # the largest |x| of each slab encodes to +-448
    assert np.all(np.isin(np.max(codes & 0x7F, axis=(1, 3)), [0x7E]))


# ------------------------------------------------------------------ paged KV (brute force)

def test_paged_append_and_gather_match_brute_force_indexing():
    rng = np.random.default_rng(4)
    L, H, D, P = 2, 3, 64, 8
    lens = [5, 17, 1, 30]
    B = len(lens)
    maxb = max((n + P - 1) // P for n in lens)
    n_pages = sum((n + P - 1) // P for n in lens) + 3
    perm = rng.permutation(n_pages).astype(np.int32)
    bt = np.full((B, maxb), -1, np.int32)
    k = 0
    for b, n in enumerate(lens):
        nb = (n + P - 1) // P
        bt[b, :nb] = perm[k:k + nb]
        k += nb
    T = sum(lens)
    x = torch.randn((L, T, 2, H, D), generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pool = np.zeros((L, n_pages, 2, H, P, D), np.uint8)
    scales, err = O.kv_quant_append(xb, cu, None, bt, pool, P)
    assert err == 0
    # brute force: codes of each (l, kv, h) from the per-head torch composition
    xf = x.float()
    sc_t = (xf.abs().amax(dim=(1, 4)).clamp_min(1e-8) / 448.0)  # [L, 2, H]
    np.testing.assert_array_equal(f32_bits(scales), f32_bits(sc_t.numpy()))
    codes = (xf / sc_t[:, None, :, :, None]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    want = np.zeros_like(pool)
    seq = np.repeat(np.arange(B), lens)
    pos = np.concatenate([np.arange(n) for n in lens])
    pages = bt[seq, pos // P]
    for l in range(L):
        want[l, pages, :, :, pos % P, :] = codes[l]
    np.testing.assert_array_equal(pool, want)
    # gather of layer 1 back: bytes and dequant vs torch decode
    out_len = maxb * P
    kk, vv, gerr = O.kv_gather_dequant(pool[1], scales[1], bt, np.array(lens, np.int32), out_len)
    assert gerr == 0
    for b in range(B):
        n = lens[b]
        t = np.arange(n)
        c = pool[1][bt[b, t // P], :, :, t % P, :]  # [n, 2, H, D]
        dq = (torch.from_numpy(c).view(torch.float8_e4m3fn).float() * torch.from_numpy(scales[1])[None, :, :, None]
              ).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        np.testing.assert_array_equal(kk[b, :, :n], dq[:, 0].transpose(1, 0, 2))
        np.testing.assert_array_equal(vv[b, :, :n], dq[:, 1].transpose(1, 0, 2))
        assert not kk[b, :, n:].any() and not vv[b, :, n:].any()


def _small_tables(rng, lens, P):
    B = len(lens)
    maxb = max((n + P - 1) // P for n in lens)
    n_pages = sum((n + P - 1) // P for n in lens) + 2
    perm = rng.permutation(n_pages).astype(np.int32)
    bt = np.full((B, maxb), -1, np.int32)
    k = 0
    for b, n in enumerate(lens):
        nb = (n + P - 1) // P
        bt[b, :nb] = perm[k:k + nb]
        k += nb
    return bt, n_pages


@pytest.mark.parametrize("saturate", [False, True])
def test_static_append_overflow_matches_torch(saturate):
    """Static scales: a finite token beyond 464 |s| gets the torch cast's NaN code and
    sets bit 8; with saturation it gets clamp(x / s, -448, 448)'s code instead.  Slabs
    with a non-finite scale keep the plain cast either way (a -inf scale: zeros signed
    opposite to x).  Pinned by torch's division and float8_e4m3fn cast (and torch.clamp
    for saturation)."""
    rng = np.random.default_rng(11)
    L, H, D, P = 2, 3, 64, 4
    lens = [3, 6, 1]
    bt, n_pages = _small_tables(rng, lens, P)
    T = sum(lens)
    x = torch.randn((L, T, 2, H, D), generator=torch.Generator().manual_seed(11)) * 8
    x[0, 0, 0, 0, :4] = torch.tensor([float("inf"), -float("inf"), float("nan"), -3.0e4])
    x[0, 1, 0, 1, :3] = torch.tensor([float("inf"), -float("inf"), float("nan")])  # negative scale below
    x = x.to(torch.bfloat16)
    x.view(torch.int16)[0, 2, 0, 1, 3] = -63  # 0xFFC1: a NaN with the sign bit set
    sc = torch.tensor([[[0.01, -0.02, 0.5], [1.0, float("inf"), -0.004]],
                       [[-float("inf"), 2.0, -0.1], [0.007, 1e3, -1e-3]]], dtype=torch.float32)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pool = np.zeros((L, n_pages, 2, H, P, D), np.uint8)
    got_sc, err = O.kv_quant_append(xb, cu, None, bt, pool, P, scales=sc.numpy(), saturate=saturate)
    np.testing.assert_array_equal(f32_bits(got_sc), f32_bits(sc.numpy()))  # static: unchanged
    xf = x.float()
    q = xf / sc[:, None, :, :, None]
    finite = torch.isfinite(xf) & torch.isfinite(sc)[:, None, :, :, None]
    plain = q.to(torch.float8_e4m3fn).view(torch.uint8)
    over = finite & ((plain & 0x7F) == 0x7F)
    assert over.any() and not over.all()
    assert err == (8 if over.any() else 0)
    codes = (torch.where(finite, q.clamp(-448.0, 448.0), q) if saturate else q).to(torch.float8_e4m3fn)
    codes = codes.view(torch.uint8).numpy()
    want = np.zeros_like(pool)
    seq = np.repeat(np.arange(len(lens)), lens)
    pos = np.concatenate([np.arange(n) for n in lens])
    for l in range(L):
        want[l, bt[seq, pos // P], :, :, pos % P, :] = codes[l]
    np.testing.assert_array_equal(pool, want)
    # dynamic scales never overflow a finite input
    x2 = (torch.randn((L, T, 2, H, D), generator=torch.Generator().manual_seed(12)) * 1e4).to(torch.bfloat16)
    pool2 = np.zeros_like(pool)
    _, err2 = O.kv_quant_append(x2.view(torch.int16).numpy().view(np.uint16), cu, None, bt, pool2, P)
    assert err2 == 0 and not ((pool2 & 0x7F) == 0x7F).any()


# ------------------------------------------------------------------ legacy int8 vs torch

def torch_reference_expr(x: torch.Tensor):
    """The expressions of zenyx/streaming/precision.py:10-11, 16 evaluated by torch on CPU."""
    scale = x.abs().amax().clamp_min(1e-8) / 127.0
    q = torch.clamp((x / scale).round(), -127, 127).to(torch.int8)
    y = (q.float() * scale).to(torch.bfloat16)
    return q, scale, y


@pytest.mark.parametrize("dt,tdt", [("bf16", torch.bfloat16), ("f16", torch.float16), ("f32", torch.float32)])
@pytest.mark.parametrize("mag", [1.0, 1e-4, 2e4, 0.0, 1e-7])
def test_int8_legacy_oracle_matches_torch(dt, tdt, mag):
    g = torch.Generator().manual_seed(int(mag * 1000) % 97)
    x = (torch.randn(3001, generator=g) * mag).to(tdt)
    q, s, y = torch_reference_expr(x)
    raw = x.view(torch.int16).numpy().view(np.uint16) if tdt != torch.float32 else x.numpy()
    wq, ws = O.int8_legacy_quant(raw, dt)
    np.testing.assert_array_equal(wq, q.numpy())
    assert np.float32(ws) == np.float32(s.float().item()) or (np.isnan(ws) and torch.isnan(s))
    assert_bf16_equal(O.int8_legacy_dequant(wq, ws), y.view(torch.int16).numpy().view(np.uint16))


def test_int8_legacy_scale_every_bf16_amax():
    """Scale rounding over every positive finite bf16 amax, against torch's 0-dim path."""
    vals = (np.arange(1, 0x7F80, 37, dtype=np.uint32) << 16).view(np.float32)
    for v in vals[::50]:
        x = torch.tensor([float(v), -float(v) / 3], dtype=torch.bfloat16)
        _, s, _ = torch_reference_expr(x)
        _, ws = O.int8_legacy_quant(x.view(torch.int16).numpy().view(np.uint16), "bf16")
        assert np.float32(ws) == np.float32(s.float().item())


# ------------------------------------------------------------------ Belady

def test_reference_belady_known_answer():
    """zenyx/tests/test_streaming.py:14-22, on the restated class."""
    cache = O.RefBeladyApproxCache(capacity=2)
    cache.update_future("a", 1)
    cache.update_future("b", 100)
    cache.update_future("c", 2)
    cache.touch("a")
    cache.touch("b")
    assert cache.touch("c") == ["b"]
    assert cache.resident == {"a", "c"}


def test_reference_belady_known_answer_as_trace():
    # The same instance as a page trace: a=0, b=1, c=2 with next uses 1, 100, 2 means the
    # trace continues a, c and b far later; capacity 2 evicts b at the miss on c.
    trace = np.array([0, 1, 2, 0, 2] + [3] * 95 + [1], np.int32)
    ep, eg, st = O.belady_simulate(trace, 4, 2)
    assert (int(ep[0]), int(eg[0])) == (2, 1)
    assert [tuple(map(int, e)) for e in zip(ep, eg)] == O.ref_belady_trace(trace, 2)


def brute_force_min_misses(trace, cap):
    """Fewest misses over every eviction choice (exhaustive; tiny traces only)."""
    from functools import lru_cache

    trace = tuple(int(p) for p in trace)

    @lru_cache(maxsize=None)
    def go(i, res):
        if i == len(trace):
            return 0
        p = trace[i]
        if p in res:
            return go(i + 1, res)
        if len(res) < cap:
            return 1 + go(i + 1, tuple(sorted(res + (p,))))
        return 1 + min(go(i + 1, tuple(sorted(tuple(r for r in res if r != v) + (p,)))) for v in res)

    return go(0, ())


@pytest.mark.parametrize("seed", range(12))
def test_belady_heap_matches_linear_scan_and_is_optimal(seed):
    rng = np.random.default_rng(seed)
    n_pages = int(rng.integers(2, 7))
    cap = int(rng.integers(1, n_pages))
    trace = rng.integers(0, n_pages, int(rng.integers(1, 14))).astype(np.int32)
    ep, eg, st = O.belady_simulate(trace, n_pages, cap)
    assert [tuple(map(int, e)) for e in zip(ep, eg)] == O.ref_belady_trace(trace, cap)
    assert st["misses"] == brute_force_min_misses(trace, cap)
    assert st["misses"] + st["hits"] == len(trace)


@pytest.mark.parametrize("seed", range(6))
def test_belady_heap_matches_linear_scan_larger(seed):
    rng = np.random.default_rng(100 + seed)
    n_pages = int(rng.integers(5, 60))
    cap = int(rng.integers(1, n_pages + 3))
    trace = rng.integers(0, n_pages, 600).astype(np.int32)
    ep, eg, st = O.belady_simulate(trace, n_pages, cap)
    assert [tuple(map(int, e)) for e in zip(ep, eg)] == O.ref_belady_trace(trace, cap)


def test_belady_argmax_matches_lexsort():
    """belady.py:44-50 semantics (largest key > -1 among residents; ties to the smallest
    rank, then the smallest slot) against numpy's lexsort on random inputs with many ties
    and negative keys; without ranks the slot index is the rank, without a residency
    array every slot is a candidate."""
    rng = np.random.default_rng(11)
    for n in (1, 5, 64, 1000):
        for _ in range(20):
            keys = rng.integers(-3, 6, n).astype(np.int64)
            res = (rng.random(n) < 0.5).astype(np.uint8)
            rank = rng.integers(0, max(2, n // 3), n).astype(np.int64)  # ties in rank too
            for r_arg, use_res in ((None, True), (rank, True), (rank, False)):
                cand = (res == 1) if use_res else np.ones(n, bool)
                ok = np.nonzero(cand & (keys > -1))[0]
                r = ok if r_arg is None else r_arg[ok]
                if ok.size == 0:
                    want = (-1, -1)
                else:
                    order = np.lexsort((ok, r, -keys[ok]))  # key descending, rank, slot ascending
                    want = (int(ok[order[0]]), int(keys[ok[order[0]]]))
                assert O.belady_argmax(keys, res if use_res else None, r_arg) == want


def test_next_use_matches_dictionary_scan():
    rng = np.random.default_rng(12)
    trace = rng.integers(0, 37, 5000).astype(np.int32)
    nu, pu = O.next_use(trace, 37)
    last, nxt = {}, [O.NEVER] * len(trace)
    for i in range(len(trace) - 1, -1, -1):
        nxt[i] = last.get(int(trace[i]), O.NEVER)
        last[int(trace[i])] = i
    prv, seen = [-1] * len(trace), {}
    for i, p in enumerate(trace.tolist()):
        prv[i] = seen.get(p, -1)
        seen[p] = i
    assert nu.tolist() == nxt and pu.tolist() == prv


def test_next_use_closed_form():
    trace = np.array([3, 1, 3, 3, 0, 1], np.int32)
    nu, pu = O.next_use(trace, 4)
    N = O.NEVER
    assert nu.tolist() == [2, 5, 3, N, N, N]
    assert pu.tolist() == [-1, -1, 0, 2, -1, 1]


def test_ring_trace_structure():
    L, R, S = 3, 8, 4
    tr = O.ring_trace(L, R, S)
    assert tr.size == 2 * L * R * R * S
    fwd, bwd = tr[: tr.size // 2], tr[tr.size // 2:]
    np.testing.assert_array_equal(bwd, fwd[::-1])
    # every page of a layer is touched once per ring step (R times per layer in forward)
    counts = np.bincount(fwd, minlength=L * R * S)
    assert np.all(counts == R)
    # step s, device d reads shard (d - s) mod R
    blk = fwd[: R * R * S].reshape(R, R, S)
    for s in range(R):
        for d in range(R):
            assert blk[s, d, 0] == ((d - s) % R) * S
    # degree-1 ring of one layer reduces to build_ring_timeline (kv_tiering.py:69-73)
    one = O.ring_trace(1, 1, 5)
    ref = O.ref_ring_timeline(5)
    assert one.tolist() == ref["forward"] + ref["backward"]


@pytest.mark.parametrize("Hq,Hkv,D,P,seed", [(8, 2, 64, 16, 0), (4, 4, 128, 5, 1), (8, 1, 256, 32, 2)])
def test_paged_attention_oracle_matches_torch_sdpa(Hq, Hkv, D, P, seed):
    """The oracle's decode attention against torch's float64 softmax(qK^T)V on K/V built by
    plain numpy indexing of the pool (codes decoded, times the per-head scale), including
    an empty sequence, a one-token one and a partial last page."""
    rng = np.random.default_rng(seed)
    lens = np.array([0, 1, 3 * P + 2, 50], np.int32)
    B, n_pages = len(lens), 64
    max_blocks = (int(lens.max()) + P - 1) // P
    pool = rng.integers(0, 256, (n_pages, 2, Hkv, P, D), dtype=np.uint8)
    pool[(pool & 0x7F) == 0x7F] = 0x12  # no NaN codes
    bt = np.stack([rng.permutation(n_pages)[:max_blocks] for _ in range(B)]).astype(np.int32)
    scales = rng.uniform(1e-3, 0.05, (2, Hkv)).astype(np.float32)
    q = torch.randn((B, Hq, D), dtype=torch.float32, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
    qb = q.view(torch.int16).numpy().view(np.uint16)
    # the softmax scale crosses the C ABI as a float: the float64 reference uses the same value
    sm = float(np.float32(1.0 / np.sqrt(D)))
    got, err = O.paged_attention_decode(qb, pool, scales, bt, lens, sm)
    assert err == 0
    dec = O.e4m3_decode(np.arange(256, dtype=np.uint8)).astype(np.float64)
    grp = Hq // Hkv
    for b in range(B):
        t = np.arange(lens[b])
        pages = bt[b, t // P]
        for hq in range(Hq):
            h = hq // grp
            K = torch.from_numpy(dec[pool[pages, 0, h, t % P, :]] * float(scales[0, h]))
            V = torch.from_numpy(dec[pool[pages, 1, h, t % P, :]] * float(scales[1, h]))
            qd = q[b, hq].double()
            if lens[b] == 0:
                want = torch.zeros(D, dtype=torch.bfloat16)
            else:
                p = torch.softmax((K @ qd) * sm, dim=0)
                want = (p @ V).float().to(torch.bfloat16)
            w = want.view(torch.int16).numpy().view(np.uint16)
            np.testing.assert_array_equal(got[b, hq], w)


@pytest.mark.parametrize("Hq,Hkv,P,causal,seed", [(8, 2, 16, 1, 0), (4, 4, 32, 0, 1), (6, 3, 16, 1, 2),
                                                   (2, 1, 48, 0, 3)])
def test_prefill_attention_oracle_matches_torch(Hq, Hkv, P, causal, seed):
    """The oracle's block attention (one ring step) against torch's float64
    softmax(qK^T)V with an explicit key range and causal mask, K/V built by numpy indexing
    of the pool; includes a query block starting mid-sequence, a key range starting
    mid-page and an empty key range (zeros, lse -inf)."""
    rng = np.random.default_rng(seed)
    D = 128
    n_q = [5, 17, 3]
    q_pos0 = np.array([0, 40, 100], np.int32)
    kv_begin = np.array([0, 9, 60], np.int32)
    kv_end = np.array([5, 61, 60], np.int32)
    cu = np.concatenate([[0], np.cumsum(n_q)]).astype(np.int32)
    max_blocks = 8
    n_pages = 40
    pool = rng.integers(0, 256, (n_pages, 2, Hkv, P, D), dtype=np.uint8)
    pool[(pool & 0x7F) == 0x7F] = 0x12
    bt = np.stack([rng.permutation(n_pages)[:max_blocks] for _ in range(3)]).astype(np.int32)
    scales = rng.uniform(1e-3, 0.05, (2, Hkv)).astype(np.float32)
    q = torch.randn((cu[-1], Hq, D), generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
    qb = q.view(torch.int16).numpy().view(np.uint16)
    sm = float(np.float32(1.0 / np.sqrt(D)))
    got, lse, err = O.paged_attention_prefill(qb, cu, q_pos0, pool, scales, bt, kv_begin, kv_end, causal, sm)
    assert err == 0
    dec = O.e4m3_decode(np.arange(256, dtype=np.uint8)).astype(np.float64)
    grp = Hq // Hkv
    for b in range(3):
        for i in range(cu[b], cu[b + 1]):
            qp = q_pos0[b] + i - cu[b]
            t = np.arange(kv_begin[b], kv_end[b])
            if causal:
                t = t[t <= qp]
            pages = bt[b, t // P]
            for hq in range(Hq):
                h = hq // grp
                w = got[i, hq]
                if t.size == 0:
                    assert np.all(w == 0) and lse[i, hq] == -np.inf
                    continue
                K = torch.from_numpy(dec[pool[pages, 0, h, t % P, :]] * float(scales[0, h]))
                V = torch.from_numpy(dec[pool[pages, 1, h, t % P, :]] * float(scales[1, h]))
                s = (K @ q[i, hq].double()) * sm
                want = (torch.softmax(s, dim=0) @ V).float().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
                np.testing.assert_array_equal(w, want)
                want_lse = float(torch.logsumexp(s, dim=0)) / np.log(2.0)
                assert abs(lse[i, hq] - want_lse) <= 2e-6 * max(1.0, abs(want_lse))


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_legacy_reciprocal_quotient_matches_division(dt):
    """The GPU's legacy quantiser forms x / s for bf16 / f16 input from r = 1 / s and one
    Markstein correction: every 97th reachable scale against every input of the format
    gives the same int8 code as IEEE division (the full set, stride 1, was run too)."""
    bad, pairs = O.legacy_reciprocal_check(dt, 97)
    assert pairs > 10_000_000
    assert bad == 0


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_legacy_fast_encoder_matches_division(dt):
    """The GPU's fast legacy encoder (no range guard, integer rounding by adding 1.5 * 2^23)
    gives the reference code for every reachable pair: every finite x with |x| at most the
    largest amax of its scale, every 61st scale (the full set, stride 1, was run too)."""
    bad, pairs = O.legacy_fast_check(dt, 61)
    assert pairs > 5_000_000
    assert bad == 0


def test_fp8_encoders_need_the_correction_step():
    """Why the FP8 encoders keep the Markstein step even with dynamic scales (|x| <= amax):
    the plain product x * RN(1 / s) gives another e4m3 code than x / s on some pairs."""
    bad, pairs = O.fp8_product_check(101)
    assert pairs > 10_000_000
    assert bad > 0


def test_torch_restatements_of_append_and_gather_match_c():
    """The torch CPU restatements bench.py times as the multi-threaded CPU baseline give
    the C oracle's scales, pool bytes and gathered values bit for bit."""
    g = torch.Generator().manual_seed(12)
    H, D, P = 4, 128, 16
    lens = [37, 16, 100]
    nb = [(n + P - 1) // P for n in lens]
    n_pages = sum(nb) + 3
    perm = torch.randperm(n_pages, generator=g).numpy().astype(np.int32)
    bt = np.full((3, max(nb)), -1, np.int32)
    k = 0
    for b in range(3):
        bt[b, :nb[b]] = perm[k:k + nb[b]]
        k += nb[b]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    x = (torch.randn((sum(lens), 2, H, D), generator=g) * 3).to(torch.bfloat16)
    x[5, 1, 2] *= 40
    sc, pool = O.kv_quant_append_torch(x, cu, bt, n_pages, P)
    wpool = np.zeros((1, n_pages, 2, H, P, D), np.uint8)
    wsc, err = O.kv_quant_append(x.view(torch.int16).numpy().view(np.uint16)[None], cu, None, bt, wpool, P)
    assert err == 0
    np.testing.assert_array_equal(sc.numpy().view(np.uint32), wsc[0].view(np.uint32))
    np.testing.assert_array_equal(pool.numpy(), wpool[0])
    out_len = max(nb) * P
    kt, vt = O.kv_gather_dequant_torch(pool, sc, bt, lens, out_len)
    wk, wv, gerr = O.kv_gather_dequant(wpool[0], wsc[0], bt, np.array(lens, np.int32), out_len)
    assert gerr == 0
    np.testing.assert_array_equal(kt.view(torch.int16).numpy().view(np.uint16), wk)
    np.testing.assert_array_equal(vt.view(torch.int16).numpy().view(np.uint16), wv)
