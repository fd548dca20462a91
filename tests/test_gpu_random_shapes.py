"""Seeded random configurations through the HIP kernels against the C oracle: shapes the
parametrized tests do not list (head counts 1-9, head dims 64 / 128 / 256, page sizes
from 1 to 48, one to six ragged sequences, prefill rows that start late and key ranges
that start or end inside a page), and a paged cache whose per-layer scales are not 16-byte
aligned.

* paged append + fused FP8 quantisation, single pass and two passes: codes and scales
  bit-exact (the oracle's restatement of the reference's e4m3fn cast);
* paged gather + dequant of every layer that append wrote: bf16 bit-exact;
* decode attention from the pages: one bf16 ulp + 2^-17 max|V| (test_gpu_attention.py);
* one prefill / ring step, and ring attention over 1-5 shards in one launch or one launch
  per shard (fp16 P, the default): two bf16 ulps + 2^-10 max|V| (test_gpu_prefill.py);
* the per-head FP8 quantiser (both paths) and the legacy int8 per-slab functions in
  every dtype: bit-exact.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from test_gpu_attention import assert_within_one_ulp, make_case, v_colmax
from test_gpu_kv import assert_bf16_equal, bits16, make_append_case
from test_gpu_prefill import assert_precision, make, run_step, vmax_rows
from zenyx_amd import kv

pytestmark = pytest.mark.gpu


def _append_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        L = int(rng.integers(1, 4))
        H = int(rng.integers(1, 10))
        D = int(rng.choice([64, 128, 256]))
        P = int(rng.choice([1, 3, 8, 16, 32, 48]))
        lens = [int(v) for v in rng.integers(0, 400, int(rng.integers(1, 7)))]
        if not any(lens):
            lens[0] = 1
        cases.append((i, L, H, D, P, lens))
    return cases


@pytest.mark.parametrize("case", _append_cases(16, 2026), ids=lambda c: f"a{c[0]}")
def test_random_append_then_gather(dev, case):
    i, L, H, D, P, lens = case
    print(f"append/gather case {i}: L={L} H={H} D={D} P={P} lens={lens}", flush=True)
    x, cu, bt, n_pages, _ = make_append_case(L, H, D, P, lens, seed=100 + i)
    pool = torch.zeros((L, n_pages, 2, H, P, D), dtype=torch.uint8)
    wpool = pool.numpy().copy()
    wsc, werr = O.kv_quant_append(bits16(x), cu.numpy(), None, bt.numpy(), wpool, P)
    assert werr == 0
    for two_pass in (False, True):
        pool_d = pool.to(dev)
        sc = kv.kv_quant_append(x.to(dev), cu.to(dev), bt.to(dev), pool_d, check=True, two_pass=two_pass,
                                single_pass=not two_pass)
        np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), wsc.view(np.uint32))
        np.testing.assert_array_equal(pool_d.cpu().numpy(), wpool)
    seq_lens = torch.tensor(lens, dtype=torch.int32)
    out_len = max(lens)
    for layer in range(L):
        wk, wv, gerr = O.kv_gather_dequant(wpool[layer], wsc[layer], bt.numpy(), seq_lens.numpy(), out_len)
        assert gerr == 0
        k, v = kv.kv_gather_dequant(pool_d[layer], sc[layer], bt.to(dev), seq_lens.to(dev), out_len, check=True)
        assert_bf16_equal(bits16(k), wk)
        assert_bf16_equal(bits16(v), wv)


def _attention_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        Hkv = int(rng.integers(1, 9))
        Hq = Hkv * int(rng.choice([1, 2, 3, 4, 8]))
        D = int(rng.choice([64, 128, 256]))
        P = int(rng.choice([5, 16, 32]))
        lens = [int(v) for v in rng.integers(0, 3000, int(rng.integers(1, 6)))]
        cases.append((i, Hq, Hkv, D, P, lens))
    return cases


@pytest.mark.parametrize("case", _attention_cases(12, 7), ids=lambda c: f"d{c[0]}")
def test_random_decode_attention(dev, case):
    i, Hq, Hkv, D, P, lens = case
    print(f"decode case {i}: Hq={Hq} Hkv={Hkv} D={D} P={P} lens={lens}", flush=True)
    q, pool, scales, bt, lens = make_case(Hq, Hkv, D, P, lens, seed=300 + i)
    sm = 1.0 / np.sqrt(D)
    want, werr = O.paged_attention_decode(bits16(q), pool, scales, bt, lens, sm)
    assert werr == 0
    got = kv.paged_attention_decode(q.to(dev), torch.from_numpy(pool).to(dev), torch.from_numpy(scales).to(dev),
                                    torch.from_numpy(bt).to(dev), torch.from_numpy(lens).to(dev), check=True)
    assert_within_one_ulp(bits16(got), want, v_colmax(pool, scales, bt, lens, Hq))


def _prefill_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        Hkv = int(rng.integers(1, 5))
        Hq = Hkv * int(rng.choice([1, 2, 3, 4]))
        P = int(rng.choice([16, 32, 48]))
        B = int(rng.integers(1, 5))
        n_q = [int(v) for v in rng.integers(0, 200, B)]
        q_pos0 = [int(v) for v in rng.integers(0, 300, B)]
        kb = [int(rng.integers(0, 40)) for _ in range(B)]
        ke = [max(k, qp + nq + int(rng.integers(-30, 30))) for k, qp, nq in zip(kb, q_pos0, n_q)]
        cases.append((i, Hq, Hkv, P, n_q, q_pos0, kb, ke, bool(rng.integers(0, 2))))
    return cases


@pytest.mark.parametrize("case", _prefill_cases(10, 11), ids=lambda c: f"p{c[0]}")
def test_random_prefill_step(case):
    i, Hq, Hkv, P, n_q, q_pos0, kb, ke, causal = case
    print(f"prefill case {i}: Hq={Hq} Hkv={Hkv} P={P} n_q={n_q} q_pos0={q_pos0} kv=[{kb}, {ke}) causal={causal}",
          flush=True)
    q, pool, scales, bt, cu, qp = make(Hq, Hkv, P, n_q, q_pos0, ke, seed=500 + i)
    kb, ke = np.asarray(kb, np.int32), np.asarray(ke, np.int32)
    out, _ = run_step(q, pool, scales, bt, cu, qp, kb, ke, causal, "f16")
    torch.cuda.synchronize()
    sm = float(np.float32(1.0 / np.sqrt(128)))
    want, _, err = O.paged_attention_prefill(bits16(q), cu, qp, pool, scales, bt, kb, ke, causal, sm)
    assert err == 0
    assert_precision(bits16(out), want, vmax_rows(pool, scales, bt, cu, kb, ke, Hq), "f16")


@pytest.mark.parametrize("H", [1, 3])
def test_paged_cache_odd_kv_head_count(dev, H):
    """With an odd number of KV heads, every other layer's [2, H] scales start 8 bytes off a
    16-byte boundary; the cache's gather and decode of such a layer match the oracle."""
    from zenyx_amd.train.fp8_kv_quantization import PagedFP8KVCache, QuantizedRingAttention

    L, D, P = 2, 128, 16
    print(f"paged cache with H={H}", flush=True)
    cache = PagedFP8KVCache(L, H, D, num_pages=40, page_size=P, device=dev)
    g = torch.Generator().manual_seed(40 + H)
    lens = [37, 100]
    x = torch.randn((L, sum(lens), 2, H, D), generator=g).to(torch.bfloat16)
    cache.append(x, ["a", "b"], lens, check=True)
    bt = np.full((2, max(len(cache.pages[s]) for s in "ab")), -1, np.int32)
    for i, s in enumerate("ab"):
        bt[i, :len(cache.pages[s])] = cache.pages[s]
    pool = np.zeros((L, 40, 2, H, P, D), np.uint8)
    sc, err = O.kv_quant_append(bits16(x), np.array([0, 37, 137], np.int32), None, bt, pool, P)
    assert err == 0
    np.testing.assert_array_equal(cache.scales.cpu().numpy().view(np.uint32), sc.view(np.uint32))
    k, v = cache.gather(1, ["a", "b"])
    wk, wv, gerr = O.kv_gather_dequant(pool[1], sc[1], bt, np.array(lens, np.int32), max(lens))
    assert gerr == 0
    assert_bf16_equal(bits16(k), wk)
    assert_bf16_equal(bits16(v), wv)
    Hq = 2 * H
    q = torch.randn((2, Hq, D), generator=g).to(torch.bfloat16)
    got = QuantizedRingAttention(cache).decode(q.to(dev), 1, ["a", "b"])
    want, werr = O.paged_attention_decode(bits16(q), pool[1], sc[1], bt, np.array(lens, np.int32),
                                          1.0 / np.sqrt(D))
    assert werr == 0
    assert_within_one_ulp(bits16(got), want, v_colmax(pool[1], sc[1], bt, np.array(lens, np.int32), Hq))


def _heads_cases(n, seed):
    rng = np.random.default_rng(seed)
    return [(i, int(rng.integers(1, 7)), int(rng.integers(1, 6)), int(rng.integers(1, 10)),
             16 * int(rng.integers(1, 1500))) for i in range(n)]  # runs are whole 16-element groups


@pytest.mark.parametrize("case", _heads_cases(10, 5), ids=lambda c: f"h{c[0]}")
def test_random_fp8_heads(dev, case):
    """The per-head quantiser ([n_outer, n_batch, n_heads, run] -> one scale per (outer,
    head)) through both paths, and its dequant, at random shapes."""
    i, n_outer, B, H, run = case
    print(f"fp8 heads case {i}: {(n_outer, B, H, run)}", flush=True)
    g = torch.Generator().manual_seed(700 + i)
    x = (torch.randn((n_outer, B, H, run), generator=g) *
         torch.exp2(torch.randint(-8, 9, (n_outer, 1, H, 1), generator=g).float())).to(torch.bfloat16)
    wc, ws = O.fp8_quant_heads(bits16(x))
    for mode in ("single", "two"):
        codes, scales = kv.fp8_quant_heads(x.to(dev), two_pass=mode == "two", single_pass=mode == "single",
                                           check=True)
        np.testing.assert_array_equal(scales.cpu().numpy().view(np.uint32), ws.view(np.uint32))
        np.testing.assert_array_equal(codes.cpu().numpy(), wc)
    assert_bf16_equal(bits16(kv.fp8_dequant_heads(codes, scales)), O.fp8_dequant_heads(wc, ws))


_LEGACY_DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _legacy_cases(n, seed):
    rng = np.random.default_rng(seed)
    return [(i, str(rng.choice(list(_LEGACY_DT))), int(rng.integers(1, 9)), int(rng.integers(1, 5000)))
            for i in range(n)]


@pytest.mark.parametrize("case", _legacy_cases(10, 9), ids=lambda c: f"l{c[0]}")
def test_random_int8_legacy_slabs(dev, case):
    """precision.py:8-16 per slab (one launch for all slabs) at random slab counts and
    lengths (aligned and not), every dtype the reference accepts."""
    i, dt, n_slabs, n = case
    print(f"legacy int8 case {i}: {dt} {n_slabs} x {n}", flush=True)
    g = torch.Generator().manual_seed(900 + i)
    x = (torch.randn((n_slabs, n), generator=g) *
         torch.exp2(torch.randint(-10, 10, (n_slabs, 1), generator=g).float())).to(_LEGACY_DT[dt])
    q, sc = kv.int8_legacy_quant_slabs(x.to(dev))
    y = kv.int8_legacy_dequant_slabs(q, sc)
    for s in range(n_slabs):
        wq, ws = O.int8_legacy_quant(x[s].numpy() if dt == "f32" else bits16(x[s]), dt)
        np.testing.assert_array_equal(q[s].cpu().numpy(), wq)
        assert np.float32(sc[s].float().item()).tobytes() == np.float32(ws).tobytes()
        assert_bf16_equal(bits16(y[s]), O.int8_legacy_dequant(wq, ws))


def _ring_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        Hkv = int(rng.integers(1, 5))
        Hq = Hkv * int(rng.choice([1, 2, 4]))
        B = int(rng.integers(1, 4))
        lens = [int(v) for v in rng.integers(1, 700, B)]
        cases.append((i, Hq, Hkv, lens, int(rng.integers(1, 6)), bool(rng.integers(0, 2)), bool(rng.integers(0, 2))))
    return cases


@pytest.mark.parametrize("case", _ring_cases(8, 13), ids=lambda c: f"r{c[0]}")
def test_random_ring_attention(dev, case):
    """Ring attention over R key shards (one launch, or one launch per shard merged through
    the running output) equals attention over all keys, causal or not."""
    i, Hq, Hkv, lens, R, single, causal = case
    print(f"ring case {i}: Hq={Hq} Hkv={Hkv} lens={lens} R={R} single={single} causal={causal}", flush=True)
    q, pool, scales, bt, cu, qp = make(Hq, Hkv, 16, lens, [0] * len(lens), lens, seed=1100 + i)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    kv_len = np.asarray(lens, np.int32)
    out = kv.ring_attention_fp8(q.to(dev), t(cu), t(qp), t(pool), t(scales), t(bt), t(kv_len), ring_degree=R,
                                causal=causal, check=True, single_launch=single)
    torch.cuda.synchronize()
    zeros = np.zeros(len(lens), np.int32)
    want, _, err = O.paged_attention_prefill(bits16(q), cu, qp, pool, scales, bt, zeros, kv_len, causal,
                                             float(np.float32(1.0 / np.sqrt(128))))
    assert err == 0
    assert_precision(bits16(out), want, vmax_rows(pool, scales, bt, cu, zeros, kv_len, Hq), "f16")
