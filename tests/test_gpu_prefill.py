"""Blocks of queries over the FP8 pages (one ring step of QuantizedRingAttention,
README.md:344) and ring attention composed from such steps on one GPU, against the C
oracle (itself pinned against torch float64 in test_oracle.py).

Tolerance: the kernel computes scores in fp32 on matrix cores (bf16 q, K codes exact in
bf16) and an exp2-domain online softmax; how P enters P.V sets the bound per output
channel (the row sums use the same P, so a row is an average of V under weights
perturbed by at most e relative, which moves it by at most 2 e max|V|):
  "f16"   (default, P x 2^7 fp16): one bf16 ulp of the exact value + 2^-10 max|V| (e = 2^-11);
  "bf16"  (P rounded to bf16):     one ulp + 2^-7 max|V|  (e = 2^-8);
  "exact" (P as bf16 hi + lo):     e = 2^-16, a worst case of one ulp + 2^-15 max|V|; the
                                   rounding errors are independent and average out, and
                                   the tests hold this mode to one ulp + 2^-17 max|V|;
the oracle value, rounded to bf16, stands for the exact one: one more ulp for the modes
whose bound is not far below an ulp.  lse2 (log2 of the softmax denominator) within 2e-5
(absolute + relative), plus log2 of the weights' perturbation, e / ln 2, for "f16" and
"bf16" (the denominator is the sum of the same rounded weights, which keeps ring steps
merged by lse2 an average under those weights).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from zenyx_amd import kv
from test_gpu_attention import assert_within_bound, bf16_to_f32

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def bits16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def make(Hq, Hkv, P, n_q, q_pos0, kv_len, seed, n_pages=None):
    rng = np.random.default_rng(seed)
    D = 128
    B = len(n_q)
    max_blocks = max(1, -(-max(kv_len) // P))
    n_pages = n_pages or B * max_blocks + 3
    pool = rng.integers(0, 256, (n_pages, 2, Hkv, P, D), dtype=np.uint8)
    pool[(pool & 0x7F) == 0x7F] = 0x3A
    perm = rng.permutation(n_pages)
    bt = perm[:B * max_blocks].reshape(B, max_blocks).astype(np.int32)
    scales = rng.uniform(1e-3, 0.05, (2, Hkv)).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(n_q)]).astype(np.int32)
    q = torch.from_numpy(rng.standard_normal((int(cu[-1]), Hq, D)).astype(np.float32)).to(torch.bfloat16)
    return q, pool, scales, bt, cu, np.asarray(q_pos0, np.int32)


def vmax_rows(pool, scales, bt, cu, kv_begin, kv_end, Hq):
    """Per (row, query head, channel): max |V| over the sequence's key range (a bound
    for the keys the row actually uses)."""
    dec = np.abs(O.e4m3_decode(np.arange(256, dtype=np.uint8)).astype(np.float64))
    n_pages, _, Hkv, P, D = pool.shape
    out = np.zeros((int(cu[-1]), Hq, D))
    for b in range(len(cu) - 1):
        t = np.arange(kv_begin[b], kv_end[b])
        if t.size == 0:
            continue
        pages = bt[b, t // P]
        for hq in range(Hq):
            h = hq // (Hq // Hkv)
            out[cu[b]:cu[b + 1], hq] = np.nanmax(dec[pool[pages, 1, h, t % P, :]], axis=0) * abs(float(scales[1, h]))
    return out


P_BOUND = {"exact": (1, 2.0 ** -17), "f16": (2, 2.0 ** -10), "bf16": (2, 2.0 ** -7)}  # (ulps, bound on |V|)
LSE_EXTRA = {"exact": 0.0, "f16": 2.0 ** -11 / np.log(2.0), "bf16": 2.0 ** -8 / np.log(2.0)}


def assert_precision(got_bits, want_bits, vmax, precision="f16"):
    ulps, e = P_BOUND[precision]
    return assert_within_bound(got_bits, want_bits, vmax, e, ulps)


def run_step(q, pool, scales, bt, cu, q_pos0, kb, ke, causal, precision="f16"):
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    o_acc = torch.empty(q.shape, dtype=torch.float32, device=DEV)
    lse = torch.empty(q.shape[:2], dtype=torch.float32, device=DEV)
    out = kv.paged_attention_prefill(q.to(DEV), t(cu), t(q_pos0), t(pool), t(scales), t(bt), t(kb), t(ke),
                                     causal=causal, o_acc=o_acc, lse2=lse, first=True, check=True,
                                     precision=precision)
    return out, lse


CASES = [  # Hq, Hkv, P, n_q, q_pos0, kv_begin, kv_end
    (8, 2, 16, [37, 5, 64], [0, 20, 100], [0, 3, 17], [37, 25, 164]),
    (32, 8, 16, [130, 1], [500, 0], [0, 0], [630, 1]),
    (4, 4, 32, [70, 33], [0, 64], [5, 70], [70, 70]),       # second: empty key range
    (6, 3, 16, [20, 0, 45], [10, 0, 5], [0, 0, 0], [30, 0, 50]),  # a sequence with no queries
    (2, 1, 48, [129], [300], [40], [429]),
]


@pytest.mark.parametrize("precision", ["f16", "exact", "bf16"])
@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_step_matches_oracle(case, causal, precision):
    Hq, Hkv, P, n_q, q_pos0, kb, ke = CASES[case]
    print(f"prefill step case {case} causal={causal} precision={precision}", flush=True)
    q, pool, scales, bt, cu, qp = make(Hq, Hkv, P, n_q, q_pos0, ke, seed=case)
    kb, ke = np.asarray(kb, np.int32), np.asarray(ke, np.int32)
    out, lse = run_step(q, pool, scales, bt, cu, qp, kb, ke, causal, precision)
    torch.cuda.synchronize()
    sm = float(np.float32(1.0 / np.sqrt(128)))
    want, wlse, err = O.paged_attention_prefill(bits16(q), cu, qp, pool, scales, bt, kb, ke, causal, sm)
    assert err == 0
    assert_precision(bits16(out), want, vmax_rows(pool, scales, bt, cu, kb, ke, Hq), precision)
    g = lse.cpu().numpy()
    fin = np.isfinite(wlse)
    np.testing.assert_array_equal(np.isfinite(g), fin)
    assert np.all(np.abs(g[fin] - wlse[fin]) <= 2e-5 * (1 + np.abs(wlse[fin])) + LSE_EXTRA[precision])


_RING_CASE = {}


def _ring_case():
    """One set of inputs and its oracle result, shared by the ring degrees."""
    if not _RING_CASE:
        Hq, Hkv, P = 32, 8, 16
        n_q, lens, q_pos0 = [256, 77, 512], [256, 300, 1024], [0, 223, 512]  # queries end at the last key
        q, pool, scales, bt, cu, qp = make(Hq, Hkv, P, n_q, q_pos0, lens, seed=41)
        zeros, lens_a = np.zeros(len(lens), np.int32), np.asarray(lens, np.int32)
        sm = float(np.float32(1.0 / np.sqrt(128)))
        want, _, err = O.paged_attention_prefill(bits16(q), cu, qp, pool, scales, bt, zeros, lens_a, True, sm)
        assert err == 0
        _RING_CASE.update(q=q, pool=pool, scales=scales, bt=bt, cu=cu, qp=qp, lens=lens_a, want=want,
                          vmax=vmax_rows(pool, scales, bt, cu, zeros, lens_a, Hq))
    return _RING_CASE


@pytest.mark.parametrize("precision", ["f16", "exact"])
@pytest.mark.parametrize("single_launch", [True, False])
@pytest.mark.parametrize("ring", [1, 3, 8, 70])  # 70: more ranges than a block keeps in LDS
def test_ring_attention_equals_full_attention(ring, single_launch, precision):
    c = _ring_case()
    print(f"ring {ring} single_launch={single_launch} precision={precision}", flush=True)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    out = kv.ring_attention_fp8(c["q"].to(DEV), t(c["cu"]), t(c["qp"]), t(c["pool"]), t(c["scales"]), t(c["bt"]),
                                t(c["lens"]), ring_degree=ring, causal=True, check=True, single_launch=single_launch,
                                precision=precision)
    torch.cuda.synchronize()
    worst = assert_precision(bits16(out), c["want"], c["vmax"], precision)
    print(f"  worst |err| / max|V| = {worst:.3g}", flush=True)


@pytest.mark.parametrize("precision", ["f16", "exact"])
def test_last_step_leaves_the_running_output(precision):
    """ZX_PREFILL_LAST: the last step of a ring writes the same bf16 rows as a merging
    step and leaves o_acc / lse2 as they were."""
    c = _ring_case()
    print(f"last step precision={precision}", flush=True)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    q, cu, qp, pool, scales, bt = c["q"].to(DEV), t(c["cu"]), t(c["qp"]), t(c["pool"]), t(c["scales"]), t(c["bt"])
    lens = c["lens"].astype(np.int64)
    R = 3
    bounds = [t((lens * r // R).astype(np.int32)) for r in range(R + 1)]
    o_acc = torch.empty(q.shape, dtype=torch.float32, device=DEV)
    lse2 = torch.empty(q.shape[:2], dtype=torch.float32, device=DEV)
    for r in range(R - 1):
        kv.paged_attention_prefill(q, cu, qp, pool, scales, bt, bounds[r], bounds[r + 1], o_acc=o_acc, lse2=lse2,
                                   first=r == 0, write_bf16=False, check=True, precision=precision)
    o_keep, l_keep = o_acc.clone(), lse2.clone()
    out_last = kv.paged_attention_prefill(q, cu, qp, pool, scales, bt, bounds[R - 1], bounds[R], o_acc=o_acc,
                                          lse2=lse2, first=False, check=True, precision=precision, last=True)
    torch.cuda.synchronize()
    assert torch.equal(o_acc.view(torch.int32), o_keep.view(torch.int32))
    assert torch.equal(lse2.view(torch.int32), l_keep.view(torch.int32))
    out_merge = kv.paged_attention_prefill(q, cu, qp, pool, scales, bt, bounds[R - 1], bounds[R], o_acc=o_acc,
                                           lse2=lse2, first=False, check=True, precision=precision)
    torch.cuda.synchronize()
    assert torch.equal(out_last.view(torch.int16), out_merge.view(torch.int16))
    assert not torch.equal(o_acc.view(torch.int32), o_keep.view(torch.int32))  # the merging step did write
    assert_precision(bits16(out_last), c["want"], c["vmax"], precision)
    with pytest.raises(ValueError):
        kv.paged_attention_prefill(q, cu, qp, pool, scales, bt, bounds[0], bounds[1], last=True)


def _steps(q, cu, qp, pool, scales, bt, lens, R, final, precision="f16"):
    """A causal ring of R launches over keys [0, lens) in ascending contiguous shards; out
    starts as a NaN pattern so that a row no step writes shows."""
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    lens = np.asarray(lens, np.int64)
    bounds = [t((lens * r // R).astype(np.int32)) for r in range(R + 1)]
    o_acc = torch.empty(q.shape, dtype=torch.float32, device=DEV)
    lse2 = torch.empty(q.shape[:2], dtype=torch.float32, device=DEV)
    out = torch.full(q.shape, 0x7FC1, dtype=torch.int16, device=DEV).view(torch.bfloat16)
    for r in range(R):
        kv.paged_attention_prefill(q, cu, qp, pool, scales, bt, bounds[r], bounds[r + 1], o_acc=o_acc, lse2=lse2,
                                   first=r == 0, out=out, write_bf16=final or r == R - 1, check=True,
                                   precision=precision, last=r == R - 1, final=final)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("shape", ["ragged", "queries_past_keys", "empty_shards"])
@pytest.mark.parametrize("R", [3, 8])
def test_final_steps_equal_the_merged_ring(shape, R):
    """ZX_PREFILL_FINAL: every step writes as bf16 the rows it completes and the last one
    converts only the rows it reaches; the output equals, bit for bit, the ring that merges
    every row into the running output and converts them all in the last step (the same
    fp32 value goes to bf16 either way), every row is written (none keeps the NaN pattern
    the output starts with), and it is within the default bound of the oracle."""
    if shape == "ragged":
        c = _ring_case()
        q, pool, scales, bt, cu, qp, lens = c["q"], c["pool"], c["scales"], c["bt"], c["cu"], c["qp"], c["lens"]
        Hq, want, vmax = 32, c["want"], c["vmax"]
    else:
        Hq, Hkv, P = 8, 2, 16
        if shape == "queries_past_keys":  # rows at positions past the last key see every key
            n_q, q_pos0, lens = [40, 70, 5], [10, 0, 30], [30, 50, 33]
        else:  # most shards empty, a sequence's only key in the last shard
            n_q, q_pos0, lens = [3, 4, 20], [0, 0, 0], [3, 1, 20]
        q, pool, scales, bt, cu, qp = make(Hq, Hkv, P, n_q, q_pos0, lens, seed=23)
        lens = np.asarray(lens, np.int32)
        zeros = np.zeros(len(lens), np.int32)
        sm = float(np.float32(1.0 / np.sqrt(128)))
        want, _, err = O.paged_attention_prefill(bits16(q), cu, qp, pool, scales, bt, zeros, lens, True, sm)
        assert err == 0
        vmax = vmax_rows(pool, scales, bt, cu, zeros, lens, Hq)
    print(f"final steps: {shape}, R={R}", flush=True)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    args = (q.to(DEV), t(cu), t(qp), t(pool), t(scales), t(bt), lens, R)
    got = _steps(*args, final=True)
    ref = _steps(*args, final=False)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert not torch.isnan(got.float()).any()
    assert_precision(bits16(got), want, vmax)
    with pytest.raises(ValueError):
        kv.paged_attention_prefill(q.to(DEV), t(cu), t(qp), t(pool), t(scales), t(bt), t(np.zeros(len(lens), np.int32)),
                                   t(np.asarray(lens, np.int32)), causal=False, o_acc=torch.empty(q.shape,
                                   dtype=torch.float32, device=DEV), lse2=torch.empty(q.shape[:2],
                                   dtype=torch.float32, device=DEV), final=True)


def test_final_first_step_writes_every_row():
    """ZX_PREFILL_FINAL on a first step (INIT) whose key range starts past some rows: no
    earlier step finished those rows, so they are written too (no key: zeros), and the
    one-step ring (INIT | LAST | FINAL) equals a plain merging step bit for bit and the
    oracle within the default bound."""
    Hq, Hkv, P = 8, 2, 16
    n_q, q_pos0, kb, ke = [40, 70], [0, 0], [10, 30], [50, 60]
    q, pool, scales, bt, cu, qp = make(Hq, Hkv, P, n_q, q_pos0, ke, seed=29)
    kb, ke = np.asarray(kb, np.int32), np.asarray(ke, np.int32)
    sm = float(np.float32(1.0 / np.sqrt(128)))
    want, _, err = O.paged_attention_prefill(bits16(q), cu, qp, pool, scales, bt, kb, ke, True, sm)
    assert err == 0
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    outs = []
    for final in (True, False):
        o_acc = torch.empty(q.shape, dtype=torch.float32, device=DEV)
        lse2 = torch.empty(q.shape[:2], dtype=torch.float32, device=DEV)
        out = torch.full(q.shape, 0x7FC1, dtype=torch.int16, device=DEV).view(torch.bfloat16)
        kv.paged_attention_prefill(q.to(DEV), t(cu), t(qp), t(pool), t(scales), t(bt), t(kb), t(ke), o_acc=o_acc,
                                   lse2=lse2, first=True, out=out, check=True, last=final, final=final)
        torch.cuda.synchronize()
        outs.append(out)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert not torch.isnan(outs[0].float()).any()
    assert_precision(bits16(outs[0]), want, vmax_rows(pool, scales, bt, cu, kb, ke, Hq))


@pytest.mark.parametrize("ring,single", [(1, True), (8, True), (3, False)])
def test_ring_attention_bf16_p(ring, single):
    """P rounded once to bf16 for P.V (ZX_PREFILL_FAST_P): within its bound of the oracle
    (one ulp + 2^-7 max|V|)."""
    c = _ring_case()
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    out = kv.ring_attention_fp8(c["q"].to(DEV), t(c["cu"]), t(c["qp"]), t(c["pool"]), t(c["scales"]), t(c["bt"]),
                                t(c["lens"]), ring_degree=ring, causal=True, check=True, single_launch=single,
                                precision="bf16")
    torch.cuda.synchronize()
    worst = assert_precision(bits16(out), c["want"], c["vmax"], "bf16")
    print(f"ring {ring} bf16 P: worst |err| / max|V| = {worst:.3g}", flush=True)


def test_f16_p_keeps_small_weights():
    """The fp16 mode on rows where one key outweighs each of the ~200 others by 2^15.5 (q all
    ones, K all ones but key 7 = 20: scores 15.5 log2 units apart): the small weights sum to
    ~2^-8 of the row and lie below fp16's normal range unless P carries its 2^7 factor, so
    losing them would miss the 2^-10 max|V| bound; within it, as the exact mode is within
    its own."""
    Hq, Hkv, P = 4, 1, 16
    _, pool, scales, bt, cu, qp = make(Hq, Hkv, P, [64], [191], [256], seed=23)
    q = torch.ones((64, Hq, 128), dtype=torch.bfloat16)
    pool[:, 0] = 0x38  # K = 1.0 (e4m3) everywhere ...
    pool[bt[0, 7 // P], 0, 0, 7 % P, :] = 0x5A  # ... but key 7 = 20.0
    scales[0, 0] = 0.05
    kb, ke = np.zeros(1, np.int32), np.full(1, 256, np.int32)
    sm = float(np.float32(1.0 / np.sqrt(128)))
    want, _, err = O.paged_attention_prefill(bits16(q), cu, qp, pool, scales, bt, kb, ke, True, sm)
    assert err == 0
    vm = vmax_rows(pool, scales, bt, cu, kb, ke, Hq)
    for precision in ("f16", "exact"):
        out, _ = run_step(q, pool, scales, bt, cu, qp, kb, ke, True, precision)
        torch.cuda.synchronize()
        worst = assert_precision(bits16(out), want, vm, precision)
        print(f"{precision}: worst |err| / max|V| = {worst:.3g}", flush=True)


@pytest.mark.parametrize("causal", [True, False])
def test_ring_ranges_in_device_order(causal):
    """zx_paged_attention_ring with the shards in the order one device of a ring of 5 sees
    them (its own shard first, then (g - r) mod 5), uneven shards, an empty shard and a
    range that starts mid-page: equal to attention over the union."""
    c = _ring_case()
    lens = c["lens"]
    R, g = 5, 3
    cuts = np.stack([np.array([0, 1, 2, 2, 4, 5]) * L // 5 for L in lens], axis=1)  # shard 2 empty
    cuts[1] = np.minimum(cuts[1] + 7, cuts[2])  # uneven: shard 0 longer, starting mid-page for shard 1
    order = [(g - r) % R for r in range(R)]
    kb = np.stack([cuts[s] for s in order]).astype(np.int32)
    ke = np.stack([cuts[s + 1] for s in order]).astype(np.int32)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    out = kv.paged_attention_ring(c["q"].to(DEV), t(c["cu"]), t(c["qp"]), t(c["pool"]), t(c["scales"]), t(c["bt"]),
                                  t(kb), t(ke), causal=causal, check=True)
    torch.cuda.synchronize()
    if causal:
        want, vmax = c["want"], c["vmax"]
    else:
        zeros = np.zeros(len(lens), np.int32)
        sm = float(np.float32(1.0 / np.sqrt(128)))
        want, _, err = O.paged_attention_prefill(bits16(c["q"]), c["cu"], c["qp"], c["pool"], c["scales"], c["bt"],
                                                 zeros, lens, False, sm)
        assert err == 0
        vmax = c["vmax"]
    assert_precision(bits16(out), want, vmax)


@pytest.mark.parametrize("precision", ["f16", "exact"])
def test_negative_scales(precision):
    """Scales of either sign (a static scale may be negative): with K's scale negative the
    scores change sign and every step takes the masked softmax path (the maximum of
    s * scale is no longer the scale times the maximum of s); V heads with a negative scale
    flip their output.  A step, causal and not, and ring attention over 3 shards in one
    launch and in separate launches."""
    Hq, Hkv, P = 8, 4, 16
    n_q, q_pos0, lens = [70, 33], [30, 0], [100, 140]
    print(f"negative scales precision={precision}", flush=True)
    q, pool, scales, bt, cu, qp = make(Hq, Hkv, P, n_q, q_pos0, lens, seed=37)
    scales[0, 0::2] *= -1.0
    scales[1, 1::2] *= -1.0
    kb, ke = np.zeros(2, np.int32), np.asarray(lens, np.int32)
    sm = float(np.float32(1.0 / np.sqrt(128)))
    vm = vmax_rows(pool, scales, bt, cu, kb, ke, Hq)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    for causal in (True, False):
        want, wlse, err = O.paged_attention_prefill(bits16(q), cu, qp, pool, scales, bt, kb, ke, causal, sm)
        assert err == 0
        out, lse = run_step(q, pool, scales, bt, cu, qp, kb, ke, causal, precision)
        torch.cuda.synchronize()
        assert_precision(bits16(out), want, vm, precision)
        g = lse.cpu().numpy()
        fin = np.isfinite(wlse)
        np.testing.assert_array_equal(np.isfinite(g), fin)
        assert np.all(np.abs(g[fin] - wlse[fin]) <= 2e-5 * (1 + np.abs(wlse[fin])) + LSE_EXTRA[precision])
        for single in (False, True):
            ring = kv.ring_attention_fp8(q.to(DEV), t(cu), t(qp), t(pool), t(scales), t(bt), t(ke), ring_degree=3,
                                         causal=causal, check=True, single_launch=single, precision=precision)
            torch.cuda.synchronize()
            assert_precision(bits16(ring), want, vm, precision)


def assert_nan_leak_only_in_window(got_bits, want_bits, vmax, precision, leak):
    """got equals want to the precision bound, NaN compared as a class, except that got may
    be NaN where want is not inside the boolean mask ``leak``."""
    g, w = bf16_to_f32(got_bits), bf16_to_f32(want_bits)
    extra = np.isnan(g) & ~np.isnan(w)
    assert not (extra & ~leak).any(), f"{(extra & ~leak).sum()} NaN outside the leak window"
    assert not (np.isnan(w) & ~np.isnan(g)).any(), "a NaN of the oracle is missing"
    keep = ~extra
    assert_precision(got_bits[keep], want_bits[keep], vmax[keep], precision)
    return int(extra.sum())


@pytest.mark.parametrize("precision", ["f16", "exact", "bf16"])
def test_nan_codes_propagate_like_the_oracle(precision):
    """NaN codes (e4m3 0x7F / 0xFF) in the pages.  A NaN K element makes every score of its
    key NaN: each row that sees the key is NaN in every channel, with lse2 -inf (the
    oracle's softmax denominator is NaN), and no other row changes (a masked score never
    reaches P).  A NaN V element makes its own channel NaN in the rows that see it; since
    the P.V product of a 64-key step multiplies the weight 0 of a key a row does not see
    by that key's V, rows before the key whose step holds it may also be NaN in that
    channel (as in tiled attention generally; the oracle skips such keys), and nothing
    else.  Checked for one step, and for ring attention over 3 shards in one launch and in
    separate launches merged through o_acc / lse2, where a NaN of the first step has to
    survive the later merges, which give it weight 0."""
    Hq, Hkv, P = 8, 2, 16
    n_q, q_pos0, lens = [48, 40], [0, 24], [48, 64]
    print(f"nan codes precision={precision}", flush=True)
    q, pool, scales, bt, cu, qp = make(Hq, Hkv, P, n_q, q_pos0, lens, seed=31)
    pool[bt[0, 5 // P], 0, 0, 5 % P, 77] = 0x7F  # K of sequence 0, key 5, KV head 0, channel 77
    pool[bt[1, 30 // P], 1, 1, 30 % P, 17] = 0xFF  # V of sequence 1, key 30, KV head 1, channel 17
    kb, ke = np.zeros(2, np.int32), np.asarray(lens, np.int32)
    sm = float(np.float32(1.0 / np.sqrt(128)))
    want, wlse, err = O.paged_attention_prefill(bits16(q), cu, qp, pool, scales, bt, kb, ke, True, sm)
    assert err == 0
    w = bf16_to_f32(want)
    # the planted codes reach exactly the rows and channels described (causal: sequence 0's
    # rows from position 5 on, query heads 0-3; sequence 1's rows from position 30 on,
    # query heads 4-7, channel 17)
    assert np.isnan(w[5:48, 0:4]).all() and not np.isnan(w[0:5]).any()
    assert np.isnan(w[48 + 6:, 4:8, 17]).all() and not np.isnan(w[48:48 + 6]).any()
    assert np.isnan(w).sum() == 43 * 4 * 128 + 34 * 4
    assert np.isneginf(wlse[5:48, 0:4]).all()
    # where the NaN V may also show: sequence 1 (positions 24 + i), heads 4-7, channel 17,
    # rows less than 64 positions before key 30
    leak = np.zeros(w.shape, bool)
    leak[48:48 + 6, 4:8, 17] = True
    vm = vmax_rows(pool, scales, bt, cu, kb, ke, Hq)
    out, lse = run_step(q, pool, scales, bt, cu, qp, kb, ke, True, precision)
    torch.cuda.synchronize()
    n = assert_nan_leak_only_in_window(bits16(out), want, vm, precision, leak)
    g = lse.cpu().numpy()
    np.testing.assert_array_equal(np.isfinite(g), np.isfinite(wlse))
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    for single in (False, True):
        ring = kv.ring_attention_fp8(q.to(DEV), t(cu), t(qp), t(pool), t(scales), t(bt), t(ke), ring_degree=3,
                                     causal=True, check=True, single_launch=single, precision=precision)
        torch.cuda.synchronize()
        n_ring = assert_nan_leak_only_in_window(bits16(ring), want, vm, precision, leak)
        print(f"  ring 3 single_launch={single}: {n_ring} NaN in the window (step: {n})", flush=True)


def test_prefill_flags_bad_pages():
    Hq, Hkv, P = 8, 2, 16
    q, pool, scales, bt, cu, qp = make(Hq, Hkv, P, [40], [0], [64], seed=9, n_pages=8)
    bt = bt.copy()
    bt[0, 1] = 1000  # keys 16..31 on a page outside the pool
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    kb, ke = np.zeros(1, np.int32), np.full(1, 64, np.int32)
    with pytest.raises(ValueError, match="block table"):
        kv.paged_attention_prefill(q.to(DEV), t(cu), t(qp), t(pool), t(scales), t(bt), t(kb), t(ke), causal=False,
                                   check=True)
    out = kv.paged_attention_prefill(q.to(DEV), t(cu), t(qp), t(pool), t(scales), t(bt), t(kb), t(ke), causal=False)
    torch.cuda.synchronize()
    sm = float(np.float32(1.0 / np.sqrt(128)))
    want, _, err = O.paged_attention_prefill(bits16(q), cu, qp, pool, scales, bt, kb, ke, False, sm)
    assert err & 1
    assert_precision(bits16(out), want, vmax_rows(pool, scales, np.where(bt < 8, bt, 0), cu, kb, ke, Hq))


def test_prefill_kv_end_past_table_is_clipped_and_flagged():
    """kv_end beyond max_blocks * page_size: the kernel clips the key range to the table
    (as the oracle does), flags ZX_KERR_POS_RANGE, and check=True raises."""
    Hq, Hkv, P = 8, 2, 16
    q, pool, scales, bt, cu, qp = make(Hq, Hkv, P, [40], [24], [64], seed=11)  # table holds 64 keys
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    kb, ke = np.zeros(1, np.int32), np.full(1, 80, np.int32)
    with pytest.raises(ValueError, match="max_blocks"):
        kv.paged_attention_prefill(q.to(DEV), t(cu), t(qp), t(pool), t(scales), t(bt), t(kb), t(ke), causal=True,
                                   check=True)
    out = kv.paged_attention_prefill(q.to(DEV), t(cu), t(qp), t(pool), t(scales), t(bt), t(kb), t(ke), causal=True)
    torch.cuda.synchronize()
    sm = float(np.float32(1.0 / np.sqrt(128)))
    want, _, err = O.paged_attention_prefill(bits16(q), cu, qp, pool, scales, bt, kb, ke, True, sm)
    assert err & 2
    assert_precision(bits16(out), want, vmax_rows(pool, scales, bt, cu, kb, np.full(1, 64, np.int32), Hq))


def test_prefill_rejects_bad_scales():
    Hq, Hkv, P = 8, 2, 16
    q, pool, scales, bt, cu, qp = make(Hq, Hkv, P, [16], [0], [16], seed=12)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    kb, ke = np.zeros(1, np.int32), np.full(1, 16, np.int32)
    with pytest.raises(ValueError, match="scales_layer"):
        kv.paged_attention_prefill(q.to(DEV), t(cu), t(qp), t(pool), t(scales[:, :1]), t(bt), t(kb), t(ke))
    with pytest.raises(ValueError, match="scales_layer"):
        kv.paged_attention_prefill(q.to(DEV), t(cu), t(qp), t(pool), t(scales.astype(np.float64)), t(bt), t(kb),
                                   t(ke))


def test_prefill_flags_rows_beyond_max_q_per_seq():
    """A max_q_per_seq below a sequence's query count leaves the extra rows unwritten and is
    flagged (ZX_KERR_POS_RANGE); the covered rows are still right."""
    Hq, Hkv, P = 8, 2, 16
    q, pool, scales, bt, cu, qp = make(Hq, Hkv, P, [200], [0], [200], seed=13)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    kb, ke = np.zeros(1, np.int32), np.full(1, 200, np.int32)
    with pytest.raises(ValueError, match="max_q_per_seq"):
        kv.paged_attention_prefill(q.to(DEV), t(cu), t(qp), t(pool), t(scales), t(bt), t(kb), t(ke),
                                   max_q_per_seq=64, check=True)
    out = kv.paged_attention_prefill(q.to(DEV), t(cu), t(qp), t(pool), t(scales), t(bt), t(kb), t(ke),
                                     max_q_per_seq=64)
    torch.cuda.synchronize()
    sm = float(np.float32(1.0 / np.sqrt(128)))
    want, _, err = O.paged_attention_prefill(bits16(q), cu, qp, pool, scales, bt, kb, ke, True, sm)
    assert err == 0
    covered = 64  # query tiles of 32 * 4 / G = 32 rows (G = 4 here): ceil(64 / 32) = 2 tiles cover rows 0..63
    assert_precision(bits16(out)[:covered], want[:covered], vmax_rows(pool, scales, bt, cu, kb, ke, Hq)[:covered])


def test_ring_degree_above_sequence_lengths():
    """Ring degree 8 over sequences of 3, 1 and 20 keys: most shards are empty (the first
    one too, which must still initialise the running output), the result is still full
    causal attention."""
    Hq, Hkv, P = 8, 2, 16
    lens = [3, 1, 20]
    q, pool, scales, bt, cu, qp = make(Hq, Hkv, P, lens, [0, 0, 0], lens, seed=17)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    kl = np.asarray(lens, np.int32)
    sm = float(np.float32(1.0 / np.sqrt(128)))
    zeros = np.zeros(3, np.int32)
    want, _, err = O.paged_attention_prefill(bits16(q), cu, qp, pool, scales, bt, zeros, kl, True, sm)
    assert err == 0
    for single in (True, False):
        out = kv.ring_attention_fp8(q.to(DEV), t(cu), t(qp), t(pool), t(scales), t(bt), t(kl), ring_degree=8,
                                    causal=True, check=True, single_launch=single)
        torch.cuda.synchronize()
        assert_precision(bits16(out), want, vmax_rows(pool, scales, bt, cu, zeros, kl, Hq))
