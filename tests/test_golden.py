"""The oracle and the host-side drop-ins against the committed fixtures of tests/golden/
(the reference's own known answers, and configs[0] / a ragged paged case as written by
tests/golden/make_golden.py)."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._golden_io import f32_from_hex, fixture, generator
from zenyx_amd.streaming import BandwidthAwareScheduler, BandwidthSample

KATS = fixture("reference_kats.json")


def test_reference_belady_kat_on_oracle_restatement():
    k = KATS["belady_farthest_next_use"]
    cache = O.RefBeladyApproxCache(capacity=k["capacity"])
    for key, nxt in k["update_future"]:
        cache.update_future(key, nxt)
    for key in k["touch"]:
        assert cache.touch(key) == []
    assert cache.touch(k["last_touch"]) == k["evicted"]


@pytest.mark.parametrize("case", KATS["bandwidth_throttle"]["cases"])
def test_reference_bandwidth_kat(case):
    sched = BandwidthAwareScheduler(max_fetch_to_compute_ratio=KATS["bandwidth_throttle"]["max_fetch_to_compute_ratio"])
    s = BandwidthSample(fetch_time_ms=case["fetch_time_ms"], compute_time_ms=case["compute_time_ms"])
    assert sched.should_throttle(s) is case["throttle"]
    want = case["fetch_time_ms"] - case["compute_time_ms"] if case["throttle"] else 0.0
    assert sched.throttle_ms(s) == want


def test_bandwidth_rule_edges():
    sched = BandwidthAwareScheduler(2.0)
    assert sched.should_throttle(BandwidthSample(0.0, 0.0))            # no compute time: always
    assert sched.throttle_ms(BandwidthSample(0.5, -1.0)) == 1.5
    assert not sched.should_throttle(BandwidthSample(2.0, 1.0))        # ratio 2 is not above 2
    assert sched.throttle_ms(BandwidthSample(3.0, 1.0)) == 2.0


def test_e4m3_boundary_fixture():
    for v, code in KATS["e4m3fn_boundaries"]["cases"]:
        x = np.array([float(v)], np.float32)
        assert int(O.e4m3_encode(x)[0]) == code, v


def test_configs0_fixture_closed_form_scales():
    """The fixture's FP8 scales are max(amax, 1e-8) / 448 of each (layer, kv, head) slab of the
    seeded input, and its int8 scales amax / 127 rounded to bf16 (precision.py:9-10)."""
    import torch

    fx = fixture("configs0.json")
    xb = generator().configs0_input()
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).float().reshape(288, -1)
    amax = x.abs().amax(dim=1)
    want8 = (amax.clamp_min(1e-8) / 448.0).numpy()
    np.testing.assert_array_equal(f32_from_hex(fx["fp8_scales_f32"]), want8)
    want_i8 = (amax.to(torch.bfloat16) / 127.0).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(f32_from_hex(fx["int8_scales_bf16_as_f32"]), want_i8)


def test_configs0_oracle_matches_fixture():
    assert generator().configs0_expected(O) == fixture("configs0.json")


def test_paged_small_oracle_matches_fixture():
    assert generator().paged_small_expected(O) == fixture("paged_small.json")


def test_paged_small_fixture_by_indexing():
    """Brute force on the fixture itself: every token's codes sit at page
    block_tables[b, pos // P], slot pos % P, and every gathered value is code * scale."""
    fx = fixture("paged_small.json")
    H, D, P, n_pages = fx["H"], fx["D"], fx["page_size"], fx["n_pages"]
    pool = np.array(fx["pool"], np.uint8).reshape(n_pages, 2, H, P, D)
    sc = f32_from_hex(fx["scales_f32"]).reshape(2, H)
    x = np.array(fx["x_bf16_bits"], np.uint16).reshape(fx["x_shape"])[0]
    bt = np.array(fx["block_tables"]).reshape(2, -1)
    cu, out_len = fx["cu_seqlens"], fx["out_len"]
    k = np.array(fx["k_bf16_bits"], np.uint16).reshape(2, H, out_len, D)
    v = np.array(fx["v_bf16_bits"], np.uint16).reshape(2, H, out_len, D)
    xf = O.bf16_to_f32(x)
    np.testing.assert_array_equal(sc, np.maximum(np.abs(xf).max(axis=(0, 3)), np.float32(1e-8)) / np.float32(448))
    used = np.zeros(n_pages, bool)
    for b in range(2):
        for pos in range(cu[b + 1] - cu[b]):
            page = bt[b, pos // P]
            used[page] = True
            codes = pool[page, :, :, pos % P, :]
            np.testing.assert_array_equal(codes, O.e4m3_encode(xf[cu[b] + pos] / sc[:, :, None]))
            vals = O.bf16_rne(O.e4m3_decode(codes) * sc[:, :, None])
            np.testing.assert_array_equal(k[b, :, pos], vals[0])
            np.testing.assert_array_equal(v[b, :, pos], vals[1])
        assert not k[b, :, cu[b + 1] - cu[b]:].any() and not v[b, :, cu[b + 1] - cu[b]:].any()
    assert not pool[~used].any()
