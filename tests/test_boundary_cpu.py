"""CPU-side checks of the drop-in boundary: the C-ABI library loads and exports every entry
point include/zenyx_kv.h declares, argument errors come back as status codes (no GPU
needed: validation precedes every HIP call), and the host-side logic (ring access
sequence, tiering sizes, reference timeline) matches the oracle and closed forms."""
import ctypes
import os
import re

import numpy as np
import pytest

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "zenyx_kv.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(zx_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    from zenyx_amd import _native

    lib = _native.load()
    syms = header_symbols()
    assert len(syms) >= 15
    for s in syms:
        assert hasattr(lib, s), f"libzenyx_kv.so does not export {s}"
        assert s in _native.SIGNATURES, f"{s} has no ctypes signature"
    assert lib.zx_abi_version() == _native.ABI_VERSION


def test_argument_errors_are_status_codes():
    from zenyx_amd import _native as N

    lib = N.load()
    rc = lib.zx_kv_gather_dequant(None, 10, 8, 128, 16, None, None, 4, None, 2, 64, None, None, None, None)
    assert rc == N.ZX_ERR_INVALID and b"null pointer" in lib.zx_last_error()
    rc = lib.zx_kv_gather_dequant(ctypes.c_void_p(16), 10, 8, 96, 16, ctypes.c_void_p(16), ctypes.c_void_p(16), 4,
                                  ctypes.c_void_p(16), 2, 64, ctypes.c_void_p(16), ctypes.c_void_p(16), None, None)
    assert rc == N.ZX_ERR_UNSUPPORTED and b"head_dim" in lib.zx_last_error()
    # bulk arrays off a 16-byte boundary are refused before any device call
    p16, p8 = ctypes.c_void_p(16), ctypes.c_void_p(24)
    rc = lib.zx_kv_gather_dequant(p8, 10, 8, 128, 16, p16, p16, 4, p16, 2, 64, p16, p16, None, None)
    assert rc == N.ZX_ERR_INVALID and b"16-byte aligned" in lib.zx_last_error()
    rc = lib.zx_kv_quant_append(p8, 16 * 2 * 8 * 128, 1, 16, 8, 128, p16, None, 1, p16, 1, 16, p16,
                                2 * 8 * 16 * 128, 1, p16, 0, None, p16, 1 << 20, None)
    assert rc == N.ZX_ERR_INVALID and b"16-byte aligned" in lib.zx_last_error()
    rc = lib.zx_int8_legacy_quant(ctypes.c_void_p(16), 0, 0, ctypes.c_void_p(16), ctypes.c_void_p(16),
                                  ctypes.c_void_p(16), 256, None)
    assert rc == N.ZX_ERR_INVALID and b"empty" in lib.zx_last_error()
    rc = lib.zx_belady_simulate(None, None, None, 10, 0, 10, 5, 0, ctypes.c_void_p(16), ctypes.c_void_p(16),
                                ctypes.c_void_p(16), None, None, 0, None, None, 0, None)
    assert rc == N.ZX_ERR_INVALID and b"capacity" in lib.zx_last_error()
    with pytest.raises(ValueError):
        N.check(N.ZX_ERR_INVALID, "x")
    with pytest.raises(N.ZenyxNativeError):
        N.check(N.ZX_ERR_HIP, "x")


def test_workspace_queries_are_host_only():
    from zenyx_amd import _native as N

    lib = N.load()
    assert lib.zx_kv_quant_append_workspace_bytes(32, 74902, 8, 128) >= 74902 * 8
    assert lib.zx_belady_simulate_workspace_bytes(20_971_520, 1_310_720) >= (20_971_520 + 1_310_720) // 8
    assert lib.zx_belady_argmax_workspace_bytes(1000) >= 16


@pytest.mark.parametrize("L,R,S", [(1, 1, 5), (3, 8, 4), (2, 4, 7)])
def test_ring_access_sequence_sizes(L, R, S):
    """The trace itself is built on the GPU (tests/test_gpu_dropin.py); here its sizes, and
    the oracle's trace against the closed form of ring step r, device d -> shard (d - r) mod R."""
    from zenyx_amd.train.belayd_kv_cache_tiering import RingAttentionAccessSequence

    seq = RingAttentionAccessSequence(L, R, S)
    tr = O.ring_trace(L, R, S)
    assert len(seq) == tr.size and seq.n_pages == L * R * S
    fwd = np.array([(l * R + (d - r) % R) * S + i for l in range(L) for r in range(R) for d in range(R)
                    for i in range(S)], np.int32)
    np.testing.assert_array_equal(tr, np.concatenate([fwd, fwd[::-1]]))


def test_tiering_manager_sizes_at_baseline_config():
    from zenyx_amd.train.belayd_kv_cache_tiering import BeladyKVCacheTieringManager

    m = BeladyKVCacheTieringManager(num_devices=8, context_length=2**20, num_layers=80, num_kv_heads=8,
                                    head_dim=128, page_tokens=64, hbm_budget_bytes=64e9)
    assert m.page_bytes == 128 * 1024
    assert m.pages_per_shard == 2048
    assert m.n_pages == 1_310_720
    assert m.capacity == 488_281
    assert len(m.sequence) == 20_971_520
    # the README constructor (README.md:93-97)
    r = BeladyKVCacheTieringManager(num_devices=8, context_length=4096, num_layers=12)
    assert r.capacity == r.n_pages == 12 * 8 * 8


def test_build_ring_timeline_matches_reference():
    from zenyx_amd.streaming import build_ring_timeline

    for n in (1, 2, 7):
        assert build_ring_timeline(n) == O.ref_ring_timeline(n)


def header_constants():
    """NAME -> value of every ZX_* constant the header defines (enum members and #defines)."""
    text = open(os.path.join(ROOT, "include", "zenyx_kv.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    consts = {}
    for name, val in re.findall(r"\b(ZX_[A-Z0-9_]+)\s*=\s*(-?\d+)", text):
        consts[name] = int(val)
    for name, val, sh in re.findall(r"#define\s+(ZX_[A-Z0-9_]+)\s+\(?(\d+)u?\s*(?:<<\s*(\d+))?", text):
        consts[name] = int(val) << int(sh or 0)
    return consts


def test_header_constants_match_the_python_binding():
    from zenyx_amd import _native as N

    consts = header_constants()
    for name in ("ZX_PREFILL_MERGE", "ZX_PREFILL_INIT", "ZX_PREFILL_BF16", "ZX_PREFILL_FAST_P", "ZX_PREFILL_EXACT_P",
                 "ZX_PREFILL_LAST", "ZX_PREFILL_FINAL",
                 "ZX_HEADS_TWO_PASS", "ZX_HEADS_SINGLE_PASS", "ZX_APPEND_STATIC_SCALES", "ZX_APPEND_SATURATE",
                 "ZX_APPEND_TWO_PASS", "ZX_KERR_PAGE_RANGE", "ZX_KERR_POS_RANGE", "ZX_KERR_SPIN", "ZX_KERR_OVERFLOW",
                 "ZX_ERR_INVALID", "ZX_ERR_UNSUPPORTED", "ZX_ERR_WORKSPACE"):
        assert name in consts, f"{name} not found in the header"
        assert getattr(N, name) == consts[name], f"{name}: header {consts[name]}, binding {getattr(N, name)}"


def test_exclusive_flags_are_refused_before_any_device_call():
    from zenyx_amd import _native as N

    lib = N.load()
    p = ctypes.c_void_p(16)
    rc = lib.zx_fp8_quant_heads(p, 1, 1, 1, 16, p, p, N.ZX_HEADS_TWO_PASS | N.ZX_HEADS_SINGLE_PASS, None, None, 0,
                                None)
    assert rc == N.ZX_ERR_INVALID and b"together" in lib.zx_last_error()
    rc = lib.zx_fp8_quant_heads(p, 1, 1, 1, 16, p, p, 64, None, None, 0, None)
    assert rc == N.ZX_ERR_INVALID and b"unknown flag" in lib.zx_last_error()
    for fl, msg in ((N.ZX_APPEND_TWO_PASS | N.ZX_APPEND_SINGLE_PASS, b"together"), (64, b"unknown flag")):
        rc = lib.zx_kv_quant_append(p, 16 * 2 * 8 * 128, 1, 16, 8, 128, p, None, 1, p, 1, 16, p, 2 * 8 * 16 * 128, 1,
                                    p, fl, None, None, 0, None)
        assert rc == N.ZX_ERR_INVALID and msg in lib.zx_last_error()
    for fn, extra in ((lib.zx_paged_attention_prefill, ()), (lib.zx_paged_attention_ring, (1,))):
        args = [p, 16, p, p, 8, p, 10, 2, 128, 16, p, p, 4] + [p, p] + list(extra) + [1, 16, 1, 0.1]
        rc = fn(*args, N.ZX_PREFILL_BF16 | N.ZX_PREFILL_FAST_P | N.ZX_PREFILL_EXACT_P, None, None, p, None, None)
        assert rc == N.ZX_ERR_INVALID and b"together" in lib.zx_last_error()
        rc = fn(*args, N.ZX_PREFILL_BF16 | N.ZX_PREFILL_LAST, None, None, p, None, None)
        assert rc == N.ZX_ERR_INVALID and b"ZX_PREFILL_LAST needs" in lib.zx_last_error()
        rc = fn(*args, N.ZX_PREFILL_BF16 | N.ZX_PREFILL_FINAL, None, None, p, None, None)
        assert rc == N.ZX_ERR_INVALID and b"ZX_PREFILL_FINAL needs" in lib.zx_last_error()
        rc = fn(*args, 128 | N.ZX_PREFILL_BF16, None, None, p, None, None)
        assert rc == N.ZX_ERR_INVALID and b"unknown flags" in lib.zx_last_error()
    # FINAL on a non-causal step
    args = [p, 16, p, p, 8, p, 10, 2, 128, 16, p, p, 4, p, p, 1, 16, 0, 0.1]
    rc = lib.zx_paged_attention_prefill(*args, N.ZX_PREFILL_MERGE | N.ZX_PREFILL_BF16 | N.ZX_PREFILL_FINAL, p, p, p,
                                        None, None)
    assert rc == N.ZX_ERR_INVALID and b"ZX_PREFILL_FINAL needs" in lib.zx_last_error()


def test_attention_precision_names():
    import torch

    from zenyx_amd import kv

    assert kv.PRECISIONS == ("f16", "bf16", "exact")
    t = torch.zeros(1)
    with pytest.raises(ValueError, match="precision"):
        kv.ring_attention_fp8(t, t, t, t, t, t, t, ring_degree=1, precision="fp8")
    with pytest.raises(ValueError, match="precision"):
        kv.paged_attention_prefill(t, t, t, t, t, t, t, t, precision="half")
