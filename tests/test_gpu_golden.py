"""The HIP kernels against the committed fixtures of tests/golden/: configs[0] through the
per-head FP8 and legacy int8 kernels (digests of all 75.5 M codes and dequantised values,
all 288 scales of each scheme), the ragged paged append + gather value for value, and the
reference's own known answers through the drop-in classes."""
import hashlib

import numpy as np
import pytest
import torch

from tests._golden_io import f32_from_hex, fixture, generator
from zenyx_amd import kv
from zenyx_amd.streaming import BeladyApproxCache, dequantize_for_bf16_compute, quantize_to_fp8_storage

pytestmark = pytest.mark.gpu


def sha(t: torch.Tensor) -> str:
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16, torch.int8):
        t = t.view(torch.uint8)
    return hashlib.sha256(t.numpy().tobytes()).hexdigest()


def f32_hex(t: torch.Tensor) -> list[str]:
    return [f"{int(b):08x}" for b in t.detach().float().cpu().numpy().reshape(-1).view(np.uint32)]


@pytest.fixture(scope="module")
def configs0(dev):
    fx = fixture("configs0.json")
    xb = generator().configs0_input()
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16)
    assert hashlib.sha256(xb.tobytes()).hexdigest() == fx["input_sha256"]
    return fx, x.to(dev)


def test_configs0_fp8_heads(configs0):
    fx, x = configs0
    codes, scales = kv.fp8_quant_heads(x)
    assert f32_hex(scales) == fx["fp8_scales_f32"]
    assert sha(codes) == fx["fp8_codes_sha256"]
    assert sha(kv.fp8_dequant_heads(codes, scales)) == fx["fp8_dequant_bf16_sha256"]


def test_configs0_int8_slabs(configs0):
    fx, x = configs0
    q, s = kv.int8_legacy_quant_slabs(x.reshape(288, -1))
    assert f32_hex(s) == fx["int8_scales_bf16_as_f32"]
    assert sha(q) == fx["int8_codes_sha256"]
    assert sha(kv.int8_legacy_dequant_slabs(q, s)) == fx["int8_dequant_bf16_sha256"]


def test_configs0_int8_per_tensor_drop_in(configs0):
    """The reference's per-tensor functions (precision.py:8-16) on three of the slabs."""
    fx, x = configs0
    want = f32_from_hex(fx["int8_scales_bf16_as_f32"])
    xs = x.reshape(288, -1)
    q_all, _ = kv.int8_legacy_quant_slabs(xs)
    for i in (0, 145, 287):
        q, s = quantize_to_fp8_storage(xs[i])
        assert s.dtype == torch.bfloat16 and s.float().item() == want[i]
        assert torch.equal(q, q_all[i])
        y = dequantize_for_bf16_compute(q, s)
        assert torch.equal(y, kv.int8_legacy_dequant_slabs(q_all[i:i + 1], s.reshape(1))[0])


def test_paged_small_append_gather(dev):
    fx = fixture("paged_small.json")
    H, D, P, n_pages, out_len = fx["H"], fx["D"], fx["page_size"], fx["n_pages"], fx["out_len"]
    x = torch.tensor(np.array(fx["x_bf16_bits"], np.uint16).view(np.int16)).view(torch.bfloat16)
    x = x.reshape(fx["x_shape"]).to(dev)
    cu = torch.tensor(fx["cu_seqlens"], dtype=torch.int32, device=dev)
    bt = torch.tensor(fx["block_tables"], dtype=torch.int32, device=dev).reshape(2, -1)
    pool = torch.full((1, n_pages, 2, H, P, D), 0, dtype=torch.uint8, device=dev)
    sc = kv.kv_quant_append(x, cu, bt, pool, check=True)
    assert f32_hex(sc) == fx["scales_f32"]
    assert pool.cpu().reshape(-1).tolist() == fx["pool"]
    sl = torch.tensor(fx["seq_lens"], dtype=torch.int32, device=dev)
    k, v = kv.kv_gather_dequant(pool[0], sc[0], bt, sl, out_len, check=True)
    assert k.cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1).tolist() == fx["k_bf16_bits"]
    assert v.cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1).tolist() == fx["v_bf16_bits"]


def test_reference_kats_through_drop_ins(dev):
    kats = fixture("reference_kats.json")
    k = kats["belady_farthest_next_use"]
    cache = BeladyApproxCache(capacity=k["capacity"])
    for key, nxt in k["update_future"]:
        cache.update_future(key, nxt)
    for key in k["touch"]:
        assert cache.touch(key) == []
    assert cache.touch(k["last_touch"]) == k["evicted"]
    r = kats["precision_roundtrip"]
    x = torch.randn(*r["shape"])
    q, scale = quantize_to_fp8_storage(x)
    y = dequantize_for_bf16_compute(q, scale)
    assert list(y.shape) == r["shape"] and y.dtype == getattr(torch, r["dequant_dtype"])
