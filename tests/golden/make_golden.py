"""Writes the golden fixtures of this directory (run from the repository root):

    python tests/golden/make_golden.py

* ``reference_kats.json``: the known answers the reference's own tests hold for this path
  (zenyx/tests/test_streaming.py:14-22, 25-28, 31-36), copied as data, plus the OCP OFP8
  e4m3fn boundary table the FP8 encoder follows.
* ``configs0.json``: the expected results of the README toy model's case (its
  KV cache ``[12, 2, 1, 12, 4096, 64]`` bf16, ``torch.manual_seed(0)``, N(0, 1) drawn in
  fp32) from the C oracle: all 288 per-(layer, kv, head) FP8 scales and legacy int8
  scales as fp32 bit patterns, and SHA-256 digests of the codes and dequantised values.
* ``paged_small.json``: one ragged paged append + gather written out in full (inputs,
  scales, the whole page pool, the gathered K / V with zeros past each length).

The fixtures are data only.  The values come from the C oracle (oracle/zx_oracle.c),
which tests/test_oracle.py pins against closed forms, torch's own e4m3 conversion and
brute force; the tests of this directory check the oracle and the HIP kernels against
these files, so a change in either shows up as a fixture mismatch.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))

CONFIGS0_SHAPE = [12, 2, 1, 12, 4096, 64]


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def f32_hex(v) -> list[str]:
    return [f"{int(b):08x}" for b in np.asarray(v, np.float32).reshape(-1).view(np.uint32)]


def configs0_input():
    """bf16 bit patterns of configs[0]'s cache, as ``[24, 1, 12, 262144]`` (slab (l, kv, h)
    at outer index 2 l + kv, head h)."""
    import torch

    torch.manual_seed(0)
    x = torch.randn(CONFIGS0_SHAPE, dtype=torch.float32).to(torch.bfloat16)
    return x.view(torch.int16).numpy().view(np.uint16).reshape(24, 1, 12, 4096 * 64)


def configs0_expected(O) -> dict:
    xb = configs0_input()
    codes, scales = O.fp8_quant_heads(xb)
    y = O.fp8_dequant_heads(codes, scales)
    slabs = xb.reshape(288, 4096 * 64)
    q = np.empty(slabs.shape, np.int8)
    s8 = np.empty(288, np.float32)
    yi = np.empty(slabs.shape, np.uint16)
    for i in range(288):
        q[i], s8[i] = O.int8_legacy_quant(slabs[i], "bf16")
        yi[i] = O.int8_legacy_dequant(q[i], s8[i])
    return {
        "shape": CONFIGS0_SHAPE,
        "seed": 0,
        "input_sha256": sha256(xb),
        "fp8_scales_f32": f32_hex(scales),
        "fp8_codes_sha256": sha256(codes),
        "fp8_dequant_bf16_sha256": sha256(y),
        "int8_scales_bf16_as_f32": f32_hex(s8),
        "int8_codes_sha256": sha256(q),
        "int8_dequant_bf16_sha256": sha256(yi),
    }


def paged_small_input():
    """A ragged batch: 2 sequences of 5 and 3 tokens, 2 heads, D 64, pages of 4 tokens,
    6 pages, non-contiguous block tables; one value per kv / head is large so the
    scales differ between heads."""
    import torch

    g = torch.Generator().manual_seed(11)
    H, D, lens = 2, 64, [5, 3]
    x = torch.randn((1, sum(lens), 2, H, D), generator=g, dtype=torch.float32)
    x[0, 1, 0, 1, 3] = 37.0
    x[0, 6, 1, 0, 5] = -0.02
    xb = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return {
        "x_bf16_bits": xb, "cu_seqlens": np.array([0, 5, 8], np.int32),
        "block_tables": np.array([[3, 0], [5, 1]], np.int32), "seq_lens": np.array(lens, np.int32),
        "H": H, "D": D, "page_size": 4, "n_pages": 6, "out_len": 6,
    }


def paged_small_expected(O) -> dict:
    inp = paged_small_input()
    H, D, P, n_pages = inp["H"], inp["D"], inp["page_size"], inp["n_pages"]
    pool = np.zeros((1, n_pages, 2, H, P, D), np.uint8)
    sc, err = O.kv_quant_append(inp["x_bf16_bits"], inp["cu_seqlens"], None, inp["block_tables"], pool, P)
    assert err == 0
    k, v, err = O.kv_gather_dequant(pool[0], sc[0], inp["block_tables"], inp["seq_lens"], inp["out_len"])
    assert err == 0
    out = {key: (val.reshape(-1).tolist() if isinstance(val, np.ndarray) else val) for key, val in inp.items()}
    out["x_shape"] = list(inp["x_bf16_bits"].shape)
    out.update({"scales_f32": f32_hex(sc), "pool": pool.reshape(-1).tolist(),
                "k_bf16_bits": k.reshape(-1).tolist(), "v_bf16_bits": v.reshape(-1).tolist()})
    return out


def reference_kats() -> dict:
    inf = float("inf")
    return {
        "belady_farthest_next_use": {
            "source": "zenyx/tests/test_streaming.py:14-22",
            "capacity": 2,
            "update_future": [["a", 1], ["b", 100], ["c", 2]],
            "touch": ["a", "b"],
            "last_touch": "c",
            "evicted": ["b"],
        },
        "bandwidth_throttle": {
            "source": "zenyx/tests/test_streaming.py:25-28",
            "max_fetch_to_compute_ratio": 1.0,
            "cases": [{"fetch_time_ms": 2.0, "compute_time_ms": 1.0, "throttle": True},
                      {"fetch_time_ms": 0.5, "compute_time_ms": 1.0, "throttle": False}],
        },
        "precision_roundtrip": {
            "source": "zenyx/tests/test_streaming.py:31-36",
            "shape": [4, 4],
            "dequant_dtype": "bfloat16",
        },
        "e4m3fn_boundaries": {
            "source": "OCP 8-bit Floating Point Specification (OFP8) v1.0, E4M3 with NaN for overflow",
            "cases": [[v if abs(v) != inf else ("inf" if v > 0 else "-inf"), c] for v, c in [
                (448.0, 0x7E), (464.0, 0x7E), (470.0, 0x7F), (2.0 ** -10, 0x00), (1.5 * 2.0 ** -9, 0x02),
                (2.0 ** -9, 0x01), (1.0625, 0x38), (1.1875, 0x3A), (240.0, 0x77), (248.0, 0x78),
                (-0.0, 0x80), (inf, 0x7F), (-inf, 0xFF), (-470.0, 0xFF), (2.0 ** -6, 0x08)]],
        },
    }


def main() -> None:
    sys.path.insert(0, ROOT)
    from oracle import oracle as O

    for name, obj in [("reference_kats.json", reference_kats()),
                      ("configs0.json", configs0_expected(O)),
                      ("paged_small.json", paged_small_expected(O))]:
        with open(os.path.join(HERE, name), "w") as f:
            json.dump(obj, f, indent=1 if name != "paged_small.json" else None)
            f.write("\n")
        print("wrote", name)


if __name__ == "__main__":
    main()
