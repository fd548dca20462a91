"""Drop-in for zenyx/streaming/precision.py: per-tensor int8 "FP8-ish" storage.

Same signatures and results as the reference (precision.py:8-16), computed by the
libzenyx_kv.so kernels (zx_int8_legacy_quant / zx_int8_legacy_dequant).  Tensors already
on the HIP device stay there; CPU tensors are staged through the device and the results
come back on the CPU, as the reference returns them on the input's device.

Arithmetic follows torch's CPU evaluation of the reference expressions (every
intermediate rounded to the input dtype, true fp32 division, half-to-even rounding),
which is what the reference's own test exercises (zenyx/tests/test_streaming.py:31-36).
"""
from __future__ import annotations

import torch

from .. import kv
from .._native import ensure_gpu


def quantize_to_fp8_storage(tensor: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Store tensor as int8 + scale (precision.py:8-12): scale = max(amax, 1e-8) / 127 as a
    0-dim tensor of the input dtype, q = clamp(round(tensor / scale), -127, 127)."""
    if tensor.device.type == "cuda":
        return kv.int8_legacy_quant(tensor.detach())
    dev = ensure_gpu()
    q, s = kv.int8_legacy_quant(tensor.detach().to(dev))
    return q.cpu(), s.cpu()


def dequantize_for_bf16_compute(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """(q.float() * scale).to(bfloat16) (precision.py:15-16)."""
    if q.device.type == "cuda":
        return kv.int8_legacy_dequant(q, scale)
    dev = ensure_gpu()
    return kv.int8_legacy_dequant(q.to(dev), scale.to(dev)).cpu()


__all__ = ["quantize_to_fp8_storage", "dequantize_for_bf16_compute"]
