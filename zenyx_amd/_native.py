"""ctypes binding of ``libzenyx_kv.so`` (the C ABI declared in include/zenyx_kv.h).

The library is the only compute path of this package: when it is missing, or no HIP
device is present, every operation raises instead of falling back to anything else.
"""
from __future__ import annotations

import atexit
import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libzenyx_kv.so")

ZX_OK = 0
ZX_ERR_INVALID = -1
ZX_ERR_HIP = -2
ZX_ERR_UNSUPPORTED = -3
ZX_ERR_WORKSPACE = -4

ZX_BF16, ZX_F16, ZX_F32 = 0, 1, 2
ZX_KERR_PAGE_RANGE, ZX_KERR_POS_RANGE, ZX_KERR_SPIN, ZX_KERR_OVERFLOW = 1, 2, 4, 8
ZX_APPEND_STATIC_SCALES = 1
ZX_APPEND_TWO_PASS = 2
ZX_APPEND_SATURATE = 4
ZX_APPEND_SINGLE_PASS = 8
ZX_PREFILL_MERGE, ZX_PREFILL_INIT, ZX_PREFILL_BF16, ZX_PREFILL_FAST_P, ZX_PREFILL_EXACT_P = 1, 2, 4, 8, 16
ZX_PREFILL_LAST = 32
ZX_PREFILL_FINAL = 64
ZX_HEADS_TWO_PASS = 1
ZX_HEADS_SINGLE_PASS = 2
ZX_NEVER = 0x7FFFFFFF
ABI_VERSION = 7

_P = ctypes.c_void_p
_I64, _I32, _SZ, _INT = ctypes.c_int64, ctypes.c_int32, ctypes.c_size_t, ctypes.c_int

# name -> (restype, argtypes); kept in the order of include/zenyx_kv.h
SIGNATURES = {
    "zx_last_error": (ctypes.c_char_p, []),
    "zx_abi_version": (_INT, []),
    "zx_set_wait_bound_us": (_INT, [_I64]),
    "zx_int8_legacy_quant": (_INT, [_P, _INT, _I64, _P, _P, _P, _SZ, _P]),
    "zx_int8_legacy_dequant": (_INT, [_P, _P, _INT, _I64, _P, _P]),
    "zx_int8_legacy_quant_slabs_workspace_bytes": (_SZ, [_I64]),
    "zx_int8_legacy_quant_slabs": (_INT, [_P, _INT, _I64, _I64, _P, _P, _P, _SZ, _P]),
    "zx_int8_legacy_dequant_slabs": (_INT, [_P, _P, _INT, _I64, _I64, _P, _P]),
    "zx_fp8_quant_heads_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "zx_fp8_quant_heads": (_INT, [_P, _I64, _I64, _I64, _I64, _P, _P, _I32, _P, _P, _SZ, _P]),
    "zx_fp8_dequant_heads": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _P, _P]),
    "zx_fp8_encode_f32": (_INT, [_P, _I64, _P, _P]),
    "zx_kv_scales": (_INT, [_P, _I64, _I32, _I64, _I32, _I32, _P, _P]),
    "zx_kv_quant_append_workspace_bytes": (_SZ, [_I32, _I64, _I32, _I32]),
    "zx_kv_quant_append": (_INT, [_P, _I64, _I32, _I64, _I32, _I32, _P, _P, _I32, _P, _I32, _I32,
                                  _P, _I64, _I64, _P, _I32, _P, _P, _SZ, _P]),
    "zx_kv_quant_append_noalloc": (_INT, [_P, _I64, _I32, _I64, _I32, _I32, _P, _P, _I32, _P, _I32, _I32,
                                          _P, _I64, _I64, _P, _I32, _P, _P]),
    "zx_kv_gather_dequant": (_INT, [_P, _I64, _I32, _I32, _I32, _P, _P, _I32, _P, _I32, _I32, _P,
                                    _P, _P, _P]),
    "zx_belady_argmax_workspace_bytes": (_SZ, [_I64]),
    "zx_belady_argmax": (_INT, [_P, _P, _P, _I64, _P, _P, _SZ, _P]),
    "zx_belady_update_slots": (_INT, [_P, _P, _P, _I64, _P, _P, _P, _P, _I64, _P, _P]),
    "zx_belady_next_use_workspace_bytes": (_SZ, [_I64, _I32]),
    "zx_belady_next_use": (_INT, [_P, _I64, _I32, _P, _P, _P, _P, _SZ, _P]),
    "zx_belady_simulate_workspace_bytes": (_SZ, [_I64, _I32]),
    "zx_belady_simulate": (_INT, [_P, _P, _P, _I64, _I64, _I64, _I32, _I64, _P, _P, _P, _P, _P,
                                  _I64, _P, _P, _SZ, _P]),
    "zx_tier_copy_runs": (_INT, [_P, _P, _P, _P, _I64, _I64, _P, _P]),
    "zx_paged_attention_decode_workspace_bytes": (ctypes.c_size_t, [_I32, _I32, _I32, _I32, _I32, _I32]),
    "zx_paged_attention_decode": (_INT, [_P, _I32, _P, _I64, _I32, _I32, _I32, _P, _P, _I32, _P, _I32,
                                         ctypes.c_float, _P, _P, _P, ctypes.c_size_t, _P]),
    "zx_tier_move_pages": (_INT, [_P, _I64, _P, _I64, _P, _P, _I64, _I64, _I32, _P, _P]),
    "zx_belady_tier_plan": (_INT, [_P, _P, _P, _I64, _P, _P, _I64, _P, _P, _I64, _P, _P, _P, _P, _P]),
    "zx_ring_curriculum_trace_len": (_I64, [_P, _P, _I32, _I32]),
    "zx_ring_curriculum_trace": (_INT, [_P, _P, _I32, _I32, _I32, _P, _I64, _P]),
    "zx_paged_attention_prefill": (_INT, [_P, _I64, _P, _P, _I32, _P, _I64, _I32, _I32, _I32, _P, _P, _I32, _P,
                                          _P, _I32, _I32, _I32, ctypes.c_float, _I32, _P, _P, _P, _P, _P]),
    "zx_paged_attention_ring": (_INT, [_P, _I64, _P, _P, _I32, _P, _I64, _I32, _I32, _I32, _P, _P, _I32, _P,
                                       _P, _I32, _I32, _I32, _I32, ctypes.c_float, _I32, _P, _P, _P, _P, _P]),
}

_lib = None
_lock = threading.Lock()


class ZenyxNativeError(RuntimeError):
    """A HIP failure inside libzenyx_kv.so."""


def load() -> ctypes.CDLL:
    """Load the library and bind every entry point; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
                    "g.build()'` (or zenyx_amd.build.build()); zenyx_amd has no CPU fallback")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.zx_abi_version() != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH} has ABI {lib.zx_abi_version()}, expected {ABI_VERSION}")
            from ._streams import teardown

            atexit.register(teardown)
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    """Map a zx status code to the Python exception the reference contract uses."""
    if rc == ZX_OK:
        return
    msg = load().zx_last_error().decode(errors="replace")
    text = f"{what}: {msg}" if msg else what
    if rc in (ZX_ERR_INVALID, ZX_ERR_UNSUPPORTED):
        raise ValueError(text)
    raise ZenyxNativeError(f"{text} (status {rc})")


def require_device(t: torch.Tensor, name: str) -> None:
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a HIP device tensor, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.data_ptr() % 16:
        raise ValueError(f"{name} must be 16-byte aligned")


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_ptr(device: torch.device | None = None):
    """The current torch stream of `device` as a hipStream_t."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ensure_gpu() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("zenyx_amd needs a HIP device (MI355X); none is visible")
    load()
    return torch.device("cuda", torch.cuda.current_device())
