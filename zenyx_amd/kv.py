"""Torch-facing operations of the KV-cache hot path, each a thin wrapper over one entry
point of libzenyx_kv.so (include/zenyx_kv.h).

Tensors must live on the HIP device; the wrappers validate dtype/shape/contiguity on the
host, pass raw pointers and the current torch stream, and never synchronise unless asked
(``check=True`` reads back the kernels' error word and raises ``ValueError``).

Layouts:
  * KV cache tensor (FP8KVQuantizer): ``[L, 2, B, H, T, D]`` bf16, scales ``[L, 2, H]``.
  * token-major append input: ``[L, n_tok, 2, H, D]`` (or one layer ``[n_tok, 2, H, D]``).
  * page pool: ``[L, n_pages, 2, H, P, D]`` uint8 e4m3fn codes (or one layer without L).
"""
from __future__ import annotations

import ctypes

import torch

from . import _native as N

_DT = {torch.bfloat16: N.ZX_BF16, torch.float16: N.ZX_F16, torch.float32: N.ZX_F32}


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16) if t.dtype in (torch.bfloat16, torch.float16) else t


def _err_word(device) -> torch.Tensor:
    return torch.zeros(1, dtype=torch.int32, device=device)


def _err_word_if(check: bool, device) -> torch.Tensor | None:
    """A fresh device error word when the call will read it (check=True), else None: the
    kernels then skip their error reports (every one is guarded), and the call saves the
    word's fill kernel."""
    return _err_word(device) if check else None


def kernel_error_text(e: int) -> str:
    """The ZX_KERR_* bits of a device error word, in words."""
    parts = []
    if e & N.ZX_KERR_PAGE_RANGE:
        parts.append("block table entry outside [0, n_pages)")
    if e & N.ZX_KERR_POS_RANGE:
        parts.append("token position beyond max_blocks * page_size (attention: or a query row beyond "
                     "max_q_per_seq)")
    if e & N.ZX_KERR_SPIN:
        parts.append("bounded wait ran out")
    if e & N.ZX_KERR_OVERFLOW:
        parts.append("a token exceeds 464 x its static FP8 scale (stored as the NaN code, or as +-448 when "
                     "saturating)")
    return "; ".join(parts)


def _raise_kernel_error(err: torch.Tensor, what: str) -> None:
    e = int(err.item())
    if e:
        raise ValueError(f"{what}: " + kernel_error_text(e))


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


# ------------------------------------------------------------------ legacy int8

def int8_legacy_quant(x: torch.Tensor):
    """zenyx/streaming/precision.py:8-12 on the GPU: (q int8, 0-dim scale in x.dtype)."""
    N.ensure_gpu()
    if x.dtype not in _DT:
        raise TypeError(f"quantize_to_fp8_storage: unsupported dtype {x.dtype}")
    if x.numel() == 0:
        # precision.py:10 -- amax of an empty tensor raises in torch
        raise RuntimeError("quantize_to_fp8_storage: cannot quantize an empty tensor (amax over zero elements)")
    x = x.contiguous()
    N.require_device(x, "x")
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    scale = torch.empty((), dtype=x.dtype, device=x.device)
    ws = _workspace(256, x.device)
    N.check(N.load().zx_int8_legacy_quant(N.ptr(x), _DT[x.dtype], x.numel(), N.ptr(q), N.ptr(scale),
                                          N.ptr(ws), ws.numel(), N.stream_ptr(x.device)),
            "quantize_to_fp8_storage")
    return q, scale


def int8_legacy_dequant(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """zenyx/streaming/precision.py:15-16 on the GPU."""
    N.ensure_gpu()
    if q.dtype != torch.int8:
        q = q.to(torch.int8)
    q = q.contiguous()
    scale = scale.reshape(()).to(q.device)
    if scale.dtype not in _DT:
        scale = scale.float()
    scale = scale.contiguous()
    N.require_device(q, "q")
    y = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    N.check(N.load().zx_int8_legacy_dequant(N.ptr(q), N.ptr(scale), _DT[scale.dtype], q.numel(), N.ptr(y),
                                            N.stream_ptr(q.device)), "dequantize_for_bf16_compute")
    return y


def int8_legacy_quant_slabs(x: torch.Tensor):
    """precision.py:8-12 applied to every slab ``x[i]`` of ``x [n_slabs, ...]`` in one launch:
    (q int8 like x, scales ``[n_slabs]`` in x.dtype), bit-identical to
    ``int8_legacy_quant(x[i])`` for every i."""
    N.ensure_gpu()
    if x.dtype not in _DT:
        raise TypeError(f"quantize_to_fp8_storage: unsupported dtype {x.dtype}")
    if x.dim() < 1 or x.shape[0] == 0 or x[0].numel() == 0:
        raise RuntimeError("quantize_to_fp8_storage: cannot quantize an empty tensor (amax over zero elements)")
    x = x.contiguous()
    N.require_device(x, "x")
    n_slabs, slab = x.shape[0], x[0].numel()
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    scales = torch.empty((n_slabs,), dtype=x.dtype, device=x.device)
    ws = _workspace(N.load().zx_int8_legacy_quant_slabs_workspace_bytes(n_slabs), x.device)
    N.check(N.load().zx_int8_legacy_quant_slabs(N.ptr(x), _DT[x.dtype], n_slabs, slab, N.ptr(q), N.ptr(scales),
                                                N.ptr(ws), ws.numel(), N.stream_ptr(x.device)),
            "int8_legacy_quant_slabs")
    return q, scales


def int8_legacy_dequant_slabs(q: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """precision.py:15-16 applied to every slab: bf16 ``y[i] = (q[i].float() * scales[i]).to(bf16)``."""
    N.ensure_gpu()
    if q.dtype != torch.int8 or q.dim() < 1:
        raise ValueError("q must be int8 [n_slabs, ...]")
    if scales.dtype not in _DT or scales.shape != (q.shape[0],):
        raise ValueError("scales must be [n_slabs] in bf16, f16 or f32")
    q, scales = q.contiguous(), scales.contiguous()
    N.require_device(q, "q")
    N.require_device(scales, "scales")
    y = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    N.check(N.load().zx_int8_legacy_dequant_slabs(N.ptr(q), N.ptr(scales), _DT[scales.dtype], q.shape[0],
                                                  q[0].numel() if q.shape[0] else 0, N.ptr(y), N.stream_ptr(q.device)),
            "int8_legacy_dequant_slabs")
    return y


# ------------------------------------------------------------------ FP8 per head

# zx_fp8_quant_heads reads inputs of this many bytes and more in one pass (its cooperative
# single-pass kernel); below it the second read of two passes comes from the Infinity Cache.
HEADS_SINGLE_PASS_BYTES = 256 << 20


def set_wait_bound_us(us: int | None) -> None:
    """Bound (microseconds) of one wait without progress inside the cooperative
    single-pass kernels; ``None`` restores the default (2 s).  0 makes the first such wait
    give up: the call then returns with ZX_KERR_SPIN in its error word and undefined
    outputs (every wave exits normally).  Process-wide; for tests and operators."""
    N.check(N.load().zx_set_wait_bound_us(-1 if us is None else int(us)), "set_wait_bound_us")


def fp8_quant_heads(x: torch.Tensor, two_pass: bool = False, check: bool = False, single_pass: bool = False):
    """x: bf16 ``[n_outer, n_batch, n_heads, run]`` -> (codes uint8 same shape, scales
    fp32 ``[n_outer, n_heads]``), one scale per (outer, head).  Inputs of 256 MiB and more
    are read once (the single-pass kernel), smaller ones in two passes (the second read
    comes from the Infinity Cache); ``two_pass`` / ``single_pass`` force either path (same
    results)."""
    N.ensure_gpu()
    if x.dtype != torch.bfloat16 or x.dim() != 4:
        raise ValueError("fp8_quant_heads: x must be bf16 [n_outer, n_batch, n_heads, run]")
    N.require_device(x, "x")
    O, B, H, R = x.shape
    codes = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    scales = torch.empty((O, H), dtype=torch.float32, device=x.device)
    lib = N.load()
    if two_pass and single_pass:
        raise ValueError("fp8_quant_heads: two_pass and single_pass are exclusive")
    ws = None if two_pass else _workspace(lib.zx_fp8_quant_heads_workspace_bytes(O, B, H, R), x.device)
    err = _err_word_if(check, x.device)
    flags = N.ZX_HEADS_TWO_PASS if two_pass else (N.ZX_HEADS_SINGLE_PASS if single_pass else 0)
    N.check(lib.zx_fp8_quant_heads(N.ptr(x), O, B, H, R, N.ptr(codes), N.ptr(scales),
                                   flags, N.ptr(err), N.ptr(ws),
                                   0 if ws is None else ws.numel(), N.stream_ptr(x.device)), "fp8_quant_heads")
    if check:
        _raise_kernel_error(err, "fp8_quant_heads")
    return codes, scales


def fp8_dequant_heads(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    N.ensure_gpu()
    if codes.dtype != torch.uint8 or codes.dim() != 4:
        raise ValueError("fp8_dequant_heads: codes must be uint8 [n_outer, n_batch, n_heads, run]")
    O, B, H, R = codes.shape
    if scales.shape != (O, H) or scales.dtype != torch.float32:
        raise ValueError(f"fp8_dequant_heads: scales must be float32 {(O, H)}")
    N.require_device(codes, "codes")
    N.require_device(scales, "scales")
    y = torch.empty(codes.shape, dtype=torch.bfloat16, device=codes.device)
    N.check(N.load().zx_fp8_dequant_heads(N.ptr(codes), N.ptr(scales), O, B, H, R, N.ptr(y),
                                          N.stream_ptr(codes.device)), "fp8_dequant_heads")
    return y


def fp8_encode_f32(v: torch.Tensor) -> torch.Tensor:
    """Already-scaled fp32 values -> e4m3fn codes (uint8), nearest-even, overflow -> NaN."""
    N.ensure_gpu()
    if v.dtype != torch.float32:
        raise ValueError("fp8_encode_f32: v must be float32")
    v = v.contiguous()
    N.require_device(v, "v")
    codes = torch.empty(v.shape, dtype=torch.uint8, device=v.device)
    N.check(N.load().zx_fp8_encode_f32(N.ptr(v), v.numel(), N.ptr(codes), N.stream_ptr(v.device)),
            "fp8_encode_f32")
    return codes


# ------------------------------------------------------------------ paged KV

def _layers(x: torch.Tensor):
    if x.dim() == 4:
        x = x.unsqueeze(0)
    if x.dim() != 5 or x.shape[2] != 2:
        raise ValueError("x must be [L, n_tok, 2, H, D] (or [n_tok, 2, H, D])")
    if x.dtype != torch.bfloat16:
        raise ValueError("x must be bfloat16")
    return x


def kv_scales(x: torch.Tensor) -> torch.Tensor:
    """Per-(layer, kv, head) FP8 scales of a token-major batch -> ``[L, 2, H]`` fp32."""
    N.ensure_gpu()
    x = _layers(x)
    N.require_device(x, "x")
    L, T, _, H, D = x.shape
    scales = torch.empty((L, 2, H), dtype=torch.float32, device=x.device)
    N.check(N.load().zx_kv_scales(N.ptr(x), T * 2 * H * D, L, T, H, D, N.ptr(scales),
                                  N.stream_ptr(x.device)), "kv_scales")
    return scales


def kv_quant_append(x: torch.Tensor, cu_seqlens: torch.Tensor, block_tables: torch.Tensor,
                    pool: torch.Tensor, scales: torch.Tensor | None = None,
                    start_pos: torch.Tensor | None = None, static_scales: bool = False,
                    check: bool = False, two_pass: bool = False, saturate: bool = False,
                    err: torch.Tensor | None = None, single_pass: bool = False) -> torch.Tensor:
    """Paged append with fused FP8 quantisation.

    x ``[L, n_tok, 2, H, D]`` bf16; cu_seqlens int32 ``[B+1]``; block_tables int32
    ``[B, max_blocks]``; pool uint8 ``[L, n_pages, 2, H, P, D]`` (written in place).
    Without ``static_scales`` the scales are computed from this batch and written into
    ``scales`` (allocated if None); returns the scales ``[L, 2, H]``.  With static scales a
    token beyond 464 x its scale is stored as the NaN code and flags an overflow, or as
    +-448 with ``saturate``.  ``err`` (device int32 ``[1]``) collects the kernels' error
    bits across calls (a fresh word by default); ``check`` reads it and raises.  Dynamic
    scales take one cooperative pass or two passes, whichever the library expects to be
    faster for the call's size; ``two_pass`` / ``single_pass`` force either (same results).
    """
    N.ensure_gpu()
    x = _layers(x)
    if pool.dim() == 5:
        pool = pool.unsqueeze(0)
    L, T, _, H, D = x.shape
    if pool.dim() != 6 or pool.shape[0] != L or pool.shape[2:4] != (2, H) or pool.shape[5] != D:
        raise ValueError(f"pool must be uint8 [L={L}, n_pages, 2, H={H}, P, D={D}]")
    if pool.dtype != torch.uint8:
        raise ValueError("pool must be uint8")
    n_pages, P = pool.shape[1], pool.shape[4]
    for name, t in (("cu_seqlens", cu_seqlens), ("block_tables", block_tables)):
        if t.dtype != torch.int32:
            raise ValueError(f"{name} must be int32")
    if block_tables.dim() != 2 or cu_seqlens.dim() != 1 or cu_seqlens.numel() != block_tables.shape[0] + 1:
        raise ValueError("block_tables must be [B, max_blocks] and cu_seqlens [B+1]")
    if start_pos is not None and (start_pos.dtype != torch.int32 or start_pos.numel() != block_tables.shape[0]):
        raise ValueError("start_pos must be int32 [B]")
    if scales is None:
        if static_scales:
            raise ValueError("static_scales needs scales")
        scales = torch.empty((L, 2, H), dtype=torch.float32, device=x.device)
    if scales.shape != (L, 2, H) or scales.dtype != torch.float32:
        raise ValueError(f"scales must be float32 [{L}, 2, {H}]")
    for name, t in (("x", x), ("cu_seqlens", cu_seqlens), ("block_tables", block_tables), ("pool", pool),
                    ("scales", scales)) + ((("start_pos", start_pos),) if start_pos is not None else ()):
        N.require_device(t, name)
    if saturate and not static_scales:
        raise ValueError("saturate applies to static scales (dynamic scales never overflow)")
    if two_pass and single_pass:
        raise ValueError("kv_quant_append: two_pass and single_pass are exclusive")
    lib = N.load()
    ws = _workspace(lib.zx_kv_quant_append_workspace_bytes(L, T, H, D), x.device)
    if err is None:
        err = _err_word_if(check, x.device)
    elif err.dtype != torch.int32 or err.numel() < 1 or err.device != x.device:
        raise ValueError("err must be an int32 tensor on x's device")
    flags = (N.ZX_APPEND_STATIC_SCALES if static_scales else 0) | (N.ZX_APPEND_TWO_PASS if two_pass else 0) | \
        (N.ZX_APPEND_SATURATE if saturate else 0) | (N.ZX_APPEND_SINGLE_PASS if single_pass else 0)
    N.check(lib.zx_kv_quant_append(N.ptr(x), T * 2 * H * D, L, T, H, D, N.ptr(cu_seqlens), N.ptr(start_pos),
                                   block_tables.shape[0], N.ptr(block_tables), block_tables.shape[1], P,
                                   N.ptr(pool), pool[0].numel(), n_pages, N.ptr(scales), flags, N.ptr(err),
                                   N.ptr(ws), ws.numel(), N.stream_ptr(x.device)), "kv_quant_append")
    if check:
        _raise_kernel_error(err, "kv_quant_append")
    return scales


def _aligned_scales(scales_layer: torch.Tensor) -> torch.Tensor:
    """One layer's ``[2, H]`` scales as the C ABI takes every pointer (contiguous, 16-byte
    aligned).  A layer of a ``[L, 2, H]`` tensor starts 8 H bytes after the previous one,
    so with H odd every other layer is not aligned: such a slice is copied (2 H floats)."""
    if scales_layer.device.type != "cuda" or (scales_layer.is_contiguous() and scales_layer.data_ptr() % 16 == 0):
        return scales_layer
    return scales_layer.clone(memory_format=torch.contiguous_format)


def kv_gather_dequant(pool_layer: torch.Tensor, scales_layer: torch.Tensor, block_tables: torch.Tensor,
                      seq_lens: torch.Tensor, out_len: int | None = None, check: bool = False,
                      out: tuple[torch.Tensor, torch.Tensor] | None = None):
    """Paged gather + dequant of one layer: pool ``[n_pages, 2, H, P, D]`` uint8, scales
    ``[2, H]`` fp32 -> (k, v), each bf16 ``[B, H, out_len, D]``; positions at or beyond
    ``seq_lens[b]`` are zeros."""
    N.ensure_gpu()
    if pool_layer.dim() != 5 or pool_layer.dtype != torch.uint8 or pool_layer.shape[1] != 2:
        raise ValueError("pool_layer must be uint8 [n_pages, 2, H, P, D]")
    n_pages, _, H, P, D = pool_layer.shape
    if scales_layer.shape != (2, H) or scales_layer.dtype != torch.float32:
        raise ValueError(f"scales_layer must be float32 [2, {H}]")
    scales_layer = _aligned_scales(scales_layer)
    if block_tables.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise ValueError("block_tables and seq_lens must be int32")
    B = block_tables.shape[0]
    if seq_lens.numel() != B:
        raise ValueError("seq_lens must have one entry per block-table row")
    if out_len is None:
        out_len = block_tables.shape[1] * P
    for name, t in (("pool_layer", pool_layer), ("scales_layer", scales_layer), ("block_tables", block_tables),
                    ("seq_lens", seq_lens)):
        N.require_device(t, name)
    if out is None:
        k = torch.empty((B, H, out_len, D), dtype=torch.bfloat16, device=pool_layer.device)
        v = torch.empty_like(k)
    else:
        k, v = out
        for t in (k, v):
            if t.shape != (B, H, out_len, D) or t.dtype != torch.bfloat16:
                raise ValueError(f"out tensors must be bf16 {(B, H, out_len, D)}")
            N.require_device(t, "out")
    err = _err_word_if(check, pool_layer.device)
    N.check(N.load().zx_kv_gather_dequant(N.ptr(pool_layer), n_pages, H, D, P, N.ptr(scales_layer),
                                          N.ptr(block_tables), block_tables.shape[1], N.ptr(seq_lens), B,
                                          out_len, N.ptr(k), N.ptr(v), N.ptr(err),
                                          N.stream_ptr(pool_layer.device)), "kv_gather_dequant")
    if check:
        _raise_kernel_error(err, "kv_gather_dequant")
    return k, v


def paged_attention_decode(q: torch.Tensor, pool_layer: torch.Tensor, scales_layer: torch.Tensor,
                           block_tables: torch.Tensor, seq_lens: torch.Tensor, sm_scale: float | None = None,
                           out: torch.Tensor | None = None, check: bool = False) -> torch.Tensor:
    """Decode attention straight from the FP8 pages: q ``[B, Hq, D]`` bf16 (one token per
    sequence), pool ``[n_pages, 2, Hkv, P, D]`` uint8, scales ``[2, Hkv]`` fp32 ->
    ``[B, Hq, D]`` bf16 = softmax(sm_scale * q K^T) V over positions < seq_lens[b], with
    K, V = decoded codes times their head's scale (query head i reads kv head
    i // (Hq / Hkv)).  ``sm_scale`` defaults to 1/sqrt(D)."""
    N.ensure_gpu()
    if pool_layer.dim() != 5 or pool_layer.dtype != torch.uint8 or pool_layer.shape[1] != 2:
        raise ValueError("pool_layer must be uint8 [n_pages, 2, Hkv, P, D]")
    n_pages, _, Hkv, P, D = pool_layer.shape
    if q.dim() != 3 or q.dtype != torch.bfloat16 or q.shape[2] != D:
        raise ValueError(f"q must be bf16 [B, Hq, {D}]")
    B, Hq, _ = q.shape
    if Hq % Hkv:
        raise ValueError("the number of query heads must be a multiple of the number of kv heads")
    if scales_layer.shape != (2, Hkv) or scales_layer.dtype != torch.float32:
        raise ValueError(f"scales_layer must be float32 [2, {Hkv}]")
    scales_layer = _aligned_scales(scales_layer)
    if block_tables.dtype != torch.int32 or seq_lens.dtype != torch.int32 or block_tables.dim() != 2:
        raise ValueError("block_tables [B, max_blocks] and seq_lens [B] must be int32")
    if block_tables.shape[0] != B or seq_lens.numel() != B:
        raise ValueError("block_tables and seq_lens need one row per sequence")
    q = q.contiguous()
    for name, t in (("q", q), ("pool_layer", pool_layer), ("scales_layer", scales_layer),
                    ("block_tables", block_tables), ("seq_lens", seq_lens)):
        N.require_device(t, name)
    if out is None:
        out = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=q.device)
    elif out.shape != (B, Hq, D) or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError(f"out must be contiguous bf16 {(B, Hq, D)}")
    lib = N.load()
    mb = block_tables.shape[1]
    ws = _workspace(lib.zx_paged_attention_decode_workspace_bytes(B, Hq, Hkv, D, mb, P), q.device)
    err = _err_word_if(check, q.device)
    N.check(lib.zx_paged_attention_decode(
        N.ptr(q), Hq, N.ptr(pool_layer), n_pages, Hkv, D, P, N.ptr(scales_layer), N.ptr(block_tables), mb,
        N.ptr(seq_lens), B, float(D ** -0.5 if sm_scale is None else sm_scale), N.ptr(out), N.ptr(err), N.ptr(ws),
        ws.numel(), N.stream_ptr(q.device)), "paged_attention_decode")
    if check:
        _raise_kernel_error(err, "paged_attention_decode")
    return out


# ------------------------------------------------------------------ Belady

# How the softmax weights P enter P.V (the row sums use the same P); bound on |got - exact|
# per output channel, beside one bf16 ulp of the exact value:
#   "f16"   (default) P * 2^7 rounded once to fp16, V in fp16: 2^-10 max|V|;
#   "bf16"  P rounded once to bf16 (ZX_PREFILL_FAST_P), the same speed: 2^-7 max|V|;
#   "exact" P as bf16 hi + lo (ZX_PREFILL_EXACT_P), ~1.3x the time: 2^-15 max|V| at worst
#           (measured within 2^-17 max|V|).
PRECISIONS = ("f16", "bf16", "exact")


def _precision_flag(precision: str) -> int:
    if precision == "f16":
        return 0
    if precision == "bf16":
        return N.ZX_PREFILL_FAST_P
    if precision == "exact":
        return N.ZX_PREFILL_EXACT_P
    raise ValueError(f"precision must be one of {PRECISIONS}, got {precision!r}")


def paged_attention_prefill(q: torch.Tensor, cu_q: torch.Tensor, q_pos0: torch.Tensor, pool_layer: torch.Tensor,
                            scales_layer: torch.Tensor, block_tables: torch.Tensor, kv_begin: torch.Tensor,
                            kv_end: torch.Tensor, causal: bool = True, sm_scale: float | None = None,
                            o_acc: torch.Tensor | None = None, lse2: torch.Tensor | None = None,
                            first: bool = True, out: torch.Tensor | None = None, write_bf16: bool = True,
                            max_q_per_seq: int | None = None, check: bool = False,
                            err: torch.Tensor | None = None, precision: str = "f16", last: bool = False,
                            final: bool = False):
    """One ring step of attention over the FP8 pages (zx_paged_attention_prefill).

    ``q`` [n_q, Hq, 128] bf16 rows of all sequences (``cu_q`` [B+1] int32 offsets,
    ``q_pos0`` [B] int32 position of each sequence's first query row); keys
    [kv_begin[b], kv_end[b]) of the pool layer through the block tables.  With ``o_acc``
    / ``lse2`` (fp32 [n_q, Hq, 128] / [n_q, Hq]) the step merges into them (``first``
    overwrites); with ``write_bf16`` the (merged) rows go to ``out`` as bf16, and ``last``
    (with both) leaves ``o_acc`` / ``lse2`` unwritten (ZX_PREFILL_LAST: a ring's last step
    whose running output is not needed afterwards).  ``final`` (with both, causal;
    ZX_PREFILL_FINAL) is for a causal ring whose steps cover each sequence's keys in
    ascending contiguous ranges from 0: rows below ``kv_begin`` are left alone (finished
    by an earlier step), rows below ``kv_end`` go to ``out`` only (no later key reaches
    them), the others merge into ``o_acc`` / ``lse2`` (and go to ``out`` too when ``last``).
    ``err`` (int32
    [1], zeroed by the caller) collects the kernel's input-error bits across several calls;
    by default each call uses a fresh one.  ``precision``: see PRECISIONS.  Returns ``out``
    (or None)."""
    p_flag = _precision_flag(precision)
    N.require_device(q, "q")
    if q.dtype != torch.bfloat16 or q.dim() != 3:
        raise ValueError("q must be [n_q, n_q_heads, head_dim] bfloat16")
    N.require_device(pool_layer, "pool_layer")
    if pool_layer.dim() != 5 or pool_layer.dtype != torch.uint8:
        raise ValueError("pool_layer must be uint8 [n_pages, 2, n_kv_heads, page_size, head_dim]")
    n_pages, two, Hkv, P, D = pool_layer.shape
    n_q, Hq, Dq = q.shape
    if two != 2 or Dq != D:
        raise ValueError("pool_layer must be [n_pages, 2, n_kv_heads, page_size, head_dim] matching q")
    scales_layer = _aligned_scales(scales_layer)
    N.require_device(scales_layer, "scales_layer")
    if scales_layer.shape != (2, Hkv) or scales_layer.dtype != torch.float32:
        raise ValueError(f"scales_layer must be float32 [2, {Hkv}]")
    if block_tables.dim() != 2:
        raise ValueError("block_tables must be int32 [n_seqs, max_blocks]")
    for t, name in ((cu_q, "cu_q"), (q_pos0, "q_pos0"), (block_tables, "block_tables"), (kv_begin, "kv_begin"),
                    (kv_end, "kv_end")):
        N.require_device(t, name)
        if t.dtype != torch.int32:
            raise ValueError(f"{name} must be int32")
    B = cu_q.numel() - 1
    if q_pos0.numel() != B or kv_begin.numel() != B or kv_end.numel() != B or block_tables.shape[0] != B:
        raise ValueError("cu_q, q_pos0, kv_begin, kv_end and block_tables disagree on the number of sequences")
    if (o_acc is None) != (lse2 is None):
        raise ValueError("o_acc and lse2 go together")
    if o_acc is not None:
        N.require_device(o_acc, "o_acc")
        N.require_device(lse2, "lse2")
        if o_acc.dtype != torch.float32 or o_acc.shape != q.shape or lse2.dtype != torch.float32 or \
                lse2.shape != (n_q, Hq):
            raise ValueError("o_acc must be float32 like q, lse2 float32 [n_q, n_q_heads]")
    if write_bf16:
        out = torch.empty_like(q) if out is None else out
        N.require_device(out, "out")
        if out.shape != q.shape or out.dtype != torch.bfloat16:
            raise ValueError("out must be bfloat16 like q")
    if max_q_per_seq is None:
        max_q_per_seq = int((cu_q[1:] - cu_q[:-1]).max().item()) if B else 0
    if last and (o_acc is None or not write_bf16):
        raise ValueError("last needs o_acc / lse2 and write_bf16")
    if final and (o_acc is None or not write_bf16 or not causal):
        raise ValueError("final needs o_acc / lse2, write_bf16 and causal")
    flags = (N.ZX_PREFILL_MERGE if o_acc is not None else 0) | (N.ZX_PREFILL_INIT if o_acc is not None and first
                                                                else 0) | (N.ZX_PREFILL_BF16 if write_bf16 else 0) | \
        (N.ZX_PREFILL_LAST if last else 0) | (N.ZX_PREFILL_FINAL if final else 0) | p_flag
    sm = float(sm_scale) if sm_scale is not None else 1.0 / float(D) ** 0.5
    dev = q.device
    if err is None:
        err = _err_word_if(check, dev)
    elif err.dtype != torch.int32 or err.numel() < 1 or err.device != dev:
        raise ValueError("err must be an int32 tensor on q's device")
    N.check(N.load().zx_paged_attention_prefill(
        N.ptr(q), n_q, N.ptr(cu_q), N.ptr(q_pos0), Hq, N.ptr(pool_layer), n_pages, Hkv, D, P, N.ptr(scales_layer),
        N.ptr(block_tables), block_tables.shape[1], N.ptr(kv_begin), N.ptr(kv_end), B, int(max_q_per_seq),
        int(bool(causal)), sm, flags, N.ptr(o_acc), N.ptr(lse2), N.ptr(out if write_bf16 else None), N.ptr(err),
        N.stream_ptr(dev)), "paged_attention_prefill")
    if check:
        _raise_kernel_error(err, "paged_attention_prefill")
    return out if write_bf16 else None


def paged_attention_ring(q: torch.Tensor, cu_q: torch.Tensor, q_pos0: torch.Tensor, pool_layer: torch.Tensor,
                         scales_layer: torch.Tensor, block_tables: torch.Tensor, kv_begin: torch.Tensor,
                         kv_end: torch.Tensor, causal: bool = True, sm_scale: float | None = None,
                         max_q_per_seq: int | None = None, check: bool = False,
                         err: torch.Tensor | None = None, precision: str = "f16") -> torch.Tensor:
    """All steps of a ring in one launch (zx_paged_attention_ring): ``kv_begin`` /
    ``kv_end`` int32 ``[R, B]`` hold step r's key range of every sequence; each block
    walks the R ranges with its running softmax state in registers and writes the bf16
    rows once.  Same arguments and result as R paged_attention_prefill steps merged;
    ``precision``: see PRECISIONS."""
    p_flag = _precision_flag(precision)
    N.require_device(q, "q")
    if q.dtype != torch.bfloat16 or q.dim() != 3:
        raise ValueError("q must be [n_q, n_q_heads, head_dim] bfloat16")
    N.require_device(pool_layer, "pool_layer")
    if pool_layer.dim() != 5 or pool_layer.dtype != torch.uint8 or pool_layer.shape[1] != 2:
        raise ValueError("pool_layer must be uint8 [n_pages, 2, n_kv_heads, page_size, head_dim]")
    n_pages, _, Hkv, P, D = pool_layer.shape
    n_q, Hq, Dq = q.shape
    if Dq != D:
        raise ValueError("q and pool_layer disagree on head_dim")
    scales_layer = _aligned_scales(scales_layer)
    N.require_device(scales_layer, "scales_layer")
    if scales_layer.shape != (2, Hkv) or scales_layer.dtype != torch.float32:
        raise ValueError(f"scales_layer must be float32 [2, {Hkv}]")
    B = cu_q.numel() - 1
    for t, name in ((cu_q, "cu_q"), (q_pos0, "q_pos0"), (block_tables, "block_tables"), (kv_begin, "kv_begin"),
                    (kv_end, "kv_end")):
        N.require_device(t, name)
        if t.dtype != torch.int32:
            raise ValueError(f"{name} must be int32")
    if kv_begin.dim() != 2 or kv_begin.shape != kv_end.shape or kv_begin.shape[1] != B:
        raise ValueError("kv_begin and kv_end must be int32 [n_ranges, n_seqs]")
    if q_pos0.numel() != B or block_tables.dim() != 2 or block_tables.shape[0] != B:
        raise ValueError("cu_q, q_pos0 and block_tables disagree on the number of sequences")
    if max_q_per_seq is None:
        max_q_per_seq = int((cu_q[1:] - cu_q[:-1]).max().item()) if B else 0
    out = torch.empty_like(q)
    sm = float(sm_scale) if sm_scale is not None else 1.0 / float(D) ** 0.5
    if err is None:
        err = _err_word_if(check, q.device)
    N.check(N.load().zx_paged_attention_ring(
        N.ptr(q), n_q, N.ptr(cu_q), N.ptr(q_pos0), Hq, N.ptr(pool_layer), n_pages, Hkv, D, P, N.ptr(scales_layer),
        N.ptr(block_tables), block_tables.shape[1], N.ptr(kv_begin), N.ptr(kv_end), kv_begin.shape[0], B,
        int(max_q_per_seq), int(bool(causal)), sm, N.ZX_PREFILL_BF16 | p_flag, None,
        None, N.ptr(out), N.ptr(err),
        N.stream_ptr(q.device)), "paged_attention_ring")
    if check:
        _raise_kernel_error(err, "paged_attention_ring")
    return out


def ring_attention_fp8(q: torch.Tensor, cu_q: torch.Tensor, q_pos0: torch.Tensor, pool_layer: torch.Tensor,
                       scales_layer: torch.Tensor, block_tables: torch.Tensor, kv_len: torch.Tensor,
                       ring_degree: int, causal: bool = True, sm_scale: float | None = None,
                       check: bool = False, single_launch: bool = True, precision: str = "f16",
                       max_q_per_seq: int | None = None, err: torch.Tensor | None = None) -> torch.Tensor:
    """Ring attention over the FP8 pages on one GPU: the keys [0, kv_len[b]) of every
    sequence are split into ``ring_degree`` shards (the KV blocks a ring would pass
    around), shard r being ring step r.  With ``single_launch`` one launch walks the R
    shards with the running softmax state in registers (zx_paged_attention_ring);
    otherwise each step is its own launch (paged_attention_prefill, the unit a ring over R
    GPUs runs) merged into a running fp32 output and log-sum-exp, the last one writing
    bf16 (causal: every step writes as bf16 the rows it completes, ZX_PREFILL_FINAL, so
    the last one converts only the rows it reaches).  Either equals attention over all keys (the exchange between devices is what
    one GPU leaves out).  ``precision``: how P enters P.V (see PRECISIONS).
    ``max_q_per_seq``: a bound on every sequence's query count, when the caller knows one
    (otherwise it is read back from ``cu_q``, which waits for the device).  The kernels
    trust it: rows of a sequence beyond it are not computed and their outputs are left
    undefined, and ZX_KERR_POS_RANGE is set in the error word when the call has one
    (``check=True`` reads a fresh one and raises; ``err``, device int32 ``[1]``, collects
    the bits for the caller to read later)."""
    _precision_flag(precision)
    if ring_degree < 1:
        raise ValueError("ring_degree must be >= 1")
    n_q, Hq, D = q.shape
    if max_q_per_seq is None:
        mq = int((cu_q[1:] - cu_q[:-1]).max().item()) if cu_q.numel() > 1 else 0
    else:
        mq = int(max_q_per_seq)
    # Shard r covers keys [kv_len * r // R, kv_len * (r + 1) // R): all bounds in one go,
    # so the loop below only launches the ring steps (rows padded to 16 bytes, the
    # alignment every pointer of the C ABI needs).
    B = kv_len.numel()
    steps = torch.arange(ring_degree + 1, dtype=torch.int64, device=kv_len.device)
    bounds = torch.empty((ring_degree + 1, (B + 3) // 4 * 4), dtype=torch.int32, device=kv_len.device)
    bounds[:, :B] = kv_len.to(torch.int64)[None, :] * steps[:, None] // ring_degree
    if err is None:
        err = _err_word_if(check, q.device)
    elif err.dtype != torch.int32 or err.numel() < 1 or err.device != q.device:
        raise ValueError("err must be an int32 tensor on q's device")
    if single_launch:
        out = paged_attention_ring(q, cu_q, q_pos0, pool_layer, scales_layer, block_tables,
                                   bounds[:-1, :B].contiguous(), bounds[1:, :B].contiguous(), causal=causal,
                                   sm_scale=sm_scale, max_q_per_seq=mq, err=err, precision=precision)
        if check:
            _raise_kernel_error(err, "ring_attention_fp8")
        return out
    o_acc = torch.empty((n_q, Hq, D), dtype=torch.float32, device=q.device)
    lse2 = torch.empty((n_q, Hq), dtype=torch.float32, device=q.device)
    out = torch.empty_like(q)
    for r in range(ring_degree):
        paged_attention_prefill(q, cu_q, q_pos0, pool_layer, scales_layer, block_tables, bounds[r, :B],
                                bounds[r + 1, :B],
                                causal=causal, sm_scale=sm_scale, o_acc=o_acc, lse2=lse2, first=r == 0, out=out,
                                write_bf16=causal or r == ring_degree - 1, max_q_per_seq=mq, err=err,
                                precision=precision, last=r == ring_degree - 1, final=causal)
    if check:
        _raise_kernel_error(err, "ring_attention_fp8")
    return out


def belady_argmax(keys: torch.Tensor, resident: torch.Tensor | None = None,
                  rank: torch.Tensor | None = None) -> torch.Tensor:
    """belady.py:39-51 over slots: device int64 ``[slot, key]`` ({-1, -1} if none).
    ``resident`` (uint8, default: every slot) selects the candidates; ``rank`` (int64,
    default: the slot index) breaks ties, smallest first."""
    N.ensure_gpu()
    if keys.dtype != torch.int64:
        raise ValueError("keys must be int64")
    N.require_device(keys, "keys")
    if resident is not None:
        if resident.dtype != torch.uint8 or resident.shape != keys.shape:
            raise ValueError("resident must be uint8 of keys' shape")
        N.require_device(resident, "resident")
    if rank is not None:
        if rank.dtype != torch.int64 or rank.shape != keys.shape:
            raise ValueError("rank must be int64 of keys' shape")
        N.require_device(rank, "rank")
    lib = N.load()
    out = torch.empty(2, dtype=torch.int64, device=keys.device)
    ws = _workspace(lib.zx_belady_argmax_workspace_bytes(keys.numel()), keys.device)
    N.check(lib.zx_belady_argmax(N.ptr(keys), N.ptr(resident), N.ptr(rank), keys.numel(), N.ptr(out), N.ptr(ws),
                                 ws.numel(), N.stream_ptr(keys.device)), "belady_argmax")
    return out


def next_use(trace: torch.Tensor, n_pages: int, check: bool = False):
    """Next/previous use of every position of an int32 page trace (ZX_NEVER / -1)."""
    N.ensure_gpu()
    if trace.dtype != torch.int32 or trace.dim() != 1:
        raise ValueError("trace must be a 1-D int32 tensor")
    N.require_device(trace, "trace")
    n = trace.numel()
    nu = torch.empty(n, dtype=torch.int32, device=trace.device)
    pu = torch.empty(n, dtype=torch.int32, device=trace.device)
    lib = N.load()
    ws = _workspace(lib.zx_belady_next_use_workspace_bytes(n, n_pages), trace.device)
    err = _err_word_if(check, trace.device)
    N.check(lib.zx_belady_next_use(N.ptr(trace), n, n_pages, N.ptr(nu), N.ptr(pu), N.ptr(err), N.ptr(ws),
                                   ws.numel(), N.stream_ptr(trace.device)), "belady_next_use")
    if check:
        _raise_kernel_error(err, "belady_next_use")
    return nu, pu


class BeladyTraceSim:
    """Belady MIN over an int32 page trace on the GPU (zx_belady_simulate).

    The cache state (resident flags, next-use keys, counters) lives in device tensors, so
    the trace can be processed in pieces with ``run(t_end)``; victims accumulate in
    ``evict_pos`` / ``evict_page`` (device int32, first ``n_evicted`` entries valid).
    """

    def __init__(self, trace: torch.Tensor, n_pages: int, capacity: int, evict_cap: int | None = None,
                 record_misses: bool = False):
        N.ensure_gpu()
        if trace.dtype != torch.int32 or trace.dim() != 1:
            raise ValueError("trace must be a 1-D int32 device tensor")
        if capacity < 1:
            raise ValueError("capacity must be >= 1")
        N.require_device(trace, "trace")
        dev = trace.device
        self.trace, self.n_pages, self.capacity = trace, int(n_pages), int(capacity)
        self.n_total = trace.numel()
        self.next_use, self.prev_use = next_use(trace, n_pages, check=True)
        self.resident = torch.zeros(self.n_pages, dtype=torch.uint8, device=dev)
        self.key = torch.full((self.n_pages,), N.ZX_NEVER, dtype=torch.int32, device=dev)
        self.state = torch.zeros(4, dtype=torch.int64, device=dev)
        cap = self.n_total if evict_cap is None else int(evict_cap)
        self.evict_cap = cap
        self.evict_pos = torch.empty(max(cap, 1), dtype=torch.int32, device=dev)
        self.evict_page = torch.empty(max(cap, 1), dtype=torch.int32, device=dev)
        self.miss_flags = torch.zeros(self.n_total, dtype=torch.uint8, device=dev) if record_misses else None
        lib = N.load()
        self._ws = _workspace(lib.zx_belady_simulate_workspace_bytes(self.n_total, self.n_pages), dev)
        self.t = 0

    def run(self, t_end: int | None = None) -> None:
        """Process trace positions [self.t, t_end) (default: to the end)."""
        t_end = self.n_total if t_end is None else int(t_end)
        if not self.t <= t_end <= self.n_total:
            raise ValueError(f"t_end must lie in [{self.t}, {self.n_total}]")
        N.check(N.load().zx_belady_simulate(
            N.ptr(self.trace), N.ptr(self.next_use), N.ptr(self.prev_use), self.n_total, self.t, t_end,
            self.n_pages, self.capacity, N.ptr(self.resident), N.ptr(self.key), N.ptr(self.state),
            N.ptr(self.evict_pos), N.ptr(self.evict_page), self.evict_cap, N.ptr(self.miss_flags),
            N.ptr(self._ws), self._ws.numel(), N.stream_ptr(self.trace.device)), "belady_simulate")
        self.t = t_end

    @property
    def n_evicted(self) -> int:
        return int(self.state[1].item())

    def stats(self) -> dict:
        s = self.state.tolist()
        return {"resident": s[0], "evictions": s[1], "misses": s[2], "hits": s[3]}

    def evictions(self):
        """(positions, pages) of the stored victims as CPU int32 tensors."""
        k = min(self.n_evicted, self.evict_cap)
        return self.evict_pos[:k].cpu(), self.evict_page[:k].cpu()


def ring_curriculum_trace(degrees, ctx_pages, n_layers: int, layer_stride: int,
                          device: torch.device | None = None) -> torch.Tensor:
    """Page trace of ring attention over training steps with per-step ring degree and
    pages per layer (zx_ring_curriculum_trace): a 1-D int32 device tensor, steps
    concatenated, each step's forward followed by its exact reverse."""
    import numpy as np

    deg = np.ascontiguousarray(degrees, dtype=np.int32)
    ctx = np.ascontiguousarray(ctx_pages, dtype=np.int32)
    if deg.ndim != 1 or deg.shape != ctx.shape:
        raise ValueError("degrees and ctx_pages must be 1-D of equal length")
    lib = N.load()
    n = lib.zx_ring_curriculum_trace_len(deg.ctypes.data, ctx.ctypes.data, deg.size, int(n_layers))
    if n < 0:
        raise ValueError("ring degrees and pages per layer must be >= 1, n_layers >= 1")
    dev = device or N.ensure_gpu()
    out = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    N.check(lib.zx_ring_curriculum_trace(deg.ctypes.data, ctx.ctypes.data, deg.size, int(n_layers),
                                         int(layer_stride), N.ptr(out), n, N.stream_ptr(dev)),
            "ring_curriculum_trace")
    return out[:n]


def tier_move_pages(dst: torch.Tensor, src: torch.Tensor, dst_offs: torch.Tensor, src_offs: torch.Tensor,
                    page_bytes: int, stream: torch.cuda.Stream | None = None, max_workgroups: int = 0,
                    err: torch.Tensor | None = None) -> None:
    """Enqueue ``dst[dst_offs[i] : +page_bytes] = src[src_offs[i] : +page_bytes]`` for every
    i with one kernel (zx_tier_move_pages).  ``dst``/``src`` are contiguous device or pinned
    host tensors; the offset tensors are int64, on the device or pinned, and must stay
    alive until the copy has run."""
    for t, name in ((dst_offs, "dst_offs"), (src_offs, "src_offs")):
        if t.dtype != torch.int64 or t.dim() != 1 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous 1-D int64 tensor")
        if not (t.is_cuda or t.is_pinned()):
            raise ValueError(f"{name} must be on the device or in pinned host memory")
    if dst_offs.numel() != src_offs.numel():
        raise ValueError("dst_offs and src_offs differ in length")
    for t, name in ((dst, "dst"), (src, "src")):
        if not t.is_contiguous() or not (t.is_cuda or t.is_pinned()):
            raise ValueError(f"{name} must be a contiguous device or pinned host tensor")
    dev = dst.device if dst.is_cuda else src.device
    st = stream if stream is not None else torch.cuda.current_stream(dev)
    N.check(N.load().zx_tier_move_pages(
        N.ptr(dst), dst.numel() * dst.element_size(), N.ptr(src), src.numel() * src.element_size(),
        N.ptr(dst_offs), N.ptr(src_offs), dst_offs.numel(), int(page_bytes), int(max_workgroups), N.ptr(err),
        ctypes.c_void_p(st.cuda_stream)), "tier_move_pages")


def belady_tier_plan(sim0: "BeladyTraceSim", sim01: "BeladyTraceSim", check: bool = False):
    """Three-tier schedule from two Belady runs over one trace (zx_belady_tier_plan):
    ``sim0`` with the T0 capacity, ``sim01`` with T0 + T1, both run to the end with
    ``record_misses=True``.  Returns device tensors (src uint8, v0 int32, v1 int32): per
    position the tier the accessed page came from (0 hit in T0, 1 from T1, 2 from T2,
    3 new), the page T0 evicts (-1: none; it goes to T1 unless v1 names it too) and the
    page T1 evicts to T2 (-1: none)."""
    for s in (sim0, sim01):
        if s.miss_flags is None or s.t != s.n_total:
            raise ValueError("both simulations must be run to the end with record_misses=True")
        if s.n_evicted > s.evict_cap:
            raise ValueError("an eviction list overflowed its capacity")
    if sim0.trace.data_ptr() != sim01.trace.data_ptr() or sim0.capacity > sim01.capacity:
        raise ValueError("sim0 and sim01 must share one trace, with sim0's capacity <= sim01's")
    dev = sim0.trace.device
    n = sim0.n_total
    src = torch.empty(n, dtype=torch.uint8, device=dev)
    v0 = torch.empty(n, dtype=torch.int32, device=dev)
    v1 = torch.empty(n, dtype=torch.int32, device=dev)
    err = _err_word_if(check, dev)
    N.check(N.load().zx_belady_tier_plan(
        N.ptr(sim0.prev_use), N.ptr(sim0.miss_flags), N.ptr(sim01.miss_flags), n,
        N.ptr(sim0.evict_pos), N.ptr(sim0.evict_page), sim0.n_evicted,
        N.ptr(sim01.evict_pos), N.ptr(sim01.evict_page), sim01.n_evicted,
        N.ptr(src), N.ptr(v0), N.ptr(v1), N.ptr(err), N.stream_ptr(dev)), "belady_tier_plan")
    if check:
        _raise_kernel_error(err, "belady_tier_plan")
    return src, v0, v1


def tier_copy_runs(dst: torch.Tensor, src: torch.Tensor, dst_offs, src_offs, run_bytes: int,
                   stream: torch.cuda.Stream | None = None) -> None:
    """Enqueue run copies ``dst[dst_offs[i] : +run_bytes] = src[src_offs[i] : +run_bytes]``
    (byte offsets into the two tensors' storage) on ``stream`` (default: the current one).
    One side is a device tensor, the other device or pinned host memory; adjacent runs are
    merged into one copy.  Replaces the ``.to(device)`` / ``.cpu()`` moves of
    kv_tiering.py:46, 54, 60."""
    import numpy as np

    d = np.ascontiguousarray(dst_offs, dtype=np.int64)
    s = np.ascontiguousarray(src_offs, dtype=np.int64)
    if d.shape != s.shape or d.ndim != 1:
        raise ValueError("dst_offs and src_offs must be 1-D of equal length")
    nb_d, nb_s = dst.numel() * dst.element_size(), src.numel() * src.element_size()
    if len(d) and (d.min() < 0 or s.min() < 0 or d.max() + run_bytes > nb_d or s.max() + run_bytes > nb_s):
        raise ValueError("run outside a buffer")
    if not (dst.is_contiguous() and src.is_contiguous()):
        raise ValueError("dst and src must be contiguous")
    dev = dst.device if dst.is_cuda else src.device
    st = stream if stream is not None else torch.cuda.current_stream(dev)
    lib = N.load()
    N.check(lib.zx_tier_copy_runs(N.ptr(dst), N.ptr(src), d.ctypes.data, s.ctypes.data, len(d), run_bytes,
                                  ctypes.c_void_p(st.cuda_stream), None), "tier_copy_runs")
