"""CPU oracle for the zenyx KV-cache hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of bench.py may
import this module; it is the checker, never the thing measured or shipped.  The product
(``zenyx_amd``) does not import it and has no CPU fallback.

Two layers:

* numpy wrappers over ``libzx_oracle.so`` (built from ``oracle/zx_oracle.c`` by
  ``oracle/Makefile``), the fast restatement used at realistic sizes;
* pure-Python restatements for tiny inputs that follow the reference line by line:
  ``RefBeladyApproxCache`` (zenyx/streaming/belady.py:14-55), ``ref_belady_trace``
  (the same per-miss linear argmax, belady.py:39-51, driven over a page trace) and
  ``ref_ring_timeline`` (zenyx/streaming/kv_tiering.py:69-73).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libzx_oracle.so")
NEVER = 0x7FFFFFFF

_lib = None


def lib() -> ctypes.CDLL:
    """Load (building first if needed) the C oracle."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            import subprocess

            subprocess.run(["make", "-s", "-C", _HERE], check=True)
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i64, i32, f32 = ctypes.c_int64, ctypes.c_int32, ctypes.c_float
        sig = {
            "zxo_e4m3_encode_array": (None, [P, P, i64]),
            "zxo_e4m3_decode_array": (None, [P, P, i64]),
            "zxo_bf16_rne_array": (None, [P, P, i64]),
            "zxo_f16_rne_array": (None, [P, P, i64]),
            "zxo_fp8_scale": (f32, [f32]),
            "zxo_fp8_quant_heads": (None, [P, i64, i64, i64, i64, P, P]),
            "zxo_fp8_dequant_heads": (None, [P, P, i64, i64, i64, i64, P]),
            "zxo_kv_scales": (None, [P, i64, i32, i64, i32, i32, P]),
            "zxo_kv_quant_append": (i32, [P, i64, i32, i64, i32, i32, P, P, i32, P, i32, i32,
                                          P, i64, i64, P, i32]),
            "zxo_kv_gather_dequant": (i32, [P, i64, i32, i32, i32, P, P, i32, P, i32, i32, P, P]),
            "zxo_int8_legacy_quant": (f32, [P, ctypes.c_int, i64, P]),
            "zxo_int8_legacy_dequant": (None, [P, f32, i64, P]),
            "zxo_belady_argmax": (None, [P, P, P, i64, P]),
            "zxo_next_use": (None, [P, i64, i32, P, P]),
            "zxo_belady_simulate": (i64, [P, i64, i32, i64, P, P, i64, P, P]),
            "zxo_belady_tiers": (i64, [P, i64, i32, i64, i64, P, P, P]),
            "zxo_ring_curriculum_trace": (i64, [P, P, i32, i32, i32, P]),
            "zxo_ring_trace": (None, [i32, i32, i32, P]),
            "zxo_paged_attention_decode": (i32, [P, i32, P, i64, i32, i32, i32, P, P, i32, P, i32, f32, P]),
            "zxo_paged_attention_prefill": (i32, [P, P, P, i32, P, i64, i32, i32, i32, P, P, i32, P, P, i32, i32,
                                                  f32, P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


# ------------------------------------------------------------------ scalar formats

def e4m3_encode(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().zxo_e4m3_encode_array(_p(x), _p(out), x.size)
    return out


def e4m3_decode(c) -> np.ndarray:
    c = np.ascontiguousarray(c, dtype=np.uint8)
    out = np.empty(c.shape, np.float32)
    lib().zxo_e4m3_decode_array(_p(c), _p(out), c.size)
    return out


def bf16_rne(x) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), nearest-even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().zxo_bf16_rne_array(_p(x), _p(out), x.size)
    return out


def f16_rne(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().zxo_f16_rne_array(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def fp8_scale(amax: float) -> float:
    return float(np.float32(lib().zxo_fp8_scale(float(amax))))


# ------------------------------------------------------------------ FP8 per head

def fp8_quant_heads(x_bits: np.ndarray):
    """x_bits: bf16 bit patterns [n_outer, n_batch, n_heads, run] -> (codes, scales)."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    n_outer, n_batch, n_heads, run = x_bits.shape
    codes = np.empty(x_bits.shape, np.uint8)
    scales = np.empty((n_outer, n_heads), np.float32)
    lib().zxo_fp8_quant_heads(_p(x_bits), n_outer, n_batch, n_heads, run, _p(codes), _p(scales))
    return codes, scales


def fp8_dequant_heads(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    n_outer, n_batch, n_heads, run = codes.shape
    y = np.empty(codes.shape, np.uint16)
    lib().zxo_fp8_dequant_heads(_p(codes), _p(scales), n_outer, n_batch, n_heads, run, _p(y))
    return y


# ------------------------------------------------------------------ paged KV

def kv_scales(x_bits: np.ndarray) -> np.ndarray:
    """x_bits: [L, n_tok, 2, H, D] bf16 bits -> scales [L, 2, H]."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    L, n_tok, _, H, D = x_bits.shape
    scales = np.empty((L, 2, H), np.float32)
    lib().zxo_kv_scales(_p(x_bits), n_tok * 2 * H * D, L, n_tok, H, D, _p(scales))
    return scales


def kv_quant_append(x_bits, cu_seqlens, start_pos, block_tables, pool, page_size,
                    scales=None, saturate=False):
    """In-place paged append into pool [L, n_pages, 2, H, P, D]; returns (scales, err).
    With ``scales`` given they are static; ``saturate`` then stores overflowing finite
    inputs as +-448 instead of the NaN code (err bit 8 is set either way)."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    L, n_tok, _, H, D = x_bits.shape
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    sp = None if start_pos is None else np.ascontiguousarray(start_pos, dtype=np.int32)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    assert pool.flags["C_CONTIGUOUS"] and pool.dtype == np.uint8
    n_pages = pool.shape[1]
    static = scales is not None
    sc = np.ascontiguousarray(scales, np.float32).copy() if static else np.empty((L, 2, H), np.float32)
    err = lib().zxo_kv_quant_append(_p(x_bits), n_tok * 2 * H * D, L, n_tok, H, D, _p(cu), _p(sp),
                                    len(cu) - 1, _p(bt), bt.shape[1], page_size, _p(pool),
                                    pool[0].size, n_pages, _p(sc), int(static) | (4 if saturate and static else 0))
    return sc, int(err)


def kv_quant_append_torch(x, cu_seqlens, block_tables, n_pages, page_size):
    """The paged append of one layer restated in torch on the CPU (the multi-threaded CPU
    baseline; same results as zxo_kv_quant_append, checked in tests/test_oracle.py):
    x bf16 [n_tok, 2, H, D] (CPU tensor) -> (scales fp32 [2, H], pool uint8 [n_pages, 2, H, P, D])
    with scale = max(amax, 1e-8) / 448 per (kv, head) and the e4m3 codes of x / scale at
    page block_tables[b, pos // P], slot pos % P."""
    import torch

    n_tok, _, H, D = x.shape
    cu = torch.as_tensor(np.asarray(cu_seqlens), dtype=torch.int64)
    lens = cu[1:] - cu[:-1]
    tok_b = torch.repeat_interleave(torch.arange(len(lens)), lens)
    pos = torch.arange(n_tok) - cu[:-1][tok_b]
    bt = torch.as_tensor(np.asarray(block_tables), dtype=torch.int64)
    page, slot = bt[tok_b, pos // page_size], pos % page_size
    xf = x.float()
    sc = xf.abs().amax(dim=(0, 3)).clamp_min(1e-8) / 448.0
    codes = (xf / sc[None, :, :, None]).to(torch.float8_e4m3fn).view(torch.uint8)
    pool = torch.zeros((n_pages, 2, H, page_size, D), dtype=torch.uint8)
    pool[page, :, :, slot, :] = codes
    return sc, pool


def kv_gather_dequant_torch(pool_layer, scales_layer, block_tables, seq_lens, out_len):
    """The paged gather + dequant of one layer restated in torch on the CPU (the
    multi-threaded CPU baseline; same results as zxo_kv_gather_dequant): -> (k, v) bf16
    [B, H, out_len, D], zeros past each sequence's length."""
    import torch

    n_pages, _, H, P, D = pool_layer.shape
    bt = torch.as_tensor(np.asarray(block_tables), dtype=torch.int64)
    B = bt.shape[0]
    k = torch.zeros((B, H, out_len, D), dtype=torch.bfloat16)
    v = torch.zeros((B, H, out_len, D), dtype=torch.bfloat16)
    for b in range(B):
        n = min(int(seq_lens[b]), out_len)
        t = torch.arange(n)
        codes = pool_layer[bt[b, t // P], :, :, t % P, :]  # [n, 2, H, D]
        vals = (codes.view(torch.float8_e4m3fn).float() * scales_layer[None, :, :, None]).to(torch.bfloat16)
        k[b, :, :n] = vals[:, 0].transpose(0, 1)
        v[b, :, :n] = vals[:, 1].transpose(0, 1)
    return k, v


def kv_gather_dequant(pool_layer, scales_layer, block_tables, seq_lens, out_len):
    """pool_layer [n_pages, 2, H, P, D] -> (k, v) bf16 bits [B, H, out_len, D], err."""
    pool_layer = np.ascontiguousarray(pool_layer, dtype=np.uint8)
    n_pages, _, H, P, D = pool_layer.shape
    sc = np.ascontiguousarray(scales_layer, dtype=np.float32)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    B = len(sl)
    k = np.empty((B, H, out_len, D), np.uint16)
    v = np.empty((B, H, out_len, D), np.uint16)
    err = lib().zxo_kv_gather_dequant(_p(pool_layer), n_pages, H, D, P, _p(sc), _p(bt), bt.shape[1],
                                      _p(sl), B, out_len, _p(k), _p(v))
    return k, v, int(err)


# ------------------------------------------------------------------ legacy int8

_DT = {"bf16": 0, "f16": 1, "f32": 2}


def paged_attention_decode(q_bits, pool_layer, scales_layer, block_tables, seq_lens, sm_scale):
    """q_bits [B, Hq, D] bf16 bits; pool_layer [n_pages, 2, Hkv, P, D] -> (out bits [B, Hq, D], err)."""
    q_bits = np.ascontiguousarray(q_bits, dtype=np.uint16)
    pool_layer = np.ascontiguousarray(pool_layer, dtype=np.uint8)
    n_pages, _, Hkv, P, D = pool_layer.shape
    B, Hq, _ = q_bits.shape
    sc = np.ascontiguousarray(scales_layer, dtype=np.float32)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    out = np.empty((B, Hq, D), np.uint16)
    err = lib().zxo_paged_attention_decode(_p(q_bits), Hq, _p(pool_layer), n_pages, Hkv, D, P, _p(sc), _p(bt),
                                           bt.shape[1], _p(sl), B, float(sm_scale), _p(out))
    return out, int(err)


def paged_attention_prefill(q_bits, cu_q, q_pos0, pool_layer, scales_layer, block_tables, kv_begin, kv_end,
                            causal: bool, sm_scale: float):
    """Block attention over the FP8 pages; q_bits [n_q, Hq, D] uint16.  Returns
    (out bf16 bits [n_q, Hq, D], lse2 float32 [n_q, Hq], error bits)."""
    q_bits = np.ascontiguousarray(q_bits, dtype=np.uint16)
    pool_layer = np.ascontiguousarray(pool_layer, dtype=np.uint8)
    n_q, Hq, D = q_bits.shape
    n_pages, _, Hkv, P, _ = pool_layer.shape
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cu = np.ascontiguousarray(cu_q, dtype=np.int32)
    out = np.zeros_like(q_bits)
    lse = np.empty((n_q, Hq), np.float32)
    err = lib().zxo_paged_attention_prefill(
        _p(q_bits), _p(cu), _p(np.ascontiguousarray(q_pos0, dtype=np.int32)), Hq, _p(pool_layer), n_pages, Hkv, D,
        P, _p(np.ascontiguousarray(scales_layer, dtype=np.float32)), _p(bt), bt.shape[1],
        _p(np.ascontiguousarray(kv_begin, dtype=np.int32)), _p(np.ascontiguousarray(kv_end, dtype=np.int32)),
        cu.size - 1, int(causal), sm_scale, _p(out), _p(lse))
    return out, lse, int(err)


def int8_legacy_quant(x: np.ndarray, dtype: str):
    """x: bit patterns (uint16) for bf16/f16 or float32 values -> (q int8, scale float)."""
    x = np.ascontiguousarray(x)
    q = np.empty(x.shape, np.int8)
    s = lib().zxo_int8_legacy_quant(_p(x), _DT[dtype], x.size, _p(q))
    return q, float(np.float32(s))


def legacy_reciprocal_check(dtype: str, scale_stride: int = 1):
    """(mismatching codes, pairs compared) of the reciprocal + Markstein quotient against
    IEEE division for the legacy quantiser (zxo_legacy_reciprocal_check)."""
    L = lib()
    L.zxo_legacy_reciprocal_check.restype = ctypes.c_int64
    L.zxo_legacy_reciprocal_check.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_int64)]
    pairs = ctypes.c_int64(0)
    bad = L.zxo_legacy_reciprocal_check(_DT[dtype], int(scale_stride), ctypes.byref(pairs))
    return int(bad), int(pairs.value)


def legacy_fast_check(dtype: str, scale_stride: int = 1):
    """(mismatching codes, pairs compared) of the GPU's fast legacy encoder (reciprocal +
    Markstein, no range guard, integer rounding by adding 1.5 * 2^23) against the reference
    code, over every reachable (scale, x) pair (zxo_legacy_fast_check)."""
    L = lib()
    L.zxo_legacy_fast_check.restype = ctypes.c_int64
    L.zxo_legacy_fast_check.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_int64)]
    pairs = ctypes.c_int64(0)
    bad = L.zxo_legacy_fast_check(_DT[dtype], int(scale_stride), ctypes.byref(pairs))
    return int(bad), int(pairs.value)


def fp8_product_check(scale_stride: int = 1):
    """(differing codes, pairs compared) of e4m3(x * RN(1 / s)) against e4m3(x / s) over
    dynamic scales s = amax / 448 and |x| <= amax (zxo_fp8_product_check)."""
    L = lib()
    L.zxo_fp8_product_check.restype = ctypes.c_int64
    L.zxo_fp8_product_check.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_int64)]
    pairs = ctypes.c_int64(0)
    bad = L.zxo_fp8_product_check(int(scale_stride), ctypes.byref(pairs))
    return int(bad), int(pairs.value)


def int8_legacy_dequant(q: np.ndarray, scale: float) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int8)
    y = np.empty(q.shape, np.uint16)
    lib().zxo_int8_legacy_dequant(_p(q), float(scale), q.size, _p(y))
    return y


# ------------------------------------------------------------------ Belady

def belady_argmax(keys: np.ndarray, resident: np.ndarray | None, rank: np.ndarray | None = None):
    keys = np.ascontiguousarray(keys, dtype=np.int64)
    if resident is not None:
        resident = np.ascontiguousarray(resident, dtype=np.uint8)
    if rank is not None:
        rank = np.ascontiguousarray(rank, dtype=np.int64)
    out = np.empty(2, np.int64)
    lib().zxo_belady_argmax(_p(keys), _p(resident), _p(rank), keys.size, _p(out))
    return int(out[0]), int(out[1])


def next_use(trace: np.ndarray, n_pages: int):
    trace = np.ascontiguousarray(trace, dtype=np.int32)
    nu = np.empty(trace.size, np.int32)
    pu = np.empty(trace.size, np.int32)
    lib().zxo_next_use(_p(trace), trace.size, n_pages, _p(nu), _p(pu))
    return nu, pu


def belady_simulate(trace: np.ndarray, n_pages: int, capacity: int, evict_cap: int | None = None,
                    miss_flags: bool = False):
    """Heap-based Belady MIN; returns (evict_pos, evict_page, stats{misses,hits,resident}
    [, miss_flags])."""
    trace = np.ascontiguousarray(trace, dtype=np.int32)
    cap = trace.size if evict_cap is None else evict_cap
    ep = np.empty(max(cap, 1), np.int32)
    eg = np.empty(max(cap, 1), np.int32)
    stats = np.zeros(3, np.int64)
    mf = np.zeros(trace.size, np.uint8) if miss_flags else None
    n_ev = lib().zxo_belady_simulate(_p(trace), trace.size, n_pages, capacity, _p(ep), _p(eg),
                                     cap, _p(stats), _p(mf))
    k = min(n_ev, cap)
    out = (ep[:k].copy(), eg[:k].copy(), {"evictions": int(n_ev), "misses": int(stats[0]),
                                          "hits": int(stats[1]), "resident": int(stats[2])})
    return out + (mf,) if miss_flags else out


def belady_tiers(trace: np.ndarray, n_pages: int, c0: int, c1: int):
    """Explicit three-tier Belady hierarchy (two heaps); returns (src uint8, v0 int32,
    v1 int32, T0 misses): per access the tier the page came from (0 hit in T0, 1 from T1,
    2 from T2, 3 new), the page T0 evicted to T1 and the page T1 evicted to T2 (-1: none)."""
    trace = np.ascontiguousarray(trace, dtype=np.int32)
    src = np.empty(trace.size, np.uint8)
    v0 = np.empty(trace.size, np.int32)
    v1 = np.empty(trace.size, np.int32)
    m = lib().zxo_belady_tiers(_p(trace), trace.size, n_pages, c0, c1, _p(src), _p(v0), _p(v1))
    return src, v0, v1, int(m)


def ring_curriculum_trace(degrees, ctx_pages, n_layers: int, layer_stride: int) -> np.ndarray:
    """Concatenated ring traces of training steps with per-step degree and pages per layer."""
    deg = np.ascontiguousarray(degrees, dtype=np.int32)
    ctx = np.ascontiguousarray(ctx_pages, dtype=np.int32)
    n = int(np.sum(2 * n_layers * deg.astype(np.int64) * ctx))
    out = np.empty(max(n, 1), np.int32)
    k = lib().zxo_ring_curriculum_trace(_p(deg), _p(ctx), deg.size, n_layers, layer_stride, _p(out))
    assert k == n
    return out[:n]


def ring_trace(n_layers: int, ring: int, shard_pages: int) -> np.ndarray:
    out = np.empty(2 * n_layers * ring * ring * shard_pages, np.int32)
    lib().zxo_ring_trace(n_layers, ring, shard_pages, _p(out))
    return out


# ------------------------------------------------------------------ pure-Python restatements

class RefBeladyApproxCache:
    """Line-by-line restatement of zenyx/streaming/belady.py:14-55.

    The one liberty: the reference iterates a ``set`` in ``_select_victim`` (belady.py:46),
    whose order Python does not fix, so ties on the farthest next use are broken here by
    first registration order of the id (the order the drop-in assigns slots in).
    """

    def __init__(self, capacity: int):
        self.capacity = capacity
        self._resident: dict = {}  # insertion-ordered set
        self._next_use: dict = {}
        self._order: dict = {}

    def _reg(self, tid):
        if tid not in self._order:
            self._order[tid] = len(self._order)

    def update_future(self, tensor_id, next_use_step: int) -> None:  # belady.py:22-23
        self._reg(tensor_id)
        self._next_use[tensor_id] = next_use_step

    def touch(self, tensor_id) -> list:  # belady.py:25-37
        self._reg(tensor_id)
        evicted = []
        if tensor_id in self._resident:
            return evicted
        if len(self._resident) >= self.capacity:
            victim = self._select_victim()
            if victim is not None:
                del self._resident[victim]
                evicted.append(victim)
        self._resident[tensor_id] = True
        return evicted

    def _select_victim(self):  # belady.py:39-51
        if not self._resident:
            return None
        victim = None
        farthest = -1
        for tid in sorted(self._resident, key=lambda t: self._order[t]):
            nxt = self._next_use.get(tid, 10**18)
            if nxt > farthest:
                farthest = nxt
                victim = tid
        return victim

    @property
    def resident(self) -> set:
        return set(self._resident)


def ref_belady_trace(trace, capacity: int):
    """Belady over a page trace with the reference's per-miss linear scan.

    For each access: next_use of the page is set to its next position in the trace
    (belady.py:22-23 driven with true future knowledge, never-again = 10**18 as in
    belady.py:47), then ``touch`` (belady.py:25-37).  Ties go to the smallest page id.
    Returns the list of (position, victim) pairs.  O(n * capacity): tiny inputs only.
    """
    trace = [int(p) for p in trace]
    n = len(trace)
    nxt = [10**18] * n
    last = {}
    for i in range(n - 1, -1, -1):
        nxt[i] = last.get(trace[i], 10**18)
        last[trace[i]] = i
    resident = set()
    next_use = {}
    out = []
    for i, p in enumerate(trace):
        next_use[p] = nxt[i]
        if p in resident:
            continue
        if len(resident) >= capacity and resident:
            victim, far = None, -1
            for q in sorted(resident):
                if next_use[q] > far:
                    far, victim = next_use[q], q
            resident.discard(victim)
            out.append((i, victim))
        resident.add(p)
    return out


def ref_ring_timeline(num_blocks: int) -> dict:
    """zenyx/streaming/kv_tiering.py:69-73."""
    forward = list(range(num_blocks))
    return {"forward": forward, "backward": list(reversed(forward))}
