"""FP8 KV quantisation (README.md:157-159, 329, 344: ``FP8KVQuantizer``; the module the
README names, zenyx/train/fp8_kv_quantization.py, is absent from the reference tree, so
its behaviour is defined here and in include/zenyx_kv.h).

* ``FP8KVQuantizer`` -- e4m3fn codes with one fp32 scale per (layer, K/V, head):
  scale = max(amax, 1e-8) / 448, code = e4m3fn_RNE(x / scale), dequant = bf16_RNE(code * scale).
* ``PagedFP8KVCache`` -- a paged FP8 KV cache: page pool ``[L, n_pages, 2, H, P, D]``,
  host-side page allocator and block tables, fused quantize+append of new tokens and
  gather+dequant of whole sequences for decode.
* ``QuantizedRingAttention`` -- ring attention (and decode) over that cache, reading the
  FP8 pages directly.
All arithmetic runs in libzenyx_kv.so on the HIP device.
"""
from __future__ import annotations

import torch

from .. import _native as N
from .. import kv
from .._native import ensure_gpu


class FP8KVQuantizer:
    """Per-(layer, kv, head) dynamic FP8 e4m3fn quantisation of a KV cache tensor."""

    E4M3_MAX = 448.0
    compression_ratio = 2.0  # bf16 -> fp8

    def __init__(self, device: torch.device | None = None):
        self.device = device

    def quantize(self, kv_cache: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """kv_cache ``[L, 2, B, H, T, D]`` bf16 -> (codes uint8 same shape, scales ``[L, 2, H]`` fp32)."""
        if kv_cache.dim() != 6 or kv_cache.shape[1] != 2:
            raise ValueError("kv_cache must be [L, 2, B, H, T, D]")
        dev = self.device or ensure_gpu()
        x = kv_cache.to(dev).contiguous()
        L, _, B, H, T, D = x.shape
        codes, scales = kv.fp8_quant_heads(x.view(2 * L, B, H, T * D))
        return codes.view(x.shape), scales.view(L, 2, H)

    def dequantize(self, codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
        """Inverse of :meth:`quantize` -> bf16 ``[L, 2, B, H, T, D]``."""
        if codes.dim() != 6 or codes.shape[1] != 2:
            raise ValueError("codes must be [L, 2, B, H, T, D]")
        L, _, B, H, T, D = codes.shape
        y = kv.fp8_dequant_heads(codes.contiguous().view(2 * L, B, H, T * D),
                                 scales.contiguous().view(2 * L, H))
        return y.view(codes.shape)


class PagedFP8KVCache:
    """Paged FP8 KV cache with fused quantize+append and gather+dequant.

    The first append computes the per-(layer, kv, head) scales from its tokens (prefill);
    later appends reuse them (decode), so pages written earlier keep decoding with the
    scale they were encoded with.  A later token beyond 464 x its slab's scale does not fit
    e4m3: with ``overflow="raise"`` (default) it is stored as the NaN code, as the torch
    cast would, and the next checked call raises; with ``overflow="saturate"`` it is
    stored as +-448 and counted in ``saturated_appends``.  Kernel error bits (bad page ids,
    positions, overflow, a timed-out wait) accumulate in one device word, read without an
    extra synchronisation by the calls that synchronise anyway (``check_errors``, the
    attention calls, ``append(check=True)``)."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, num_pages: int,
                 page_size: int = 16, device: torch.device | None = None, overflow: str = "raise"):
        if overflow not in ("raise", "saturate"):
            raise ValueError('overflow must be "raise" or "saturate"')
        self.device = device or ensure_gpu()
        self.L, self.H, self.D, self.P = num_layers, num_kv_heads, head_dim, page_size
        self.num_pages = num_pages
        self.overflow = overflow
        self.pool = torch.zeros((num_layers, num_pages, 2, num_kv_heads, page_size, head_dim),
                                dtype=torch.uint8, device=self.device)
        self.scales = torch.ones((num_layers, 2, num_kv_heads), dtype=torch.float32, device=self.device)
        self.has_scales = False
        self.err = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.saturated_appends = 0
        self._free = list(range(num_pages - 1, -1, -1))
        self.pages: dict = {}    # seq id -> list of page ids
        self.lengths: dict = {}  # seq id -> tokens stored

    def _reserve(self, seq_id, new_len: int, taken: list) -> None:
        pages = self.pages.setdefault(seq_id, [])
        need = -(-new_len // self.P)
        while len(pages) < need:
            if not self._free:
                raise MemoryError("PagedFP8KVCache: out of pages")
            p = self._free.pop()
            pages.append(p)
            taken.append((seq_id, p))

    def _release(self, taken: list) -> None:
        for seq_id, p in reversed(taken):
            self.pages[seq_id].remove(p)
            if not self.pages[seq_id]:
                del self.pages[seq_id]
            self._free.append(p)

    def _tables(self, seq_ids) -> torch.Tensor:
        width = max(1, max(len(self.pages.get(s, [])) for s in seq_ids))
        rows = [self.pages.get(s, []) + [-1] * (width - len(self.pages.get(s, []))) for s in seq_ids]
        return torch.tensor(rows, dtype=torch.int32).to(self.device)

    def append(self, x: torch.Tensor, seq_ids: list, lengths: list[int], dynamic_scales: bool | None = None,
               check: bool = False):
        """Append new tokens of several sequences.  x: ``[L, n_tok, 2, H, D]`` bf16, tokens of
        sequence ``seq_ids[i]`` packed in order with ``lengths[i]`` tokens each.  Scales are
        computed from this batch on the first append and reused afterwards (static); asking
        for dynamic scales once pages hold tokens is refused, since it would change the
        scale of pages already written.  ``check`` synchronises and raises on any kernel
        error bit (see ``check_errors``)."""
        if sum(lengths) != x.shape[1]:
            raise ValueError("sum(lengths) must equal x.shape[1]")
        stored = any(n > 0 for n in self.lengths.values())
        dyn = (not self.has_scales) if dynamic_scales is None else dynamic_scales
        if dyn and stored:
            raise ValueError("dynamic scales on a cache that already holds tokens would re-scale pages written "
                             "with the old scales; free the sequences first")
        start = [self.lengths.get(s, 0) for s in seq_ids]
        taken: list = []
        try:
            for s, st, n in zip(seq_ids, start, lengths):
                self._reserve(s, st + n, taken)
            cu = [0]
            for n in lengths:
                cu.append(cu[-1] + n)
            kv.kv_quant_append(x.to(self.device), torch.tensor(cu, dtype=torch.int32).to(self.device),
                               self._tables(seq_ids), self.pool, scales=self.scales,
                               start_pos=torch.tensor(start, dtype=torch.int32).to(self.device),
                               static_scales=not dyn, saturate=(not dyn) and self.overflow == "saturate",
                               err=self.err)
        except BaseException:
            self._release(taken)
            raise
        self.has_scales = True
        for s, st, n in zip(seq_ids, start, lengths):
            self.lengths[s] = st + n
        if check:
            self.check_errors()
        return self.scales

    def check_errors(self) -> None:
        """Read (and clear) the cache's device error word; raise ValueError for any bit, except
        an overflow in ``overflow="saturate"`` mode, which only counts ``saturated_appends``.
        Synchronises with the cache's device."""
        e = int(self.err.item())
        if not e:
            return
        self.err.zero_()
        if self.overflow == "saturate" and e & N.ZX_KERR_OVERFLOW:
            self.saturated_appends += 1
            e &= ~N.ZX_KERR_OVERFLOW
        if e:
            raise ValueError("PagedFP8KVCache: " + kv.kernel_error_text(e))

    def gather(self, layer: int, seq_ids: list, out_len: int | None = None):
        """bf16 ``(k, v)``, each ``[B, H, out_len, D]``, of one layer for decode; positions past a
        sequence's length are zeros."""
        lens = torch.tensor([self.lengths.get(s, 0) for s in seq_ids], dtype=torch.int32).to(self.device)
        bt = self._tables(seq_ids)
        if out_len is None:
            out_len = max(1, max(self.lengths.get(s, 0) for s in seq_ids))
        return kv.kv_gather_dequant(self.pool[layer], self.scales[layer].contiguous(), bt, lens, out_len)

    def free(self, seq_id) -> None:
        for p in self.pages.pop(seq_id, []):
            self._free.append(p)
        self.lengths.pop(seq_id, None)


class QuantizedRingAttention:
    """Ring attention over a paged FP8 KV cache.  README.md:344 imports it beside
    ``FP8KVQuantizer``; its code is absent from the reference, so the behaviour is defined
    here.  The cached keys of each sequence are split into ``ring_degree`` shards (the KV
    blocks a ring passes between devices); each shard is one ring step that attends the
    queries to it straight from the FP8 pages (no bf16 copy of K/V) and merges by
    log-sum-exp into a running fp32 output, so the result is softmax(sm_scale q K^T) V over
    all cached keys (causal: keys up to each query's position).  On one GPU the steps run
    in sequence.  ``decode`` is the one-token case (split-K decode kernel)."""

    def __init__(self, cache: PagedFP8KVCache, ring_degree: int = 8, causal: bool = True,
                 sm_scale: float | None = None, precision: str = "f16"):
        if ring_degree < 1:
            raise ValueError("ring_degree must be >= 1")
        self.cache = cache
        self.ring_degree = ring_degree
        self.causal = causal
        self.sm_scale = sm_scale
        if precision not in kv.PRECISIONS:
            raise ValueError(f"precision must be one of {kv.PRECISIONS}")
        self.precision = precision  # how the softmax weights enter P.V (kv.PRECISIONS)

    def __call__(self, q: torch.Tensor, layer: int, seq_ids: list, q_lens: list[int]) -> torch.Tensor:
        """q ``[n_q, Hq, D]`` bf16: the queries of ``seq_ids[i]`` packed in order, ``q_lens[i]``
        rows each, standing for that sequence's newest ``q_lens[i]`` cached tokens (the
        tokens just appended, as in prefill).  Returns bf16 ``[n_q, Hq, D]``."""
        c = self.cache
        if len(q_lens) != len(seq_ids) or sum(q_lens) != q.shape[0]:
            raise ValueError("q_lens must give the row count of every sequence in seq_ids, summing to q.shape[0]")
        lens = [c.lengths.get(s, 0) for s in seq_ids]
        if any(n > m for n, m in zip(q_lens, lens)):
            raise ValueError("a sequence has more query rows than cached tokens")
        cu = [0]
        for n in q_lens:
            cu.append(cu[-1] + n)
        dev = c.device
        out = kv.ring_attention_fp8(
            q.to(dev).contiguous(), torch.tensor(cu, dtype=torch.int32).to(dev),
            torch.tensor([m - n for n, m in zip(q_lens, lens)], dtype=torch.int32).to(dev), c.pool[layer],
            c.scales[layer].contiguous(), c._tables(seq_ids), torch.tensor(lens, dtype=torch.int32).to(dev),
            ring_degree=self.ring_degree, causal=self.causal, sm_scale=self.sm_scale, check=True,
            precision=self.precision, max_q_per_seq=max(q_lens, default=0))
        c.check_errors()  # the appends behind these pages (the check above has synchronised)
        return out

    def decode(self, q: torch.Tensor, layer: int, seq_ids: list) -> torch.Tensor:
        """q ``[B, Hq, D]`` bf16, one query token per sequence over all its cached tokens."""
        c = self.cache
        lens = torch.tensor([c.lengths.get(s, 0) for s in seq_ids], dtype=torch.int32).to(c.device)
        out = kv.paged_attention_decode(q.to(c.device).contiguous(), c.pool[layer], c.scales[layer].contiguous(),
                                        c._tables(seq_ids), lens, sm_scale=self.sm_scale, check=True)
        c.check_errors()
        return out


__all__ = ["FP8KVQuantizer", "PagedFP8KVCache", "QuantizedRingAttention"]
