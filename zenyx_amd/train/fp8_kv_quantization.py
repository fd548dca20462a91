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

    def quantize(self, kv_cache: torch.Tensor, check: bool | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """kv_cache ``[L, 2, B, H, T, D]`` bf16 -> (codes uint8 same shape, scales ``[L, 2, H]`` fp32).

        ``check`` (default: whenever the input is large enough for the library's
        single-pass kernel, 256 MiB and up) passes an error word, synchronises and raises
        ValueError if the kernel reported an error; the single pass's workgroups wait for
        each other, and a wait that runs out leaves the outputs undefined."""
        if kv_cache.dim() != 6 or kv_cache.shape[1] != 2:
            raise ValueError("kv_cache must be [L, 2, B, H, T, D]")
        dev = self.device or ensure_gpu()
        x = kv_cache.to(dev).contiguous()
        L, _, B, H, T, D = x.shape
        if check is None:
            check = x.numel() * x.element_size() >= kv.HEADS_SINGLE_PASS_BYTES
        codes, scales = kv.fp8_quant_heads(x.view(2 * L, B, H, T * D), check=check)
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
    stored as +-448 and ``saturated_appends`` counts the appends that stored at least one
    such token.  Each append ORs its kernel error bits (bad page ids, positions, overflow,
    a timed-out wait) into a device word of its own; the calls that synchronise anyway
    (``check_errors``, the attention calls, ``append(check=True)``) read them.  An append
    found faulty by an unchecked append's later check stays stored; ``append(check=True)``
    undoes its own faulty append (lengths, pages, scales) before raising."""

    _ERR_WORDS = 64

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
        # one error word per append since the last check (a ring; a full ring is checked
        # before it is reused), so saturation is counted per append
        self._err = torch.zeros(self._ERR_WORDS, dtype=torch.int32, device=self.device)
        self._n_err = 0
        self.saturated_appends = 0
        self._free = list(range(num_pages - 1, -1, -1))
        self.pages: dict = {}    # seq id -> list of page ids
        self.lengths: dict = {}  # seq id -> tokens stored
        # Device-resident block tables: one row per live sequence (rows are reused after
        # free), -1 past its pages, and each row's length.  Reserving pages writes only the
        # new entries; a call gathers its sequences' rows on the device, so host work per
        # call is O(sequences in the call), not O(pages).
        self._row: dict = {}  # seq id -> row
        self._free_rows: list = []
        self._bt = torch.full((16, 64), -1, dtype=torch.int32, device=self.device)
        self._len = torch.zeros(16, dtype=torch.int32, device=self.device)
        self._rows_cache: tuple = ((), None)  # (seq_ids, device int64 rows) of the last call
        self._ones_cache: dict = {}  # n -> device int32 ones [n] / arange [n + 1] (one-token steps)

    # ---------------------------------------------------------------- block tables

    def _row_of(self, seq_id) -> int:
        r = self._row.get(seq_id)
        if r is None:
            r = self._free_rows.pop() if self._free_rows else len(self._row)
            if r >= self._bt.shape[0]:
                self._grow(rows=max(2 * self._bt.shape[0], r + 1))
            self._row[seq_id] = r
        return r

    def _grow(self, rows: int | None = None, width: int | None = None) -> None:
        old = self._bt
        rows = rows or old.shape[0]
        width = width or old.shape[1]
        bt = torch.full((rows, width), -1, dtype=torch.int32, device=self.device)
        bt[:old.shape[0], :old.shape[1]].copy_(old)
        self._bt = bt
        if rows > self._len.shape[0]:
            ln = torch.zeros(rows, dtype=torch.int32, device=self.device)
            ln[:self._len.shape[0]].copy_(self._len)
            self._len = ln

    def _write_entries(self, entries: list) -> None:
        """entries: (row, column, page id or -1) -> the device tables (one small upload)."""
        if not entries:
            return
        width = max(c for _, c, _ in entries) + 1
        if width > self._bt.shape[1]:
            self._grow(width=max(2 * self._bt.shape[1], width))
        t = torch.tensor(entries, dtype=torch.int64).t().contiguous().to(self.device)
        self._bt.index_put_((t[0], t[1]), t[2].to(torch.int32))

    def _rows(self, seq_ids) -> torch.Tensor:
        """Device int64 row indices of seq_ids (cached for a repeated batch)."""
        key = tuple(seq_ids)
        if self._rows_cache[0] != key:
            rows = torch.tensor([self._row_of(s) for s in seq_ids], dtype=torch.int64).to(self.device)
            self._rows_cache = (key, rows)
        return self._rows_cache[1]

    def _tables(self, seq_ids) -> torch.Tensor:
        """Device int32 ``[len(seq_ids), width]`` block tables of seq_ids, -1 past their pages;
        width = the most pages any of them holds (the kernels size their work by it)."""
        width = max(1, max(len(self.pages.get(s, ())) for s in seq_ids))
        return self._bt[:, :width].index_select(0, self._rows(seq_ids))

    def _lengths(self, seq_ids) -> torch.Tensor:
        """Device int32 tokens stored per sequence of seq_ids."""
        return self._len.index_select(0, self._rows(seq_ids))

    def _counts(self, lengths: list) -> tuple:
        """Device (int32 [B] token counts, int32 [B + 1] cu_seqlens) of an append."""
        n = len(lengths)
        if all(v == 1 for v in lengths):  # a decode step: cached
            c = self._ones_cache.get(n)
            if c is None:
                c = (torch.ones(n, dtype=torch.int32, device=self.device),
                     torch.arange(n + 1, dtype=torch.int32, device=self.device))
                self._ones_cache[n] = c
            return c
        cu = [0]
        for v in lengths:
            cu.append(cu[-1] + v)
        w = (n + 4) // 4 * 4  # rows padded to 16 bytes: each part starts 16-byte aligned
        t = torch.tensor([list(lengths) + [0] * (w - n), cu + [0] * (w - n - 1)], dtype=torch.int32).to(self.device)
        return t[0, :n], t[1, :n + 1]

    def _reserve(self, seq_id, new_len: int, taken: list, entries: list) -> None:
        pages = self.pages.setdefault(seq_id, [])
        need = -(-new_len // self.P)
        row = self._row_of(seq_id) if len(pages) < need else None
        while len(pages) < need:
            if not self._free:
                raise MemoryError("PagedFP8KVCache: out of pages")
            p = self._free.pop()
            entries.append((row, len(pages), p))
            pages.append(p)
            taken.append((seq_id, p))

    def _release(self, taken: list) -> None:
        """Return pages just reserved (newest first) to the free list; their table entries
        go back to -1 and rows left without pages or tokens are freed."""
        entries = []
        for seq_id, p in reversed(taken):
            pages = self.pages[seq_id]
            entries.append((self._row[seq_id], len(pages) - 1, -1))
            pages.pop()
            if not pages:
                del self.pages[seq_id]
            self._free.append(p)
        self._write_entries(entries)
        for seq_id in {s for s, _ in taken}:
            if seq_id not in self.pages and not self.lengths.get(seq_id):
                self._drop_row(seq_id)

    def _drop_row(self, seq_id) -> None:
        r = self._row.pop(seq_id, None)
        if r is None:
            return
        self._bt[r].fill_(-1)
        self._len[r] = 0
        self._free_rows.append(r)
        self._rows_cache = ((), None)

    # ---------------------------------------------------------------- API

    def append(self, x: torch.Tensor, seq_ids: list, lengths: list[int], dynamic_scales: bool | None = None,
               check: bool = False, single_pass: bool = False):
        """Append new tokens of several sequences.  x: ``[L, n_tok, 2, H, D]`` bf16, tokens of
        sequence ``seq_ids[i]`` packed in order with ``lengths[i]`` tokens each.  Scales are
        computed from this batch on the first append and reused afterwards (static); asking
        for dynamic scales once pages hold tokens is refused, since it would change the
        scale of pages already written.  ``check`` synchronises and raises on any kernel
        error bit (see ``check_errors``).  ``single_pass`` makes dynamic scales take the
        cooperative single pass whatever the batch's size (kv.kv_quant_append)."""
        if len(lengths) != len(seq_ids) or len(set(seq_ids)) != len(seq_ids):
            raise ValueError("seq_ids must be distinct, one per entry of lengths")
        if sum(lengths) != x.shape[1]:
            raise ValueError("sum(lengths) must equal x.shape[1]")
        stored = any(n > 0 for n in self.lengths.values())
        dyn = (not self.has_scales) if dynamic_scales is None else dynamic_scales
        if dyn and stored:
            raise ValueError("dynamic scales on a cache that already holds tokens would re-scale pages written "
                             "with the old scales; free the sequences first")
        if check or self._n_err == self._ERR_WORDS:
            self.check_errors()  # earlier appends first, so the word read below is this call's own
        start = [self.lengths.get(s, 0) for s in seq_ids]
        word = self._err[self._n_err:self._n_err + 1]
        had_scales = self.has_scales
        taken: list = []
        try:
            entries: list = []
            for s, st, n in zip(seq_ids, start, lengths):
                self._reserve(s, st + n, taken, entries)
            self._write_entries(entries)
            counts, cu = self._counts(lengths)
            rows = self._rows(seq_ids)
            kv.kv_quant_append(x.to(self.device), cu, self._tables(seq_ids), self.pool, scales=self.scales,
                               start_pos=self._len.index_select(0, rows),
                               static_scales=not dyn, saturate=(not dyn) and self.overflow == "saturate",
                               err=word, single_pass=single_pass and dyn)
        except BaseException:
            self._release(taken)
            raise
        if check:  # the word is this call's own (earlier ones were checked above)
            e = int(word.item())
            if e:
                word.zero_()
                e = self._count_saturation([e])
                if e:  # undo this append: its tokens are not part of the cache
                    self._release(taken)
                    self.has_scales = had_scales
                    raise ValueError("PagedFP8KVCache.append: " + kv.kernel_error_text(e))
        else:
            self._n_err += 1
        self.has_scales = True
        for s, st, n in zip(seq_ids, start, lengths):
            self.lengths[s] = st + n
        self._len.index_add_(0, rows, counts)
        return self.scales

    def _count_saturation(self, words) -> int:
        """Count the appends whose word holds only a saturation event (overflow in
        ``overflow="saturate"`` mode); return the other bits ORed together."""
        bits = 0
        for w in words:
            if self.overflow == "saturate" and w & N.ZX_KERR_OVERFLOW:
                self.saturated_appends += 1
                w &= ~N.ZX_KERR_OVERFLOW
            bits |= w
        return bits

    def check_errors(self) -> None:
        """Read (and clear) the error words of the appends since the last check; raise
        ValueError for any bit, except an overflow in ``overflow="saturate"`` mode, which
        only counts ``saturated_appends``.  Synchronises with the cache's device."""
        n, self._n_err = self._n_err, 0
        if n == 0:
            return
        words = [int(w) for w in self._err[:n].cpu().tolist()]
        if any(words):
            self._err[:n].zero_()
        e = self._count_saturation(words)
        if e:
            raise ValueError("PagedFP8KVCache: " + kv.kernel_error_text(e))

    def gather(self, layer: int, seq_ids: list, out_len: int | None = None):
        """bf16 ``(k, v)``, each ``[B, H, out_len, D]``, of one layer for decode; positions past a
        sequence's length are zeros."""
        if out_len is None:
            out_len = max(1, max(self.lengths.get(s, 0) for s in seq_ids))
        return kv.kv_gather_dequant(self.pool[layer], self.scales[layer], self._tables(seq_ids),
                                    self._lengths(seq_ids), out_len)

    def free(self, seq_id) -> None:
        for p in self.pages.pop(seq_id, []):
            self._free.append(p)
        self.lengths.pop(seq_id, None)
        self._drop_row(seq_id)


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
                 sm_scale: float | None = None, precision: str = "f16", check: bool = True):
        if ring_degree < 1:
            raise ValueError("ring_degree must be >= 1")
        self.cache = cache
        self.ring_degree = ring_degree
        self.causal = causal
        self.sm_scale = sm_scale
        if precision not in kv.PRECISIONS:
            raise ValueError(f"precision must be one of {kv.PRECISIONS}")
        self.precision = precision  # how the softmax weights enter P.V (kv.PRECISIONS)
        # check: every call synchronises, reads the kernels' error word and the cache's
        # append words, and raises on any error bit; without it calls stay asynchronous
        # and errors surface at the cache's next check_errors
        self.check = check

    def __call__(self, q: torch.Tensor, layer: int, seq_ids: list, q_lens: list[int]) -> torch.Tensor:
        """q ``[n_q, Hq, D]`` bf16: the queries of ``seq_ids[i]`` packed in order, ``q_lens[i]``
        rows each, standing for that sequence's newest ``q_lens[i]`` cached tokens (the
        tokens just appended, as in prefill).  Returns bf16 ``[n_q, Hq, D]``."""
        c = self.cache
        if len(q_lens) != len(seq_ids) or sum(q_lens) != q.shape[0]:
            raise ValueError("q_lens must give the row count of every sequence in seq_ids, summing to q.shape[0]")
        if any(n > c.lengths.get(s, 0) for n, s in zip(q_lens, seq_ids)):
            raise ValueError("a sequence has more query rows than cached tokens")
        counts, cu = c._counts(q_lens)
        lens = c._lengths(seq_ids)
        out = kv.ring_attention_fp8(
            q.to(c.device).contiguous(), cu, lens - counts, c.pool[layer], c.scales[layer], c._tables(seq_ids), lens,
            ring_degree=self.ring_degree, causal=self.causal, sm_scale=self.sm_scale, check=self.check,
            precision=self.precision, max_q_per_seq=max(q_lens, default=0))
        if self.check:
            c.check_errors()  # the appends behind these pages (the check above has synchronised)
        return out

    def decode(self, q: torch.Tensor, layer: int, seq_ids: list) -> torch.Tensor:
        """q ``[B, Hq, D]`` bf16, one query token per sequence over all its cached tokens."""
        c = self.cache
        out = kv.paged_attention_decode(q.to(c.device).contiguous(), c.pool[layer], c.scales[layer],
                                        c._tables(seq_ids), c._lengths(seq_ids), sm_scale=self.sm_scale,
                                        check=self.check)
        if self.check:
            c.check_errors()
        return out


__all__ = ["FP8KVQuantizer", "PagedFP8KVCache", "QuantizedRingAttention"]
