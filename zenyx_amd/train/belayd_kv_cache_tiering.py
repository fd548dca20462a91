"""Belady KV-cache tiering (README.md:61, 93-97, 343: ``BeladyKVCacheTieringManager``,
``RingAttentionAccessSequence``; the README's module path, including its spelling, is
kept: zenyx.train.belayd_kv_cache_tiering).  The reference tree does not contain this
module, so its behaviour is defined here:

* ``RingAttentionAccessSequence`` -- the KV page accesses of ring attention of degree R
  simulated on one GPU, generalising build_ring_timeline (zenyx/streaming/kv_tiering.py:
  69-73): per layer, for ring step s and simulated device d, the pages of shard
  (d - s) mod R in order; the backward pass is the exact reverse of the forward pass.
* ``BeladyKVCacheTieringManager`` -- sizes the page set from the model (context length,
  layers, KV heads, head_dim, page tokens, FP8 bytes) and the HBM budget, computes the
  Belady MIN schedule of that sequence on the GPU (zx_belady_next_use +
  zx_belady_simulate; victims are farthest-next-use, ties to the smallest page id), and
  replays the tier moves it implies between a device page pool and pinned host memory
  with hipMemcpyAsync on a side stream (zx_tier_copy_runs).
"""
from __future__ import annotations

import math
import time

import numpy as np
import torch

from .. import _native as N
from .. import kv
from .._streams import copy_stream


class RingAttentionAccessSequence:
    """Page access order of a degree-``ring_degree`` ring over ``num_layers`` layers."""

    def __init__(self, num_layers: int, ring_degree: int = 8, pages_per_shard: int = 2048):
        if num_layers < 1 or ring_degree < 1 or pages_per_shard < 1:
            raise ValueError("num_layers, ring_degree and pages_per_shard must be positive")
        self.num_layers, self.ring_degree, self.pages_per_shard = num_layers, ring_degree, pages_per_shard

    @property
    def n_pages(self) -> int:
        return self.num_layers * self.ring_degree * self.pages_per_shard

    def __len__(self) -> int:
        return 2 * self.num_layers * self.ring_degree * self.ring_degree * self.pages_per_shard

    def trace(self, device: torch.device | str | None = None) -> torch.Tensor:
        """int32 page ids, forward then backward: layer l's page of shard k, index i is
        (l R + k) S + i.  Built on the GPU by zx_ring_curriculum_trace as one step of
        constant degree R over R S pages per layer (shard k of that step is exactly pages
        [k S, (k + 1) S)); ``device="cpu"`` returns a host copy."""
        L, R, S = self.num_layers, self.ring_degree, self.pages_per_shard
        dev = torch.device(device) if device is not None else N.ensure_gpu()
        gdev = dev if dev.type == "cuda" else N.ensure_gpu()
        t = kv.ring_curriculum_trace([R], [R * S], L, R * S, device=gdev)
        return t if dev.type == "cuda" else t.cpu()


class BeladyKVCacheTieringManager:
    """Belady-optimal HBM <-> pinned-host tiering of FP8 KV pages for a ring schedule.

    ``BeladyKVCacheTieringManager(num_devices=8, context_length=4096, num_layers=12)`` is the
    README's call (README.md:93-97); ``num_devices`` is the ring degree.
    """

    def __init__(self, num_devices: int = 8, context_length: int = 4096, num_layers: int = 12,
                 num_kv_heads: int = 8, head_dim: int = 128, page_tokens: int = 64,
                 hbm_budget_bytes: float | None = None, kv_bytes_per_element: int = 1,
                 device: torch.device | None = None):
        self.num_devices, self.context_length, self.num_layers = num_devices, context_length, num_layers
        self.num_kv_heads, self.head_dim, self.page_tokens = num_kv_heads, head_dim, page_tokens
        shard_tokens = math.ceil(context_length / num_devices)
        self.pages_per_shard = max(1, math.ceil(shard_tokens / page_tokens))
        self.page_bytes = page_tokens * num_kv_heads * head_dim * 2 * kv_bytes_per_element  # K and V
        self.sequence = RingAttentionAccessSequence(num_layers, num_devices, self.pages_per_shard)
        self.n_pages = self.sequence.n_pages
        if hbm_budget_bytes is None:
            self.capacity = self.n_pages
        else:
            self.capacity = max(1, min(self.n_pages, int(hbm_budget_bytes // self.page_bytes)))
        self.device = device
        self.sim: kv.BeladyTraceSim | None = None
        self.timings: dict = {}

    # ------------------------------------------------------------------ schedule
    def plan(self, record_misses: bool = True) -> dict:
        """Build the access trace and its Belady schedule on the GPU; returns counters."""
        dev = self.device or N.ensure_gpu()
        trace = self.sequence.trace(dev)
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        self.sim = kv.BeladyTraceSim(trace, self.n_pages, self.capacity, record_misses=record_misses)
        torch.cuda.synchronize(dev)
        t1 = time.perf_counter()
        self.sim.run()
        torch.cuda.synchronize(dev)
        t2 = time.perf_counter()
        self.timings = {"next_use_s": t1 - t0, "simulate_s": t2 - t1}
        return self.sim.stats()

    def eviction_schedule(self):
        """(trace positions, page ids) of every eviction, in order (CPU int32)."""
        if self.sim is None:
            raise RuntimeError("call plan() first")
        return self.sim.evictions()

    # ------------------------------------------------------------------ tier moves
    def _moves(self, t_begin: int, t_end: int):
        """Trace positions and page ids of the window's D2H and H2D moves (see transfers)."""
        if self.sim is None or self.sim.miss_flags is None:
            raise RuntimeError("call plan(record_misses=True) first")
        trace = self.sim.trace
        pos, page = self.eviction_schedule()
        pos, page = pos.numpy().astype(np.int64), page.numpy().astype(np.int64)
        # a page is written back once, at its first eviction: KV pages do not change after
        # they are written, so a page fetched back from host memory is clean and is dropped
        # without a copy when it is evicted again
        first = np.zeros(len(page), bool)
        first[np.unique(page, return_index=True)[1]] = True
        sel = (pos >= t_begin) & (pos < t_end) & first
        last = torch.full((self.n_pages,), -1, dtype=torch.int64, device=trace.device)
        last.scatter_reduce_(0, trace.long(), torch.arange(trace.numel(), device=trace.device), reduce="amax")
        last = last.cpu().numpy()
        keep = last[page[sel]] > pos[sel]
        d2h_pos, d2h = pos[sel][keep], page[sel][keep]
        miss = self.sim.miss_flags[t_begin:t_end].bool()
        seen = self.sim.prev_use[t_begin:t_end] >= 0
        k = (miss & seen).cpu().numpy()
        h2d_pos = t_begin + np.nonzero(k)[0].astype(np.int64)
        h2d = trace[t_begin:t_end].cpu().numpy()[k].astype(np.int64)
        return d2h_pos, d2h, h2d_pos, h2d

    def transfers(self, t_begin: int, t_end: int):
        """Pages moved for trace positions [t_begin, t_end): (d2h, h2d) page-id arrays.
        D2H: a page's first eviction when it is used again later (the only time its bytes
        exist on the device alone: pages do not change once written, so later evictions of
        a page fetched back drop it without a copy); H2D: misses on pages seen before
        (first touches create pages on the device and need no copy)."""
        _, d2h, _, h2d = self._moves(t_begin, t_end)
        return d2h, h2d

    @staticmethod
    def _chunks(kind: np.ndarray, page: np.ndarray, max_len: int) -> list:
        """Split moves sorted by trace position into per-direction chunks of at most
        ``max_len`` moves, in issue order: a list of (direction, move indices, chunk index
        of the other direction to wait for or -1).  A move depends on its page's previous
        move when that one went the other way (a page written back, then fetched again);
        if that move is still in the other direction's open chunk, both open chunks are
        closed first (this direction's, whose waits point at closed chunks only, then the
        other's), so every wait points at a chunk issued earlier and the two copy streams
        never wait for each other in a cycle."""
        out = []
        cur = {0: [], 1: []}
        n_closed = {0: 0, 1: 0}
        dep = {0: -1, 1: -1}
        last: dict = {}  # page -> (direction, chunk index) of its latest move

        def close(k):
            if cur[k]:
                out.append((k, cur[k], dep[k]))
                n_closed[k] += 1
                cur[k], dep[k] = [], -1

        for i in range(len(page)):
            k, p = int(kind[i]), int(page[i])
            prev = last.get(p)
            if prev is not None and prev[0] != k:
                if prev[1] == n_closed[1 - k]:  # still in the other direction's open chunk
                    close(k)
                    close(1 - k)
                dep[k] = max(dep[k], prev[1])
            cur[k].append(i)
            last[p] = (k, n_closed[k])
            if len(cur[k]) >= max_len:
                close(k)
        close(0)
        close(1)
        return out

    def replay_transfers(self, t_begin: int, t_end: int, compute=None, max_pool_pages: int | None = None,
                         max_batch: int = 1024, check_bytes: bool = False) -> dict:
        """Execute the window's tier moves with real page buffers: a device pool and a pinned
        host pool with one slot per page the window moves (page p in slot rank(p) on both
        sides).  The moves, in trace order, go out in chunks of up to ``max_batch`` pages
        per direction: D2H chunks on the library's d2h copy stream and H2D chunks on its
        h2d copy stream, so PCIe carries both directions at once; a chunk holding a page
        whose previous move went the other way first waits for the chunk that made it
        (an event between the two streams).  ``compute`` (a callable launching kernels on
        the current stream) runs concurrently.  Returns pages moved, each direction's copy
        time (first to last copy) and the window's span over both.  ``max_pool_pages``
        below the window's page count is refused: pages would share slots and overwrite
        each other (ThreeTierReplay schedules slots access by access for windows larger
        than the pool).
        ``check_bytes``: before the window, each page's bytes (a pattern of its id) are put
        where the page is (the device slot if its first move is D2H, the host slot if it is
        H2D) and filler everywhere else; afterwards both slots of every page must hold the
        pattern, which fails if a copy ran before the copy that brought its page in."""
        dev = self.device or N.ensure_gpu()
        d2h_pos, d2h, h2d_pos, h2d = self._moves(t_begin, t_end)
        pages = np.unique(np.concatenate([d2h, h2d]))
        if max_pool_pages is not None and max_pool_pages < len(pages):
            raise ValueError(f"the window moves {len(pages)} distinct pages, more than max_pool_pages="
                             f"{max_pool_pages} device slots")
        pb = self.page_bytes
        slot = np.full(self.n_pages, -1, np.int64)
        slot[pages] = np.arange(len(pages))
        dev_pool = torch.empty(max(len(pages), 1) * pb, dtype=torch.uint8, device=dev)
        host_pool = torch.empty(max(len(pages), 1) * pb, dtype=torch.uint8, pin_memory=True)
        pos = np.concatenate([d2h_pos, h2d_pos])
        kind = np.concatenate([np.zeros(len(d2h), np.int8), np.ones(len(h2d), np.int8)])
        page = np.concatenate([d2h, h2d])
        order = np.lexsort((kind, pos))
        pos, kind, page = pos[order], kind[order], page[order]
        chunks = self._chunks(kind, page, max_batch)
        if check_bytes and len(pages):
            first_kind = np.full(self.n_pages, -1, np.int8)
            first_kind[page[::-1]] = kind[::-1]  # the earliest move of each page wins
            want = _page_pattern(torch.from_numpy(pages).to(dev), pb)
            on_dev = torch.from_numpy(first_kind[pages] == 0).to(dev)
            dev_pool.view(-1, pb).copy_(torch.where(on_dev[:, None], want, torch.full_like(want, 0xEE)))
            host_pool.view(-1, pb).copy_(torch.where(on_dev[:, None], torch.full_like(want, 0xEE), want).cpu())
        streams = (copy_stream(dev, "d2h"), copy_stream(dev, "h2d"))
        cur = torch.cuda.current_stream(dev)
        for st in streams:
            st.wait_stream(cur)
        done = {0: [], 1: []}  # end event of each chunk, per direction
        ev_first = [None, None]
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        if compute is not None:
            compute()
        for k, idx, wait in chunks:
            st = streams[k]
            if wait >= 0:
                st.wait_event(done[1 - k][wait])
            if ev_first[k] is None:
                ev_first[k] = torch.cuda.Event(enable_timing=True)
                ev_first[k].record(st)
            p = np.sort(page[idx])  # page order: adjacent slots merge into one copy
            if k == 0:
                kv.tier_copy_runs(host_pool, dev_pool, slot[p] * pb, slot[p] * pb, pb, stream=st)
            else:
                kv.tier_copy_runs(dev_pool, host_pool, slot[p] * pb, slot[p] * pb, pb, stream=st)
            e = torch.cuda.Event(enable_timing=True)
            e.record(st)
            done[k].append(e)
        torch.cuda.synchronize(dev)
        wall = time.perf_counter() - t0
        # each direction: from its first copy to its last; the span: first copy to last copy
        d2h_ms = ev_first[0].elapsed_time(done[0][-1]) if done[0] else 0.0
        h2d_ms = ev_first[1].elapsed_time(done[1][-1]) if done[1] else 0.0
        starts = [e for e in ev_first if e is not None]
        ends = [done[k][-1] for k in (0, 1) if done[k]]
        span_ms = 0.0
        if starts:
            first = starts[0] if len(starts) == 1 or starts[0].elapsed_time(starts[1]) >= 0 else starts[1]
            span_ms = max(first.elapsed_time(e) for e in ends)
        nd, nh = int(len(d2h)), int(len(h2d))
        if check_bytes and len(pages):
            bad_dev = int((dev_pool.view(-1, pb) != want).any(dim=1).sum())
            bad_host = int((host_pool.view(-1, pb).to(dev) != want).any(dim=1).sum())
            if bad_dev or bad_host:
                raise RuntimeError(f"replay_transfers: {bad_dev} device and {bad_host} host slots do not hold "
                                   "their page's bytes")
        gb = lambda n, ms: n * pb / max(ms, 1e-9) / 1e6  # noqa: E731
        return {"d2h_pages": nd, "h2d_pages": nh, "page_bytes": pb, "chunks": len(chunks),
                "d2h_GBps": gb(nd, d2h_ms), "h2d_GBps": gb(nh, h2d_ms),
                "d2h_ms": d2h_ms, "h2d_ms": h2d_ms, "copy_span_ms": span_ms,
                "both_GBps": gb(nd + nh, span_ms), "copy_ms": d2h_ms + h2d_ms, "wall_ms": wall * 1e3}


def _page_pattern(pages: torch.Tensor, pb: int) -> torch.Tensor:
    """uint8 [len(pages), pb]: bytes that identify each page id."""
    i = torch.arange(pb, device=pages.device, dtype=torch.int64)
    return ((pages.to(torch.int64)[:, None] * 2654435761 + i[None, :] * 40503) >> 7).to(torch.uint8)


__all__ = ["BeladyKVCacheTieringManager", "RingAttentionAccessSequence"]
