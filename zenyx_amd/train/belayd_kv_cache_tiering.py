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

import ctypes
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
    def transfers(self, t_begin: int, t_end: int):
        """Pages moved for trace positions [t_begin, t_end): (d2h, h2d) page-id arrays.
        D2H: evicted pages that are used again later; H2D: misses on pages seen before
        (first touches create pages on the device and need no copy)."""
        if self.sim is None or self.sim.miss_flags is None:
            raise RuntimeError("call plan(record_misses=True) first")
        trace = self.sim.trace
        pos, page = self.eviction_schedule()
        pos, page = pos.numpy(), page.numpy()
        sel = (pos >= t_begin) & (pos < t_end)
        last = torch.full((self.n_pages,), -1, dtype=torch.int64, device=trace.device)
        last.scatter_reduce_(0, trace.long(), torch.arange(trace.numel(), device=trace.device), reduce="amax")
        last = last.cpu().numpy()
        d2h = page[sel][last[page[sel]] > pos[sel]]
        miss = self.sim.miss_flags[t_begin:t_end].bool()
        seen = self.sim.prev_use[t_begin:t_end] >= 0
        h2d = trace[t_begin:t_end][miss & seen].cpu().numpy()
        return d2h.astype(np.int64), h2d.astype(np.int64)

    def replay_transfers(self, t_begin: int, t_end: int, compute=None, max_pool_pages: int | None = None) -> dict:
        """Execute the window's tier moves with real page buffers: a device pool and a pinned
        host pool with one slot per page the window moves (page p in slot rank(p) on both
        sides).  All D2H copies are queued, then all H2D copies, on a side stream; ``compute``
        (a callable launching kernels on the current stream) runs concurrently.  Returns
        bytes moved and times.  ``max_pool_pages`` below the window's page count is refused:
        pages would share slots and overwrite each other (ThreeTierReplay schedules slots
        access by access for windows larger than the pool)."""
        dev = self.device or N.ensure_gpu()
        d2h, h2d = self.transfers(t_begin, t_end)
        # batch the window's moves in page order: adjacent pages have adjacent slots on both
        # sides, so zx_tier_copy_runs merges them into few large copies
        d2h, h2d = np.sort(d2h), np.sort(h2d)
        pages = np.unique(np.concatenate([d2h, h2d]))
        if max_pool_pages is not None and max_pool_pages < len(pages):
            raise ValueError(f"the window moves {len(pages)} distinct pages, more than max_pool_pages="
                             f"{max_pool_pages} device slots")
        slots = max(len(pages), 1)
        host_rank = {int(p): i for i, p in enumerate(pages)}
        pb = self.page_bytes
        dev_pool = torch.empty(slots * pb, dtype=torch.uint8, device=dev)
        host_pool = torch.empty(len(pages) * pb if len(pages) else pb, dtype=torch.uint8, pin_memory=True)
        lib = N.load()
        side = copy_stream(dev, "h2d")

        def offs(ids, on_host):
            if on_host:
                return (ctypes.c_int64 * len(ids))(*[host_rank[int(p)] * pb for p in ids])
            return (ctypes.c_int64 * len(ids))(*[host_rank[int(p)] * pb for p in ids])

        cur = torch.cuda.current_stream(dev)
        side.wait_stream(cur)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        ev[0].record(side)
        if len(d2h):
            N.check(lib.zx_tier_copy_runs(N.ptr(host_pool), N.ptr(dev_pool), offs(d2h, True), offs(d2h, False),
                                          len(d2h), pb, ctypes.c_void_p(side.cuda_stream), None), "d2h")
        ev[1].record(side)
        if len(h2d):
            N.check(lib.zx_tier_copy_runs(N.ptr(dev_pool), N.ptr(host_pool), offs(h2d, False), offs(h2d, True),
                                          len(h2d), pb, ctypes.c_void_p(side.cuda_stream), None), "h2d")
        ev[2].record(side)
        if compute is not None:
            compute()
        torch.cuda.synchronize(dev)
        wall = time.perf_counter() - t0
        d2h_ms = ev[0].elapsed_time(ev[1])
        h2d_ms = ev[1].elapsed_time(ev[2])
        return {"d2h_pages": int(len(d2h)), "h2d_pages": int(len(h2d)), "page_bytes": pb,
                "d2h_GBps": len(d2h) * pb / max(d2h_ms, 1e-9) / 1e6, "h2d_GBps": len(h2d) * pb / max(h2d_ms, 1e-9) / 1e6,
                "copy_ms": d2h_ms + h2d_ms, "wall_ms": wall * 1e3}


__all__ = ["BeladyKVCacheTieringManager", "RingAttentionAccessSequence"]
