"""Three-tier Belady KV tiering: HBM (T0) / pinned host DRAM (T1) / NVMe file (T2).

README.md:150-154 describes Phase 7 as a three-tier hierarchy (HBM / DRAM / NVMe) with
offline-optimal replacement; the reference's own tier manager (zenyx/streaming/
kv_tiering.py:18-66) has the same three tiers with LRU spill and synchronous copies.
Here the policy is Belady at both levels and the copies are asynchronous:

* ``ThreeTierPlan`` -- the schedule.  Belady MIN is a stack algorithm, so in the exclusive
  hierarchy where T0 sends its farthest page to T1 and T1 its farthest to T2, T0 is MIN
  with capacity c0 and T0 + T1 is MIN with capacity c0 + c1.  Two runs of the GPU
  simulator (zx_belady_simulate) and one plan kernel (zx_belady_tier_plan) give, per
  trace position, the tier the page comes from and the pages T0 and T1 evict.  Slots
  are then assigned on the host: each tier reuses its freed slots first-in first-out
  behind ``spare`` extra slots, so a slot freed at position i is reused no earlier than
  ``spare`` positions later.
* ``ThreeTierReplay`` -- moves real page bytes for a window of the trace: T0 is a device
  pool, T1 a pinned host pool, T2 a file (O_DIRECT through per-thread bounce buffers
  when the file system allows it, else buffered).
  The window is cut into batches in which every page moves at most once and no slot is
  freed and reused, so all of a batch's copies are independent: T0 -> T1 runs on one
  side stream, T1 -> T0 and T2 -> T0 on another (pages that form long runs on both
  sides as merged hipMemcpyAsync copies, zx_tier_copy_runs; scattered pages as one
  zx_tier_move_pages kernel per batch that reads pinned host memory over PCIe), NVMe
  reads and writes on host threads, all while the caller's kernels run on the compute
  stream.  Victims that are never used again are dropped without a copy.
"""
from __future__ import annotations

import concurrent.futures as cf
import mmap
import os
import threading
import time

import numpy as np
import torch

from .. import _native as N
from .. import kv
from .._streams import copy_stream

SRC_HIT, SRC_T1, SRC_T2, SRC_NEW = 0, 1, 2, 3


def _rank_in_runs(keys_sorted: np.ndarray) -> np.ndarray:
    """0, 1, 2, ... within each run of equal keys of a sorted array."""
    n = keys_sorted.size
    if n == 0:
        return np.zeros(0, np.int64)
    start = np.ones(n, bool)
    start[1:] = keys_sorted[1:] != keys_sorted[:-1]
    idx = np.arange(n, dtype=np.int64)
    return idx - np.maximum.accumulate(np.where(start, idx, 0))


def fifo_slots(adm_pos, adm_page, dep_pos, dep_page, n_slots: int):
    """Slots of one tier whose freed slots are reused first-in first-out.

    ``adm_*`` are the tier's admissions and ``dep_*`` its departures, each in position
    order; a page's admissions and departures alternate, admission first.  Admission k
    takes the k-th slot of the queue [0, 1, ..., n_slots - 1, then every freed slot in the
    order it was freed].  Returns (slot of each admission, slot of each departure)."""
    adm_pos = np.asarray(adm_pos, np.int64)
    dep_pos = np.asarray(dep_pos, np.int64)
    adm_page = np.asarray(adm_page, np.int64)
    dep_page = np.asarray(dep_page, np.int64)
    M, D = adm_pos.size, dep_pos.size
    if M == 0:
        return np.zeros(0, np.int64), np.zeros(0, np.int64)
    # the k-th departure of a page ends its k-th admission
    oa = np.argsort(adm_page, kind="stable")
    od = np.argsort(dep_page, kind="stable")
    ka = adm_page[oa] * (M + 1) + _rank_in_runs(adm_page[oa])
    kd = dep_page[od] * (M + 1) + _rank_in_runs(dep_page[od])
    j = np.searchsorted(ka, kd)
    if D and (j.max() >= M or not np.array_equal(ka[j], kd)):
        raise ValueError("a departure without a matching admission")
    dep_adm = np.empty(D, np.int64)
    dep_adm[od] = oa[j]
    if D and np.any(adm_pos[dep_adm] > dep_pos):
        raise ValueError("a page departs before it was admitted")
    # admission k >= n_slots reuses the slot freed by departure k - n_slots
    ptr = np.arange(M, dtype=np.int64)
    extra = M - n_slots
    if extra > 0:
        if extra > D:
            raise ValueError("more pages resident than the tier has slots")
        if np.any(dep_pos[:extra] > adm_pos[n_slots:]):
            raise ValueError("a slot is reused before it is freed")
        ptr[n_slots:] = dep_adm[:extra]
    while True:  # pointer jumping to the first occupant of the slot
        nxt = ptr[ptr]
        if np.array_equal(nxt, ptr):
            break
        ptr = nxt
    adm_slot = ptr
    return adm_slot, adm_slot[dep_adm]


class ThreeTierPlan:
    """Belady schedule of a page trace over T0 (``t0_pages``), T1 (``t1_pages``) and T2.

    Per position i (host numpy arrays of length n): ``src[i]`` (0 hit in T0, 1 from T1,
    2 from T2, 3 new), ``v0[i]`` / ``v1[i]`` (the page T0 / T1 evicts, -1 for none; a T0
    victim with v1 == v0 goes straight to T2), the T0 slot the accessed page occupies
    (``slot0``), and the slots of every move."""

    def __init__(self, trace: torch.Tensor, n_pages: int, t0_pages: int, t1_pages: int, spare: int = 4096):
        """Plans ``trace`` (a 1-D int32 device tensor) on the GPU."""
        self._check_sizes(t0_pages, t1_pages, spare)
        N.ensure_gpu()
        self.n_pages, self.c0, self.c1, self.spare = int(n_pages), int(t0_pages), int(t1_pages), int(spare)
        dev = trace.device
        t0 = time.perf_counter()
        sim0 = kv.BeladyTraceSim(trace, n_pages, self.c0, record_misses=True)
        sim0.run()
        if self.c1 > 0:
            sim01 = kv.BeladyTraceSim(trace, n_pages, self.c0 + self.c1, record_misses=True)
            sim01.run()
        else:
            sim01 = sim0
        src, v0, v1 = kv.belady_tier_plan(sim0, sim01, check=True)
        torch.cuda.synchronize(dev)
        t1 = time.perf_counter()
        self.gpu_s = t1 - t0
        self.stats0, self.stats01 = sim0.stats(), sim01.stats()
        self.trace = trace.cpu().numpy()
        self.src, self.v0, self.v1 = src.cpu().numpy(), v0.cpu().numpy(), v1.cpu().numpy()
        nu = sim0.next_use.cpu().numpy()
        prev = sim0.prev_use.cpu().numpy()
        del sim0, sim01
        self._assign_slots(nu, prev)
        self.host_s = time.perf_counter() - t1

    @staticmethod
    def _check_sizes(t0_pages, t1_pages, spare):
        if t0_pages < 1 or t1_pages < 0 or spare < 1:
            raise ValueError("t0_pages >= 1, t1_pages >= 0 and spare >= 1 are required")

    @classmethod
    def from_schedule(cls, trace: np.ndarray, n_pages: int, t0_pages: int, t1_pages: int, spare: int,
                      src: np.ndarray, v0: np.ndarray, v1: np.ndarray, next_use: np.ndarray,
                      prev_use: np.ndarray) -> "ThreeTierPlan":
        """The host bookkeeping (slots, moves, batches) of a schedule computed elsewhere
        (zx_belady_tier_plan's layout); no device work."""
        cls._check_sizes(t0_pages, t1_pages, spare)
        self = cls.__new__(cls)
        self.n_pages, self.c0, self.c1, self.spare = int(n_pages), int(t0_pages), int(t1_pages), int(spare)
        self.trace = np.ascontiguousarray(trace, np.int32)
        self.src = np.ascontiguousarray(src, np.uint8)
        self.v0 = np.ascontiguousarray(v0, np.int32)
        self.v1 = np.ascontiguousarray(v1, np.int32)
        self.gpu_s, self.stats0, self.stats01 = 0.0, None, None
        t1 = time.perf_counter()
        self._assign_slots(np.asarray(next_use), np.asarray(prev_use))
        self.host_s = time.perf_counter() - t1
        return self

    # ------------------------------------------------------------------ host bookkeeping
    def _assign_slots(self, next_use: np.ndarray, prev_use: np.ndarray) -> None:
        n = self.trace.size
        pos = np.arange(n, dtype=np.int64)
        tr, src, v0, v1 = self.trace, self.src, self.v0, self.v1
        last = np.full(self.n_pages, -1, np.int64)
        fin = np.nonzero(next_use == N.ZX_NEVER)[0]
        last[tr[fin]] = fin
        self.last_use = last
        # T0: admissions at misses, departures at T0 evictions
        a0 = np.nonzero(src != SRC_HIT)[0]
        d0 = np.nonzero(v0 >= 0)[0]
        s_a0, s_d0 = fifo_slots(a0, tr[a0], d0, v0[d0], self.c0 + self.spare)
        self.adm0 = np.full(n, -1, np.int64)
        self.adm0[a0] = s_a0
        self.dep0 = np.full(n, -1, np.int64)
        self.dep0[d0] = s_d0
        # T0 slot of every access: that of the admission that started its residency
        ptr = np.where(src != SRC_HIT, pos, prev_use.astype(np.int64))
        if np.any(ptr < 0):
            raise ValueError("a hit without an earlier access")
        while True:
            nxt = ptr[ptr]
            if np.array_equal(nxt, ptr):
                break
            ptr = nxt
        self.slot0 = self.adm0[ptr]
        # T1: admissions = T0 victims that stay in T1; departures = promotions to T0 and
        # T1 evictions to T2 (at most one of the two per position)
        into1 = (v0 >= 0) & (v1 != v0)
        a1 = np.nonzero(into1)[0]
        prom = src == SRC_T1
        ev1 = (v1 >= 0) & (v1 != v0)
        d1 = np.nonzero(prom | ev1)[0]
        d1_page = np.where(prom[d1], tr[d1], v1[d1])
        s_a1, s_d1 = fifo_slots(a1, v0[a1], d1, d1_page, max(self.c1, 0) + self.spare)
        self.adm1 = np.full(n, -1, np.int64)
        self.adm1[a1] = s_a1
        self.dep1 = np.full(n, -1, np.int64)
        self.dep1[d1] = s_d1

    def live(self, pages: np.ndarray, at: np.ndarray) -> np.ndarray:
        """Whether each page is accessed again after position ``at``."""
        return self.last_use[pages] > at

    def moves(self, a: int, b: int) -> dict:
        """The moves of positions [a, b): dict of (page, from, to) arrays per kind.
        Slots for T0/T1, page ids for T2 (file offset page * page_bytes)."""
        sl = slice(a, b)
        pos = np.arange(a, b, dtype=np.int64)
        tr, src, v0, v1 = self.trace[sl], self.src[sl], self.v0[sl], self.v1[sl]
        adm0, dep0, adm1, dep1 = self.adm0[sl], self.dep0[sl], self.adm1[sl], self.dep1[sl]
        m = {}
        k = src == SRC_T1
        m["t1_t0"] = (tr[k], dep1[k], adm0[k])
        k = src == SRC_T2
        m["t2_t0"] = (tr[k], tr[k], adm0[k])
        k = src == SRC_NEW
        m["new"] = (tr[k], tr[k], adm0[k])
        k = (v0 >= 0) & (v1 != v0)
        k &= self.live(np.maximum(v0, 0), pos)
        m["t0_t1"] = (v0[k], dep0[k], adm1[k])
        k = (v0 >= 0) & (v1 == v0)
        k &= self.live(np.maximum(v0, 0), pos)
        m["t0_t2"] = (v0[k], dep0[k], v0[k])
        k = (v1 >= 0) & (v1 != v0)
        k &= self.live(np.maximum(v1, 0), pos)
        m["t1_t2"] = (v1[k], dep1[k], v1[k])
        return m

    def batches(self, a: int, b: int, max_len: int | None = None) -> list:
        """Cut [a, b) into batches of at most ``max_len`` (<= spare) positions in which no
        page has more than one move (admission to T0, or leaving T0, or leaving T1)."""
        max_len = self.spare if max_len is None else min(int(max_len), self.spare)
        sl = slice(a, b)
        tr, src, v0, v1 = self.trace[sl], self.src[sl], self.v0[sl], self.v1[sl]
        # pages moving at each position (up to three)
        m_adm = np.where(src != SRC_HIT, tr, -1)
        m_v0 = v0
        m_v1 = np.where(v1 != v0, v1, -1)
        out = []
        start = 0
        n = b - a
        seen: set = set()
        i = 0
        while i < n:
            pages = [int(p) for p in (m_adm[i], m_v0[i], m_v1[i]) if p >= 0]
            if i - start >= max_len or any(p in seen for p in pages):
                out.append((a + start, a + i))
                start = i
                seen = set()
            seen.update(pages)
            i += 1
        if start < n:
            out.append((a + start, a + n))
        return out

    def stats(self) -> dict:
        s = self.src
        return {"accesses": int(s.size), "t0_hits": int(np.sum(s == SRC_HIT)), "from_t1": int(np.sum(s == SRC_T1)),
                "from_t2": int(np.sum(s == SRC_T2)), "new": int(np.sum(s == SRC_NEW)),
                "t0_evictions": int(np.sum(self.v0 >= 0)), "t1_evictions": int(np.sum((self.v1 >= 0) & (self.v1 != self.v0))),
                "t0_to_t2": int(np.sum((self.v0 >= 0) & (self.v1 == self.v0))),
                "gpu_plan_s": self.gpu_s, "host_slots_s": self.host_s}


class ThreeTierReplay:
    """Executes a ThreeTierPlan with real buffers: T0 device pool (c0 + spare slots),
    T1 pinned host pool (c1 + spare slots), T2 file of n_pages pages (sparse)."""

    def __init__(self, plan: ThreeTierPlan, page_bytes: int, t2_path: str, device: torch.device | None = None,
                 io_threads: int = 8, direct_io: bool = True, move_workgroups: int = 32):
        if page_bytes <= 0 or page_bytes % 16:
            raise ValueError("page_bytes must be a positive multiple of 16")
        self.plan, self.pb = plan, int(page_bytes)
        self.move_workgroups = int(move_workgroups)
        self.device = device or N.ensure_gpu()
        self.t0 = torch.empty((plan.c0 + plan.spare) * self.pb, dtype=torch.uint8, device=self.device)
        self.t1 = torch.empty((plan.c1 + plan.spare) * self.pb, dtype=torch.uint8, pin_memory=True)
        self._t1_np = self.t1.numpy()
        self.t2_path = t2_path
        self._tls = threading.local()
        flags = os.O_RDWR | os.O_CREAT
        self.direct = False
        self.fd = None
        # O_DIRECT (bypassing the page cache) needs 4 KiB-aligned buffers, offsets and
        # sizes, and memory the kernel can pin for DMA -- not HIP's pinned pages -- so
        # direct I/O goes through a per-thread anonymous bounce buffer
        if direct_io and hasattr(os, "O_DIRECT") and self.pb % 4096 == 0:
            try:
                fd = os.open(t2_path, flags | os.O_DIRECT, 0o600)
                probe = mmap.mmap(-1, self.pb)
                try:
                    os.pwritev(fd, [probe], 0)
                    os.preadv(fd, [probe], 0)
                    self.fd, self.direct = fd, True
                except OSError:
                    os.close(fd)
                finally:
                    probe.close()
            except OSError:
                pass
        if self.fd is None:
            self.fd = os.open(t2_path, flags, 0o600)
        self.pool = cf.ThreadPoolExecutor(max(1, io_threads))
        self.s_out = copy_stream(self.device, "d2h")  # T0 -> host
        self.s_in = copy_stream(self.device, "h2d")   # host -> T0
        self._stage_in = torch.empty(0, dtype=torch.uint8, pin_memory=True)
        self._stage_out = torch.empty(0, dtype=torch.uint8, pin_memory=True)
        self._err = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._keep: list = []  # offset tables of copies in flight

    def _move(self, dst: torch.Tensor, src: torch.Tensor, dst_offs: np.ndarray, src_offs: np.ndarray,
              stream: torch.cuda.Stream) -> None:
        """Pages that form long runs on both sides go as merged hipMemcpyAsync copies (the
        DMA engines, no compute units); scattered pages as one zx_tier_move_pages launch."""
        n = len(dst_offs)
        if n == 0:
            return
        pb = self.pb
        runs = 1 + int(np.count_nonzero((np.diff(dst_offs) != pb) | (np.diff(src_offs) != pb)))
        if n >= 8 * runs:
            kv.tier_copy_runs(dst, src, dst_offs, src_offs, pb, stream=stream)
            return
        d = torch.from_numpy(np.ascontiguousarray(dst_offs, np.int64)).pin_memory()
        s = torch.from_numpy(np.ascontiguousarray(src_offs, np.int64)).pin_memory()
        self._keep.append((d, s))
        kv.tier_move_pages(dst, src, d, s, pb, stream=stream, max_workgroups=self.move_workgroups, err=self._err)

    def close(self) -> None:
        self.pool.shutdown(wait=True)
        if self.fd is not None:
            os.close(self.fd)
            self.fd = None

    def __enter__(self) -> "ThreeTierReplay":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def _stage(self, which: str, n: int) -> torch.Tensor:
        cur = getattr(self, which)
        if cur.numel() < n * self.pb:
            cur = torch.empty(max(n, 1) * self.pb, dtype=torch.uint8, pin_memory=True)
            setattr(self, which, cur)
        return cur

    def _bounce(self) -> tuple:
        b = getattr(self._tls, "buf", None)
        if b is None:
            mm = mmap.mmap(-1, self.pb)
            b = (mm, np.frombuffer(mm, dtype=np.uint8))
            self._tls.buf = b
        return b

    def _write_page(self, buf: np.ndarray, o: int, page: int) -> None:
        if self.direct:
            mm, arr = self._bounce()
            arr[:] = buf[o:o + self.pb]
            n = os.pwritev(self.fd, [mm], page * self.pb)
        else:
            n = os.pwritev(self.fd, [memoryview(buf[o:o + self.pb])], page * self.pb)
        if n != self.pb:
            raise OSError("short write to the T2 file")

    def _read_page(self, buf: np.ndarray, o: int, page: int) -> None:
        if self.direct:
            mm, arr = self._bounce()
            n = os.preadv(self.fd, [mm], page * self.pb)
            buf[o:o + n] = arr[:n]
        else:
            n = os.preadv(self.fd, [memoryview(buf[o:o + self.pb])], page * self.pb)
        if n < self.pb:  # past the end of the file: a page this replay never wrote
            buf[o + n:o + self.pb] = 0

    def _pwrite(self, buf: np.ndarray, offs: np.ndarray, pages: np.ndarray) -> None:
        for f in [self.pool.submit(self._write_page, buf, int(o), int(p)) for o, p in zip(offs, pages)]:
            f.result()

    def _pread(self, buf: np.ndarray, offs: np.ndarray, pages: np.ndarray) -> None:
        for f in [self.pool.submit(self._read_page, buf, int(o), int(p)) for o, p in zip(offs, pages)]:
            f.result()

    def run(self, a: int, b: int, compute=None, create=None, after_batch=None, max_batch: int | None = None) -> dict:
        """Replay positions [a, b).  ``compute()`` (optional) launches kernels on the
        current stream once, before the first batch, to overlap with the moves;
        ``create(pages, t0_slots)`` fills new pages (default: left as they are);
        ``after_batch(a_i, b_i)`` runs after each batch has completed."""
        plan, pb = self.plan, self.pb
        cur = torch.cuda.current_stream(self.device)
        batches = plan.batches(a, b, max_batch)
        tot = {"t0_t1": 0, "t1_t0": 0, "t2_t0": 0, "t0_t2": 0, "t1_t2": 0, "new": 0}
        t_io = {"d2h_s": 0.0, "h2d_s": 0.0, "disk_write_s": 0.0, "disk_read_s": 0.0}
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(6)]
        self.s_out.wait_stream(cur)
        self.s_in.wait_stream(cur)
        torch.cuda.synchronize(self.device)
        t_start = time.perf_counter()
        if compute is not None:
            compute()
        for (ba, bb) in batches:
            m = plan.moves(ba, bb)
            for k in tot:
                tot[k] += len(m[k][0])
            # T0 -> T1 and T0 -> staging (for T0 -> T2) on the outgoing stream
            ev[0].record(self.s_out)
            pg, fr, to = m["t0_t1"]
            self._move(self.t1, self.t0, to * pb, fr * pb, self.s_out)
            pg2, fr2, _ = m["t0_t2"]
            so = None
            if len(pg2):
                so = self._stage("_stage_out", len(pg2))
                self._move(so, self.t0, np.arange(len(pg2)) * pb, fr2 * pb, self.s_out)
            ev[1].record(self.s_out)
            # T1 -> T0 on the incoming stream
            ev[2].record(self.s_in)
            pg, fr, to = m["t1_t0"]
            self._move(self.t0, self.t1, to * pb, fr * pb, self.s_in)
            # T1 -> T2 from host memory (slots this batch's copies do not touch)
            pg, fr, _ = m["t1_t2"]
            if len(pg):
                t0 = time.perf_counter()
                self._pwrite(self._t1_np, fr * pb, pg)
                t_io["disk_write_s"] += time.perf_counter() - t0
            ev[3].record(self.s_in)
            # T2 -> staging -> T0
            pg, _, to = m["t2_t0"]
            if len(pg):
                si = self._stage("_stage_in", len(pg))
                t0 = time.perf_counter()
                self._pread(si.numpy(), np.arange(len(pg)) * pb, pg)
                t_io["disk_read_s"] += time.perf_counter() - t0
            ev[4].record(self.s_in)
            if len(pg):
                self._move(self.t0, si, to * pb, np.arange(len(pg)) * pb, self.s_in)
            ev[5].record(self.s_in)
            pg, _, to = m["new"]
            if len(pg) and create is not None:
                with torch.cuda.stream(self.s_in):
                    create(pg, to)
            # staged T0 -> T2 pages go to the file once their copy is done
            if so is not None:
                self.s_out.synchronize()
                t0 = time.perf_counter()
                self._pwrite(so.numpy(), np.arange(len(pg2)) * pb, pg2)
                t_io["disk_write_s"] += time.perf_counter() - t0
            self.s_out.synchronize()
            self.s_in.synchronize()
            self._keep.clear()
            t_io["d2h_s"] += ev[0].elapsed_time(ev[1]) / 1e3
            t_io["h2d_s"] += (ev[2].elapsed_time(ev[3]) + ev[4].elapsed_time(ev[5])) / 1e3
            if after_batch is not None:
                after_batch(ba, bb)
        torch.cuda.synchronize(self.device)
        wall = time.perf_counter() - t_start
        if int(self._err.item()):
            raise RuntimeError("tier_move_pages skipped a page outside its buffer")
        out = {"positions": b - a, "batches": len(batches), "wall_s": wall, "page_bytes": pb, "direct_io": self.direct}
        out.update({f"{k}_pages": v for k, v in tot.items()})
        out.update(t_io)
        gb = lambda pages, s: pages * pb / s / 1e9 if s > 0 else 0.0  # noqa: E731
        out["d2h_GBps"] = gb(tot["t0_t1"] + tot["t0_t2"], t_io["d2h_s"])
        out["h2d_GBps"] = gb(tot["t1_t0"] + tot["t2_t0"], t_io["h2d_s"])
        out["disk_write_GBps"] = gb(tot["t1_t2"] + tot["t0_t2"], t_io["disk_write_s"])
        out["disk_read_GBps"] = gb(tot["t2_t0"], t_io["disk_read_s"])
        return out


__all__ = ["ThreeTierPlan", "ThreeTierReplay", "fifo_slots", "SRC_HIT", "SRC_T1", "SRC_T2", "SRC_NEW"]
