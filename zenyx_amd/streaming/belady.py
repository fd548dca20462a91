"""Drop-in for zenyx/streaming/belady.py: Belady approximation by next-use distance.

``BeladyApproxCache`` keeps the reference contract (belady.py:14-55): ``update_future``
records an id's next use, ``touch`` admits an id and, when the cache is full, evicts the
resident id whose next use is farthest (unknown ids count as 10**18, belady.py:47).  The
farthest-next-use scan runs on the GPU (zx_belady_argmax over dense device tables of the
resident ids' keys and registration numbers, kept in place and updated slot by slot);
the id <-> slot bookkeeping stays on the host.

Kept reference behaviour (belady.py:30-36, 45-51):
  * a victim must have next use > -1, so if every resident id has next use <= -1 nothing is
    evicted and the resident set grows past the capacity;
  * capacity 0 behaves like capacity 1 (the size test is ``len >= capacity``).
One liberty: the reference breaks ties by iterating a Python ``set`` (order unspecified);
here ties go to the id registered first (first seen by ``update_future`` or ``touch``).
Not thread-safe, like the reference.
"""
from __future__ import annotations

import ctypes
import time
from dataclasses import dataclass

import torch

from .. import _native as N
from .._native import ensure_gpu

_INF = 10**18
_PENDING = -2  # the argmax's result word before the kernel writes it (it writes a slot >= -1)
_I64_MAX = 2**63 - 1
_I64_MIN = -(2**63)


@dataclass
class AccessEvent:
    """belady.py:8-11 (unused by the reference itself; kept for the import surface)."""

    tensor_id: str
    step: int


class BeladyApproxCache:
    """Evict tensors with farthest known next-use (Belady approximation), on the GPU.

    The device tables hold the resident ids only, one slot each: the next-use key and the
    id's registration number (the tie-break).  Admitting an id appends a slot; evicting
    one moves the last slot into the freed one, so the tables stay dense and at most the
    resident count long however many distinct ids pass through.  ``update_future`` and
    ``touch`` only change host dictionaries and mark slots dirty; a miss on a full cache
    first writes the dirty slots (one zx_belady_update_slots launch reading them from
    pinned host memory), then runs the argmax (zx_belady_argmax, ties to the smaller
    registration number) over the resident slots, whose {slot, key} lands in pinned host
    memory, and waits for that stream once.  Host work per eviction is O(1) plus the
    slots changed since the previous one; device work is O(resident)."""

    def __init__(self, capacity: int, device: torch.device | None = None):
        self.capacity = capacity
        self._device = device
        self._rank: dict = {}   # id -> registration number (first update_future or touch)
        self._key: dict = {}    # id -> next use, for every id given one (the reference's next_use)
        self._slot: dict = {}   # resident id -> its slot in the device tables
        self._at: list = []     # slot -> resident id
        self._dirty: set = set()  # slots whose device entry is stale
        self._cap = 0  # slots the device tables hold
        self._keys_dev: torch.Tensor | None = None
        self._rank_dev: torch.Tensor | None = None
        self._ws: torch.Tensor | None = None
        self._stage = None  # pinned (slot, key, rank) staging arrays and their numpy views
        self._out: torch.Tensor | None = None  # pinned int64 [2]: {slot, key} of the last argmax
        self._out_np = None  # its numpy view (read without a torch call)

    def _reg(self, tensor_id) -> None:
        if tensor_id not in self._rank:
            self._rank[tensor_id] = len(self._rank)

    def update_future(self, tensor_id, next_use_step: int) -> None:  # belady.py:22-23
        self._reg(tensor_id)
        self._key[tensor_id] = min(max(int(next_use_step), _I64_MIN), _I64_MAX)
        s = self._slot.get(tensor_id)
        if s is not None:
            self._dirty.add(s)

    def touch(self, tensor_id) -> list:  # belady.py:25-37
        self._reg(tensor_id)
        if tensor_id in self._slot:
            return []
        evicted: list = []
        if len(self._at) >= self.capacity:
            victim = self._select_victim()
            if victim is not None:
                self._remove(victim)
                evicted.append(victim)
        self._slot[tensor_id] = len(self._at)
        self._dirty.add(len(self._at))
        self._at.append(tensor_id)
        return evicted

    def _remove(self, tensor_id) -> None:
        """Free the id's slot; the last slot's id moves into it (the tables stay dense)."""
        s = self._slot.pop(tensor_id)
        last = self._at.pop()
        if s < len(self._at):
            self._at[s] = last
            self._slot[last] = s
            self._dirty.add(s)
        self._dirty.discard(len(self._at))  # beyond the live slots now: never scanned

    def _tables(self, dev: torch.device) -> None:
        """Grow the device tables (geometrically) to hold every resident slot."""
        n = len(self._at)
        if n <= self._cap:
            return
        cap = max(1024, 2 * n)
        keys = torch.empty(cap, dtype=torch.int64, device=dev)
        rank = torch.empty(cap, dtype=torch.int64, device=dev)
        if self._cap:
            keys[:self._cap].copy_(self._keys_dev)
            rank[:self._cap].copy_(self._rank_dev)
        self._keys_dev, self._rank_dev, self._cap = keys, rank, cap
        lib = N.load()
        self._ws = torch.empty(max(256, lib.zx_belady_argmax_workspace_bytes(cap)), dtype=torch.uint8, device=dev)
        if self._out is None:
            self._out = torch.empty(2, dtype=torch.int64, pin_memory=True)
            self._out_np = self._out.numpy()

    def _flush(self, stream) -> None:
        """Write the dirty slots into the device tables (one launch)."""
        m = len(self._dirty)
        if not m:
            return
        if self._stage is None or self._stage[0].numel() < m:
            size = max(64, 2 * m)
            st = tuple(torch.empty(size, dtype=torch.int64, pin_memory=True) for _ in range(3))
            self._stage = st + tuple(t.numpy() for t in st)
        t_slot, t_key, t_rank, a_slot, a_key, a_rank = self._stage
        slots = sorted(self._dirty)
        ids = [self._at[s] for s in slots]
        a_slot[:m] = slots
        a_key[:m] = [self._key.get(t, _INF) for t in ids]
        a_rank[:m] = [self._rank[t] for t in ids]
        N.check(N.load().zx_belady_update_slots(N.ptr(self._keys_dev), None, N.ptr(self._rank_dev), self._cap,
                                                N.ptr(t_slot), N.ptr(t_key), None, N.ptr(t_rank), m, None, stream),
                "belady_update_slots")
        self._dirty.clear()

    def _select_victim(self):  # belady.py:39-51, as one GPU argmax
        if not self._at:
            return None
        dev = self._device or ensure_gpu()
        self._tables(dev)
        cur = torch.cuda.current_stream(dev)
        stream = ctypes.c_void_p(cur.cuda_stream)
        self._flush(stream)
        lib = N.load()
        self._out_np[0] = _PENDING
        N.check(lib.zx_belady_argmax(N.ptr(self._keys_dev), None, N.ptr(self._rank_dev), len(self._at),
                                     N.ptr(self._out), N.ptr(self._ws), self._ws.numel(), stream), "belady_argmax")
        # The argmax writes its result into pinned host memory, after the slot updates that
        # read the staging arrays have run (same stream): watching that word returns as soon
        # as it lands, ~7 us sooner per eviction than a stream synchronisation (33k -> 40k
        # evictions/s at 488,281 resident ids).  Work queued on the stream before this call
        # can delay it for longer; after a while the wait becomes a synchronisation.
        t0 = time.perf_counter()
        spins = 0
        while self._out_np[0] == _PENDING:
            spins += 1
            if spins % 4096 == 0 and time.perf_counter() - t0 > 0.1:
                cur.synchronize()
                break
        slot = int(self._out_np[0])
        if slot == _PENDING:
            raise RuntimeError("belady_argmax: the kernel did not write its result")
        return None if slot < 0 else self._at[slot]

    @property
    def resident(self) -> set:
        return set(self._slot)


__all__ = ["BeladyApproxCache", "AccessEvent"]
