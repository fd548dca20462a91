"""Drop-in for zenyx/streaming/belady.py: Belady approximation by next-use distance.

``BeladyApproxCache`` keeps the reference contract (belady.py:14-55): ``update_future``
records an id's next use, ``touch`` admits an id and, when the cache is full, evicts the
resident id whose next use is farthest (unknown ids count as 10**18, belady.py:47).  The
farthest-next-use scan runs on the GPU (zx_belady_argmax over device tables of keys and
residency flags, kept in place and updated slot by slot); the id <-> slot bookkeeping
stays on the host.

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
from dataclasses import dataclass

import torch

from .. import _native as N
from .._native import ensure_gpu

_INF = 10**18
_I64_MAX = 2**63 - 1
_I64_MIN = -(2**63)


@dataclass
class AccessEvent:
    """belady.py:8-11 (unused by the reference itself; kept for the import surface)."""

    tensor_id: str
    step: int


class BeladyApproxCache:
    """Evict tensors with farthest known next-use (Belady approximation), on the GPU.

    The next-use keys and residency flags live in device tables indexed by slot (one slot
    per id, in registration order).  ``update_future`` and ``touch`` only change a host
    mirror and mark the slot dirty; a miss on a full cache first writes the dirty slots
    (one zx_belady_update_slots launch reading them from pinned host memory), then runs
    the argmax (zx_belady_argmax) over the tables, whose {slot, key} result lands in
    pinned host memory, and waits for that stream once.  Host work per eviction is O(1)
    plus the slots changed since the previous one."""

    def __init__(self, capacity: int, device: torch.device | None = None):
        self.capacity = capacity
        self._device = device
        self._slot: dict = {}
        self._ids: list = []
        self._keys: list[int] = []  # host mirror of the next-use keys, by slot
        self._resident: dict = {}  # insertion-ordered set of resident ids
        self._dirty: set = set()  # slots whose device entry is stale
        self._cap = 0  # slots the device tables hold
        self._keys_dev: torch.Tensor | None = None
        self._res_dev: torch.Tensor | None = None
        self._ws: torch.Tensor | None = None
        self._stage = None  # pinned (slot, key, res) staging arrays and their numpy views
        self._out: torch.Tensor | None = None  # pinned int64 [2]: {slot, key} of the last argmax

    def _reg(self, tensor_id) -> int:
        s = self._slot.get(tensor_id)
        if s is None:
            s = len(self._ids)
            self._slot[tensor_id] = s
            self._ids.append(tensor_id)
            self._keys.append(_INF)
            self._dirty.add(s)
        return s

    def update_future(self, tensor_id, next_use_step: int) -> None:  # belady.py:22-23
        s = self._reg(tensor_id)
        v = int(next_use_step)
        self._keys[s] = min(max(v, _I64_MIN), _I64_MAX)
        self._dirty.add(s)

    def touch(self, tensor_id) -> list:  # belady.py:25-37
        s = self._reg(tensor_id)
        evicted: list = []
        if tensor_id in self._resident:
            return evicted
        if len(self._resident) >= self.capacity:
            victim = self._select_victim()
            if victim is not None:
                del self._resident[victim]
                self._dirty.add(self._slot[victim])
                evicted.append(victim)
        self._resident[tensor_id] = True
        self._dirty.add(s)
        return evicted

    def _tables(self, dev: torch.device) -> None:
        """Grow the device tables (geometrically) to hold every registered slot."""
        n = len(self._ids)
        if n <= self._cap:
            return
        cap = max(1024, 2 * n)
        keys = torch.full((cap,), _INF, dtype=torch.int64, device=dev)
        res = torch.zeros(cap, dtype=torch.uint8, device=dev)
        if self._cap:
            keys[:self._cap].copy_(self._keys_dev)
            res[:self._cap].copy_(self._res_dev)
        self._keys_dev, self._res_dev, self._cap = keys, res, cap
        lib = N.load()
        self._ws = torch.empty(max(256, lib.zx_belady_argmax_workspace_bytes(cap)), dtype=torch.uint8, device=dev)
        if self._out is None:
            self._out = torch.empty(2, dtype=torch.int64, pin_memory=True)

    def _flush(self, dev: torch.device, stream) -> None:
        """Write the dirty slots into the device tables (one launch)."""
        m = len(self._dirty)
        if not m:
            return
        if self._stage is None or self._stage[0].numel() < m:
            size = max(64, 2 * m)
            st = (torch.empty(size, dtype=torch.int64, pin_memory=True),
                  torch.empty(size, dtype=torch.int64, pin_memory=True),
                  torch.empty(size, dtype=torch.uint8, pin_memory=True))
            self._stage = st + tuple(t.numpy() for t in st)
        t_slot, t_key, t_res, a_slot, a_key, a_res = self._stage
        slots = sorted(self._dirty)
        a_slot[:m] = slots
        a_key[:m] = [self._keys[s] for s in slots]
        a_res[:m] = [self._ids[s] in self._resident for s in slots]
        N.check(N.load().zx_belady_update_slots(N.ptr(self._keys_dev), N.ptr(self._res_dev), self._cap,
                                                N.ptr(t_slot), N.ptr(t_key), N.ptr(t_res), m, None, stream),
                "belady_update_slots")
        self._dirty.clear()

    def _select_victim(self):  # belady.py:39-51, as one GPU argmax
        if not self._resident:
            return None
        dev = self._device or ensure_gpu()
        self._tables(dev)
        cur = torch.cuda.current_stream(dev)
        stream = ctypes.c_void_p(cur.cuda_stream)
        self._flush(dev, stream)
        lib = N.load()
        N.check(lib.zx_belady_argmax(N.ptr(self._keys_dev), N.ptr(self._res_dev), len(self._ids), N.ptr(self._out),
                                     N.ptr(self._ws), self._ws.numel(), stream), "belady_argmax")
        cur.synchronize()  # the staging arrays are free again and the result is in pinned memory
        slot = int(self._out[0])
        return None if slot < 0 else self._ids[slot]

    @property
    def resident(self) -> set:
        return set(self._resident)


__all__ = ["BeladyApproxCache", "AccessEvent"]
