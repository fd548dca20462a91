"""Drop-in for zenyx/streaming/belady.py: Belady approximation by next-use distance.

``BeladyApproxCache`` keeps the reference contract (belady.py:14-55): ``update_future``
records an id's next use, ``touch`` admits an id and, when the cache is full, evicts the
resident id whose next use is farthest (unknown ids count as 10**18, belady.py:47).  The
farthest-next-use scan runs on the GPU (zx_belady_argmax over a device table of keys and
residency flags); the id <-> slot bookkeeping stays on the host.

Kept reference behaviour (belady.py:30-36, 45-51):
  * a victim must have next use > -1, so if every resident id has next use <= -1 nothing is
    evicted and the resident set grows past the capacity;
  * capacity 0 behaves like capacity 1 (the size test is ``len >= capacity``).
One liberty: the reference breaks ties by iterating a Python ``set`` (order unspecified);
here ties go to the id registered first (first seen by ``update_future`` or ``touch``).
Not thread-safe, like the reference.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import kv
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
    """Evict tensors with farthest known next-use (Belady approximation), on the GPU."""

    def __init__(self, capacity: int, device: torch.device | None = None):
        self.capacity = capacity
        self._device = device
        self._slot: dict = {}
        self._ids: list = []
        self._resident: dict = {}  # insertion-ordered set of resident ids
        self._keys_host: list[int] = []
        self._dirty = True
        self._keys_dev: torch.Tensor | None = None
        self._res_dev: torch.Tensor | None = None

    def _reg(self, tensor_id) -> int:
        s = self._slot.get(tensor_id)
        if s is None:
            s = len(self._ids)
            self._slot[tensor_id] = s
            self._ids.append(tensor_id)
            self._keys_host.append(_INF)
            self._dirty = True
        return s

    def update_future(self, tensor_id, next_use_step: int) -> None:  # belady.py:22-23
        s = self._reg(tensor_id)
        v = int(next_use_step)
        self._keys_host[s] = min(max(v, _I64_MIN), _I64_MAX)
        self._dirty = True

    def touch(self, tensor_id) -> list:  # belady.py:25-37
        self._reg(tensor_id)
        evicted: list = []
        if tensor_id in self._resident:
            return evicted
        if len(self._resident) >= self.capacity:
            victim = self._select_victim()
            if victim is not None:
                del self._resident[victim]
                self._dirty = True
                evicted.append(victim)
        self._resident[tensor_id] = True
        self._dirty = True
        return evicted

    def _select_victim(self):  # belady.py:39-51, as one GPU argmax
        if not self._resident:
            return None
        dev = self._device or ensure_gpu()
        if self._dirty:
            res = [0] * len(self._ids)
            for tid in self._resident:
                res[self._slot[tid]] = 1
            self._keys_dev = torch.tensor(self._keys_host, dtype=torch.int64).to(dev)
            self._res_dev = torch.tensor(res, dtype=torch.uint8).to(dev)
            self._dirty = False
        slot, _ = kv.belady_argmax(self._keys_dev, self._res_dev).tolist()
        return None if slot < 0 else self._ids[slot]

    @property
    def resident(self) -> set:
        return set(self._resident)


__all__ = ["BeladyApproxCache", "AccessEvent"]
