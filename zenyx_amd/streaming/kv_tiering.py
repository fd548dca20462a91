"""Drop-in for zenyx/streaming/kv_tiering.py: T0 (HBM) / T1 (host DRAM) / T2 (cold) KV
tiers with LRU spill, and the ring-attention access timeline.

Same public surface as the reference (kv_tiering.py:11-73): ``KVBlockRef``,
``KVTierManager(t0_capacity, t1_capacity)`` with the ``t0``/``t1``/``t2`` dicts, ``put``,
``prefetch_to_t0``, ``evict_from_t0``, and ``build_ring_timeline``.  The copies the
reference does with ``.to(device)`` / ``.cpu()`` (kv_tiering.py:46, 54, 60) go through
zx_tier_copy_runs (hipMemcpyAsync) on a side stream:
  * host -> device: the side stream waits for the caller's stream, copies, and the caller's
    stream waits for the copy, so the returned tensor is ready for the caller's kernels
    without blocking the host;
  * device -> host: the destination is pinned host memory; the copy runs on the side stream
    (overlapping kernels on other streams) and the host waits only for that copy, because
    the reference hands back a CPU tensor that is ready to read.
Eviction policy, capacities, KeyError on unknown ids and the aliasing of CPU tensors by
``put`` (``.cpu()`` of a CPU tensor is the same tensor) follow the reference.
"""
from __future__ import annotations

import threading

import ctypes
from collections import OrderedDict
from dataclasses import dataclass

import torch

from .. import _native as N
from .._streams import all_copy_streams, copy_stream


@dataclass
class KVBlockRef:
    """kv_tiering.py:11-15."""

    block_id: int
    seq_start: int
    seq_end: int


class _SideStream:
    """The tier copies' side stream of a device (the library's shared h2d copy stream)."""

    @staticmethod
    def get(device: torch.device) -> torch.cuda.Stream:
        return copy_stream(device, "h2d")


def _copy(dst: torch.Tensor, src: torch.Tensor, stream: torch.cuda.Stream) -> None:
    nbytes = src.numel() * src.element_size()
    if nbytes == 0:
        return
    off = (ctypes.c_int64 * 1)(0)
    N.check(N.load().zx_tier_copy_runs(N.ptr(dst), N.ptr(src), off, off, 1, nbytes,
                                       ctypes.c_void_p(stream.cuda_stream), None), "tier copy")


class _HostKeepAlive:
    """Host tensors read by copies still queued on a stream.

    A copy issued through hipMemcpyAsync is invisible to torch's pinned-memory caching
    allocator, which would hand a freed pinned block to the next pin_memory() request
    (another tier move, a DataLoader) while the DMA still reads it.  Each source is held
    here with an event recorded after its copy and dropped once the event has completed;
    completed entries are released whenever a new one is added or ``release_done`` runs.
    """

    _pending: list = []  # (event, tensor), in the order the copies were queued
    _lock = threading.Lock()  # the list is shared by every mover of the process

    @classmethod
    def hold(cls, tensor: torch.Tensor, stream: torch.cuda.Stream) -> None:
        ev = torch.cuda.Event()
        ev.record(stream)
        with cls._lock:
            cls._pending = [(e, t) for e, t in cls._pending if not e.query()]
            cls._pending.append((ev, tensor))

    @classmethod
    def release_done(cls) -> None:
        with cls._lock:
            cls._pending = [(ev, t) for ev, t in cls._pending if not ev.query()]

    @classmethod
    def release_all(cls) -> None:
        with cls._lock:
            pending, cls._pending = cls._pending, []
        for ev, _ in pending:
            ev.synchronize()


def keep_host_alive(tensor: torch.Tensor, stream: torch.cuda.Stream) -> None:
    """Keep ``tensor`` (the host side of a copy just queued on ``stream``) referenced until
    that copy has run."""
    _HostKeepAlive.hold(tensor, stream)


def to_device(cpu_tensor: torch.Tensor, device: torch.device) -> torch.Tensor:
    """Host tensor -> new device tensor, copied on the side stream, ordered before any later
    work on the caller's current stream.  The host tensor stays referenced until the copy
    has run, so the caller may drop it at once."""
    N.ensure_gpu()
    src = cpu_tensor.contiguous()
    cur = torch.cuda.current_stream(device)
    side = _SideStream.get(device)
    out = torch.empty(src.shape, dtype=src.dtype, device=device)
    side.wait_stream(cur)
    _copy(out, src, side)
    keep_host_alive(src, side)
    out.record_stream(side)
    cur.wait_stream(side)
    return out


def to_host(gpu_tensor: torch.Tensor) -> torch.Tensor:
    """Device tensor -> pinned host tensor; returns once the copy (on the side stream) is done."""
    N.ensure_gpu()
    src = gpu_tensor.detach().contiguous()
    dev = src.device
    cur = torch.cuda.current_stream(dev)
    side = _SideStream.get(dev)
    out = torch.empty(src.shape, dtype=src.dtype, pin_memory=True)
    side.wait_stream(cur)
    _copy(out, src, side)
    src.record_stream(side)
    done = torch.cuda.Event()
    done.record(side)
    done.synchronize()
    return out


class KVTierManager:
    """Three places a KV block can live, with least-recently-used spill between them
    (behaviour of kv_tiering.py:18-66).

    ``t0`` maps block ids to device tensors, at most ``t0_capacity`` of them; ``t1`` maps
    ids to pinned host copies, at most ``t1_capacity``; ``t2`` keeps every block that was
    ``put`` plus whatever overflows ``t1``, with no bound.  Each ordered dict lists its
    blocks oldest use first, so an overflow always spills the front entry one level down.
    """

    def __init__(self, t0_capacity: int = 2, t1_capacity: int = 32):
        self.t0: OrderedDict[int, torch.Tensor] = OrderedDict()
        self.t1: OrderedDict[int, torch.Tensor] = OrderedDict()
        self.t2: dict[int, torch.Tensor] = {}
        self.t0_capacity = t0_capacity
        self.t1_capacity = t1_capacity

    def put(self, block_id: int, tensor: torch.Tensor) -> None:  # kv_tiering.py:33-34
        data = tensor.detach()
        # a host tensor is kept as it is (no copy), as .cpu() would return it
        self.t2[block_id] = data if data.device.type == "cpu" else to_host(data)

    def prefetch_to_t0(self, block_id: int, device: torch.device) -> torch.Tensor:  # :36-49
        hit = self.t0.get(block_id)
        if hit is not None:
            self.t0.move_to_end(block_id)  # now the most recent use
            return hit
        # a T1 block leaves T1; a T2 block stays in T2 (only read); an unknown id is a KeyError
        host = self.t1.pop(block_id) if block_id in self.t1 else self.t2[block_id]
        target = torch.device(device)
        self.t0[block_id] = resident = to_device(host, target) if target.type == "cuda" else host.to(target)
        self._spill()
        return resident

    def evict_from_t0(self, block_id: int) -> None:  # :51-55
        if block_id not in self.t0:
            return
        self.t1[block_id] = _host_copy(self.t0.pop(block_id))
        self._spill()

    def synchronize(self, device: torch.device | None = None) -> None:
        """Wait until the tier copies queued on the side stream (of ``device``, or of every
        device used so far) are done.  Copies to host already complete before returning, as
        ``.cpu()`` does in the reference; copies to the device are ordered before later
        work on the caller's stream and need this only when another stream or the host
        reads them."""
        streams = [_SideStream.get(torch.device(device))] if device is not None else all_copy_streams()
        for s in streams:
            s.synchronize()
        _HostKeepAlive.release_done()

    def _spill(self) -> None:
        """Restore both capacity bounds: the oldest T0 blocks go to T1 (copied to the host),
        then the oldest T1 blocks go to T2 (moved as they are).  Moving every T0 overflow
        first and trimming T1 afterwards leaves the same tiers, in the same orders, as
        trimming T1 after each single move (:57-66): both take T1's oldest entries."""
        while len(self.t0) > self.t0_capacity:
            block_id, tensor = self.t0.popitem(last=False)
            self.t1[block_id] = _host_copy(tensor)
        while len(self.t1) > self.t1_capacity:
            block_id, tensor = self.t1.popitem(last=False)
            self.t2[block_id] = tensor


def _host_copy(tensor: torch.Tensor) -> torch.Tensor:
    return to_host(tensor) if tensor.device.type == "cuda" else tensor.detach()


def build_ring_timeline(num_blocks: int) -> dict[str, list[int]]:
    """Block ids in ring order for the forward sweep, and the same ids reversed for the
    backward sweep (behaviour of kv_tiering.py:69-73)."""
    forward = list(range(num_blocks))
    backward = list(reversed(forward))
    return {"forward": forward, "backward": backward}


__all__ = ["KVTierManager", "KVBlockRef", "build_ring_timeline", "keep_host_alive"]
