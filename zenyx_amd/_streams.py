"""The library's copy streams: two per device, shared by every tier mover, weight streamer
and replay (``"h2d"`` for host -> device and general tier copies, ``"d2h"`` for device ->
host write-backs), all at the default priority.

A process gets a few hardware queues (4 by default on ROCm) and HIP hands them to
streams round-robin, so creating a stream per object or per call eventually puts a copy
stream on the compute stream's queue, where the two serialise and copies stop overlapping
kernels.  Reusing two streams keeps the library at three queues with the compute stream.
"""
from __future__ import annotations

import threading

import torch

_pool: dict = {}
_lock = threading.Lock()


def copy_stream(device: torch.device | int | str | None = None, direction: str = "h2d") -> torch.cuda.Stream:
    """The shared copy stream of ``device`` (default: the current one) for ``direction``."""
    if direction not in ("h2d", "d2h"):
        raise ValueError('direction must be "h2d" or "d2h"')
    if device is None:
        idx = torch.cuda.current_device()
    else:
        d = torch.device(device) if not isinstance(device, int) else torch.device("cuda", device)
        idx = d.index if d.index is not None else torch.cuda.current_device()
    key = (idx, direction)
    s = _pool.get(key)
    if s is None:
        with _lock:
            s = _pool.get(key)
            if s is None:
                s = torch.cuda.Stream(device=idx)  # default priority
                _pool[key] = s
    return s


def all_copy_streams() -> list:
    return list(_pool.values())


def teardown() -> None:
    """Finish the library's device work before the interpreter shuts down: wait for the
    copy streams and the devices they belong to (and the current one), then drop the host tensors and
    events kept for copies in flight (they would otherwise be destroyed during
    finalisation, after the HIP runtime may have begun its own teardown).  Registered
    with atexit when the library is first loaded; safe to call more than once."""
    if not torch.cuda.is_initialized():
        return
    used = {torch.cuda.current_device()} | {idx for idx, _ in _pool}
    for s in all_copy_streams():
        s.synchronize()
    for idx in sorted(used):
        with torch.cuda.device(idx):
            torch.cuda.synchronize()
    from .streaming.kv_tiering import _HostKeepAlive

    _HostKeepAlive.release_all()
