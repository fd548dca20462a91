"""Drop-in for zenyx/streaming/parameter_streamer.py: layer-wise weight streaming with
prefetch and a bounded set of resident layers, on the same pinned-DRAM -> HBM transfer
engine as the KV tiers.

Same public surface as the reference (parameter_streamer.py:13-87): ``LayerBlock``,
``ParameterStore`` (``register``, ``load``, ``blocks``) and ``LayerWeightStreamer(store,
device, min_block_bytes, max_resident_layers)`` with ``prefetch``, ``get`` and ``evict``;
resident layers are evicted least recently used first beyond ``max_resident_layers``,
and an unknown layer id raises KeyError, as in the reference.  What changes:

* ``ParameterStore.register`` copies the weights into pinned host memory once; the
  reference pins a fresh copy on every load (parameter_streamer.py:85).
* a load is one zx_tier_copy_runs (hipMemcpyAsync) of the whole layer on a side stream,
  not a ``.to(device, non_blocking=True)`` from a worker thread; ``get`` makes the
  caller's current stream wait for that copy through an event instead of blocking the
  host, so a prefetched layer streams in while the previous layer computes.
* ``min_block_bytes`` is accepted for compatibility; the reference only uses it to call
  ``.contiguous()`` on an already contiguous tensor (parameter_streamer.py:82-83).
"""
from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass

import torch

from .. import _native as N
from .. import kv
from .._streams import copy_stream
from .kv_tiering import keep_host_alive


@dataclass
class LayerBlock:
    """parameter_streamer.py:13-16."""

    layer_id: str
    tensor: torch.Tensor


class ParameterStore:
    """Every layer's weights kept in pinned host memory, by layer id (the role of
    parameter_streamer.py:19-29); ``load`` hands back the pinned tensor itself."""

    def __init__(self):
        self.blocks: dict[str, torch.Tensor] = {}

    def register(self, layer_id: str, tensor: torch.Tensor) -> None:
        t = tensor.detach()
        host = torch.empty(t.shape, dtype=t.dtype, pin_memory=torch.cuda.is_available())
        host.copy_(t)
        self.blocks[layer_id] = host

    def load(self, layer_id: str) -> torch.Tensor:
        return self.blocks[layer_id]


class LayerWeightStreamer:
    """Device copies of layer weights, fetched ahead of use on the library's copy stream;
    at most ``max_resident_layers`` are kept, the least recently used dropped first (the
    role of parameter_streamer.py:32-87)."""

    def __init__(self, store: ParameterStore, device: torch.device, min_block_bytes: int = 5 * 1024 * 1024,
                 max_resident_layers: int = 2):
        self.store = store
        self.device = torch.device(device)
        self.min_block_bytes = min_block_bytes
        self.max_resident_layers = max_resident_layers
        self._resident: OrderedDict[str, torch.Tensor] = OrderedDict()
        self._prefetch: dict = {}  # layer id -> (tensor, copy-done event), or the KeyError to raise
        self._side = None
        if self.device.type == "cuda":
            N.ensure_gpu()
            self._side = copy_stream(self.device, "h2d")

    def prefetch(self, layer_id: str) -> None:
        if layer_id in self._resident or layer_id in self._prefetch:
            return
        try:
            self._prefetch[layer_id] = self._start_load(layer_id)
        except KeyError as e:  # the reference's future raises at get(), not here
            self._prefetch[layer_id] = e

    def get(self, layer_id: str) -> torch.Tensor:
        if layer_id in self._resident:
            self._resident.move_to_end(layer_id)
            return self._resident[layer_id]
        pending = self._prefetch.pop(layer_id, None)
        if isinstance(pending, KeyError):
            raise pending
        if pending is None:
            pending = self._start_load(layer_id)
        tensor, done = pending
        if done is not None:
            torch.cuda.current_stream(self.device).wait_event(done)
        self._resident[layer_id] = tensor
        self._evict_if_needed()
        return tensor

    def evict(self, layer_id: str) -> None:
        self._resident.pop(layer_id, None)

    def _evict_if_needed(self) -> None:
        while len(self._resident) > self.max_resident_layers:
            self._resident.popitem(last=False)

    def _start_load(self, layer_id: str):
        host = self.store.load(layer_id)  # KeyError for an unknown layer, as the reference
        if self.device.type != "cuda":
            return host.to(self.device), None
        if not host.is_pinned():
            host = host.pin_memory()
        out = torch.empty(host.shape, dtype=host.dtype, device=self.device)
        nbytes = host.numel() * host.element_size()
        cur = torch.cuda.current_stream(self.device)
        done = torch.cuda.Event()
        self._side.wait_stream(cur)  # `out` may reuse memory the current stream just freed
        if nbytes:
            kv.tier_copy_runs(out, host, [0], [0], nbytes, stream=self._side)
            keep_host_alive(host, self._side)  # a temporary pinned copy must outlive the DMA
        out.record_stream(self._side)
        done.record(self._side)
        return out, done


__all__ = ["ParameterStore", "LayerWeightStreamer", "LayerBlock"]
