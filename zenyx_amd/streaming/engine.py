"""Drop-in for zenyx/streaming/engine.py: the layer-streamed forward/backward driver, the
only in-tree caller of the Belady cache, the KV tiers and the weight streamer.

``StreamingConfig`` (engine.py:18-22) and ``StreamingExecutionEngine(model, device,
config)`` with ``run_forward_backward(x, target, loss_fn) -> float`` (engine.py:59-103)
keep the reference's call order, which is what this path has to reproduce:

* at construction each direct child of the model is one layer; its flattened state goes
  into the ParameterStore (an empty state registers one zero, as the reference does);
* per layer i in order: prefetch layer i + 1, ``get`` layer i, run the layer on the
  previous activation, ``update_future(name, i + 1)`` then ``touch(name)`` on the Belady
  cache, and ``evict`` every returned victim from the weight streamer;
* the loss, its backward, then the backward ring timeline over the KV tier manager:
  each block found in T2 is prefetched to T0 and evicted again (engine.py:96-101).

The layers compute with their own parameters, as in the reference (the streamed copy
is fetched but not bound into the module).  The engine holds the reference's
``BandwidthAwareScheduler`` as ``bandwidth`` (engine.py:46) but does not sleep on it (the
host sleep of engine.py:79-85): ``get`` here never blocks the host, so its fetch time is
~0 and the rule would never ask for a delay.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import torch
import torch.nn as nn

from .bandwidth import BandwidthAwareScheduler
from .belady import BeladyApproxCache
from .kv_tiering import KVTierManager, build_ring_timeline
from .parameter_streamer import LayerWeightStreamer, ParameterStore


@dataclass
class StreamingConfig:
    """engine.py:18-22."""

    max_hbm_layers: int = 2
    kv_t0_blocks: int = 2
    kv_t1_blocks: int = 64


class StreamingExecutionEngine:
    """Prefetch -> compute -> evict per layer, then backward (engine.py:25-103)."""

    def __init__(self, model: nn.Module, device: torch.device, config: StreamingConfig | None = None):
        self.model = model
        self.device = torch.device(device)
        self.config = config or StreamingConfig()
        self.store = ParameterStore()
        self.layer_names: list[str] = []
        self.layers: list[nn.Module] = []
        for name, module in model.named_children():
            self.layer_names.append(name)
            self.layers.append(module)
            state = [t.detach().reshape(-1).cpu() for t in module.state_dict().values()]
            self.store.register(name, torch.cat(state) if state else torch.zeros(1))
        self.weight_streamer = LayerWeightStreamer(self.store, device=self.device,
                                                   max_resident_layers=self.config.max_hbm_layers)
        self.kv_manager = KVTierManager(t0_capacity=self.config.kv_t0_blocks, t1_capacity=self.config.kv_t1_blocks)
        self.cache = BeladyApproxCache(capacity=self.config.max_hbm_layers)
        self.bandwidth = BandwidthAwareScheduler(max_fetch_to_compute_ratio=1.0)

    def run_forward_backward(self, x: torch.Tensor, target: torch.Tensor,
                             loss_fn: Callable[[torch.Tensor, torch.Tensor], torch.Tensor]) -> float:
        act = x.to(self.device)
        target = target.to(self.device)
        n = len(self.layer_names)
        for i, (name, layer) in enumerate(zip(self.layer_names, self.layers)):
            if i + 1 < n:
                self.weight_streamer.prefetch(self.layer_names[i + 1])
            self.weight_streamer.get(name)
            act = layer(act)
            self.cache.update_future(name, i + 1)
            for victim in self.cache.touch(name):
                self.weight_streamer.evict(victim)
        loss = loss_fn(act, target)
        loss.backward()
        for block_id in build_ring_timeline(num_blocks=max(1, n))["backward"]:
            if block_id in self.kv_manager.t2:
                self.kv_manager.prefetch_to_t0(block_id, self.device)
                self.kv_manager.evict_from_t0(block_id)
        return float(loss.item())


__all__ = ["StreamingExecutionEngine", "StreamingConfig"]
