"""A paged FP8 KV cache of many layers streamed through a few HBM layer slots and pinned
host DRAM (README.md:151-154, Phase 7: "Streams 516 GB KV cache through 16 GB HBM"; the
module behind that claim is absent from the reference tree, so the behaviour is defined
here).

The cache serves one training step's layer sweep: a forward pass appends every layer in
order 0 .. L-1, a backward pass gathers them in order L-1 .. 0.  Only ``hbm_layers`` = S
layer pools fit in HBM.  When layer l >= S needs a slot, the resident layer whose next use
is farthest goes (Belady): in the backward sweep that is the lowest-numbered resident
layer, i.e. layer l - S.  So the layers 0 .. L-S-1 are the spilled ones, known in advance:
each is written back to pinned host memory on the library's d2h copy stream right after
its own append (write-behind), and the append that reuses its slot waits only for that
copy.  In the backward sweep, the slot a gather frees at once receives the H2D prefetch of
the spilled layer S positions later in the sweep (layer l - S), on the h2d copy stream,
and that layer's gather waits for its copy.  Every wait is an event between the caller's
stream and a copy stream; the host never blocks.
"""
from __future__ import annotations

import torch

from .. import _native as N
from .. import kv
from .._streams import copy_stream


class LayerStreamedKVCache:
    """``num_layers`` layers of a paged FP8 KV cache (each ``[n_pages, 2, H, P, D]`` codes,
    scales ``[L, 2, H]``), ``hbm_layers`` of them in HBM at a time, the rest in pinned DRAM.

    ``append_layer(l, ...)`` for l = 0 .. L-1, then ``gather_layer(l, ...)`` for l = L-1 .. 0;
    ``reset()`` starts the next step with the same buffers.  With ``timing=True`` every
    append, gather and tier copy is bracketed by events (``events``)."""

    def __init__(self, num_layers: int, hbm_layers: int, n_pages: int, num_kv_heads: int = 8,
                 head_dim: int = 128, page_size: int = 16, device: torch.device | None = None,
                 timing: bool = False):
        if num_layers < 1 or hbm_layers < 1 or n_pages < 1:
            raise ValueError("num_layers, hbm_layers and n_pages must be positive")
        self.device = device or N.ensure_gpu()
        self.L, self.S = num_layers, min(hbm_layers, num_layers)
        self.n_spill = self.L - self.S
        shape = (n_pages, 2, num_kv_heads, page_size, head_dim)
        self.layer_shape = shape
        self.layer_bytes = n_pages * 2 * num_kv_heads * page_size * head_dim
        self.slots = torch.empty((self.S,) + shape, dtype=torch.uint8, device=self.device)
        self.host = (torch.empty((self.n_spill,) + shape, dtype=torch.uint8, pin_memory=True)
                     if self.n_spill else None)
        self.scales = torch.empty((self.L, 2, num_kv_heads), dtype=torch.float32, device=self.device)
        self.err = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.d2h = copy_stream(self.device, "d2h")  # write-behind of the spilled layers
        self.h2d = copy_stream(self.device, "h2d")  # prefetch back into freed slots
        self.timing = timing
        self.reset()

    def reset(self) -> None:
        """Start a new sweep (forward from layer 0) over the same buffers."""
        self.slot_of: dict[int, int] = {}
        self._d2h_done: dict[int, torch.cuda.Event] = {}
        self._h2d_done: dict[int, torch.cuda.Event] = {}
        self._next_fwd, self._next_bwd = 0, self.L - 1
        self.events = {"append": [], "gather": [], "d2h": [], "h2d": []}

    def _event(self):
        return torch.cuda.Event(enable_timing=self.timing)

    def _copy(self, dst: torch.Tensor, src: torch.Tensor, kind: str) -> torch.cuda.Event:
        side = self.d2h if kind == "d2h" else self.h2d
        e0 = self._event()
        e0.record(side)
        kv.tier_copy_runs(dst, src, [0], [0], self.layer_bytes, stream=side)
        e1 = self._event()
        e1.record(side)
        if self.timing:
            self.events[kind].append((e0, e1))
        return e1

    def append_layer(self, layer: int, x: torch.Tensor, cu_seqlens: torch.Tensor, block_tables: torch.Tensor,
                     start_pos: torch.Tensor | None = None) -> None:
        """Forward step: quantise and append layer ``layer``'s tokens x ``[n_tok, 2, H, D]``
        bf16 (dynamic per-(kv, head) scales) into its HBM slot; a layer that will be spilled
        is written back to pinned DRAM right after."""
        if layer != self._next_fwd:
            raise ValueError(f"append_layer expects layer {self._next_fwd} next (forward order), got {layer}")
        comp = torch.cuda.current_stream(self.device)
        if layer >= self.S:  # the slot of layer - S, whose write-behind must be done
            comp.wait_event(self._d2h_done[layer - self.S])
            slot = self.slot_of.pop(layer - self.S)
        else:
            slot = layer
        self.slot_of[layer] = slot
        e0, e1 = self._event(), self._event()
        e0.record(comp)
        kv.kv_quant_append(x, cu_seqlens, block_tables, self.slots[slot], scales=self.scales[layer:layer + 1],
                           start_pos=start_pos, err=self.err)
        e1.record(comp)
        if self.timing:
            self.events["append"].append((e0, e1))
        if layer < self.n_spill:  # a future victim: write it back now
            self.d2h.wait_event(e1)
            self._d2h_done[layer] = self._copy(self.host[layer], self.slots[slot], "d2h")
        self._next_fwd += 1

    def gather_layer(self, layer: int, block_tables: torch.Tensor, seq_lens: torch.Tensor, out_len: int,
                     out: tuple[torch.Tensor, torch.Tensor] | None = None):
        """Backward step: gather + dequantise layer ``layer`` -> bf16 (k, v) ``[B, H, out_len, D]``
        (into ``out`` if given); the freed slot receives the next spilled layer."""
        if self._next_fwd != self.L:
            raise ValueError("gather_layer needs the forward sweep (every append_layer) first")
        if layer != self._next_bwd:
            raise ValueError(f"gather_layer expects layer {self._next_bwd} next (backward order), got {layer}")
        comp = torch.cuda.current_stream(self.device)
        if layer < self.n_spill:
            comp.wait_event(self._h2d_done[layer])
        slot = self.slot_of.pop(layer)
        e0, e1 = self._event(), self._event()
        e0.record(comp)
        k, v = kv.kv_gather_dequant(self.slots[slot], self.scales[layer], block_tables, seq_lens, out_len, out=out)
        e1.record(comp)
        if self.timing:
            self.events["gather"].append((e0, e1))
        nxt = layer - self.S
        if 0 <= nxt < self.n_spill:  # prefetch that layer into the slot just freed
            self.h2d.wait_event(e1)
            self._h2d_done[nxt] = self._copy(self.slots[slot], self.host[nxt], "h2d")
            self.slot_of[nxt] = slot
        self._next_bwd -= 1
        return k, v

    def check_errors(self) -> None:
        """Raise ValueError if any append flagged a bad page id or position (synchronises)."""
        e = int(self.err.item())
        if e:
            self.err.zero_()
            raise ValueError("LayerStreamedKVCache: " + kv.kernel_error_text(e))


__all__ = ["LayerStreamedKVCache"]
