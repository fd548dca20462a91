"""Dynamic ring curriculum (README.md:19, 162-165, 192, 330, 345: ``RingDegreeScheduler``,
``CurriculumPhase``, "progressive ring degree expansion", "adaptive scheduling based on
loss landscape", "smooth interpolation between training phases"; the module
zenyx/train/dynamic_ring_curriculum.py is absent from the reference tree, so its
behaviour is defined here).

What it feeds on this path: the ring degree and context length of every training step
fix the order in which ring attention touches the KV pages, and that order is what the
Belady tiering plans over.  ``RingDegreeScheduler.access_trace`` builds the page trace of
any run of steps on the GPU (zx_ring_curriculum_trace), with page ids that stay the same
across phases (layer l owns ``layer_stride`` page ids, enough for the longest context),
so one Belady schedule can span phase changes.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Sequence

import torch

from .. import kv


@dataclass(frozen=True)
class CurriculumPhase:
    """One phase: ``steps`` training steps at ring degree ``ring_degree`` over
    ``context_length`` tokens.  ``steps = 0`` makes a phase open-ended (last phase only).
    During its first ``ramp_steps`` steps the context grows linearly from the previous
    phase's length (the smooth interpolation); the degree switches at the phase start."""

    name: str
    ring_degree: int
    context_length: int
    steps: int = 0
    ramp_steps: int = 0


class RingDegreeScheduler:
    """Ring degree and context length per training step.

    ``phases`` lists the curriculum; without it, the degree doubles from ``min_degree`` to
    ``num_devices`` in equal phases of ``total_steps`` with the context scaled with the
    degree (``context_length`` at the full degree).  With ``patience > 0`` the scheduler
    is adaptive: ``observe_loss`` advances to the next phase as soon as the loss has not
    improved by a relative ``min_delta`` over ``patience`` observations in a row (the
    later phases shift earlier)."""

    def __init__(self, phases: Sequence[CurriculumPhase] | None = None, *, num_devices: int = 8,
                 context_length: int | None = None, total_steps: int | None = None, min_degree: int = 1,
                 patience: int = 0, min_delta: float = 0.0):
        if phases is None:
            if context_length is None or total_steps is None:
                raise ValueError("give phases, or context_length and total_steps")
            degrees = []
            d = max(1, min_degree)
            while d < num_devices:
                degrees.append(d)
                d *= 2
            degrees.append(num_devices)
            per = max(1, total_steps // len(degrees))
            phases = [CurriculumPhase(f"ring{r}", r, max(1, context_length * r // num_devices),
                                      per if i + 1 < len(degrees) else 0)
                      for i, r in enumerate(degrees)]
        phases = list(phases)
        if not phases:
            raise ValueError("a curriculum needs at least one phase")
        for i, p in enumerate(phases):
            if p.ring_degree < 1 or p.context_length < 1 or p.steps < 0 or p.ramp_steps < 0:
                raise ValueError(f"phase {p.name!r}: degree and context must be >= 1, steps >= 0")
            if p.ring_degree > num_devices:
                raise ValueError(f"phase {p.name!r}: ring degree {p.ring_degree} > {num_devices} devices")
            if p.steps == 0 and i + 1 < len(phases):
                raise ValueError("only the last phase may be open-ended (steps = 0)")
            if p.steps and p.ramp_steps > p.steps:
                raise ValueError(f"phase {p.name!r}: ramp longer than the phase")
        self.phases = phases
        self.num_devices = num_devices
        self.patience, self.min_delta = int(patience), float(min_delta)
        self._starts = []
        s = 0
        for p in phases:
            self._starts.append(s)
            s += p.steps
        self._best = math.inf
        self._stale = 0

    # ------------------------------------------------------------------ lookup
    def phase_index(self, step: int) -> int:
        if step < 0:
            raise ValueError("step must be >= 0")
        i = 0
        while i + 1 < len(self.phases) and step >= self._starts[i + 1]:
            i += 1
        return i

    def phase_at(self, step: int) -> CurriculumPhase:
        return self.phases[self.phase_index(step)]

    def degree_at(self, step: int) -> int:
        return self.phase_at(step).ring_degree

    def context_at(self, step: int) -> int:
        i = self.phase_index(step)
        p = self.phases[i]
        into = step - self._starts[i]
        if i == 0 or p.ramp_steps == 0 or into >= p.ramp_steps:
            return p.context_length
        prev = self.phases[i - 1].context_length
        return prev + (p.context_length - prev) * (into + 1) // (p.ramp_steps + 1)

    def phase_start(self, i: int) -> int:
        return self._starts[i]

    # ------------------------------------------------------------------ adaptation
    def observe_loss(self, step: int, loss: float) -> bool:
        """Record the loss of ``step``; returns True when the curriculum moved on to the
        next phase (starting at step + 1)."""
        if self.patience <= 0:
            return False
        i = self.phase_index(step)
        if self._best == math.inf or loss < self._best - self.min_delta * abs(self._best):
            self._best, self._stale = float(loss), 0
            return False
        self._stale += 1
        if self._stale < self.patience or i + 1 >= len(self.phases) or self._starts[i + 1] <= step + 1:
            return False
        shift = self._starts[i + 1] - (step + 1)
        for j in range(i + 1, len(self.phases)):
            self._starts[j] -= shift
        self._best, self._stale = math.inf, 0
        return True

    # ------------------------------------------------------------------ KV page traces
    def pages_per_layer(self, step: int, page_tokens: int = 64) -> int:
        return -(-self.context_at(step) // page_tokens)

    def layer_stride(self, page_tokens: int = 64) -> int:
        """Page ids per layer: enough for the longest context of any phase."""
        return max(-(-p.context_length // page_tokens) for p in self.phases)

    def access_trace(self, steps: Sequence[int], num_layers: int, page_tokens: int = 64,
                     device: torch.device | None = None) -> torch.Tensor:
        """Device int32 page trace of the given training steps, concatenated; each step is
        its ring-attention forward (per layer, ring step, simulated device) and the exact
        reverse.  Page ids are [0, num_layers * layer_stride(page_tokens))."""
        steps = list(steps)
        deg = [self.degree_at(s) for s in steps]
        ctx = [self.pages_per_layer(s, page_tokens) for s in steps]
        return kv.ring_curriculum_trace(deg, ctx, num_layers, self.layer_stride(page_tokens), device=device)


__all__ = ["CurriculumPhase", "RingDegreeScheduler"]
