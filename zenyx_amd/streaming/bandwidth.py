"""Drop-in for zenyx/streaming/bandwidth.py:8-29: the fetch-versus-compute throttle rule.

``BandwidthSample(fetch_time_ms, compute_time_ms)`` and
``BandwidthAwareScheduler(max_fetch_to_compute_ratio=1.0)`` keep the reference's names and
decisions (its test, zenyx/tests/test_streaming.py:25-28, holds here unchanged):

* a sample with no compute time (``<= 0``) always throttles;
* otherwise it throttles when fetch / compute exceeds the ratio;
* the delay is the part of the fetch that compute did not cover, never negative, and 0
  when the sample does not throttle.

Host logic only.  ``StreamingExecutionEngine`` holds one as ``bandwidth`` for callers
that consult it, but does not sleep on it: its weight fetches are enqueued on a side
stream and never block the host, so a host-timed fetch is ~0 and the rule would never
ask for a delay.
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass
class BandwidthSample:
    """One layer's measured fetch and compute time (bandwidth.py:8-11)."""

    fetch_time_ms: float
    compute_time_ms: float


class BandwidthAwareScheduler:
    """Throttle decision when transfers dominate compute (bandwidth.py:14-29)."""

    def __init__(self, max_fetch_to_compute_ratio: float = 1.0):
        self.max_ratio = max_fetch_to_compute_ratio

    def should_throttle(self, sample: BandwidthSample) -> bool:
        compute = sample.compute_time_ms
        return True if compute <= 0 else sample.fetch_time_ms / compute > self.max_ratio

    def throttle_ms(self, sample: BandwidthSample) -> float:
        if not self.should_throttle(sample):
            return 0.0
        return max(0.0, sample.fetch_time_ms - sample.compute_time_ms)


__all__ = ["BandwidthSample", "BandwidthAwareScheduler"]
