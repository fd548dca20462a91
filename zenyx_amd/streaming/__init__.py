"""MI355X drop-in for ``zenyx.streaming`` (zenyx/streaming/__init__.py:1-20), the KV path
and the weight streaming that shares its transfer engine.

Kept names: ``quantize_to_fp8_storage``, ``dequantize_for_bf16_compute``,
``BeladyApproxCache``, ``KVTierManager``, ``KVBlockRef``, ``build_ring_timeline``,
``ParameterStore``, ``LayerWeightStreamer``, ``LayerBlock``, the caller that drives
them, ``StreamingExecutionEngine`` / ``StreamingConfig``, and the throttle rule
``BandwidthAwareScheduler`` / ``BandwidthSample`` (host logic).
"""
from .bandwidth import BandwidthAwareScheduler, BandwidthSample
from .belady import AccessEvent, BeladyApproxCache
from .engine import StreamingConfig, StreamingExecutionEngine
from .kv_tiering import KVBlockRef, KVTierManager, build_ring_timeline
from .parameter_streamer import LayerBlock, LayerWeightStreamer, ParameterStore
from .precision import dequantize_for_bf16_compute, quantize_to_fp8_storage

__all__ = [
    "AccessEvent",
    "BandwidthAwareScheduler",
    "BandwidthSample",
    "BeladyApproxCache",
    "KVBlockRef",
    "KVTierManager",
    "build_ring_timeline",
    "LayerBlock",
    "StreamingConfig",
    "StreamingExecutionEngine",
    "LayerWeightStreamer",
    "ParameterStore",
    "quantize_to_fp8_storage",
    "dequantize_for_bf16_compute",
]
