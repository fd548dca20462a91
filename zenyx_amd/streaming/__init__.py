"""MI355X drop-in for the KV-cache part of ``zenyx.streaming`` (zenyx/streaming/__init__.py:1-20).

Kept names: ``quantize_to_fp8_storage``, ``dequantize_for_bf16_compute``,
``BeladyApproxCache``, ``KVTierManager``, ``KVBlockRef``, ``build_ring_timeline``.
The reference's weight streaming (``LayerWeightStreamer``, ``ParameterStore``), bandwidth
throttle and training engine are not part of the KV hot path and are not provided.
"""
from .belady import AccessEvent, BeladyApproxCache
from .kv_tiering import KVBlockRef, KVTierManager, build_ring_timeline
from .precision import dequantize_for_bf16_compute, quantize_to_fp8_storage

__all__ = [
    "AccessEvent",
    "BeladyApproxCache",
    "KVBlockRef",
    "KVTierManager",
    "build_ring_timeline",
    "quantize_to_fp8_storage",
    "dequantize_for_bf16_compute",
]
