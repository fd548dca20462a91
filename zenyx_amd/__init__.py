"""zenyx_amd -- MI355X-native (gfx950) KV-cache hot path of zenyx.

``zenyx_amd.streaming`` keeps the call signatures of ``zenyx.streaming`` (precision,
Belady cache, KV tiers, ring timeline); ``zenyx_amd.train`` holds the README-documented
``BeladyKVCacheTieringManager`` and ``FP8KVQuantizer``.  All compute runs in
libzenyx_kv.so (hand-written HIP kernels behind a C ABI, include/zenyx_kv.h); there is
no CPU fallback.
"""
__version__ = "0.1.0"

from . import kv  # noqa: F401
