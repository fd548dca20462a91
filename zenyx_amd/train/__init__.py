"""README-documented Phase-7/8/9 modules of zenyx, MI355X-native:
``belayd_kv_cache_tiering`` (Belady KV tiering over a ring schedule), ``belady_tiers``
(the three-tier HBM / DRAM / NVMe hierarchy with Belady at both levels),
``dynamic_ring_curriculum`` (ring degree per training step and the page traces it
implies) and ``fp8_kv_quantization`` (per-head FP8 KV quantisation, a paged FP8 KV
cache and ring attention reading it)."""
