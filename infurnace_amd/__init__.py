"""infurnace_amd: MI355X-native (gfx950) KV-cache hot path for Infurnace.

``infurnace_amd.kernels`` -- store_kv / paged_attention (HIP kernels via the C ABI
in include/infurnace_amd.h); ``infurnace_amd.cache`` -- block pool, block tables,
slot mappings and the paged device pool.
"""
__version__ = "0.1.0"
