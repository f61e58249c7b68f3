"""Hot-path kernels, drop-in for the reference's ``infurnace.kernels``.

``store_kv`` and ``paged_attention`` keep the documented names and positional
arguments (reference docs/architecture.md:245-246); every call goes through
the C ABI of libinfurnace_hip.so to hand-written gfx950 HIP kernels.  Array
arguments may be torch tensors or any DLPack / CUDA-array-interface carrier
(``DeviceArray`` describes raw memory), taken without a copy.
"""
from ._carrier import DeviceArray, as_tensor
from ._common import KVStoreError, PagedAttentionError
from .kv_prep import (copy_pages, qk_norm_rope_append, qk_norm_rope_append_and_prefill, qk_norm_rope_store_and_decode,
                      rope_table, zero_pages)
from .kv_store import store_kv, store_kv_layers
from .paged_attention import DecodePlan, decode_plan, paged_attention, store_kv_and_decode, store_kv_and_prefill

__all__ = ["store_kv", "store_kv_layers", "paged_attention", "store_kv_and_decode", "store_kv_and_prefill",
           "decode_plan", "DecodePlan", "qk_norm_rope_append", "qk_norm_rope_store_and_decode",
           "qk_norm_rope_append_and_prefill", "rope_table",
           "zero_pages", "copy_pages",
           "KVStoreError", "PagedAttentionError", "DeviceArray", "as_tensor"]
