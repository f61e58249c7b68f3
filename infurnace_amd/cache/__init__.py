"""Host-side page pool and KV bookkeeping, drop-in for the reference's ``infurnace.cache``.

The reference's cache/ modules are 0-byte placeholders; the contract is
docs/roadmap.md:325-337 and docs/architecture.md:225-240, 255-257.
"""
from .block_pool import (OWNERS, BlockPool, BlockPoolError, PoolExhausted, build_block_table, slot_mapping,
                         slot_mapping_for_positions)
from .kv_manager import KVCacheError, KVManager, PagedKVCache
from .prefix_cache import PrefixCache, PrefixCacheError

__all__ = ["BlockPool", "BlockPoolError", "PoolExhausted", "OWNERS", "build_block_table", "slot_mapping",
           "slot_mapping_for_positions", "KVManager", "PagedKVCache", "KVCacheError", "PrefixCache",
           "PrefixCacheError"]
