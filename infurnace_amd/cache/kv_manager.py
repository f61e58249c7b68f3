"""Paged KV storage and per-sequence page bookkeeping.

Drop-in for the reference's planned ``infurnace.cache.kv_manager`` (a 0-byte
placeholder).  ``PagedKVCache`` is the persistent device pool
``kv_pool[layer, K_or_V, physical_page, page_offset, kv_head, head_dim]``
(docs/architecture.md:225-232), zero-initialised like the contiguous
ContiguousKVCache it replaces (src/infurnace/executor/tinygrad/buffers.py:24-45).
``KVManager`` owns the logical side: which pages each sequence holds, its
length, atomic growth for appended tokens, release on completion/cancel, and
the int32 block tables and slot mappings handed to the kernels
(docs/architecture.md:234-240).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Hashable, Sequence

import numpy as np
import torch

from .block_pool import BlockPool, BlockPoolError, PoolExhausted, build_block_table

__all__ = ["PagedKVCache", "KVManager", "KVCacheError"]


class KVCacheError(ValueError):
    """KV cache configuration or bookkeeping violates the contract (reference buffers.py:6)."""


class PagedKVCache:
    """Persistent fp16 pool [layers, 2, num_blocks, block_size, num_kv_heads, head_dim] on one GPU."""

    def __init__(self, num_layers: int, num_blocks: int, num_kv_heads: int, head_dim: int,
                 block_size: int = 16, device: str | torch.device = "cuda", zero: bool = True):
        for name, v in (("num_layers", num_layers), ("num_blocks", num_blocks), ("num_kv_heads", num_kv_heads),
                        ("head_dim", head_dim), ("block_size", block_size)):
            if v < 1:
                raise KVCacheError(f"{name} must be positive, got {v}")
        if head_dim % 8 != 0:
            raise KVCacheError(f"head_dim must be a multiple of 8 (16-byte rows), got {head_dim}")
        shape = (num_layers, 2, num_blocks, block_size, num_kv_heads, head_dim)
        alloc = torch.zeros if zero else torch.empty
        self.kv = alloc(shape, dtype=torch.float16, device=device)
        self.num_layers, self.num_blocks, self.block_size = num_layers, num_blocks, block_size
        self.num_kv_heads, self.head_dim = num_kv_heads, head_dim

    @property
    def shape(self) -> tuple[int, ...]:
        return tuple(self.kv.shape)

    @property
    def size_bytes(self) -> int:
        return self.kv.numel() * self.kv.element_size()

    @property
    def page_bytes(self) -> int:
        """Bytes of one page (K+V, all kv heads) in one layer."""
        return 2 * self.block_size * self.num_kv_heads * self.head_dim * self.kv.element_size()

    def layer(self, i: int) -> torch.Tensor:
        return self.kv[i]

    def clear_pages(self, ids: Sequence[int]) -> None:
        """Zero the given pages in every layer (slot reuse without stale state, buffers.py:67-81)."""
        if len(ids) == 0:
            return
        arr = np.asarray(ids, np.int64)
        if int(arr.min()) < 0 or int(arr.max()) >= self.num_blocks:
            raise KVCacheError("page id outside the pool")
        from ..kernels import zero_pages  # the HIP page kernel (ifn_zero_pages)
        zero_pages(self.kv, torch.as_tensor(arr.astype(np.int32), device=self.kv.device))

    def copy_pages(self, src: Sequence[int], dst: Sequence[int]) -> None:
        """Copy page src[i] to dst[i] in every layer (a private copy of a shared partial block)."""
        if len(src) != len(dst):
            raise KVCacheError("copy_pages needs as many destinations as sources")
        if len(src) == 0:
            return
        s, d = np.asarray(src, np.int64), np.asarray(dst, np.int64)
        if min(s.min(), d.min()) < 0 or max(s.max(), d.max()) >= self.num_blocks:
            raise KVCacheError("page id outside the pool")
        from ..kernels import copy_pages
        copy_pages(self.kv, torch.as_tensor(s.astype(np.int32), device=self.kv.device),
                   torch.as_tensor(d.astype(np.int32), device=self.kv.device))


@dataclass
class _Seq:
    blocks: list[int] = field(default_factory=list)
    length: int = 0
    shared: int = 0  # leading blocks borrowed from a shared prefix (not owned by "active" alloc)


class KVManager:
    """Sequence -> pages bookkeeping over a ``BlockPool``."""

    def __init__(self, pool: BlockPool, max_pages_per_seq: int | None = None):
        self.pool = pool
        self.block_size = pool.block_size
        self.max_pages_per_seq = max_pages_per_seq
        self._seqs: dict[Hashable, _Seq] = {}

    # ---- lifecycle -----------------------------------------------------------
    def add_sequence(self, seq_id: Hashable, prefix_blocks: Sequence[int] = (), prefix_len: int = 0) -> None:
        """Register a sequence, optionally starting from shared prefix pages.

        The prefix pages get one more "active" reference each (shared, refcounted
        ids appear in several block tables); ``prefix_len`` tokens of them count
        as already stored.  Only whole pages may be shared.
        """
        if seq_id in self._seqs:
            raise KVCacheError(f"sequence {seq_id!r} already exists")
        prefix_blocks = [int(b) for b in prefix_blocks]
        if prefix_len != len(prefix_blocks) * self.block_size:
            raise KVCacheError("a shared prefix must cover whole pages (prefix_len = pages * block_size)")
        self.pool.retain(prefix_blocks, owner="active")
        self._seqs[seq_id] = _Seq(blocks=list(prefix_blocks), length=prefix_len, shared=len(prefix_blocks))

    def free_sequence(self, seq_id: Hashable) -> list[int]:
        """Drop the sequence's references; returns pages that became free."""
        self._get(seq_id)
        s = self._seqs.pop(seq_id)
        return self.pool.free(s.blocks, owner="active")

    def __contains__(self, seq_id: Hashable) -> bool:
        return seq_id in self._seqs

    def length(self, seq_id: Hashable) -> int:
        return self._get(seq_id).length

    def blocks(self, seq_id: Hashable) -> list[int]:
        return list(self._get(seq_id).blocks)

    # ---- growth ----------------------------------------------------------------
    def append(self, seq_id: Hashable, n: int) -> np.ndarray:
        """Reserve ``n`` more positions of one sequence; returns their int32 slots."""
        return self.append_batch([seq_id], [n])[0]

    def append_batch(self, seq_ids: Sequence[Hashable], counts: Sequence[int]) -> list[np.ndarray]:
        """Reserve positions for several sequences at once, atomically.

        Either every sequence grows (new pages taken from the pool) or
        ``PoolExhausted`` is raised and nothing changes.
        """
        if len(seq_ids) != len(counts) or len(set(seq_ids)) != len(seq_ids):
            raise KVCacheError("seq_ids must be distinct and match counts")
        plans = []
        total_new = 0
        for sid, n in zip(seq_ids, counts):
            s = self._get(sid)
            if n < 0:
                raise KVCacheError("cannot append a negative number of tokens")
            need_pages = -(-(s.length + n) // self.block_size)
            if self.max_pages_per_seq is not None and need_pages > self.max_pages_per_seq:
                raise KVCacheError(f"sequence {sid!r} would need {need_pages} pages > {self.max_pages_per_seq}")
            new = max(0, need_pages - len(s.blocks))
            plans.append((s, n, new))
            total_new += new
        if total_new > self.pool.num_free:
            raise PoolExhausted(f"need {total_new} pages, {self.pool.num_free} free")
        out = []
        for s, n, new in plans:
            s.blocks.extend(self.pool.allocate(new, owner="active"))
            pos = np.arange(s.length, s.length + n, dtype=np.int64)
            row = np.asarray(s.blocks, np.int64)
            out.append((row[pos // self.block_size] * self.block_size + pos % self.block_size).astype(np.int32))
            s.length += n
        return out

    def replace_blocks(self, seq_id: Hashable, block_indices: Sequence[int]) -> list[int]:
        """Release some of a sequence's private pages and replace them with fresh ones (page churn).

        Used to model pool churn (free and reallocate suffix pages): the sequence
        keeps its length; the replaced pages' contents must be rewritten by the
        caller.  Atomic: on exhaustion nothing changes.
        """
        s = self._get(seq_id)
        idx = [int(i) for i in block_indices]
        if any(i < s.shared or i >= len(s.blocks) for i in idx) or len(set(idx)) != len(idx):
            raise KVCacheError("block indices must be distinct private pages of the sequence")
        if len(idx) > self.pool.num_free:
            # fresh pages are taken before the old ones are released
            raise PoolExhausted(f"need {len(idx)} pages, {self.pool.num_free} free")
        fresh = self.pool.allocate(len(idx), owner="active")
        old = [s.blocks[i] for i in idx]
        for i, b in zip(idx, fresh):
            s.blocks[i] = b
        self.pool.free(old, owner="active")
        return fresh

    # ---- tables ------------------------------------------------------------------
    def block_tables(self, seq_ids: Sequence[Hashable], max_pages: int | None = None) -> np.ndarray:
        pad = 0 if self.pool.dummy_block is None else self.pool.dummy_block
        return build_block_table([self._get(s).blocks for s in seq_ids], max_pages=max_pages, pad=pad)

    def seq_lens(self, seq_ids: Sequence[Hashable]) -> np.ndarray:
        return np.asarray([self._get(s).length for s in seq_ids], np.int32)

    def _get(self, seq_id: Hashable) -> _Seq:
        try:
            return self._seqs[seq_id]
        except KeyError:
            raise KVCacheError(f"unknown sequence {seq_id!r}") from None


# re-exported for callers that catch pool errors through this module
__all__ += ["BlockPoolError", "PoolExhausted"]
