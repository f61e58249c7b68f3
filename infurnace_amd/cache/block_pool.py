"""Logical page pool: free list, per-owner reference counts, dummy page, block tables, slot mapping.

Drop-in for the reference's planned ``infurnace.cache.block_pool`` (a 0-byte
placeholder), built to the contract of docs/roadmap.md:325-337 (Phase 5A) and
docs/architecture.md:234-240, 255-257:

  * a reserved dummy page gives inactive/padded rows a valid address to read
    (never to write: store_kv skips inactive rows);
  * multi-page allocation is atomic -- it either returns every page or raises
    ``PoolExhausted`` with no state change (admission rollback);
  * active-request, prefix-cache and in-flight ownership are counted
    separately; a page returns to the free list only when all three counts are
    zero ("pages referenced by submitted device work are in flight and cannot
    return to the free pool");
  * stale or foreign ids are rejected before any state changes.

``block_table[request, logical_page] = physical_page`` and
``slot_mapping[token] = physical_page * page_size + page_offset``
(docs/architecture.md:234-235) are built here on the host as int32 arrays.
All state is plain host memory; nothing here touches the GPU.
"""
from __future__ import annotations

from collections import deque
from typing import Iterable, Sequence

import numpy as np

__all__ = ["BlockPool", "BlockPoolError", "PoolExhausted", "OWNERS",
           "build_block_table", "slot_mapping", "slot_mapping_for_positions"]

OWNERS = ("active", "prefix", "inflight")


class BlockPoolError(ValueError):
    """Invalid pool operation (bad id, double free, unknown owner)."""


class PoolExhausted(BlockPoolError):
    """Not enough free pages; the pool is unchanged."""


class BlockPool:
    """Fixed pool of ``num_blocks`` physical pages of ``block_size`` tokens.

    ``order`` optionally fixes the order in which free pages are handed out
    (e.g. a seeded permutation, so tables are non-contiguous); by default ids
    come out ascending.  With ``reserve_dummy`` the first id of that order (page
    0 by default) is the dummy page: never allocated, never freed.
    """

    def __init__(self, num_blocks: int, block_size: int = 16, reserve_dummy: bool = True,
                 order: Sequence[int] | None = None):
        if num_blocks < 1 or block_size < 1:
            raise BlockPoolError("num_blocks and block_size must be positive")
        if reserve_dummy and num_blocks < 2:
            raise BlockPoolError("a pool with a dummy page needs at least 2 blocks")
        ids = list(range(num_blocks)) if order is None else [int(i) for i in order]
        if sorted(ids) != list(range(num_blocks)):
            raise BlockPoolError("order must be a permutation of range(num_blocks)")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.dummy_block: int | None = ids[0] if reserve_dummy else None
        self._free: deque[int] = deque(ids[1:] if reserve_dummy else ids)
        self._counts = {o: np.zeros(num_blocks, np.int64) for o in OWNERS}
        self._is_free = np.zeros(num_blocks, bool)
        self._is_free[list(self._free)] = True

    # ---- queries -------------------------------------------------------------
    @property
    def num_free(self) -> int:
        return len(self._free)

    @property
    def num_used(self) -> int:
        return self.capacity - self.num_free

    @property
    def capacity(self) -> int:
        """Allocatable pages (excludes the dummy page)."""
        return self.num_blocks - (1 if self.dummy_block is not None else 0)

    def refcount(self, block_id: int, owner: str | None = None) -> int:
        """Owners of ``block_id``: one owner kind, or the sum over all kinds."""
        self._check_ids([block_id])
        if owner is None:
            return int(sum(c[block_id] for c in self._counts.values()))
        return int(self._owner(owner)[block_id])

    def is_free(self, block_id: int) -> bool:
        self._check_ids([block_id])
        return bool(self._is_free[block_id])

    # ---- mutation ------------------------------------------------------------
    def allocate(self, n: int, owner: str = "active") -> list[int]:
        """Take ``n`` free pages for ``owner`` (refcount 1 each), all or nothing."""
        counts = self._owner(owner)
        if n < 0:
            raise BlockPoolError(f"cannot allocate {n} blocks")
        if n > len(self._free):
            raise PoolExhausted(f"requested {n} blocks, {len(self._free)} free")
        ids = [self._free.popleft() for _ in range(n)]
        self._is_free[ids] = False
        counts[ids] += 1
        return ids

    def retain(self, ids: Iterable[int], owner: str = "active") -> None:
        """Add one ``owner`` reference to each (allocated) page, e.g. a shared prefix."""
        counts = self._owner(owner)
        arr = self._as_ids(ids)
        if arr.size and self._is_free[arr].any():
            i = int(arr[np.argmax(self._is_free[arr])])
            raise BlockPoolError(f"block {i} is free; cannot retain it")
        np.add.at(counts, arr, 1)

    def free(self, ids: Iterable[int], owner: str = "active") -> list[int]:
        """Drop one ``owner`` reference per id; returns the pages that became free.

        Validated as a whole before anything changes, so a stale id or a double
        free leaves the pool untouched.  A page still held by another owner kind
        (prefix cache, in-flight work) stays allocated.  Pages return to the free
        list in the order of their last occurrence in ``ids``.
        """
        counts = self._owner(owner)
        arr = self._as_ids(ids)
        if arr.size == 0:
            return []
        uniq, need = np.unique(arr, return_counts=True)
        short = counts[uniq] < need
        if short.any():
            j = int(np.argmax(short))
            raise BlockPoolError(f"block {int(uniq[j])} has {int(counts[uniq[j]])} {owner} reference(s), "
                                 f"cannot drop {int(need[j])}")
        np.subtract.at(counts, arr, 1)
        total = sum(c[uniq] for c in self._counts.values())
        newly = uniq[(total == 0) & ~self._is_free[uniq]]
        if newly.size == 0:
            return []
        # last occurrence of each id in ``ids``: the moment its count reached zero
        rev_first = np.unique(arr[::-1], return_index=True)[1]
        last = (arr.size - 1 - rev_first)[np.searchsorted(uniq, newly)]
        released = [int(i) for i in newly[np.argsort(last, kind="stable")]]
        self._is_free[released] = True
        self._free.extend(released)
        return released

    def mark_in_flight(self, ids: Iterable[int]) -> None:
        """Pages read or written by submitted device work (released by ``release_in_flight``)."""
        self.retain(ids, owner="inflight")

    def release_in_flight(self, ids: Iterable[int]) -> list[int]:
        return self.free(ids, owner="inflight")

    def check_invariants(self) -> None:
        """Raise if the free list, flags and counts disagree (used by randomized tests)."""
        total = sum(self._counts.values())
        free_set = set(self._free)
        if len(free_set) != len(self._free):
            raise AssertionError("duplicate id in free list")
        for i in range(self.num_blocks):
            if i == self.dummy_block:
                if i in free_set or total[i] != 0:
                    raise AssertionError("dummy block entered circulation")
                continue
            if (i in free_set) != bool(self._is_free[i]):
                raise AssertionError(f"free flag of block {i} disagrees with the free list")
            if (total[i] == 0) != (i in free_set):
                raise AssertionError(f"block {i}: refcount {int(total[i])} but free={i in free_set}")
        for o, c in self._counts.items():
            if (c < 0).any():
                raise AssertionError(f"negative {o} count")

    # ---- helpers -------------------------------------------------------------
    def _owner(self, owner: str) -> np.ndarray:
        try:
            return self._counts[owner]
        except KeyError:
            raise BlockPoolError(f"unknown owner {owner!r}; expected one of {OWNERS}") from None

    def _check_ids(self, ids: Sequence[int]) -> None:
        self._as_ids(ids)

    def _as_ids(self, ids: Iterable[int]) -> np.ndarray:
        """``ids`` as an int64 array, every entry a valid, non-dummy page id (else BlockPoolError)."""
        if isinstance(ids, np.ndarray):
            arr = ids.reshape(-1)
        else:
            ids = list(ids)
            for i in ids:
                if not isinstance(i, (int, np.integer)) or isinstance(i, bool):
                    raise BlockPoolError(f"block id {i!r} outside [0, {self.num_blocks})")
            arr = np.asarray(ids, np.int64)
        if arr.size and arr.dtype.kind not in "iu":
            raise BlockPoolError(f"block ids must be integers, got dtype {arr.dtype}")
        arr = arr.astype(np.int64, copy=False)
        if arr.size:
            bad = (arr < 0) | (arr >= self.num_blocks)
            if bad.any():
                raise BlockPoolError(f"block id {int(arr[np.argmax(bad)])} outside [0, {self.num_blocks})")
            if self.dummy_block is not None and (arr == self.dummy_block).any():
                raise BlockPoolError("the dummy block cannot be retained or freed")
        return arr

    def build_block_table(self, seqs: Sequence[Sequence[int]], max_pages: int | None = None) -> np.ndarray:
        pad = 0 if self.dummy_block is None else self.dummy_block
        return build_block_table(seqs, max_pages=max_pages, pad=pad)


def build_block_table(seqs: Sequence[Sequence[int]], max_pages: int | None = None, pad: int = 0) -> np.ndarray:
    """int32 [B, max_pages]: row b lists sequence b's physical pages in logical order, padded with ``pad``."""
    width = max((len(s) for s in seqs), default=0) if max_pages is None else int(max_pages)
    width = max(width, 1)
    table = np.full((len(seqs), width), pad, np.int32)
    for b, s in enumerate(seqs):
        if len(s) > width:
            raise BlockPoolError(f"sequence {b} has {len(s)} pages > max_pages {width}")
        table[b, :len(s)] = np.asarray(s, np.int32)
    return table


def slot_mapping(block_table: np.ndarray, seq_idx: Sequence[int], positions: Sequence[int],
                 block_size: int = 16) -> np.ndarray:
    """int32 [T]: ``table[seq][pos // bs] * bs + pos % bs`` (docs/architecture.md:235)."""
    bt = np.asarray(block_table)
    si = np.asarray(seq_idx, np.int64)
    pos = np.asarray(positions, np.int64)
    if si.shape != pos.shape:
        raise BlockPoolError("seq_idx and positions must have the same shape")
    if pos.size and (pos.min() < 0 or (pos // block_size).max() >= bt.shape[1]):
        raise BlockPoolError("position beyond the block table")
    if si.size and (si.min() < 0 or si.max() >= bt.shape[0]):
        raise BlockPoolError("sequence index outside the block table")
    slots = bt[si, pos // block_size].astype(np.int64) * block_size + pos % block_size
    return slots.astype(np.int32)


def slot_mapping_for_positions(block_table_row: Sequence[int], start: int, count: int,
                               block_size: int = 16) -> np.ndarray:
    """Slots of ``count`` consecutive positions from ``start`` of one sequence (a prefill chunk)."""
    row = np.asarray(block_table_row, np.int32)[None]
    pos = np.arange(start, start + count, dtype=np.int64)
    return slot_mapping(row, np.zeros(count, np.int64), pos, block_size)
