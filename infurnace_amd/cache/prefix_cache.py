"""Prefix cache over the page pool: identity, sharing and eviction of complete KV blocks.

Implements the reference's Phase 8 contract (docs/roadmap.md:442-470;
docs/architecture.md:381-391), whose module is not written yet:

* Only complete, immutable token blocks are published; a partial tail block is
  never shared (no copy-on-write ambiguity at the active tail).
* Identity covers the namespace -- the checkpoint and every execution setting
  that changes KV values (dtype, RoPE base and scaling, adapters) -- and the
  whole token history: a block is found by a digest of (namespace, parent
  block, token ids of the block), and a digest match is verified against the
  stored token ids and the parent entry, so a collision can never select
  unrelated tokens.
* A published block holds one "prefix" reference on its page
  (``BlockPool`` owner kinds).  Dropping it never frees a page that still has
  active or in-flight owners; eviction only reclaims entries whose page has no
  other owner, least recently used first, leaves before their parents.
* Changing the namespace (model reload) invalidates every entry.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass
from typing import Callable, Hashable, Sequence

from .block_pool import BlockPool, BlockPoolError

__all__ = ["PrefixCache", "PrefixCacheError"]


class PrefixCacheError(ValueError):
    """Bad prefix-cache request (wrong page count, foreign page, ...)."""


def _blake2b(data: bytes) -> bytes:
    return hashlib.blake2b(data, digest_size=16).digest()


@dataclass
class _Entry:
    uid: int
    parent: int | None  # uid of the previous block of the chain
    tokens: tuple[int, ...]
    page: int
    children: int = 0
    last_use: int = 0
    order: int = 0


@dataclass
class _Stats:
    lookups: int = 0
    hit_blocks: int = 0
    published: int = 0
    evicted: int = 0
    collisions: int = 0  # digest matches whose tokens or parent differed


class PrefixCache:
    """Map from token-block chains to pages of a ``BlockPool``.

    ``namespace`` is any value whose ``repr`` identifies the checkpoint and the
    KV-affecting settings.  ``hasher`` (bytes -> bytes) exists so tests can force
    collisions; the default is a 128-bit BLAKE2b.
    """

    def __init__(self, pool: BlockPool, namespace: Hashable, capacity_blocks: int | None = None,
                 hasher: Callable[[bytes], bytes] | None = None):
        if capacity_blocks is not None and capacity_blocks < 0:
            raise PrefixCacheError("capacity_blocks must be non-negative")
        self.pool = pool
        self.block_size = pool.block_size
        self.capacity_blocks = capacity_blocks
        self._hash = hasher or _blake2b
        self._ns = repr(namespace).encode()
        self.namespace = namespace
        self._buckets: dict[bytes, list[_Entry]] = {}
        self._entries: dict[int, _Entry] = {}
        self._clock = 0
        self._order = 0
        self.stats = _Stats()

    # -- identity ---------------------------------------------------------------------------

    def _digest(self, parent: int | None, tokens: tuple[int, ...]) -> bytes:
        body = b"".join(int(t).to_bytes(8, "little", signed=True) for t in tokens)
        head = b"<root>" if parent is None else parent.to_bytes(8, "little")
        return self._hash(self._ns + b"|" + head + b"|" + body)

    def _find(self, parent: int | None, tokens: tuple[int, ...]) -> _Entry | None:
        bucket = self._buckets.get(self._digest(parent, tokens), ())
        for e in bucket:
            if e.parent == parent and e.tokens == tokens:  # verify: a digest match alone is not identity
                return e
        if bucket:
            self.stats.collisions += 1
        return None

    def _blocks(self, token_ids: Sequence[int]) -> list[tuple[int, ...]]:
        bs = self.block_size
        toks = [int(t) for t in token_ids]
        return [tuple(toks[i * bs:(i + 1) * bs]) for i in range(len(toks) // bs)]

    # -- queries ----------------------------------------------------------------------------

    def __len__(self) -> int:
        return len(self._entries)

    def lookup(self, token_ids: Sequence[int]) -> tuple[list[int], int]:
        """Longest cached chain of complete blocks that prefixes ``token_ids``.

        Returns ``(pages, num_tokens)``.  No reference is taken: pass the pages to
        ``KVManager.add_sequence(..., prefix_blocks=pages, prefix_len=num_tokens)``,
        which retains them for the new sequence.
        """
        self.stats.lookups += 1
        self._clock += 1
        pages: list[int] = []
        parent = None
        for blk in self._blocks(token_ids):
            e = self._find(parent, blk)
            if e is None:
                break
            e.last_use = self._clock
            pages.append(e.page)
            parent = e.uid
        self.stats.hit_blocks += len(pages)
        return pages, len(pages) * self.block_size

    # -- publication and eviction -----------------------------------------------------------

    def insert(self, token_ids: Sequence[int], pages: Sequence[int]) -> int:
        """Publish the complete blocks of a sequence whose block i is stored in ``pages[i]``.

        The trailing partial block is never published.  Blocks already cached are left
        as they are (the chain continues through the cached entry).  Each new entry
        takes a "prefix" reference on its page.  When the cache is at capacity the
        least recently used evictable leaf makes room; if none can, publication stops.
        Returns the number of newly published blocks.
        """
        blocks = self._blocks(token_ids)
        if len(pages) < len(blocks):
            raise PrefixCacheError(f"{len(blocks)} complete blocks need as many pages, got {len(pages)}")
        for p in pages[:len(blocks)]:
            if not 0 <= int(p) < self.pool.num_blocks or self.pool.is_free(int(p)):
                raise PrefixCacheError(f"page {p} is not an allocated page of the pool")
        self._clock += 1
        parent = None
        new = 0
        parent_entry: _Entry | None = None
        for blk, page in zip(blocks, pages):
            e = self._find(parent, blk)
            if e is None:
                if self.capacity_blocks is not None and len(self._entries) >= self.capacity_blocks:
                    protect = {parent_entry.uid} if parent_entry is not None else set()
                    if self._evict_one(protect) is None:
                        break
                e = self._publish(parent, blk, int(page))
                if parent_entry is not None:
                    parent_entry.children += 1
                new += 1
            e.last_use = self._clock
            parent, parent_entry = e.uid, e
        return new

    def _publish(self, parent: int | None, tokens: tuple[int, ...], page: int) -> _Entry:
        self.pool.retain([page], owner="prefix")
        self._order += 1
        e = _Entry(self._order, parent, tokens, page, order=self._order)
        self._buckets.setdefault(self._digest(parent, tokens), []).append(e)
        self._entries[e.uid] = e
        self.stats.published += 1
        return e

    def _evictable(self, e: _Entry) -> bool:
        # a leaf whose page no active sequence or in-flight work still references
        return e.children == 0 and self.pool.refcount(e.page) == self.pool.refcount(e.page, "prefix")

    def _drop(self, e: _Entry) -> list[int]:
        d = self._digest(e.parent, e.tokens)
        self._buckets[d].remove(e)
        if not self._buckets[d]:
            del self._buckets[d]
        del self._entries[e.uid]
        if e.parent is not None:
            self._entries[e.parent].children -= 1
        self.stats.evicted += 1
        return self.pool.free([e.page], owner="prefix")

    def _evict_one(self, protect: set[int] = frozenset()) -> list[int] | None:
        cands = [e for e in self._entries.values() if e.uid not in protect and self._evictable(e)]
        if not cands:
            return None
        victim = min(cands, key=lambda e: (e.last_use, e.order))
        return self._drop(victim)

    def evict(self, n_blocks: int) -> list[int]:
        """Evict up to ``n_blocks`` entries (LRU leaves with no other owners); returns freed pages."""
        freed: list[int] = []
        for _ in range(max(0, n_blocks)):
            got = self._evict_one()
            if got is None:
                break
            freed.extend(got)
        return freed

    def invalidate(self, namespace: Hashable | None = None) -> list[int]:
        """Drop every entry (model reload or settings change); optionally switch namespace.

        Only the cache's own references are released: pages still used by active
        sequences or in-flight work stay allocated.  Returns the pages that became free.
        """
        freed: list[int] = []
        for e in list(self._entries.values()):
            try:
                freed.extend(self.pool.free([e.page], owner="prefix"))
            except BlockPoolError as err:  # the pool lost track of a reference: a caller bug
                raise PrefixCacheError(str(err)) from err
        self._buckets.clear()
        self._entries.clear()
        if namespace is not None:
            self.namespace = namespace
            self._ns = repr(namespace).encode()
        return freed

    def check_invariants(self) -> None:
        """Every entry holds one prefix reference; child counts match; digests match content."""
        per_page: dict[int, int] = {}
        children: dict[int, int] = {}
        for uid, e in self._entries.items():
            assert e.uid == uid and len(e.tokens) == self.block_size
            assert e in self._buckets[self._digest(e.parent, e.tokens)]
            assert e.parent is None or e.parent in self._entries
            per_page[e.page] = per_page.get(e.page, 0) + 1
            if e.parent is not None:
                children[e.parent] = children.get(e.parent, 0) + 1
        for page, n in per_page.items():
            assert self.pool.refcount(page, "prefix") >= n
        for e in self._entries.values():
            assert e.children == children.get(e.uid, 0)
