"""KV side of a runner on the paged cache: slots, pages, plans, and per-layer store + attend.

The reference's ``Runner`` (src/infurnace/executor/runner.py:5-45) owns model
execution through ``prefill(input_ids, slot, start_position)``,
``decode(input_ids, position, slot)`` and ``clear_slot(slot)``, and today keeps
one contiguous cache row per slot (src/infurnace/executor/tinygrad/buffers.py).
``PagedKVRunner`` is the part of such a runner that touches KV bytes, built on
this package's pool, tables and kernels:

* a slot is a sequence in a ``KVManager``; pages are allocated per prefill chunk
  and per decode step (one new page every ``block_size`` tokens), all-or-nothing;
* ``fill_block_tables(plan)`` produces ``DecodePlan.block_tables`` for the
  scheduler (src/infurnace/scheduler/plan.py:30-31; the scheduler leaves it
  empty at src/infurnace/scheduler/scheduler.py:160-172);
* a prefill chunk or a decode step returns a step object whose
  ``store_attend(layer, q, k, v)`` appends that layer's K/V and runs paged
  attention -- the per-layer replacement of model.py:116-138 (prefill) and
  :191-200 (decode); ``prep_store_attend`` does the same from fp32 projections
  through the fused norm + rotary + append kernel (model.py:183-196);
* ``clear_slot(slot)`` releases the slot's pages (zeroing them on request:
  buffers.py:67-81), which is what the engine calls on every terminal transition
  (src/infurnace/engine/engine.py:89,130,166);
* a decode batch whose live rows start with the same pages (prefix-cache hits)
  reads those pages once for the batch (``paged_attention(...,
  shared_prefix_pages=...)``) when they are at least ``shared_prefix_min_pages``;
  a batch whose rows share pages otherwise keeps its page loads cached (an empty
  ``shared_prefix_pages``), since the default decode streams every page once.

The model itself (projections, MLP, logits) stays with the caller.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Sequence

import numpy as np
import torch

from .cache import BlockPool, KVCacheError, KVManager, PagedKVCache, PrefixCache
from .kernels import paged_attention, qk_norm_rope_append, store_kv, store_kv_and_decode, store_kv_and_prefill

__all__ = ["PagedKVRunner", "RunnerError"]


class RunnerError(ValueError):
    """A prefill or decode request that does not fit the runner's state (as RunnerError in
    src/infurnace/executor/runner.py's implementations)."""


@dataclass
class _Step:
    runner: "PagedKVRunner"
    slot_mapping: torch.Tensor        # int32 [T]
    block_tables: torch.Tensor        # int32 [B, max_pages] (prefill: [max_pages])
    seq_lens: torch.Tensor | None     # int32 [B] (decode only)
    active: torch.Tensor | None       # uint8 [T] (decode only)
    positions: torch.Tensor           # int32 [T]
    query_start: int | None           # prefill only
    max_len: int
    # int32 pages every live decode row starts with; empty: rows share pages elsewhere (cached page loads)
    shared_prefix: torch.Tensor | None = None

    def store_attend(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     out: torch.Tensor | None = None) -> torch.Tensor:
        """Append this step's k, v (fp16 [T, Hkv, D]) for ``layer``, then attend with q (fp16 [T, Hq, D]).

        A prefill chunk, and a decode step without a shared prefix, do both in one launch
        (``store_kv_and_prefill`` / ``store_kv_and_decode``).
        """
        kv = self.runner.cache.kv
        if self.query_start is not None:
            return store_kv_and_prefill(q, kv, self.block_tables, k, v, query_start=self.query_start, layer=layer,
                                        out=out)
        if self.shared_prefix is None:
            return store_kv_and_decode(q, kv, self.block_tables, self.seq_lens, self.active, self.slot_mapping, k, v,
                                       layer=layer, max_seq_len=self.max_len, out=out)
        store_kv(kv, self.slot_mapping, self.active, k, v, layer=layer)
        if self.query_start is not None:
            return paged_attention(q, kv, self.block_tables, None, None, layer=layer, query_start=self.query_start,
                                   out=out)
        return paged_attention(q, kv, self.block_tables, self.seq_lens, self.active, layer=layer,
                               max_seq_len=self.max_len, out=out, shared_prefix_pages=self.shared_prefix)

    def prep_store_attend(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor, rope: torch.Tensor,
                          eps: float = 1e-6, out: torch.Tensor | None = None) -> torch.Tensor:
        """The same from fp32 projections: q/k RMSNorm + rotary, fp16 cast and append in one launch."""
        kv = self.runner.cache.kv
        q16 = qk_norm_rope_append(q, k, v, q_norm_weight, k_norm_weight, rope, self.positions, self.slot_mapping,
                                  self.active, kv, layer=layer, eps=eps)
        if self.query_start is not None:
            return paged_attention(q16, kv, self.block_tables, None, None, layer=layer,
                                   query_start=self.query_start, out=out)
        return paged_attention(q16, kv, self.block_tables, self.seq_lens, self.active, layer=layer,
                               max_seq_len=self.max_len, out=out, shared_prefix_pages=self.shared_prefix)


class PagedKVRunner:
    """Paged KV state for ``num_slots`` concurrent sequences of up to ``max_context`` tokens."""

    def __init__(self, num_layers: int, num_slots: int, max_context: int, num_kv_heads: int, head_dim: int,
                 num_blocks: int, device: str | torch.device = "cuda", block_size: int = 16,
                 prefix_namespace=None, prefix_capacity_blocks: int | None = None,
                 shared_prefix_min_pages: int = 64):
        if num_slots < 1 or max_context < 1:
            raise RunnerError("num_slots and max_context must be positive")
        self._num_slots, self._max_context = num_slots, max_context
        self.block_size = block_size
        self.max_pages = math.ceil(max_context / block_size)
        self.device = torch.device(device)
        self.cache = PagedKVCache(num_layers, num_blocks, num_kv_heads, head_dim, block_size, self.device)
        self.pool = BlockPool(num_blocks, block_size)
        self.mgr = KVManager(self.pool, max_pages_per_seq=self.max_pages)
        # prefix cache (docs/roadmap.md:442-470) when a namespace -- checkpoint and KV-affecting
        # settings -- is given; PrefillPlan.prefix_token_ids / prefix_cache_hit (plan.py:14-15)
        self.prefix = (PrefixCache(self.pool, prefix_namespace, prefix_capacity_blocks)
                       if prefix_namespace is not None else None)
        # below this many common leading pages, decode re-reads them per row (from cache) instead
        # of paying the shared-prefix path's two extra launches
        self.shared_prefix_min_pages = max(1, int(shared_prefix_min_pages))

    # Runner contract (runner.py:11-21)
    @property
    def num_slots(self) -> int:
        return self._num_slots

    @property
    def max_context(self) -> int:
        return self._max_context

    def _check_slot(self, slot: int) -> None:
        if not 0 <= slot < self._num_slots:
            raise RunnerError(f"slot {slot} out of range [0, {self._num_slots})")

    def length(self, slot: int) -> int:
        """Tokens whose K/V the slot holds."""
        return self.mgr.length(slot) if slot in self.mgr else 0

    def _table(self, slots: Sequence[int]) -> np.ndarray:
        pad = self.pool.dummy_block if self.pool.dummy_block is not None else 0
        t = np.full((len(slots), self.max_pages), pad, np.int32)
        for i, s in enumerate(slots):
            if s in self.mgr:
                b = self.mgr.blocks(s)
                t[i, :len(b)] = b
        return t

    def _dev(self, a: np.ndarray) -> torch.Tensor:
        return torch.from_numpy(np.ascontiguousarray(a)).to(self.device)

    # -- prefill ----------------------------------------------------------------------------

    def begin_prefill(self, slot: int, start_position: int, num_tokens: int) -> _Step:
        """Reserve pages for tokens [start_position, start_position + num_tokens) of ``slot``.

        Chunks arrive in order (the scheduler's chunk bounds cover the prompt without
        gaps, plan.py:9-13): ``start_position`` must equal the tokens already stored.
        """
        self._check_slot(slot)
        if num_tokens < 1:
            raise RunnerError("a prefill chunk needs at least one token")
        if start_position != self.length(slot):
            raise RunnerError(f"slot {slot} holds {self.length(slot)} tokens; chunk starts at {start_position}")
        if start_position + num_tokens > self._max_context:
            raise RunnerError(f"chunk ends at {start_position + num_tokens} > max_context {self._max_context}")
        if slot not in self.mgr:
            self.mgr.add_sequence(slot)
        try:
            slots = self.mgr.append(slot, num_tokens)
        except KVCacheError as e:
            raise RunnerError(str(e)) from e
        pos = np.arange(start_position, start_position + num_tokens, dtype=np.int32)
        return _Step(self, self._dev(slots.astype(np.int32)), self._dev(self._table([slot])[0]), None, None,
                     self._dev(pos), start_position, start_position + num_tokens)

    def attach_prefix(self, slot: int, token_ids: Sequence[int]) -> int:
        """Start an empty slot from the longest cached prefix of ``token_ids`` (complete blocks).

        Returns the number of tokens whose K/V the slot now shares; prefill resumes there
        (``begin_prefill(slot, n, ...)``).  At least one token is always left to prefill, so
        the last prompt token's logits are produced.
        """
        self._check_slot(slot)
        if self.prefix is None:
            raise RunnerError("this runner has no prefix cache (prefix_namespace was not given)")
        if slot in self.mgr:
            raise RunnerError(f"slot {slot} is not empty")
        pages, n = self.prefix.lookup(list(token_ids)[:max(0, len(token_ids) - 1)])
        self.mgr.add_sequence(slot, prefix_blocks=pages, prefix_len=n)
        return n

    def publish_prefix(self, slot: int, token_ids: Sequence[int]) -> int:
        """Publish the complete blocks of the slot's first ``len(token_ids)`` tokens."""
        self._check_slot(slot)
        if self.prefix is None:
            raise RunnerError("this runner has no prefix cache (prefix_namespace was not given)")
        if len(token_ids) > self.length(slot):
            raise RunnerError(f"slot {slot} holds {self.length(slot)} tokens, not {len(token_ids)}")
        return self.prefix.insert(list(token_ids), self.mgr.blocks(slot))

    # -- decode -----------------------------------------------------------------------------

    def fill_block_tables(self, plan) -> tuple[tuple[int, ...], ...]:
        """``DecodePlan.block_tables`` for ``plan`` (pages of each row's slot, padded)."""
        return tuple(tuple(int(x) for x in row) for row in self._table(list(plan.slots)))

    def begin_decode(self, plan) -> _Step:
        """Append one token per active row of a ``DecodePlan`` (plan.py:16-28) at ``positions[i]``.

        Inactive rows (padding) store nothing and produce no output.  Pages for all
        active rows are allocated together or not at all.
        """
        slots, positions, active = list(plan.slots), list(plan.positions), list(plan.active_mask)
        if not (len(slots) == len(positions) == len(active)):
            raise RunnerError("plan slots, positions and active_mask differ in length")
        live = [i for i, a in enumerate(active) if a]
        for i in live:
            self._check_slot(slots[i])
            if slots[i] not in self.mgr or positions[i] != self.length(slots[i]):
                raise RunnerError(f"row {i}: slot {slots[i]} holds {self.length(slots[i])} tokens, "
                                  f"decode writes position {positions[i]}")
            if positions[i] + 1 > self._max_context:
                raise RunnerError(f"row {i}: position {positions[i]} is past max_context")
        if len({slots[i] for i in live}) != len(live):
            raise RunnerError("two active rows share a slot")
        try:
            new_slots = self.mgr.append_batch([slots[i] for i in live], [1] * len(live))
        except KVCacheError as e:
            raise RunnerError(str(e)) from e
        sm = np.full(len(slots), -1, np.int32)
        for j, i in enumerate(live):
            sm[i] = int(new_slots[j][0])
        lens = np.zeros(len(slots), np.int32)
        for i in live:
            lens[i] = positions[i] + 1
        act = np.asarray(active, np.uint8)
        table = self._table(slots)
        shared = self._common_pages(table[live], lens[live])
        if len(shared) >= self.shared_prefix_min_pages:
            prefix = self._dev(shared)
        elif self._any_shared(table[live], lens[live]):
            prefix = self._dev(np.zeros(0, np.int32))
        else:
            prefix = None
        return _Step(self, self._dev(sm), self._dev(table), self._dev(lens), self._dev(act),
                     self._dev(np.asarray(positions, np.int32)), None, int(lens.max()) if len(lens) else 0, prefix)

    def _common_pages(self, table: np.ndarray, lens: np.ndarray) -> np.ndarray:
        """Leading page ids that every row of ``table`` holds at the same columns (at least two
        rows), limited to pages complete in every row (``lens`` keys)."""
        if table.shape[0] < 2:
            return np.zeros(0, np.int32)
        limit = int(lens.min()) // self.block_size
        same = (table[:, :limit] == table[0, :limit]).all(axis=0)
        n = int(np.argmin(same)) if not same.all() else limit
        return np.ascontiguousarray(table[0, :n], dtype=np.int32)

    def _any_shared(self, table: np.ndarray, lens: np.ndarray) -> bool:
        """Whether a page id occurs in more than one of the rows' used table entries (``lens`` keys)."""
        if table.shape[0] < 2:
            return False
        used = -(-lens.astype(np.int64) // self.block_size)
        pages = np.concatenate([table[i, :used[i]] for i in range(table.shape[0])])
        return len(np.unique(pages)) != len(pages)

    # -- lifecycle --------------------------------------------------------------------------

    def clear_slot(self, slot: int, zero: bool = False) -> list[int]:
        """Release the slot's pages (runner.py:38-43); ``zero`` also zeroes the freed pages."""
        self._check_slot(slot)
        if slot not in self.mgr:
            return []
        freed = self.mgr.free_sequence(slot)
        if zero and freed:
            self.cache.clear_pages(freed)
        return freed
