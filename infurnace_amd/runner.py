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
* pages referenced by submitted device work are in flight and do not return to
  the free pool until that work has completed (docs/architecture.md:255-257;
  the "delayed in-flight reclamation" of docs/roadmap.md:331-337,356-359): a
  step marks the pages it reads or writes in flight when it begins, records an
  event after each of its launches, and its pages are released once it is closed
  (a later step began or a slot was cleared) and its last event has completed -- checked
  without blocking at every ``begin_*``, ``clear_slot`` and ``reclaim()``, or
  waited for by ``synchronize()``.  A page freed by ``clear_slot`` while in
  flight is reused only after that; with ``zero=True`` it is zeroed when it is
  released;
* a decode step builds its step plan (``decode_plan``) once, at its first layer,
  and every later layer reuses it;
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

from .cache import BlockPool, KVCacheError, KVManager, PagedKVCache, PoolExhausted, PrefixCache
from .kernels import (decode_plan, paged_attention, qk_norm_rope_append, qk_norm_rope_store_and_decode, store_kv,
                      store_kv_and_decode, store_kv_and_prefill)

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
    pages: np.ndarray | None = None   # page ids this step reads or writes (held in flight)
    event: object | None = None       # recorded after the step's latest launch
    closed: bool = False              # no further launch will be recorded
    plan: object | None = None        # decode step plan, built at the first layer

    def _launched(self) -> None:
        """Record the step's completion event after a launch on the current stream."""
        if self.event is None:
            self.event = self.runner._event_factory()
        self.event.record()

    def _decode_plan(self, q: torch.Tensor):
        # (lazy: the step's first layer decodes unplanned and writes the plan the others read)
        if self.plan is None:
            self.plan = decode_plan(q.shape, self.runner.cache.kv, self.block_tables, self.seq_lens, self.active,
                                    self.slot_mapping, max_seq_len=self.max_len, lazy=True)
        return self.plan

    def store_attend(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     out: torch.Tensor | None = None) -> torch.Tensor:
        """Append this step's k, v (fp16 [T, Hkv, D]) for ``layer``, then attend with q (fp16 [T, Hq, D]).

        A prefill chunk, and a decode step without a shared prefix, do both in one launch
        (``store_kv_and_prefill`` / ``store_kv_and_decode``).
        """
        if self.closed:
            raise RunnerError("this step is closed: a later step has begun")
        kv = self.runner.cache.kv
        if self.query_start is not None:
            o = store_kv_and_prefill(q, kv, self.block_tables, k, v, query_start=self.query_start, layer=layer,
                                     out=out)
        elif self.shared_prefix is None:
            o = store_kv_and_decode(q, kv, self.block_tables, self.seq_lens, self.active, self.slot_mapping, k, v,
                                    layer=layer, max_seq_len=self.max_len, out=out, plan=self._decode_plan(q))
        else:
            store_kv(kv, self.slot_mapping, self.active, k, v, layer=layer)
            # (unplanned: a shared-prefix step plan measures no faster than the kernel's own split)
            o = paged_attention(q, kv, self.block_tables, self.seq_lens, self.active, layer=layer,
                                max_seq_len=self.max_len, out=out, shared_prefix_pages=self.shared_prefix)
        self._launched()
        return o

    def prep_store_attend(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor, rope: torch.Tensor,
                          eps: float = 1e-6, out: torch.Tensor | None = None) -> torch.Tensor:
        """The same from fp32 projections: q/k RMSNorm + rotary, fp16 cast and append.

        A decode step without a shared prefix does all of it and the attention in one launch
        (``qk_norm_rope_store_and_decode``); otherwise the pre-append is its own launch.  (A prefill
        chunk keeps two launches: ``qk_norm_rope_append_and_prefill`` does it in one, but every
        workgroup then prepares the chunk rows it reads itself, which measures slower.)
        """
        if self.closed:
            raise RunnerError("this step is closed: a later step has begun")
        kv = self.runner.cache.kv
        if self.query_start is None and self.shared_prefix is None:
            o = qk_norm_rope_store_and_decode(q, k, v, q_norm_weight, k_norm_weight, rope, self.positions,
                                              self.slot_mapping, self.active, kv, self.block_tables, self.seq_lens,
                                              layer=layer, eps=eps, max_seq_len=self.max_len, out=out,
                                              plan=self._decode_plan(q))
            self._launched()
            return o
        q16 = qk_norm_rope_append(q, k, v, q_norm_weight, k_norm_weight, rope, self.positions, self.slot_mapping,
                                  self.active, kv, layer=layer, eps=eps)
        if self.query_start is not None:  # a prefill chunk
            o = paged_attention(q16, kv, self.block_tables, None, None, layer=layer, query_start=self.query_start,
                                out=out)
        else:  # a decode step over a shared prefix
            o = paged_attention(q16, kv, self.block_tables, self.seq_lens, self.active, layer=layer,
                                max_seq_len=self.max_len, out=out, shared_prefix_pages=self.shared_prefix)
        self._launched()
        return o


class PagedKVRunner:
    """Paged KV state for ``num_slots`` concurrent sequences of up to ``max_context`` tokens."""

    def __init__(self, num_layers: int, num_slots: int, max_context: int, num_kv_heads: int, head_dim: int,
                 num_blocks: int, device: str | torch.device = "cuda", block_size: int = 16,
                 prefix_namespace=None, prefix_capacity_blocks: int | None = None,
                 shared_prefix_min_pages: int = 64, event_factory=None):
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
        # completion events of submitted steps (an object with record() and query(); on a GPU a
        # torch.cuda.Event recorded on the current stream)
        self._event_factory = event_factory or (
            (lambda: torch.cuda.Event()) if self.device.type == "cuda" else _CompletedEvent)
        self._inflight: list[_Step] = []  # steps whose pages are held in flight
        self._zero_on_release: set[int] = set()

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
        self._close_steps()
        if slot not in self.mgr:
            self.mgr.add_sequence(slot)
        slots = self._reserve(lambda: self.mgr.append(slot, num_tokens))
        pos = np.arange(start_position, start_position + num_tokens, dtype=np.int32)
        table = self._table([slot])[0]
        used = table[:-(-(start_position + num_tokens) // self.block_size)]
        return self._submit(_Step(self, self._dev(slots.astype(np.int32)), self._dev(table), None, None,
                                  self._dev(pos), start_position, start_position + num_tokens), used)

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
        self._close_steps()
        new_slots = self._reserve(lambda: self.mgr.append_batch([slots[i] for i in live], [1] * len(live)))
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
        used = [table[i, :-(-int(lens[i]) // self.block_size)] for i in live]
        return self._submit(_Step(self, self._dev(sm), self._dev(table), self._dev(lens), self._dev(act),
                                  self._dev(np.asarray(positions, np.int32)), None,
                                  int(lens.max()) if len(lens) else 0, prefix),
                            np.concatenate(used) if used else np.zeros(0, np.int32))

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
        """Release the slot's pages (runner.py:38-43); ``zero`` also zeroes the freed pages.

        Returns the pages that returned to the free pool now.  Pages that submitted work still
        reads or writes return (and, with ``zero``, are zeroed) once that work has completed.
        """
        self._check_slot(slot)
        if slot not in self.mgr:
            return []
        for st in self._inflight:  # the engine clears slots between steps: no step takes more launches
            st.closed = True
        owned = self.mgr.blocks(slot)
        freed = self.mgr.free_sequence(slot)
        if zero:
            if freed:
                self.cache.clear_pages(freed)
            held = set(owned) - set(freed)
            self._zero_on_release.update(p for p in held if self.pool.refcount(p, "inflight") > 0)
        return freed + self.reclaim()

    # -- in-flight pages ----------------------------------------------------------------------

    def _submit(self, step: _Step, pages: np.ndarray) -> _Step:
        """Hold the step's pages in flight until its work has completed."""
        ids = np.unique(np.asarray(pages, np.int64))
        if self.pool.dummy_block is not None:
            ids = ids[ids != self.pool.dummy_block]
        step.pages = ids
        if ids.size:
            self.pool.mark_in_flight(ids)
        self._inflight.append(step)
        return step

    def _close_steps(self) -> None:
        """A new step begins: earlier steps take no further launches; release what has completed."""
        for st in self._inflight:
            st.closed = True
        self.reclaim()

    def _reserve(self, take):
        """Run a page reservation (all or nothing).  When the pool is exhausted while submitted
        steps still hold pages in flight, wait for them, release their pages and try once more;
        an exhausted pool raises PoolExhausted, any other refusal RunnerError."""
        try:
            return take()
        except PoolExhausted:
            if not self._inflight:
                raise
            self.synchronize()
        except KVCacheError as e:
            raise RunnerError(str(e)) from e
        try:
            return take()
        except KVCacheError as e:
            raise RunnerError(str(e)) from e

    def reclaim(self) -> list[int]:
        """Release the pages of closed steps whose work has completed (no blocking); returns the
        pages that returned to the free pool."""
        released: list[int] = []
        keep = []
        for st in self._inflight:
            if st.closed and (st.event is None or st.event.query()):
                if st.pages is not None and st.pages.size:
                    released += self.pool.release_in_flight(st.pages)
            else:
                keep.append(st)
        self._inflight = keep
        if released and self._zero_on_release:
            z = [p for p in released if p in self._zero_on_release]
            if z:
                self._zero_on_release.difference_update(z)
                self.cache.clear_pages(z)
        return released

    def synchronize(self) -> list[int]:
        """Wait for every submitted step's work, close all steps and release their pages."""
        for st in self._inflight:
            st.closed = True
            if st.event is not None:
                st.event.synchronize()
        return self.reclaim()

    @property
    def pages_in_flight(self) -> int:
        """Distinct pages held by submitted, unreleased steps."""
        if not self._inflight:
            return 0
        return int(np.unique(np.concatenate([st.pages for st in self._inflight if st.pages is not None])).size)


class _CompletedEvent:
    """Completion event for a runner without a GPU: work is complete as soon as it is recorded."""

    def record(self, stream=None) -> None:
        pass

    def query(self) -> bool:
        return True

    def synchronize(self) -> None:
        pass
