"""paged_attention: GQA attention that gathers K/V pages through block tables (HIP, gfx950).

Mirrors the reference's documented operation
``paged_attention(query, kv_pool, block_tables, sequence_lengths, active_mask)``
(docs/architecture.md:242-246; src/infurnace/kernels/paged_attention.py is a
0-byte placeholder).  It replaces the contiguous attention of
src/infurnace/executor/tinygrad/model.py:

  * decode (model.py:196-200): one query per sequence at position L-1 reads
    keys [0, L) -- ``query`` [B, Hq, D], ``sequence_lengths`` = L per row;
  * chunked prefill (model.py:116-132): ``query`` [T, Hq, D] of one sequence
    with ``query_start`` = start_position; row i attends keys
    [0, query_start + i] (mask key_pos <= query_pos, model.py:128-132).  The
    chunk's K/V must already be in the pool (store_kv first).

Both compute softmax(scale * q k^T) v with fp16 inputs, fp32 accumulation and
fp16 output; query head h reads kv head h // (Hq // Hkv) (enable_gqa=True);
``scale`` defaults to 1/sqrt(D) (tinygrad's default).  Inactive rows write
nothing.
"""
from __future__ import annotations

import math

import torch

from .. import _capi
from ._common import PagedAttentionError, check_pool, current_stream, ptr
from ._carrier import accepts_carriers

__all__ = ["paged_attention", "store_kv_and_decode", "store_kv_and_prefill", "PagedAttentionError",
           "workspace_for", "DecodePlan", "decode_plan"]

# One zero-initialised workspace per (device, stream): every kernel call leaves
# the workspace's ticket counters at zero, so the buffer is reused as is.
_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def workspace_for(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """Zero-filled uint8 scratch of at least ``nbytes`` for calls on ``stream``."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        # grow geometrically so ragged batches do not reallocate every call
        # (the caching allocator keeps the old block alive for work queued on this stream)
        size = max(nbytes, 2 * ws.numel() if ws is not None else 0, 1 << 20)
        ws = torch.zeros(size, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


class DecodePlan:
    """The split of one decode step's keys over the CUs (``ifn_paged_decode_plan``).

    Every layer of a decode step attends with the same block tables, lengths,
    active mask and appended slots, and the decode kernel's split depends on
    nothing else; a plan built once per step lets each layer's launch start its
    page loads one round trip after launch.  It is valid only for calls with the
    tensors it was built from, unchanged: the wrappers check that the same
    tensors and shapes are passed (any layer of the same pool), and with
    ``validate=True`` also their contents (the plan is rebuilt and compared byte
    for byte).

    A lazy plan (``decode_plan(..., lazy=True)``) is built by the first decode call
    that takes it (``ifn_paged_decode_planning`` and its append / pre-append forms):
    that call decodes unplanned and writes the plan, so the step needs no plan
    launch of its own.  It takes the form of that call: built by a call without
    slots, it serves the fused-append calls only as an unplanned split.
    """

    def __init__(self, buf, nbytes: int, key: tuple, rebuild=None, pending: bool = False):
        self.buf, self.nbytes, self.key, self._rebuild = buf, nbytes, key, rebuild
        self.pending = pending and buf is not None

    def check_current(self) -> None:
        """Validate mode: raise unless a plan built now from the same tensors is identical
        (their contents were not changed since this one was built)."""
        if self.buf is None or self._rebuild is None or self.pending:
            return
        fresh = self._rebuild()
        if not torch.equal(fresh.buf, self.buf):
            raise PagedAttentionError("stale DecodePlan: the tables, lengths, mask or slots it was built from "
                                      "have changed since; build a new plan for this step")

    def ptr_for(self, key: tuple, need_slots: bool):
        """The plan's device address for a call with ``key``; None when these shapes need no plan."""
        if need_slots and self.key[1] is None:
            raise PagedAttentionError("this DecodePlan was built without slot_mapping; the fused append needs it")
        if key[0] != self.key[0] or key[2:] != self.key[2:] or (need_slots and key[1] != self.key[1]):
            raise PagedAttentionError("this DecodePlan was built for other tensors or shapes")
        return None if self.buf is None else self.buf.data_ptr()

    def entry(self, planned: str, planning: str) -> str:
        """The C entry point for the next call: ``planning`` while the plan is still to be built."""
        return planning if self.pending else planned

    def built(self) -> None:
        """The call that builds a lazy plan has been enqueued."""
        self.pending = False


def _plan_key(query_shape, slot_mapping, pool_layer, block_tables, sequence_lengths, active_mask, max_seq_len,
              shared_pages=None):
    """What a plan depends on, by tensor identity: shapes, the pool's page geometry, the tables,
    lengths, mask, slots, the length cap and (shared-prefix plans) the number of shared pages."""
    return (tuple(query_shape), None if slot_mapping is None else slot_mapping.data_ptr(),
            tuple(pool_layer.shape), block_tables.data_ptr(), tuple(block_tables.shape),
            sequence_lengths.data_ptr(), None if active_mask is None else active_mask.data_ptr(), int(max_seq_len),
            None if shared_pages is None else int(shared_pages))


@accepts_carriers
def decode_plan(query_shape, kv_pool: torch.Tensor, block_tables: torch.Tensor, sequence_lengths: torch.Tensor,
                active_mask: torch.Tensor | None = None, slot_mapping: torch.Tensor | None = None, *,
                layer: int = 0, block_size: int = 16, max_seq_len: int | None = None,
                shared_prefix_pages: torch.Tensor | None = None, lazy: bool = False) -> DecodePlan:
    """Build the step plan for decode calls with these tables, lengths, mask and (optionally) slots.

    ``query_shape`` is the decode query's shape [B, Hq, D].  The plan is computed on the
    current stream.  Pass it as ``plan=`` to ``paged_attention`` / ``store_kv_and_decode`` for
    every layer of the step; with ``slot_mapping`` it also serves the fused append.  With
    ``shared_prefix_pages`` (the tensor the step's ``paged_attention`` calls pass; only its
    length matters here) it is the plan of the shared-prefix decode
    (``ifn_paged_decode_shared_prefix_plan``) and takes no slots.  Shapes that decode without a
    plan give an empty plan, which the calls accept and ignore.  ``lazy``: allocate the plan
    only; the step's first decode call builds it (not for the shared-prefix decode).
    """
    pool_layer, (P, bs, hkv, d) = check_pool(kv_pool, layer, PagedAttentionError)
    dev = pool_layer.device
    if bs != block_size:
        raise PagedAttentionError(f"kv_pool block_size {bs} != block_size argument {block_size}")
    n, hq, qd = (int(x) for x in query_shape)
    if qd != d or hq % hkv != 0:
        raise PagedAttentionError(f"query [B, {hq}, {qd}] does not match kv heads {hkv} x {d}")
    if not isinstance(block_tables, torch.Tensor) or block_tables.ndim != 2:
        raise PagedAttentionError("block_tables must be a rank-2 [B, max_pages] int32 tensor")
    max_pages = block_tables.shape[1]
    _check("block_tables", block_tables, (n, max_pages), (torch.int32,), dev)
    _check("sequence_lengths", sequence_lengths, (n,), (torch.int32,), dev)
    if active_mask is not None:
        _check("active_mask", active_mask, (n,), (torch.bool, torch.uint8), dev)
    if slot_mapping is not None:
        _check("slot_mapping", slot_mapping, (n,), (torch.int32,), dev)
    if max_pages < 1:
        raise PagedAttentionError("block_tables must have at least one column")
    cap = max_pages * bs
    msl = cap if max_seq_len is None else min(int(max_seq_len), cap)
    if msl < 0:
        raise PagedAttentionError("max_seq_len must be non-negative")
    sp = None
    if shared_prefix_pages is not None:
        if not isinstance(shared_prefix_pages, torch.Tensor) or shared_prefix_pages.ndim != 1:
            raise PagedAttentionError("shared_prefix_pages must be a rank-1 int32 tensor")
        sp = shared_prefix_pages.shape[0]
        if sp > max_pages:
            raise PagedAttentionError(f"{sp} shared pages exceed the table's {max_pages} columns")
        if slot_mapping is not None:
            raise PagedAttentionError("a shared-prefix plan takes no slot_mapping (that decode has no fused append)")
        if lazy:
            raise PagedAttentionError("a shared-prefix plan is built by decode_plan itself (lazy=False)")
    key = _plan_key((n, hq, d), slot_mapping, pool_layer, block_tables, sequence_lengths, active_mask, msl, sp)
    if n == 0:
        return DecodePlan(None, 0, key)
    lib = _capi.lib()
    nbytes = lib.ifn_paged_decode_plan_bytes(n, hq, hkv, d, bs, max_pages, msl)
    if nbytes == 0:
        return DecodePlan(None, 0, key)
    # zero-filled, so that words the kernel leaves unwritten compare equal between two plans
    buf = torch.zeros(nbytes, dtype=torch.uint8, device=dev)

    def rebuild():
        return decode_plan(query_shape, kv_pool, block_tables, sequence_lengths, active_mask, slot_mapping,
                           layer=layer, block_size=block_size, max_seq_len=max_seq_len,
                           shared_prefix_pages=shared_prefix_pages)
    if lazy:
        return DecodePlan(buf, nbytes, key, rebuild, pending=True)
    if sp is None:
        _capi.call("ifn_paged_decode_plan", buf.data_ptr(), nbytes, ptr(block_tables), max_pages,
                   ptr(sequence_lengths), ptr(active_mask), ptr(slot_mapping), P, n, hq, hkv, d, bs, msl,
                   current_stream(dev))
    else:
        _capi.call("ifn_paged_decode_shared_prefix_plan", buf.data_ptr(), nbytes, ptr(block_tables), max_pages,
                   ptr(sequence_lengths), ptr(active_mask), sp, P, n, hq, hkv, d, bs, msl, current_stream(dev))
    return DecodePlan(buf, nbytes, key, rebuild)


def _row_keys(sequence_lengths: torch.Tensor, active_mask, msl: int) -> torch.Tensor:
    """Keys each decode row attends (0 for inactive rows), on the device."""
    keys = sequence_lengths.to(torch.int64).clamp(0, msl)
    if active_mask is not None:
        keys = keys * active_mask.to(torch.bool)
    return keys


def _validate_pages(table: torch.Tensor, keys: torch.Tensor, num_pages: int, bs: int, what: str) -> None:
    """Validate mode: every table entry a row reads (its first ceil(keys / bs) entries) names a page of
    the pool.  The kernels read an entry outside the pool as a page without keys; here it raises.
    ``table`` is [rows, max_pages], ``keys`` [rows] (int64, on the device)."""
    need = (keys + bs - 1) // bs
    used = torch.arange(table.shape[1], device=table.device)[None, :] < need[:, None]
    bad = used & ((table < 0) | (table >= num_pages))
    if bool(bad.any()):
        row, col = (int(x) for x in bad.nonzero()[0])
        raise PagedAttentionError(f"{what}: block table row {row} entry {col} = {int(table[row, col])} "
                                  f"is not a page of the {num_pages}-page pool")


def _validate_shared_prefix(table: torch.Tensor, keys: torch.Tensor, pages: torch.Tensor, bs: int) -> None:
    """Validate mode: every row of at least S * bs keys starts its table with the S declared pages."""
    sp = pages.shape[0]
    if sp == 0:
        return
    casc = keys >= sp * bs
    bad = casc[:, None] & (table[:, :sp] != pages[None, :])
    if bool(bad.any()):
        row, col = (int(x) for x in bad.nonzero()[0])
        raise PagedAttentionError(f"shared_prefix_pages: row {row} of {int(keys[row])} keys has page "
                                  f"{int(table[row, col])} at entry {col}, not the declared {int(pages[col])}")


def _check(name: str, t, shape: tuple, dtypes: tuple, device) -> None:
    if not isinstance(t, torch.Tensor):
        raise PagedAttentionError(f"{name} must be a torch.Tensor")
    if t.dtype not in dtypes:
        raise PagedAttentionError(f"{name} dtype must be one of {dtypes}, got {t.dtype}")
    if tuple(t.shape) != tuple(shape):
        raise PagedAttentionError(f"{name} shape must be {tuple(shape)}, got {tuple(t.shape)}")
    if t.device != device:
        raise PagedAttentionError(f"{name} must be on {device}, got {t.device}")
    if not t.is_contiguous():
        raise PagedAttentionError(f"{name} must be contiguous")


@accepts_carriers
def paged_attention(query: torch.Tensor, kv_pool: torch.Tensor, block_tables: torch.Tensor,
                    sequence_lengths: torch.Tensor | None, active_mask: torch.Tensor | None = None, *,
                    layer: int = 0, scale: float | None = None, query_start: int | None = None,
                    out: torch.Tensor | None = None, block_size: int = 16,
                    max_seq_len: int | None = None, shared_prefix_pages: torch.Tensor | None = None,
                    plan: DecodePlan | None = None, validate: bool = False) -> torch.Tensor:
    """Paged GQA attention; returns ``out`` (allocated when None).

    Decode (``query_start is None``): ``query`` [B, Hq, D] fp16,
    ``block_tables`` int32 [B, max_pages], ``sequence_lengths`` int32 [B] on the
    device, ``active_mask`` bool/uint8 [B] or None.  ``max_seq_len`` is an
    optional host-side upper bound of ``sequence_lengths`` (default
    max_pages * block_size); every row's length is clamped to it, so a smaller
    value truncates attention.  ``shared_prefix_pages``
    (int32 [S] on the device) declares that every row of at least
    S * block_size keys starts its table with these S pages (a prefix-cache
    hit); they are then read once for the whole batch instead of once per row.
    The declaration is trusted unless ``validate``.  Without it the decode streams its
    pages (non-temporal loads, each page expected to be read by one row); an
    empty ``shared_prefix_pages`` declares rows that share pages outside a
    common leading run, and the decode then keeps pages in the caches.
    ``plan`` (decode only, from ``decode_plan`` over the same tensors, with the same
    ``shared_prefix_pages`` when they are given) is the step's precomputed split; the result is
    bit-identical without it.

    ``validate=True`` (a debug mode: it synchronises) checks, before the launch,
    what the kernels otherwise trust: that every table entry a row reads names a
    page of the pool, that ``shared_prefix_pages`` heads the table of every row
    long enough to include it, and that ``plan`` is current (rebuilt and compared
    byte for byte); it raises ``PagedAttentionError`` on a mismatch.  The launch
    itself, and so the result, is the same as without it.

    Prefill (``query_start`` given): ``query`` [T, Hq, D] of one sequence,
    ``block_tables`` int32 [max_pages] or [1, max_pages]; ``sequence_lengths`` is
    unused on the device (keys = query_start + T) and, when it is a host value,
    must equal query_start + T.  ``active_mask`` of one False row makes the call
    a no-op.
    """
    pool_layer, (P, bs, hkv, d) = check_pool(kv_pool, layer, PagedAttentionError)
    dev = pool_layer.device
    if bs != block_size:
        raise PagedAttentionError(f"kv_pool block_size {bs} != block_size argument {block_size}")
    if not isinstance(query, torch.Tensor) or query.ndim != 3:
        raise PagedAttentionError("query must be a rank-3 tensor ([B, Hq, D] decode or [T, Hq, D] prefill)")
    n, hq, qd = query.shape
    if qd != d:
        raise PagedAttentionError(f"query head_dim {qd} != kv head_dim {d}")
    if hq % hkv != 0:
        raise PagedAttentionError(f"num_q_heads {hq} is not a multiple of num_kv_heads {hkv}")
    _check("query", query, (n, hq, d), (torch.float16,), dev)
    if out is None:
        out = torch.zeros_like(query) if active_mask is not None else torch.empty_like(query)
    else:
        _check("out", out, (n, hq, d), (torch.float16,), dev)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if not scale > 0:
        raise PagedAttentionError(f"scale must be positive, got {scale}")
    stream = current_stream(dev)
    lib = _capi.lib()

    if query_start is None:
        if not isinstance(block_tables, torch.Tensor) or block_tables.ndim != 2:
            raise PagedAttentionError("block_tables must be a rank-2 [B, max_pages] int32 tensor")
        max_pages = block_tables.shape[1]
        _check("block_tables", block_tables, (n, max_pages), (torch.int32,), dev)
        _check("sequence_lengths", sequence_lengths, (n,), (torch.int32,), dev)
        if active_mask is not None:
            _check("active_mask", active_mask, (n,), (torch.bool, torch.uint8), dev)
        if max_pages < 1:
            raise PagedAttentionError("block_tables must have at least one column")
        cap = max_pages * bs
        msl = cap if max_seq_len is None else min(int(max_seq_len), cap)
        if msl < 0:
            raise PagedAttentionError("max_seq_len must be non-negative")
        if n == 0:
            return out
        if validate:
            keys = _row_keys(sequence_lengths, active_mask, msl)
            _validate_pages(block_tables, keys, P, bs, "paged_attention")
            if plan is not None:
                plan.check_current()
        if shared_prefix_pages is not None:
            if not isinstance(shared_prefix_pages, torch.Tensor) or shared_prefix_pages.ndim != 1:
                raise PagedAttentionError("shared_prefix_pages must be a rank-1 int32 tensor")
            sp = shared_prefix_pages.shape[0]
            _check("shared_prefix_pages", shared_prefix_pages, (sp,), (torch.int32,), dev)
            if sp > max_pages:
                raise PagedAttentionError(f"{sp} shared pages exceed the table's {max_pages} columns")
            if validate:
                _validate_shared_prefix(block_tables, keys, shared_prefix_pages, bs)
            nbytes = lib.ifn_paged_decode_shared_prefix_workspace_bytes(n, hq, hkv, d, bs, sp)
            ws = workspace_for(dev, stream, nbytes)
            if plan is not None:  # a plan from decode_plan(..., shared_prefix_pages=...)
                if plan.pending:
                    raise PagedAttentionError("a lazy DecodePlan cannot serve the shared-prefix decode")
                key = _plan_key((n, hq, d), None, pool_layer, block_tables, sequence_lengths, active_mask, msl, sp)
                pp = plan.ptr_for(key, False)
                _capi.call("ifn_paged_decode_shared_prefix_planned", ptr(out), ptr(query), ptr(pool_layer), P,
                           ptr(shared_prefix_pages), sp, ptr(block_tables), max_pages, ptr(sequence_lengths),
                           ptr(active_mask), n, hq, hkv, d, bs, msl, float(scale), pp, plan.nbytes if pp else 0,
                           ptr(ws), ws.numel(), stream)
                return out
            _capi.call("ifn_paged_decode_shared_prefix", ptr(out), ptr(query), ptr(pool_layer), P,
                       ptr(shared_prefix_pages), sp, ptr(block_tables), max_pages, ptr(sequence_lengths),
                       ptr(active_mask), n, hq, hkv, d, bs, msl, float(scale), ptr(ws), ws.numel(), stream)
            return out
        nbytes = lib.ifn_paged_decode_workspace_bytes(n, hq, hkv, d, bs, msl)
        ws = workspace_for(dev, stream, nbytes)
        if plan is not None:
            key = _plan_key((n, hq, d), None, pool_layer, block_tables, sequence_lengths, active_mask, msl)
            pp = plan.ptr_for(key, False)
            _capi.call(plan.entry("ifn_paged_decode_planned", "ifn_paged_decode_planning"), ptr(out), ptr(query),
                       ptr(pool_layer), P, ptr(block_tables), max_pages, ptr(sequence_lengths), ptr(active_mask), n,
                       hq, hkv, d, bs, msl, float(scale), pp, plan.nbytes if pp else 0, ptr(ws), ws.numel(), stream)
            plan.built()
            return out
        _capi.call("ifn_paged_decode", ptr(out), ptr(query), ptr(pool_layer), P, ptr(block_tables),
                   max_pages, ptr(sequence_lengths), ptr(active_mask), n, hq, hkv, d, bs, msl,
                   float(scale), ptr(ws), ws.numel(), stream)
        return out

    # chunked prefill of one sequence
    query_start = int(query_start)
    if query_start < 0:
        raise PagedAttentionError(f"query_start must be non-negative, got {query_start}")
    if not isinstance(block_tables, torch.Tensor):
        raise PagedAttentionError("block_tables must be a torch.Tensor")
    table = block_tables.reshape(-1) if block_tables.ndim == 2 and block_tables.shape[0] == 1 else block_tables
    if table.ndim != 1:
        raise PagedAttentionError("prefill block_tables must be [max_pages] or [1, max_pages]")
    max_pages = table.shape[0]
    _check("block_tables", table, (max_pages,), (torch.int32,), dev)
    total = query_start + n
    if total > max_pages * bs:
        raise PagedAttentionError(f"query_start + T = {total} exceeds the table's {max_pages * bs} slots")
    if isinstance(sequence_lengths, torch.Tensor) and sequence_lengths.device.type == "cpu":
        if sequence_lengths.numel() != 1 or int(sequence_lengths.reshape(-1)[0]) != total:
            raise PagedAttentionError(f"sequence_lengths must be [{total}] (= query_start + T)")
    elif isinstance(sequence_lengths, (list, tuple)):
        if list(sequence_lengths) != [total]:
            raise PagedAttentionError(f"sequence_lengths must be [{total}] (= query_start + T)")
    if active_mask is not None:
        if active_mask.numel() != 1:
            raise PagedAttentionError("prefill active_mask must have exactly one element")
        if not bool(active_mask.reshape(-1)[0]):
            return out
    if n == 0:
        return out
    if validate:
        _validate_pages(table[None, :], torch.full((1,), total, dtype=torch.int64, device=dev), P, bs,
                        "paged_attention (prefill)")
    nbytes = lib.ifn_paged_prefill_workspace_bytes(n, query_start, hq, hkv, d, bs)
    ws = workspace_for(dev, stream, nbytes)
    _capi.call("ifn_paged_prefill", ptr(out), ptr(query), ptr(pool_layer), P, ptr(table), max_pages,
               query_start, n, hq, hkv, d, bs, float(scale), ptr(ws), ws.numel(), stream)
    return out


@accepts_carriers
def store_kv_and_decode(query: torch.Tensor, kv_pool: torch.Tensor, block_tables: torch.Tensor,
                        sequence_lengths: torch.Tensor, active_mask: torch.Tensor | None,
                        slot_mapping: torch.Tensor, new_k: torch.Tensor, new_v: torch.Tensor, *, layer: int = 0,
                        scale: float | None = None, out: torch.Tensor | None = None, block_size: int = 16,
                        max_seq_len: int | None = None, plan: DecodePlan | None = None,
                        validate: bool = False) -> torch.Tensor:
    """One decode step's append and attention in one launch (``ifn_paged_decode_append``).

    Same result, in ``out`` and in the pool, as ``store_kv(kv_pool, slot_mapping, active_mask,
    new_k, new_v, layer=layer)`` followed by ``paged_attention(query, kv_pool, block_tables,
    sequence_lengths, active_mask, layer=layer, ...)`` -- the store of model.py:191-196 and the
    attention of :196-200.  ``new_k``/``new_v`` are fp16 [B, Hkv, D], ``slot_mapping`` int32 [B].
    An appended slot must not be read by another row of the call (true of any paged KV state).
    ``plan``: the step's ``decode_plan`` built with this ``slot_mapping``.  ``validate`` as for
    ``paged_attention``, plus the slots (as ``store_kv(..., validate=True)``).
    """
    from .kv_store import _check_index, _check_rows
    if slot_mapping is None:
        raise PagedAttentionError("store_kv_and_decode needs a slot_mapping")
    pool_layer, (P, bs, hkv, d) = check_pool(kv_pool, layer, PagedAttentionError)
    dev = pool_layer.device
    if bs != block_size:
        raise PagedAttentionError(f"kv_pool block_size {bs} != block_size argument {block_size}")
    if not isinstance(query, torch.Tensor) or query.ndim != 3:
        raise PagedAttentionError("query must be a rank-3 [B, Hq, D] tensor")
    n, hq, qd = query.shape
    if qd != d or hq % hkv != 0:
        raise PagedAttentionError(f"query [B, {hq}, {qd}] does not match kv heads {hkv} x {d}")
    _check("query", query, (n, hq, d), (torch.float16,), dev)
    if not isinstance(block_tables, torch.Tensor) or block_tables.ndim != 2:
        raise PagedAttentionError("block_tables must be a rank-2 [B, max_pages] int32 tensor")
    max_pages = block_tables.shape[1]
    _check("block_tables", block_tables, (n, max_pages), (torch.int32,), dev)
    _check("sequence_lengths", sequence_lengths, (n,), (torch.int32,), dev)
    if active_mask is not None:
        _check("active_mask", active_mask, (n,), (torch.bool, torch.uint8), dev)
    _check_rows("new_k", new_k, (n,), hkv, d, dev)
    _check_rows("new_v", new_v, (n,), hkv, d, dev)
    sm = _check_index("slot_mapping", slot_mapping, n, dev, (torch.int32,))
    if max_pages < 1:
        raise PagedAttentionError("block_tables must have at least one column")
    if out is None:
        out = torch.zeros_like(query) if active_mask is not None else torch.empty_like(query)
    else:
        _check("out", out, (n, hq, d), (torch.float16,), dev)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if not scale > 0:
        raise PagedAttentionError(f"scale must be positive, got {scale}")
    cap = max_pages * bs
    msl = cap if max_seq_len is None else min(int(max_seq_len), cap)
    if msl < 0:
        raise PagedAttentionError("max_seq_len must be non-negative")
    if n == 0:
        return out
    if validate:
        from .kv_store import _debug_validate
        _debug_validate(sm, active_mask, P * bs)
        _validate_pages(block_tables, _row_keys(sequence_lengths, active_mask, msl), P, bs, "store_kv_and_decode")
        if plan is not None:
            plan.check_current()
    stream = current_stream(dev)
    lib = _capi.lib()
    nbytes = lib.ifn_paged_decode_workspace_bytes(n, hq, hkv, d, bs, msl)
    ws = workspace_for(dev, stream, nbytes)
    if plan is not None:
        key = _plan_key((n, hq, d), sm, pool_layer, block_tables, sequence_lengths, active_mask, msl)
        pp = plan.ptr_for(key, True)
        _capi.call(plan.entry("ifn_paged_decode_append_planned", "ifn_paged_decode_append_planning"), ptr(out),
                   ptr(query), ptr(pool_layer), P, ptr(block_tables), max_pages, ptr(sequence_lengths),
                   ptr(active_mask), ptr(sm), ptr(new_k), ptr(new_v), n, hq, hkv, d, bs, msl, float(scale), pp,
                   plan.nbytes if pp else 0, ptr(ws), ws.numel(), stream)
        plan.built()
        return out
    _capi.call("ifn_paged_decode_append", ptr(out), ptr(query), ptr(pool_layer), P, ptr(block_tables), max_pages,
               ptr(sequence_lengths), ptr(active_mask), ptr(sm), ptr(new_k), ptr(new_v), n, hq, hkv, d, bs, msl,
               float(scale), ptr(ws), ws.numel(), stream)
    return out


@accepts_carriers
def store_kv_and_prefill(query: torch.Tensor, kv_pool: torch.Tensor, block_table: torch.Tensor, new_k: torch.Tensor,
                         new_v: torch.Tensor, *, query_start: int, layer: int = 0, scale: float | None = None,
                         out: torch.Tensor | None = None, block_size: int = 16, validate: bool = False) -> torch.Tensor:
    """One prefill chunk's append and causal attention (``ifn_paged_prefill_append``).

    Same result, in ``out`` and in the pool, as ``store_kv`` of ``new_k``/``new_v`` [T, Hkv, D] at
    the table's slots for positions query_start .. query_start + T - 1 followed by
    ``paged_attention(query, ..., query_start=query_start)`` -- the store of model.py:134-138 and
    the attention of :116-132.  One launch when query_start % 32 == 0, else the store and the
    attention as two launches.  ``validate``: every table entry the chunk's keys use names a page
    of the pool (checked before the launch; a debug mode that synchronises).
    """
    from .kv_store import _check_rows
    pool_layer, (P, bs, hkv, d) = check_pool(kv_pool, layer, PagedAttentionError)
    dev = pool_layer.device
    if bs != block_size:
        raise PagedAttentionError(f"kv_pool block_size {bs} != block_size argument {block_size}")
    if not isinstance(query, torch.Tensor) or query.ndim != 3:
        raise PagedAttentionError("query must be a rank-3 [T, Hq, D] tensor")
    n, hq, qd = query.shape
    if qd != d or hq % hkv != 0:
        raise PagedAttentionError(f"query [T, {hq}, {qd}] does not match kv heads {hkv} x {d}")
    _check("query", query, (n, hq, d), (torch.float16,), dev)
    _check_rows("new_k", new_k, (n,), hkv, d, dev)
    _check_rows("new_v", new_v, (n,), hkv, d, dev)
    query_start = int(query_start)
    if query_start < 0:
        raise PagedAttentionError(f"query_start must be non-negative, got {query_start}")
    if not isinstance(block_table, torch.Tensor):
        raise PagedAttentionError("block_table must be a torch.Tensor")
    table = block_table.reshape(-1) if block_table.ndim == 2 and block_table.shape[0] == 1 else block_table
    if table.ndim != 1:
        raise PagedAttentionError("block_table must be [max_pages] or [1, max_pages]")
    max_pages = table.shape[0]
    _check("block_table", table, (max_pages,), (torch.int32,), dev)
    if query_start + n > max_pages * bs:
        raise PagedAttentionError(f"query_start + T = {query_start + n} exceeds the table's {max_pages * bs} slots")
    if out is None:
        out = torch.empty_like(query)
    else:
        _check("out", out, (n, hq, d), (torch.float16,), dev)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if not scale > 0:
        raise PagedAttentionError(f"scale must be positive, got {scale}")
    if n == 0:
        return out
    if validate:
        _validate_pages(table[None, :], torch.full((1,), query_start + n, dtype=torch.int64, device=dev), P, bs,
                        "store_kv_and_prefill")
    stream = current_stream(dev)
    lib = _capi.lib()
    nbytes = lib.ifn_paged_prefill_workspace_bytes(n, query_start, hq, hkv, d, bs)
    ws = workspace_for(dev, stream, nbytes)
    _capi.call("ifn_paged_prefill_append", ptr(out), ptr(query), ptr(pool_layer), P, ptr(table), max_pages,
               query_start, n, ptr(new_k), ptr(new_v), hq, hkv, d, bs, float(scale), ptr(ws), ws.numel(), stream)
    return out

