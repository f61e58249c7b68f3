"""Pre-append step and page utilities of the KV-cache path (HIP, gfx950).

``qk_norm_rope_append`` fuses the steps between the Q/K/V projections and the
cache write in the reference's forward pass
(src/infurnace/executor/tinygrad/model.py:183-196 for decode, :109-137 for
prefill): per-head RMSNorm of q and k (``_rms_norm``, :11-13), the half-split
rotary embedding (``_apply_rope`` :24-27 over the table of ``_precompute_rope``
:19-23), the fp32 -> fp16 cast, and the slot-mapped store of k and v.  One
launch replaces a norm, a rope and a store pass over K.

``zero_pages`` is the paged form of ``ContiguousKVCache.clear_slot``
(src/infurnace/executor/tinygrad/buffers.py:67-81): a released sequence's pages
return to the freshly allocated (zero) state.  ``copy_pages`` gives a sequence a
private copy of a block (partial tail blocks are never shared,
docs/architecture.md:381-391).
"""
from __future__ import annotations

import math

import numpy as np
import torch

from .. import _capi
from ._common import KVStoreError, PagedAttentionError, check_pool, current_stream, ptr
from ._carrier import accepts_carriers

__all__ = ["qk_norm_rope_append", "qk_norm_rope_store_and_decode", "qk_norm_rope_append_and_prefill", "rope_table",
           "zero_pages", "copy_pages"]


def rope_table(max_positions: int, head_dim: int, base: float, device=None) -> torch.Tensor:
    """fp32 [max_positions, head_dim] rows ``[cos(p f_i) | sin(p f_i)]``, f_i = base^(-2i/D), i < D/2.

    ``_precompute_rope`` (model.py:18-22) in its own order and precision: the exponents
    2i/D, base^(2i/D), the inverse frequencies f_i and the angles p * f_i are float32 values,
    each rounded once; cos and sin of those float32 angles are then rounded once to float32
    (the reference's float32 cos/sin may differ from these by an ulp).
    """
    if max_positions < 1 or head_dim < 2 or head_dim % 2 or not base > 0:
        raise ValueError("rope_table needs max_positions >= 1, an even head_dim and base > 0")
    f32 = np.float32
    expo = (np.arange(0, head_dim, 2, dtype=f32) / f32(head_dim)).astype(f32)
    inv = (f32(1.0) / np.power(f32(base), expo).astype(f32)).astype(f32)
    ang = (np.arange(max_positions, dtype=f32)[:, None] * inv[None, :]).astype(f32)
    a64 = ang.astype(np.float64)
    table = np.concatenate([np.cos(a64), np.sin(a64)], axis=1).astype(f32)
    return torch.from_numpy(table).to(device) if device is not None else torch.from_numpy(table)


def _f32(name: str, t, shape: tuple, device) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise KVStoreError(f"{name} must be a torch.Tensor")
    if t.dtype != torch.float32:
        raise KVStoreError(f"{name} dtype must be float32, got {t.dtype}")
    if tuple(t.shape) != shape:
        raise KVStoreError(f"{name} shape must be {shape}, got {tuple(t.shape)}")
    if t.device != device or not t.is_contiguous():
        raise KVStoreError(f"{name} must be a contiguous tensor on {device}")
    return t


def _i32(name: str, t, n: int, device, dtypes=(torch.int32,)) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or t.dtype not in dtypes or tuple(t.shape) != (n,):
        raise KVStoreError(f"{name} must be a {dtypes} tensor of shape ({n},)")
    if t.device != device or not t.is_contiguous():
        raise KVStoreError(f"{name} must be a contiguous tensor on {device}")
    return t


@accepts_carriers
def qk_norm_rope_append(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_norm_weight: torch.Tensor,
                        k_norm_weight: torch.Tensor, rope: torch.Tensor, positions: torch.Tensor,
                        slot_mapping: torch.Tensor, active_mask: torch.Tensor | None, kv_pool: torch.Tensor, *,
                        layer: int = 0, eps: float = 1e-6, q_out: torch.Tensor | None = None) -> torch.Tensor:
    """Normalise and rotate q, k; store k and v (fp16) at their slots; return q as fp16.

    q fp32 [T, Hq, D]; k, v fp32 [T, Hkv, D]; norm weights fp32 [D]; ``rope`` from
    ``rope_table``; positions and slot_mapping int32 [T]; active_mask bool/uint8 [T] or
    None.  A token whose position is outside the table stores nothing and gets a zero
    q row.
    """
    pool_layer, (P, bs, hkv, d) = check_pool(kv_pool, layer, KVStoreError)
    dev = pool_layer.device
    if not isinstance(q, torch.Tensor) or q.ndim != 3:
        raise KVStoreError("q must be a rank-3 [T, Hq, D] tensor")
    T, hq = q.shape[0], q.shape[1]
    if hq % hkv:
        raise KVStoreError(f"num_q_heads {hq} is not a multiple of num_kv_heads {hkv}")
    _f32("q", q, (T, hq, d), dev)
    _f32("k", k, (T, hkv, d), dev)
    _f32("v", v, (T, hkv, d), dev)
    _f32("q_norm_weight", q_norm_weight, (d,), dev)
    _f32("k_norm_weight", k_norm_weight, (d,), dev)
    if not isinstance(rope, torch.Tensor) or rope.ndim != 2:
        raise KVStoreError("rope must be the rank-2 table of rope_table()")
    _f32("rope", rope, (rope.shape[0], d), dev)
    _i32("positions", positions, T, dev)
    _i32("slot_mapping", slot_mapping, T, dev)
    if active_mask is not None:
        _i32("active_mask", active_mask, T, dev, (torch.bool, torch.uint8))
    if not (eps >= 0 and math.isfinite(eps)):
        raise KVStoreError("eps must be a finite non-negative number")
    if q_out is None:
        q_out = torch.empty((T, hq, d), dtype=torch.float16, device=dev)
    elif q_out.dtype != torch.float16 or tuple(q_out.shape) != (T, hq, d) or q_out.device != dev or \
            not q_out.is_contiguous():
        raise KVStoreError(f"q_out must be a contiguous float16 [{T}, {hq}, {d}] tensor on {dev}")
    if T == 0:
        return q_out
    _capi.call("ifn_qk_norm_rope_append", ptr(q_out), ptr(q), ptr(k), ptr(v), ptr(q_norm_weight),
               ptr(k_norm_weight), ptr(rope), rope.shape[0], ptr(positions), ptr(slot_mapping), ptr(active_mask),
               ptr(pool_layer), P, T, hq, hkv, d, bs, float(eps), current_stream(dev))
    return q_out


def _full_pool(kv_pool) -> tuple:
    if not isinstance(kv_pool, torch.Tensor) or kv_pool.ndim != 6:
        raise KVStoreError("kv_pool must be the rank-6 [layers, 2, pages, block_size, Hkv, D] pool")
    check_pool(kv_pool, 0, KVStoreError)
    return kv_pool.shape


@accepts_carriers
def zero_pages(kv_pool: torch.Tensor, page_ids: torch.Tensor) -> None:
    """Zero K and V of every listed page in every layer (ids outside the pool are skipped)."""
    L, _, P, bs, hkv, d = _full_pool(kv_pool)
    ids = _i32("page_ids", page_ids, page_ids.numel() if isinstance(page_ids, torch.Tensor) else -1,
               kv_pool.device)
    _capi.call("ifn_zero_pages", ptr(kv_pool), L, P, ptr(ids), ids.numel(), hkv, d, bs,
               current_stream(kv_pool.device))


@accepts_carriers
def copy_pages(kv_pool: torch.Tensor, src_ids: torch.Tensor, dst_ids: torch.Tensor) -> None:
    """Copy page src_ids[i] to dst_ids[i] in every layer.  Destinations must be distinct and
    disjoint from the sources (checked here on the host)."""
    L, _, P, bs, hkv, d = _full_pool(kv_pool)
    n = src_ids.numel() if isinstance(src_ids, torch.Tensor) else -1
    src = _i32("src_ids", src_ids, n, kv_pool.device)
    dst = _i32("dst_ids", dst_ids, n, kv_pool.device)
    s, t = src.cpu().tolist(), dst.cpu().tolist()
    if len(set(t)) != len(t) or set(t) & set(s):
        raise KVStoreError("copy_pages destinations must be distinct and not among the sources")
    _capi.call("ifn_copy_pages", ptr(kv_pool), L, P, ptr(src), ptr(dst), n, hkv, d, bs,
               current_stream(kv_pool.device))


@accepts_carriers
def qk_norm_rope_store_and_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_norm_weight: torch.Tensor,
                                  k_norm_weight: torch.Tensor, rope: torch.Tensor, positions: torch.Tensor,
                                  slot_mapping: torch.Tensor, active_mask: torch.Tensor | None,
                                  kv_pool: torch.Tensor, block_tables: torch.Tensor,
                                  sequence_lengths: torch.Tensor, *, layer: int = 0, eps: float = 1e-6,
                                  scale: float | None = None, out: torch.Tensor | None = None,
                                  block_size: int = 16, max_seq_len: int | None = None, plan=None) -> torch.Tensor:
    """A decode step of one layer from fp32 projections: pre-append and attention in one launch.

    ``ifn_paged_decode_prep_append``: the same ``out`` and pool as ``qk_norm_rope_append(q, k, v,
    ..., positions, slot_mapping, active_mask, kv_pool, layer=layer, eps=eps)`` followed by
    ``paged_attention(q16, kv_pool, block_tables, sequence_lengths, active_mask, ...)`` -- the
    norm / rope / cast / store of model.py:183-196 and the attention of :196-200.  q fp32
    [B, Hq, D], k / v fp32 [B, Hkv, D]; ``plan`` a ``decode_plan`` built with ``slot_mapping``.
    Row b's appended token is at ``positions[b]`` and ``slot_mapping[b]`` is that position's slot
    in the row's table (the decode step's invariant).  Shapes the fused kernel does not cover
    (token row other than 2 KiB, head_dim > 128) run the two launches instead.
    """
    from .paged_attention import _check, _plan_key, paged_attention, workspace_for
    from .kv_store import _check_index
    pool_layer, (P, bs, hkv, d) = check_pool(kv_pool, layer, PagedAttentionError)
    dev = pool_layer.device
    if bs != block_size:
        raise PagedAttentionError(f"kv_pool block_size {bs} != block_size argument {block_size}")
    if not isinstance(q, torch.Tensor) or q.ndim != 3:
        raise PagedAttentionError("q must be a rank-3 [B, Hq, D] tensor")
    n, hq = q.shape[0], q.shape[1]
    if hq % hkv:
        raise PagedAttentionError(f"num_q_heads {hq} is not a multiple of num_kv_heads {hkv}")
    _f32("q", q, (n, hq, d), dev)
    _f32("k", k, (n, hkv, d), dev)
    _f32("v", v, (n, hkv, d), dev)
    _f32("q_norm_weight", q_norm_weight, (d,), dev)
    _f32("k_norm_weight", k_norm_weight, (d,), dev)
    if not isinstance(rope, torch.Tensor) or rope.ndim != 2:
        raise KVStoreError("rope must be the rank-2 table of rope_table()")
    _f32("rope", rope, (rope.shape[0], d), dev)
    _i32("positions", positions, n, dev)
    sm = _check_index("slot_mapping", slot_mapping, n, dev, (torch.int32,))
    if sm is None:
        raise PagedAttentionError("qk_norm_rope_store_and_decode needs a slot_mapping")
    if active_mask is not None:
        _i32("active_mask", active_mask, n, dev, (torch.bool, torch.uint8))
    if not isinstance(block_tables, torch.Tensor) or block_tables.ndim != 2:
        raise PagedAttentionError("block_tables must be a rank-2 [B, max_pages] int32 tensor")
    max_pages = block_tables.shape[1]
    _check("block_tables", block_tables, (n, max_pages), (torch.int32,), dev)
    _check("sequence_lengths", sequence_lengths, (n,), (torch.int32,), dev)
    if max_pages < 1:
        raise PagedAttentionError("block_tables must have at least one column")
    if not (eps >= 0 and math.isfinite(eps)):
        raise KVStoreError("eps must be a finite non-negative number")
    if out is None:
        out = torch.zeros((n, hq, d), dtype=torch.float16, device=dev) if active_mask is not None else \
            torch.empty((n, hq, d), dtype=torch.float16, device=dev)
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
    stream = current_stream(dev)
    lib = _capi.lib()
    nbytes = lib.ifn_paged_decode_workspace_bytes(n, hq, hkv, d, bs, msl)
    ws = workspace_for(dev, stream, nbytes)
    pp, pbytes, entry = None, 0, lib.ifn_paged_decode_prep_append
    if plan is not None:
        key = _plan_key((n, hq, d), sm, pool_layer, block_tables, sequence_lengths, active_mask, msl)
        pp = plan.ptr_for(key, True)
        pbytes = plan.nbytes if pp else 0
        entry = getattr(lib, plan.entry("ifn_paged_decode_prep_append", "ifn_paged_decode_prep_append_planning"))
    status = entry(
        ptr(out), ptr(q), ptr(k), ptr(v), ptr(q_norm_weight), ptr(k_norm_weight), ptr(rope), rope.shape[0],
        ptr(positions), ptr(sm), ptr(pool_layer), P, ptr(block_tables), max_pages, ptr(sequence_lengths),
        ptr(active_mask), n, hq, hkv, d, bs, msl, float(scale), float(eps), pp, pbytes, ptr(ws), ws.numel(), stream)
    if status == _capi.IFN_ERR_UNSUPPORTED:
        q16 = qk_norm_rope_append(q, k, v, q_norm_weight, k_norm_weight, rope, positions, sm, active_mask, kv_pool,
                                  layer=layer, eps=eps)
        return paged_attention(q16, kv_pool, block_tables, sequence_lengths, active_mask, layer=layer, scale=scale,
                               out=out, block_size=block_size, max_seq_len=max_seq_len, plan=plan)
    _capi.check("ifn_paged_decode_prep_append", status)
    if plan is not None:
        plan.built()
    return out


def qk_norm_rope_append_and_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_norm_weight: torch.Tensor,
                                    k_norm_weight: torch.Tensor, rope: torch.Tensor, kv_pool: torch.Tensor,
                                    block_table: torch.Tensor, *, query_start: int, layer: int = 0,
                                    eps: float = 1e-6, scale: float | None = None, out: torch.Tensor | None = None,
                                    block_size: int = 16, validate: bool = False) -> torch.Tensor:
    """A prefill chunk of one layer from fp32 projections: pre-append and attention in one launch.

    ``ifn_paged_prefill_prep_append``: the same ``out`` and pool as ``qk_norm_rope_append(q, k, v,
    ..., positions, slots, None, kv_pool, layer=layer, eps=eps)`` with positions query_start + t and
    their slots in ``block_table``, followed by ``paged_attention(q16, kv_pool, block_table, None,
    None, query_start=query_start)`` -- the norm / rope / attention / cache write of a prefill
    chunk, model.py:109-138.  q fp32 [T, Hq, D], k / v fp32 [T, Hkv, D].  A chunk the fused kernel
    does not take (query_start not a multiple of 32, an unaligned input) runs the two launches
    instead.  ``validate``: every table entry the chunk's keys use names a page of the pool
    (checked before the launch; a debug mode that synchronises).
    """
    from .paged_attention import _check, _validate_pages, paged_attention, workspace_for
    pool_layer, (P, bs, hkv, d) = check_pool(kv_pool, layer, PagedAttentionError)
    dev = pool_layer.device
    if bs != block_size:
        raise PagedAttentionError(f"kv_pool block_size {bs} != block_size argument {block_size}")
    if not isinstance(q, torch.Tensor) or q.ndim != 3:
        raise PagedAttentionError("q must be a rank-3 [T, Hq, D] tensor")
    n, hq = q.shape[0], q.shape[1]
    if hq % hkv:
        raise PagedAttentionError(f"num_q_heads {hq} is not a multiple of num_kv_heads {hkv}")
    _f32("q", q, (n, hq, d), dev)
    _f32("k", k, (n, hkv, d), dev)
    _f32("v", v, (n, hkv, d), dev)
    _f32("q_norm_weight", q_norm_weight, (d,), dev)
    _f32("k_norm_weight", k_norm_weight, (d,), dev)
    if not isinstance(rope, torch.Tensor) or rope.ndim != 2:
        raise KVStoreError("rope must be the rank-2 table of rope_table()")
    _f32("rope", rope, (rope.shape[0], d), dev)
    if not (eps >= 0 and math.isfinite(eps)):
        raise KVStoreError("eps must be a finite non-negative number")
    query_start = int(query_start)
    if query_start < 0:
        raise PagedAttentionError(f"query_start must be non-negative, got {query_start}")
    if query_start + n > rope.shape[0]:
        raise PagedAttentionError(f"positions up to {query_start + n - 1} are past the rope table's "
                                  f"{rope.shape[0]} rows")
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
        out = torch.empty((n, hq, d), dtype=torch.float16, device=dev)
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
                        "qk_norm_rope_append_and_prefill")
    stream = current_stream(dev)
    lib = _capi.lib()
    status = _capi.IFN_ERR_UNSUPPORTED
    aligned = all(t.data_ptr() % 16 == 0 for t in (q, k, v, q_norm_weight, k_norm_weight, rope, out, pool_layer))
    if query_start % 32 == 0 and aligned:
        nbytes = lib.ifn_paged_prefill_workspace_bytes(n, query_start, hq, hkv, d, bs)
        ws = workspace_for(dev, stream, nbytes)
        status = lib.ifn_paged_prefill_prep_append(
            ptr(out), ptr(q), ptr(k), ptr(v), ptr(q_norm_weight), ptr(k_norm_weight), ptr(rope), rope.shape[0],
            ptr(pool_layer), P, ptr(table), max_pages, query_start, n, hq, hkv, d, bs, float(eps), float(scale),
            ptr(ws), ws.numel(), stream)
    if status == _capi.IFN_ERR_UNSUPPORTED:
        pos = torch.arange(query_start, query_start + n, dtype=torch.int32, device=dev)
        slots = table[torch.div(pos, bs, rounding_mode="floor").long()] * bs + pos % bs
        q16 = qk_norm_rope_append(q, k, v, q_norm_weight, k_norm_weight, rope, pos, slots.to(torch.int32), None,
                                  kv_pool, layer=layer, eps=eps)
        return paged_attention(q16, kv_pool, table, None, None, layer=layer, query_start=query_start, scale=scale,
                               out=out, block_size=block_size)
    _capi.check("ifn_paged_prefill_prep_append", status)
    return out
