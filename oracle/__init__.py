"""CPU oracle for the KV-cache hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or the timed CPU
baseline).  The product path (``infurnace_amd``) never imports it.

It wraps ``ifn_oracle.c`` (plain C, built by ``oracle/build.py``) with numpy
arrays.  fp16 tensors travel as ``numpy.float16`` arrays and are handed to C as
their raw uint16 bit patterns, so byte-level results are exact.

Reference anchors (the reference's own path modules are 0-byte placeholders):
  * layout / slot mapping / store / attention contract:
    docs/architecture.md:225-235, 245-253
  * decode semantics: src/infurnace/executor/tinygrad/model.py:191-200
  * chunked-prefill semantics: src/infurnace/executor/tinygrad/model.py:116-138
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from .build import LIB_PATH, build as build_library

_lib = None


def lib() -> ctypes.CDLL:
    """Load (building on first use when absent) the oracle shared library."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build_library()
        L = ctypes.CDLL(LIB_PATH)
        p = ctypes.c_void_p
        i32, i64, f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float
        L.orc_half_to_float_array.argtypes = [p, p, i64]
        L.orc_float_to_half_array.argtypes = [p, p, i64]
        L.orc_slot_mapping.argtypes = [p, i32, p, p, i32, i32, p]
        L.orc_slot_mapping.restype = ctypes.c_int
        L.orc_store_kv.argtypes = [p, i64, p, p, p, p, i32, i32, i32, i32]
        L.orc_paged_attention.argtypes = [p, p, p, i64, p, i32, p, p, i32, i32, i32, i32, i32, i32, f32]
        L.orc_paged_attention.restype = ctypes.c_int
        L.orc_qk_norm_rope_append.argtypes = [p, p, i64, p, p, p, p, p, p, i32, p, p, p, i32, i32, i32, i32, i32,
                                              f32]
        L.orc_qk_norm_rope_append.restype = ctypes.c_int
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype != dtype:
        raise TypeError(f"expected {np.dtype(dtype)}, got {a.dtype}")
    return np.ascontiguousarray(a)


def half_to_float(h: np.ndarray) -> np.ndarray:
    h = _c(h, np.float16)
    out = np.empty(h.shape, np.float32)
    lib().orc_half_to_float_array(_ptr(h), _ptr(out), h.size)
    return out


def float_to_half(f: np.ndarray) -> np.ndarray:
    f = _c(f, np.float32)
    out = np.empty(f.shape, np.float16)
    lib().orc_float_to_half_array(_ptr(f), _ptr(out), f.size)
    return out


def slot_mapping(block_tables, seq_idx, positions, block_size: int = 16) -> np.ndarray:
    """``slot = table[seq][pos // bs] * bs + pos % bs`` (docs/architecture.md:235)."""
    bt = _c(block_tables, np.int32)
    si = _c(seq_idx, np.int32)
    pos = _c(positions, np.int32)
    out = np.empty(pos.shape, np.int32)
    rc = lib().orc_slot_mapping(_ptr(bt), bt.shape[1], _ptr(si), _ptr(pos), pos.size, block_size, _ptr(out))
    if rc != 0:
        raise ValueError("position beyond the block table")
    return out


def store_kv(pool_layer: np.ndarray, slot_mapping, active_mask, new_k, new_v) -> None:
    """In-place slot-mapped append into ``pool_layer`` [2, P, bs, Hkv, D] fp16."""
    if pool_layer.dtype != np.float16 or not pool_layer.flags.c_contiguous or pool_layer.ndim != 5:
        raise TypeError("pool_layer must be a C-contiguous [2,P,bs,Hkv,D] float16 array")
    _, P, bs, hkv, d = pool_layer.shape
    sm = _c(slot_mapping, np.int32)
    am = None if active_mask is None else _c(np.asarray(active_mask).astype(np.uint8), np.uint8)
    k = _c(new_k, np.float16)
    v = _c(new_v, np.float16)
    lib().orc_store_kv(_ptr(pool_layer), P, _ptr(sm), _ptr(am), _ptr(k), _ptr(v), sm.size, hkv, d, bs)


def paged_attention(q, pool_layer, block_tables, seq_lens, active_mask=None, scale=None,
                    out: np.ndarray | None = None) -> np.ndarray:
    """fp32-accumulation paged attention.

    ``q`` is [B, Hq, D] (decode, one query per sequence at position len-1) or
    [B, Tq, Hq, D] (Tq causal queries ending at position len-1).  Returns fp16
    of the same shape; inactive rows keep ``out``'s prior contents (zeros when
    ``out`` is None).
    """
    q = _c(q, np.float16)
    decode = q.ndim == 3
    q4 = q[:, None] if decode else q
    B, Tq, Hq, D = q4.shape
    pool_layer = _c(pool_layer, np.float16)
    _, P, bs, hkv, d2 = pool_layer.shape
    assert d2 == D and Hq % hkv == 0
    bt = _c(block_tables, np.int32)
    sl = _c(seq_lens, np.int32)
    am = None if active_mask is None else _c(np.asarray(active_mask).astype(np.uint8), np.uint8)
    o = np.zeros(q4.shape, np.float16) if out is None else _c(out, np.float16).reshape(q4.shape).copy()
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    rc = lib().orc_paged_attention(_ptr(o), _ptr(np.ascontiguousarray(q4)), _ptr(pool_layer), P, _ptr(bt),
                                   bt.shape[1], _ptr(sl), _ptr(am), B, Tq, Hq, hkv, D, bs, float(scale))
    if rc != 0:
        raise ValueError(f"oracle rejected inputs (code {rc})")
    return o[:, 0] if decode else o


def host_threads() -> int:
    """Threads for the row-parallel oracle: the cores this process may run on, capped at the
    host's thread budget (OMP_NUM_THREADS when set -- the CPU share of a one-GPU box -- else 16)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    try:
        cap = int(os.environ.get("OMP_NUM_THREADS") or 16)
    except ValueError:
        cap = 16
    return max(1, min(n, cap))


def paged_attention_rows(q, pool_layer, block_tables, seq_lens, active_mask=None, scale=None,
                         threads: int | None = None) -> np.ndarray:
    """``paged_attention`` with its rows split over host threads (the C call releases the GIL).

    Each thread runs the same oracle on a contiguous block of rows, so the result is identical
    to one ``paged_attention`` call on all rows.
    """
    import concurrent.futures as cf
    q = _c(q, np.float16)
    B = q.shape[0]
    n = max(1, min(threads or host_threads(), B))
    bounds = [B * i // n for i in range(n + 1)]
    pool_layer = _c(pool_layer, np.float16)
    bt, sl = _c(block_tables, np.int32), _c(seq_lens, np.int32)
    am = None if active_mask is None else np.asarray(active_mask)

    def run(i):
        lo, hi = bounds[i], bounds[i + 1]
        return paged_attention(q[lo:hi], pool_layer, bt[lo:hi], sl[lo:hi], None if am is None else am[lo:hi], scale)

    with cf.ThreadPoolExecutor(max_workers=n) as ex:
        parts = list(ex.map(run, range(n)))
    return np.concatenate(parts, axis=0)


def qk_norm_rope_append(q, k, v, q_norm_weight, k_norm_weight, rope_table, positions, slot_mapping,
                        active_mask, pool_layer: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """Pre-append step: returns q (fp16 [T, Hq, D]) after RMSNorm + rotary; stores k (normed,
    rotated) and v (cast) into ``pool_layer`` [2, P, bs, Hkv, D] fp16 in place."""
    if pool_layer.dtype != np.float16 or not pool_layer.flags.c_contiguous or pool_layer.ndim != 5:
        raise TypeError("pool_layer must be a C-contiguous [2,P,bs,Hkv,D] float16 array")
    _, P, bs, hkv, d = pool_layer.shape
    qf, kf, vf = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    T, hq, _ = qf.shape
    qw, kw = _c(q_norm_weight, np.float32), _c(k_norm_weight, np.float32)
    rope = _c(rope_table, np.float32)
    pos = _c(positions, np.int32)
    sm = _c(slot_mapping, np.int32)
    am = None if active_mask is None else _c(np.asarray(active_mask).astype(np.uint8), np.uint8)
    out = np.zeros((T, hq, d), np.float16)
    rc = lib().orc_qk_norm_rope_append(_ptr(out), _ptr(pool_layer), P, _ptr(qf), _ptr(kf), _ptr(vf), _ptr(qw),
                                       _ptr(kw), _ptr(rope), rope.shape[0], _ptr(pos), _ptr(sm), _ptr(am), T, hq,
                                       hkv, d, bs, float(eps))
    if rc != 0:
        raise ValueError(f"orc_qk_norm_rope_append failed: {rc}")
    return out
