"""store_kv: slot-mapped KV append into the paged pool (HIP, gfx950).

Mirrors the reference's documented operation
``store_kv(kv_pool, slot_mapping, active_mask, new_k, new_v)``
(docs/architecture.md:242-253; the module src/infurnace/kernels/kv_store.py is
a 0-byte placeholder).  It replaces the contiguous per-layer store of
src/infurnace/executor/tinygrad/model.py:191-196 (decode) and :134-138
(prefill): new K/V rows land at ``pool[layer, 0|1, slot // bs, slot % bs]``
instead of ``kv[layer, 0|1, slot, position]``.

Semantics (bit-exact copy):
  * token t writes iff ``active_mask[t]`` (when given) and
    ``0 <= slot_mapping[t] < num_pages * block_size``;
  * inactive rows write nothing at all -- never a shared dummy location
    (docs/architecture.md:250-253);
  * the launch is asynchronous on the current HIP stream, so a following
    ``paged_attention`` on the same stream reads the stored rows
    (write-before-read, docs/architecture.md:249-250).
"""
from __future__ import annotations

import torch

from .. import _capi
from ._common import KVStoreError, check_pool, current_stream, ptr
from ._carrier import accepts_carriers

__all__ = ["store_kv", "store_kv_layers", "KVStoreError"]


def _check_rows(name: str, t: torch.Tensor, lead: tuple, hkv: int, d: int, device) -> None:
    if not isinstance(t, torch.Tensor):
        raise KVStoreError(f"{name} must be a torch.Tensor")
    if t.dtype != torch.float16:
        raise KVStoreError(f"{name} dtype must be float16, got {t.dtype}")
    if tuple(t.shape) != (*lead, hkv, d):
        raise KVStoreError(f"{name} shape must be {(*lead, hkv, d)}, got {tuple(t.shape)}")
    if t.device != device:
        raise KVStoreError(f"{name} must be on {device}, got {t.device}")
    if not t.is_contiguous():
        raise KVStoreError(f"{name} must be contiguous")


def _check_index(name: str, t, n: int, device, dtypes) -> torch.Tensor | None:
    if t is None:
        return None
    if not isinstance(t, torch.Tensor):
        raise KVStoreError(f"{name} must be a torch.Tensor or None")
    if t.dtype not in dtypes:
        raise KVStoreError(f"{name} dtype must be one of {dtypes}, got {t.dtype}")
    if tuple(t.shape) != (n,):
        raise KVStoreError(f"{name} shape must be ({n},), got {tuple(t.shape)}")
    if t.device != device:
        raise KVStoreError(f"{name} must be on {device}, got {t.device}")
    if not t.is_contiguous():
        raise KVStoreError(f"{name} must be contiguous")
    return t


def _debug_validate(slot_mapping: torch.Tensor, active_mask, num_slots: int) -> None:
    """Host-side check (synchronises): active slots in range and pairwise distinct."""
    slots = slot_mapping.detach().cpu().long()
    act = torch.ones_like(slots, dtype=torch.bool) if active_mask is None else active_mask.detach().cpu().bool()
    live = slots[act]
    if live.numel() and (int(live.min()) < 0 or int(live.max()) >= num_slots):
        raise KVStoreError(f"active slot outside [0, {num_slots})")
    if live.numel() != torch.unique(live).numel():
        raise KVStoreError("two active rows map to the same slot")


@accepts_carriers
def store_kv(kv_pool: torch.Tensor, slot_mapping: torch.Tensor, active_mask: torch.Tensor | None,
             new_k: torch.Tensor, new_v: torch.Tensor, *, layer: int = 0, validate: bool = False) -> None:
    """Append ``new_k``/``new_v`` [T, Hkv, D] fp16 into ``kv_pool`` in place.

    ``kv_pool`` is the full pool [layers, 2, pages, block_size, Hkv, D] (``layer``
    selects one) or one layer's [2, pages, block_size, Hkv, D].  ``slot_mapping``
    is int32 [T]; ``active_mask`` is bool/uint8 [T] or None.  ``validate=True``
    adds a synchronising host check for out-of-range and duplicate active slots.
    """
    pool_layer, (P, bs, hkv, d) = check_pool(kv_pool, layer, KVStoreError)
    dev = pool_layer.device
    if not isinstance(new_k, torch.Tensor) or new_k.ndim != 3:
        raise KVStoreError("new_k must be a rank-3 [T, Hkv, D] tensor")
    T = new_k.shape[0]
    _check_rows("new_k", new_k, (T,), hkv, d, dev)
    _check_rows("new_v", new_v, (T,), hkv, d, dev)
    sm = _check_index("slot_mapping", slot_mapping, T, dev, (torch.int32,))
    am = _check_index("active_mask", active_mask, T, dev, (torch.bool, torch.uint8))
    if validate:
        _debug_validate(sm, am, P * bs)
    if T == 0:
        return
    _capi.call("ifn_store_kv", ptr(pool_layer), P, ptr(sm), ptr(am), ptr(new_k), ptr(new_v),
               T, hkv, d, bs, current_stream(dev))


@accepts_carriers
def store_kv_layers(kv_pool: torch.Tensor, slot_mapping: torch.Tensor, active_mask: torch.Tensor | None,
                    new_k: torch.Tensor, new_v: torch.Tensor, *, validate: bool = False) -> None:
    """Append one token batch into every layer with a single launch.

    ``kv_pool`` [L, 2, P, bs, Hkv, D]; ``new_k``/``new_v`` [L, T, Hkv, D]; the slot
    mapping and mask are shared by all layers.  Equivalent to ``store_kv`` once
    per layer (the layer loop of model.py:98 with the store of :134-138).
    """
    if not isinstance(kv_pool, torch.Tensor) or kv_pool.ndim != 6:
        raise KVStoreError("kv_pool must be the rank-6 [layers, 2, pages, block_size, Hkv, D] pool")
    check_pool(kv_pool, 0, KVStoreError)
    L, _, P, bs, hkv, d = kv_pool.shape
    dev = kv_pool.device
    if not isinstance(new_k, torch.Tensor) or new_k.ndim != 4:
        raise KVStoreError("new_k must be a rank-4 [L, T, Hkv, D] tensor")
    T = new_k.shape[1]
    _check_rows("new_k", new_k, (L, T), hkv, d, dev)
    _check_rows("new_v", new_v, (L, T), hkv, d, dev)
    sm = _check_index("slot_mapping", slot_mapping, T, dev, (torch.int32,))
    am = _check_index("active_mask", active_mask, T, dev, (torch.bool, torch.uint8))
    if validate:
        _debug_validate(sm, am, P * bs)
    if T == 0:
        return
    _capi.call("ifn_store_kv_layers", ptr(kv_pool), L, P, ptr(sm), ptr(am), ptr(new_k), ptr(new_v),
               T, hkv, d, bs, current_stream(dev))
