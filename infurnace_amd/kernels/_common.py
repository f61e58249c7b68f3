"""Shared argument checks for the kernel wrappers."""
from __future__ import annotations

import torch


class KVStoreError(ValueError):
    """store_kv inputs do not satisfy the contract (cf. KVCacheError, reference buffers.py:6)."""


class PagedAttentionError(ValueError):
    """paged_attention inputs do not satisfy the contract (cf. Qwen3ModelError, reference model.py:8)."""


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def current_stream(device: torch.device) -> int:
    """hipStream_t of torch's current stream on ``device`` (as an int for ctypes)."""
    return torch.cuda.current_stream(device).cuda_stream


def check_pool(kv_pool, layer: int, err: type[ValueError]):
    """Validate a pool and return (one layer's [2, P, bs, Hkv, D] view, (P, bs, Hkv, D)).

    Layout ``kv_pool[layer, K_or_V, physical_page, page_offset, kv_head, head_dim]``
    (docs/architecture.md:225-232), fp16, contiguous.
    """
    if not isinstance(kv_pool, torch.Tensor):
        raise err("kv_pool must be a torch.Tensor")
    if kv_pool.dtype != torch.float16:
        raise err(f"kv_pool dtype must be float16, got {kv_pool.dtype}")
    if kv_pool.ndim == 6:
        if not 0 <= layer < kv_pool.shape[0]:
            raise err(f"layer {layer} out of range [0, {kv_pool.shape[0]})")
        pool_layer = kv_pool[layer]
    elif kv_pool.ndim == 5:
        if layer != 0:
            raise err("a single-layer [2, P, bs, Hkv, D] pool only has layer 0")
        pool_layer = kv_pool
    else:
        raise err(f"kv_pool must be rank 6 [layers, 2, pages, block_size, Hkv, D] or rank 5, got rank {kv_pool.ndim}")
    if pool_layer.shape[0] != 2:
        raise err(f"kv_pool K_or_V axis must have size 2, got {pool_layer.shape[0]}")
    if not kv_pool.is_contiguous():
        raise err("kv_pool must be contiguous")
    if kv_pool.device.type != "cuda":
        raise err(f"kv_pool must be a GPU tensor, got device {kv_pool.device}")
    _, P, bs, hkv, d = pool_layer.shape
    if P < 1 or bs < 1 or hkv < 1 or d < 1:
        raise err(f"kv_pool has an empty axis: {tuple(kv_pool.shape)}")
    return pool_layer, (P, bs, hkv, d)
