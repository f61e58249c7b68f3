"""Helpers shared by the GPU parity tests (device plumbing + oracle adapters)."""
import sys

import numpy as np
import torch

import oracle

ATOL, RTOL = 2e-3, 1e-2  # fp16 attention tolerance vs the fp32-accumulation oracle


def say(msg: str) -> None:
    """Name the case before a GPU step (flushed, so a fault still shows which case ran)."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def to_dev(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def randn16(shape, gen: torch.Generator, dev, tail_frac: float = 0.0, tail_scale: float = 1.0) -> torch.Tensor:
    x = torch.randn(shape, generator=gen, device=dev, dtype=torch.float32)
    if tail_frac > 0:
        x = torch.where(torch.rand(shape, generator=gen, device=dev) < tail_frac, x * tail_scale, x)
    return x.to(torch.float16)


def compact_for_oracle(pool_layer: torch.Tensor, table: np.ndarray, lens: np.ndarray, bs: int = 16):
    """Copy only the pages the rows reference to host memory; remap the table onto them."""
    used = sorted({int(p) for b in range(table.shape[0]) for p in table[b, :-(-int(lens[b]) // bs)]})
    idx = torch.as_tensor(used, dtype=torch.long, device=pool_layer.device)
    sub = pool_layer.index_select(1, idx).cpu().numpy()
    remap = {p: i for i, p in enumerate(used)}
    t2 = np.zeros_like(table)
    for b in range(table.shape[0]):
        n = -(-int(lens[b]) // bs)
        t2[b, :n] = [remap[int(p)] for p in table[b, :n]]
    return sub, t2


def assert_attn_close(got: torch.Tensor, ref: np.ndarray, what: str = "") -> None:
    g = got.detach().cpu().numpy().astype(np.float64)
    r = ref.astype(np.float64)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    err = np.abs(g - r)
    bound = ATOL + RTOL * np.abs(r)
    bad = err > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} outside atol {ATOL}/rtol {RTOL}; "
                           f"max abs err {err.max():.3g}")


def oracle_decode(pool_layer: torch.Tensor, table: np.ndarray, lens: np.ndarray, q: torch.Tensor,
                  rows=None) -> np.ndarray:
    """The oracle's decode of ``rows`` (all by default), over host threads; only the pages those rows
    read are copied to the host (the whole pool when they read most of it)."""
    rows = np.arange(table.shape[0]) if rows is None else np.asarray(rows)
    qh = q[torch.as_tensor(rows, device=q.device)].cpu().numpy()
    used = -(-lens[rows].astype(np.int64) // 16)
    if int(used.sum()) >= pool_layer.shape[1] // 2:
        return oracle.paged_attention_rows(qh, pool_layer.cpu().numpy(), table[rows], lens[rows].astype(np.int32))
    sub, t2 = compact_for_oracle(pool_layer, table[rows], lens[rows])
    return oracle.paged_attention_rows(qh, sub, t2, lens[rows].astype(np.int32))
