"""Seeded synthetic workloads for the five measured configurations.

The reference defines no inputs for this path (its fixture generator
tools/generate_fixtures.py is a 0-byte placeholder), so the generators here
are the contract: ``numpy.random.default_rng(seed)`` (PCG64) for all host-side
metadata (lengths, page permutations, churn order) and for small tensors;
large pools are filled on the GPU from a seeded ``torch.Generator`` so a 28 GB
pool does not go through host memory.

Shapes are the Qwen3 contracts (reference src/infurnace/models/qwen3.py:15-23:
16 Q heads, 8 KV heads, head_dim 128, 28 layers; Qwen3-8B: 32 Q / 8 KV, 36
layers), fp16, 16-token pages.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

BLOCK = 16


@dataclass
class DecodeWorkload:
    """Host-side description of a batched decode step (one layer's view)."""
    name: str
    num_layers: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    num_pages: int
    seq_lens: np.ndarray            # int32 [B], tokens attended after the append
    block_tables: np.ndarray        # int32 [B, max_pages]
    seed: int
    tail_frac: float = 0.0          # fraction of values scaled by tail_scale
    tail_scale: float = 1.0
    shared_prefix_pages: int = 0    # leading table columns shared by every row
    extra: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return int(self.seq_lens.shape[0])

    @property
    def max_pages(self) -> int:
        return int(self.block_tables.shape[1])

    @property
    def append_slots(self) -> np.ndarray:
        """Slot of each sequence's newest token (position L-1): one append per row per layer."""
        pos = self.seq_lens.astype(np.int64) - 1
        pages = self.block_tables[np.arange(self.batch), pos // BLOCK].astype(np.int64)
        return (pages * BLOCK + pos % BLOCK).astype(np.int32)

    def unique_pages(self) -> int:
        used = set()
        for b in range(self.batch):
            used.update(self.block_tables[b, :-(-int(self.seq_lens[b]) // BLOCK)].tolist())
        return len(used)

    def decode_bytes(self, unique: bool = False) -> int:
        """Algorithmic HBM bytes of one decode launch (one layer).

        K+V once per kv head per token (2*Hkv*D*2 B/token) + Q + O (B*Hq*D*2 B each)
        + block-table entries read (4 B per page used) + sequence lengths (4 B/row).
        With ``unique`` a page shared by several rows is counted once.
        """
        tok_bytes = 2 * self.num_kv_heads * self.head_dim * 2
        pages = -(-self.seq_lens.astype(np.int64) // BLOCK)
        if unique:
            kv = self.unique_pages() * BLOCK * tok_bytes
            # a shared page holds 16 valid tokens; private tails may be partial
            kv -= int(np.sum(pages * BLOCK - self.seq_lens)) * tok_bytes
        else:
            kv = int(np.sum(self.seq_lens.astype(np.int64))) * tok_bytes
        qo = 2 * self.batch * self.num_q_heads * self.head_dim * 2
        return int(kv + qo + 4 * int(np.sum(pages)) + 4 * self.batch)

    def append_bytes(self) -> int:
        """Algorithmic bytes of one append launch: read + write K/V rows + one slot per token."""
        return self.batch * (2 * 2 * self.num_kv_heads * self.head_dim * 2 + 4)


def config1(seed: int = 1) -> dict:
    """Single-layer decode, B=1, context 512, pool of 64 pages (CPU-runnable case).

    Draw order: pool [2,64,16,8,128], block table (first 32 of a permutation of
    64), q [1,16,128], new_k [1,8,128], new_v [1,8,128]; all N(0,1) -> fp16.
    The new token is stored at position 511, then attention reads 512 tokens.
    """
    rng = np.random.default_rng(seed)
    f16 = lambda *s: rng.standard_normal(s, dtype=np.float32).astype(np.float16)
    pool = f16(2, 64, BLOCK, 8, 128)
    table = rng.permutation(64)[:32].astype(np.int32)[None]
    q = f16(1, 16, 128)
    new_k = f16(1, 8, 128)
    new_v = f16(1, 8, 128)
    pos = 511
    slot = np.asarray([int(table[0, pos // BLOCK]) * BLOCK + pos % BLOCK], np.int32)
    return dict(pool=pool, block_tables=table, q=q, new_k=new_k, new_v=new_v,
                seq_lens=np.asarray([512], np.int32), slot_mapping=slot, scale=1.0 / np.sqrt(128.0))


def config2(seed: int = 2) -> DecodeWorkload:
    """Ragged batched decode: B=32, L ~ U[128, 4096], 16384 pages per layer, 28 layers.

    Each sequence takes ceil(L/16) consecutive ids of one seeded permutation of
    the pool (drawn without replacement, so tables are non-contiguous).
    """
    rng = np.random.default_rng(seed)
    lens = rng.integers(128, 4096, endpoint=True, size=32).astype(np.int32)
    perm = rng.permutation(16384).astype(np.int32)
    pages = -(-lens // BLOCK)
    table = np.zeros((32, 4096 // BLOCK), np.int32)
    off = 0
    for b in range(32):
        table[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    return DecodeWorkload("qwen3-0.6b ragged decode B=32 ctx U[128,4096]", 28, 16, 8, 128, 16384,
                          lens, table, seed)


def config4(seed: int = 4) -> DecodeWorkload:
    """Bandwidth stress: B=256, L=8192, 131072 pages per layer, tables = permutation.reshape(256, 512).

    5% of the pool/query values are scaled by 8 (softmax range).
    """
    rng = np.random.default_rng(seed)
    table = rng.permutation(131072).astype(np.int32).reshape(256, 512)
    lens = np.full(256, 8192, np.int32)
    return DecodeWorkload("qwen3-0.6b stress decode B=256 ctx 8192", 1, 16, 8, 128, 131072, lens, table, seed,
                          tail_frac=0.05, tail_scale=8.0)


def config5(seed: int = 5) -> DecodeWorkload:
    """Qwen3-8B shapes (32 Q / 8 KV), 64 sequences sharing a 4096-token prefix + 512 private tokens.

    Pool of 4096 pages per layer: the first 256 ids of a seeded permutation are
    the shared prefix (identical in every table), each row then takes 32
    private pages.  ``extra['churn']`` lists, per step, the (row, column) table
    entries whose pages are freed and reallocated (10% of the suffix pages).
    """
    rng = np.random.default_rng(seed)
    perm = rng.permutation(4096).astype(np.int32)
    prefix = perm[:256]
    table = np.zeros((64, 288), np.int32)
    table[:, :256] = prefix
    table[:, 256:] = perm[256:256 + 64 * 32].reshape(64, 32)
    lens = np.full(64, 4096 + 512, np.int32)
    n_churn = (64 * 32) // 10
    churn = [np.stack(np.unravel_index(rng.permutation(64 * 32)[:n_churn], (64, 32)), 1) for _ in range(4)]
    for c in churn:
        c[:, 1] += 256
    return DecodeWorkload("qwen3-8b prefix-shared decode B=64 ctx 4096+512", 36, 32, 8, 128, 4096, lens, table,
                          seed, shared_prefix_pages=256, extra={"churn": churn, "free_ids": perm[256 + 64 * 32:]})


@dataclass
class PrefillWorkload:
    name: str
    num_layers: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    num_pages: int
    prompt_len: int
    chunk: int
    block_table: np.ndarray  # int32 [max_pages]
    seed: int

    def chunk_flops(self, c: int) -> int:
        """MFMA work of chunk c: 4*Hq*D per (query, visible key) pair (QK^T and PV, multiply+add)."""
        start = c * self.chunk
        visible = sum(start + i + 1 for i in range(self.chunk))
        return 4 * self.num_q_heads * self.head_dim * visible

    def chunk_bytes(self, c: int) -> int:
        """Algorithmic bytes of chunk c's attention: K/V of visible tokens once + Q + O."""
        keys = (c + 1) * self.chunk
        return keys * 2 * self.num_kv_heads * self.head_dim * 2 + 2 * self.chunk * self.num_q_heads * self.head_dim * 2


def config3(seed: int = 3) -> PrefillWorkload:
    """Chunked prefill: 2048-token prompt in four 512-token chunks, 28 layers, 128 pages of a 1024-page pool."""
    rng = np.random.default_rng(seed)
    table = rng.permutation(1024)[:128].astype(np.int32)
    return PrefillWorkload("qwen3-0.6b chunked prefill 2048 = 4x512", 28, 16, 8, 128, 1024, 2048, 512, table, seed)
