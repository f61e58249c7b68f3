"""Writes the small golden fixtures of tests/golden/ from the pinned CPU oracle.

The reference holds no vectors for this path (its tools/generate_fixtures.py is a
0-byte placeholder), so these fixtures are regression pins of the oracle, which
tests/test_oracle.py pins against numpy, torch SDPA (float64), brute force and
closed forms.  Run: python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from infurnace_amd import workloads  # noqa: E402


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def config1():
    c = workloads.config1()
    pool = c["pool"].copy()
    oracle.store_kv(pool, c["slot_mapping"], None, c["new_k"], c["new_v"])
    out = oracle.paged_attention(c["q"], pool, c["block_tables"], c["seq_lens"])
    return dict(inputs_sha256=np.asarray(digest(c["pool"], c["block_tables"], c["q"], c["new_k"], c["new_v"])),
                pool_after_sha256=np.asarray(digest(pool)), slot_mapping=c["slot_mapping"],
                block_tables=c["block_tables"], out=out)


def tiny(seed=7):
    rng = np.random.default_rng(seed)
    hq, hkv, d, P = 4, 2, 64, 9
    pool = rng.standard_normal((2, P, 16, hkv, d), dtype=np.float32).astype(np.float16)
    table = rng.permutation(P)[:8].astype(np.int32).reshape(2, 4)
    lens = np.asarray([17, 61], np.int32)
    # append one token per row at position len-1, then decode
    slots = oracle.slot_mapping(table, np.arange(2, dtype=np.int32), lens - 1, 16)
    nk = rng.standard_normal((2, hkv, d), dtype=np.float32).astype(np.float16)
    nv = rng.standard_normal((2, hkv, d), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal((2, hq, d), dtype=np.float32).astype(np.float16)
    after = pool.copy()
    oracle.store_kv(after, slots, None, nk, nv)
    dec = oracle.paged_attention(q, after, table, lens)
    # causal prefill of 13 queries ending at position 60 of row 1
    qp = rng.standard_normal((1, 13, hq, d), dtype=np.float32).astype(np.float16)
    pre = oracle.paged_attention(qp, after, table[1:], lens[1:])
    return dict(pool=pool, block_tables=table, seq_lens=lens, slot_mapping=slots, new_k=nk, new_v=nv, q=q,
                pool_after=after, decode_out=dec, prefill_q=qp[0], prefill_start=np.asarray(61 - 13),
                prefill_out=pre[0])


if __name__ == "__main__":
    np.savez_compressed(os.path.join(HERE, "config1.npz"), **config1())
    np.savez_compressed(os.path.join(HERE, "tiny.npz"), **tiny())
    for f in ("config1.npz", "tiny.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
