"""Golden fixtures (tests/golden/, written by tests/golden/make_golden.py from the pinned oracle).

CPU: the seeded generators and the oracle still reproduce the fixtures bit for bit.
GPU: the HIP kernels match them (store_kv bit-exact, attention atol 2e-3 / rtol 1e-2).
"""
import os

import numpy as np
import pytest
import torch

import oracle
from infurnace_amd import workloads

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(HERE, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _digest(*arrays):
    import hashlib
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def test_config1_fixture_reproduces_on_cpu():
    g = load("config1.npz")
    c = workloads.config1()
    assert _digest(c["pool"], c["block_tables"], c["q"], c["new_k"], c["new_v"]) == str(g["inputs_sha256"])
    assert np.array_equal(c["slot_mapping"], g["slot_mapping"])
    pool = c["pool"].copy()
    oracle.store_kv(pool, c["slot_mapping"], None, c["new_k"], c["new_v"])
    assert _digest(pool) == str(g["pool_after_sha256"])
    out = oracle.paged_attention(c["q"], pool, c["block_tables"], c["seq_lens"])
    assert np.array_equal(out.view(np.uint16), g["out"].view(np.uint16))


def test_tiny_fixture_reproduces_on_cpu():
    g = load("tiny.npz")
    after = g["pool"].copy()
    oracle.store_kv(after, g["slot_mapping"], None, g["new_k"], g["new_v"])
    assert np.array_equal(after.view(np.uint16), g["pool_after"].view(np.uint16))
    dec = oracle.paged_attention(g["q"], after, g["block_tables"], g["seq_lens"])
    assert np.array_equal(dec.view(np.uint16), g["decode_out"].view(np.uint16))
    pre = oracle.paged_attention(g["prefill_q"][None], after, g["block_tables"][1:], g["seq_lens"][1:])[0]
    assert np.array_equal(pre.view(np.uint16), g["prefill_out"].view(np.uint16))


@pytest.mark.gpu
def test_kernels_match_golden_fixtures(dev):
    from gpu_util import assert_attn_close, say, to_dev
    from infurnace_amd.kernels import paged_attention, store_kv
    say("golden fixtures on GPU")
    g = load("tiny.npz")
    pool = to_dev(g["pool"], dev)
    store_kv(pool, to_dev(g["slot_mapping"], dev), None, to_dev(g["new_k"], dev), to_dev(g["new_v"], dev))
    torch.cuda.synchronize()
    assert np.array_equal(pool.cpu().numpy().view(np.uint16), g["pool_after"].view(np.uint16))
    out = paged_attention(to_dev(g["q"], dev), pool, to_dev(g["block_tables"], dev), to_dev(g["seq_lens"], dev),
                          None)
    assert_attn_close(out, g["decode_out"], "golden decode")
    pre = paged_attention(to_dev(g["prefill_q"], dev), pool, to_dev(g["block_tables"][1], dev), None, None,
                          query_start=int(g["prefill_start"]))
    assert_attn_close(pre, g["prefill_out"], "golden prefill")
    c = load("config1.npz")
    cw = workloads.config1()
    p1 = to_dev(cw["pool"], dev)
    store_kv(p1, to_dev(cw["slot_mapping"], dev), None, to_dev(cw["new_k"], dev), to_dev(cw["new_v"], dev))
    o1 = paged_attention(to_dev(cw["q"], dev), p1, to_dev(cw["block_tables"], dev), to_dev(cw["seq_lens"], dev), None)
    assert_attn_close(o1, c["out"], "golden config1")
