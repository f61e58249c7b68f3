"""Paged decode attention on the GPU vs the fp32-accumulation oracle.

Tolerance atol 2e-3 / rtol 1e-2 in fp16 (the reference's own tiny-model
tolerance, tests/test_runner.py:77-81,194).  Cases follow the Phase 5C gate
(docs/roadmap.md:346-354): page boundaries, partial pages, GQA head mappings,
independence of physical page assignment -- plus the measured configurations
at full size.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_attn_close, oracle_decode, randn16, say, to_dev
from infurnace_amd import workloads
from infurnace_amd.kernels import paged_attention, store_kv

pytestmark = pytest.mark.gpu


def _ragged(rng, lens, hq, hkv, d, extra_pages=5):
    pages = [-(-int(L) // 16) for L in lens]
    P = sum(pages) + extra_pages
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((len(lens), max(pages)), np.int32)
    off = 0
    for b, n in enumerate(pages):
        table[b, :n] = perm[off:off + n]
        off += n
    pool = rng.standard_normal((2, P, 16, hkv, d), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal((len(lens), hq, d), dtype=np.float32).astype(np.float16)
    return pool, table, np.asarray(lens, np.int32), q


def test_config1_append_then_decode(dev):
    say("decode config1")
    c = workloads.config1()
    pool = to_dev(c["pool"], dev)
    store_kv(pool, to_dev(c["slot_mapping"], dev), None, to_dev(c["new_k"], dev), to_dev(c["new_v"], dev))
    out = paged_attention(to_dev(c["q"], dev), pool, to_dev(c["block_tables"], dev), to_dev(c["seq_lens"], dev),
                          None)
    exp_pool = c["pool"].copy()
    oracle.store_kv(exp_pool, c["slot_mapping"], None, c["new_k"], c["new_v"])
    ref = oracle.paged_attention(c["q"], exp_pool, c["block_tables"], c["seq_lens"])
    assert_attn_close(out, ref, "config1")


EDGE_LENS = [1, 2, 15, 16, 17, 31, 33, 64, 100, 255, 256, 257, 1000, 1024, 4096]


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (8, 8, 128), (64, 8, 128), (16, 8, 64),
                                      (16, 4, 256), (4, 1, 64)])
def test_ragged_edges_and_gqa_groups(dev, hq, hkv, d):
    say(f"decode ragged hq={hq} hkv={hkv} d={d}")
    rng = np.random.default_rng(hq * 1000 + hkv * 10 + d)
    pool, table, lens, q = _ragged(rng, EDGE_LENS, hq, hkv, d)
    out = paged_attention(to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev), None)
    assert_attn_close(out, oracle.paged_attention(q, pool, table, lens), f"hq={hq} hkv={hkv} d={d}")


def test_independent_of_physical_page_assignment(dev):
    """Same logical K/V under two physical layouts -> bit-identical outputs."""
    say("decode page relabel")
    rng = np.random.default_rng(11)
    pool, table, lens, q = _ragged(rng, [300, 4096, 17, 2000], 16, 8, 128)
    perm = rng.permutation(pool.shape[1])
    pool2 = np.empty_like(pool)
    pool2[:, perm] = pool
    table2 = perm[table].astype(np.int32)
    a = paged_attention(to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev), None)
    b = paged_attention(to_dev(q, dev), to_dev(pool2, dev), to_dev(table2, dev), to_dev(lens, dev), None)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_inactive_rows_zero_len_and_bad_pages(dev):
    say("decode inactive/zero/bad-page")
    rng = np.random.default_rng(12)
    pool, table, lens, q = _ragged(rng, [50, 700, 33, 90], 16, 8, 128)
    lens_dev = lens.copy()
    lens_dev[2] = 0
    active = np.asarray([True, False, True, True])
    sentinel = torch.full((4, 16, 128), 7.0, dtype=torch.float16, device=dev)
    out = paged_attention(to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), to_dev(lens_dev, dev),
                          to_dev(active, dev), out=sentinel)
    torch.cuda.synchronize()
    assert torch.all(out[1] == 7.0)          # inactive row: no write
    assert torch.all(out[2] == 0.0)          # active row with no keys: zeros
    ref = oracle.paged_attention(q[[0, 3]], pool, table[[0, 3]], lens[[0, 3]])
    assert_attn_close(out[[0, 3]], ref, "active rows")
    # an out-of-range page id contributes nothing and never faults
    bad = table.copy()
    bad[0, 1] = pool.shape[1] + 1000
    bad[0, 2] = -5
    out2 = paged_attention(to_dev(q, dev), to_dev(pool, dev), to_dev(bad, dev), to_dev(lens, dev), None)
    torch.cuda.synchronize()
    assert_attn_close(out2[1:], oracle.paged_attention(q[1:], pool, table[1:], lens[1:]), "rows with good pages")
    # row 0 attends keys 0..49 with logical pages 1 and 2 (keys 16..47) left out
    keys = [k for k in range(int(lens[0])) if k // 16 not in (1, 2)]
    kk = np.stack([pool[0, table[0, k // 16], k % 16] for k in keys]).astype(np.float64)
    vv = np.stack([pool[1, table[0, k // 16], k % 16] for k in keys]).astype(np.float64)
    ref0 = np.zeros((16, 128))
    for h in range(16):
        sc = kk[:, h // 2] @ q[0, h].astype(np.float64) / np.sqrt(128)
        pr = np.exp(sc - sc.max())
        ref0[h] = (pr[:, None] * vv[:, h // 2]).sum(0) / pr.sum()
    assert_attn_close(out2[0], ref0.astype(np.float32), "row with invalid pages")


def test_workspace_reuse_across_calls_and_batches(dev):
    """Split-KV tickets reset themselves: repeated and differently-shaped calls stay exact."""
    say("decode workspace reuse")
    rng = np.random.default_rng(13)
    pool, table, lens, q = _ragged(rng, [4096, 3000, 1500, 800, 4000], 16, 8, 128)
    args = (to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev))
    qd = to_dev(q, dev)
    first = paged_attention(qd, *args, None).clone()
    for _ in range(3):
        again = paged_attention(qd, *args, None)
        assert torch.equal(first.view(torch.int16), again.view(torch.int16))
    # a smaller batch may be partitioned differently (pages per partition follow the batch
    # size), so it agrees to the tolerance rather than bit for bit
    sub = paged_attention(qd[1:3].contiguous(), args[0], args[1][1:3].contiguous(), args[2][1:3].contiguous(), None)
    ref = oracle.paged_attention(q, pool, table, lens)
    assert_attn_close(sub, ref[1:3], "sub-batch")
    assert_attn_close(first, ref, "workspace reuse")


def test_workspace_shared_across_shapes(dev):
    """One workspace serves decode and prefill calls of alternating shapes (ticket area is fixed)."""
    say("workspace shared across shapes")
    rng = np.random.default_rng(14)
    cases = []
    for lens, hq in [([40, 3000], 16), (list(rng.integers(100, 4096, 40)), 16), ([5000], 32), ([900] * 70, 16)]:
        cases.append((_ragged(rng, lens, hq, 8, 128), hq))
    for rep in range(2):
        for (pool, table, lens, q), hq in cases:
            out = paged_attention(to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev), None)
            assert_attn_close(out, oracle.paged_attention(q, pool, table, lens), f"rep {rep} B={len(lens)}")
            # a prefill call in between uses the same workspace
            t = min(int(lens[0]), 300)
            qp = rng.standard_normal((t, hq, 128), dtype=np.float32).astype(np.float16)
            o2 = paged_attention(to_dev(qp, dev), to_dev(pool, dev), to_dev(table[0], dev), None, None,
                                 query_start=int(lens[0]) - t)
            ref2 = oracle.paged_attention(qp[None], pool, table[:1], lens[:1])[0]
            assert_attn_close(o2, ref2, f"prefill rep {rep}")


def test_config2_full_size_one_layer(dev):
    say("decode config2 full")
    w = workloads.config2()
    g = torch.Generator(device=dev).manual_seed(202)
    pool = randn16((2, w.num_pages, 16, 8, 128), g, dev)
    q = randn16((w.batch, 16, 128), g, dev)
    out = paged_attention(q, pool, to_dev(w.block_tables, dev), to_dev(w.seq_lens, dev), None,
                          max_seq_len=int(w.seq_lens.max()))
    assert_attn_close(out, oracle_decode(pool, w.block_tables, w.seq_lens, q), "config2")


def test_config2_append_then_decode_28_layers(dev):
    """Full step at config 2: per layer store_kv then paged_attention on one stream."""
    say("decode config2 28 layers")
    w = workloads.config2()
    g = torch.Generator(device=dev).manual_seed(2020)
    layers = 3  # parity on 3 of the 28 layers (pool per layer 1 GiB); the bench runs all 28
    pool = randn16((layers, 2, w.num_pages, 16, 8, 128), g, dev)
    slots = to_dev(w.append_slots, dev)
    bt, sl = to_dev(w.block_tables, dev), to_dev(w.seq_lens, dev)
    for layer in range(layers):
        k, v, q = randn16((32, 8, 128), g, dev), randn16((32, 8, 128), g, dev), randn16((32, 16, 128), g, dev)
        store_kv(pool, slots, None, k, v, layer=layer)
        out = paged_attention(q, pool, bt, sl, None, layer=layer)
        torch.cuda.synchronize()
        flat = pool[layer].view(2, -1, 8, 128)
        assert torch.equal(flat[0, slots.long()].view(torch.int16), k.view(torch.int16))
        assert_attn_close(out, oracle_decode(pool[layer], w.block_tables, w.seq_lens, q), f"layer {layer}")


def test_config4_stress_full_size(dev):
    """B=256, L=8192, 131072 pages (8.6 GB pool), 5% x8 tail: every row against the oracle."""
    say("decode config4 full")
    w = workloads.config4()
    g = torch.Generator(device=dev).manual_seed(404)
    pool = randn16((2, w.num_pages, 16, 8, 128), g, dev, w.tail_frac, w.tail_scale)
    q = randn16((w.batch, 16, 128), g, dev, w.tail_frac, w.tail_scale)
    out = paged_attention(q, pool, to_dev(w.block_tables, dev), to_dev(w.seq_lens, dev), None,
                          max_seq_len=8192)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert_attn_close(out, oracle_decode(pool, w.block_tables, w.seq_lens, q), "config4 all rows")
    # every output is a convex combination of V rows: bounded by the row-wise V extremes
    vmax = pool[1].abs().amax().float()
    assert float(out.float().abs().max()) <= float(vmax) * (1 + 1e-3)


def test_config5_prefix_shared_with_churn(dev):
    """Qwen3-8B shapes (G=4), shared 4096-token prefix, 10% suffix pages churned per step."""
    say("decode config5 churn")
    w = workloads.config5()
    g = torch.Generator(device=dev).manual_seed(505)
    pool = randn16((2, w.num_pages, 16, 8, 128), g, dev)
    table = w.block_tables.copy()
    free_ids = list(w.extra["free_ids"])
    for step, churn in enumerate(w.extra["churn"][:2]):
        # free 10% of the suffix pages and reallocate them from the free list, then rewrite their K/V
        old = [int(table[r, c]) for r, c in churn]
        new = free_ids[:len(old)]
        free_ids = free_ids[len(old):] + old
        for (r, c), pid in zip(churn, new):
            table[r, c] = pid
        idx = torch.as_tensor(new, dtype=torch.long, device=dev)
        pool[:, idx] = randn16((2, len(new), 16, 8, 128), g, dev)
        q = randn16((w.batch, 32, 128), g, dev)
        out = paged_attention(q, pool, to_dev(table, dev), to_dev(w.seq_lens, dev), None)
        assert_attn_close(out, oracle_decode(pool, table, w.seq_lens, q), f"config5 step {step}, all rows")


def test_long_context_uses_many_partitions(dev):
    """A 60,000-token row splits into 64 partitions (the merge bound) beside a short row."""
    say("decode long context 60000")
    rng = np.random.default_rng(15)
    pool, table, lens, q = _ragged(rng, [60000, 1000], 16, 8, 128)
    out = paged_attention(to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev), None)
    assert_attn_close(out, oracle.paged_attention(q, pool, table, lens), "long context")
