"""Fused append + decode (ifn_paged_decode_append) against the two-launch step on the GPU.

The fused launch must leave the same bytes in the pool as store_kv and produce the same
output as store_kv followed by paged decode -- bit for bit, since the appended token's
values are the same fp16 numbers whether read back from the pool or taken from new_k /
new_v, and the arithmetic is the same.  The decode oracle (atol 2e-3 / rtol 1e-2) pins the
result as well.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_attn_close, randn16, say, to_dev
from infurnace_amd import workloads
from infurnace_amd.kernels import paged_attention, store_kv, store_kv_and_decode, store_kv_and_prefill

pytestmark = pytest.mark.gpu


def _case(rng, lens, hq, hkv, d, extra_pages=6):
    """Ragged rows whose last token (position L-1) is the appended one."""
    pages = [max(1, -(-int(L) // 16)) for L in lens]
    P = sum(pages) + extra_pages
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((len(lens), max(pages)), np.int32)
    off = 0
    slots = np.full(len(lens), -1, np.int32)
    for b, n in enumerate(pages):
        table[b, :n] = perm[off:off + n]
        off += n
        if lens[b] > 0:
            pos = int(lens[b]) - 1
            slots[b] = table[b, pos // 16] * 16 + pos % 16
    pool = rng.standard_normal((2, P, 16, hkv, d), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal((len(lens), hq, d), dtype=np.float32).astype(np.float16)
    nk = rng.standard_normal((len(lens), hkv, d), dtype=np.float32).astype(np.float16)
    nv = rng.standard_normal((len(lens), hkv, d), dtype=np.float32).astype(np.float16)
    return pool, table, np.asarray(lens, np.int32), slots, q, nk, nv


def _both(dev, pool, table, lens, slots, q, nk, nv, active=None):
    args = dict(table=to_dev(table, dev), lens=to_dev(lens, dev), slots=to_dev(slots, dev), q=to_dev(q, dev),
                nk=to_dev(nk, dev), nv=to_dev(nv, dev), am=None if active is None else to_dev(active, dev))
    p1, p2 = to_dev(pool, dev), to_dev(pool, dev)
    out1 = torch.full_like(args["q"], 5.0)
    out2 = torch.full_like(args["q"], 5.0)
    store_kv(p1, args["slots"], args["am"], args["nk"], args["nv"])
    paged_attention(args["q"], p1, args["table"], args["lens"], args["am"], out=out1)
    store_kv_and_decode(args["q"], p2, args["table"], args["lens"], args["am"], args["slots"], args["nk"], args["nv"],
                        out=out2)
    return p1, out1, p2, out2


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (8, 8, 128), (64, 8, 128), (16, 8, 64),
                                      (16, 4, 256), (4, 1, 64)])
def test_fused_equals_store_then_decode(dev, hq, hkv, d):
    say(f"fused append hq={hq} hkv={hkv} d={d}")
    rng = np.random.default_rng(hq * 31 + hkv + d)
    lens = [1, 2, 15, 16, 17, 33, 100, 256, 257, 1000, 4096]
    pool, table, lens, slots, q, nk, nv = _case(rng, lens, hq, hkv, d)
    p1, out1, p2, out2 = _both(dev, pool, table, lens, slots, q, nk, nv)
    assert torch.equal(p1.view(torch.int16), p2.view(torch.int16)), "pool differs from store_kv's"
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16)), "output differs from the two-launch step"
    exp_pool = pool.copy()
    oracle.store_kv(exp_pool, slots, None, nk, nv)
    assert_attn_close(out2, oracle.paged_attention(q, exp_pool, table, lens), f"hq={hq} d={d}")


def test_inactive_rows_bad_slots_and_empty_rows(dev):
    """Inactive rows store nothing and write nothing; an out-of-range slot stores nothing; an
    active row with no keys writes zeros -- exactly as store_kv then decode."""
    say("fused append: inactive / bad slot / empty rows")
    rng = np.random.default_rng(41)
    pool, table, lens, slots, q, nk, nv = _case(rng, [70, 300, 45, 90, 128, 5], 16, 8, 128)
    active = np.asarray([1, 0, 1, 1, 1, 0], np.uint8)
    slots[2] = -1                      # active row appending nowhere (its last key is the old pool value)
    slots[3] = pool.shape[1] * 16 + 3  # out of range: skipped
    lens[4] = 0                        # active row with no keys
    p1, out1, p2, out2 = _both(dev, pool, table, lens, slots, q, nk, nv, active)
    assert torch.equal(p1.view(torch.int16), p2.view(torch.int16))
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))
    assert bool((out2[[1, 5]] == 5.0).all()), "inactive rows were written"
    assert bool((out2[4] == 0).all())


def test_config2_full_size_28_layer_step(dev):
    """Config 2 (B=32, L=U[128,4096]) over 4 layers of a full 16384-page pool: bit-identical to
    the two-launch step, layer by layer."""
    say("fused append config2")
    w = workloads.config2()
    g = torch.Generator(device=dev).manual_seed(77)
    L = 4
    pool1 = randn16((L, 2, w.num_pages, 16, 8, 128), g, dev)
    pool2 = pool1.clone()
    bt, sl = to_dev(w.block_tables, dev), to_dev(w.seq_lens, dev)
    slots = to_dev(w.append_slots, dev)
    for layer in range(L):
        q = randn16((w.batch, 16, 128), g, dev)
        nk = randn16((w.batch, 8, 128), g, dev)
        nv = randn16((w.batch, 8, 128), g, dev)
        store_kv(pool1, slots, None, nk, nv, layer=layer)
        o1 = paged_attention(q, pool1, bt, sl, None, layer=layer)
        o2 = store_kv_and_decode(q, pool2, bt, sl, None, slots, nk, nv, layer=layer)
        assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), f"layer {layer}"
    assert torch.equal(pool1.view(torch.int16), pool2.view(torch.int16))


def _prefill_both(dev, pool, table, qs, q, nk, nv):
    T = q.shape[0]
    p1, p2 = to_dev(pool, dev), to_dev(pool, dev)
    tb = to_dev(table, dev)
    pos = np.arange(qs, qs + T)
    slots = (table[pos // 16].astype(np.int64) * 16 + pos % 16)
    slots = np.where((table[pos // 16] >= 0) & (table[pos // 16] < pool.shape[1]), slots, -1).astype(np.int32)
    qd, kd, vd = to_dev(q, dev), to_dev(nk, dev), to_dev(nv, dev)
    store_kv(p1, to_dev(slots, dev), None, kd, vd)
    o1 = paged_attention(qd, p1, tb, None, None, query_start=qs)
    o2 = store_kv_and_prefill(qd, p2, tb, kd, vd, query_start=qs)
    return p1, o1, p2, o2, slots


@pytest.mark.parametrize("qs,T", [(0, 512), (512, 512), (1536, 512), (0, 37), (64, 100), (96, 200), (2016, 33),
                                  (16, 50), (40, 90)])
@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (8, 8, 128), (16, 8, 64)])
def test_fused_prefill_equals_store_then_prefill(dev, qs, T, hq, hkv, d):
    """Aligned starts (one launch) and unaligned ones (two launches); chunk ends inside a tile."""
    say(f"fused prefill qs={qs} T={T} hq={hq} hkv={hkv} d={d}")
    rng = np.random.default_rng(qs * 7 + T + hq + d)
    pages = -(-(qs + T) // 16)
    P = pages + 9
    table = rng.permutation(P)[:pages].astype(np.int32)
    pool = rng.standard_normal((2, P, 16, hkv, d), dtype=np.float32).astype(np.float16)
    f = lambda *s: rng.standard_normal(s, dtype=np.float32).astype(np.float16)
    q, nk, nv = f(T, hq, d), f(T, hkv, d), f(T, hkv, d)
    p1, o1, p2, o2, slots = _prefill_both(dev, pool, table, qs, q, nk, nv)
    assert torch.equal(p1.view(torch.int16), p2.view(torch.int16)), "pool differs from store_kv's"
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), "output differs from the two-launch chunk"
    exp_pool = pool.copy()
    oracle.store_kv(exp_pool, slots, None, nk, nv)
    lens = np.asarray([qs + T], np.int32)
    assert_attn_close(o2, oracle.paged_attention(q[None], exp_pool, table[None], lens)[0], f"qs={qs} T={T}")


def test_fused_prefill_bad_chunk_page(dev):
    """A chunk page id outside the pool: nothing stored there, its keys contribute nothing -- as
    store_kv (slot skipped) then prefill (page masked)."""
    say("fused prefill bad chunk page")
    rng = np.random.default_rng(51)
    qs, T, hq, hkv, d = 64, 96, 16, 8, 128
    pages = (qs + T) // 16
    P = pages + 4
    table = rng.permutation(P)[:pages].astype(np.int32)
    table[6] = P + 100  # a chunk page (keys 96..111)
    pool = rng.standard_normal((2, P, 16, hkv, d), dtype=np.float32).astype(np.float16)
    f = lambda *s: rng.standard_normal(s, dtype=np.float32).astype(np.float16)
    q, nk, nv = f(T, hq, d), f(T, hkv, d), f(T, hkv, d)
    p1, o1, p2, o2, _ = _prefill_both(dev, pool, table, qs, q, nk, nv)
    assert torch.equal(p1.view(torch.int16), p2.view(torch.int16))
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))


def test_fused_prefill_config3_chunks(dev):
    """Config 3: four 512-token chunks of a 2048-token prompt, fused, vs the two-launch chunks."""
    say("fused prefill config3")
    w = workloads.config3()
    g = torch.Generator(device=dev).manual_seed(33)
    pool1 = randn16((2, w.num_pages, 16, 8, 128), g, dev)
    pool2 = pool1.clone()
    tb = to_dev(w.block_table, dev)
    for c in range(4):
        qs = c * w.chunk
        q = randn16((w.chunk, 16, 128), g, dev)
        nk = randn16((w.chunk, 8, 128), g, dev)
        nv = randn16((w.chunk, 8, 128), g, dev)
        pos = np.arange(qs, qs + w.chunk)
        slots = to_dev((w.block_table[pos // 16].astype(np.int64) * 16 + pos % 16).astype(np.int32), dev)
        store_kv(pool1, slots, None, nk, nv)
        o1 = paged_attention(q, pool1, tb, None, None, query_start=qs)
        o2 = store_kv_and_prefill(q, pool2, tb, nk, nv, query_start=qs)
        assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), f"chunk {c}"
    assert torch.equal(pool1.view(torch.int16), pool2.view(torch.int16))
