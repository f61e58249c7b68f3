"""Causal chunked-prefill paged attention (MFMA) on the GPU vs the oracle.

Semantics: src/infurnace/executor/tinygrad/model.py:116-132 (query i at
start_position + i sees key_pos <= query_pos), append-then-attend as in the
measured configuration.  Tolerance atol 2e-3 / rtol 1e-2 in fp16.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_attn_close, compact_for_oracle, randn16, say, to_dev
from infurnace_amd import workloads
from infurnace_amd.cache import slot_mapping_for_positions
from infurnace_amd.kernels import paged_attention, store_kv

pytestmark = pytest.mark.gpu


def _seq(rng, total, hq, hkv, d, extra=6):
    pages = -(-total // 16)
    P = pages + extra
    table = rng.permutation(P)[:pages].astype(np.int32)
    pool = rng.standard_normal((2, P, 16, hkv, d), dtype=np.float32).astype(np.float16)
    return pool, table


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (8, 8, 128), (64, 8, 128), (16, 8, 64),
                                      (4, 1, 64)])
@pytest.mark.parametrize("start,T", [(0, 1), (0, 37), (0, 128), (45, 38), (100, 300), (512, 512), (17, 1),
                                     (3000, 40), (1500, 100)])
def test_prefill_matches_oracle(dev, hq, hkv, d, start, T):
    say(f"prefill hq={hq} hkv={hkv} d={d} start={start} T={T}")
    rng = np.random.default_rng(start * 1000 + T + hq + d)
    pool, table = _seq(rng, start + T, hq, hkv, d)
    q = rng.standard_normal((T, hq, d), dtype=np.float32).astype(np.float16)
    out = paged_attention(to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), None, None, query_start=start)
    ref = oracle.paged_attention(q[None], pool, table[None], np.asarray([start + T], np.int32))[0]
    assert_attn_close(out, ref, f"start={start} T={T}")


@pytest.mark.parametrize("hq,hkv,d,start,T", [(16, 8, 128, 8192, 512), (16, 8, 64, 4000, 544), (32, 8, 128, 4200, 512),
                                             (16, 8, 128, 16600, 512)])
def test_long_context_rows_match_oracle(dev, hq, hkv, d, start, T):
    """Chunks long enough that each wave runs past 32 tiles (its page-id window is reloaded), in
    both kernel configurations (32-row/8-wave and 64-row/4-wave).  Every row is checked: row r of
    the chunk is the single query at position start + r, i.e. the last row of a sequence of
    start + r + 1 keys, so the chunk is T decode rows over one table, which the oracle runs split
    over the host's threads."""
    say(f"prefill long context hq={hq} hkv={hkv} d={d} start={start} T={T}")
    rng = np.random.default_rng(start + T + d)
    pool, table = _seq(rng, start + T, hq, hkv, d)
    q = rng.standard_normal((T, hq, d), dtype=np.float32).astype(np.float16)
    out = paged_attention(to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), None, None, query_start=start)
    lens = (start + 1 + np.arange(T)).astype(np.int32)
    ref = oracle.paged_attention_rows(q, pool, np.repeat(table[None], T, axis=0), lens)
    assert_attn_close(out, ref, f"start={start} T={T}")


def test_chunked_equals_unchunked_and_decode(dev):
    """Chunked prefill == one-shot prefill (reference tests/test_cached_forward.py:107-117) and the
    last query row == paged decode at that position."""
    say("prefill chunked vs unchunked")
    rng = np.random.default_rng(21)
    total = 700
    pool, table = _seq(rng, total, 16, 8, 128)
    q = rng.standard_normal((total, 16, 128), dtype=np.float32).astype(np.float16)
    P, T = to_dev(pool, dev), to_dev(table, dev)
    Q = to_dev(q, dev)
    full = paged_attention(Q, P, T, None, None, query_start=0)
    parts = [paged_attention(Q[s:e].contiguous(), P, T, None, None, query_start=s)
             for s, e in [(0, 256), (256, 257), (257, 700)]]
    chunked = torch.cat(parts)
    ref = oracle.paged_attention(q[None], pool, table[None], np.asarray([total], np.int32))[0]
    assert_attn_close(full, ref, "one-shot")
    assert_attn_close(chunked, ref, "chunked")
    dec = paged_attention(Q[-1:].contiguous(), P, T[None], torch.tensor([total], dtype=torch.int32, device=dev), None)
    assert_attn_close(dec, ref[-1:], "decode at the last position")


def test_config3_append_then_attend_all_chunks(dev):
    """Config 3 on one layer: four 512-token chunks, each appended with store_kv then attended causally.

    The oracle keeps its own host pool, written by its own store at the host-computed slots, so a
    wrong store or slot on the GPU shows up both as a pool difference and in the attention.
    """
    say("prefill config3")
    w = workloads.config3()
    g = torch.Generator(device=dev).manual_seed(303)
    pool = randn16((2, w.num_pages, 16, 8, 128), g, dev)
    host_pool = pool.cpu().numpy()
    table = to_dev(w.block_table, dev)
    for c in range(4):
        start = c * w.chunk
        k = randn16((w.chunk, 8, 128), g, dev)
        v = randn16((w.chunk, 8, 128), g, dev)
        q = randn16((w.chunk, 16, 128), g, dev)
        host_slots = oracle.slot_mapping(w.block_table[None], np.zeros(w.chunk, np.int32),
                                         np.arange(start, start + w.chunk, dtype=np.int32))
        assert np.array_equal(host_slots, slot_mapping_for_positions(w.block_table, start, w.chunk))
        store_kv(pool, to_dev(host_slots, dev), None, k, v)
        oracle.store_kv(host_pool, host_slots, None, k.cpu().numpy(), v.cpu().numpy())
        out = paged_attention(q, pool, table, None, None, query_start=start)
        total = start + w.chunk
        assert np.array_equal(pool.cpu().numpy().view(np.uint16), host_pool.view(np.uint16)), f"chunk {c}: pool"
        ref = oracle.paged_attention(q.cpu().numpy()[None], host_pool, w.block_table[None],
                                     np.asarray([total], np.int32))[0]
        assert_attn_close(out, ref, f"chunk {c}")


def test_workspace_reuse_and_bad_pages(dev):
    say("prefill workspace reuse / bad pages")
    rng = np.random.default_rng(22)
    pool, table = _seq(rng, 2048, 16, 8, 128)
    q = rng.standard_normal((512, 16, 128), dtype=np.float32).astype(np.float16)
    P, T, Q = to_dev(pool, dev), to_dev(table, dev), to_dev(q, dev)
    a = paged_attention(Q, P, T, None, None, query_start=1536).clone()
    for _ in range(3):
        b = paged_attention(Q, P, T, None, None, query_start=1536)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    bad = table.copy()
    bad[3] = pool.shape[1] + 7
    c = paged_attention(Q, P, to_dev(bad, dev), None, None, query_start=1536)
    torch.cuda.synchronize()
    assert torch.isfinite(c.float()).all()


def _masked_reference(q, pool, table, start, skip_pages):
    """float64 causal attention over keys [0, start + i], leaving out every key of the logical pages in
    skip_pages (the documented meaning of a page id outside [0, num_pages): it contributes no keys)."""
    T, hq, d = q.shape
    hkv = pool.shape[3]
    g = hq // hkv
    total = start + T
    keys = [k for k in range(total) if k // 16 not in skip_pages]
    kk = np.stack([pool[0, table[k // 16], k % 16] for k in keys]).astype(np.float64)  # [n, hkv, d]
    vv = np.stack([pool[1, table[k // 16], k % 16] for k in keys]).astype(np.float64)
    kpos = np.asarray(keys)
    out = np.zeros((T, hq, d))
    for i in range(T):
        vis = kpos <= start + i
        for h in range(hq):
            s = kk[vis, h // g] @ q[i, h].astype(np.float64) / np.sqrt(d)
            p = np.exp(s - s.max())
            out[i, h] = (p[:, None] * vv[vis, h // g]).sum(0) / p.sum()
    return out


def test_invalid_page_contributes_no_keys(dev):
    say("prefill invalid page id -> its keys are skipped")
    rng = np.random.default_rng(31)
    start, T = 40, 30
    pool, table = _seq(rng, start + T, 16, 8, 128)
    q = rng.standard_normal((T, 16, 128), dtype=np.float32).astype(np.float16)
    bad = table.copy()
    bad[2] = pool.shape[1] + 3  # logical page 2 = keys 32..47
    out = paged_attention(to_dev(q, dev), to_dev(pool, dev), to_dev(bad, dev), None, None, query_start=start)
    ref = _masked_reference(q, pool, table, start, {2})
    assert_attn_close(out, ref.astype(np.float32), "invalid page 2")
    # negative ids too
    bad[2] = -1
    out = paged_attention(to_dev(q, dev), to_dev(pool, dev), to_dev(bad, dev), None, None, query_start=start)
    assert_attn_close(out, ref.astype(np.float32), "page id -1")
