"""Decode over 32- and 64-token pages (the page-size choice, docs/roadmap.md:327) vs the oracle.

The whole-row decode kernel and its step plan are compiled for pages of 16, 32 and 64 tokens
for the Qwen3 decode shapes (head_dim 128, 8 KV heads, GQA groups 2 and 4).  Each page size is
checked against the oracle (which addresses any page size) at atol 2e-3 / rtol 1e-2; planned
and unplanned calls must agree bit for bit, and the fused append must equal store_kv followed by
the decode, in the pool and in the output.  The same keys in 16-token pages must give the same
attention (paged == contiguous, whatever the page size) within the tolerance.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_attn_close, randn16, say, to_dev
from infurnace_amd.kernels import decode_plan, paged_attention, store_kv, store_kv_and_decode

pytestmark = pytest.mark.gpu


def _tables(rng, lens, bs, extra=5):
    pages = [max(1, -(-int(L) // bs)) for L in lens]
    P = sum(pages) + extra
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((len(lens), max(pages)), np.int32)
    off = 0
    for b, n in enumerate(pages):
        table[b, :n] = perm[off:off + n]
        off += n
    return table, P


@pytest.mark.parametrize("bs", [32, 64])
@pytest.mark.parametrize("hq", [16, 32])
def test_decode_pages_vs_oracle(dev, bs, hq):
    say(f"decode page size {bs} hq={hq}")
    rng = np.random.default_rng(bs * 7 + hq)
    g = torch.Generator(device=dev).manual_seed(bs + hq)
    hkv, d = 8, 128
    lens = np.asarray([1, bs - 1, bs, bs + 1, 3 * bs + 5, 700, 2049, 4096, 63, 1500], np.int32)
    table, P = _tables(rng, lens, bs)
    pool = randn16((2, P, bs, hkv, d), g, dev)
    q = randn16((len(lens), hq, d), g, dev)
    T, L = to_dev(table, dev), to_dev(lens, dev)
    out = paged_attention(q, pool, T, L, None, block_size=bs)
    ref = oracle.paged_attention_rows(q.cpu().numpy(), pool.cpu().numpy(), table, lens)
    assert_attn_close(out, ref, f"page size {bs}")
    plan = decode_plan(q.shape, pool, T, L, block_size=bs)
    out2 = paged_attention(q, pool, T, L, None, block_size=bs, plan=plan)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), "planned differs from unplanned"


@pytest.mark.parametrize("bs", [32, 64])
def test_fused_append_pages(dev, bs):
    say(f"fused append, page size {bs}")
    rng = np.random.default_rng(100 + bs)
    g = torch.Generator(device=dev).manual_seed(100 + bs)
    hq, hkv, d = 16, 8, 128
    lens = np.asarray([5, bs, bs + 1, 999, 3000, 64], np.int32)
    table, P = _tables(rng, lens, bs)
    slots = np.asarray([table[b, (L - 1) // bs] * bs + (L - 1) % bs for b, L in enumerate(lens)], np.int32)
    pool = randn16((2, P, bs, hkv, d), g, dev)
    q = randn16((len(lens), hq, d), g, dev)
    nk, nv = randn16((len(lens), hkv, d), g, dev), randn16((len(lens), hkv, d), g, dev)
    T, L, S = to_dev(table, dev), to_dev(lens, dev), to_dev(slots, dev)
    p1, p2 = pool.clone(), pool.clone()
    store_kv(p1, S, None, nk, nv)
    o1 = paged_attention(q, p1, T, L, None, block_size=bs)
    plan = decode_plan(q.shape, p2, T, L, None, S, block_size=bs)
    o2 = store_kv_and_decode(q, p2, T, L, None, S, nk, nv, block_size=bs, plan=plan)
    assert torch.equal(p1.view(torch.int16), p2.view(torch.int16)), "pools differ"
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), "outputs differ"
    ref = oracle.paged_attention_rows(q.cpu().numpy(), p1.cpu().numpy(), table, lens)
    assert_attn_close(o2, ref, f"fused append page size {bs}")


def test_same_keys_in_16_token_pages(dev):
    """Rows laid out in 32-token pages and the same keys in 16-token pages attend alike."""
    say("page size 32 vs 16, same keys")
    rng = np.random.default_rng(7)
    g = torch.Generator(device=dev).manual_seed(7)
    hq, hkv, d = 16, 8, 128
    lens = np.asarray([33, 500, 1024, 2047], np.int32)
    t32, P32 = _tables(rng, lens, 32)
    pool32 = randn16((2, P32, 32, hkv, d), g, dev)
    pool16 = pool32.reshape(2, P32 * 2, 16, hkv, d)  # page p of 32 tokens = pages 2p, 2p + 1 of 16
    t16 = np.zeros((len(lens), t32.shape[1] * 2), np.int32)
    t16[:, 0::2], t16[:, 1::2] = 2 * t32, 2 * t32 + 1
    q = randn16((len(lens), hq, d), g, dev)
    L = to_dev(lens, dev)
    o32 = paged_attention(q, pool32, to_dev(t32, dev), L, None, block_size=32)
    o16 = paged_attention(q, pool16, to_dev(t16, dev), L, None, block_size=16)
    ref = oracle.paged_attention_rows(q.cpu().numpy(), pool16.cpu().numpy(), t16, lens)
    assert_attn_close(o32, ref, "32-token pages")
    assert_attn_close(o16, ref, "16-token pages")
