"""Validate mode of the attention wrappers: the inputs the kernels trust are checked on request.

The reference's cache contract keeps block identities "verified, never trusted"
(docs/architecture.md:381-391).  The kernels trust three things for speed: that
``shared_prefix_pages`` heads every long-enough row's table, that a ``DecodePlan``
was built from the current contents of its tensors, and that every table entry a
row reads names a page of the pool.  With ``validate=True`` the wrappers check
all three before the launch and raise ``PagedAttentionError``; a valid call
gives exactly the output of the same call without validation.
"""
import numpy as np
import pytest
import torch

from gpu_util import randn16, say, to_dev
from infurnace_amd.kernels import PagedAttentionError, decode_plan, paged_attention, store_kv_and_decode

pytestmark = pytest.mark.gpu


def _batch(dev, seed=41, B=12, P=600, hkv=8, d=128, hq=16):
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=dev).manual_seed(seed)
    lens = rng.integers(20, 700, size=B).astype(np.int32)
    pages = -(-lens // 16)
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((B, int(pages.max())), np.int32)
    off = 0
    for b in range(B):
        table[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    pool = randn16((2, P, 16, hkv, d), gen, dev)
    q = randn16((B, hq, d), gen, dev)
    return pool, q, to_dev(table, dev), to_dev(lens, dev), table, lens


def test_validated_decode_is_bit_identical(dev):
    say("validate: decode, plain and planned, bit-identical")
    pool, q, T, L, _, _ = _batch(dev)
    ref = paged_attention(q, pool, T, L, None)
    got = paged_attention(q, pool, T, L, None, validate=True)
    assert torch.equal(ref.view(torch.int16), got.view(torch.int16))
    plan = decode_plan(q.shape, pool, T, L)
    got2 = paged_attention(q, pool, T, L, None, plan=plan, validate=True)
    assert torch.equal(ref.view(torch.int16), got2.view(torch.int16))


def test_stale_plan_raises(dev):
    say("validate: a plan whose lengths were rewritten in place")
    pool, q, T, L, _, _ = _batch(dev, seed=42)
    plan = decode_plan(q.shape, pool, T, L)
    L[0] -= 16  # same tensor, new contents: the plan's split no longer matches
    with pytest.raises(PagedAttentionError, match="stale DecodePlan"):
        paged_attention(q, pool, T, L, None, plan=plan, validate=True)
    fresh = decode_plan(q.shape, pool, T, L)
    paged_attention(q, pool, T, L, None, plan=fresh, validate=True)


def test_stale_plan_raises_for_the_fused_append(dev):
    say("validate: store_kv_and_decode with a stale plan")
    pool, q, T, L, table, lens = _batch(dev, seed=43)
    gen = torch.Generator(device=dev).manual_seed(43)
    B, hkv, d = q.shape[0], pool.shape[3], pool.shape[4]
    slots = to_dev(np.asarray([table[b, (lens[b] - 1) // 16] * 16 + (lens[b] - 1) % 16 for b in range(B)], np.int32),
                   dev)
    nk, nv = randn16((B, hkv, d), gen, dev), randn16((B, hkv, d), gen, dev)
    plan = decode_plan(q.shape, pool, T, L, None, slots)
    ok = store_kv_and_decode(q, pool.clone(), T, L, None, slots, nk, nv, plan=plan, validate=True)
    ref = store_kv_and_decode(q, pool.clone(), T, L, None, slots, nk, nv, plan=plan)
    assert torch.equal(ok.view(torch.int16), ref.view(torch.int16))
    L[1] -= 16  # lengths rewritten in place
    with pytest.raises(PagedAttentionError, match="stale DecodePlan"):
        store_kv_and_decode(q, pool, T, L, None, slots, nk, nv, plan=plan, validate=True)


def test_wrong_shared_prefix_declaration_raises(dev):
    say("validate: shared_prefix_pages against the tables")
    rng = np.random.default_rng(44)
    gen = torch.Generator(device=dev).manual_seed(44)
    B, S, P, hkv, d, hq = 6, 8, 400, 8, 128, 16
    perm = rng.permutation(P).astype(np.int32)
    prefix = perm[:S]
    lens = np.asarray([S * 16 + 40 * (b + 1) for b in range(B)], np.int32)
    lens[5] = 50  # a short row: its own table, not the prefix
    pages = -(-lens // 16)
    table = np.zeros((B, int(pages.max())), np.int32)
    off = S
    for b in range(B):
        if b == 5:
            table[b, :pages[b]] = perm[off:off + pages[b]]
            off += pages[b]
            continue
        table[b, :S] = prefix
        table[b, S:pages[b]] = perm[off:off + pages[b] - S]
        off += pages[b] - S
    pool = randn16((2, P, 16, hkv, d), gen, dev)
    q = randn16((B, hq, d), gen, dev)
    T, L, SP = to_dev(table, dev), to_dev(lens, dev), to_dev(prefix, dev)
    ref = paged_attention(q, pool, T, L, None, shared_prefix_pages=SP)
    got = paged_attention(q, pool, T, L, None, shared_prefix_pages=SP, validate=True)
    assert torch.equal(ref.view(torch.int16), got.view(torch.int16))
    wrong = SP.clone()
    wrong[3] = int(perm[-1])
    with pytest.raises(PagedAttentionError, match="shared_prefix_pages"):
        paged_attention(q, pool, T, L, None, shared_prefix_pages=wrong, validate=True)


def test_page_outside_the_pool_raises(dev):
    say("validate: a table entry outside the pool (decode and prefill)")
    pool, q, T, L, table, lens = _batch(dev, seed=45)
    P = pool.shape[1]
    bad = T.clone()
    bad[4, int(lens[4] - 1) // 16] = P  # the row's last used entry
    paged_attention(q, pool, bad, L, None)  # trusted: such a page holds no keys
    with pytest.raises(PagedAttentionError, match="not a page"):
        paged_attention(q, pool, bad, L, None, validate=True)
    bad2 = T.clone()
    bad2[4, int(lens[4] - 1) // 16 + 1:] = -7  # entries past the row's keys are never read
    paged_attention(q, pool, bad2, L, None, validate=True)
    qp = q[:1].expand(64, -1, -1).contiguous()
    tab = T[0].clone()
    paged_attention(qp, pool, tab, None, None, query_start=0, validate=True)
    tab[1] = -1
    with pytest.raises(PagedAttentionError, match="not a page"):
        paged_attention(qp, pool, tab, None, None, query_start=0, validate=True)
