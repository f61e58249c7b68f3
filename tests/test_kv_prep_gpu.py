"""Pre-append step (q/k RMSNorm + rotary + fp16 cast + slot append) and the page zero/copy
utilities on the GPU, against the oracle (tests/test_oracle.py pins the oracle).

q and k rows: within one fp16 ulp of the oracle (both round an fp32 result once; the
fp32 sums differ in order); v rows: bit-exact (a plain cast); pages the call does not
address: bit-identical.  Page zero/copy: bit-exact.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_attn_close, say, to_dev
from infurnace_amd.kernels import copy_pages, paged_attention, qk_norm_rope_append, rope_table, zero_pages

pytestmark = pytest.mark.gpu


def _ulps(a16, b16):
    a = a16.astype(np.float64)
    b = b16.astype(np.float64)
    ulp = np.spacing(np.abs(b16)).astype(np.float64)
    return np.abs(a - b) / np.maximum(ulp, 2.0 ** -24)


def _case(rng, T, hq, hkv, d, P=40, bs=16, max_pos=8192):
    q = (rng.standard_normal((T, hq, d)) * 3).astype(np.float32)
    k = rng.standard_normal((T, hkv, d)).astype(np.float32)
    v = rng.standard_normal((T, hkv, d)).astype(np.float32)
    qw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    pos = rng.integers(0, max_pos, T).astype(np.int32)
    slots = rng.permutation(P * bs)[:T].astype(np.int32)
    pool = rng.standard_normal((2, P, bs, hkv, d)).astype(np.float16)
    return q, k, v, qw, kw, pos, slots, pool


@pytest.mark.parametrize("T,hq,hkv,d", [(1, 16, 8, 128), (32, 16, 8, 128), (7, 32, 8, 128), (5, 8, 8, 64),
                                        (3, 4, 1, 256), (512, 16, 8, 128)])
def test_prep_matches_oracle(dev, T, hq, hkv, d):
    say(f"qk_norm_rope_append T={T} hq={hq} hkv={hkv} d={d}")
    rng = np.random.default_rng(T * 7 + d)
    q, k, v, qw, kw, pos, slots, pool = _case(rng, T, hq, hkv, d)
    rope = rope_table(8192, d, 1e6)
    active = (rng.random(T) > 0.2).astype(np.uint8)
    if T > 2:
        slots[1] = pool.shape[1] * 16 + 5   # out of range: stores nothing
        pos[2] = 9000                        # outside the table: zero q row, no store
    ref_pool = pool.copy()
    ref_q = oracle.qk_norm_rope_append(q, k, v, qw, kw, rope.numpy(), pos, slots, active, ref_pool, eps=1e-6)
    P = to_dev(pool, dev)
    out = qk_norm_rope_append(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), to_dev(qw, dev), to_dev(kw, dev),
                              rope.to(dev), to_dev(pos, dev), to_dev(slots, dev), to_dev(active, dev), P, eps=1e-6)
    got_q = out.cpu().numpy()
    got_pool = P.cpu().numpy()
    assert _ulps(got_q, ref_q).max() <= 1.0
    assert _ulps(got_pool[0], ref_pool[0]).max() <= 1.0                      # K: normed + rotated
    assert np.array_equal(got_pool[1].view(np.uint16), ref_pool[1].view(np.uint16))  # V: cast only
    # rows the call must not touch are bit-identical to the input pool
    flat_in = pool.reshape(2, -1, hkv, d).view(np.uint16)
    flat_out = got_pool.reshape(2, -1, hkv, d).view(np.uint16)
    live = {int(s) for t, s in enumerate(slots) if active[t] and 0 <= s < pool.shape[1] * 16 and 0 <= pos[t] < 8192}
    others = np.array([i for i in range(flat_in.shape[1]) if i not in live])
    assert np.array_equal(flat_in[:, others], flat_out[:, others])


def test_prep_then_decode_equals_oracle_pipeline(dev):
    """The fused step feeding paged decode gives the oracle's attention over the oracle's cache."""
    say("qk_norm_rope_append -> paged decode")
    rng = np.random.default_rng(77)
    B, hq, hkv, d, P = 4, 16, 8, 128, 64
    lens = np.array([40, 17, 64, 5], np.int32)
    table = rng.permutation(P)[:16].reshape(4, 4).astype(np.int32)
    pool = rng.standard_normal((2, P, 16, hkv, d)).astype(np.float16)
    q = rng.standard_normal((B, hq, d)).astype(np.float32)
    k = rng.standard_normal((B, hkv, d)).astype(np.float32)
    v = rng.standard_normal((B, hkv, d)).astype(np.float32)
    w = np.ones(d, np.float32)
    pos = (lens - 1).astype(np.int32)
    slots = (table[np.arange(B), pos // 16] * 16 + pos % 16).astype(np.int32)
    rope = rope_table(128, d, 1e6)
    ref_pool = pool.copy()
    ref_q = oracle.qk_norm_rope_append(q, k, v, w, w, rope.numpy(), pos, slots, None, ref_pool)
    ref = oracle.paged_attention(ref_q, ref_pool, table, lens)
    Pd = to_dev(pool, dev)
    qd = qk_norm_rope_append(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), to_dev(w, dev), to_dev(w, dev),
                             rope.to(dev), to_dev(pos, dev), to_dev(slots, dev), None, Pd)
    out = paged_attention(qd, Pd, to_dev(table, dev), to_dev(lens, dev), None)
    assert_attn_close(out, ref, "fused append -> decode")


def test_zero_and_copy_pages_bit_exact(dev):
    say("zero_pages / copy_pages")
    rng = np.random.default_rng(5)
    pool = rng.standard_normal((3, 2, 12, 16, 8, 128)).astype(np.float16)
    P = to_dev(pool, dev)
    zero_pages(P, to_dev(np.array([2, 7, 99, -1], np.int32), dev))
    exp = pool.copy()
    exp[:, :, [2, 7]] = 0
    assert np.array_equal(P.cpu().numpy().view(np.uint16), exp.view(np.uint16))
    copy_pages(P, to_dev(np.array([0, 5, 3], np.int32), dev), to_dev(np.array([9, 11, 2], np.int32), dev))
    exp[:, :, [9, 11, 2]] = exp[:, :, [0, 5, 3]]
    assert np.array_equal(P.cpu().numpy().view(np.uint16), exp.view(np.uint16))
    with pytest.raises(ValueError):
        copy_pages(P, to_dev(np.array([1, 2], np.int32), dev), to_dev(np.array([2, 4], np.int32), dev))


def test_paged_cache_clear_and_copy_use_the_page_kernels(dev):
    say("PagedKVCache.clear_pages / copy_pages")
    from infurnace_amd.cache import PagedKVCache
    cache = PagedKVCache(2, 10, 8, 128, device=dev, zero=False)
    g = torch.Generator(device=dev).manual_seed(3)
    cache.kv.normal_(generator=g)
    before = cache.kv.clone()
    cache.copy_pages([1, 4], [6, 8])
    cache.clear_pages([1, 3])
    exp = before.clone()
    exp[:, :, [6, 8]] = before[:, :, [1, 4]]
    exp[:, :, [1, 3]] = 0
    assert torch.equal(cache.kv.view(torch.int16), exp.view(torch.int16))
