"""Fused pre-append + prefill (ifn_paged_prefill_prep_append) against the two-launch chunk on the GPU.

One launch takes a prefill chunk's fp32 projections through the q/k RMSNorm, the rotary embedding,
the fp16 cast and the append at positions query_start + t, then runs the causal attention.  It must
leave the same bytes in the pool as ``qk_norm_rope_append`` (positions query_start + t, the table's
slots) and produce the same output as that followed by ``paged_attention(..., query_start=...)`` --
bit for bit.  The two-launch path is pinned against the oracle elsewhere
(tests/test_kv_prep_gpu.py, tests/test_paged_prefill_gpu.py); one case here also checks the fused
result against the oracle pipeline directly (attention atol 2e-3 / rtol 1e-2, K at most one fp16
value apart or within 1e-6, V bit-exact).
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_attn_close, say, to_dev
from infurnace_amd import _capi
from infurnace_amd.kernels import paged_attention, qk_norm_rope_append, qk_norm_rope_append_and_prefill, rope_table

pytestmark = pytest.mark.gpu

MAX_POS = 20000


def _case(rng, start, T, hq, hkv, d, extra=6, bad_pages=()):
    """One sequence of start + T keys (the first start already in the pool), fp32 projections."""
    pages = -(-(start + T) // 16)
    P = pages + extra
    table = rng.permutation(P)[:pages].astype(np.int32)
    for i, bad in bad_pages:
        table[i] = bad
    pool = rng.standard_normal((2, P, 16, hkv, d), dtype=np.float32).astype(np.float16)
    q = (rng.standard_normal((T, hq, d)) * 2).astype(np.float32)
    k = rng.standard_normal((T, hkv, d)).astype(np.float32)
    v = rng.standard_normal((T, hkv, d)).astype(np.float32)
    qw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    return dict(pool=pool, table=table, q=q, k=k, v=v, qw=qw, kw=kw, start=start)


def _slots(table, start, T):
    pos = np.arange(start, start + T, dtype=np.int64)
    return pos.astype(np.int32), (table[pos // 16].astype(np.int64) * 16 + pos % 16).astype(np.int32)


def _both(dev, c, rope):
    """(pool, out) of the two launches and of the fused launch (called through the C ABI, so the
    fused kernel is the one measured), from the same inputs."""
    t = {n: to_dev(c[n], dev) for n in ("table", "q", "k", "v", "qw", "kw")}
    T, hq, d = c["q"].shape
    hkv = c["k"].shape[1]
    start = c["start"]
    pos, slots = _slots(c["table"], start, T)
    p1, p2 = to_dev(c["pool"], dev), to_dev(c["pool"], dev)
    out1 = torch.full((T, hq, d), 5.0, dtype=torch.float16, device=dev)
    out2 = torch.full_like(out1, 5.0)
    q16 = qk_norm_rope_append(t["q"], t["k"], t["v"], t["qw"], t["kw"], rope, to_dev(pos, dev), to_dev(slots, dev),
                              None, p1)
    paged_attention(q16, p1, t["table"], None, None, query_start=start, out=out1)
    L = _capi.lib()
    P = p2.shape[1]
    nb = L.ifn_paged_prefill_workspace_bytes(T, start, hq, hkv, d, 16)
    ws = torch.zeros(max(nb, 256), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = L.ifn_paged_prefill_prep_append(out2.data_ptr(), t["q"].data_ptr(), t["k"].data_ptr(), t["v"].data_ptr(),
                                         t["qw"].data_ptr(), t["kw"].data_ptr(), rope.data_ptr(), rope.shape[0],
                                         p2.data_ptr(), P, t["table"].data_ptr(), t["table"].shape[0], start, T, hq,
                                         hkv, d, 16, 1e-6, 0.0, ws.data_ptr(), ws.numel(), stream)
    assert rc == 0, _capi.status_string(rc)
    torch.cuda.synchronize()
    return p1, out1, p2, out2


def _steps(a16, b16):
    """Distance in representable fp16 values (0: equal, 1: neighbours, also across a power of two)."""
    def ordinal(x):
        i = x.view(np.int16).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFF), i)
    return np.abs(ordinal(a16) - ordinal(b16))


def _assert_same(p1, out1, p2, out2, what):
    assert torch.equal(p1.view(torch.int16), p2.view(torch.int16)), f"{what}: pools differ"
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16)), f"{what}: outputs differ"


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (8, 8, 128), (64, 8, 128), (16, 8, 64),
                                      (4, 1, 64), (32, 4, 64)])
@pytest.mark.parametrize("start,T", [(0, 1), (0, 37), (0, 512), (32, 100), (96, 33), (512, 512), (1536, 512),
                                     (3008, 40), (4096, 300)])
def test_fused_prefill_prep_equals_two_launches(dev, hq, hkv, d, start, T):
    say(f"fused prep+prefill hq={hq} hkv={hkv} d={d} start={start} T={T}")
    rng = np.random.default_rng(start * 7 + T * 3 + hq + hkv * 5 + d)
    rope = rope_table(MAX_POS, d, 1e6, device=dev)
    _assert_same(*_both(dev, _case(rng, start, T, hq, hkv, d), rope), f"start={start} T={T}")


def test_fused_prefill_prep_invalid_pages(dev):
    """Chunk pages outside the pool (negative, past the end): nothing is written there and their keys
    are not attended, exactly as in the two launches."""
    say("fused prep+prefill invalid pages")
    rng = np.random.default_rng(91)
    c = _case(rng, 64, 200, 16, 8, 128, bad_pages=[(5, -1), (9, 1 << 20)])
    rope = rope_table(MAX_POS, 128, 1e6, device=dev)
    _assert_same(*_both(dev, c, rope), "invalid pages")


def test_fused_prefill_prep_config3_prompt(dev):
    """Config 3 (Qwen3-0.6B, a 2048-token prompt in four 512-token chunks): every chunk of the fused
    path equals the two launches, with the pool carried from chunk to chunk."""
    hq, hkv, d, n = 16, 8, 128, 2048
    rng = np.random.default_rng(3)
    P = n // 16 + 8
    table = to_dev(rng.permutation(P)[:n // 16].astype(np.int32), dev)
    p1 = torch.zeros((2, P, 16, hkv, d), dtype=torch.float16, device=dev)
    p2 = torch.zeros_like(p1)
    rope = rope_table(MAX_POS, d, 1e6, device=dev)
    g = torch.Generator(device=dev).manual_seed(3)
    qw = 1 + 0.1 * torch.randn(d, generator=g, device=dev)
    kw = 1 + 0.1 * torch.randn(d, generator=g, device=dev)
    for start in range(0, n, 512):
        say(f"fused prep+prefill config3 chunk at {start}")
        q = 2 * torch.randn((512, hq, d), generator=g, device=dev)
        k = torch.randn((512, hkv, d), generator=g, device=dev)
        v = torch.randn((512, hkv, d), generator=g, device=dev)
        pos = torch.arange(start, start + 512, dtype=torch.int32, device=dev)
        slots = (table[(pos // 16).long()] * 16 + pos % 16).to(torch.int32)
        q16 = qk_norm_rope_append(q, k, v, qw, kw, rope, pos, slots, None, p1)
        out1 = paged_attention(q16, p1, table, None, None, query_start=start)
        out2 = qk_norm_rope_append_and_prefill(q, k, v, qw, kw, rope, p2, table, query_start=start)
        torch.cuda.synchronize()
        _assert_same(p1, out1, p2, out2, f"chunk at {start}")


def test_fused_prefill_prep_matches_oracle_pipeline(dev):
    """The fused chunk against the oracle's pre-append then the oracle's causal attention over the
    oracle's pool (host copies): K at most one fp16 value apart (the two sum the squares in
    different orders, so the fp32 results can round to neighbouring fp16 values) or within 1e-6
    where the rotation cancels, V bit-exact, the attention within atol 2e-3 / rtol 1e-2."""
    say("fused prep+prefill vs oracle pipeline")
    hq, hkv, d, start, T = 16, 8, 128, 320, 200
    rng = np.random.default_rng(17)
    c = _case(rng, start, T, hq, hkv, d)
    rope = rope_table(MAX_POS, d, 1e6, device=dev)
    pool = to_dev(c["pool"], dev)
    t = {n: to_dev(c[n], dev) for n in ("table", "q", "k", "v", "qw", "kw")}
    out = qk_norm_rope_append_and_prefill(t["q"], t["k"], t["v"], t["qw"], t["kw"], rope, pool, t["table"],
                                          query_start=start)
    torch.cuda.synchronize()
    ref_pool = c["pool"].copy()
    pos, slots = _slots(c["table"], start, T)
    ref_q = oracle.qk_norm_rope_append(c["q"], c["k"], c["v"], c["qw"], c["kw"], rope.cpu().numpy(), pos, slots, None,
                                       ref_pool, eps=1e-6)
    ref = oracle.paged_attention(ref_q[None], ref_pool, c["table"][None], np.asarray([start + T], np.int32))[0]
    assert_attn_close(out, ref, "fused prep+prefill vs oracle")
    got = pool.cpu().numpy()
    # adjacent fp16 values at most -- or within 1e-6 where the rotation's two products nearly cancel
    # (their fp32 roundings, ~6e-8 of O(1) terms, then decide the last bits of a small result)
    near = np.abs(got[0].astype(np.float64) - ref_pool[0].astype(np.float64)) <= 1e-6
    assert ((_steps(got[0], ref_pool[0]) <= 1) | near).all()
    assert np.array_equal(got[1].view(np.uint16), ref_pool[1].view(np.uint16))


def test_unaligned_chunk_runs_two_launches(dev):
    """query_start not a multiple of 32: the C entry point declines (IFN_ERR_UNSUPPORTED) and the
    Python entry runs the two launches, with the same result."""
    say("fused prep+prefill unaligned start")
    hq, hkv, d, start, T = 16, 8, 128, 45, 70
    rng = np.random.default_rng(45)
    c = _case(rng, start, T, hq, hkv, d)
    rope = rope_table(MAX_POS, d, 1e6, device=dev)
    t = {n: to_dev(c[n], dev) for n in ("table", "q", "k", "v", "qw", "kw")}
    L = _capi.lib()
    p0 = to_dev(c["pool"], dev)
    o0 = torch.empty((T, hq, d), dtype=torch.float16, device=dev)
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    rc = L.ifn_paged_prefill_prep_append(o0.data_ptr(), t["q"].data_ptr(), t["k"].data_ptr(), t["v"].data_ptr(),
                                         t["qw"].data_ptr(), t["kw"].data_ptr(), rope.data_ptr(), rope.shape[0],
                                         p0.data_ptr(), p0.shape[1], t["table"].data_ptr(), t["table"].shape[0], start,
                                         T, hq, hkv, d, 16, 1e-6, 0.0, ws.data_ptr(), ws.numel(),
                                         torch.cuda.current_stream(dev).cuda_stream)
    assert rc == _capi.IFN_ERR_UNSUPPORTED
    pos, slots = _slots(c["table"], start, T)
    p1, p2 = to_dev(c["pool"], dev), to_dev(c["pool"], dev)
    q16 = qk_norm_rope_append(t["q"], t["k"], t["v"], t["qw"], t["kw"], rope, to_dev(pos, dev), to_dev(slots, dev),
                              None, p1)
    out1 = paged_attention(q16, p1, t["table"], None, None, query_start=start)
    out2 = qk_norm_rope_append_and_prefill(t["q"], t["k"], t["v"], t["qw"], t["kw"], rope, p2, t["table"],
                                           query_start=start)
    torch.cuda.synchronize()
    _assert_same(p1, out1, p2, out2, "unaligned start")
