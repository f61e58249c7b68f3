"""Fused pre-append + decode (ifn_paged_decode_prep_append) against the two-launch step on the GPU.

One launch takes the step's fp32 projections through the q/k RMSNorm, the rotary embedding,
the fp16 cast and the slot append, then attends.  It must leave the same bytes in the pool as
``qk_norm_rope_append`` and produce the same output as ``qk_norm_rope_append`` followed by the
paged decode -- bit for bit, since both kernels round every norm / rotary operation alike and
the attention reads the same fp16 numbers.  The two-launch path is itself pinned against the
oracle (tests/test_kv_prep_gpu.py, tests/test_paged_decode_gpu.py); one case here also checks
the fused result against the oracle directly (atol 2e-3 / rtol 1e-2).
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_attn_close, compact_for_oracle, say, to_dev
from infurnace_amd import workloads
from infurnace_amd.kernels import (decode_plan, paged_attention, qk_norm_rope_append, qk_norm_rope_store_and_decode,
                                   rope_table)

pytestmark = pytest.mark.gpu

MAX_POS = 8192


def _case(rng, lens, hq, hkv, d, extra_pages=6):
    """Ragged rows whose appended token is their last (position L - 1), fp32 projections."""
    pages = [max(1, -(-int(L) // 16)) for L in lens]
    P = sum(pages) + extra_pages
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((len(lens), max(pages)), np.int32)
    off = 0
    slots = np.full(len(lens), -1, np.int32)
    pos = np.zeros(len(lens), np.int32)
    for b, n in enumerate(pages):
        table[b, :n] = perm[off:off + n]
        off += n
        if lens[b] > 0:
            pos[b] = int(lens[b]) - 1
            slots[b] = table[b, pos[b] // 16] * 16 + pos[b] % 16
    pool = rng.standard_normal((2, P, 16, hkv, d), dtype=np.float32).astype(np.float16)
    q = (rng.standard_normal((len(lens), hq, d)) * 2).astype(np.float32)
    k = rng.standard_normal((len(lens), hkv, d)).astype(np.float32)
    v = rng.standard_normal((len(lens), hkv, d)).astype(np.float32)
    qw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    return dict(pool=pool, table=table, lens=np.asarray(lens, np.int32), slots=slots, pos=pos, q=q, k=k, v=v,
                qw=qw, kw=kw)


def _both(dev, c, active=None, planned=False):
    """(pool, out) of the two launches and of the fused launch, from the same inputs."""
    t = {n: to_dev(c[n], dev) for n in ("table", "lens", "slots", "pos", "q", "k", "v", "qw", "kw")}
    am = None if active is None else to_dev(active, dev)
    rope = rope_table(MAX_POS, c["q"].shape[2], 1e6, device=dev)
    if isinstance(c["pool"], torch.Tensor):
        p1, p2 = c["pool"], c["pool"].clone()
    else:
        p1, p2 = to_dev(c["pool"], dev), to_dev(c["pool"], dev)
    out1 = torch.full(c["q"].shape, 5.0, dtype=torch.float16, device=dev)
    out2 = torch.full_like(out1, 5.0)
    plan = decode_plan(c["q"].shape, p2, t["table"], t["lens"], am, t["slots"]) if planned else None
    q16 = qk_norm_rope_append(t["q"], t["k"], t["v"], t["qw"], t["kw"], rope, t["pos"], t["slots"], am, p1)
    paged_attention(q16, p1, t["table"], t["lens"], am, out=out1)
    qk_norm_rope_store_and_decode(t["q"], t["k"], t["v"], t["qw"], t["kw"], rope, t["pos"], t["slots"], am, p2,
                                  t["table"], t["lens"], out=out2, plan=plan)
    torch.cuda.synchronize()
    return p1, out1, p2, out2, q16


def _assert_same(p1, out1, p2, out2, what):
    assert torch.equal(p1.view(torch.int16), p2.view(torch.int16)), f"{what}: pools differ"
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16)), f"{what}: outputs differ"


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (8, 8, 128), (16, 16, 64), (32, 16, 64)])
@pytest.mark.parametrize("planned", [False, True])
def test_fused_prep_equals_two_launches(dev, hq, hkv, d, planned):
    say(f"fused prep+decode hq={hq} hkv={hkv} d={d} planned={planned}")
    rng = np.random.default_rng(hq * 131 + hkv * 7 + d + planned)
    lens = [1, 2, 15, 16, 17, 33, 100, 256, 257, 1000, 4096]
    c = _case(rng, lens, hq, hkv, d)
    _assert_same(*_both(dev, c, planned=planned)[:4], f"hq={hq} hkv={hkv} d={d}")


def test_fused_prep_edge_rows(dev):
    """Inactive rows, a position outside the rotary table (zero query, nothing stored), a slot
    outside the pool (nothing stored, the pool row is attended), rows without keys, and an
    appended token that is not the row's last."""
    say("fused prep+decode edge rows")
    rng = np.random.default_rng(5)
    lens = [0, 5, 40, 64, 300, 17, 1, 96]
    c = _case(rng, lens, 16, 8, 128)
    active = np.array([1, 1, 0, 1, 1, 1, 1, 1], np.uint8)
    c["pos"][3] = MAX_POS + 3                                 # outside the table
    c["slots"][4] = c["pool"].shape[1] * 16 + 7              # outside the pool
    c["pos"][7], c["slots"][7] = 40, c["table"][7, 2] * 16 + 8   # appended at 40 of 96 keys
    for planned in (False, True):
        p1, o1, p2, o2, _ = _both(dev, c, active=active, planned=planned)
        _assert_same(p1, o1, p2, o2, f"edge rows planned={planned}")
        assert torch.equal(o2[2], torch.full_like(o2[2], 5.0)), "an inactive row was written"


def test_fused_prep_config2_full_size(dev):
    """Config 2 (B=32, ragged contexts up to 4096, 16384 pages) at full size, planned as the runner
    calls it; every row against the oracle's own pipeline.  The oracle copies the pages the rows
    read before the launch, runs its own pre-append (orc_qk_norm_rope_append) from the fp32
    projections into that copy at the rows' slots, then its attention: nothing it reads comes
    from the GPU's pre-append.  The appended K rows must match the oracle's within one fp16 ulp
    and the V rows bit for bit."""
    say("fused prep+decode config 2")
    w = workloads.config2()
    rng = np.random.default_rng(2)
    B, hq, hkv, d = w.batch, 16, 8, 128
    gen = torch.Generator(device=dev)
    gen.manual_seed(2)
    pool = torch.randn((2, w.num_pages, 16, hkv, d), generator=gen, device=dev, dtype=torch.float32).half()
    c = dict(pool=pool, table=w.block_tables, lens=w.seq_lens.astype(np.int32), slots=w.append_slots,
             pos=(w.seq_lens - 1).astype(np.int32),
             q=rng.standard_normal((B, hq, d)).astype(np.float32),
             k=rng.standard_normal((B, hkv, d)).astype(np.float32),
             v=rng.standard_normal((B, hkv, d)).astype(np.float32),
             qw=(1 + 0.1 * rng.standard_normal(d)).astype(np.float32),
             kw=(1 + 0.1 * rng.standard_normal(d)).astype(np.float32))
    lens = c["lens"]
    sub, t2 = compact_for_oracle(pool, w.block_tables, lens)  # before the launches append into `pool`
    p1, o1, p2, o2, q16 = _both(dev, c, planned=True)
    _assert_same(p1, o1, p2, o2, "config 2")
    pos = c["pos"]
    slots_sub = np.asarray([t2[b, pos[b] // 16] * 16 + pos[b] % 16 for b in range(B)], np.int32)
    rope = rope_table(MAX_POS, d, 1e6).numpy()
    q16_orc = oracle.qk_norm_rope_append(c["q"], c["k"], c["v"], c["qw"], c["kw"], rope, pos, slots_sub, None, sub)
    ref = oracle.paged_attention_rows(q16_orc, sub, t2, lens)
    assert_attn_close(o2, ref, "config 2 fused prep vs the oracle pipeline")
    got_k = p2[0].reshape(-1, hkv, d)[torch.as_tensor(w.append_slots.astype(np.int64), device=dev)].cpu().numpy()
    got_v = p2[1].reshape(-1, hkv, d)[torch.as_tensor(w.append_slots.astype(np.int64), device=dev)].cpu().numpy()
    exp_k = sub[0].reshape(-1, hkv, d)[slots_sub]
    exp_v = sub[1].reshape(-1, hkv, d)[slots_sub]
    assert np.array_equal(got_v.view(np.uint16), exp_v.view(np.uint16)), "appended V rows differ from the oracle"
    ulps = np.abs(got_k.view(np.uint16).astype(np.int32) - exp_k.view(np.uint16).astype(np.int32))
    assert int(ulps.max()) <= 1, "appended K rows differ from the oracle by more than one fp16 ulp"


def test_fused_prep_unsupported_shape_runs_two_launches(dev):
    """head_dim 256 is outside the fused kernel; the wrapper runs the two launches (same result)."""
    say("fused prep+decode d=256 (two launches)")
    rng = np.random.default_rng(9)
    c = _case(rng, [3, 40, 200], 8, 4, 256)
    _assert_same(*_both(dev, c)[:4], "d=256")
