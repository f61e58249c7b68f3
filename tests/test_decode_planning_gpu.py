"""A step's first decode builds the step plan (ifn_paged_decode_planning and its append and
pre-append forms, ``decode_plan(..., lazy=True)``).

The call decodes unplanned and writes, as it goes, the words the plan kernel
(``ifn_paged_decode_plan``) writes for the same inputs.  Checked here: its output (and pool,
for the fused forms) equals the unplanned call's bit for bit; the plan it leaves equals the plan
kernel's byte for byte (both buffers start zeroed); and the later layers' planned calls with it
equal the unplanned ones.  Cases cover ragged rows, inactive and empty rows, pages outside the
pool, ranges holding more pieces than a record describes, calls with fewer ranges than
workgroups (short batches), 32-token pages and config 2 at full size.
"""
import numpy as np
import pytest
import torch

from gpu_util import say, to_dev
from infurnace_amd import workloads
from infurnace_amd.kernels import (decode_plan, paged_attention, qk_norm_rope_store_and_decode, rope_table,
                                   store_kv_and_decode)

pytestmark = pytest.mark.gpu


def _case(rng, lens, hq, hkv, d, bs=16, extra_pages=5):
    pages = [max(1, -(-int(L) // bs)) for L in lens]
    P = sum(pages) + extra_pages
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((len(lens), max(pages)), np.int32)
    off = 0
    for b, n in enumerate(pages):
        table[b, :n] = perm[off:off + n]
        off += n
    pool = rng.standard_normal((2, P, bs, hkv, d), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal((len(lens), hq, d), dtype=np.float32).astype(np.float16)
    return pool, table, np.asarray(lens, np.int32), q


def _same(a: torch.Tensor, b: torch.Tensor, what: str):
    assert torch.equal(a.view(torch.int16), b.view(torch.int16)), what


def _check(dev, pool, table, lens, q, active=None, append=False, bs=16, what=""):
    """Unplanned, planning (lazy plan) and then planned calls: outputs and pools bit-equal, and the
    lazily built plan equal to the plan kernel's."""
    qd, bt, sl = to_dev(q, dev), to_dev(table, dev), to_dev(lens, dev)
    act = None if active is None else to_dev(active, dev)
    B, hkv, d = q.shape[0], pool.shape[3], pool.shape[4]
    slots = k = v = None
    if append:
        g = torch.Generator(device=dev).manual_seed(int(lens.sum()) % 1000)
        pos = np.maximum(lens - 1, 0)
        slots = to_dev((table[np.arange(B), pos // bs].astype(np.int64) * bs + pos % bs).astype(np.int32), dev)
        k = torch.randn((B, hkv, d), generator=g, device=dev).half()
        v = torch.randn((B, hkv, d), generator=g, device=dev).half()

    def run(plan):
        p = to_dev(pool, dev)
        out = torch.full(qd.shape, 7.0, dtype=torch.float16, device=dev)
        if append:
            store_kv_and_decode(qd, p, bt, sl, act, slots, k, v, out=out, block_size=bs, plan=plan)
        else:
            paged_attention(qd, p, bt, sl, act, out=out, block_size=bs, plan=plan)
        torch.cuda.synchronize()
        return out, p

    ref_out, ref_pool = run(None)
    eager = decode_plan(qd.shape, to_dev(pool, dev), bt, sl, act, slots, block_size=bs)
    lazy = decode_plan(qd.shape, to_dev(pool, dev), bt, sl, act, slots, block_size=bs, lazy=True)
    assert lazy.pending or lazy.buf is None
    out1, pool1 = run(lazy)  # builds the plan
    assert not lazy.pending
    _same(ref_out, out1, f"{what}: the planning call differs from the unplanned one")
    _same(ref_pool, pool1, f"{what}: the planning call's pool differs")
    if eager.buf is not None:
        torch.cuda.synchronize()
        assert torch.equal(eager.buf, lazy.buf), f"{what}: the plan written differs from the plan kernel's"
    out2, pool2 = run(lazy)  # planned with it
    _same(ref_out, out2, f"{what}: planned with the written plan differs")
    _same(ref_pool, pool2, f"{what}: planned pool differs")


@pytest.mark.parametrize("append", [False, True])
@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (32, 16, 64), (8, 4, 256)])
def test_planning_ragged(dev, hq, hkv, d, append):
    say(f"planning ragged hq={hq} hkv={hkv} d={d} append={append}")
    rng = np.random.default_rng(hq * 7 + d + append)
    lens = [1, 2, 15, 16, 17, 31, 33, 64, 100, 255, 256, 257, 1000, 1024, 4096]
    pool, table, lens, q = _case(rng, lens, hq, hkv, d)
    _check(dev, pool, table, lens, q, append=append, what=f"hq={hq} d={d}")


@pytest.mark.parametrize("append", [False, True])
def test_planning_inactive_empty_and_bad_pages(dev, append):
    say(f"planning inactive/empty/bad pages append={append}")
    rng = np.random.default_rng(77)
    pool, table, lens, q = _case(rng, [50, 700, 33, 90, 0, 300, 1, 2000], 16, 8, 128)
    active = np.asarray([1, 0, 1, 1, 1, 1, 1, 0], np.uint8)
    table[5, 1] = pool.shape[1] + 1000
    table[5, 3] = -7
    _check(dev, pool, table, lens, q, active=active, append=append, what="inactive/empty/bad")


@pytest.mark.parametrize("batch", [3, 700])
def test_planning_short_and_many_rows(dev, batch):
    """3 rows: fewer ranges than workgroups (the rest write empty records); 700 rows of a few keys:
    ranges with more pieces than a record holds."""
    say(f"planning batch={batch}")
    rng = np.random.default_rng(batch)
    lens = rng.integers(1, 40 if batch > 100 else 90, size=batch)
    pool, table, lens, q = _case(rng, lens, 16, 8, 128)
    _check(dev, pool, table, lens, q, what=f"batch {batch}")
    _check(dev, pool, table, lens, q, append=True, what=f"batch {batch} append")


def test_planning_32_token_pages(dev):
    say("planning 32-token pages")
    rng = np.random.default_rng(32)
    pool, table, lens, q = _case(rng, [40, 31, 32, 33, 1000, 2047, 5], 16, 8, 128, bs=32)
    _check(dev, pool, table, lens, q, bs=32, what="32-token pages")
    _check(dev, pool, table, lens, q, append=True, bs=32, what="32-token pages append")


def test_planning_config2_full_size(dev):
    say("planning config 2")
    w = workloads.config2()
    rng = np.random.default_rng(2)
    pool = rng.standard_normal((2, w.num_pages, 16, w.num_kv_heads, w.head_dim), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal((w.batch, w.num_q_heads, w.head_dim), dtype=np.float32).astype(np.float16)
    _check(dev, pool, w.block_tables, w.seq_lens, q, what="config 2")
    _check(dev, pool, w.block_tables, w.seq_lens, q, append=True, what="config 2 append")


def test_planning_pre_append(dev):
    """The pre-append form: a lazy plan built by the first qk_norm_rope_store_and_decode call gives
    the same output and pool as an eager plan, and the same plan bytes."""
    say("planning pre-append")
    rng = np.random.default_rng(5)
    hq, hkv, d = 16, 8, 128
    pool, table, lens, q = _case(rng, [300, 17, 1, 900, 64, 2500], hq, hkv, d)
    B = len(lens)
    g = torch.Generator(device=dev).manual_seed(5)
    qf = torch.randn((B, hq, d), generator=g, device=dev)
    kf = torch.randn((B, hkv, d), generator=g, device=dev)
    vf = torch.randn((B, hkv, d), generator=g, device=dev)
    qw = 1 + 0.1 * torch.randn(d, generator=g, device=dev)
    kw = 1 + 0.1 * torch.randn(d, generator=g, device=dev)
    rope = rope_table(8192, d, 1e6, device=dev)
    pos = lens - 1
    positions = to_dev(pos.astype(np.int32), dev)
    slots = to_dev((table[np.arange(B), pos // 16].astype(np.int64) * 16 + pos % 16).astype(np.int32), dev)
    bt, sl = to_dev(table, dev), to_dev(lens, dev)
    res = []
    for lazy in (False, True):
        p = to_dev(pool, dev)
        plan = decode_plan((B, hq, d), p, bt, sl, None, slots, lazy=lazy)
        outs = []
        for _ in range(2):  # the first call builds a lazy plan, the second reads it
            out = qk_norm_rope_store_and_decode(qf, kf, vf, qw, kw, rope, positions, slots, None, p, bt, sl, plan=plan)
            torch.cuda.synchronize()
            outs.append(out.clone())
        res.append((outs, p, plan))
    (e_outs, e_pool, e_plan), (l_outs, l_pool, l_plan) = res
    for i in range(2):
        _same(e_outs[i], l_outs[i], f"pre-append call {i}")
    _same(e_pool, l_pool, "pre-append pool")
    assert torch.equal(e_plan.buf, l_plan.buf), "pre-append: the plan written differs from the plan kernel's"


def test_lazy_plan_under_validate(dev):
    """validate=True skips a plan not yet built, then checks the built one against a fresh plan."""
    say("lazy plan validate")
    rng = np.random.default_rng(9)
    pool, table, lens, q = _case(rng, [120, 4000, 7, 640], 16, 8, 128)
    qd, p, bt, sl = to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev)
    plan = decode_plan(qd.shape, p, bt, sl, lazy=True)
    a = paged_attention(qd, p, bt, sl, plan=plan, validate=True)
    b = paged_attention(qd, p, bt, sl, plan=plan, validate=True)
    torch.cuda.synchronize()
    _same(a, b, "validated planning and planned calls")
