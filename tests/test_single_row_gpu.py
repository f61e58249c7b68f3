"""Single-row decode calls (batch 1) on the GPU.

A call of one row is split over the CUs without the per-row start cost that the split charges a
call of several rows (every range then holds one piece of that row): a row of L keys takes
min(CUs, ceil(L / 32)) ranges, and the last arrival merges that many split states.  Checked at
lengths around the page, burst, range and merge-batch edges (512 is config 1, whose 16 ranges
make exactly one 16-state merge batch; 513 is the first length that needs 17):

- the unplanned call against the oracle (16-token pages, and 32- and 64-token pages);
- planned and planning calls (the step's first decode, which writes the plan) bit-identical to
  the unplanned one, and the written plan byte-identical to the plan kernel's;
- the fused append bit-identical to its planned and planning forms, and close to the oracle on
  the appended pool;
- the shared-prefix entry with one cascade row against the oracle.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_attn_close, say, to_dev
from infurnace_amd.kernels import decode_plan, paged_attention, store_kv_and_decode

pytestmark = pytest.mark.gpu

LENS = [1, 4, 15, 16, 31, 32, 33, 100, 255, 256, 257, 511, 512, 513, 544, 1000, 4096, 8191]


def _row(rng, L, hq, hkv, d, extra_pages=3, bs=16):
    n = max(1, -(-L // bs))
    P = n + extra_pages
    table = rng.permutation(P)[:n].astype(np.int32)[None, :]
    pool = rng.standard_normal((2, P, bs, hkv, d), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal((1, hq, d), dtype=np.float32).astype(np.float16)
    return pool, table, np.asarray([L], np.int32), q


def _bits(a: torch.Tensor) -> torch.Tensor:
    return a.view(torch.int16)


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (32, 16, 64)])
def test_single_row_decode_forms(dev, hq, hkv, d):
    for L in LENS:
        say(f"single row L={L} hq={hq} hkv={hkv} d={d}")
        rng = np.random.default_rng(L * 31 + hq + d)
        pool, table, lens, q = _row(rng, L, hq, hkv, d)
        qd, p, bt, sl = to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev)
        ref = paged_attention(qd, p, bt, sl)
        torch.cuda.synchronize()
        assert_attn_close(ref, oracle.paged_attention(q, pool, table, lens), f"L={L}")
        eager = decode_plan(qd.shape, p, bt, sl)
        planned = paged_attention(qd, p, bt, sl, plan=eager)
        lazy = decode_plan(qd.shape, p, bt, sl, lazy=True)
        planning = paged_attention(qd, p, bt, sl, plan=lazy)  # writes the plan
        after = paged_attention(qd, p, bt, sl, plan=lazy)     # reads it
        torch.cuda.synchronize()
        for got, what in ((planned, "planned"), (planning, "planning"), (after, "planned with the written plan")):
            assert torch.equal(_bits(got), _bits(ref)), f"L={L}: {what} differs from unplanned"
        if eager.buf is not None:
            assert torch.equal(eager.buf, lazy.buf), f"L={L}: the written plan differs from the plan kernel's"


@pytest.mark.parametrize("bs", [32, 64])
def test_single_row_larger_pages(dev, bs):
    """The 32- and 64-token page instantiations (their own kernels and plan kernels) split a single
    row the same way."""
    for L in (1, 31, 33, 512, 513, 2047, 5000):
        say(f"single row L={L} page {bs}")
        rng = np.random.default_rng(L + bs)
        pool, table, lens, q = _row(rng, L, 16, 8, 128, bs=bs)
        qd, p, bt, sl = to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev)
        ref = paged_attention(qd, p, bt, sl, block_size=bs)
        torch.cuda.synchronize()
        assert_attn_close(ref, oracle.paged_attention(q, pool, table, lens), f"L={L} page {bs}")
        eager = decode_plan(qd.shape, p, bt, sl, block_size=bs)
        planned = paged_attention(qd, p, bt, sl, block_size=bs, plan=eager)
        lazy = decode_plan(qd.shape, p, bt, sl, block_size=bs, lazy=True)
        planning = paged_attention(qd, p, bt, sl, block_size=bs, plan=lazy)
        torch.cuda.synchronize()
        assert torch.equal(_bits(planned), _bits(ref)), f"L={L} page {bs}: planned differs"
        assert torch.equal(_bits(planning), _bits(ref)), f"L={L} page {bs}: planning differs"
        assert torch.equal(eager.buf, lazy.buf), f"L={L} page {bs}: the written plan differs"


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128)])
def test_single_row_fused_append(dev, hq, hkv, d):
    for L in (1, 17, 512, 513, 3000):
        say(f"single row fused append L={L} hq={hq}")
        rng = np.random.default_rng(L + 7 * hq)
        pool, table, lens, q = _row(rng, L, hq, hkv, d)
        pos = L - 1
        slot = int(table[0, pos // 16]) * 16 + pos % 16
        kn = rng.standard_normal((1, hkv, d), dtype=np.float32).astype(np.float16)
        vn = rng.standard_normal((1, hkv, d), dtype=np.float32).astype(np.float16)
        qd, bt, sl = to_dev(q, dev), to_dev(table, dev), to_dev(lens, dev)
        slots = to_dev(np.asarray([slot], np.int32), dev)
        k, v = to_dev(kn, dev), to_dev(vn, dev)
        res = []
        for mode in ("unplanned", "planned", "planning"):
            p = to_dev(pool, dev)
            plan = None if mode == "unplanned" else decode_plan(qd.shape, p, bt, sl, None, slots,
                                                                lazy=mode == "planning")
            out = store_kv_and_decode(qd, p, bt, sl, None, slots, k, v, plan=plan)
            torch.cuda.synchronize()
            res.append((out, p))
        for (o, p), mode in zip(res[1:], ("planned", "planning")):
            assert torch.equal(_bits(o), _bits(res[0][0])), f"L={L}: {mode} output differs"
            assert torch.equal(_bits(p), _bits(res[0][1])), f"L={L}: {mode} pool differs"
        host = pool.copy()
        host[0, slot // 16, slot % 16] = kn[0]
        host[1, slot // 16, slot % 16] = vn[0]
        assert np.array_equal(res[0][1].cpu().numpy(), host), f"L={L}: appended pool"
        assert_attn_close(res[0][0], oracle.paged_attention(q, host, table, lens), f"L={L} fused")


@pytest.mark.parametrize("hq", [16, 32])
@pytest.mark.parametrize("suffix", [0, 1, 100, 513, 600])
def test_single_row_shared_prefix(dev, hq, suffix):
    say(f"single row shared prefix hq={hq} suffix={suffix}")
    hkv, d, n_shared = 8, 128, 40
    rng = np.random.default_rng(hq + suffix)
    L = n_shared * 16 + suffix
    pool, table, lens, q = _row(rng, L, hq, hkv, d)
    prefix = to_dev(np.ascontiguousarray(table[0, :n_shared]), dev)
    args = (to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev), None)
    out = paged_attention(*args, shared_prefix_pages=prefix)
    torch.cuda.synchronize()
    assert_attn_close(out, oracle.paged_attention(q, pool, table, lens), f"shared prefix suffix={suffix}")
