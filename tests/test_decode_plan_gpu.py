"""Decode step plans on the GPU: a planned call equals the unplanned one bit for bit.

The step plan (``decode_plan`` / ``ifn_paged_decode_plan``) precomputes the split of a decode
batch's keys over the CUs once per step; every layer's decode (and fused append) then starts its
page loads earlier.  It changes no arithmetic, so planned and unplanned outputs -- and pools,
for the fused append -- must be identical, and both must match the oracle.  A plan built for
another batch is detected through its header and ignored.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_attn_close, oracle_decode, randn16, say, to_dev
from infurnace_amd import _capi, workloads
from infurnace_amd.kernels import decode_plan, paged_attention, store_kv_and_decode
from infurnace_amd.kernels.paged_attention import workspace_for

pytestmark = pytest.mark.gpu


def _ragged(rng, lens, hq, hkv, d, extra_pages=5):
    pages = [max(1, -(-int(L) // 16)) for L in lens]
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


def _both(dev, q, pool, table, lens, active=None, slots=None, k=None, v=None, msl=None):
    """(unplanned, planned) outputs -- and pools when k/v are given (fused append)."""
    qd, bt, sl = to_dev(q, dev), to_dev(table, dev), to_dev(lens, dev)
    act = None if active is None else to_dev(active, dev)
    res = []
    for planned in (False, True):
        p = to_dev(pool, dev) if isinstance(pool, np.ndarray) else pool.clone()
        plan = decode_plan(qd.shape, p, bt, sl, act, None if slots is None else slots, max_seq_len=msl) if planned \
            else None
        out = torch.full(qd.shape, 7.0, dtype=torch.float16, device=dev)
        if k is None:
            paged_attention(qd, p, bt, sl, act, out=out, max_seq_len=msl, plan=plan)
        else:
            store_kv_and_decode(qd, p, bt, sl, act, slots, k, v, out=out, max_seq_len=msl, plan=plan)
        torch.cuda.synchronize()
        res.append((out, p))
    return res


def _assert_same(a: torch.Tensor, b: torch.Tensor, what: str):
    assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"{what}: planned differs from unplanned"


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (8, 8, 128), (32, 16, 64), (8, 4, 256)])
def test_plan_matches_unplanned_on_ragged_edges(dev, hq, hkv, d):
    say(f"plan ragged hq={hq} hkv={hkv} d={d}")
    rng = np.random.default_rng(hq * 100 + d)
    lens = [1, 2, 15, 16, 17, 31, 33, 64, 100, 255, 256, 257, 1000, 1024, 4096]
    pool, table, lens, q = _ragged(rng, lens, hq, hkv, d)
    (u, _), (p, _) = _both(dev, q, pool, table, lens)
    _assert_same(u, p, f"hq={hq} d={d}")
    assert_attn_close(p, oracle.paged_attention(q, pool, table, lens), f"planned hq={hq} hkv={hkv} d={d}")


def test_plan_inactive_zero_and_bad_pages(dev):
    say("plan inactive/zero/bad-page")
    rng = np.random.default_rng(31)
    pool, table, lens, q = _ragged(rng, [50, 700, 33, 90, 0, 300], 16, 8, 128)
    lens_dev = lens.copy()
    lens_dev[2] = 0
    active = np.asarray([True, False, True, True, True, True])
    bad = table.copy()
    bad[5, 1] = pool.shape[1] + 1000
    bad[5, 3] = -7
    (u, _), (p, _) = _both(dev, q, pool, bad, lens_dev, active=active)
    _assert_same(u, p, "inactive/zero/bad")
    assert torch.all(p[1] == 7.0)  # inactive: untouched
    assert torch.all(p[2] == 0.0) and torch.all(p[4] == 0.0)  # active without keys: zeros
    assert_attn_close(p[[0, 3]], oracle.paged_attention(q[[0, 3]], pool, table[[0, 3]], lens[[0, 3]]), "good rows")


@pytest.mark.parametrize("batch", [200, 700])
def test_plan_many_short_rows(dev, batch):
    """Ranges hold more rows than a plan record describes (and > 512 rows: offsets copied in a loop)."""
    say(f"plan many short rows batch={batch}")
    rng = np.random.default_rng(batch)
    lens = rng.integers(0, 41, size=batch)
    pool, table, lens, q = _ragged(rng, lens, 16, 8, 128)
    active = rng.random(batch) < 0.9
    (u, _), (p, _) = _both(dev, q, pool, table, lens, active=active)
    _assert_same(u, p, f"batch {batch}")
    live = np.nonzero(active & (lens > 0))[0]
    assert_attn_close(p[torch.as_tensor(live, device=dev)],
                      oracle.paged_attention(q[live], pool, table[live], lens[live]), "live rows")


def test_plan_config2_full_size_decode_and_fused_append(dev):
    say("plan config2 full")
    w = workloads.config2()
    g = torch.Generator(device=dev).manual_seed(2121)
    pool = randn16((2, w.num_pages, 16, 8, 128), g, dev)
    q = randn16((w.batch, 16, 128), g, dev)
    msl = int(w.seq_lens.max())
    (u, _), (p, _) = _both(dev, q.cpu().numpy(), pool, w.block_tables, w.seq_lens, msl=msl)
    _assert_same(u, p, "config2 decode")
    assert_attn_close(p, oracle_decode(pool, w.block_tables, w.seq_lens, q), "config2 planned")
    slots = to_dev(w.append_slots, dev)
    k, v = randn16((w.batch, 8, 128), g, dev), randn16((w.batch, 8, 128), g, dev)
    (u, pu), (p, pp) = _both(dev, q.cpu().numpy(), pool, w.block_tables, w.seq_lens, slots=slots, k=k, v=v, msl=msl)
    _assert_same(u, p, "config2 fused append")
    assert torch.equal(pu.view(torch.int16), pp.view(torch.int16)), "fused append: pools differ"
    flat = pp.view(2, -1, 8, 128)
    assert torch.equal(flat[0, slots.long()].view(torch.int16), k.view(torch.int16))


def test_plan_for_another_batch_is_ignored(dev):
    """A plan whose header names another batch size is not used (the C entry falls back)."""
    say("plan header mismatch")
    rng = np.random.default_rng(77)
    pool, table, lens, q = _ragged(rng, [300, 900, 40, 2000], 16, 8, 128)
    L = _capi.lib()
    poold, bt, sl, qd = to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev), to_dev(q, dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    P, mp, msl = pool.shape[1], table.shape[1], table.shape[1] * 16
    big = max(L.ifn_paged_decode_plan_bytes(n, 16, 8, 128, 16, mp, msl) for n in (3, 4))
    plan = torch.zeros(big, dtype=torch.uint8, device=dev)
    assert L.ifn_paged_decode_plan(plan.data_ptr(), big, bt.data_ptr(), mp, sl.data_ptr(), None, None, P, 3, 16, 8,
                                   128, 16, msl, stream) == 0  # plan of the first 3 rows
    nb = L.ifn_paged_decode_workspace_bytes(4, 16, 8, 128, 16, msl)
    ws = workspace_for(dev, stream, nb)
    out = torch.empty_like(qd)
    assert L.ifn_paged_decode_planned(out.data_ptr(), qd.data_ptr(), poold.data_ptr(), P, bt.data_ptr(), mp,
                                      sl.data_ptr(), None, 4, 16, 8, 128, 16, msl, 0.0, plan.data_ptr(), big,
                                      ws.data_ptr(), ws.numel(), stream) == 0
    ref = paged_attention(qd, poold, bt, sl, None)
    torch.cuda.synchronize()
    _assert_same(ref, out, "mismatched plan")
    # a plan buffer too small for a record per workgroup is rejected on the host
    assert L.ifn_paged_decode_planned(out.data_ptr(), qd.data_ptr(), poold.data_ptr(), P, bt.data_ptr(), mp,
                                      sl.data_ptr(), None, 4, 16, 8, 128, 16, msl, 0.0, plan.data_ptr(), 64,
                                      ws.data_ptr(), ws.numel(), stream) == _capi.IFN_ERR_WORKSPACE


def test_plan_reused_across_layers(dev):
    """One plan serves every layer of a step (the runner builds one per step)."""
    say("plan reused across layers")
    w = workloads.config2()
    g = torch.Generator(device=dev).manual_seed(99)
    layers = 2
    pool = randn16((layers, 2, w.num_pages, 16, 8, 128), g, dev)
    bt, sl = to_dev(w.block_tables, dev), to_dev(w.seq_lens, dev)
    q = randn16((layers, w.batch, 16, 128), g, dev)
    plan = decode_plan(q[0].shape, pool, bt, sl, None)
    for layer in range(layers):
        a = paged_attention(q[layer], pool, bt, sl, None, layer=layer, plan=plan)
        b = paged_attention(q[layer], pool, bt, sl, None, layer=layer)
        torch.cuda.synchronize()
        _assert_same(a, b, f"layer {layer}")
