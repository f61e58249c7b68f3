"""Shared-prefix decode (ifn_paged_decode_shared_prefix) on the GPU vs the oracle.

The prefix cache (docs/roadmap.md:442-470) makes rows share their leading pages;
config 5 of the benchmark is 64 rows over one 4096-token prefix.  The shared
entry point reads those pages once for the batch, then merges each row's own
pages in.  Its result is the ordinary paged decode of the same tables, so the
checks are the decode oracle (atol 2e-3 / rtol 1e-2 in fp16) plus agreement
with ifn_paged_decode on the same inputs.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_attn_close, oracle_decode, randn16, say, to_dev
from infurnace_amd import workloads
from infurnace_amd.kernels import paged_attention

pytestmark = pytest.mark.gpu


def _shared(rng, n_shared, suffix_lens, hq, hkv, d, short_rows=()):
    """Tables whose first n_shared pages are the same ids; rows in short_rows get their own
    tables and lengths below the prefix."""
    B = len(suffix_lens)
    lens = np.asarray([n_shared * 16 + s for s in suffix_lens], np.int32)
    for b, L in short_rows:
        lens[b] = L
    pages = [-(-int(L) // 16) for L in lens]
    P = n_shared + sum(pages) + 7
    perm = rng.permutation(P).astype(np.int32)
    prefix = perm[:n_shared]
    table = np.zeros((B, max(max(pages), n_shared, 1)), np.int32)
    off = n_shared
    short = {b for b, _ in short_rows}
    for b in range(B):
        if b in short:
            table[b, :pages[b]] = perm[off:off + pages[b]]
            off += pages[b]
        else:
            own = pages[b] - n_shared
            table[b, :n_shared] = prefix
            table[b, n_shared:pages[b]] = perm[off:off + own]
            off += own
    pool = rng.standard_normal((2, P, 16, hkv, d), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal((B, hq, d), dtype=np.float32).astype(np.float16)
    return pool, table, lens, q, prefix.copy()


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (8, 8, 128), (64, 8, 128), (16, 8, 64),
                                      (4, 1, 64)])
@pytest.mark.parametrize("n_shared", [1, 3, 8, 40])
def test_matches_oracle_and_plain_decode(dev, hq, hkv, d, n_shared):
    say(f"shared-prefix hq={hq} hkv={hkv} d={d} shared={n_shared}")
    rng = np.random.default_rng(hq * 7 + hkv * 3 + d + n_shared)
    suffix = [0, 1, 15, 16, 17, 100, 333, 1000]  # 0: the row is exactly the prefix
    pool, table, lens, q, prefix = _shared(rng, n_shared, suffix, hq, hkv, d)
    args = (to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev), None)
    out = paged_attention(*args, shared_prefix_pages=to_dev(prefix, dev))
    ref = oracle.paged_attention(q, pool, table, lens)
    assert_attn_close(out, ref, f"hq={hq} hkv={hkv} d={d} shared={n_shared}")
    plain = paged_attention(*args)
    assert_attn_close(out, plain.cpu().numpy(), "vs ifn_paged_decode")


def test_short_rows_inactive_rows_and_padding(dev):
    """Rows shorter than the prefix use their own tables; inactive rows are not written."""
    say("shared-prefix short/inactive rows")
    rng = np.random.default_rng(21)
    suffix = [5, 200, 0, 64, 77, 1, 300, 31, 9]
    pool, table, lens, q, prefix = _shared(rng, 12, suffix, 16, 8, 128, short_rows=[(1, 40), (4, 191), (7, 0)])
    active = np.ones(len(suffix), np.uint8)
    active[[3, 6]] = 0
    q_d = to_dev(q, dev)
    out = torch.full_like(q_d, 7.0)
    paged_attention(q_d, to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev), to_dev(active, dev), out=out,
                    shared_prefix_pages=to_dev(prefix, dev))
    live = [i for i in range(len(suffix)) if active[i] and lens[i] > 0]
    ref = oracle.paged_attention(q[live], pool, table[live], lens[live])
    assert_attn_close(out[live], ref, "live rows")
    assert bool((out[[3, 6]] == 7.0).all()), "inactive rows were written"
    assert bool((out[7] == 0).all()), "an active row with no keys must be zero"


@pytest.mark.parametrize("hq", [8, 16, 32])
def test_rows_at_prefix_length_only(dev, hq):
    """Every cascade row is exactly the prefix: no private key in the call, so the decode's token
    list is empty and each output is the prefix states alone; then the same with rows shorter than
    the prefix beside them (attended in full)."""
    say(f"shared-prefix rows at the prefix length only hq={hq}")
    rng = np.random.default_rng(40 + hq)
    for suffix, short in (([0] * 6, []), ([0, 0, 0, 0, 0], [(1, 17), (3, 1)])):
        pool, table, lens, q, prefix = _shared(rng, 9, suffix, hq, 8, 128, short_rows=short)
        args = (to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev), None)
        out = paged_attention(*args, shared_prefix_pages=to_dev(prefix, dev))
        assert_attn_close(out, oracle.paged_attention(q, pool, table, lens), f"short rows {short}")
        assert_attn_close(out, paged_attention(*args).cpu().numpy(), "vs ifn_paged_decode")


def test_deterministic_and_workspace_reuse(dev):
    """Repeated calls are bit-identical; one workspace serves changing shapes."""
    say("shared-prefix determinism + workspace reuse")
    rng = np.random.default_rng(22)
    outs = []
    for n_shared, suffix in ((64, [10, 500, 3]), (5, [1000, 0, 16, 70, 2]), (64, [10, 500, 3])):
        pool, table, lens, q, prefix = _shared(np.random.default_rng(n_shared), n_shared, suffix, 32, 8, 128)
        args = (to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev), None)
        o1 = paged_attention(*args, shared_prefix_pages=to_dev(prefix, dev))
        o2 = paged_attention(*args, shared_prefix_pages=to_dev(prefix, dev))
        assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
        assert_attn_close(o1, oracle.paged_attention(q, pool, table, lens), f"shared={n_shared}")
        outs.append(o1)
    assert torch.equal(outs[0].view(torch.int16), outs[2].view(torch.int16))


def test_config5_full_size_with_churn(dev):
    """Config 5 (64 rows, 4096-token prefix + 512 own tokens, G=4) with suffix page churn."""
    say("shared-prefix config5 churn")
    w = workloads.config5()
    g = torch.Generator(device=dev).manual_seed(505)
    pool = randn16((2, w.num_pages, 16, 8, 128), g, dev)
    table = w.block_tables.copy()
    prefix = to_dev(table[0, :w.shared_prefix_pages].copy(), dev)
    free_ids = list(w.extra["free_ids"])
    for step, churn in enumerate(w.extra["churn"][:2]):
        old = [int(table[r, c]) for r, c in churn]
        new = free_ids[:len(old)]
        free_ids = free_ids[len(old):] + old
        for (r, c), pid in zip(churn, new):
            table[r, c] = pid
        idx = torch.as_tensor(new, dtype=torch.long, device=dev)
        pool[:, idx] = randn16((2, len(new), 16, 8, 128), g, dev)
        q = randn16((w.batch, 32, 128), g, dev)
        tdev, ldev = to_dev(table, dev), to_dev(w.seq_lens, dev)
        out = paged_attention(q, pool, tdev, ldev, None, shared_prefix_pages=prefix)
        assert_attn_close(out, oracle_decode(pool, table, w.seq_lens, q), f"config5 step {step}, all rows")
        plain = paged_attention(q, pool, tdev, ldev, None)
        assert_attn_close(out, plain.cpu().numpy(), f"config5 step {step} vs ifn_paged_decode")


def test_config5_one_launch_deterministic(dev):
    """Config 5 decodes in one launch whose prefix and private-page workgroups finish at about the same
    time, so which of them merges a (row, kv head) varies from call to call; the output must not.
    Ten calls bit-identical, and the G = 2 form (Qwen3-0.6B heads over the same tables) too."""
    say("shared-prefix config5 one-launch determinism")
    w = workloads.config5()
    g = torch.Generator(device=dev).manual_seed(55)
    prefix = to_dev(w.block_tables[0, :w.shared_prefix_pages].copy(), dev)
    tdev, ldev = to_dev(w.block_tables, dev), to_dev(w.seq_lens, dev)
    for hq in (32, 16):
        pool = randn16((2, w.num_pages, 16, 8, 128), g, dev)
        q = randn16((w.batch, hq, 128), g, dev)
        first = paged_attention(q, pool, tdev, ldev, None, shared_prefix_pages=prefix)
        for i in range(9):
            again = paged_attention(q, pool, tdev, ldev, None, shared_prefix_pages=prefix)
            assert torch.equal(first.view(torch.int16), again.view(torch.int16)), f"hq={hq}: call {i + 1} differs"
        rows = [0, 17, 40, 63]
        assert_attn_close(first[rows], oracle_decode(pool, w.block_tables, w.seq_lens, q, rows=rows),
                          f"hq={hq} rows")


def test_large_batch_many_splits(dev):
    """200 rows over a 2000-token prefix: several query blocks and key splits in the prefix pass."""
    say("shared-prefix B=200 prefix 2000")
    rng = np.random.default_rng(23)
    suffix = list(rng.integers(0, 300, size=200))
    pool, table, lens, q, prefix = _shared(rng, 125, suffix, 16, 8, 128)
    args = (to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev), None)
    out = paged_attention(*args, shared_prefix_pages=to_dev(prefix, dev))
    rows = [0, 1, 63, 64, 127, 128, 199]
    ref = oracle.paged_attention(q[rows], pool, table[rows], lens[rows])
    assert_attn_close(out[rows], ref, "B=200")
    assert_attn_close(out, paged_attention(*args).cpu().numpy(), "B=200 vs ifn_paged_decode")


def test_workspace_shared_with_other_entry_points(dev):
    """Shared-prefix, plain decode and prefill calls alternate on one workspace (fixed ticket area)."""
    say("shared-prefix workspace alternation")
    rng = np.random.default_rng(24)
    for rep in range(2):
        for n_shared, suffix, hq in ((40, [3, 900, 64, 0], 16), (200, list(rng.integers(0, 500, 33)), 32)):
            pool, table, lens, q, prefix = _shared(rng, n_shared, suffix, hq, 8, 128)
            args = (to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev), None)
            ref = oracle.paged_attention(q, pool, table, lens)
            assert_attn_close(paged_attention(*args, shared_prefix_pages=to_dev(prefix, dev)), ref,
                              f"rep {rep} shared={n_shared}")
            assert_attn_close(paged_attention(*args), ref, f"rep {rep} plain")
            t = 200
            qp = rng.standard_normal((t, hq, 128), dtype=np.float32).astype(np.float16)
            o2 = paged_attention(to_dev(qp, dev), args[1], to_dev(table[1], dev), None, None,
                                 query_start=int(lens[1]) - t)
            ref2 = oracle.paged_attention(qp[None], pool, table[1:2], lens[1:2])[0]
            assert_attn_close(o2, ref2, f"rep {rep} prefill")


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (16, 8, 64)])
def test_no_common_prefix_cached_loads_equal_streaming(dev, hq, hkv, d):
    """shared_pages == 0 is the plain decode with cached page loads: bit-identical to
    ifn_paged_decode (streaming loads) on tables whose rows share pages, and to the oracle."""
    say(f"cached plain decode hq={hq} hkv={hkv} d={d}")
    rng = np.random.default_rng(hq + hkv + d)
    pool, table, lens, q, prefix = _shared(rng, 12, [0, 3, 40, 160, 700], hq, hkv, d)
    # two rows swap their shared pages' order, so the shared pages form no common leading run
    table[1, :12] = table[1, :12][::-1]
    args = (to_dev(q, dev), to_dev(pool, dev), to_dev(table, dev), to_dev(lens, dev), None)
    cached = paged_attention(*args, shared_prefix_pages=torch.zeros(0, dtype=torch.int32, device=dev))
    streamed = paged_attention(*args)
    assert torch.equal(cached.view(torch.int16), streamed.view(torch.int16))
    assert_attn_close(cached, oracle.paged_attention(q, pool, table, lens), f"hq={hq} hkv={hkv} d={d}")


def _planned_equal(dev, pool, table, lens, q, prefix, active=None, what=""):
    """The planned shared-prefix decode equals the unplanned one bit for bit."""
    from infurnace_amd.kernels import decode_plan
    t, l = to_dev(table, dev), to_dev(lens, dev)
    p, qd = (pool if isinstance(pool, torch.Tensor) else to_dev(pool, dev)), to_dev(q, dev)
    pf = to_dev(prefix, dev) if not isinstance(prefix, torch.Tensor) else prefix
    am = None if active is None else to_dev(active, dev)
    o1 = torch.full_like(qd, 7.0)
    o2 = torch.full_like(qd, 7.0)
    paged_attention(qd, p, t, l, am, out=o1, shared_prefix_pages=pf)
    plan = decode_plan(qd.shape, p, t, l, am, shared_prefix_pages=pf)
    for _ in range(2):  # the plan serves every layer of the step
        paged_attention(qd, p, t, l, am, out=o2, shared_prefix_pages=pf, plan=plan)
        torch.cuda.synchronize()
        assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), f"{what}: planned differs"
    return o2


@pytest.mark.parametrize("hq", [16, 32])
def test_planned_equals_unplanned(dev, hq):
    """A step plan of the shared-prefix decode (ifn_paged_decode_shared_prefix_plan): rows longer
    than the prefix, exactly the prefix, shorter than it, inactive and empty; with rows split over
    several workgroups and with ranges holding more rows than a plan record describes."""
    say(f"shared-prefix planned == unplanned hq={hq}")
    rng = np.random.default_rng(60 + hq)
    suffix = [5, 200, 0, 64, 77, 1, 3000, 31, 9, 0, 450] + [2] * 40
    pool, table, lens, q, prefix = _shared(rng, 12, suffix, hq, 8, 128, short_rows=[(1, 40), (4, 191), (7, 0)])
    active = np.ones(len(suffix), np.uint8)
    active[[3, 6]] = 0
    out = _planned_equal(dev, pool, table, lens, q, prefix, active, "ragged")
    live = [i for i in range(len(suffix)) if active[i] and lens[i] > 0]
    assert_attn_close(out[live], oracle.paged_attention(q[live], pool, table[live], lens[live]), "planned ragged")
    # every cascade row exactly the prefix (the token list holds only the short rows)
    pool, table, lens, q, prefix = _shared(rng, 9, [0, 0, 0, 0], hq, 8, 128, short_rows=[(2, 17)])
    _planned_equal(dev, pool, table, lens, q, prefix, None, "prefix only")
    # 1500 rows of one private key: about 8 pieces per range, past the 3 a plan record holds
    pool, table, lens, q, prefix = _shared(rng, 2, [1] * 1500 + [2000], hq, 8, 128)
    out = _planned_equal(dev, pool, table, lens, q, prefix, None, "many pieces per range")
    rows = [0, 1, 700, 1499, 1500]
    assert_attn_close(out[rows], oracle.paged_attention(q[rows], pool, table[rows], lens[rows]), "many pieces")


def test_planned_config5_and_mismatched_plans(dev):
    """Config 5 at full size: planned == unplanned.  A plan built for a different shared-page count is
    refused by the wrapper; passed to the C entry point it is detected there and ignored (same bits)."""
    from infurnace_amd import _capi
    from infurnace_amd.kernels import decode_plan
    say("shared-prefix planned config5")
    w = workloads.config5()
    g = torch.Generator(device=dev).manual_seed(515)
    pool = randn16((2, w.num_pages, 16, 8, 128), g, dev)
    q = randn16((w.batch, 32, 128), g, dev)
    sp = w.shared_prefix_pages
    prefix = to_dev(w.block_tables[0, :sp].copy(), dev)
    out = _planned_equal(dev, pool, w.block_tables, w.seq_lens, q.cpu().numpy(), prefix, None, "config5")
    rows = [0, 31, 63]
    assert_attn_close(out[rows], oracle_decode(pool, w.block_tables, w.seq_lens, q, rows=rows), "config5 rows")
    t, l = to_dev(w.block_tables, dev), to_dev(w.seq_lens, dev)
    other = decode_plan(q.shape, pool, t, l, shared_prefix_pages=prefix[:sp - 1])
    with pytest.raises(Exception):
        paged_attention(q, pool, t, l, None, shared_prefix_pages=prefix, plan=other)
    L = _capi.lib()
    nb = L.ifn_paged_decode_shared_prefix_workspace_bytes(w.batch, 32, 8, 128, 16, sp)
    ws = torch.zeros(nb, dtype=torch.uint8, device=dev)
    o3 = torch.empty_like(q)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = L.ifn_paged_decode_shared_prefix_planned(o3.data_ptr(), q.data_ptr(), pool.data_ptr(), w.num_pages,
                                                  prefix.data_ptr(), sp, t.data_ptr(), t.shape[1], l.data_ptr(), None,
                                                  w.batch, 32, 8, 128, 16, int(w.seq_lens.max()), 0.0,
                                                  other.buf.data_ptr(), other.nbytes, ws.data_ptr(), nb, stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(o3.view(torch.int16), out.view(torch.int16)), "a plan for another prefix was not ignored"
