"""The allocation-free decode entry point (ifn_paged_decode_noalloc) against ifn_paged_decode.

Called through the C ABI, twice in a row (the second call smaller, on other shapes), its output
must equal the workspace entry point's bit for bit; a batch whose split state exceeds the fixed
scratch array is rejected on the host.
"""
import numpy as np
import pytest
import torch

from gpu_util import randn16, say, to_dev
from infurnace_amd import _capi, workloads

pytestmark = pytest.mark.gpu


def _inputs(dev, g, lens, hq, hkv, d, pages):
    B = len(lens)
    mp = max(1, max(-(-int(x) // 16) for x in lens))
    rng = np.random.default_rng(len(lens) * 7 + hq)
    perm = rng.permutation(pages).astype(np.int32)
    table = np.zeros((B, mp), np.int32)
    off = 0
    for b, n in enumerate(-(-np.asarray(lens) // 16)):
        table[b, :n] = perm[off:off + n]
        off += int(n)
    pool = randn16((2, pages, 16, hkv, d), g, dev)
    q = randn16((B, hq, d), g, dev)
    return pool, q, to_dev(table, dev), to_dev(np.asarray(lens, np.int32), dev), mp


def _pair(L, dev, pool, q, bt, sl, act, mp, hq, hkv, d, msl):
    stream = torch.cuda.current_stream(dev).cuda_stream
    B, P = q.shape[0], pool.shape[1]
    nb = L.ifn_paged_decode_workspace_bytes(B, hq, hkv, d, 16, msl)
    ws = torch.zeros(nb, dtype=torch.uint8, device=dev)
    ref = torch.full_like(q, 7.0)
    got = torch.full_like(q, 7.0)
    a = None if act is None else act.data_ptr()
    assert L.ifn_paged_decode(ref.data_ptr(), q.data_ptr(), pool.data_ptr(), P, bt.data_ptr(), mp, sl.data_ptr(), a,
                              B, hq, hkv, d, 16, msl, 0.0, ws.data_ptr(), nb, stream) == 0
    assert L.ifn_paged_decode_noalloc(got.data_ptr(), q.data_ptr(), pool.data_ptr(), P, bt.data_ptr(), mp,
                                      sl.data_ptr(), a, B, hq, hkv, d, 16, msl, 0.0, stream) == 0
    torch.cuda.synchronize()
    return ref, got


def test_noalloc_decode_matches_workspace_entry_twice(dev):
    L = _capi.lib()
    g = torch.Generator(device=dev).manual_seed(7)
    # 1. config 2 at full size (Qwen3-0.6B shapes, 16384-page pool)
    say("noalloc decode config2")
    w = workloads.config2()
    pool = randn16((2, w.num_pages, 16, 8, 128), g, dev)
    q = randn16((w.batch, 16, 128), g, dev)
    bt, sl = to_dev(w.block_tables, dev), to_dev(w.seq_lens, dev)
    ref, got = _pair(L, dev, pool, q, bt, sl, None, w.max_pages, 16, 8, 128, int(w.seq_lens.max()))
    assert torch.equal(ref.view(torch.int16), got.view(torch.int16)), "config 2: noalloc differs"
    del pool
    # 2. a smaller call on other shapes (group 4), with an inactive row and an empty row
    say("noalloc decode small")
    lens = [700, 0, 33, 1500, 16]
    pool, q, bt, sl, mp = _inputs(dev, g, lens, 32, 8, 128, 200)
    act = to_dev(np.asarray([1, 1, 0, 1, 1], np.uint8), dev)
    ref, got = _pair(L, dev, pool, q, bt, sl, act, mp, 32, 8, 128, mp * 16)
    assert torch.equal(ref.view(torch.int16), got.view(torch.int16)), "small call: noalloc differs"
    assert torch.all(got[2] == 7.0) and torch.all(got[1] == 0.0)


def test_noalloc_rejects_batches_beyond_its_scratch(dev):
    L = _capi.lib()
    cap = L.ifn_paged_decode_noalloc_max_bytes()
    B, hq = 4096, 32
    assert L.ifn_paged_decode_workspace_bytes(B, hq, 8, 128, 16, 4096) > cap
    t = torch.zeros(16, dtype=torch.float16, device=dev)
    i = torch.zeros(16, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    assert L.ifn_paged_decode_noalloc(t.data_ptr(), t.data_ptr(), t.data_ptr(), 1, i.data_ptr(), 256, i.data_ptr(),
                                      None, B, hq, 8, 128, 16, 4096, 0.0, stream) == _capi.IFN_ERR_WORKSPACE


def test_noalloc_per_segment_kernel_repeated(dev):
    """Token rows other than 2 KiB take the per-segment kernel, which also keeps its tickets and
    partial states in the static scratch: repeated calls (leftover tickets would show up as a
    wrong merge) equal ifn_paged_decode bit for bit."""
    L = _capi.lib()
    g = torch.Generator(device=dev).manual_seed(11)
    for hq, hkv, d in ((8, 2, 128), (8, 4, 64)):
        say(f"noalloc per-segment hq={hq} hkv={hkv} d={d}")
        lens = [900, 1, 64, 2000, 333, 17]
        pool, q, bt, sl, mp = _inputs(dev, g, lens, hq, hkv, d, 400)
        for rep in range(3):
            ref, got = _pair(L, dev, pool, q, bt, sl, None, mp, hq, hkv, d, mp * 16)
            assert torch.equal(ref.view(torch.int16), got.view(torch.int16)), f"rep {rep}: noalloc differs"


def test_noalloc_under_graph_capture(dev):
    """A call captured into a HIP graph (the callers this entry point is for) records only the
    decode; every replay, with eager work and synchronisations between replays, equals the
    workspace entry point's output bit for bit."""
    L = _capi.lib()
    g = torch.Generator(device=dev).manual_seed(12)
    say("noalloc under graph capture")
    lens = [300, 1200, 45, 700]
    pool, q, bt, sl, mp = _inputs(dev, g, lens, 16, 8, 128, 300)
    B, P, msl = q.shape[0], pool.shape[1], mp * 16
    stream = torch.cuda.current_stream(dev).cuda_stream
    nb = L.ifn_paged_decode_workspace_bytes(B, 16, 8, 128, 16, msl)
    ws = torch.zeros(nb, dtype=torch.uint8, device=dev)
    ref = torch.empty_like(q)
    assert L.ifn_paged_decode(ref.data_ptr(), q.data_ptr(), pool.data_ptr(), P, bt.data_ptr(), mp, sl.data_ptr(),
                              None, B, 16, 8, 128, 16, msl, 0.0, ws.data_ptr(), nb, stream) == 0
    got = torch.full_like(q, 7.0)
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        s = torch.cuda.current_stream(dev).cuda_stream
        assert L.ifn_paged_decode_noalloc(got.data_ptr(), q.data_ptr(), pool.data_ptr(), P, bt.data_ptr(), mp,
                                          sl.data_ptr(), None, B, 16, 8, 128, 16, msl, 0.0, s) == 0
    for rep in range(4):
        got.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ref.view(torch.int16), got.view(torch.int16)), f"replay {rep} differs"
        other = torch.full_like(q, 7.0)  # eager work between replays
        assert L.ifn_paged_decode_noalloc(other.data_ptr(), q.data_ptr(), pool.data_ptr(), P, bt.data_ptr(), mp,
                                          sl.data_ptr(), None, B, 16, 8, 128, 16, msl, 0.0, stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(ref.view(torch.int16), other.view(torch.int16))
