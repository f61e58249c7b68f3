"""PagedKVRunner: the KV side of a Runner (src/infurnace/executor/runner.py:5-45) driven the way
the engine drives it -- chunked prefill, batched decode plans with padding rows, clear_slot and
slot reuse -- against the oracle on a contiguous per-slot cache.  Tolerance atol 2e-3 / rtol
1e-2 (fp16 outputs, fp32 accumulation)."""
from dataclasses import dataclass

import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_attn_close, say, to_dev
from infurnace_amd.runner import PagedKVRunner, RunnerError

pytestmark = pytest.mark.gpu

L, HQ, HKV, D = 2, 16, 8, 128


@dataclass(frozen=True)
class Plan:  # the fields of DecodePlan (src/infurnace/scheduler/plan.py:16-28) the runner reads
    slots: tuple
    positions: tuple
    active_mask: tuple
    block_tables: tuple = ()


class Reference:
    """Contiguous fp16 K/V per (slot, layer), attention by the oracle over an identity table."""

    def __init__(self):
        self.k, self.v = {}, {}

    def clear(self, slot):
        for l in range(L):
            self.k.pop((slot, l), None)
            self.v.pop((slot, l), None)

    def append(self, slot, layer, k, v):
        key = (slot, layer)
        self.k[key] = np.concatenate([self.k.get(key, np.zeros((0, HKV, D), np.float16)), k])
        self.v[key] = np.concatenate([self.v.get(key, np.zeros((0, HKV, D), np.float16)), v])

    def attend(self, slot, layer, q, start):
        kk, vv = self.k[(slot, layer)], self.v[(slot, layer)]
        n = kk.shape[0]
        pages = -(-n // 16)
        pool = np.zeros((2, pages, 16, HKV, D), np.float16)
        pool[0].reshape(-1, HKV, D)[:n] = kk
        pool[1].reshape(-1, HKV, D)[:n] = vv
        table = np.arange(pages, dtype=np.int32)
        if start is None:  # decode: one query [Hq, D] at position n - 1
            return oracle.paged_attention(q[None], pool, table[None], np.asarray([n], np.int32))[0]
        # prefill: the T causal queries [T, Hq, D] end at position n - 1
        return oracle.paged_attention(q[None], pool, table[None], np.asarray([n], np.int32))[0]


def _qkv(rng, T):
    f = lambda *s: rng.standard_normal(s, dtype=np.float32).astype(np.float16)
    return f(T, HQ, D), f(T, HKV, D), f(T, HKV, D)


def test_engine_sequence_of_prefills_decodes_and_slot_reuse(dev):
    say("runner: chunked prefill, batched decode with padding, clear_slot, reuse")
    rng = np.random.default_rng(9)
    run = PagedKVRunner(L, num_slots=3, max_context=256, num_kv_heads=HKV, head_dim=D, num_blocks=64, device=dev)
    ref = Reference()

    def prefill(slot, start, T):
        step = run.begin_prefill(slot, start, T)
        for l in range(L):
            q, k, v = _qkv(rng, T)
            out = step.store_attend(l, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev))
            ref.append(slot, l, k, v)
            assert_attn_close(out, ref.attend(slot, l, q, start), f"prefill slot {slot} start {start} layer {l}")

    def decode(rows):  # rows: list of (slot, active)
        plan = Plan(tuple(s for s, _ in rows), tuple(run.length(s) if a else 0 for s, a in rows),
                    tuple(a for _, a in rows))
        filled = run.fill_block_tables(plan)
        step = run.begin_decode(plan)
        for l in range(L):
            q, k, v = _qkv(rng, len(rows))
            sentinel = torch.full((len(rows), HQ, D), 3.0, dtype=torch.float16, device=dev)
            out = step.store_attend(l, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), out=sentinel)
            for i, (s, a) in enumerate(rows):
                if not a:
                    assert torch.all(out[i] == 3.0), "a padding row was written"
                    continue
                ref.append(s, l, k[i:i + 1], v[i:i + 1])
                assert_attn_close(out[i:i + 1], ref.attend(s, l, q[i], None)[None], f"decode slot {s} layer {l}")
        return filled

    prefill(0, 0, 32)
    prefill(0, 32, 8)          # second chunk of the same prompt
    prefill(1, 0, 20)
    for _ in range(5):
        filled = decode([(0, True), (1, True), (2, False)])
    assert list(filled[0][:3]) == run.mgr.blocks(0)[:3]
    owned = run.mgr.blocks(0)
    freed = run.clear_slot(0, zero=True)   # pages the last step still uses come back once it completes
    freed += run.synchronize()
    assert sorted(freed) == sorted(owned)
    assert all(torch.all(run.cache.kv[:, :, p] == 0) for p in freed)
    ref.clear(0)
    prefill(0, 0, 10)          # the slot is reused from position 0
    for _ in range(3):
        decode([(1, True), (0, True)])
    run.pool.check_invariants()


def test_runner_rejects_out_of_order_work(dev):
    say("runner error paths")
    run = PagedKVRunner(1, num_slots=2, max_context=64, num_kv_heads=HKV, head_dim=D, num_blocks=8, device=dev)
    run.begin_prefill(0, 0, 16)
    with pytest.raises(RunnerError):
        run.begin_prefill(0, 8, 4)                     # chunk does not start at the stored length
    with pytest.raises(RunnerError):
        run.begin_decode(Plan((0,), (15,), (True,)))  # position must be the stored length (16)
    with pytest.raises(RunnerError):
        run.begin_decode(Plan((1,), (0,), (True,)))   # slot 1 was never prefilled
    with pytest.raises(RunnerError):
        run.begin_prefill(1, 0, 65)                    # past max_context
    with pytest.raises(RunnerError):
        run.begin_prefill(3, 0, 1)                     # slot out of range


def test_prefix_cache_hit_shares_pages_and_matches_full_prefill(dev):
    say("runner: prefix-cache hit")
    rng = np.random.default_rng(21)
    run = PagedKVRunner(1, num_slots=2, max_context=256, num_kv_heads=HKV, head_dim=D, num_blocks=32, device=dev,
                        prefix_namespace=("toy", "fp16"))
    prompt = list(range(1000, 1048))                 # 48 tokens = 3 complete blocks
    q, k, v = _qkv(rng, 48)
    step = run.begin_prefill(0, 0, 48)
    step.store_attend(0, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev))
    assert run.publish_prefix(0, prompt) == 3
    # a second prompt extends the first: its first 48 tokens (3 pages) are shared
    n = run.attach_prefix(1, prompt + [7, 8, 9, 10, 11])
    assert n == 48 and run.mgr.blocks(1)[:3] == run.mgr.blocks(0)[:3]
    q2, k2, v2 = _qkv(rng, 5)
    step = run.begin_prefill(1, 48, 5)
    out = step.store_attend(0, to_dev(q2, dev), to_dev(k2, dev), to_dev(v2, dev))
    ref = Reference()
    ref.append(1, 0, np.concatenate([k, k2]), np.concatenate([v, v2]))
    assert_attn_close(out, ref.attend(1, 0, q2, 48), "suffix prefill over shared prefix pages")
    # the shared pages outlive both slots while the cache holds them
    shared = run.mgr.blocks(0)[:3]
    run.clear_slot(0)
    run.clear_slot(1)
    assert all(not run.pool.is_free(p) for p in shared)
    assert sorted(run.prefix.evict(3)) == sorted(shared)
    run.pool.check_invariants()


@pytest.mark.parametrize("min_pages", [2, 64])
def test_decode_batch_over_shared_prefix_uses_one_read(dev, min_pages):
    """Rows attached to one cached prompt decode through the shared-prefix path (6 common pages,
    min_pages 2), or with cached page loads when the common run is below the threshold
    (min_pages 64); outputs match in both."""
    say(f"runner: decode over a shared prefix, min_pages={min_pages}")
    rng = np.random.default_rng(31)
    run = PagedKVRunner(L, num_slots=4, max_context=512, num_kv_heads=HKV, head_dim=D, num_blocks=128, device=dev,
                        prefix_namespace=("toy", "fp16"), shared_prefix_min_pages=min_pages)
    ref = Reference()
    prompt = list(range(500, 500 + 100))              # 6 complete blocks + 4 tokens
    step = run.begin_prefill(0, 0, 100)
    for l in range(L):
        q, k, v = _qkv(rng, 100)
        step.store_attend(l, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev))
        ref.append(0, l, k, v)
    run.publish_prefix(0, prompt)
    for s, extra in ((1, 9), (2, 30), (3, 1)):
        n = run.attach_prefix(s, prompt[:96] + list(range(extra)))
        assert n == 96
        for l in range(L):
            ref.k[(s, l)], ref.v[(s, l)] = ref.k[(0, l)][:96].copy(), ref.v[(0, l)][:96].copy()
        step = run.begin_prefill(s, n, extra)
        for l in range(L):
            q, k, v = _qkv(rng, extra)
            step.store_attend(l, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev))
            ref.append(s, l, k, v)
    for it in range(3):
        rows = [(1, True), (2, True), (0, True), (3, True)]
        plan = Plan(tuple(s for s, _ in rows), tuple(run.length(s) for s, _ in rows), tuple(a for _, a in rows))
        step = run.begin_decode(plan)
        assert step.shared_prefix is not None and step.shared_prefix.numel() == (6 if min_pages == 2 else 0)
        for l in range(L):
            q, k, v = _qkv(rng, len(rows))
            out = step.store_attend(l, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev))
            for i, (s, _) in enumerate(rows):
                ref.append(s, l, k[i:i + 1], v[i:i + 1])
                assert_attn_close(out[i:i + 1], ref.attend(s, l, q[i], None)[None], f"shared decode slot {s} l {l}")
    run.pool.check_invariants()


def test_randomized_engine_trace(dev):
    """A seeded random engine trace: prompts with prefix-cache hits, chunked prefills of varied
    sizes (aligned and unaligned starts), batched decodes with padding rows, shared-prefix
    decode batches, releases and slot reuse -- every attention output checked against the
    contiguous-cache oracle."""
    say("runner: randomized engine trace")
    rng = np.random.default_rng(2026)
    n_slots = 5
    run = PagedKVRunner(L, num_slots=n_slots, max_context=768, num_kv_heads=HKV, head_dim=D, num_blocks=400,
                        device=dev, prefix_namespace=("toy", "fp16"), shared_prefix_min_pages=2)
    ref = Reference()
    prompts = {}
    block_kv = {}  # (token prefix through block i) -> per-layer K/V of block i, first publisher's
    base_prompt = [int(t) for t in rng.integers(0, 1000, size=160)]  # shared by several requests
    seen = {"shared_steps": 0, "unaligned_chunks": 0}

    def prefill_prompt(slot, toks):
        n = run.attach_prefix(slot, toks)
        for l in range(L):  # a cache hit's pages hold the K/V of the request that published them
            if n:
                blocks = [block_kv[(tuple(toks[:16 * (i + 1)]), l)] for i in range(n // 16)]
                ref.k[(slot, l)] = np.concatenate([kb for kb, _ in blocks])
                ref.v[(slot, l)] = np.concatenate([vb for _, vb in blocks])
        pos = n
        while pos < len(toks):
            T = int(min(len(toks) - pos, rng.choice([16, 32, 37, 64, 100])))
            seen["unaligned_chunks"] += pos % 32 != 0
            step = run.begin_prefill(slot, pos, T)
            for l in range(L):
                q, k, v = _qkv(rng, T)
                out = step.store_attend(l, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev))
                ref.append(slot, l, k, v)
                assert_attn_close(out, ref.attend(slot, l, q, pos), f"prefill slot {slot} pos {pos} T {T}")
            pos += T
        prompts[slot] = list(toks)
        run.publish_prefix(slot, toks)
        for i in range(len(toks) // 16):  # blocks already cached keep their first publisher's K/V
            for l in range(L):
                key = (tuple(toks[:16 * (i + 1)]), l)
                if key not in block_kv:
                    block_kv[key] = (ref.k[(slot, l)][16 * i:16 * (i + 1)].copy(),
                                     ref.v[(slot, l)][16 * i:16 * (i + 1)].copy())

    for rnd in range(6):
        free = [s for s in range(n_slots) if s not in prompts]
        for s in free[:int(rng.integers(1, len(free) + 1)) if free else 0]:
            extra = [int(t) for t in rng.integers(0, 1000, size=int(rng.integers(1, 90)))]
            toks = (base_prompt[:int(rng.choice([16, 48, 96, 160]))] if rng.random() < 0.8 else []) + extra
            prefill_prompt(s, toks)
        live = sorted(prompts)
        sharing = [s for s in live if prompts[s][:32] == base_prompt[:32]]
        for _ in range(int(rng.integers(2, 5))):
            # every live slot, or only those that started from the shared prompt (a batch whose
            # rows can share leading pages)
            batch = sharing if len(sharing) >= 2 and rng.random() < 0.5 else live
            rows = [(s, True) for s in batch] + [(int(rng.integers(0, n_slots)), False)]
            plan = Plan(tuple(s for s, _ in rows), tuple(run.length(s) if a else 0 for s, a in rows),
                        tuple(a for _, a in rows))
            step = run.begin_decode(plan)
            seen["shared_steps"] += step.shared_prefix is not None
            for l in range(L):
                q, k, v = _qkv(rng, len(rows))
                out = step.store_attend(l, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev))
                for i, (s, a) in enumerate(rows):
                    if not a:
                        continue
                    ref.append(s, l, k[i:i + 1], v[i:i + 1])
                    assert_attn_close(out[i:i + 1], ref.attend(s, l, q[i], None)[None], f"decode round {rnd} slot {s}")
            for s, a in rows:
                if a:
                    prompts[s] = prompts[s] + [-1]  # decoded tokens never match a prompt
        for s in list(prompts)[:int(rng.integers(1, 3))]:
            run.clear_slot(s, zero=bool(rng.random() < 0.5))
            ref.clear(s)
            del prompts[s]
        run.pool.check_invariants()
        run.prefix.check_invariants()
    # the trace went through every path: prefix-cache hits, shared-prefix decode, unaligned chunks
    assert run.prefix.stats.hit_blocks > 0 and seen["shared_steps"] > 0 and seen["unaligned_chunks"] > 0, \
        (run.prefix.stats, seen)
