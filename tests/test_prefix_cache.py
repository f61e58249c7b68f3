"""Prefix cache (docs/roadmap.md:442-470 Phase 8 gates; docs/architecture.md:381-391):
only complete blocks are published, identity includes the namespace and the whole token
history, hash matches are verified (forced collisions cannot select unrelated tokens),
references stay valid under cancellation / eviction / in-flight work, eviction is
deterministic (LRU leaves with no other owner), and a namespace change invalidates."""
import random

import numpy as np
import pytest

from infurnace_amd.cache import BlockPool, KVManager, PrefixCache, PrefixCacheError


def _fill(mgr, seq, n):
    """Append n tokens to a sequence; returns its pages."""
    mgr.append(seq, n)
    return mgr.blocks(seq)


def test_publish_complete_blocks_only_and_lookup_longest_prefix():
    pool = BlockPool(32)
    mgr = KVManager(pool)
    pc = PrefixCache(pool, ("qwen3-0.6b", "fp16", 1e6))
    toks = list(range(100, 140))                    # 40 tokens: 2 complete blocks + 8
    mgr.add_sequence("a")
    pages = _fill(mgr, "a", 40)
    assert pc.insert(toks, pages) == 2              # the partial third block is never published
    assert len(pc) == 2
    assert pc.lookup(toks) == (pages[:2], 32)
    assert pc.lookup(toks[:31]) == (pages[:1], 16)  # only complete blocks match
    assert pc.lookup(toks[:16] + [0] * 16) == (pages[:1], 16)  # diverges inside block 2
    assert pc.lookup([7] + toks[1:]) == ([], 0)     # diverges in block 1: nothing
    assert pc.insert(toks, pages) == 0              # already cached
    pc.check_invariants()
    pool.check_invariants()


def test_namespace_and_history_are_part_of_identity():
    pool = BlockPool(32)
    mgr = KVManager(pool)
    a = PrefixCache(pool, ("ckpt-A", 1e6))
    b = PrefixCache(pool, ("ckpt-A", 5e5))          # different RoPE base: different KV values
    toks = list(range(32))
    mgr.add_sequence(0)
    pages = _fill(mgr, 0, 32)
    a.insert(toks, pages)
    assert b.lookup(toks) == ([], 0)
    # the same second block after a different first block is a different identity
    other = [999] * 16 + toks[16:]
    assert a.lookup(other) == ([], 0)


def test_forced_collisions_never_select_unrelated_tokens():
    pool = BlockPool(64)
    mgr = KVManager(pool)
    pc = PrefixCache(pool, "ns", hasher=lambda b: b"\0")   # every digest collides
    rng = random.Random(3)
    truth = {}
    for s in range(6):
        toks = [rng.randrange(50) for _ in range(48)]
        mgr.add_sequence(s)
        pages = _fill(mgr, s, 48)
        pc.insert(toks, pages)
        for i in range(3):
            truth[pages[i]] = tuple(toks[: (i + 1) * 16])
    for _ in range(200):
        toks = [rng.randrange(50) for _ in range(48)]
        if rng.random() < 0.5:                           # re-query a known history, maybe perturbed
            toks = list(rng.choice(list(truth.values()))) + [0] * 48
            toks = toks[:48]
            if rng.random() < 0.5:
                toks[rng.randrange(48)] += 1
        pages, n = pc.lookup(toks)
        for i, p in enumerate(pages):
            assert truth[p] == tuple(toks[: (i + 1) * 16]), "a lookup returned a page holding other tokens"
    assert pc.stats.collisions > 0
    pc.check_invariants()


def test_references_survive_cancellation_and_in_flight_work():
    pool = BlockPool(16)
    mgr = KVManager(pool)
    pc = PrefixCache(pool, "ns")
    toks = list(range(48))
    mgr.add_sequence("x")
    pages = _fill(mgr, "x", 48)
    pc.insert(toks, pages)
    pool.mark_in_flight(pages[:1])
    mgr.free_sequence("x")                    # cancellation: the cache still owns all 3 pages
    assert all(not pool.is_free(p) for p in pages)
    hit, n = pc.lookup(toks)
    mgr.add_sequence("y", prefix_blocks=hit, prefix_len=n)   # a hit shares the pages
    assert pc.evict(10) == []                 # every entry is protected (active "y" and in-flight)
    mgr.free_sequence("y")
    freed = pc.evict(10)                      # leaves first: pages[2], pages[1]; pages[0] is in flight
    assert sorted(freed) == sorted(pages[1:]) and len(pc) == 1
    assert pool.release_in_flight(pages[:1]) == []   # the cache still holds page 0
    assert pc.evict(1) == pages[:1]
    pool.check_invariants()
    assert pool.num_free == pool.capacity


def test_capacity_eviction_is_lru_and_deterministic():
    def run():
        pool = BlockPool(64)
        mgr = KVManager(pool)
        pc = PrefixCache(pool, "ns", capacity_blocks=6)   # three 2-block sequences
        order = []
        for s in range(5):
            toks = [s] * 32
            mgr.add_sequence(s)
            pages = _fill(mgr, s, 32)
            pc.insert(toks, pages)
            mgr.free_sequence(s)
            order.append(pages)
            if s == 2:
                pc.lookup([0] * 32)           # touch sequence 0: it becomes most recent
        return pc, order, pool
    pc, order, pool = run()
    assert len(pc) == 6
    # sequence 0 was touched after 2 was inserted, so 1 and 2 were the least recently used
    assert [pc.lookup([s] * 32)[1] for s in range(5)] == [32, 0, 0, 32, 32]
    pc2, order2, _ = run()
    assert [pc2.lookup([s] * 32)[1] for s in range(5)] == [pc.lookup([s] * 32)[1] for s in range(5)]
    pool.check_invariants()


def test_invalidate_on_reload_releases_only_cache_references():
    pool = BlockPool(16)
    mgr = KVManager(pool)
    pc = PrefixCache(pool, "v1")
    toks = list(range(32))
    mgr.add_sequence("live")
    pages = _fill(mgr, "live", 32)
    pc.insert(toks, pages)
    assert pc.invalidate(namespace="v2") == []     # "live" still owns its pages
    assert pc.lookup(toks) == ([], 0) and len(pc) == 0
    assert mgr.free_sequence("live") == pages
    with pytest.raises(PrefixCacheError):
        pc.insert(toks, pages)                     # freed pages cannot be published
    pool.check_invariants()


@pytest.mark.parametrize("seed", range(4))
def test_randomized_sharing_trace(seed):
    rng = random.Random(seed)
    pool = BlockPool(96)
    mgr = KVManager(pool)
    pc = PrefixCache(pool, "ns", capacity_blocks=24)
    page_tokens = {}
    vocab = [list(range(b, b + 16)) for b in range(0, 80, 16)]
    live = {}
    for step in range(300):
        op = rng.random()
        if op < 0.4 and len(live) < 6:
            sid = step
            toks = [t for _ in range(rng.randint(1, 4)) for t in rng.choice(vocab)] + [rng.randrange(9)] * rng.randint(0, 15)
            hit, n = pc.lookup(toks)
            for i, p in enumerate(hit):
                assert page_tokens[p] == tuple(toks[: (i + 1) * 16])
            try:
                mgr.add_sequence(sid, prefix_blocks=hit, prefix_len=n)
                mgr.append(sid, len(toks) - n)
            except Exception:
                if sid in mgr:
                    mgr.free_sequence(sid)
                continue
            pages = mgr.blocks(sid)
            for i in range(len(toks) // 16):
                page_tokens.setdefault(pages[i], tuple(toks[: (i + 1) * 16]))
                assert page_tokens[pages[i]] == tuple(toks[: (i + 1) * 16]) or pages[i] not in hit
            live[sid] = toks
        elif op < 0.7 and live:
            sid = rng.choice(list(live))
            pc.insert(live[sid], mgr.blocks(sid))
        elif op < 0.9 and live:
            sid = rng.choice(list(live))
            del live[sid]
            for p in mgr.free_sequence(sid):
                page_tokens.pop(p, None)
        else:
            for p in pc.evict(rng.randint(1, 4)):
                page_tokens.pop(p, None)
        pc.check_invariants()
        pool.check_invariants()
