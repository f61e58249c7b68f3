"""Host page pool, block tables and slot mappings (docs/roadmap.md:325-337 Phase 5A gate:
randomized allocate / retain / release / cancel / exhaustion / stale-ID traces preserve the
allocator and ownership invariants, including atomic failure and delayed in-flight reclamation)."""
import random

import numpy as np
import pytest

from infurnace_amd.cache import (OWNERS, BlockPool, BlockPoolError, KVCacheError, KVManager, PoolExhausted,
                                 build_block_table, slot_mapping, slot_mapping_for_positions)


def test_dummy_block_is_reserved_and_never_handed_out():
    pool = BlockPool(8)
    assert pool.dummy_block == 0 and pool.capacity == 7 and pool.num_free == 7
    got = pool.allocate(7)
    assert 0 not in got and sorted(got) == list(range(1, 8))
    with pytest.raises(PoolExhausted):
        pool.allocate(1)
    for bad in (lambda: pool.free([0]), lambda: pool.retain([0])):
        with pytest.raises(BlockPoolError):
            bad()
    pool.check_invariants()


def test_allocation_is_atomic_on_exhaustion():
    pool = BlockPool(10)
    a = pool.allocate(6)
    snapshot = (pool.num_free, [pool.refcount(i) for i in range(1, 10)])
    with pytest.raises(PoolExhausted):
        pool.allocate(4)
    assert (pool.num_free, [pool.refcount(i) for i in range(1, 10)]) == snapshot
    pool.free(a)
    assert pool.num_free == 9
    pool.check_invariants()


def test_free_validates_everything_before_changing_state():
    pool = BlockPool(10)
    a = pool.allocate(3)
    with pytest.raises(BlockPoolError):
        pool.free([a[0], a[1], a[1]])  # a[1] only has one reference
    assert all(pool.refcount(i) == 1 for i in a)
    with pytest.raises(BlockPoolError):
        pool.free([a[0], 99])  # foreign id
    assert pool.refcount(a[0]) == 1
    pool.free(a)
    with pytest.raises(BlockPoolError):
        pool.free([a[0]])  # stale id: double free
    pool.check_invariants()


def test_in_flight_pages_return_only_after_release():
    pool = BlockPool(6)
    a = pool.allocate(2)
    pool.mark_in_flight(a)
    assert pool.free(a) == []          # request finished, device work still reads the pages
    assert pool.num_free == 3 and not pool.is_free(a[0])
    assert sorted(pool.release_in_flight(a)) == sorted(a)
    assert pool.num_free == 5
    pool.check_invariants()


def test_prefix_owner_keeps_shared_pages():
    pool = BlockPool(6)
    a = pool.allocate(2)
    pool.retain(a, owner="prefix")
    assert pool.refcount(a[0]) == 2 and pool.refcount(a[0], "prefix") == 1
    assert pool.free(a) == []
    assert sorted(pool.free(a, owner="prefix")) == sorted(a)
    with pytest.raises(BlockPoolError):
        pool.retain(a)  # free pages cannot be retained
    with pytest.raises(BlockPoolError):
        pool.allocate(1, owner="bogus")


def test_seeded_order_gives_non_contiguous_tables():
    order = np.random.default_rng(0).permutation(64)
    pool = BlockPool(64, order=order, reserve_dummy=False)
    assert pool.allocate(5) == [int(x) for x in order[:5]]
    with pytest.raises(BlockPoolError):
        BlockPool(4, order=[0, 1, 1, 2])


@pytest.mark.parametrize("seed", range(6))
def test_randomized_trace_matches_brute_force_model(seed):
    rnd = random.Random(seed)
    n = 40
    pool = BlockPool(n, reserve_dummy=bool(seed % 2))
    model = {o: {} for o in OWNERS}  # owner -> {page: count}
    free = set(range(n)) - ({pool.dummy_block} if pool.dummy_block is not None else set())
    live = []  # pages with at least one owner
    for _ in range(600):
        op = rnd.random()
        if op < 0.35:
            k = rnd.randint(0, 6)
            owner = rnd.choice(["active", "prefix"])
            if k > len(free):
                with pytest.raises(PoolExhausted):
                    pool.allocate(k, owner)
            else:
                got = pool.allocate(k, owner)
                assert len(set(got)) == k and set(got) <= free
                for p in got:
                    free.discard(p)
                    model[owner][p] = 1
                    live.append(p)
        elif op < 0.55 and live:
            p = rnd.choice(live)
            owner = rnd.choice(OWNERS)
            pool.retain([p], owner)
            model[owner][p] = model[owner].get(p, 0) + 1
        elif op < 0.9 and live:
            p = rnd.choice(live)
            owner = rnd.choice(OWNERS)
            if model[owner].get(p, 0) == 0:
                with pytest.raises(BlockPoolError):
                    pool.free([p], owner)
            else:
                model[owner][p] -= 1
                released = pool.free([p], owner)
                if all(model[o].get(p, 0) == 0 for o in OWNERS):
                    assert released == [p]
                    free.add(p)
                    live = [x for x in live if x != p]
                else:
                    assert released == []
        else:
            # stale / foreign ids are rejected without side effects
            bad = rnd.choice([n, -1, n + 5])
            with pytest.raises(BlockPoolError):
                pool.free([bad])
        assert pool.num_free == len(free)
        for p in range(n):
            if p == pool.dummy_block:
                continue
            assert pool.refcount(p) == sum(model[o].get(p, 0) for o in OWNERS)
        pool.check_invariants()


def test_block_table_and_slot_mapping_closed_form():
    table = build_block_table([[5, 9], [3], [7, 1, 2]], pad=0)
    assert table.dtype == np.int32 and table.tolist() == [[5, 9, 0], [3, 0, 0], [7, 1, 2]]
    seq = np.array([0, 0, 2, 2, 1])
    pos = np.array([0, 17, 33, 15, 4])
    assert slot_mapping(table, seq, pos).tolist() == [80, 9 * 16 + 1, 2 * 16 + 1, 7 * 16 + 15, 52]
    walk = [p * 16 + o for p in [7, 1, 2] for o in range(16)]
    assert slot_mapping_for_positions([7, 1, 2], 10, 30).tolist() == walk[10:40]
    with pytest.raises(BlockPoolError):
        slot_mapping(table, [0], [48])
    with pytest.raises(BlockPoolError):
        build_block_table([[1, 2, 3]], max_pages=2)


def test_kv_manager_append_atomic_across_sequences_and_free():
    pool = BlockPool(10)  # 9 usable pages
    mgr = KVManager(pool, max_pages_per_seq=8)
    mgr.add_sequence("a")
    mgr.add_sequence("b")
    sa = mgr.append("a", 20)            # 2 pages
    assert sa.tolist() == [mgr.blocks("a")[p // 16] * 16 + p % 16 for p in range(20)]
    state = (pool.num_free, mgr.length("a"), mgr.length("b"))
    with pytest.raises(PoolExhausted):  # a needs 1 more page, b needs 7: 8 > 7 free
        mgr.append_batch(["a", "b"], [13, 100])
    assert (pool.num_free, mgr.length("a"), mgr.length("b")) == state
    sa2, sb = mgr.append_batch(["a", "b"], [13, 16])
    assert len(sa2) == 13 and len(sb) == 16 and mgr.length("a") == 33
    table = mgr.block_tables(["a", "b"])
    assert table.shape == (2, 3) and table[1, 1] == pool.dummy_block
    assert mgr.seq_lens(["a", "b"]).tolist() == [33, 16]
    with pytest.raises(KVCacheError):
        mgr.append("a", 16 * 8)          # beyond max_pages_per_seq
    released = mgr.free_sequence("a")
    assert len(released) == 3 and "a" not in mgr
    pool.check_invariants()


def test_kv_manager_shared_prefix_and_page_churn():
    pool = BlockPool(64)
    mgr = KVManager(pool)
    mgr.add_sequence("root")
    mgr.append("root", 64)              # 4 full pages: the shared prefix
    prefix = mgr.blocks("root")
    for s in range(3):
        mgr.add_sequence(s, prefix_blocks=prefix, prefix_len=64)
        mgr.append(s, 40)
    assert all(pool.refcount(p) == 4 for p in prefix)
    t = mgr.block_tables([0, 1, 2])
    assert (t[:, :4] == np.asarray(prefix)).all()
    with pytest.raises(KVCacheError):
        mgr.replace_blocks(0, [0])       # shared prefix pages cannot be churned
    old = mgr.blocks(1)[5]
    fresh = mgr.replace_blocks(1, [5])
    assert mgr.blocks(1)[5] == fresh[0] != old and pool.is_free(old)
    with pytest.raises(KVCacheError):
        mgr.add_sequence(9, prefix_blocks=prefix, prefix_len=60)  # partial pages are never shared
    for s in (0, 1, 2, "root"):
        mgr.free_sequence(s)
    assert pool.num_free == pool.capacity
    pool.check_invariants()
