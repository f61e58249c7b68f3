"""In-flight page ownership of PagedKVRunner, on the host with fake completion events.

Pages referenced by submitted device work must not return to the free pool until that work has
completed (reference docs/architecture.md:255-257; the "delayed in-flight reclamation" of the
Phase 5A/5D gates, docs/roadmap.md:331-337,356-359).  The runner marks a step's pages in flight
when the step begins, records an event after each launch, and releases the pages once the step
is closed (a later step began) and its event has completed.  Here the events are controlled by
the test and no kernel runs (the pool lives in host memory).
"""
from collections import namedtuple

import numpy as np
import pytest

from infurnace_amd.cache import PoolExhausted
from infurnace_amd.runner import PagedKVRunner, RunnerError

Plan = namedtuple("Plan", "slots positions active_mask")


class FakeEvent:
    """A completion event the test completes by hand (synchronize() completes it, as a wait would)."""
    created = []

    def __init__(self):
        self.done = False
        self.records = 0
        FakeEvent.created.append(self)

    def record(self, stream=None):
        self.records += 1
        self.done = False

    def query(self):
        return self.done

    def synchronize(self):
        self.done = True


def _runner(num_blocks=6, slots=3):
    FakeEvent.created = []
    return PagedKVRunner(1, num_slots=slots, max_context=64, num_kv_heads=2, head_dim=8, num_blocks=num_blocks,
                         device="cpu", event_factory=FakeEvent)


def test_cleared_pages_stay_allocated_while_their_work_runs():
    run = _runner()
    st = run.begin_prefill(0, 0, 32)          # 2 pages
    st._launched()                             # a kernel was submitted
    pages = run.mgr.blocks(0)
    assert run.clear_slot(0) == []             # the step still reads / writes them
    assert all(not run.pool.is_free(p) for p in pages)
    assert run.pages_in_flight == 2
    # a later step closes the first one; its event has not completed: still held
    run.begin_prefill(1, 0, 16)
    assert all(not run.pool.is_free(p) for p in pages)
    st.event.done = True
    released = run.reclaim()
    assert sorted(released) == sorted(pages)
    assert all(run.pool.is_free(p) for p in pages)
    run.pool.check_invariants()


def test_open_step_is_not_released_even_when_its_event_completed():
    run = _runner()
    st = run.begin_prefill(0, 0, 16)
    st._launched()
    st.event.done = True
    assert run.reclaim() == [] and run.pages_in_flight == 1   # open: it may still take launches
    run.begin_prefill(1, 0, 16)                # closes it; its event completed -> released now
    assert run.pages_in_flight == 1            # only the new step's page
    with pytest.raises(RunnerError):
        st.store_attend(0, None, None, None)   # a closed step takes no further launches
    st2 = run._inflight[-1]
    st2._launched()
    run.clear_slot(0)                          # clearing a slot closes the open step too
    assert st2.closed


def test_freed_page_is_not_reallocated_before_completion():
    run = _runner(num_blocks=4)                # 3 allocatable pages
    st = run.begin_prefill(0, 0, 48)           # all 3 pages
    st._launched()
    held = set(run.mgr.blocks(0))
    run.clear_slot(0)
    assert run.pool.num_free == 0
    # allocation would need a held page: the runner waits for the running work, then reuses it
    st2 = run.begin_prefill(1, 0, 16)
    assert st.event.done                       # it waited (synchronize)
    assert set(run.mgr.blocks(1)) <= held
    st2._launched()
    run.pool.check_invariants()


def test_exhaustion_without_inflight_work_raises():
    run = _runner(num_blocks=3)
    run.begin_prefill(0, 0, 32)
    run.synchronize()
    with pytest.raises(PoolExhausted):
        run.begin_prefill(1, 0, 16)


def test_decode_step_holds_every_live_rows_pages_and_zeroes_on_release(monkeypatch):
    run = _runner(num_blocks=16)
    zeroed = []
    monkeypatch.setattr(run.cache, "clear_pages", lambda ids: zeroed.append(sorted(int(i) for i in ids)))
    for s, n in ((0, 20), (1, 40)):
        run.begin_prefill(s, 0, n)._launched()
    run.synchronize()
    st = run.begin_decode(Plan((0, 1, 2), (20, 40, 0), (True, True, False)))
    st._launched()
    expect = set(run.mgr.blocks(0)) | set(run.mgr.blocks(1))
    assert set(st.pages.tolist()) == expect    # both live rows' pages, padding row none
    owned0 = run.mgr.blocks(0)
    assert run.clear_slot(0, zero=True) == []  # in flight: neither freed nor zeroed yet
    assert zeroed == []
    run.synchronize()
    assert zeroed == [sorted(owned0)]          # zeroed when released
    assert all(run.pool.is_free(p) for p in owned0)
    run.pool.check_invariants()


def test_randomized_trace_never_reuses_an_inflight_page():
    """Random prefill / decode / clear sequences: a page held by uncompleted work is never handed out."""
    rng = np.random.default_rng(0)
    run = _runner(num_blocks=24, slots=4)
    lens = {}
    live_steps = []
    for it in range(400):
        op = rng.integers(0, 4)
        if op == 0:
            s = int(rng.integers(0, 4))
            n = int(rng.integers(1, 20))
            start = lens.get(s, 0)
            if start + n > 64:
                continue
            try:
                st = run.begin_prefill(s, start, n)
            except (PoolExhausted, RunnerError):
                continue
            lens[s] = start + n
        elif op == 1 and lens:
            s = [x for x in lens if lens[x] < 64]
            if not s:
                continue
            try:
                st = run.begin_decode(Plan(tuple(s), tuple(lens[x] for x in s), (True,) * len(s)))
            except (PoolExhausted, RunnerError):
                continue
            for x in s:
                lens[x] += 1
        elif op == 2 and lens:
            s = list(lens)[int(rng.integers(0, len(lens)))]
            run.clear_slot(s)
            del lens[s]
            continue
        else:
            for ev in FakeEvent.created:
                if rng.random() < 0.5:
                    ev.done = True
            run.reclaim()
            continue
        st._launched()
        live_steps.append(st)
        # invariant: every page of a step whose work has not completed is allocated
        for old in live_steps:
            if old.event is not None and not old.event.done and old.pages is not None:
                assert all(not run.pool.is_free(int(p)) for p in old.pages)
        live_steps = [o for o in live_steps if o.event is None or not o.event.done]
        run.pool.check_invariants()
