"""Host-side decode routing of PagedKVRunner (no GPU): which decode path a batch takes.

A batch whose live rows start with a long common run of pages reads it once (shared-prefix
path); a batch whose rows share pages elsewhere keeps its page loads cached; otherwise the
decode streams every page.  These helpers decide it from the host block tables.
"""
import types

import numpy as np

from infurnace_amd.runner import PagedKVRunner


def _runner(block_size=16):
    return types.SimpleNamespace(block_size=block_size)


def test_any_shared_counts_only_used_entries():
    r = _runner()
    t = np.array([[1, 2, 3, 0], [4, 5, 0, 0], [6, 2, 0, 0]], np.int32)
    assert PagedKVRunner._any_shared(r, t, np.array([40, 20, 17]))      # row 2's second page is page 2
    assert not PagedKVRunner._any_shared(r, t, np.array([40, 20, 16]))  # row 2 uses one page only
    assert not PagedKVRunner._any_shared(r, t[:1], np.array([64]))      # one row never shares
    # padding entries (page 0 repeated past each row's length) are not shares
    assert not PagedKVRunner._any_shared(r, np.array([[7, 0], [8, 0]], np.int32), np.array([16, 16]))


def test_any_shared_matches_brute_force():
    rng = np.random.default_rng(5)
    r = _runner()
    for _ in range(200):
        B, P = int(rng.integers(1, 6)), int(rng.integers(1, 9))
        t = rng.integers(0, 12, size=(B, P)).astype(np.int32)
        lens = rng.integers(0, P * 16 + 1, size=B)
        used = [list(t[b, :-(-int(lens[b]) // 16)]) for b in range(B)]
        flat = [p for u in used for p in u]
        assert PagedKVRunner._any_shared(r, t, lens) == (B >= 2 and len(set(flat)) != len(flat))


def test_common_pages_is_the_common_leading_run():
    r = _runner()
    t = np.array([[9, 8, 7, 1], [9, 8, 6, 2], [9, 8, 7, 3]], np.int32)
    assert PagedKVRunner._common_pages(r, t, np.array([64, 64, 64])).tolist() == [9, 8]
    # limited to pages complete in every row
    assert PagedKVRunner._common_pages(r, t, np.array([64, 20, 64])).tolist() == [9]
