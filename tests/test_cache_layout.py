"""CPU tests of the host allocator (known answers of the reference's
tests/test_cache_layout.py and tests/test_prepared_layout.py)."""
import json
from pathlib import Path

import pytest

from moba_hip.cache_layout import IncrementalLayout, PageAllocator

GOLD = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())


def state(a):
    return a.tables, a.lengths, a.free_pages, a.version


def test_plans_do_not_publish_state():
    g = GOLD["allocator_plan"]
    a = PageAllocator(*g["init"])
    before = state(a)
    plan = a.plan_append(g["ids"], g["counts"])
    assert state(a) == before
    assert list(plan.token_sequences) == g["token_sequences"]
    assert list(plan.token_positions) == g["token_positions"]
    assert [list(x) for x in plan.completed_chunks] == g["completed_chunks"]
    a.commit(plan)
    assert list(a.lengths) == g["lengths_after"]
    assert list(a.tables[1][:2]) == g["table1_prefix"]
    assert list(a.tables[0][:3]) == g["table0_prefix"]
    with pytest.raises(RuntimeError, match="stale"):
        a.commit(plan)


def test_page_reuse_is_lifo_and_noncontiguous():
    g = GOLD["allocator_reuse"]
    a = PageAllocator(*g["init"])
    a.commit(a.plan_append(g["first"]["ids"], g["first"]["counts"]))
    a.reset(g["reset"])
    a.commit(a.plan_append(g["second"]["ids"], g["second"]["counts"]))
    assert list(a.tables[2][:2]) == g["table2_prefix"]
    assert a.tables[1][0] == g["table1_first"]
    assert len(a.free_pages) == g["free_after"]


def test_exhaustion_and_invalid_append_are_atomic():
    a = PageAllocator(2, 12, 3, 2, 4)
    a.commit(a.plan_append([0], [4]))
    before = state(a)
    for ids, counts in [([1], [1]), ([0], [20]), ([0, 0], [1, 1]), ([2], [1]), ([0], [0])]:
        with pytest.raises(ValueError):
            a.plan_append(ids, counts)
        assert state(a) == before
    # a huge count is refused by the length bound before anything is sized by it
    for n in (2 ** 31 - 1, 2 ** 40):
        with pytest.raises(ValueError, match="exceeds max_seq_len"):
            a.plan_append([0], [n])
        assert state(a) == before


def test_closed_chunks_follow_logical_positions():
    g = GOLD["allocator_closed_chunks"]
    a = PageAllocator(*g["init"])
    a.commit(a.plan_append([0], [g["first"]]))
    p = a.plan_append([0], [g["second"]])
    assert [list(x) for x in p.completed_chunks] == g["expected"]
    a.commit(p)
    assert a.plan_append([0], [g["third"]]).completed_chunks == ()


@pytest.mark.parametrize("p", [1, 3, 7, 16, 31])
def test_page_math_for_nondivisible_sizes(p):
    a = PageAllocator(2, 65, p, 2 * (-(-65 // p)), 24)
    a.commit(a.plan_append([0, 1], [65, 33]))
    owned = [x for row in a.tables for x in row if x >= 0]
    assert len(owned) == len(set(owned))
    assert len(owned) + len(a.free_pages) == a.num_pages
    a.reset([0, 1])
    assert len(a.free_pages) == a.num_pages and a.lengths == (0, 0)


@pytest.mark.parametrize("page", [1, 3, 7, 16])
def test_incremental_matches_transactional(page):
    old = PageAllocator(3, 41, page, 3 * (-(-41 // page)), 8)
    old.commit(old.plan_append([1, 0], [5, 7]))
    old.reset([1])
    fast = IncrementalLayout(old, [2, 0, 1])
    for _ in range(30):
        plan = fast.plan()
        snap = (tuple(map(tuple, fast.tables)), tuple(fast.lengths), tuple(fast.free))
        assert fast.plan() == plan
        assert snap == (tuple(map(tuple, fast.tables)), tuple(fast.lengths), tuple(fast.free))
        fast.commit(plan)
        old.commit(old.plan_append([2, 0, 1], [1, 1, 1]))
        assert tuple(map(tuple, fast.tables)) == old.tables
        assert tuple(fast.lengths) == old.lengths and tuple(fast.free) == old.free_pages
    fast.publish(old)
    assert list(old.lengths) == GOLD["incremental_layout"]["lengths_after_30_steps"]
    with pytest.raises(RuntimeError, match="stale"):
        fast.commit(plan)


def test_incremental_failures_do_not_mutate():
    old = PageAllocator(2, 4, 2, 1, 2)
    old.commit(old.plan_append([0], [2]))
    fast = IncrementalLayout(old, [0, 1])
    with pytest.raises(ValueError, match="pool exhausted"):
        fast.plan()
    assert fast.lengths == [2, 0] and fast.free == []
    old = PageAllocator(1, 1, 1, 1, 1)
    old.commit(old.plan_append([0], [1]))
    with pytest.raises(ValueError, match="max_seq_len"):
        IncrementalLayout(old, [0]).plan()


def test_fused_schedule_covers_every_split_once():
    """Decode split schedule: every (row, kv head) gets 1..max splits, each
    split exactly once, over a fixed grid; longer rows get more splits."""
    from moba_hip.ops.decode import fused_schedule, sched_workgroups, expected_union_tokens
    for positions, hkv, group, remote, chunk in (
            ([15883, 8359, 14466, 8938, 2711, 6290, 10424, 10009], 2, 6, 3, 512),
            ([0, 5, 31000, 2000] * 8, 1, 16, 7, 1024),
            ([3, 4], 2, 4, 2, 4)):
        entries, splits, n = fused_schedule(positions, hkv, group, remote, chunk)
        rows = len(positions) * hkv
        assert n == sched_workgroups(len(positions), hkv)
        assert len(entries) == 3 * n + rows and entries[3 * n:] == splits
        assert sum(splits) == n and all(1 <= s <= 64 for s in splits)
        seen = set()
        for w in range(n):
            r, s, c = entries[3 * w: 3 * w + 3]
            assert c == splits[r] and 0 <= s < c and (r, s) not in seen
            seen.add((r, s))
        assert len(seen) == n
        w = [expected_union_tokens(positions[r // hkv], group, remote, chunk) for r in range(rows)]
        for a in range(rows):
            for b in range(rows):
                if w[a] > 1.5 * w[b] and splits[b] < 64:
                    assert splits[a] >= splits[b]


def test_pool_c_abi_rejects_bad_ids_and_shapes():
    """The C-ABI page pool checks what a direct caller could get wrong: step
    ids outside the batch, pools of different geometry in assign, a null
    pool in the view getters.  Nothing changes on a refused call."""
    import ctypes
    import numpy as np
    from moba_hip.ops import _lib
    lib = _lib.load()
    pool, other = ctypes.c_void_p(), ctypes.c_void_p()
    assert lib.moba_pool_create(2, 32, 4, 16, 8, ctypes.byref(pool)) == 0
    assert lib.moba_pool_create(2, 32, 8, 16, 8, ctypes.byref(other)) == 0  # other page size
    try:
        ids = np.array([0, 5], dtype=np.int32)
        delta = np.zeros(4, dtype=np.int32)
        n_grants, version = ctypes.c_int(), ctypes.c_int64()
        rc = lib.moba_pool_plan_step(pool, ids.ctypes.data, 2, None, delta.ctypes.data,
                                     ctypes.byref(n_grants), ctypes.byref(version))
        assert rc == _lib.MOBA_ERR_ARG
        assert "outside cache batch slots" in lib.moba_hip_last_error().decode()
        rc = lib.moba_pool_commit_step(pool, ids.ctypes.data, 2, delta.ctypes.data, 0)
        assert rc == _lib.MOBA_ERR_ARG
        assert lib.moba_pool_assign(pool, other) == _lib.MOBA_ERR_ARG
        assert not lib.moba_pool_table(None) and not lib.moba_pool_lengths(None)
        info = (ctypes.c_int64 * 8)()
        assert lib.moba_pool_info(pool, info) == 0
        assert info[6] == 0 and info[7] == 16  # version and free pages untouched
    finally:
        lib.moba_pool_destroy(pool)
        lib.moba_pool_destroy(other)
