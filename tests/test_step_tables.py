"""Per-step block tables (host C++, no GPU): the scheduler's reservation loop
(src/scheduler/scheduler.rs:422-449) and the change-only upload plan.

A mirror of the device tables is updated from nothing but the pending
(row, col, page) triples of each step; after every step its valid entries
must equal the block manager's block tables, whatever the joins, growth,
forks, failures and releases in between. The GPU test in test_gpu_kv.py
runs the same plan through rlse_st_upload into device memory.
"""
import random

import numpy as np
import pytest


def test_growth_follows_the_scheduler_loop(kv):
    """A sequence grows by a block exactly when blocks_needed(next_len)
    exceeds the blocks it holds (scheduler.rs:427-433); one triple per page
    added, the whole row for a request new to its row."""
    bm = kv.BlockManager(64)
    st = kv.StepTables(4, 16)
    bm.allocate("a", 15)                   # 1 block
    bm.allocate("b", 40)                   # 3 blocks
    assert st.prepare(bm, ["a", "b"], [16, 41]) == [0, 0]
    assert len(bm.block_table("a")) == 1 and len(bm.block_table("b")) == 3
    tables, lens, batch, pend = st.host()
    assert batch == 2 and list(lens[:2]) == [16, 41]
    assert sorted(map(tuple, pend.tolist())) == sorted(
        [(0, 0, bm.block_table("a")[0])] + [(1, j, p) for j, p in enumerate(bm.block_table("b"))])
    st.mark_uploaded()
    assert st.prepare(bm, ["a", "b"], [17, 42]) == [0, 0]   # a crosses into block 2
    assert len(bm.block_table("a")) == 2
    _, lens, _, pend = st.host()
    assert pend.tolist() == [[0, 1, bm.block_table("a")[1]]]
    assert list(lens[:2]) == [17, 42]
    st.mark_uploaded()
    assert st.prepare(bm, ["a", "b"], [18, 43]) == [0, 0]   # no new block: nothing to send
    assert len(st.host()[3]) == 0
    st.mark_uploaded()
    # Rows swap (the scheduler's swap_remove reorders its list): both rows resent.
    assert st.prepare(bm, ["b", "a"], [44, 19]) == [0, 0]
    assert len(st.host()[3]) == 3 + 2
    st.mark_uploaded()
    st.reset()
    assert st.prepare(bm, ["b", "a"], [44, 19]) == [0, 0]
    assert len(st.host()[3]) == 3 + 2


def test_a_sequence_that_cannot_grow_is_released(kv):
    """scheduler.rs:438-443: a failed reservation drops the sequence and
    releases its blocks; the others keep their rows. Unknown ids and lengths
    past the table width are refused per row."""
    bm = kv.BlockManager(4)
    st = kv.StepTables(4, 8)
    bm.allocate("a", 16)
    bm.allocate("b", 32)
    bm.allocate("c", 16)   # every block in use
    status = st.prepare(bm, ["a", "b", "c", "zz"], [16, 33, 16, 5])
    assert status == [0, kv.ERR_CACHE_PRESSURE, 0, kv.ERR_UNKNOWN_REQUEST]
    _, lens, batch, _ = st.host()
    assert list(lens[:4]) == [16, 0, 16, 0] and batch == 4
    assert bm.free_count() == 2              # b's two blocks came back
    with pytest.raises(kv.RlseError):
        bm.block_table("b")
    assert st.prepare(bm, ["a"], [16 * 8 + 1]) == [kv.ERR_INVALID_VALUE]  # 9 blocks > 8
    assert bm.release_all() == 2 and bm.free_count() == 4
    with pytest.raises(kv.RlseError):
        st.prepare(bm, ["a"] * 5, [1] * 5)   # batch > max_batch


def test_change_only_plan_keeps_a_device_mirror_exact(kv):
    """300 random steps of joins, growth, forks, failures and finishes: the
    mirror built from triples alone equals every live row's block table."""
    rnd = random.Random(3)
    bm = kv.BlockManager(160)
    B, W = 12, 40
    st = kv.StepTables(B, W)
    mirror = np.full((B, W), -7, np.int32)
    live, nid, sent_total, full_total = {}, 0, 0, 0
    order, dev_row = [], [None] * B   # dev_row[i]: the request whose pages row i holds
    for step in range(300):
        # Joins and forks (the scheduler admits new sequences between steps).
        while len(order) < B and rnd.random() < 0.4:
            rid = f"r{nid}"
            nid += 1
            if order and rnd.random() < 0.3:
                parent = rnd.choice(order)
                n = rnd.randint(1, live[parent])
                try:
                    bm.fork(parent, rid, n)
                except kv.CachePressure:
                    continue
                live[rid] = n
            else:
                n = rnd.randint(1, 200)
                try:
                    bm.allocate(rid, n)
                except kv.CachePressure:
                    continue
                live[rid] = n
            order.append(rid)
        if rnd.random() < 0.2 and len(order) > 1:   # swap_remove of a finished one
            i = rnd.randrange(len(order))
            bm.release(order[i])
            del live[order[i]]
            order[i] = order[-1]
            order.pop()
        pages_before = {r: len(bm.block_table(r)) for r in order}
        next_lens = [min(live[r] + 1, W * 16) for r in order]
        status = st.prepare(bm, order, next_lens)
        tables, lens, batch, pend = st.host()
        for row, col, page in pend.tolist():
            mirror[row, col] = page
        per_row = np.bincount(pend[:, 0], minlength=B) if len(pend) else np.zeros(B, int)
        sent_total += len(pend)
        st.mark_uploaded()
        assert batch == len(order)
        keep = []
        for i, (r, s_) in enumerate(zip(order, status)):
            if s_ != 0:
                assert s_ == kv.ERR_CACHE_PRESSURE and lens[i] == 0 and per_row[i] == 0
                del live[r]
                continue
            live[r] = next_lens[i]
            bt = bm.block_table(r)
            assert len(bt) == max(bm.blocks_needed(next_lens[i]), pages_before[r])
            assert list(mirror[i, :len(bt)]) == bt == list(tables[i, :len(bt)])
            assert lens[i] == next_lens[i]
            expected = len(bt) - pages_before[r] if dev_row[i] == r else len(bt)
            assert per_row[i] == expected, (step, i, r)
            dev_row[i] = r
            full_total += len(bt)
            keep.append(r)
        order = keep
    assert sent_total < 0.2 * full_total, (sent_total, full_total)
    bm.release_all()
    assert bm.free_count() == 160


def test_reprepared_rows_leave_one_page_per_cell(kv):
    """A step abandoned after prepare and prepared again (no upload between)
    must not leave two pending triples for one (row, col): a row that
    restarts -- another request now sits in it -- supersedes its earlier
    pending triples, and one upload applies exactly the latest pages."""
    bm = kv.BlockManager(64)
    st = kv.StepTables(3, 8)
    for r, n in (("a", 40), ("b", 20), ("c", 70)):
        bm.allocate(r, n)
    st.prepare(bm, ["a", "b", "c"], [41, 21, 71])
    # abandoned: row 0 now holds c, row 1 a, row 2 b (no upload in between)
    st.prepare(bm, ["c", "a", "b"], [71, 41, 22])
    _, _, batch, pend = st.host()
    cells = [(int(r), int(c)) for r, c, _ in pend.tolist()]
    assert len(cells) == len(set(cells)), "two pages pending for one cell"
    mirror = {}
    for row, col, page in pend.tolist():
        mirror[(row, col)] = page
    for i, r in enumerate(["c", "a", "b"]):
        bt = bm.block_table(r)
        assert [mirror[(i, j)] for j in range(len(bt))] == bt
    # the same request prepared twice keeps its first triples and adds the growth
    st.mark_uploaded()
    st.prepare(bm, ["c", "a", "b"], [81, 41, 22])
    st.prepare(bm, ["c", "a", "b"], [97, 41, 22])
    _, _, _, pend = st.host()
    cells = [(int(r), int(c)) for r, c, _ in pend.tolist()]
    assert len(cells) == len(set(cells))
    assert sorted(c for r, c in cells if r == 0) == list(range(5, 7))
    assert [p for r, c, p in sorted(pend.tolist()) if r == 0] == bm.block_table("c")[5:7]
