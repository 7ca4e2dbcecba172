"""Tensor memory budget with page-based KV charges (host C++, no GPU).

The budget restates TensorMemoryBudget (src/cache/tensor_memory.rs:41-125);
the first two tests restate tests/test_tensor_memory.rs:9-58 and :113-146
with pages in place of contiguous snapshot copies. The page charges replace
the contiguous-capacity KV term of memory_charge (src/backends/candle.rs:
241-282): a request is charged for the pages it holds, a shared prefix page
once, and a page held only by prefix-cache chunks as retained prefix.
"""
import threading

import pytest


def test_budget_creation_and_leases(kv):
    """tensor_memory.rs tests: invalid budgets, 16 racing leases of 25 bytes on
    100 available bytes (exactly 4 fit), a prefix lease, an overflowing charge."""
    for budget, headroom in [(0, 0), (100, 100), (100, 200)]:
        with pytest.raises(kv.RlseError):
            kv.MemoryBudget(budget, headroom)
    mb = kv.MemoryBudget(108, 8)
    start, seen = threading.Barrier(16), threading.Barrier(16)
    leases, peaks = [None] * 16, [None] * 16

    def worker(i):
        start.wait()
        leases[i] = mb.try_reserve(active_kv=20, execution=5)
        seen.wait()  # every lease that fit is still held here
        peaks[i] = mb.stats().reserved_bytes
        start.wait()

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(16)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    won = [l for l in leases if l is not None]
    assert len(won) == 4 and len(set(won)) == 4
    assert peaks == [108] * 16
    st = mb.stats()
    assert (st.active_kv_reserved_bytes, st.execution_reserved_bytes) == (80, 20)
    assert st.available_bytes == 0 and st.peak_reserved_bytes == 108
    for l in won:
        mb.release(l)
    assert mb.stats().reserved_bytes == 8
    lease = mb.try_reserve(prefix=32)
    assert mb.stats().prefix_retained_bytes == 32
    mb.release(lease)
    st = mb.stats()
    assert st.available_bytes == 100 and st.prefix_retained_bytes == 0
    assert mb.try_reserve(active_kv=2**63 - 1, execution=1) is None
    with pytest.raises(kv.RlseError):
        mb.release(lease)  # released twice
    assert mb.stats().rejections == 0  # try_reserve itself records none


PAGE = 100


def _setup(kv, blocks=16, budget=1064, headroom=64, chunk=16):
    mb = kv.MemoryBudget(budget, headroom)
    bm = kv.BlockManager(blocks)
    bm.attach_budget(mb, PAGE)
    pc = kv.PrefixCache(bm, chunk_size=chunk, max_chunks=8)
    return mb, bm, pc


def _close(pc, bm, mb):
    pc.close()
    bm.close()
    assert mb.stats().reserved_bytes == mb.stats().headroom_bytes
    mb.close()


def test_admission_evicts_prefixes_and_cannot_reclaim_borrowed_pages(kv):
    """test_tensor_memory.rs:113-146 with pages: reserve_memory evicts LRU
    chunks until a charge fits; pages a live request still shares stay
    charged, so the eviction frees nothing and the admission is rejected."""
    mb, bm, pc = _setup(kv)
    prompt = list(range(32))
    bm.allocate("r", 32)                          # two pages
    pc.insert_kv(prompt, "r")                     # chunks [0,16) and [0,32)
    assert mb.stats().active_kv_reserved_bytes == 2 * PAGE
    bm.release("r")                               # now held only by the cache
    st = mb.stats()
    assert (st.active_kv_reserved_bytes, st.prefix_retained_bytes) == (0, 2 * PAGE)
    assert pc.fork(prompt, 32, "child") == []     # the borrower shares both pages
    st = mb.stats()
    assert (st.active_kv_reserved_bytes, st.prefix_retained_bytes) == (2 * PAGE, 0)
    with pytest.raises(kv.CachePressure, match="Tensor memory budget exhausted"):
        pc.reserve_memory(active_kv=600, execution=300)  # 900 > 800 available
    assert pc.stats().kv_evictions == 2 and pc.stats().chunks == 0
    st = mb.stats()
    assert st.active_kv_reserved_bytes == 2 * PAGE and st.rejections == 1
    bm.release("child")                           # the last holder: pages freed
    assert mb.stats().reserved_bytes == 64
    lease = pc.reserve_memory(active_kv=600, execution=300)
    st = mb.stats()
    assert (st.active_kv_reserved_bytes, st.execution_reserved_bytes) == (600, 300)
    # A new prefix is retained while it fits; reclaim evicts it under pressure.
    bm.allocate("r2", 16)
    pc.insert_kv(prompt[:16], "r2")
    bm.release("r2")
    assert mb.stats().prefix_retained_bytes == PAGE
    assert mb.stats().reserved_bytes <= 1064
    with pytest.raises(kv.CachePressure):
        pc.reclaim(2)  # 2 pages need 200 bytes; only 100 are left after eviction
    assert pc.stats().chunks == 0 and mb.stats().prefix_retained_bytes == 0
    mb.release(lease)
    pc.reclaim(2)
    assert mb.stats().peak_reserved_bytes <= mb.stats().budget_bytes
    _close(pc, bm, mb)


def test_page_charges_follow_allocation_fork_and_release(kv):
    """The KV charge is the pages held, not the contiguous capacity: growth
    by allocate_block, a fork sharing full pages (charged once) plus a
    copy-on-write page, release of a parent whose pages a child keeps."""
    mb, bm, pc = _setup(kv, budget=564)  # 500 available: 5 pages
    bm.allocate("p", 40)                                  # 3 pages
    assert mb.stats().active_kv_reserved_bytes == 3 * PAGE
    bm.allocate_block("p")                                # 4 pages
    assert mb.stats().active_kv_reserved_bytes == 4 * PAGE
    cow = bm.fork("p", "c", 40)                           # 2 shared + 1 copy-on-write
    assert len(cow) == 1
    assert mb.stats().active_kv_reserved_bytes == 5 * PAGE
    st_before, free_before = mb.stats(), bm.free_count()
    with pytest.raises(kv.CachePressure, match="Tensor memory budget exhausted"):
        bm.allocate_block("c")                            # a 6th page does not fit
    with pytest.raises(kv.CachePressure):
        bm.allocate("q", 1)
    st = mb.stats()
    assert bm.free_count() == free_before and st.reserved_bytes == st_before.reserved_bytes
    assert st.rejections == st_before.rejections + 2
    assert bm.block_table("c") == bm.block_table("p")[:2] + [cow[0][1]]
    bm.release("p")                                       # the child keeps 3 pages
    assert mb.stats().active_kv_reserved_bytes == 3 * PAGE
    bm.release("c")
    assert mb.stats().reserved_bytes == 64
    # Attaching charges pages already held; detaching uncharges them.
    bm2 = kv.BlockManager(8)
    bm2.allocate("x", 33)
    bm2.attach_budget(mb, PAGE)
    assert mb.stats().active_kv_reserved_bytes == 3 * PAGE
    with pytest.raises(kv.CachePressure):
        bm2.attach_budget(kv.MemoryBudget(200, 1), PAGE)  # 300 bytes do not fit
    assert mb.stats().active_kv_reserved_bytes == 3 * PAGE  # still attached to mb
    bm2.attach_budget(None)
    assert mb.stats().active_kv_reserved_bytes == 0
    bm2.attach_budget(mb, PAGE)
    bm2.close()                                           # destroy uncharges
    assert mb.stats().reserved_bytes == 64
    _close(pc, bm, mb)


QWEN3_06B = dict(num_layers=28, num_heads=16, num_kv_heads=8, head_dim=128, hidden_size=1024,
                 intermediate_size=3072, vocab_size=151936, dtype_bytes=2, context_length=40960,
                 block_size=16)


def test_memory_charge(kv):
    """memory_charge for paged KV on the Qwen3-0.6B shape in bf16. Constants
    worked out by hand from the terms of candle.rs:257-271 (P=512, T=640):
    page 2*28*8*128*16*2; attention 8*16*512*640*4; hidden 16*1024*512*2;
    mlp 8*3072*512*2; decode 8*16*640*128*2; logits 16*151936*4."""
    shape = kv.ModelShape(**QWEN3_06B)
    kvb, ex, page = kv.memory_charge(shape, 512, 128)
    assert page == 1_835_008
    assert kvb == 40 * 1_835_008 == 73_400_320  # = the contiguous 2*L*Hkv*d*T*B at T=640
    assert ex == 167_772_160 + 16_777_216 + 25_165_824 + 20_971_520 + 9_723_904
    kvb, _, _ = kv.memory_charge(shape, 512, 138)  # T = 650: whole pages, 41 of them
    assert kvb == 41 * 1_835_008
    for prompt, mx in [(0, 8), (8, 0), (40000, 961)]:
        with pytest.raises(kv.TokenLimitExceeded, match="exceeds model context"):
            kv.memory_charge(shape, prompt, mx)
    kv.memory_charge(shape, 40000, 960)  # exactly the context: admitted
    big = kv.ModelShape(**dict(QWEN3_06B, context_length=2**31 - 1, hidden_size=2**31 - 1,
                               vocab_size=2**31 - 1, intermediate_size=2**31 - 1))
    with pytest.raises(kv.CachePressure, match="overflows"):
        kv.memory_charge(big, 2**30, 2**30 - 1)  # T = the context; the products overflow
    with pytest.raises(kv.RlseError):
        kv.memory_charge(kv.ModelShape(**dict(QWEN3_06B, head_dim=0)), 1, 1)


def test_workers_sharing_a_budget_never_overdraw_it(kv):
    """Eight block managers (one per worker) charge pages to one budget from
    eight threads until it refuses: every page is charged exactly once and
    the budget never goes past its limit."""
    mb = kv.MemoryBudget(64 + 37 * PAGE, 64)  # room for 37 pages, shared
    bms = [kv.BlockManager(64) for _ in range(8)]
    for bm in bms:
        bm.attach_budget(mb, PAGE)
    start = threading.Barrier(8)
    held = [0] * 8

    def worker(i):
        start.wait()
        while True:
            try:
                bms[i].allocate_block(f"w{i}")
            except kv.CachePressure:
                return
            held[i] += 1

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    st = mb.stats()
    assert sum(held) == 37
    assert st.active_kv_reserved_bytes == 37 * PAGE and st.available_bytes == 0
    assert st.peak_reserved_bytes == st.budget_bytes and st.rejections == 8
    for bm in bms:
        bm.close()
    assert mb.stats().reserved_bytes == 64


def test_random_operations_keep_page_classes_exact(kv):
    """Random allocate / grow / fork / release / insert_kv / cache fork /
    eviction: after every step the active-KV charge is PAGE x the pages in
    live requests' block tables and the retained-prefix charge is PAGE x the
    other allocated pages (held only by cache chunks)."""
    import random
    rnd = random.Random(7)
    mb, bm, pc = _setup(kv, blocks=48, budget=64 + 40 * PAGE, chunk=16)
    live, inserted, nid, restored = {}, [], 0, 0
    for step in range(600):
        op = rnd.choice(["alloc", "grow", "fork", "release", "insert", "restore", "reclaim"])
        try:
            if op == "alloc":
                n = rnd.randint(1, 70)
                bm.allocate(f"r{nid}", n)
                live[f"r{nid}"] = [rnd.randrange(1000) for _ in range(n)]
                nid += 1
            elif op == "grow" and live:
                r = rnd.choice(sorted(live))
                if len(live[r]) % 16 == 0:
                    bm.allocate_block(r)
                live[r].append(rnd.randrange(1000))
            elif op == "fork" and live:
                r = rnd.choice(sorted(live))
                n = rnd.randint(1, len(live[r]))
                bm.fork(r, f"r{nid}", n)
                live[f"r{nid}"] = live[r][:n]
                nid += 1
            elif op == "release" and live:
                r = rnd.choice(sorted(live))
                bm.release(r)
                del live[r]
            elif op == "insert" and live:
                r = rnd.choice(sorted(live))
                n = len(live[r]) // 16 * 16
                if n:
                    pc.insert_kv(live[r][:n], r)
                    inserted.append(live[r][:n])
            elif op == "restore" and inserted:
                toks = rnd.choice(inserted)  # its request may be gone: cache-only pages
                m, _ = pc.lookup_kv(toks)
                if m:
                    k = rnd.randint(1, m)
                    pc.fork(toks, k, f"r{nid}")
                    live[f"r{nid}"] = toks[:k]
                    nid += 1
                    restored += 1
            elif op == "reclaim":
                pc.reclaim(rnd.randint(0, 8))
        except kv.CachePressure:
            pass
        request_pages = set()
        for r in live:
            request_pages.update(bm.block_table(r))
        st = mb.stats()
        allocated = bm.allocated_count()
        assert st.active_kv_reserved_bytes == PAGE * len(request_pages), (step, op)
        assert st.prefix_retained_bytes == PAGE * (allocated - len(request_pages)), (step, op)
        assert st.reserved_bytes == 64 + PAGE * allocated and st.available_bytes >= 0
    assert restored > 10 and pc.stats().kv_evictions > 10 and mb.stats().rejections > 10
    for r in list(live):
        bm.release(r)
    pc.clear()
    _close(pc, bm, mb)
