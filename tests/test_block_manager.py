"""Host block manager (KVCache successor) through the C ABI.

The first three tests restate the reference's tests/test_kv_cache.rs; the
random-sequence test cross-checks ids and stats against a pure-Python
restatement of src/cache/kv_cache.rs; the rest cover the refcounted fork
with copy-on-write that physical pages add.
"""
import random

import pytest

import oracle as O


def test_cache_allocate_and_release(kv):
    cache = kv.BlockManager(100, 16)
    assert cache.free_count() == 100
    assert cache.allocated_count() == 0
    blocks = cache.allocate("req-1", 32)  # 32 tokens requires 2 blocks
    assert len(blocks) == 2
    assert cache.free_count() == 98
    assert cache.allocated_count() == 2
    assert cache.release("req-1") == 2
    assert cache.free_count() == 100
    assert cache.allocated_count() == 0


def test_cache_pressure_error(kv):
    cache = kv.BlockManager(4, 16)
    with pytest.raises(kv.CachePressure) as e:
        cache.allocate("req-over", 80)  # 5 blocks needed
    assert "Requested 5 blocks" in e.value.message
    assert e.value.status == kv.ERR_CACHE_PRESSURE


def test_fragmentation_stats(kv):
    cache = kv.BlockManager(10, 16)
    assert cache.allocate("req-1", 16) == [0]
    assert cache.allocate("req-2", 16) == [1]
    assert cache.allocate("req-3", 16) == [2]
    cache.release("req-2")
    stats = cache.stats()
    assert stats.total_blocks == 10
    assert stats.free_blocks == 8
    assert stats.utilization > 0.0
    assert stats.fragmentation == pytest.approx(0.125)


def test_blocks_needed_and_incremental_growth(kv):
    cache = kv.BlockManager(8, 16)
    assert [cache.blocks_needed(t) for t in (0, 1, 16, 17, 37)] == [1, 1, 1, 2, 3]
    assert cache.allocate("r", 37) == [0, 1, 2]  # the reference record: 37 tokens -> [.., 3]
    assert cache.allocate_block("r") == 3
    assert cache.block_table("r") == [0, 1, 2, 3]
    with pytest.raises(kv.CachePressure, match="no free blocks"):
        big = kv.BlockManager(1, 16)
        big.allocate("a", 1)
        big.allocate_block("a")


def test_random_sequences_match_reference_model(kv):
    rnd = random.Random(1234)
    for trial in range(20):
        total = rnd.randint(1, 64)
        cache, model = kv.BlockManager(total, 16), O.KVCacheModel(total, 16)
        live = []
        for step in range(200):
            op = rnd.random()
            if op < 0.4:
                rid, toks = f"r{trial}-{step}", rnd.randint(0, 100)
                try:
                    want = model.allocate(rid, toks)
                except MemoryError as e:
                    with pytest.raises(kv.CachePressure) as got:
                        cache.allocate(rid, toks)
                    assert got.value.message == str(e)
                    continue
                assert cache.allocate(rid, toks) == want
                live.append(rid)
            elif op < 0.7 and live:
                rid = rnd.choice(live)
                try:
                    want = model.allocate_block(rid)
                except MemoryError:
                    with pytest.raises(kv.CachePressure):
                        cache.allocate_block(rid)
                    continue
                assert cache.allocate_block(rid) == want
            elif live:
                rid = live.pop(rnd.randrange(len(live)))
                assert cache.release(rid) == model.release(rid)
            s = cache.stats()
            assert (s.total_blocks, s.allocated_blocks, s.free_blocks) == model.stats()[:3]
            assert s.utilization == pytest.approx(model.stats()[3], abs=1e-6)
            assert s.fragmentation == pytest.approx(model.stats()[4], abs=1e-6)
        assert cache.release("never-allocated") == 0


def test_fork_shares_full_blocks_and_copies_partial(kv):
    cache = kv.BlockManager(200, 16)
    prefix = cache.allocate("prefix", 1030)  # 64 full blocks + 6 tokens
    assert len(prefix) == 65
    cows = {}
    for i in range(3):
        pairs = cache.fork("prefix", f"s{i}", 1030)
        assert len(pairs) == 1 and pairs[0][0] == prefix[64]
        cows[i] = pairs[0][1]
        table = cache.block_table(f"s{i}")
        assert table[:64] == prefix[:64] and table[64] == pairs[0][1]
    assert all(cache.refcount(b) == 4 for b in prefix[:64])
    assert cache.refcount(prefix[64]) == 1
    assert len(set(cows.values())) == 3
    # releasing the prefix keeps shared blocks alive for the forks
    assert cache.release("prefix") == 65
    assert all(cache.refcount(b) == 3 for b in prefix[:64])
    assert cache.refcount(prefix[64]) == 0
    for i in range(3):
        cache.release(f"s{i}")
    assert cache.free_count() == 200
    assert cache.stats().allocated_blocks == 0


def test_aligned_fork_is_pure_refcount(kv):
    cache = kv.BlockManager(100, 16)
    prefix = cache.allocate("p", 1024)
    free_before = cache.free_count()
    assert cache.fork("p", "c", 1024) == []
    assert cache.free_count() == free_before
    assert cache.block_table("c") == prefix


def test_fork_rejects_bad_requests_without_change(kv):
    cache = kv.BlockManager(4, 16)
    cache.allocate("p", 40)  # 3 blocks
    with pytest.raises(kv.RlseError):
        cache.fork("p", "c", 60)  # parent holds too few blocks
    with pytest.raises(kv.RlseError):
        cache.fork("missing", "c", 16)
    cache.allocate("full", 16)  # pool now exhausted
    with pytest.raises(kv.CachePressure):
        cache.fork("p", "c", 40)  # partial block needs a free block
    assert cache.refcount(0) == 1 and cache.free_count() == 0
    with pytest.raises(kv.RlseError):
        cache.block_table("c")
