"""Prefix cache over refcounted pages (CPU: host C++ behind the C ABI).

Reference: PrefixCache (src/cache/prefix_cache.rs:58-394) and its tests
(tests/test_prefix_cache.rs:4-102), restated below; the chunk keys are checked
against hashlib's SHA-256 of the reference's construction, and random
operation sequences against oracle.PrefixCacheModel, a pure-Python
restatement of the reference's LRU and lookup rules. The page side -- a chunk
holding references instead of a copy -- is checked against the block
manager's refcounts and free count.
"""
import numpy as np
import pytest

import oracle as O


def test_chunk_hashes_match_reference_construction(kv):
    rng = np.random.default_rng(0)
    for n, cs in [(32, 16), (48, 16), (47, 16), (100, 32), (0, 16), (15, 16)]:
        toks = rng.integers(0, 2**32, n, dtype=np.uint64).tolist()
        assert kv.PrefixCache.compute_chunk_hashes(toks, cs) == O.PrefixCacheModel.chunk_hashes(
            toks, cs)


def test_prefix_chunk_hashing(kv):  # test_prefix_cache.rs:4-9
    chunks = kv.PrefixCache.compute_chunk_hashes(list(range(32)), 16)
    assert len(chunks) == 2 and chunks[0] != chunks[1]


def test_prefix_cache_insert_and_lookup(kv):  # test_prefix_cache.rs:11-31
    bm = kv.BlockManager(64)
    cache = kv.PrefixCache(bm, 16, 100)
    prompt = list(range(48))
    assert cache.lookup(prompt) == 0
    cache.insert(prompt)
    assert cache.lookup(prompt) == 48
    st = cache.stats()
    assert (st.hits, st.misses, st.tokens_saved) == (0, 0, 0)
    assert st.chunks == 3 and st.held_pages == 0  # metadata only
    cache.close()


def test_prefix_cache_lru_eviction(kv):  # test_prefix_cache.rs:33-52
    bm = kv.BlockManager(64)
    cache = kv.PrefixCache(bm, 16, 2)
    seq_a, seq_b = list(range(32)), list(range(100, 132))
    cache.insert(seq_a)
    assert cache.lookup(seq_a) == 32
    cache.insert(seq_b)
    assert cache.lookup(seq_b) == 32
    assert cache.lookup(seq_a) == 0
    cache.close()


def test_prefix_cache_insert_and_lookup_kv(kv):  # test_prefix_cache.rs:54-102
    bm = kv.BlockManager(64)
    cache = kv.PrefixCache(bm, 16, 100)
    prompt = list(range(48))
    bm.allocate("a", 48)
    assert cache.lookup_kv(prompt) == (0, None)
    cache.insert_kv(prompt, "a", logits_handle=77)
    assert cache.lookup_kv(prompt) == (48, 77)
    assert cache.lookup_kv(list(range(32)) + [999, 1000, 1001]) == (32, None)
    cache.close()


def test_cached_chunks_hold_pages_not_copies(kv):
    """insert_kv takes references on the request's pages: nothing is
    allocated, the pages outlive the request, and they return to the free
    list only when the last chunk holding them is evicted."""
    bm = kv.BlockManager(32)
    cache = kv.PrefixCache(bm, 16, 100)
    prompt = list(range(50))                       # 3 whole chunks + 2 tokens
    pages = bm.allocate("a", 50)                    # 4 pages
    free0 = bm.free_count()
    cache.insert_kv(prompt, "a")
    assert bm.free_count() == free0                 # no copies
    # chunk i references pages 0..i: page 0 is held by 3 chunks + the request
    assert [bm.refcount(p) for p in pages] == [4, 3, 2, 1]
    assert cache.stats().held_pages == 1 + 2 + 3
    bm.release("a")
    assert [bm.refcount(p) for p in pages] == [3, 2, 1, 0]
    assert bm.free_count() == free0 + 1             # only the partial 4th page returned
    cache.clear()
    assert bm.free_count() == 32 and cache.stats().kv_evictions == 3
    cache.close()


def test_restore_shares_pages_and_copies_a_partial_page(kv):
    """fork restores a cached prefix into a new request: whole pages shared,
    a trailing partial page copied on write (the matched - 1 restore of an
    exact hit without logits, src/backends/candle.rs:449-455)."""
    bm = kv.BlockManager(32)
    cache = kv.PrefixCache(bm, 16, 100)
    prompt = list(range(48))
    pages = bm.allocate("a", 48)
    cache.insert_kv(prompt, "a")
    assert cache.fork(prompt, 48, "b") == []
    assert bm.block_table("b") == pages
    cow = cache.fork(prompt, 47, "c")
    assert len(cow) == 1 and cow[0][0] == pages[2]
    assert bm.block_table("c") == pages[:2] + [cow[0][1]]
    with pytest.raises(kv.RlseError):
        cache.fork(prompt, 49, "d")                 # more than the cache holds
    with pytest.raises(kv.RlseError):
        cache.fork(prompt, 16, "b")                 # child already holds pages
    # an evicted intermediate chunk does not break a longer restore
    cache2 = kv.PrefixCache(bm, 16, 2)              # keeps only the 2 newest chunks
    cache2.insert_kv(prompt, "a")
    assert cache2.lookup_kv(prompt)[0] == 48
    assert cache2.fork(prompt, 48, "e") == [] and bm.block_table("e") == pages
    cache2.close()
    cache.close()


def test_reclaim_evicts_lru_until_enough_pages_are_free(kv):
    bm = kv.BlockManager(8)
    cache = kv.PrefixCache(bm, 16, 100)
    for i, rid in enumerate(["x", "y"]):
        bm.allocate(rid, 64)                        # 4 pages each: pool full
        cache.insert_kv([1000 * i + t for t in range(64)], rid)
        bm.release(rid)
    assert bm.free_count() == 0
    assert cache.reclaim(4) == 4                    # x's four chunks, oldest first
    assert bm.free_count() == 4
    assert cache.lookup_kv([t for t in range(64)])[0] == 0
    assert cache.lookup_kv([1000 + t for t in range(64)])[0] == 64
    with pytest.raises(kv.CachePressure):
        cache.reclaim(9)
    cache.close()


def test_random_operations_match_reference_model(kv):
    rng = np.random.default_rng(2024)
    bm = kv.BlockManager(4096)
    for max_chunks in (0, 3, 17):
        cache = kv.PrefixCache(bm, 16, max_chunks)
        model = O.PrefixCacheModel(16, max_chunks)
        bases = [rng.integers(0, 50, 200).tolist() for _ in range(4)]
        for step in range(300):
            base = bases[rng.integers(0, len(bases))]
            toks = base[:int(rng.integers(0, 120))]
            if rng.random() < 0.3:
                toks = toks + rng.integers(0, 50, int(rng.integers(1, 20))).tolist()
            op = rng.integers(0, 5)
            if op == 0:
                assert cache.lookup(toks) == model.lookup(toks)
            elif op == 1:
                cache.insert(toks)
                model.insert(toks)
            elif op == 2:
                rid = f"r{step}"
                bm.allocate(rid, max(len(toks), 1))
                handle = int(rng.integers(1, 10**6)) if rng.random() < 0.5 else None
                cache.insert_kv(toks, rid, handle)
                model.insert_kv(toks, handle)
                bm.release(rid)
            elif op == 3:
                assert cache.lookup_kv(toks) == model.lookup_kv(toks)
            else:
                skipped = int(rng.integers(0, 3)) * 16
                cache.record_reuse(skipped)
                model.record_reuse(skipped)
            st = cache.stats()
            assert (st.hits, st.misses, st.tokens_saved, st.kv_evictions, st.chunks) == (
                model.hits, model.misses, model.tokens_saved, model.kv_evictions,
                len(model.chunks))
            total = model.hits + model.misses
            want = np.float32(model.hits) / np.float32(total) * np.float32(100) if total else 0.0
            assert st.hit_rate == pytest.approx(float(want), rel=1e-6)
        cache.close()
        assert bm.free_count() == 4096  # every page back once requests and chunks let go
