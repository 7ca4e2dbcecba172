"""KV data movement on the GPU, bit-exact against the reference layout.

The reference keeps each request's K/V in a contiguous [1, Hkv, cap, d] buffer
written by KvCache::append (src/backends/qwen2.rs:349-361), restores prefix
snapshots by copying (set_kv_snapshot, :373-377, 547-574) and requires the
cached snapshot bytes to be unchanged after reuse (src/backends/candle.rs:
1281-1292). Here the same bytes must come out of the paged pool.
"""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import DEV, NP_OF, build_tables, random_values, to_dev, to_host

pytestmark = pytest.mark.gpu

DTYPES = ["bf16", "f32", "f16"]
SHAPES = [(8, 128), (2, 64)]  # (Hkv, head_dim): Qwen3-0.6B, Qwen2.5-0.5B


def _pool(num_blocks, hkv, d, dtype):
    return torch.zeros((num_blocks, hkv, 16, d), dtype={"bf16": torch.bfloat16,
                                                        "f32": torch.float32,
                                                        "f16": torch.float16}[dtype], device=DEV)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hkv,d", SHAPES)
def test_append_is_bit_exact(kv, dtype, hkv, d):
    rng = np.random.default_rng(100)
    nb, mbps = 64, 8
    prompts = [1, 15, 16, 17, 40]
    steps = 20
    b = len(prompts)
    tables = build_tables(rng, [p + steps for p in prompts], nb, mbps)
    t_dev = to_dev(tables)
    kp, vp = _pool(nb, hkv, d, dtype), _pool(nb, hkv, d, dtype)
    np_dt = NP_OF[dtype]
    pool_k = np.zeros((nb, hkv, 16, d), np_dt)
    pool_v = np.zeros_like(pool_k)
    caches = [(O.KvCacheC(hkv, 128, d, np_dt), O.KvCacheC(hkv, 128, d, np_dt)) for _ in range(b)]

    # prefill-style multi-token append: every prompt token of every sequence
    seq_index = np.concatenate([np.full(p, i, np.int32) for i, p in enumerate(prompts)])
    positions = np.concatenate([np.arange(p, dtype=np.int32) for p in prompts])
    n = len(positions)
    k_new = random_values(rng, (n, hkv, d), dtype)
    v_new = random_values(rng, (n, hkv, d), dtype)
    kv.kv_append(to_dev(k_new, dtype), to_dev(v_new, dtype), kp, vp, t_dev, b,
                 to_dev(seq_index), to_dev(positions), n, hkv, d, mbps, nb, dtype)
    for t in range(n):
        s, p = seq_index[t], positions[t]
        O.paged_write_token(pool_k, tables[s], p, k_new[t])
        O.paged_write_token(pool_v, tables[s], p, v_new[t])
        caches[s][0].append(k_new[t][:, None], k_new[t][:, None])
        caches[s][1].append(v_new[t][:, None], v_new[t][:, None])

    # decode-style appends: one token per sequence per step
    lens = np.array(prompts, np.int32)
    for _ in range(steps):
        k1 = random_values(rng, (b, hkv, d), dtype)
        v1 = random_values(rng, (b, hkv, d), dtype)
        kv.kv_append(to_dev(k1, dtype), to_dev(v1, dtype), kp, vp, t_dev, b, None,
                     to_dev(lens), b, hkv, d, mbps, nb, dtype)
        for s in range(b):
            O.paged_write_token(pool_k, tables[s], int(lens[s]), k1[s])
            O.paged_write_token(pool_v, tables[s], int(lens[s]), v1[s])
            caches[s][0].append(k1[s][:, None], k1[s][:, None])
            caches[s][1].append(v1[s][:, None], v1[s][:, None])
        lens += 1

    np.testing.assert_array_equal(to_host(kp), pool_k)
    np.testing.assert_array_equal(to_host(vp), pool_v)
    for s in range(b):
        length = int(lens[s])
        ko = torch.empty((hkv, length, d), dtype=kp.dtype, device=DEV)
        vo = torch.empty_like(ko)
        kv.kv_gather(kp, vp, 0, 1, to_dev(tables[s]), length, ko, vo, hkv, d, nb, dtype)
        np.testing.assert_array_equal(to_host(ko), caches[s][0].snapshot()[0])
        np.testing.assert_array_equal(to_host(vo), caches[s][1].snapshot()[0])


def test_append_skips_out_of_range_slots(kv):
    rng = np.random.default_rng(101)
    nb, mbps, hkv, d = 8, 2, 2, 64
    tables = np.array([[3, 99], [5, -1]], np.int32)  # invalid ids in the second page
    kp, vp = _pool(nb, hkv, d, "bf16"), _pool(nb, hkv, d, "bf16")
    k = random_values(rng, (4, hkv, d), "bf16")
    # positions: valid, invalid block id, beyond max_blocks_per_seq*16, negative
    pos = np.array([2, 20, 40, -1], np.int32)
    seq = np.array([0, 1, 0, 1], np.int32)
    kv.kv_append(to_dev(k, "bf16"), to_dev(k, "bf16"), kp, vp, to_dev(tables), 2, to_dev(seq),
                 to_dev(pos), 4, hkv, d, mbps, nb, "bf16")
    got = to_host(kp)
    want = np.zeros_like(got)
    want[3, :, 2] = k[0]
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_pool_handle_scatter_gather_round_trip(kv, dtype):
    rng = np.random.default_rng(102)
    layers, nb, hkv, d = 3, 40, 8, 128
    pool = kv.KVPool(layers, nb, hkv, d, dtype)
    k0, v0 = pool.layer(0)
    k2, _ = pool.layer(2)
    es = {"bf16": 2, "f32": 4}[dtype]
    assert k2 - k0 == 2 * pool.layer_stride_elems * es
    table = rng.permutation(nb)[:5].astype(np.int32)
    snap_k = random_values(rng, (layers, hkv, 70, d), dtype)
    snap_v = random_values(rng, (layers, hkv, 70, d), dtype)
    t_dev = to_dev(table)
    kv.kv_scatter(to_dev(snap_k, dtype), to_dev(snap_v, dtype), k0, v0, pool.layer_stride_elems,
                  layers, t_dev, 0, 70, hkv, d, nb, dtype)
    tail = random_values(rng, (layers, hkv, 9, d), dtype)
    kv.kv_scatter(to_dev(tail, dtype), to_dev(tail, dtype), k0, v0, pool.layer_stride_elems,
                  layers, t_dev, 70, 9, hkv, d, nb, dtype)
    tdt = {"bf16": torch.bfloat16, "f32": torch.float32}[dtype]
    ko = torch.empty((layers, hkv, 79, d), dtype=tdt, device=DEV)
    vo = torch.empty_like(ko)
    kv.kv_gather(k0, v0, pool.layer_stride_elems, layers, t_dev, 79, ko, vo, hkv, d, nb, dtype)
    np.testing.assert_array_equal(to_host(ko), np.concatenate([snap_k, tail], axis=2))
    np.testing.assert_array_equal(to_host(vo), np.concatenate([snap_v, tail], axis=2))
    pool.close()


@pytest.mark.parametrize("prefix_len", [1024, 1030])
def test_prefix_fork_copy_on_write_is_bit_exact(kv, prefix_len):
    """Prefix-fork semantics at reduced size: a shared prefix held by refcounted
    blocks, forks with copy-on-write of the trailing partial block, per-fork
    suffix appends; every fork must read back exactly "copy the prefix snapshot
    into a fresh buffer, then append" and the prefix must stay untouched."""
    rng = np.random.default_rng(103)
    layers, nb, hkv, d, dtype = 2, 256, 8, 128, "bf16"
    pool = kv.KVPool(layers, nb, hkv, d, dtype)
    k0, v0 = pool.layer(0)
    stride = pool.layer_stride_elems
    bm = kv.BlockManager(nb, 16)
    bm.allocate("prefix", prefix_len)
    ptable = np.array(bm.block_table("prefix"), np.int32)
    pk = random_values(rng, (layers, hkv, prefix_len, d), dtype)
    pv = random_values(rng, (layers, hkv, prefix_len, d), dtype)
    kv.kv_scatter(to_dev(pk, dtype), to_dev(pv, dtype), k0, v0, stride, layers, to_dev(ptable),
                  0, prefix_len, hkv, d, nb, dtype)
    suffix = [64, 77, 100, 5]
    expect = {}
    for i, s in enumerate(suffix):
        rid = f"seq{i}"
        pairs = bm.fork("prefix", rid, prefix_len)
        assert len(pairs) == (1 if prefix_len % 16 else 0)
        if pairs:
            src = to_dev(np.array([p[0] for p in pairs], np.int32))
            dst = to_dev(np.array([p[1] for p in pairs], np.int32))
            kv.kv_copy_blocks(k0, v0, stride, layers, src, dst, len(pairs), hkv, d, nb, dtype)
        sk = random_values(rng, (layers, s, hkv, d), dtype)
        sv = random_values(rng, (layers, s, hkv, d), dtype)
        while len(bm.block_table(rid)) * 16 < prefix_len + s:
            bm.allocate_block(rid)
        table = np.array(bm.block_table(rid), np.int32)
        t_dev = to_dev(table)
        pos = to_dev(np.arange(prefix_len, prefix_len + s, dtype=np.int32))
        seq = to_dev(np.zeros(s, np.int32))
        for layer in range(layers):
            kl = k0 + layer * stride * 2
            vl = v0 + layer * stride * 2
            kv.kv_append(to_dev(sk[layer], dtype), to_dev(sv[layer], dtype), kl, vl, t_dev, 1,
                         seq, pos, s, hkv, d, len(table), nb, dtype)
        expect[rid] = (table, np.concatenate([pk, sk.transpose(0, 2, 1, 3)], axis=2),
                       np.concatenate([pv, sv.transpose(0, 2, 1, 3)], axis=2))
    for rid, (table, ek, ev) in expect.items():
        length = ek.shape[2]
        ko = torch.empty((layers, hkv, length, d), dtype=torch.bfloat16, device=DEV)
        vo = torch.empty_like(ko)
        kv.kv_gather(k0, v0, stride, layers, to_dev(table), length, ko, vo, hkv, d, nb, dtype)
        np.testing.assert_array_equal(to_host(ko), ek)
        np.testing.assert_array_equal(to_host(vo), ev)
    # the cached prefix snapshot is unchanged after reuse
    ko = torch.empty((layers, hkv, prefix_len, d), dtype=torch.bfloat16, device=DEV)
    vo = torch.empty_like(ko)
    kv.kv_gather(k0, v0, stride, layers, to_dev(ptable), prefix_len, ko, vo, hkv, d, nb, dtype)
    np.testing.assert_array_equal(to_host(ko), pk)
    np.testing.assert_array_equal(to_host(vo), pv)
    pool.close()


@pytest.mark.parametrize("prefix_len", [1024, 1030])
def test_forked_decode_step_equals_private_copies(kv, prefix_len):
    """Prefix-fork decode step at reduced batch: decode steps over forked sequences
    (prefix pages shared by refcount, partial page copied on write) give
    bit-for-bit the output of the same step over private copies of every
    sequence, the appended tokens land in private pages, and the shared
    prefix bytes stay unchanged."""
    import math
    rng = np.random.default_rng(404)
    layers, hq, hkv, d, dtype, b = 2, 16, 8, 128, "bf16", 6
    suffix = rng.integers(20, 90, b).astype(np.int32)
    lens = prefix_len + suffix + 1
    nb = 600  # the private-copy layout alone needs b * ceil(lens/16) pages
    bf = torch.bfloat16
    pa = kv.KVPool(layers, nb, hkv, d, dtype)   # forked layout
    pb = kv.KVPool(layers, nb, hkv, d, dtype)   # private copies
    stride = pa.layer_stride_elems
    ka0, va0 = pa.layer(0)
    kb0, vb0 = pb.layer(0)
    bma, bmb = kv.BlockManager(nb), kv.BlockManager(nb)
    pk = random_values(rng, (layers, hkv, prefix_len, d), dtype)
    pv = random_values(rng, (layers, hkv, prefix_len, d), dtype)
    bma.allocate("prefix", prefix_len)
    ptab = np.array(bma.block_table("prefix"), np.int32)
    kv.kv_scatter(to_dev(pk, dtype), to_dev(pv, dtype), ka0, va0, stride, layers, to_dev(ptab), 0,
                  prefix_len, hkv, d, nb, dtype)
    pairs = []
    for i in range(b):
        pairs += bma.fork("prefix", f"r{i}", prefix_len)
        while len(bma.block_table(f"r{i}")) * 16 < int(lens[i]):
            bma.allocate_block(f"r{i}")
        bmb.allocate(f"r{i}", int(lens[i]))
    assert len(pairs) == (b if prefix_len % 16 else 0)
    if pairs:
        kv.kv_copy_blocks(ka0, va0, stride, layers, to_dev(np.array([p[0] for p in pairs], np.int32)),
                          to_dev(np.array([p[1] for p in pairs], np.int32)), len(pairs), hkv, d,
                          nb, dtype)
    mbps = max(len(bma.block_table(f"r{i}")) for i in range(b))
    ta = np.zeros((b, mbps), np.int32)
    tb = np.zeros((b, mbps), np.int32)
    sks, svs = [], []
    for i in range(b):
        a_t, b_t = bma.block_table(f"r{i}"), bmb.block_table(f"r{i}")
        ta[i, :len(a_t)] = a_t
        tb[i, :len(b_t)] = b_t
        n = int(suffix[i])
        sk = random_values(rng, (layers, hkv, n, d), dtype)
        sv = random_values(rng, (layers, hkv, n, d), dtype)
        sks.append(sk)
        svs.append(sv)
        kv.kv_scatter(to_dev(sk, dtype), to_dev(sv, dtype), ka0, va0, stride, layers,
                      to_dev(ta[i]), prefix_len, n, hkv, d, nb, dtype)
        kv.kv_scatter(to_dev(np.concatenate([pk, sk], axis=2), dtype),
                      to_dev(np.concatenate([pv, sv], axis=2), dtype), kb0, vb0, stride, layers,
                      to_dev(tb[i]), 0, prefix_len + n, hkv, d, nb, dtype)
    max_pos = mbps * 16
    cos_b, sin_b = kv.rope_tables(1e6, d, max_pos, dtype)
    cos_t = torch.frombuffer(bytearray(cos_b), dtype=torch.int16).to(DEV).view(bf)
    sin_t = torch.frombuffer(bytearray(sin_b), dtype=torch.int16).to(DEV).view(bf)
    lens_dev = to_dev(lens.astype(np.int32))
    qw = to_dev(random_values(rng, (d,), dtype), dtype)
    kw = to_dev(random_values(rng, (d,), dtype), dtype)
    scale = 1 / math.sqrt(d)
    tad, tbd = to_dev(ta), to_dev(tb)
    for layer in range(layers):
        q = to_dev(random_values(rng, (b, hq, d), dtype), dtype)
        kn = to_dev(random_values(rng, (b, hkv, d), dtype), dtype)
        vn = to_dev(random_values(rng, (b, hkv, d), dtype), dtype)
        outs = []
        for (k0, v0), tab in (((ka0, va0), tad), ((kb0, vb0), tbd)):
            kl, vl = k0 + layer * stride * 2, v0 + layer * stride * 2
            out = torch.empty((b, hq, d), dtype=bf, device=DEV)
            print(f"fork decode step layer {layer} prefix {prefix_len}", flush=True)
            kv.decode_step(q, kn, vn, qw, kw, 1e-6, cos_t, sin_t, max_pos, kl, vl, tab, lens_dev,
                           out, b, hq, hkv, d, mbps, nb, scale, dtype)
            outs.append(to_host(out))
        np.testing.assert_array_equal(outs[0], outs[1])
    # every sequence reads back identically from both layouts
    for i in range(b):
        n = int(lens[i])
        got = []
        for (k0, v0), tab in (((ka0, va0), ta), ((kb0, vb0), tb)):
            ko = torch.empty((layers, hkv, n, d), dtype=bf, device=DEV)
            vo = torch.empty_like(ko)
            kv.kv_gather(k0, v0, stride, layers, to_dev(tab[i]), n, ko, vo, hkv, d, nb, dtype)
            got.append((to_host(ko), to_host(vo)))
        np.testing.assert_array_equal(got[0][0], got[1][0])
        np.testing.assert_array_equal(got[0][1], got[1][1])
    # the shared prefix is untouched by the forks' appends
    ko = torch.empty((layers, hkv, prefix_len, d), dtype=bf, device=DEV)
    vo = torch.empty_like(ko)
    kv.kv_gather(ka0, va0, stride, layers, to_dev(ptab), prefix_len, ko, vo, hkv, d, nb, dtype)
    np.testing.assert_array_equal(to_host(ko), pk)
    np.testing.assert_array_equal(to_host(vo), pv)
    pa.close()
    pb.close()


def test_prefix_cache_restore_reads_back_the_cached_prefix(kv):
    """A prompt's KV cached through the prefix cache (page references, no
    copy) and restored into a new request after the original request is gone:
    the restored tokens read back byte for byte, a restore ending mid-page
    copies that page, and appends to the restored request leave the cached
    pages untouched."""
    rng = np.random.default_rng(77)
    layers, nb, hkv, d, dtype = 3, 64, 8, 128, "bf16"
    pool = kv.KVPool(layers, nb, hkv, d, dtype)
    k0, v0 = pool.layer(0)
    stride = pool.layer_stride_elems
    bm = kv.BlockManager(nb)
    cache = kv.PrefixCache(bm, 16, 64)
    prompt = rng.integers(0, 30000, 70).tolist()
    table = np.array(bm.allocate("a", 70), np.int32)
    ka = random_values(rng, (layers, hkv, 70, d), dtype)
    va = random_values(rng, (layers, hkv, 70, d), dtype)
    kv.kv_scatter(to_dev(ka, dtype), to_dev(va, dtype), k0, v0, stride, layers, to_dev(table), 0,
                  70, hkv, d, nb, dtype)
    cache.insert_kv(prompt, "a")
    bm.release("a")
    assert cache.lookup_kv(prompt)[0] == 64
    for child, restore in [("b", 64), ("c", 63), ("d", 40)]:
        print(f"restore {restore} tokens into {child}", flush=True)
        cow = cache.fork(prompt, restore, child)
        assert len(cow) == (1 if restore % 16 else 0)
        if cow:
            kv.kv_copy_blocks(k0, v0, stride, layers, to_dev(np.array([cow[0][0]], np.int32)),
                              to_dev(np.array([cow[0][1]], np.int32)), 1, hkv, d, nb, dtype)
        ctab = np.array(bm.block_table(child), np.int32)
        ko = torch.empty((layers, hkv, restore, d), dtype=torch.bfloat16, device=DEV)
        vo = torch.empty_like(ko)
        kv.kv_gather(k0, v0, stride, layers, to_dev(ctab), restore, ko, vo, hkv, d, nb, dtype)
        np.testing.assert_array_equal(to_host(ko), ka[:, :, :restore])
        np.testing.assert_array_equal(to_host(vo), va[:, :, :restore])
        # the restored request appends its next token into its own page
        while len(bm.block_table(child)) * 16 < restore + 1:
            bm.allocate_block(child)
        ctab = np.array(bm.block_table(child), np.int32)
        nk = random_values(rng, (1, hkv, d), dtype)
        for layer in range(layers):
            kv.kv_append(to_dev(nk, dtype), to_dev(nk, dtype), k0 + layer * stride * 2,
                         v0 + layer * stride * 2, to_dev(ctab), 1,
                         to_dev(np.zeros(1, np.int32)), to_dev(np.array([restore], np.int32)), 1,
                         hkv, d, len(ctab), nb, dtype)
    # the cached pages still hold the original prompt
    cow = cache.fork(prompt, 64, "z")
    ztab = np.array(bm.block_table("z"), np.int32)
    ko = torch.empty((layers, hkv, 64, d), dtype=torch.bfloat16, device=DEV)
    vo = torch.empty_like(ko)
    kv.kv_gather(k0, v0, stride, layers, to_dev(ztab), 64, ko, vo, hkv, d, nb, dtype)
    np.testing.assert_array_equal(to_host(ko), ka[:, :, :64])
    np.testing.assert_array_equal(to_host(vo), va[:, :, :64])
    cache.close()
    pool.close()


def test_step_table_uploads_match_host_and_feed_decode(kv):
    """The change-only upload (rlse_st_upload: pinned staging, one copy, one
    scatter kernel) over 24 steps of joins, growth, forks and finishes: the
    device rows equal the host image in every valid entry, the lengths match,
    and decode through the uploaded tables equals decode through a full upload
    of the same image, bit for bit."""
    import random
    rnd = random.Random(11)
    hq, hkv, d, dtype = 16, 8, 128, "bf16"
    nb, B, W = 300, 16, 64
    bm = kv.BlockManager(nb)
    st = kv.StepTables(B, W)
    dev_tables = torch.full((B, W), -1, dtype=torch.int32, device=DEV)
    dev_lens = torch.zeros(B, dtype=torch.int32, device=DEV)
    rng = np.random.default_rng(4)
    kp = to_dev(random_values(rng, (nb, hkv, 16, d), dtype), dtype)
    vp = to_dev(random_values(rng, (nb, hkv, 16, d), dtype), dtype)
    q = to_dev(random_values(rng, (B, hq, d), dtype), dtype)
    live, order, nid = {}, [], 0
    for step in range(24):
        while len(order) < B and rnd.random() < 0.5:
            rid = f"r{nid}"
            nid += 1
            try:
                if order and rnd.random() < 0.3:
                    parent = rnd.choice(order)
                    n = rnd.randint(1, live[parent])
                    bm.fork(parent, rid, n)
                else:
                    n = rnd.randint(1, 600)
                    bm.allocate(rid, n)
            except kv.CachePressure:
                continue
            live[rid] = n
            order.append(rid)
        if rnd.random() < 0.25 and len(order) > 1:
            i = rnd.randrange(len(order))
            bm.release(order[i])
            del live[order[i]]
            order[i] = order[-1]
            order.pop()
        next_lens = [min(live[r] + 1, W * 16) for r in order]
        status = st.prepare(bm, order, next_lens)
        tables, lens, batch, pend = st.host()
        print(f"step {step}: batch {batch}, {len(pend)} triples", flush=True)
        st.upload(dev_tables, dev_lens)
        torch.cuda.synchronize()
        got_t, got_l = to_host(dev_tables), to_host(dev_lens)
        np.testing.assert_array_equal(got_l[:batch], lens[:batch])
        for i in range(batch):
            n = -(-int(lens[i]) // 16)
            np.testing.assert_array_equal(got_t[i, :n], tables[i, :n], err_msg=f"row {i}")
        if step in (8, 23) and batch:
            out_a = torch.empty_like(q)
            out_b = torch.empty_like(q)
            kv.paged_gqa_decode(q, kp, vp, dev_tables, dev_lens, out_a, batch, hq, hkv, d, W, nb,
                                0.0883, dtype)
            kv.paged_gqa_decode(q, kp, vp, to_dev(tables), to_dev(lens), out_b, batch, hq, hkv,
                                d, W, nb, 0.0883, dtype)
            np.testing.assert_array_equal(to_host(out_a)[:batch], to_host(out_b)[:batch])
        keep = []
        for r, s_, nl in zip(order, status, next_lens):
            if s_ == 0:
                live[r] = nl
                keep.append(r)
            else:
                del live[r]
        order = keep
    bm.release_all()
    st.close()
