"""Paged GQA decode attention on the GPU against the oracle.

Reference: decode_attention_gqa_zero_copy (src/backends/qwen2.rs:177-203) over
the buffers KvCache::append builds (:349-361), batched as in
step_decode_batch (:723-744). The oracle is the C restatement of that Candle
CPU path (oracle/rlse_oracle.c), itself pinned against float64 forms in
tests/test_oracle.py. Bars: max-abs 2e-3 for f32, 2e-2 for bf16/f16; the
relative error (max-abs / max |reference|) is printed beside it.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import (DEV, TOL, as_f32, build_tables, err_report, random_values, to_dev,
                         to_host)

pytestmark = pytest.mark.gpu


def run_decode(kv, q, kp, vp, tables, lens, hq, hkv, d, dtype, scale, workspace=None):
    b, mbps, nb = q.shape[0], tables.shape[1], kp.shape[0]
    out = torch.empty_like(q)
    ws, wsb = None, 0
    if workspace is not None:
        ws, wsb = workspace, workspace.numel()
    kv.paged_gqa_decode(q, kp, vp, to_dev(tables), to_dev(lens), out, b, hq, hkv, d, mbps, nb,
                        scale, dtype, ws, wsb)
    return to_host(out)


def check(name, got, want, dtype):
    mx, rel = err_report(got, want)
    print(f"[{name}] dtype={dtype} max_abs={mx:.3e} rel={rel:.3e}")
    assert np.isfinite(got).all()
    assert mx <= TOL[dtype], (name, mx)
    return mx, rel


def make_case(rng, lens, hq, hkv, d, dtype, extra_blocks=7):
    lens = np.asarray(lens, np.int32)
    mbps = max(1, int(max((int(n) + 15) // 16 for n in lens)))
    nb = int(sum((int(n) + 15) // 16 for n in lens)) + extra_blocks
    tables = build_tables(rng, lens, nb, mbps)
    kpool = random_values(rng, (nb, hkv, 16, d), dtype)
    vpool = random_values(rng, (nb, hkv, 16, d), dtype)
    q = random_values(rng, (len(lens), hq, d), dtype)
    return q, kpool, vpool, tables, lens


def oracle_decode(q, kpool, vpool, tables, lens, dtype, scale):
    return O.decode_paged_f32(as_f32(q, dtype), as_f32(kpool, dtype), as_f32(vpool, dtype),
                              tables, lens, scale)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("fixture", ["decode_f32.npz", "decode_gqa7_f32.npz"])
def test_golden_case_matrix(kv, dtype, fixture):
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", fixture))
    q, kpool, vpool = g["q"], g["k_pool"], g["v_pool"]
    if dtype == "f32":
        q, kpool, vpool = (O.bf16_bits_to_f32(x) for x in (q, kpool, vpool))
    hq, d = q.shape[1], q.shape[2]
    hkv = kpool.shape[1]
    got = run_decode(kv, to_dev(q, dtype), to_dev(kpool, dtype), to_dev(vpool, dtype),
                     g["tables"], g["lens"], hq, hkv, d, dtype, float(g["scale"]))
    check(f"golden {fixture}", as_f32(got, dtype), g["out_f64"], dtype)


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (14, 2, 64), (32, 8, 128), (8, 8, 64),
                                      (24, 3, 128), (40, 5, 64), (48, 8, 128), (64, 8, 64)])
def test_group_sizes_and_ragged_lengths(kv, dtype, hq, hkv, d):
    rng = np.random.default_rng(hq * 131 + d)
    lens = [1, 2, 15, 16, 17, 33, 64, 127, 300, 513]
    q, kp, vp, tables, lens = make_case(rng, lens, hq, hkv, d, dtype)
    scale = 1.0 / math.sqrt(d)
    got = run_decode(kv, to_dev(q, dtype), to_dev(kp, dtype), to_dev(vp, dtype), tables, lens,
                     hq, hkv, d, dtype, scale)
    want = oracle_decode(q, kp, vp, tables, lens, dtype, scale)
    check(f"G={hq // hkv} d={d}", as_f32(got, dtype), want, dtype)


def test_qwen3_f32_single_sequence_decode_step(kv):
    """Single-layer Qwen3-0.6B decode step, f32, batch 1: 16 query heads, 8 KV
    heads, head_dim 128, 512 cached tokens; q and the new k go through
    q_norm/k_norm (eps 1e-6, weights 1 + 0.1 N(0,1)) and RoPE (theta 1e6) at
    position 512; the new k/v are appended and attention runs over 513 keys
    (Attention::forward order, src/backends/qwen2.rs:291-328)."""
    rng = np.random.default_rng(1)
    hq, hkv, d, cached, theta, eps = 16, 8, 128, 512, 1e6, 1e-6
    nb, mbps = 48, 33
    tables = build_tables(rng, [cached + 1], nb, mbps)
    k_cache = rng.standard_normal((hkv, cached, d)).astype(np.float32)
    v_cache = rng.standard_normal((hkv, cached, d)).astype(np.float32)
    q_raw = rng.standard_normal((1, hq, d)).astype(np.float32)
    k_raw = rng.standard_normal((1, hkv, d)).astype(np.float32)
    v_raw = rng.standard_normal((1, hkv, d)).astype(np.float32)
    qw = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kw = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    scale = 1.0 / math.sqrt(d)

    # oracle: the reference's Candle CPU op sequence
    cos_t, sin_t = O.rope_tables_f32(theta, d, cached + 1)
    pos = np.full(hq, cached, np.int32)
    q_o = O.apply_rope_f32(O.rmsnorm_f32(q_raw[0], qw, eps), pos, cos_t, sin_t)
    k_o = O.apply_rope_f32(O.rmsnorm_f32(k_raw[0], kw, eps), pos[:hkv], cos_t, sin_t)
    cache_k = O.KvCacheC(hkv, cached + 1, d, np.float32)
    cache_v = O.KvCacheC(hkv, cached + 1, d, np.float32)
    cache_k.append(k_cache, k_cache)
    cache_v.append(v_cache, v_cache)
    cache_k.append(k_o[:, None], k_o[:, None])
    cache_v.append(v_raw[0][:, None], v_raw[0][:, None])
    want = O.decode_batch_f32(q_o[None], cache_k.snapshot()[0][None], cache_v.snapshot()[0][None],
                              np.array([cached + 1], np.int32), scale)

    # device: restore the cached tokens, fused norm + RoPE + append, decode
    kp = torch.zeros((nb, hkv, 16, d), dtype=torch.float32, device=DEV)
    vp = torch.zeros_like(kp)
    t_dev = to_dev(tables)
    kv.kv_scatter(to_dev(k_cache), to_dev(v_cache), kp, vp, 0, 1, t_dev, 0, cached, hkv, d, nb,
                  "f32")
    cos_b, sin_b = kv.rope_tables(theta, d, cached + 1, "f32")
    cos_d = to_dev(np.frombuffer(cos_b, np.float32).copy())
    sin_d = to_dev(np.frombuffer(sin_b, np.float32).copy())
    q_rot = torch.empty((1, hq, d), dtype=torch.float32, device=DEV)
    kv.qk_norm_rope_append(to_dev(q_raw), to_dev(k_raw), to_dev(v_raw), to_dev(qw), to_dev(kw),
                           eps, cos_d, sin_d, cached + 1, to_dev(np.array([cached], np.int32)),
                           t_dev, 1, None, 1, hq, hkv, d, mbps, nb, q_rot, kp, vp, "f32")
    np.testing.assert_allclose(to_host(q_rot)[0], q_o, rtol=2e-6, atol=2e-6)
    got = run_decode(kv, q_rot, kp, vp, tables, np.array([cached + 1], np.int32), hq, hkv, d,
                     "f32", scale)
    check("qwen3 f32 B=1 L=513", got, want, "f32")


@pytest.mark.parametrize("hq,hkv,d,batch,lmin,lmax", [
    (16, 8, 128, 32, 128, 2048),   # Qwen3-0.6B batched decode, one layer
    (14, 2, 64, 64, 4096, 4096),   # Qwen2.5-0.5B, 4096 cached tokens
])
def test_full_batch_one_layer_bf16(kv, hq, hkv, d, batch, lmin, lmax):
    """One layer of the batched-decode workloads at their full batch and
    length mix: ragged lengths + 1 appended token, 16-token blocks drawn
    from a seeded random permutation."""
    rng = np.random.default_rng(2 if hq == 16 else 3)
    lens = rng.integers(lmin, lmax + 1, batch) + 1
    q, kp, vp, tables, lens = make_case(rng, lens, hq, hkv, d, "bf16")
    scale = 1.0 / math.sqrt(d)
    got = run_decode(kv, to_dev(q, "bf16"), to_dev(kp, "bf16"), to_dev(vp, "bf16"), tables, lens,
                     hq, hkv, d, "bf16", scale)
    want = oracle_decode(q, kp, vp, tables, lens, "bf16", scale)
    check(f"batch{batch} G={hq // hkv}", as_f32(got, "bf16"), want, "bf16")


def test_edge_lengths_and_invalid_blocks(kv):
    rng = np.random.default_rng(9)
    hq, hkv, d, dtype = 16, 8, 128, "bf16"
    q, kp, vp, tables, _ = make_case(rng, [48, 48, 48, 48], hq, hkv, d, dtype)
    nb = kp.shape[0]
    tables = tables.copy()
    tables[2, 1] = nb + 5  # middle page outside the pool: skipped
    # an empty row; a row longer than its table (3 pages * 16) is invalid
    lens = np.array([0, 48, 48, 1000], np.int32)
    kv.workspace_flags()  # clear anything earlier tests left in the library-owned workspace
    got = as_f32(run_decode(kv, to_dev(q, dtype), to_dev(kp, dtype), to_dev(vp, dtype), tables,
                            lens, hq, hkv, d, dtype, 0.088), dtype)
    assert np.all(got[0] == 0.0)
    assert np.all(got[3] == 0.0)
    assert kv.workspace_flags() == kv.WS_ERR_LENGTH
    with pytest.raises(kv.TokenLimitExceeded):
        run_decode(kv, to_dev(q, dtype), to_dev(kp, dtype), to_dev(vp, dtype), tables, lens, hq,
                   hkv, d, dtype, 0.088)
        kv.workspace_check()
    assert kv.workspace_flags() == 0
    want1 = oracle_decode(q[1:2], kp, vp, tables[1:2], np.array([48], np.int32), dtype, 0.088)
    check("plain row", got[1:2], want1, dtype)
    # row 2 without its second page: keys 0-15 and 32-47
    kf, vf = as_f32(kp, dtype), as_f32(vp, dtype)
    t2 = tables[2]
    k2 = np.concatenate([O.paged_to_contiguous(kf, t2[:1], 16),
                         O.paged_to_contiguous(kf, t2[2:3], 16)], axis=1)
    v2 = np.concatenate([O.paged_to_contiguous(vf, t2[:1], 16),
                         O.paged_to_contiguous(vf, t2[2:3], 16)], axis=1)
    want2 = O.decode_batch_f32(as_f32(q[2:3], dtype), k2[None], v2[None],
                               np.array([32], np.int32), 0.088)
    check("skipped page", got[2:3], want2, dtype)


def test_workspace_paths_and_prototype_launcher_agree(kv):
    rng = np.random.default_rng(10)
    hq, hkv, d, dtype = 16, 8, 128, "bf16"
    lens = rng.integers(100, 900, 12) + 1
    q, kp, vp, tables, lens = make_case(rng, lens, hq, hkv, d, dtype)
    qd, kd, vd = to_dev(q, dtype), to_dev(kp, dtype), to_dev(vp, dtype)
    a = run_decode(kv, qd, kd, vd, tables, lens, hq, hkv, d, dtype, 0.0883)
    ws = torch.zeros(kv.decode_workspace_size(len(lens), hq, hkv, d), dtype=torch.uint8,
                     device=DEV)
    b = run_decode(kv, qd, kd, vd, tables, lens, hq, hkv, d, dtype, 0.0883, workspace=ws)
    out = torch.empty_like(qd)
    t_dev, l_dev = to_dev(tables), to_dev(lens)  # keep the buffers alive until the kernel ran
    rc = kv.load().launch_paged_gqa_decode_tiled_bf16(
        qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), t_dev.data_ptr(), l_dev.data_ptr(),
        out.data_ptr(), len(lens), hq, hkv, tables.shape[1], 0.0883)
    assert rc == 0
    c = to_host(out)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(a, c)
    # repeated launches are deterministic
    np.testing.assert_array_equal(a, run_decode(kv, qd, kd, vd, tables, lens, hq, hkv, d, dtype,
                                                0.0883))
    with pytest.raises(kv.RlseError):
        small = torch.empty(16, dtype=torch.uint8, device=DEV)
        run_decode(kv, qd, kd, vd, tables, lens, hq, hkv, d, dtype, 0.0883, workspace=small)


def test_physical_placement_does_not_change_result(kv):
    """Moving every page to a different physical block (and rewriting the
    table) must give bit-identical output: the kernel sees only the table."""
    rng = np.random.default_rng(11)
    hq, hkv, d, dtype = 16, 8, 128, "bf16"
    lens = rng.integers(1, 700, 9) + 1
    q, kp, vp, tables, lens = make_case(rng, lens, hq, hkv, d, dtype)
    nb = kp.shape[0]
    perm = rng.permutation(nb)
    kp2, vp2 = np.empty_like(kp), np.empty_like(vp)
    kp2[perm], vp2[perm] = kp, vp
    t2 = perm[tables].astype(np.int32)
    for i, n in enumerate(lens):
        t2[i, (int(n) + 15) // 16:] = 0
    a = run_decode(kv, to_dev(q, dtype), to_dev(kp, dtype), to_dev(vp, dtype), tables, lens, hq,
                   hkv, d, dtype, 0.0883)
    b = run_decode(kv, to_dev(q, dtype), to_dev(kp2, dtype), to_dev(vp2, dtype), t2, lens, hq,
                   hkv, d, dtype, 0.0883)
    np.testing.assert_array_equal(a, b)


def _decode_ws_layout(kv, batch, hq, hkv, d):
    """(record offset in bytes, counter words) of a decode workspace: the
    256-byte header, one launch counter per wave of the 2 x CUs workgroups
    (4 waves each, rounded up to 64 words), then the tagged records."""
    w = 2 * torch.cuda.get_device_properties(0).multi_processor_count
    ctr = (w * 4 + 63) // 64 * 64
    off = (64 + ctr) * 4
    assert off + 2 * w * (hq // hkv * d + 2 * (hq // hkv)) * 8 == \
        kv.decode_workspace_size(batch, hq, hkv, d)
    return off, w * 4


def _plant_stale_records(ws, rec_off, n_ctr, rng):
    """Fills the record area with plausible partials whose tags are never the
    next launch's epoch: the last launch's (a publication that landed after
    its merge), the one after the next, and random others. Also checks the
    counter invariant: every counter word holds the last launch's epoch."""
    words = ws.view(torch.int32)
    ctr = words[64:64 + n_ctr].cpu().numpy().astype(np.uint32)
    assert (ctr == ctr[0]).all() and ctr[0] != 0, "launch counters diverged"
    ep = int(ctr[0])
    recs = ws[rec_off:].view(torch.int64)
    n = recs.numel()
    tags = rng.choice(np.array([ep, (ep + 2) & 0xFFFFFFFF], np.uint64), n)
    rand = rng.integers(1, 2**32, n, dtype=np.uint64)
    rand[rand == ep + 1] = ep
    tags = np.where(rng.random(n) < 0.2, rand, tags)
    vals = (np.abs(rng.standard_normal(n)) * 3).astype(np.float32).view(np.uint32).astype(np.uint64)
    recs.copy_(torch.from_numpy(((tags << np.uint64(32)) | vals).view(np.int64)).to(DEV))
    torch.cuda.synchronize()


def test_stale_records_are_never_taken(kv):
    """Rows cut between workgroups leave tagged partial records in the
    workspace, merged in the same launch. Records never need clearing: a
    merge takes only words carrying its launch's epoch. Between launches of
    different shapes the record area is filled with stale partials (tagged
    with the previous launch's epoch, a later one or random tags) and every
    output must still match the first pass bit for bit. Rows here span up
    to ~60 groups, so merges take several batches of records."""
    rng = np.random.default_rng(12)
    dtype = "bf16"
    cases = []
    for (hq, hkv, d), lens in [((16, 8, 128), [2049, 1500, 17, 800]),
                               ((16, 8, 128), [5, 4096, 300]),
                               ((16, 8, 128), [1] * 20 + [3000]),
                               ((32, 4, 128), [7, 8000, 33]),
                               ((8, 8, 64), [4096, 3, 1000])]:
        q, kp, vp, tables, lens = make_case(rng, lens, hq, hkv, d, dtype)
        cases.append(((hq, hkv, d), to_dev(q, dtype), to_dev(kp, dtype), to_dev(vp, dtype), tables,
                      lens, oracle_decode(q, kp, vp, tables, lens, dtype, 0.0883)))
    size = max(kv.decode_workspace_size(len(c[5]), *c[0]) for c in cases)
    ws = torch.zeros(size, dtype=torch.uint8, device=DEV)
    first = []
    for rep in range(2):
        for i, ((hq, hkv, d), qd, kd, vd, tables, lens, want) in enumerate(cases):
            print(f"case{i} rep{rep} Hq={hq} Hkv={hkv} d={d} lens={list(lens)[:4]}", flush=True)
            got = run_decode(kv, qd, kd, vd, tables, lens, hq, hkv, d, dtype, 0.0883,
                             workspace=ws)
            check(f"case{i} rep{rep}", as_f32(got, dtype), want, dtype)
            if rep == 0:
                first.append(got)
            else:
                np.testing.assert_array_equal(got, first[i])
            assert kv.workspace_flags(ws) == 0
            off, n_ctr = _decode_ws_layout(kv, len(lens), hq, hkv, d)
            _plant_stale_records(ws, off, n_ctr, rng)


def test_merge_timeout_is_reported_and_later_launches_are_exact(kv):
    """A merge that gives up waiting writes NaN for its row and raises
    RLSE_WS_ERR_MERGE_TIMEOUT; rows it did not touch are exact. The bound is
    forced to zero from the host (give up at the first miss), so every
    kernel still ends normally; publications that land after their merge
    gave up stay in the workspace, and the next launches -- with the
    default bound -- must not take them."""
    rng = np.random.default_rng(41)
    hq, hkv, d, dtype = 16, 8, 128, "bf16"
    lens = rng.integers(128, 2049, 32) + 1
    q, kp, vp, tables, lens = make_case(rng, lens, hq, hkv, d, dtype)
    qd, kd, vd = to_dev(q, dtype), to_dev(kp, dtype), to_dev(vp, dtype)
    ws = torch.zeros(kv.decode_workspace_size(len(lens), hq, hkv, d), dtype=torch.uint8,
                     device=DEV)
    print("timeout: B=32 U[128,2048] Hq=16 Hkv=8 d=128 bf16, reference launch", flush=True)
    ref = run_decode(kv, qd, kd, vd, tables, lens, hq, hkv, d, dtype, 0.0883, workspace=ws)
    assert kv.workspace_flags(ws) == 0
    kv.set_merge_wait_ns(0)
    try:
        print("timeout: launch with a zero wait bound", flush=True)
        got = run_decode(kv, qd, kd, vd, tables, lens, hq, hkv, d, dtype, 0.0883, workspace=ws)
    finally:
        kv.set_merge_wait_ns(100_000_000)
    flags = kv.workspace_flags(ws)
    gf = as_f32(got, dtype)
    nan_heads = np.isnan(gf).any(axis=2)
    print(f"timeout: flags={flags} NaN heads={int(nan_heads.sum())}", flush=True)
    assert bool(flags & kv.WS_ERR_MERGE_TIMEOUT) == bool(nan_heads.any())
    assert flags & ~kv.WS_ERR_MERGE_TIMEOUT == 0
    assert np.isnan(gf[nan_heads]).all()      # a timed-out head is NaN throughout
    np.testing.assert_array_equal(got[~nan_heads], ref[~nan_heads])
    for rep in range(3):
        again = run_decode(kv, qd, kd, vd, tables, lens, hq, hkv, d, dtype, 0.0883, workspace=ws)
        np.testing.assert_array_equal(again, ref, err_msg=f"launch {rep} after the timeout")
        assert kv.workspace_flags(ws) == 0


def test_over_capacity_row_is_invalid_in_the_fused_step(kv):
    """A sequence whose length exceeds its block table's capacity is an
    invalid row for rlse_decode_step: nothing is appended for it (its pages
    are unchanged), its output is zeros and RLSE_WS_ERR_LENGTH is raised;
    the other rows are computed as usual."""
    rng = np.random.default_rng(43)
    hq, hkv, d, dtype = 16, 8, 128, "bf16"
    lens = np.array([40, 300, 47], np.int32)
    q, kp, vp, tables, lens = make_case(rng, lens, hq, hkv, d, dtype)
    b, mbps, nb = len(lens), tables.shape[1], kp.shape[0]
    bad = lens.copy()
    bad[2] = mbps * 16 + 1   # one past what row 2's table can hold
    k_new = random_values(rng, (b, hkv, d), dtype)
    v_new = random_values(rng, (b, hkv, d), dtype)
    max_pos = (mbps + 1) * 16
    c, s = _rope_tables_dev(kv, 1e6, d, max_pos, dtype)
    args = lambda kp_, vp_, out_, l_: (to_dev(q, dtype), to_dev(k_new, dtype),  # noqa: E731
                                       to_dev(v_new, dtype), None, None, 1e-6, to_dev(c, dtype),
                                       to_dev(s, dtype), max_pos, kp_, vp_, to_dev(tables),
                                       to_dev(l_), out_, b, hq, hkv, d, mbps, nb, 0.0883, dtype)
    ws = torch.zeros(kv.decode_workspace_size(b, hq, hkv, d), dtype=torch.uint8, device=DEV)
    outs, pools = [], []
    for l_ in (lens, bad):
        kp_, vp_ = to_dev(kp, dtype), to_dev(vp, dtype)
        out_ = torch.full((b, hq, d), 3.0, dtype=torch.bfloat16, device=DEV)
        kv.decode_step(*args(kp_, vp_, out_, l_), ws, ws.numel())
        outs.append(to_host(out_))
        pools.append((to_host(kp_), to_host(vp_)))
        assert kv.workspace_flags(ws) == (0 if l_ is lens else kv.WS_ERR_LENGTH)
    np.testing.assert_array_equal(outs[1][:2], outs[0][:2])
    assert (as_f32(outs[1][2], dtype) == 0).all()
    # rows 0 and 1 appended as before; row 2's pages hold the original K/V
    pk0, pv0 = pools[0]
    pk1, pv1 = pools[1]
    rows2 = tables[2, :(int(lens[2]) + 15) // 16]
    np.testing.assert_array_equal(pk1[rows2], kp[rows2])
    np.testing.assert_array_equal(pv1[rows2], vp[rows2])
    others = np.setdiff1d(np.arange(nb), rows2)
    np.testing.assert_array_equal(pk1[others], pk0[others])
    np.testing.assert_array_equal(pv1[others], pv0[others])


def test_decode_is_deterministic_across_launches(kv):
    """Rows cut between workgroups are merged in the same launch with their
    pieces combined in a fixed order, whatever order the groups finish in, so
    repeated launches on the same inputs give bit-identical outputs."""
    rng = np.random.default_rng(21)
    hq, hkv, d, dtype = 16, 8, 128, "bf16"
    lens = rng.integers(128, 2049, 32)
    q, kp, vp, tables, lens = make_case(rng, lens, hq, hkv, d, dtype)
    qd, kd, vd = to_dev(q, dtype), to_dev(kp, dtype), to_dev(vp, dtype)
    print("determinism: B=32 U[128,2048] Hq=16 Hkv=8 d=128 bf16, 10 launches", flush=True)
    first = run_decode(kv, qd, kd, vd, tables, lens, hq, hkv, d, dtype, 0.0883)
    check("determinism vs oracle", as_f32(first, dtype),
          oracle_decode(q, kp, vp, tables, lens, dtype, 0.0883), dtype)
    for rep in range(9):
        again = run_decode(kv, qd, kd, vd, tables, lens, hq, hkv, d, dtype, 0.0883)
        np.testing.assert_array_equal(again, first, err_msg=f"launch {rep + 1}")


# ------------------------------------------------------------- fused step ----
def _rope_tables_dev(kv, theta, d, max_pos, dtype):
    np_dt = {"f32": np.float32, "bf16": np.uint16, "f16": np.float16}[dtype]
    cb, sb = kv.rope_tables(theta, d, max_pos, dtype)
    c = np.frombuffer(cb, np_dt).reshape(max_pos, d // 2).copy()
    s = np.frombuffer(sb, np_dt).reshape(max_pos, d // 2).copy()
    return c, s


@pytest.mark.parametrize("dtype,hq,hkv,d,norm,lens", [
    ("bf16", 16, 8, 128, True, [1, 2, 16, 17, 300, 513, 2049, 1000, 31]),   # Qwen3-0.6B
    ("bf16", 14, 2, 64, False, [5, 4097, 100, 16, 33]),                       # Qwen2.5, no qk-norm
    ("f32", 16, 8, 128, True, [513]),                                          # Qwen3 f32, one sequence of 513 keys
    ("f16", 32, 8, 128, True, [70, 1, 900]),                                   # Qwen3-8B heads
])
def test_fused_decode_step_matches_two_kernel_path_and_oracle(kv, dtype, hq, hkv, d, norm, lens):
    """rlse_decode_step (norm + RoPE + append + decode in one launch) against
    rlse_qk_norm_rope_append followed by rlse_paged_gqa_decode, and against
    the oracle's Candle op chain (RmsNorm, apply_rope, KvCache append, zero-copy
    GQA decode; src/backends/qwen2.rs:291-328)."""
    rng = np.random.default_rng(31 + d + hq)
    lens = np.asarray(lens, np.int32)
    q, kp, vp, tables, lens = make_case(rng, lens, hq, hkv, d, dtype)
    b, mbps, nb = len(lens), tables.shape[1], kp.shape[0]
    k_new = random_values(rng, (b, hkv, d), dtype)
    v_new = random_values(rng, (b, hkv, d), dtype)
    w = lambda: random_values(rng, (d,), dtype) if norm else None  # noqa: E731
    qw, kw = w(), w()
    if norm and dtype != "bf16":
        qw = (1 + 0.1 * rng.standard_normal(d)).astype(qw.dtype)
        kw = (1 + 0.1 * rng.standard_normal(d)).astype(kw.dtype)
    elif norm:
        qw = O.f32_to_bf16_bits(1 + 0.1 * rng.standard_normal(d))
        kw = O.f32_to_bf16_bits(1 + 0.1 * rng.standard_normal(d))
    max_pos = mbps * 16
    c, s = _rope_tables_dev(kv, 1e6, d, max_pos, dtype)
    scale = 1.0 / math.sqrt(d)
    dev = lambda a: None if a is None else to_dev(a, dtype)  # noqa: E731
    t_dev, l_dev = to_dev(tables), to_dev(lens)
    c_dev, s_dev = to_dev(c, dtype), to_dev(s, dtype)

    # fused
    kp1, vp1 = to_dev(kp, dtype), to_dev(vp, dtype)
    out1 = torch.empty_like(to_dev(q, dtype))
    kv.decode_step(dev(q), dev(k_new), dev(v_new), dev(qw), dev(kw), 1e-6, c_dev, s_dev, max_pos,
                   kp1, vp1, t_dev, l_dev, out1, b, hq, hkv, d, mbps, nb, scale, dtype)
    # two kernels
    kp2, vp2 = to_dev(kp, dtype), to_dev(vp, dtype)
    qrot = torch.empty_like(out1)
    pos = lens - 1
    kv.qk_norm_rope_append(dev(q), dev(k_new), dev(v_new), dev(qw), dev(kw), 1e-6, c_dev, s_dev,
                           max_pos, to_dev(pos), t_dev, b, None, b, hq, hkv, d, mbps, nb, qrot,
                           kp2, vp2, dtype)
    out2 = run_decode(kv, qrot, kp2, vp2, tables, lens, hq, hkv, d, dtype, scale)
    got = as_f32(to_host(out1), dtype)
    check(f"fused vs two-kernel {dtype} G={hq // hkv}", got, as_f32(out2, dtype), dtype)
    # both entry points write the same pool bytes: the RMSNorm of k follows
    # one reduction order in every K writer
    pk1, pv1, pk2, pv2 = (to_host(x) for x in (kp1, vp1, kp2, vp2))
    np.testing.assert_array_equal(pv1, pv2)
    np.testing.assert_array_equal(pk1, pk2)
    # oracle chain on the appended pool
    norm_f = (O.rmsnorm_bf16 if dtype == "bf16" else None)
    if dtype == "bf16":
        qn = q.reshape(-1, d) if not norm else norm_f(q.reshape(-1, d), qw, 1e-6)
        q_ref = O.bf16_bits_to_f32(O.apply_rope_bf16(qn, np.repeat(pos, hq), c, s))
    else:
        qf = q.astype(np.float32).reshape(-1, d)
        qn = O.rmsnorm_f32(qf, qw.astype(np.float32), 1e-6) if norm else qf
        q_ref = O.apply_rope_f32(qn, np.repeat(pos, hq), c.astype(np.float32),
                                 s.astype(np.float32))
        if dtype == "f16":
            q_ref = q_ref.astype(np.float16).astype(np.float32)
    want = O.decode_paged_f32(q_ref.reshape(b, hq, d), as_f32(pk1, dtype), as_f32(pv1, dtype),
                              tables, lens, scale)
    check(f"fused vs oracle {dtype} G={hq // hkv}", got, want, dtype)


@pytest.mark.parametrize("hq,hkv,d,lens", [
    (16, 8, 128, [1, 2, 15, 16, 17, 33, 300, 2049, 0, 64]),     # Qwen3 shape, ragged, an empty row
    (14, 2, 64, [4097] * 6 + [5, 0]),                           # Qwen2.5 shape, G = 7
    (8, 8, 64, [20]),                                           # most workgroups idle
    (2, 2, 64, [16384] * 72),                                   # > 64 blocks per wave
])
def test_planned_step_equals_unplanned(kv, hq, hkv, d, lens):
    """rlse_decode_step_planned with a plan from rlse_decode_plan, with
    cacheable or streamed (RLSE_DECODE_STREAM) pages, gives the outputs and
    pool contents of rlse_decode_step bit for bit, including rows
    of length 0, idle workgroups and waves whose range spans several 64-block
    chunks."""
    dtype = "bf16"
    rng = np.random.default_rng(len(lens) * 7 + d)
    lens = np.asarray(lens, np.int32)
    b = len(lens)
    mbps = max(1, int(max((int(n) + 15) // 16 for n in lens)))
    nb = int(sum((int(n) + 15) // 16 for n in lens)) + 3
    tables = build_tables(rng, lens, nb, mbps)
    g = torch.Generator(device=DEV)
    g.manual_seed(5)
    bf = torch.bfloat16
    kp = torch.randn((nb, hkv, 16, d), generator=g, device=DEV).to(bf)
    vp = torch.randn((nb, hkv, 16, d), generator=g, device=DEV).to(bf)
    q = torch.randn((b, hq, d), generator=g, device=DEV).to(bf)
    kn = torch.randn((b, hkv, d), generator=g, device=DEV).to(bf)
    vn = torch.randn((b, hkv, d), generator=g, device=DEV).to(bf)
    qw = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(bf)
    kw = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(bf)
    max_pos = mbps * 16
    cos_b, sin_b = kv.rope_tables(1e6, d, max_pos, "bf16")
    c = torch.frombuffer(bytearray(cos_b), dtype=torch.int16).to(DEV).view(bf)
    s = torch.frombuffer(bytearray(sin_b), dtype=torch.int16).to(DEV).view(bf)
    t_dev, l_dev = to_dev(tables), to_dev(lens)
    scale = 1.0 / math.sqrt(d)
    outs, pools = [], []
    plan = torch.zeros(kv.decode_plan_size(), dtype=torch.uint8, device=DEV)
    # unplanned; planned with cacheable pages; planned streaming (twice)
    for planned, stream_pages in ((False, False), (True, False), (True, True), (True, True)):
        kp_i, vp_i = kp.clone(), vp.clone()
        out = torch.full((b, hq, d), 3.0, dtype=bf, device=DEV)
        args = (q, kn, vn, qw, kw, 1e-6, c, s, max_pos, kp_i, vp_i, t_dev, l_dev, out, b, hq, hkv,
                d, mbps, nb, scale, "bf16")
        if planned:
            kv.decode_plan(t_dev, l_dev, b, hkv, mbps, nb, plan, plan.numel())
            kv.decode_step_planned(*args, plan, stream_pages=stream_pages)
        else:
            kv.decode_step(*args)
        torch.cuda.synchronize()
        outs.append(out)
        pools.append((kp_i, vp_i))
    for i in (1, 2, 3):
        assert torch.equal(outs[0].view(torch.int16), outs[i].view(torch.int16)), i
        assert torch.equal(pools[0][0].view(torch.int16), pools[i][0].view(torch.int16)), i
        assert torch.equal(pools[0][1].view(torch.int16), pools[i][1].view(torch.int16)), i
    print(f"[planned] hq={hq} hkv={hkv} d={d} B={b}: outputs and pools identical")


def test_workspace_check_races_library_workspace_growth(kv):
    """rlse_workspace_check on the library-owned workspace while another
    host thread grows it (decode calls with no workspace at growing group
    sizes: each growth frees and reallocates the buffer). The check holds the
    workspace's mutex until its read and clear are queued, so it never
    touches a freed buffer; every call returns OK and no flag is raised."""
    import threading
    rng = np.random.default_rng(29)
    hkv, d, lens = 2, 128, np.array([40, 200, 17], np.int32)
    cases = []
    for g in range(1, 9):          # the workspace's records grow with the group size
        q, kp, vp, tables, _ = make_case(rng, lens, g * hkv, hkv, d, "bf16")
        cases.append((g, to_dev(q, "bf16"), to_dev(kp, "bf16"), to_dev(vp, "bf16"), tables))
    errors = []

    def grow():
        try:
            for g, q, kp, vp, tables in cases:
                out = torch.empty_like(q)
                kv.paged_gqa_decode(q, kp, vp, to_dev(tables), to_dev(lens), out, len(lens),
                                    g * hkv, hkv, d, tables.shape[1], kp.shape[0],
                                    1.0 / math.sqrt(d), "bf16")
                torch.cuda.synchronize()
        except Exception as e:  # noqa: BLE001 -- reported below
            errors.append(e)

    t = threading.Thread(target=grow)
    t.start()
    checks = 0
    while t.is_alive() or checks < 20:
        assert kv.workspace_flags() == 0
        checks += 1
    t.join()
    assert not errors, errors
    print(f"workspace growth x {len(cases)} with {checks} concurrent checks: clean")
