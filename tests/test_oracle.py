"""Pins the oracle (oracle/rlse_oracle.c + oracle/oracle.py) before it is trusted.

How each oracle function is pinned (no stored numeric vectors exist in the
reference for this path, and the reference cannot be built here):

* decode_batch_f32 (qwen2.rs:177-203): against the float64 textbook form;
  L=1 gives the V row; q=0 gives the mean of V; zero-copy GQA equals
  repeat_kv (the reference's own test, qwen2.rs:822-879, same shape, 1e-5);
  a planted head-mapping mistake is caught; golden vectors.
* prefill_f32 (qwen2.rs:329-345, 476-503): float64 textbook; a one-token
  chunk equals decode over offset+1 keys; with offset 0 the first query sees
  only key 0; golden vectors.
* rmsnorm_f32/bf16/f16 (qwen2.rs:68-75): constant-row closed form; float64
  form; scale invariance; golden vectors. The sum of squares follows one
  fixed order (sumsq_tree: 16-byte packets, then a pairwise tree), pinned by
  exact integer rows, a row built so that the packet split and the tree
  decide the rounded result (a sequential sum or another packet size gives
  other bits), a float64 error bound and an independent numpy restatement.
* rope tables / apply_rope (qwen2.rs:90-142): position 0 is the identity
  (bit-exact); rotations preserve the pair norms; inv_freq against
  theta^(-2i/d); float64 rotation; golden vectors.
* KvCache append/narrow (qwen2.rs:349-361): buffer capacity and contents
  against numpy slicing; over-capacity append rejected.
* paged layout (mini_serve_kernels.cu:68-70): a paged write followed by the
  contiguous read-out equals the KvCache snapshot byte for byte.
* KVCacheModel (kv_cache.rs): the reference's own tests (test_kv_cache.rs).
"""
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- decode ----
def _contig(rng, b, hkv, cap, d):
    return rng.standard_normal((b, hkv, cap, d)).astype(np.float32)


def test_decode_matches_float64_textbook():
    rng = _rng(1)
    b, hq, hkv, d, cap = 3, 16, 8, 128, 70
    q = rng.standard_normal((b, hq, d)).astype(np.float32)
    k, v = _contig(rng, b, hkv, cap, d), _contig(rng, b, hkv, cap, d)
    lens = np.array([1, 33, 70], dtype=np.int32)
    scale = 1.0 / np.sqrt(d)
    out = O.decode_batch_f32(q, k, v, lens, scale)
    for i in range(b):
        ref = O.decode_f64(q[i], k[i, :, :lens[i]], v[i, :, :lens[i]], scale)
        np.testing.assert_allclose(out[i], ref, rtol=1e-5, atol=2e-6)


def test_decode_single_key_returns_value_row():
    rng = _rng(2)
    q = rng.standard_normal((1, 4, 64)).astype(np.float32)
    k, v = _contig(rng, 1, 2, 5, 64), _contig(rng, 1, 2, 5, 64)
    out = O.decode_batch_f32(q, k, v, np.array([1], np.int32), 0.125)
    # softmax over one key is exactly 1, so every head returns its KV head's V[0]
    np.testing.assert_array_equal(out[0, 0], v[0, 0, 0])
    np.testing.assert_array_equal(out[0, 3], v[0, 1, 0])


def test_decode_zero_query_averages_values():
    rng = _rng(3)
    q = np.zeros((1, 14, 64), np.float32)
    k, v = _contig(rng, 1, 2, 100, 64), _contig(rng, 1, 2, 100, 64)
    out = O.decode_batch_f32(q, k, v, np.array([100], np.int32), 0.125)
    np.testing.assert_allclose(out[0, 0], v[0, 0].mean(axis=0), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out[0, 13], v[0, 1].mean(axis=0), rtol=1e-5, atol=1e-6)


def test_zero_copy_gqa_equals_repeat_kv():
    """Reference test test_gqa_broadcast_matmul (qwen2.rs:822-879): Hq=14, Hkv=2,
    d=64, L=100; max diff between zero-copy GQA and repeat_kv < 1e-5."""
    rng = _rng(4)
    q = rng.standard_normal((2, 14, 64)).astype(np.float32)
    k, v = _contig(rng, 2, 2, 100, 64), _contig(rng, 2, 2, 100, 64)
    lens = np.array([100, 100], np.int32)
    scale = 1.0 / np.sqrt(64)
    zc = O.decode_batch_f32(q, k, v, lens, scale)
    for i in range(2):
        # repeat_kv: materialise the repeated K/V and run plain MHA per head
        kr = np.repeat(k[i], 7, axis=0)
        vr = np.repeat(v[i], 7, axis=0)
        s = np.einsum("hd,hld->hl", q[i].astype(np.float64), kr) * scale
        rep = np.einsum("hl,hld->hd", O.softmax_f64(s), vr)
        assert np.abs(zc[i] - rep).max() < 1e-5


def test_planted_head_mapping_mistake_is_caught():
    """A decode that maps query head h to KV head h % Hkv (instead of h // G)
    must fail the repeat_kv comparison above."""
    rng = _rng(5)
    q = rng.standard_normal((14, 64)).astype(np.float32)
    k = rng.standard_normal((2, 100, 64)).astype(np.float32)
    v = rng.standard_normal((2, 100, 64)).astype(np.float32)
    good = O.decode_f64(q, k, v, 0.125)
    wrong_k = k[np.arange(14) % 2]
    wrong_v = v[np.arange(14) % 2]
    s = np.einsum("hd,hld->hl", q.astype(np.float64), wrong_k) * 0.125
    bad = np.einsum("hl,hld->hd", O.softmax_f64(s), wrong_v)
    assert np.abs(good - bad).max() > 1e-2


# --------------------------------------------------------------- prefill ----
def test_prefill_matches_float64_textbook():
    rng = _rng(6)
    hq, hkv, d, offset, ql = 8, 2, 64, 40, 24
    q = rng.standard_normal((hq, ql, d)).astype(np.float32)
    k = rng.standard_normal((hkv, offset + ql, d)).astype(np.float32)
    v = rng.standard_normal((hkv, offset + ql, d)).astype(np.float32)
    out = O.prefill_f32(q, k, v, offset, 0.125)
    ref = O.prefill_f64(q, k, v, offset, 0.125)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=2e-6)


def test_prefill_single_token_chunk_equals_decode():
    rng = _rng(7)
    hq, hkv, d, offset = 16, 8, 128, 37
    q = rng.standard_normal((hq, 1, d)).astype(np.float32)
    k = rng.standard_normal((hkv, offset + 1, d)).astype(np.float32)
    v = rng.standard_normal((hkv, offset + 1, d)).astype(np.float32)
    pf = O.prefill_f32(q, k, v, offset, 0.09)
    dc = O.decode_batch_f32(q[:, 0][None], k[None], v[None], np.array([offset + 1], np.int32),
                            0.09)
    np.testing.assert_allclose(pf[:, 0], dc[0], rtol=1e-6, atol=1e-7)


def test_prefill_first_query_sees_only_first_key():
    rng = _rng(8)
    q = rng.standard_normal((4, 5, 32)).astype(np.float32)
    k = rng.standard_normal((2, 5, 32)).astype(np.float32)
    v = rng.standard_normal((2, 5, 32)).astype(np.float32)
    out = O.prefill_f32(q, k, v, 0, 0.2)
    np.testing.assert_array_equal(out[0, 0], v[0, 0])
    np.testing.assert_array_equal(out[3, 0], v[1, 0])


# --------------------------------------------------------------- rmsnorm ----
def test_rmsnorm_constant_row_closed_form():
    # x = c everywhere: out = c / sqrt(c^2 + eps) * w
    c, eps, n = -3.5, 1e-6, 128
    x = np.full((1, n), c, np.float32)
    w = (1.0 + 0.1 * _rng(9).standard_normal(n)).astype(np.float32)
    out = O.rmsnorm_f32(x, w, eps)
    expect = (c / np.sqrt(c * c + eps)) * w.astype(np.float64)
    np.testing.assert_allclose(out[0], expect, rtol=2e-7, atol=0)


def test_rmsnorm_matches_float64_and_is_scale_invariant():
    rng = _rng(10)
    for n in (128, 1024):
        x = rng.standard_normal((17, n)).astype(np.float32)
        w = rng.standard_normal(n).astype(np.float32)
        out = O.rmsnorm_f32(x, w, 1e-6)
        np.testing.assert_allclose(out, O.rmsnorm_f64(x, w, 1e-6), rtol=2e-6, atol=2e-6)
        out4 = O.rmsnorm_f32(x * np.float32(4.0), w, 0.0)
        np.testing.assert_allclose(out4, O.rmsnorm_f32(x, w, 0.0), rtol=1e-6, atol=1e-6)


def _sumsq_tree_numpy(x, epl):
    """The packet-then-tree order written with numpy array operations."""
    x = np.asarray(x, np.float32)
    n = x.shape[-1]
    np_ = -(-n // epl)
    p2 = 1 << (np_ - 1).bit_length()
    pad = np.zeros(x.shape[:-1] + (p2 * epl,), np.float32)
    pad[..., :n] = x
    sq = (pad * pad).reshape(x.shape[:-1] + (p2, epl))
    acc = np.zeros(x.shape[:-1] + (p2,), np.float32)
    for e in range(epl):
        acc = acc + sq[..., e]
    while acc.shape[-1] > 1:
        acc = acc[..., 0::2] + acc[..., 1::2]
    return acc[..., 0]


@pytest.mark.parametrize("epl", [4, 8])
def test_sumsq_tree_order(epl):
    rng = _rng(40 + epl)
    for n in (1, 3, 8, 9, 64, 100, 128, 896, 1024, 5000):
        x = (rng.standard_normal((6, n)) * rng.uniform(0.1, 30, (6, 1))).astype(np.float32)
        got = O.sumsq_tree(x, epl)
        np.testing.assert_array_equal(got, _sumsq_tree_numpy(x, epl))
        exact = (x.astype(np.float64) ** 2).sum(-1)
        # pairwise summation error bound: (epl + log2(packets)) ulps of the sum
        depth = epl + int(np.ceil(np.log2(max(1, -(-n // epl))))) + 1
        assert np.all(np.abs(got - exact) <= depth * 2.0 ** -24 * exact)
        ints = rng.integers(-5, 6, (3, n)).astype(np.float32)   # every partial sum exact
        np.testing.assert_array_equal(O.sumsq_tree(ints, epl), (ints.astype(np.int64) ** 2).sum(-1))


def test_sumsq_tree_packet_split_decides_rounding():
    # x^2 = 2^24 then ones: inside a packet each 1 is lost to 2^24 (ties to
    # even), across packets the tree adds the other packets' sums exactly.
    x = np.ones(16, np.float32)
    x[0] = 4096.0
    assert O.sumsq_tree(x, 4) == 2.0 ** 24 + 12   # packets [2^24, 4, 4, 4]
    assert O.sumsq_tree(x, 8) == 2.0 ** 24 + 8    # packets [2^24, 8]
    seq = np.float32(0)
    for v in x:
        seq = np.float32(seq + v * v)
    assert seq == 2.0 ** 24                      # a sequential sum loses all 15
    # the f32 norm uses 4-element packets, the 16-bit norms 8-element ones
    w = np.ones(16, np.float32)
    assert O.rmsnorm_f32(x[None], w, 0.0)[0, 1] == np.float32(1.0) / np.sqrt(
        np.float32(2.0 ** 24 + 12) * np.float32(1.0 / 16))


def test_rmsnorm_bf16_within_bf16_rounding():
    rng = _rng(11)
    x = O.f32_to_bf16_bits(rng.standard_normal((4, 128)))
    w = O.f32_to_bf16_bits(1.0 + 0.1 * rng.standard_normal(128))
    out = O.bf16_bits_to_f32(O.rmsnorm_bf16(x, w, 1e-6))
    ref = O.rmsnorm_f64(O.bf16_bits_to_f32(x), O.bf16_bits_to_f32(w), 1e-6)
    # two bf16 roundings (x_normed, then the product): < 2 * 2^-8 relative
    np.testing.assert_allclose(out, ref, rtol=2 ** -7, atol=1e-6)


def test_bf16_rounding_is_nearest_even():
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9, -2.5, np.inf],
                    np.float32)
    bits = O.f32_to_bf16_bits(vals)
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: rounds to the even (1.0)
    assert O.bf16_bits_to_f32(bits).tolist() == [1.0, 1.0, 1.0 + 2 ** -6, 1.0, -2.5, np.inf]


# ------------------------------------------------------------------ rope ----
def test_rope_tables_follow_reference_formula():
    theta, d = 1e6, 128
    c, s = O.rope_tables_f32(theta, d, 600)
    inv = theta ** (-(2.0 * np.arange(d // 2)) / d)
    np.testing.assert_allclose(np.arctan2(s[1], c[1]), inv, rtol=1e-6)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)


def test_rope_position_zero_is_identity_and_norm_preserving():
    rng = _rng(12)
    d = 128
    c, s = O.rope_tables_f32(1e6, d, 1024)
    x = rng.standard_normal((6, d)).astype(np.float32)
    y0 = O.apply_rope_f32(x, np.zeros(6, np.int32), c, s)
    np.testing.assert_array_equal(y0, x)
    pos = np.array([1, 5, 17, 100, 512, 1023], np.int32)
    y = O.apply_rope_f32(x, pos, c, s)
    half = d // 2
    n_in = x[:, :half] ** 2 + x[:, half:] ** 2
    n_out = y[:, :half].astype(np.float64) ** 2 + y[:, half:].astype(np.float64) ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(y, O.rope_f64(x, pos, 1e6), rtol=0, atol=2e-4)


def test_rope_bf16_matches_float64_within_rounding():
    rng = _rng(13)
    d = 128
    c, s = O.rope_tables_f32(1e6, d, 600)
    cb, sb = O.f32_to_bf16_bits(c), O.f32_to_bf16_bits(s)
    x = O.f32_to_bf16_bits(rng.standard_normal((4, d)))
    pos = np.array([0, 3, 300, 512], np.int32)
    y = O.bf16_bits_to_f32(O.apply_rope_bf16(x, pos, cb, sb))
    ref = O.rope_f64(O.bf16_bits_to_f32(x), pos, 1e6)
    np.testing.assert_allclose(y, ref, rtol=0, atol=0.05)
    np.testing.assert_array_equal(y[0], O.bf16_bits_to_f32(x[0]))


# --------------------------------------------------------- kv movement ----
def test_kvcache_append_and_capacity():
    rng = _rng(14)
    hkv, cap, d = 2, 24, 8
    kc = O.KvCacheC(hkv, cap, d, np.float32)
    assert kc.k.size == hkv * d * cap  # candle.rs:1347-1361 capacity fact (2*8*24)
    rows = [rng.standard_normal((hkv, q, d)).astype(np.float32) for q in (16, 1, 1, 5)]
    for r in rows:
        kc.append(r, -r)
    k, v = kc.snapshot()
    np.testing.assert_array_equal(k, np.concatenate(rows, axis=1))
    np.testing.assert_array_equal(v, -np.concatenate(rows, axis=1))
    assert kc.cur_len == 23
    with pytest.raises(ValueError):
        kc.append(rows[3][:, :2], rows[3][:, :2])


def test_paged_layout_round_trip_equals_kvcache_bytes():
    rng = _rng(15)
    hkv, d, nb = 8, 128, 40
    pool = np.zeros((nb, hkv, 16, d), np.uint16)
    table = rng.permutation(nb).astype(np.int32)
    kc = O.KvCacheC(hkv, 600, d, np.uint16)
    for pos in range(333):
        row = rng.integers(0, 65535, (hkv, d), dtype=np.uint16)
        O.paged_write_token(pool, table, pos, row)
        kc.append(row[:, None, :], row[:, None, :])
    np.testing.assert_array_equal(O.paged_to_contiguous(pool, table, 333), kc.snapshot()[0])


# ------------------------------------------------------------ block model ----
def test_kvcache_model_reference_tests():
    c = O.KVCacheModel(100, 16)
    assert c.allocate("req-1", 32) == [0, 1]
    assert len(c.free) == 98
    assert c.release("req-1") == 2 and len(c.free) == 100
    c = O.KVCacheModel(4, 16)
    with pytest.raises(MemoryError, match="Requested 5 blocks"):
        c.allocate("req-over", 80)
    c = O.KVCacheModel(10, 16)
    for r in ("req-1", "req-2", "req-3"):
        c.allocate(r, 16)
    c.release("req-2")
    total, alloc, free, util, frag = c.stats()
    assert (total, free) == (10, 8) and util > 0
    # free = {1, 3..9}: runs {1}, {3..9} -> (2 - 1) / 8 = 0.125
    assert frag == pytest.approx(0.125)


# --------------------------------------------------------------- golden ----
def _golden(name):
    path = os.path.join(GOLDEN, name)
    return np.load(path, allow_pickle=False)


def test_golden_decode_vectors():
    for name in ("decode_f32.npz", "decode_gqa7_f32.npz"):
        g = _golden(name)
        f = O.bf16_bits_to_f32
        out = O.decode_paged_f32(f(g["q"]), f(g["k_pool"]), f(g["v_pool"]), g["tables"],
                                 g["lens"], float(g["scale"]))
        np.testing.assert_allclose(out, g["out_f64"], rtol=1e-5, atol=3e-6)


def test_golden_prefill_vectors():
    g = _golden("prefill_f32.npz")
    out = O.prefill_f32(g["q"], g["k"], g["v"], int(g["offset"]), float(g["scale"]))
    np.testing.assert_allclose(out, g["out_f64"], rtol=1e-5, atol=3e-6)


def test_golden_norm_rope_vectors():
    g = _golden("norm_rope_f32.npz")
    out = O.rmsnorm_f32(g["x"], g["w"], float(g["eps"]))
    np.testing.assert_allclose(out, g["rms_f64"], rtol=2e-6, atol=2e-6)
    c, s = O.rope_tables_f32(float(g["theta"]), g["x"].shape[1], int(g["pos"].max()) + 1)
    y = O.apply_rope_f32(g["x"], g["pos"], c, s)
    # The f32 angle t * inv_freq carries up to t * 2^-24 rad of rounding (the
    # reference tables are f32 too), so the bound grows with the position.
    bound = 2.0 * float(g["pos"].max()) * 2.0 ** -24 * float(np.abs(g["x"]).max()) + 1e-5
    np.testing.assert_allclose(y, g["rope_f64"], rtol=0, atol=bound)


# ------------------------------------------------------------ checksums ----
def _mix_py(w, t, j):
    m = 0xFFFFFFFF
    return ((w ^ ((t * 0x9E3779B1 + j * 0x85EBCA77) & m)) * 0xC2B2AE3D) & m


def test_mix_words_wraps_like_integer_arithmetic():
    """mix_words in numpy uint32 equals the definition in Python integers
    reduced mod 2^32, extreme operands included."""
    rng = np.random.default_rng(3)
    w = np.concatenate([rng.integers(0, 2**32, 500, dtype=np.uint64),
                        np.array([0, 1, 2**31, 2**32 - 1], np.uint64)]).astype(np.uint32)
    t = rng.integers(0, 2**31, w.size).astype(np.uint32)
    j = rng.integers(0, 64, w.size).astype(np.uint32)
    got = O.mix_words(w, t, j)
    want = np.array([_mix_py(int(a), int(b), int(c)) for a, b, c in zip(w, t, j)], np.uint64)
    np.testing.assert_array_equal(got.astype(np.uint64), want)


def _checksum_brute(kp, vp, tables, lens):
    nb, hkv = kp.shape[:2]
    kw = kp.view(np.uint32).reshape(nb, hkv, 16, -1)
    vw = vp.view(np.uint32).reshape(nb, hkv, 16, -1)
    out = np.zeros((len(lens), hkv, 2), np.uint64)
    for b, n in enumerate(lens):
        if n <= 0 or n > 16 * tables.shape[1]:
            continue
        for t in range(n):
            pid = int(tables[b, t // 16])
            if not 0 <= pid < nb:
                continue
            for h in range(hkv):
                for j in range(kw.shape[-1]):
                    out[b, h, 0] += _mix_py(int(kw[pid, h, t % 16, j]), t, j)
                    out[b, h, 1] += _mix_py(int(vw[pid, h, t % 16, j]), t, j)
    return (out & 0xFFFFFFFF).astype(np.uint32)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_kv_checksum_ref_matches_brute_force(dt):
    """kv_checksum_ref against a position-by-position loop: ragged lengths,
    a page id outside the pool (skipped), an empty row and a row longer than
    its table (both 0)."""
    rng = np.random.default_rng(5)
    nb, hkv, d, mbps = 9, 2, 8, 3
    shape = (nb, hkv, 16, d)
    if dt == "f32":
        kp, vp = (rng.standard_normal(shape).astype(np.float32) for _ in range(2))
    else:
        kp, vp = (O.f32_to_bf16_bits(rng.standard_normal(shape)) for _ in range(2))
    tables = np.array([[3, 7, 1], [0, 12, 5], [2, 4, 6], [8, 8, 8]], np.int32)  # 12: not a page
    lens = np.array([37, 40, 0, 49], np.int32)                                # 49 > 3 * 16
    got = O.kv_checksum_ref(kp, vp, tables, lens)
    np.testing.assert_array_equal(got, _checksum_brute(kp, vp, tables, lens))
    assert (got[2] == 0).all() and (got[3] == 0).all()


def test_kv_checksum_ref_sees_attended_bytes_only():
    """A flipped bit of an attended element changes its row's sum and no
    other; a flipped bit past the row's length changes nothing; swapping two
    attended positions' rows changes the sum (the position enters the mix)."""
    rng = np.random.default_rng(6)
    nb, hkv, d = 6, 2, 8
    kp = O.f32_to_bf16_bits(rng.standard_normal((nb, hkv, 16, d)))
    vp = O.f32_to_bf16_bits(rng.standard_normal((nb, hkv, 16, d)))
    tables = np.array([[0, 1], [2, 3]], np.int32)
    lens = np.array([20, 30], np.int32)
    base = O.kv_checksum_ref(kp, vp, tables, lens)
    k2 = kp.copy()
    k2[1, 1, 2, 5] ^= np.uint16(1 << 3)                 # seq 0, head 1, position 18
    s2 = O.kv_checksum_ref(k2, vp, tables, lens)
    assert s2[0, 1, 0] != base[0, 1, 0]
    s2[0, 1, 0] = base[0, 1, 0]
    np.testing.assert_array_equal(s2, base)
    v3 = vp.copy()
    v3[1, 0, 10, 0] ^= np.uint16(1)                      # seq 0 position 26 >= 20
    np.testing.assert_array_equal(O.kv_checksum_ref(kp, v3, tables, lens), base)
    k4 = kp.copy()
    k4[2, 0, [3, 4]] = k4[2, 0, [4, 3]]                  # seq 1, head 0, positions 3 and 4
    if not np.array_equal(kp[2, 0, 3], kp[2, 0, 4]):
        assert O.kv_checksum_ref(k4, vp, tables, lens)[1, 0, 0] != base[1, 0, 0]
