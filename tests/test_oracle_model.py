"""Pins the decode-step oracle (oracle/oracle.py, ``*_ref``) before it is trusted.

The element-wise rules come from candle-core / candle-nn 0.11.0 and half 2.7.1
(Cargo.lock), which the reference does not vendor; the reference holds no
stored vectors for these ops. Each function is pinned here by what the
mathematics fixes, chosen so that a dropped term, a swapped operand or a wrong
rounding step fails:

* round_to: bf16 ties-to-even cases by hand; f16 equals numpy's half cast.
* embedding_ref: table rows; out-of-range ids give zero rows.
* rmsnorm_ref (qwen2.rs:68-75): f32 and bf16 bit-exact against the C
  restatement (rlse_oracle.c, itself pinned in test_oracle.py); constant-row
  closed form c / sqrt(c^2 + eps) * w.
* add_rmsnorm_ref (qwen2.rs:748-756): the sum is the rounded sum; the norm
  is rmsnorm_ref of it.
* silu_ref: silu(0) = 0, silu(x) - silu(-x) = x, silu(x) -> x and -> -0 at
  the ends; every value within one dtype ulp of the float64 x * sigmoid(x).
* linear_ref: identity weights return x exactly; bias rows; float64 bound.
* argmax_ref (candle.rs:737-751): ties, NaN at 0 / later, all -inf by hand;
  equals numpy's argmax on NaN-free rows.
* rope_ref (qwen2.rs:701-719): f32/bf16 bit-exact against the C restatement;
  position 0 is the identity.
* model_step_ref (qwen2.rs:628-764): token-by-token decoding from empty
  caches equals the last row of an independent float64 causal forward of
  the whole sequence (Model::forward, :519-541), with Qwen3 (q/k norm) and
  Qwen2 (q/k/v bias) layers; zeroed o_proj and down_proj reduce the model to
  norm(embedding) . lm_head; a planted swap of gate and up is caught.
"""
import math

import numpy as np
import pytest

import oracle as O


def _rng(s):
    return np.random.default_rng(s)


def test_round_to_bf16_and_f16_by_hand():
    # 1 + 2^-8 is halfway between 1 and 1 + 2^-7: ties to even -> 1.
    x = np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8), 65504.0, 1e-40], np.float32)
    got = O.round_to(x, "bf16")
    assert got[0] == 1.0 and got[1] == 1 + 2 ** -6 and got[2] == -1.0
    assert got[3] == 65536.0
    r = _rng(1).standard_normal(1000).astype(np.float32) * 100
    np.testing.assert_array_equal(O.round_to(r, "f16"), r.astype(np.float16).astype(np.float32))
    np.testing.assert_array_equal(O.round_to(r, "f32"), r)
    with pytest.raises(ValueError):
        O.round_to(r, "f64")


def test_embedding_rows_and_out_of_range_ids():
    table = _rng(2).standard_normal((10, 8)).astype(np.float32)
    out = O.embedding_ref([3, 0, 9, -1, 10], table)
    np.testing.assert_array_equal(out[:3], table[[3, 0, 9]])
    assert not out[3:].any()


@pytest.mark.parametrize("n", [1, 64, 1024, 896])
def test_rmsnorm_matches_c_restatement_bit_exact(n):
    rng = _rng(n)
    x = rng.standard_normal((5, n)).astype(np.float32) * 3
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    np.testing.assert_array_equal(O.rmsnorm_ref(x, w, 1e-6, "f32"), O.rmsnorm_f32(x, w, 1e-6))
    xb, wb = O.f32_to_bf16_bits(x), O.f32_to_bf16_bits(w)
    want = O.bf16_bits_to_f32(O.rmsnorm_bf16(xb, wb, 1e-6))
    got = O.rmsnorm_ref(O.bf16_bits_to_f32(xb), O.bf16_bits_to_f32(wb), 1e-6, "bf16")
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("dt", O.DTYPES)
def test_rmsnorm_constant_row_closed_form(dt):
    c, eps, n = 0.75, 1e-2, 256
    w = O.round_to(np.linspace(0.5, 1.5, n), dt)
    got = O.rmsnorm_ref(np.full((2, n), c, np.float32), w, eps, dt)
    want = c / math.sqrt(c * c + eps) * w.astype(np.float64)
    tol = {"f32": 1e-6, "bf16": 1.6e-2, "f16": 2e-3}[dt]
    np.testing.assert_allclose(got[0], want, rtol=tol)
    np.testing.assert_array_equal(got[0], got[1])


@pytest.mark.parametrize("dt", O.DTYPES)
def test_add_rmsnorm_is_rounded_sum_then_norm(dt):
    rng = _rng(5)
    x = O.round_to(rng.standard_normal((3, 128)), dt)
    r = O.round_to(rng.standard_normal((3, 128)), dt)
    w = O.round_to(1 + 0.1 * rng.standard_normal(128), dt)
    h, out = O.add_rmsnorm_ref(x, r, w, 1e-6, dt)
    np.testing.assert_array_equal(h, O.round_to(x + r, dt))
    np.testing.assert_array_equal(out, O.rmsnorm_ref(h, w, 1e-6, dt))
    # with a zero x the norm is of the residual itself
    h0, out0 = O.add_rmsnorm_ref(np.zeros_like(x), r, w, 1e-6, dt)
    np.testing.assert_array_equal(h0, r)
    np.testing.assert_array_equal(out0, O.rmsnorm_ref(r, w, 1e-6, dt))


ULP = {"f32": 2.0 ** -23, "bf16": 2.0 ** -7, "f16": 2.0 ** -10}


@pytest.mark.parametrize("dt", O.DTYPES)
def test_silu_special_values_and_float64_bound(dt):
    s = O.silu_ref(np.array([0.0, 200.0, -200.0], np.float32), dt)
    assert s[0] == 0 and s[1] == 200.0 and s[2] == 0 and np.signbit(s[2])
    # f16's exp(-x) overflows for x < -ln(65504) = -11.09 (silu -> -0 there)
    lo = -11.0 if dt == "f16" else -12.0
    x = O.round_to(np.linspace(lo, 12, 4001), dt)
    got = O.silu_ref(x, dt).astype(np.float64)
    exact = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    # three roundings (exp, 1 + e, quotient): within a few ulps of the value
    err = np.abs(got - exact) / np.maximum(np.abs(exact), 2.0 ** -14)
    assert err.max() <= 4 * ULP[dt], err.max()
    # silu(x) - silu(-x) = x (sigmoid(x) + sigmoid(-x) = 1), to rounding
    diff = O.silu_ref(x, dt).astype(np.float64) - O.silu_ref(-x, dt).astype(np.float64)
    np.testing.assert_allclose(diff, x, rtol=8 * ULP[dt], atol=8 * ULP[dt])


@pytest.mark.parametrize("dt", O.DTYPES)
def test_silu_mul_is_linear_in_up(dt):
    g = O.round_to(_rng(6).standard_normal((4, 64)), dt)
    np.testing.assert_array_equal(O.silu_mul_ref(g, np.ones_like(g), dt), O.silu_ref(g, dt))
    np.testing.assert_array_equal(O.silu_mul_ref(g, np.zeros_like(g), dt), 0 * g)
    two = O.silu_mul_ref(g, np.full_like(g, 2.0), dt)
    np.testing.assert_array_equal(two, 2 * O.silu_ref(g, dt))   # scaling by 2 is exact


@pytest.mark.parametrize("dt", O.DTYPES)
def test_linear_identity_bias_and_float64_bound(dt):
    rng = _rng(7)
    x = O.round_to(rng.standard_normal((3, 32)), dt)
    np.testing.assert_array_equal(O.linear_ref(x, np.eye(32, dtype=np.float32), None, dt), x)
    b = O.round_to(rng.standard_normal(32), dt)
    np.testing.assert_array_equal(O.linear_ref(np.zeros_like(x), np.eye(32), b, dt),
                                  np.broadcast_to(b, x.shape))
    w = O.round_to(rng.standard_normal((48, 32)), dt)
    y = O.linear_ref(x, w, None, dt)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    assert y.shape == (3, 48)
    assert (np.abs(y - exact) <= ULP[dt] * np.abs(exact) + 1e-30).all()
    # y = x W^T, not x W: a transposed operand fails here
    assert not np.allclose(y[:, :32], O.round_to(x.astype(np.float64) @ w[:32], dt))


def test_argmax_scan_rule_by_hand():
    nan, inf = np.nan, np.inf
    rows = np.array([
        [1, 3, 3, 2],          # tie: first maximum
        [nan, 5, 9, 1],        # NaN at 0: never left
        [1, nan, 2, nan],      # later NaNs never taken
        [-inf, -inf, -inf, -inf],
        [-inf, nan, -inf, -5],
        [2, 2, 2, 2],
    ], np.float32)
    assert O.argmax_ref(rows).tolist() == [1, 0, 2, 0, 3, 0]
    r = _rng(8).standard_normal((50, 777)).astype(np.float32)
    r[:, 100] = r.max(1) + 1
    r[:, 200] = r[:, 100]           # a tie behind the first maximum
    np.testing.assert_array_equal(O.argmax_ref(r), np.argmax(r, axis=1))


def test_rope_matches_c_restatement_and_position_zero():
    rng = _rng(9)
    d, rows = 64, 6
    cos_t, sin_t = O.rope_tables_f32(1e6, d, 40)
    x = rng.standard_normal((rows, d)).astype(np.float32)
    pos = np.array([0, 1, 5, 17, 39, 2], np.int32)
    np.testing.assert_array_equal(O.rope_ref(x, pos, cos_t, sin_t, "f32"),
                                  O.apply_rope_f32(x, pos, cos_t, sin_t))
    cb, sb = O.f32_to_bf16_bits(cos_t), O.f32_to_bf16_bits(sin_t)
    xb = O.f32_to_bf16_bits(x)
    want = O.bf16_bits_to_f32(O.apply_rope_bf16(xb, pos, cb, sb))
    got = O.rope_ref(O.bf16_bits_to_f32(xb), pos, O.bf16_bits_to_f32(cb),
                     O.bf16_bits_to_f32(sb), "bf16")
    np.testing.assert_array_equal(got, want)
    z = O.rope_ref(x, np.zeros(rows, np.int32), cos_t, sin_t, "f32")
    np.testing.assert_array_equal(z, x)


# ------------------------------------------------------------ whole step ----
def _f64_causal_forward(spec, w, tokens):
    """Independent float64 textbook of Model::forward over a whole sequence
    (qwen2.rs:519-541, DecoderLayer::forward :414-428): causal attention with
    repeat_kv, RoPE from theta directly, logits of the last position."""
    h, d, hq, hkv = spec.hidden, spec.head_dim, spec.heads, spec.kv_heads
    n = len(tokens)
    f = {k: v.astype(np.float64) for k, v in w.items()}
    x = f["embed"][np.asarray(tokens)]
    pos = np.arange(n)
    for l in range(spec.layers):
        p = f"l{l}."
        hn = O.rmsnorm_f64(x, f[p + "in_norm"], spec.eps)
        q = hn @ f[p + "q_w"].T + f.get(p + "q_b", 0)
        k = hn @ f[p + "k_w"].T + f.get(p + "k_b", 0)
        v = hn @ f[p + "v_w"].T + f.get(p + "v_b", 0)
        q, k, v = q.reshape(n, hq, d), k.reshape(n, hkv, d), v.reshape(n, hkv, d)
        if spec.qk_norm:
            q = O.rmsnorm_f64(q, f[p + "q_norm"], spec.eps)
            k = O.rmsnorm_f64(k, f[p + "k_norm"], spec.eps)
        q = np.stack([O.rope_f64(q[:, i], pos, spec.theta) for i in range(hq)], 0)
        k = np.stack([O.rope_f64(k[:, i], pos, spec.theta) for i in range(hkv)], 0)
        a = O.prefill_f64(q, k, v.transpose(1, 0, 2), 0, 1 / math.sqrt(d))  # [hq, n, d]
        x = x + a.transpose(1, 0, 2).reshape(n, hq * d) @ f[p + "o_w"].T
        hn = O.rmsnorm_f64(x, f[p + "post_norm"], spec.eps)
        g, u = hn @ f[p + "gate_w"].T, hn @ f[p + "up_w"].T
        x = x + (g / (1 + np.exp(-g)) * u) @ f[p + "down_w"].T
    x = O.rmsnorm_f64(x, f["norm"], spec.eps)
    return x[-1] @ f["lm_head"].T


def _decode_all(spec, w, seqs, dt):
    """Decodes every sequence token by token from empty caches, batched."""
    b_sz, n = len(seqs), len(seqs[0])
    kc = [[np.zeros((spec.kv_heads, 0, spec.head_dim), np.float32) for _ in range(b_sz)]
          for _ in range(spec.layers)]
    vc = [[np.zeros((spec.kv_heads, 0, spec.head_dim), np.float32) for _ in range(b_sz)]
          for _ in range(spec.layers)]
    cos_t, sin_t = O.rope_tables_f32(spec.theta, spec.head_dim, n + 1)
    cos_t, sin_t = O.round_to(cos_t, dt), O.round_to(sin_t, dt)
    logits = None
    for t in range(n):
        logits = O.model_step_ref(spec, w, [s[t] for s in seqs], kc, vc, cos_t, sin_t, dt)
    return logits, kc


SPECS = {
    "qwen3": O.ModelSpec(hidden=64, layers=2, heads=4, kv_heads=2, head_dim=16, inter=96,
                         vocab=50, qk_norm=True, qkv_bias=False, tied=True),
    "qwen2": O.ModelSpec(hidden=64, layers=2, heads=6, kv_heads=2, head_dim=16, inter=80,
                         vocab=40, theta=1e4, qk_norm=False, qkv_bias=True, tied=False),
}


@pytest.mark.parametrize("arch", sorted(SPECS))
def test_step_by_step_decode_equals_float64_causal_forward(arch):
    spec = SPECS[arch]
    rng = _rng(10)
    w = O.random_weights(spec, rng, "f32")
    seqs = [list(rng.integers(0, spec.vocab, 7)) for _ in range(3)]
    logits, kc = _decode_all(spec, w, seqs, "f32")
    assert kc[1][2].shape == (spec.kv_heads, 7, spec.head_dim)
    for b, s in enumerate(seqs):
        want = _f64_causal_forward(spec, w, s)
        np.testing.assert_allclose(logits[b], want, rtol=0, atol=2e-5 * np.abs(want).max())


def test_bf16_step_stays_within_its_bar_of_float64():
    spec = SPECS["qwen3"]
    rng = _rng(11)
    w = O.random_weights(spec, rng, "bf16")
    seqs = [list(rng.integers(0, spec.vocab, 5)) for _ in range(2)]
    logits, _ = _decode_all(spec, w, seqs, "bf16")
    for b, s in enumerate(seqs):
        want = _f64_causal_forward(spec, w, s)
        err = np.abs(logits[b] - want).max() / np.abs(want).max()
        assert 0 < err < 5e-2, err     # rounded per op, so not exact


def test_zero_projections_reduce_to_norm_of_embedding():
    spec = SPECS["qwen3"]
    w = O.random_weights(spec, _rng(12), "f32")
    for l in range(spec.layers):
        w[f"l{l}.o_w"] = np.zeros_like(w[f"l{l}.o_w"])
        w[f"l{l}.down_w"] = np.zeros_like(w[f"l{l}.down_w"])
    ids = [3, 17, 42]
    logits, _ = _decode_all(spec, w, [[i] for i in ids], "f32")
    x = O.rmsnorm_ref(w["embed"][ids], w["norm"], spec.eps, "f32")
    np.testing.assert_allclose(logits, x.astype(np.float64) @ w["lm_head"].T.astype(np.float64),
                               rtol=1e-6, atol=1e-6)


def test_a_planted_gate_up_swap_is_caught():
    spec = SPECS["qwen3"]
    rng = _rng(13)
    w = O.random_weights(spec, rng, "f32")
    seq = [list(rng.integers(0, spec.vocab, 4))]
    want = _f64_causal_forward(spec, w, seq[0])
    bad = dict(w)
    for l in range(spec.layers):
        bad[f"l{l}.gate_w"], bad[f"l{l}.up_w"] = w[f"l{l}.up_w"], w[f"l{l}.gate_w"]
    logits, _ = _decode_all(spec, bad, seq, "f32")
    assert np.abs(logits[0] - want).max() > 1e-2 * np.abs(want).max()
