"""RMSNorm, RoPE and the fused q/k-norm + RoPE + append on the GPU.

Reference: RmsNorm::forward (src/backends/qwen2.rs:68-75), RotaryEmbedding and
apply_rope (:84-142), Attention::forward's norm -> transpose -> RoPE -> append
order (:291-313). RoPE uses the same host-built tables as the oracle, and the
kernels round at the same points as Candle; the sum of squares of RMSNorm
follows the oracle's fixed order (orc_sumsq_tree), so RMSNorm, RoPE and the
fused q/k-norm + RoPE + append are all checked bit for bit. The case matrix
rows {1, 4, 17, 64} x n {128, 1024} is the reference harness's
(scripts/validate_cuda_kernels.py:132-160).
"""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import DEV, as_f32, build_tables, random_values, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows", [1, 4, 17, 64])
@pytest.mark.parametrize("n", [128, 1024, 100, 896, 8192])
def test_rmsnorm_matrix(kv, dtype, rows, n):
    rng = np.random.default_rng(rows * 7 + n)
    x = random_values(rng, (rows, n), dtype)
    w = random_values(rng, (n,), dtype)
    out = torch.empty((rows, n), dtype=to_dev(x, dtype).dtype, device=DEV)
    kv.rmsnorm(to_dev(x, dtype), to_dev(w, dtype), out, rows, n, 1e-6, dtype)
    got = to_host(out)
    if dtype == "bf16":
        want = O.rmsnorm_bf16(x, w, 1e-6)
    elif dtype == "f16":
        want = O.rmsnorm_f16(x, w, 1e-6)
    else:
        want = O.rmsnorm_f32(x, w, 1e-6)
    np.testing.assert_array_equal(got, want)
    # the reference harness's bar (validate_cuda_kernels.py:126-129)
    atol, rtol = (1e-5, 1e-4) if dtype == "f32" else (5e-3, 5e-3)
    ref = O.rmsnorm_f64(as_f32(x, dtype), as_f32(w, dtype), 1e-6)
    assert np.all(np.abs(as_f32(got, dtype) - ref) <= atol + rtol * np.abs(ref) +
                  (0 if dtype == "f32" else 2.0 ** -7 * np.abs(ref)))


def test_prototype_rmsnorm_launchers(kv):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 1024)).astype(np.float32)
    w = rng.standard_normal(1024).astype(np.float32)
    a = torch.empty((4, 1024), dtype=torch.float32, device=DEV)
    xd, wd = to_dev(x), to_dev(w)  # keep the buffers alive until the kernel ran
    assert kv.load().launch_rmsnorm_f32(xd.data_ptr(), wd.data_ptr(), a.data_ptr(), 4, 1024,
                                        1e-6) == 0
    np.testing.assert_array_equal(to_host(a), O.rmsnorm_f32(x, w, 1e-6))
    xb, wb = O.f32_to_bf16_bits(x), O.f32_to_bf16_bits(w)
    b = torch.empty((4, 1024), dtype=torch.bfloat16, device=DEV)
    xbd, wbd = to_dev(xb, "bf16"), to_dev(wb, "bf16")
    assert kv.load().launch_rmsnorm_bf16(xbd.data_ptr(), wbd.data_ptr(), b.data_ptr(), 4, 1024,
                                         1e-6) == 0
    np.testing.assert_array_equal(to_host(b), O.rmsnorm_bf16(xb, wb, 1e-6))


def _tables(kv, theta, d, max_pos, dtype):
    np_dt = {"f32": np.float32, "bf16": np.uint16, "f16": np.float16}[dtype]
    cb, sb = kv.rope_tables(theta, d, max_pos, dtype)
    c = np.frombuffer(cb, np_dt).reshape(max_pos, d // 2).copy()
    s = np.frombuffer(sb, np_dt).reshape(max_pos, d // 2).copy()
    return c, s


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("d", [64, 128])
def test_rope_bit_exact(kv, dtype, d):
    rng = np.random.default_rng(d)
    ntok, hq, hkv, theta, max_pos = 6, 16, 8, 1e6, 4096
    c, s = _tables(kv, theta, d, max_pos, dtype)
    q = random_values(rng, (ntok, hq, d), dtype)
    k = random_values(rng, (ntok, hkv, d), dtype)
    pos = np.array([0, 1, 17, 512, 2047, 4095], np.int32)
    qd, kd = to_dev(q, dtype), to_dev(k, dtype)
    kv.rope(qd, kd, to_dev(c, dtype), to_dev(s, dtype), to_dev(pos), ntok, hq, hkv, d, max_pos,
            dtype)
    for x, dev, h in ((q, qd, hq), (k, kd, hkv)):
        rows = x.reshape(ntok * h, d)
        rpos = np.repeat(pos, h)
        if dtype == "bf16":
            want = O.apply_rope_bf16(rows, rpos, c, s)
        else:
            want = O.apply_rope_f32(rows, rpos, c, s)
        np.testing.assert_array_equal(to_host(dev).reshape(ntok * h, d), want)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_qk_norm_rope_append_matches_reference_order(kv, dtype):
    rng = np.random.default_rng(21)
    b, hq, hkv, d, eps, theta = 5, 16, 8, 128, 1e-6, 1e6
    pos = np.array([0, 15, 16, 200, 511], np.int32)
    nb, mbps = 64, 32
    tables = build_tables(rng, pos + 1, nb, mbps)
    q = random_values(rng, (b, hq, d), dtype)
    k = random_values(rng, (b, hkv, d), dtype)
    v = random_values(rng, (b, hkv, d), dtype)
    qw = O.f32_to_bf16_bits(1 + 0.1 * rng.standard_normal(d)) if dtype == "bf16" else \
        (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kw = O.f32_to_bf16_bits(1 + 0.1 * rng.standard_normal(d)) if dtype == "bf16" else \
        (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    c, s = _tables(kv, theta, d, 600, dtype)
    tdt = {"bf16": torch.bfloat16, "f32": torch.float32}[dtype]
    kp = torch.zeros((nb, hkv, 16, d), dtype=tdt, device=DEV)
    vp = torch.zeros_like(kp)
    q_out = torch.empty((b, hq, d), dtype=tdt, device=DEV)
    kv.qk_norm_rope_append(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), to_dev(qw, dtype),
                           to_dev(kw, dtype), eps, to_dev(c, dtype), to_dev(s, dtype), 600,
                           to_dev(pos), to_dev(tables), b, None, b, hq, hkv, d, mbps, nb, q_out,
                           kp, vp, dtype)
    norm = O.rmsnorm_bf16 if dtype == "bf16" else O.rmsnorm_f32
    rope = O.apply_rope_bf16 if dtype == "bf16" else O.apply_rope_f32
    q_ref = rope(norm(q.reshape(-1, d), qw, eps), np.repeat(pos, hq), c, s).reshape(b, hq, d)
    k_ref = rope(norm(k.reshape(-1, d), kw, eps), np.repeat(pos, hkv), c, s).reshape(b, hkv, d)
    np.testing.assert_array_equal(to_host(q_out), q_ref)
    pool_k, pool_v = to_host(kp), to_host(vp)
    for i in range(b):
        blk, slot = tables[i, pos[i] // 16], pos[i] % 16
        np.testing.assert_array_equal(pool_k[blk, :, slot], k_ref[i])
        np.testing.assert_array_equal(pool_v[blk, :, slot], v[i])  # V is appended raw


def test_qwen2_path_without_qk_norm(kv):
    """Qwen2 has no q_norm/k_norm (qwen2.rs:251-260): null weights skip the norm,
    and the result equals plain RoPE + append."""
    rng = np.random.default_rng(22)
    b, hq, hkv, d, dtype = 3, 14, 2, 64, "bf16"
    pos = np.array([3, 40, 100], np.int32)
    nb, mbps = 16, 8
    tables = build_tables(rng, pos + 1, nb, mbps)
    q, k, v = (random_values(rng, (b, h, d), dtype) for h in (hq, hkv, hkv))
    c, s = _tables(kv, 1e6, d, 128, dtype)
    kp = torch.zeros((nb, hkv, 16, d), dtype=torch.bfloat16, device=DEV)
    vp = torch.zeros_like(kp)
    q_out = torch.empty((b, hq, d), dtype=torch.bfloat16, device=DEV)
    kv.qk_norm_rope_append(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), None, None, 1e-6,
                           to_dev(c, dtype), to_dev(s, dtype), 128, to_dev(pos), to_dev(tables), b,
                           None, b, hq, hkv, d, mbps, nb, q_out, kp, vp, dtype)
    np.testing.assert_array_equal(
        to_host(q_out), O.apply_rope_bf16(q.reshape(-1, d), np.repeat(pos, hq), c, s)
        .reshape(b, hq, d))
    k_ref = O.apply_rope_bf16(k.reshape(-1, d), np.repeat(pos, hkv), c, s).reshape(b, hkv, d)
    pool_k = to_host(kp)
    for i in range(b):
        np.testing.assert_array_equal(pool_k[tables[i, pos[i] // 16], :, pos[i] % 16], k_ref[i])
