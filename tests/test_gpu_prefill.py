"""Chunked-prefill attention (MFMA tiles) on the GPU against the oracle.

Reference: the prefill branch of Attention::forward (src/backends/qwen2.rs:
329-345) with prepare_causal_attention_mask (:476-503): the chunk's queries
at positions offset .. offset+Tq-1 see keys 0 .. offset+t, query head hq
reading KV head hq // G. The oracle is orc_prefill_f32 (the C restatement of
that Candle CPU path, pinned against float64 in tests/test_oracle.py), run on
the same bf16/f16-rounded inputs laid out contiguously as KvCache holds them.
Bars: max-abs 2e-2 for bf16 and f16 (the probabilities enter the P.V product
rounded to the pool dtype), 2e-3 for f32 (the reference CPU path's dtype: f32
products on f32 MFMAs); the relative error is printed beside it.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import TOL, as_f32, err_report, random_values, to_dev, to_host

pytestmark = pytest.mark.gpu


def make_case(rng, hq, hkv, d, tq, offset, dtype, spare_blocks=9):
    """Random pool + one sequence of ctx_len = offset + tq keys on shuffled pages."""
    L = offset + tq
    npages = (L + 15) // 16
    nb = npages + spare_blocks
    table = rng.permutation(nb)[:npages].astype(np.int32)
    kp = random_values(rng, (nb, hkv, 16, d), dtype)
    vp = random_values(rng, (nb, hkv, 16, d), dtype)
    q = random_values(rng, (tq, hq, d), dtype)
    return q, kp, vp, table, L


def run_prefill(kv, q, kp, vp, table, L, hq, hkv, d, dtype, scale, max_blocks=None):
    tq = q.shape[0]
    qd, kd, vd = to_dev(q, dtype), to_dev(kp, dtype), to_dev(vp, dtype)
    out = torch.empty_like(qd)
    td = to_dev(table)
    mb = max_blocks if max_blocks is not None else table.shape[0]
    kv.prefill_attn(qd, kd, vd, td, L, tq, out, hq, hkv, d, mb, kp.shape[0], scale, dtype)
    return to_host(out)


def oracle_prefill(q, kp, vp, table, L, hq, hkv, d, dtype, scale, heads=None):
    """orc_prefill_f32 on the contiguous [Hkv, L, d] buffers; q token-major
    [Tq, Hq, d] is transposed to the oracle's [Hq, Tq, d]. heads = a KV-head
    subset to evaluate (returns [Tq, len(heads)*G, d])."""
    tq = q.shape[0]
    g = hq // hkv
    kc = as_f32(O.paged_to_contiguous(kp, table, L), dtype)
    vc = as_f32(O.paged_to_contiguous(vp, table, L), dtype)
    qf = as_f32(q, dtype)
    heads = list(range(hkv)) if heads is None else heads
    outs = []
    for h in heads:
        qh = np.ascontiguousarray(qf[:, h * g:(h + 1) * g, :].transpose(1, 0, 2))
        o = O.prefill_f32(qh, kc[h:h + 1], vc[h:h + 1], L - tq, scale)
        outs.append(o.transpose(1, 0, 2))
    return np.concatenate(outs, axis=1)


def check(name, got, want, dtype):
    mx, rel = err_report(got, want)
    print(f"[{name}] dtype={dtype} max_abs={mx:.3e} rel={rel:.3e}")
    assert np.isfinite(got).all()
    assert mx <= TOL[dtype], (name, mx)


SHAPES = [(32, 8, 128), (14, 2, 64), (8, 8, 128), (16, 2, 128)]
CHUNKS = [(1, 0), (1, 37), (7, 0), (64, 100), (130, 5), (300, 1000)]


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"Hq{s[0]}-Hkv{s[1]}-d{s[2]}")
def test_prefill_matches_oracle(kv, dtype, shape):
    hq, hkv, d = shape
    rng = np.random.default_rng(hq * 1000 + d)
    scale = 1.0 / math.sqrt(d)
    for tq, offset in CHUNKS:
        q, kp, vp, table, L = make_case(rng, hq, hkv, d, tq, offset, dtype)
        print(f"case Hq={hq} Hkv={hkv} d={d} Tq={tq} offset={offset} {dtype}", flush=True)
        got = as_f32(run_prefill(kv, q, kp, vp, table, L, hq, hkv, d, dtype, scale), dtype)
        want = oracle_prefill(q, kp, vp, table, L, hq, hkv, d, dtype, scale)
        check(f"prefill Tq={tq} off={offset}", got, want, dtype)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_prefill_split_keys_path(kv, dtype):
    """Few row tiles over a long context: the keys are split across
    workgroups and merged; the result must not depend on the split."""
    hq, hkv, d = 8, 8, 128
    rng = np.random.default_rng(11)
    for tq, offset in [(16, 3000), (64, 5000), (3, 9000)]:
        q, kp, vp, table, L = make_case(rng, hq, hkv, d, tq, offset, dtype)
        ws = kv.prefill_workspace_size(tq, L, hq, hkv, d)
        print(f"split case Tq={tq} offset={offset} workspace={ws}", flush=True)
        assert ws > 0  # this shape must take the split path
        got = as_f32(run_prefill(kv, q, kp, vp, table, L, hq, hkv, d, dtype, 1 / math.sqrt(d)),
                     dtype)
        want = oracle_prefill(q, kp, vp, table, L, hq, hkv, d, dtype, 1 / math.sqrt(d))
        check(f"split Tq={tq} off={offset}", got, want, dtype)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_prefill_skips_invalid_pages(kv, dtype):
    """Keys on pages whose id is outside the pool are skipped, as the decode
    kernel does; checked against a float64 evaluation with those keys masked."""
    hq, hkv, d = 4, 2, 64
    rng = np.random.default_rng(5)
    tq, offset = 20, 80
    q, kp, vp, table, L = make_case(rng, hq, hkv, d, tq, offset, dtype)
    nb = kp.shape[0]
    bad = table.copy()
    bad[1] = nb + 3      # out of range
    bad[3] = -1          # negative
    scale = 1 / math.sqrt(d)
    print("invalid-page case", flush=True)
    got = as_f32(run_prefill(kv, q, kp, vp, bad, L, hq, hkv, d, dtype, scale), dtype)
    kc = as_f32(O.paged_to_contiguous(kp, table, L), dtype).astype(np.float64)
    vc = as_f32(O.paged_to_contiguous(vp, table, L), dtype).astype(np.float64)
    qf = as_f32(q, dtype).astype(np.float64)
    g = hq // hkv
    keep = np.ones(L, bool)
    keep[16:32] = False
    keep[48:64] = False
    want = np.zeros_like(qf)
    for t in range(tq):
        for hh in range(hq):
            s = kc[hh // g] @ qf[t, hh] * scale
            vis = keep & (np.arange(L) <= offset + t)
            s = np.where(vis, s, -np.inf)
            p = np.exp(s - s.max())
            want[t, hh] = (p / p.sum()) @ vc[hh // g]
    check("invalid pages skipped", got, want, dtype)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_prefill_qwen3_8b_chunk(kv, dtype):
    """The Qwen3-8B chunk: 512 queries after 8192 cached tokens, 32 q / 8 kv
    heads, d=128, bf16 and f32; KV heads 0 and 7 checked against the oracle."""
    hq, hkv, d = 32, 8, 128
    rng = np.random.default_rng(8)
    q, kp, vp, table, L = make_case(rng, hq, hkv, d, 512, 8192, dtype)
    print(f"qwen3-8b chunk Tq=512 offset=8192 {dtype}", flush=True)
    got = as_f32(run_prefill(kv, q, kp, vp, table, L, hq, hkv, d, dtype, 1 / math.sqrt(d)),
                 dtype)
    assert np.isfinite(got).all()
    g = hq // hkv
    want = oracle_prefill(q, kp, vp, table, L, hq, hkv, d, dtype, 1 / math.sqrt(d), heads=[0, 7])
    sub = np.concatenate([got[:, 0:g], got[:, 7 * g:8 * g]], axis=1)
    check("qwen3-8b chunk heads 0,7", sub, want, dtype)
    # Every KV head (each one's row tiles on their own XCD and key splits) on
    # the tokens at the edges of the 64-token row tiles and at the chunk ends.
    tq = q.shape[0]
    kc = as_f32(O.paged_to_contiguous(kp, table, L), dtype)
    vc = as_f32(O.paged_to_contiguous(vp, table, L), dtype)
    qf = as_f32(q, dtype)
    toks = [0, 1, 63, 64, 127, 128, 191, 255, 256, 319, 383, 384, 447, 448, 510, 511]
    worst = 0.0
    for h in range(hkv):
        for t in toks:
            qh = np.ascontiguousarray(qf[t:t + 1, h * g:(h + 1) * g, :].transpose(1, 0, 2))
            o = O.prefill_f32(qh, kc[h:h + 1], vc[h:h + 1], L - tq + t, 1 / math.sqrt(d))
            mx, _ = err_report(got[t, h * g:(h + 1) * g], o[:, 0, :])
            worst = max(worst, mx)
            assert mx <= TOL[dtype], (h, t, mx)
    print(f"qwen3-8b chunk: all {hkv} KV heads x {len(toks)} tokens within {worst:.3e}")


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_prefill_single_token_equals_decode(kv, dtype):
    """A one-token chunk is the decode of that token over its prefix."""
    hq, hkv, d = 16, 8, 128
    rng = np.random.default_rng(3)
    q, kp, vp, table, L = make_case(rng, hq, hkv, d, 1, 200, dtype)
    scale = 1 / math.sqrt(d)
    print("single-token chunk vs decode", flush=True)
    got = run_prefill(kv, q, kp, vp, table, L, hq, hkv, d, dtype, scale)
    out = torch.empty_like(to_dev(q, dtype))
    qd, kd, vd = to_dev(q, dtype), to_dev(kp, dtype), to_dev(vp, dtype)
    td, ld = to_dev(table.reshape(1, -1)), to_dev(np.array([L], np.int32))
    kv.paged_gqa_decode(qd, kd, vd, td, ld, out, 1, hq, hkv, d, table.shape[0], kp.shape[0],
                        scale, dtype)
    dec = to_host(out)
    mx, rel = err_report(as_f32(got, dtype), as_f32(dec, dtype))
    print(f"[prefill(1) vs decode] max_abs={mx:.3e} rel={rel:.3e}")
    assert mx <= TOL[dtype]
