"""Writes the golden fixtures of this directory (inputs + float64 expectations).

The reference ships no numeric vectors for its KV-cache path, and its Rust
code cannot be built here, so the expectations are the float64 textbook forms
of the reference's math (numpy), evaluated on the case matrix of the
reference's kernel validation harness (scripts/validate_cuda_kernels.py:
162-251): Qwen3-0.6B decode shape (16 query heads, 8 KV heads, head_dim 128),
a 32-block pool with the fragmented table [29, 3, 18, 0, 25, 11, 7, 14],
lengths 1, 15, 16, 17, 31, 32, 33, 64, 128, and the ragged shared-page batch
[1, 15, 16, 17, 31, 32, 33] over pages 7 and 12. The paged read follows
reference_paged_gqa (validate_cuda_kernels.py:29-46). K/V/q values are
N(0, 1) rounded to bf16 and stored as bf16 bit patterns (uint16), so the
same fixture serves f32 and bf16 tests.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def bf16_round(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def bf16_bits(x):
    """Bit patterns of values that are already bf16-representable."""
    return (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def softmax(s):
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    return e / e.sum(axis=-1, keepdims=True)


def paged_decode_f64(q, k_pool, v_pool, tables, lens, scale):
    b, hq, d = q.shape
    hkv = k_pool.shape[1]
    g = hq // hkv
    out = np.zeros((b, hq, d))
    for i in range(b):
        n = int(lens[i])
        pages = tables[i, : (n + 15) // 16]
        k = k_pool[pages].transpose(1, 0, 2, 3).reshape(hkv, -1, d)[:, :n].astype(np.float64)
        v = v_pool[pages].transpose(1, 0, 2, 3).reshape(hkv, -1, d)[:, :n].astype(np.float64)
        for h in range(hq):
            s = k[h // g] @ q[i, h].astype(np.float64) * scale
            out[i, h] = softmax(s) @ v[h // g]
    return out


def decode_case():
    rng = np.random.default_rng(42)
    hq, hkv, d, nblk = 16, 8, 128, 32
    k_pool = bf16_round(rng.standard_normal((nblk, hkv, 16, d)))
    v_pool = bf16_round(rng.standard_normal((nblk, hkv, 16, d)))
    frag = [29, 3, 18, 0, 25, 11, 7, 14]
    single = [1, 15, 16, 17, 31, 32, 33, 64, 128]
    ragged = [1, 15, 16, 17, 31, 32, 33]
    ragged_tables = [[7, 0, 0, 0], [7, 0, 0, 0], [7, 0, 0, 0], [7, 19, 0, 0], [7, 12, 0, 0],
                     [7, 12, 0, 0], [7, 12, 28, 0]]
    tables = [frag for _ in single] + [t + [0] * 4 for t in ragged_tables]
    lens = single + ragged
    b = len(lens)
    q = bf16_round(rng.standard_normal((b, hq, d)))
    tables = np.array(tables, np.int32)
    lens = np.array(lens, np.int32)
    scale = 1.0 / np.sqrt(d)
    out = paged_decode_f64(q, k_pool, v_pool, tables, lens, scale)
    np.savez_compressed(os.path.join(HERE, "decode_f32.npz"), q=bf16_bits(q),
                        k_pool=bf16_bits(k_pool), v_pool=bf16_bits(v_pool), tables=tables,
                        lens=lens, scale=np.float32(scale), out_f64=out)


def decode_gqa7_case():
    """Qwen2.5-0.5B head shape (14 query heads, 2 KV heads, head_dim 64)."""
    rng = np.random.default_rng(7)
    hq, hkv, d, nblk = 14, 2, 64, 48
    k_pool = bf16_round(rng.standard_normal((nblk, hkv, 16, d)))
    v_pool = bf16_round(rng.standard_normal((nblk, hkv, 16, d)))
    lens = np.array([1, 100, 257, 16], np.int32)
    perm = rng.permutation(nblk).astype(np.int32)
    tables = np.zeros((4, 17), np.int32)
    used = 0
    for i, n in enumerate(lens):
        nb = (n + 15) // 16
        tables[i, :nb] = perm[used:used + nb]
        used += nb
    q = bf16_round(rng.standard_normal((4, hq, d)))
    scale = 1.0 / np.sqrt(d)
    out = paged_decode_f64(q, k_pool, v_pool, tables, lens, scale)
    np.savez_compressed(os.path.join(HERE, "decode_gqa7_f32.npz"), q=bf16_bits(q),
                        k_pool=bf16_bits(k_pool), v_pool=bf16_bits(v_pool), tables=tables,
                        lens=lens, scale=np.float32(scale), out_f64=out)


def prefill_case():
    rng = np.random.default_rng(43)
    hq, hkv, d, offset, ql = 8, 2, 64, 40, 24
    q = bf16_round(rng.standard_normal((hq, ql, d)))
    k = bf16_round(rng.standard_normal((hkv, offset + ql, d)))
    v = bf16_round(rng.standard_normal((hkv, offset + ql, d)))
    scale = 0.125
    g = hq // hkv
    s = np.einsum("hid,hjd->hij", q.astype(np.float64), np.repeat(k, g, 0).astype(np.float64))
    s = s * scale
    i = np.arange(ql)[:, None]
    j = np.arange(offset + ql)[None, :]
    s = np.where(j - offset > i, -np.inf, s)
    out = np.einsum("hij,hjd->hid", softmax(s), np.repeat(v, g, 0).astype(np.float64))
    np.savez_compressed(os.path.join(HERE, "prefill_f32.npz"), q=q, k=k, v=v,
                        offset=np.int32(offset), scale=np.float32(scale), out_f64=out)


def norm_rope_case():
    rng = np.random.default_rng(44)
    rows, d, eps, theta = 17, 128, 1e-6, 1e6
    x = rng.standard_normal((rows, d)).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    xd = x.astype(np.float64)
    rms = xd / np.sqrt((xd * xd).mean(axis=-1, keepdims=True) + eps) * w
    pos = rng.integers(0, 4096, rows).astype(np.int32)
    half = d // 2
    inv = theta ** (-(2.0 * np.arange(half)) / d)
    ang = pos[:, None].astype(np.float64) * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    rope = np.concatenate([xd[:, :half] * c - xd[:, half:] * s,
                           xd[:, half:] * c + xd[:, :half] * s], axis=-1)
    np.savez_compressed(os.path.join(HERE, "norm_rope_f32.npz"), x=x, w=w, eps=np.float32(eps),
                        theta=np.float64(theta), pos=pos, rms_f64=rms, rope_f64=rope)


if __name__ == "__main__":
    decode_case()
    decode_gqa7_case()
    prefill_case()
    norm_rope_case()
    print("fixtures written to", HERE, file=sys.stderr)
