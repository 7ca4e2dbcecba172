"""Oracle for the KV-cache hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use this
module, and only as the reference results are compared with (or the timed
CPU baseline). The product path (librlse_kv.so and its binding) never
imports it.

Two layers:

1. ``C`` -- ctypes binding of liboracle.so (oracle/rlse_oracle.c), a C
   restatement of the reference's Candle CPU path in f32: KvCache
   append/narrow, the prototype's paged layout, zero-copy GQA decode, masked
   prefill, RmsNorm with Candle's cast order, RoPE tables and apply_rope.
2. numpy float64 textbook forms (``*_f64``) of the same math, used to pin the
   C restatement: softmax(q K^T * scale) V with GQA head mapping h // G,
   the causal mask with an offset, RMSNorm and NeoX RoPE in exact arithmetic.

Plus ``KVCacheModel``, a pure-Python restatement of the reference block
allocator (src/cache/kv_cache.rs:15-145) used to cross-check the C++ block
manager on random operation sequences.

Parity status of each function (how it is pinned) is listed in the module
docstring of tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import math
import os
from typing import Dict, List, Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} missing: run `make -C oracle`")
    lib = ctypes.CDLL(LIB_PATH)
    vp, i, f, d, ll = (ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_double,
                       ctypes.c_longlong)
    sigs = {
        "orc_bf16_to_f32_array": (None, [vp, vp, ll]),
        "orc_f32_to_bf16_array": (None, [vp, vp, ll]),
        "orc_kvcache_append": (i, [vp, i, i, i, i, i, vp, i]),
        "orc_kvcache_narrow": (None, [vp, i, i, i, i, i, vp]),
        "orc_paged_write_token": (None, [vp, i, i, i, vp, i, vp]),
        "orc_paged_to_contiguous": (None, [vp, i, i, i, vp, i, vp]),
        "orc_decode_gqa_f32": (None, [vp, vp, vp, i, i, i, i, i, f, vp]),
        "orc_decode_batch_f32": (None, [vp, vp, vp, vp, i, i, i, i, i, f, vp, i]),
        "orc_prefill_f32": (None, [vp, vp, vp, i, i, i, i, i, i, f, vp, i]),
        "orc_rmsnorm_f32": (None, [vp, vp, vp, i, i, f]),
        "orc_rmsnorm_bf16": (None, [vp, vp, vp, i, i, f]),
        "orc_sumsq_tree_rows": (None, [vp, i, i, i, vp]),
        "orc_rope_tables_f32": (None, [d, i, i, vp, vp]),
        "orc_apply_rope_f32": (None, [vp, vp, vp, vp, i, i]),
        "orc_apply_rope_bf16": (None, [vp, vp, vp, vp, i, i]),
        "orc_decode_step_f32": (None, [vp, vp, vp, vp, vp, vp, i, i, i, i, i, f, vp, i]),
        "orc_max_threads": (i, []),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


# ---------------------------------------------------------------------------
# bf16 helpers (numpy), identical rounding to the C restatement
# ---------------------------------------------------------------------------
def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    load().orc_f32_to_bf16_array(_p(x), _p(out), x.size)
    return out


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ---------------------------------------------------------------------------
# C restatement wrappers
# ---------------------------------------------------------------------------
class KvCacheC:
    """candle_nn KvCache over dim 2 of [1, Hkv, cap, d], bytes of any dtype."""

    def __init__(self, hkv: int, cap: int, d: int, np_dtype):
        self.hkv, self.cap, self.d = hkv, cap, d
        self.dtype = np.dtype(np_dtype)
        self.k = np.zeros((hkv, cap, d), dtype=self.dtype)
        self.v = np.zeros((hkv, cap, d), dtype=self.dtype)
        self.cur_len = 0

    def append(self, k_new: np.ndarray, v_new: np.ndarray) -> None:
        """k_new, v_new [Hkv, q, d] (Attention::append_kv, qwen2.rs:349-361)."""
        k_new = np.ascontiguousarray(k_new, dtype=self.dtype)
        v_new = np.ascontiguousarray(v_new, dtype=self.dtype)
        q = k_new.shape[1]
        es = self.dtype.itemsize
        lib = load()
        n1 = lib.orc_kvcache_append(_p(self.k), self.hkv, self.cap, self.d, es, self.cur_len,
                                    _p(k_new), q)
        n2 = lib.orc_kvcache_append(_p(self.v), self.hkv, self.cap, self.d, es, self.cur_len,
                                    _p(v_new), q)
        if n1 < 0 or n2 < 0:
            raise ValueError("kv-cache: above max-seq-len")
        self.cur_len = n1

    def snapshot(self):
        """get_kv_snapshot: narrow(2, 0, cur_len), contiguous copies."""
        es = self.dtype.itemsize
        k = np.empty((self.hkv, self.cur_len, self.d), dtype=self.dtype)
        v = np.empty_like(k)
        lib = load()
        lib.orc_kvcache_narrow(_p(self.k), self.hkv, self.cap, self.d, es, self.cur_len, _p(k))
        lib.orc_kvcache_narrow(_p(self.v), self.hkv, self.cap, self.d, es, self.cur_len, _p(v))
        return k, v


def paged_write_token(pool: np.ndarray, table: np.ndarray, pos: int, row: np.ndarray) -> None:
    """pool [nb, Hkv, 16, d]; row [Hkv, d]; prototype index formula."""
    nb, hkv, bs, d = pool.shape
    table = np.ascontiguousarray(table, dtype=np.int32)
    row = np.ascontiguousarray(row, dtype=pool.dtype)
    load().orc_paged_write_token(_p(pool), hkv, d, pool.dtype.itemsize, _p(table), pos, _p(row))


def paged_to_contiguous(pool: np.ndarray, table: np.ndarray, length: int) -> np.ndarray:
    nb, hkv, bs, d = pool.shape
    table = np.ascontiguousarray(table, dtype=np.int32)
    out = np.empty((hkv, length, d), dtype=pool.dtype)
    load().orc_paged_to_contiguous(_p(pool), hkv, d, pool.dtype.itemsize, _p(table), length,
                                   _p(out))
    return out


# Checksums of the pool's rows (rlse_kv_checksum): the definition itself,
# in numpy uint32 arithmetic (every product and sum wraps mod 2^32).
_MIX_T, _MIX_J, _MIX_M = np.uint32(0x9E3779B1), np.uint32(0x85EBCA77), np.uint32(0xC2B2AE3D)


def mix_words(w: np.ndarray, t: np.ndarray, j: np.ndarray) -> np.ndarray:
    """(w ^ (t * 0x9E3779B1 + j * 0x85EBCA77)) * 0xC2B2AE3D mod 2^32, with
    t and j broadcast against w."""
    with np.errstate(over="ignore"):
        key = (np.asarray(t, np.uint32) * _MIX_T + np.asarray(j, np.uint32) * _MIX_J)
        return (np.asarray(w, np.uint32) ^ key) * _MIX_M


def kv_checksum_ref(k_pool: np.ndarray, v_pool: np.ndarray, tables: np.ndarray,
                    lens: np.ndarray) -> np.ndarray:
    """Per (sequence, KV head) row: the sums mod 2^32, over the attended
    positions t < L (L = 0 for L <= 0 or beyond the table's capacity) and the
    32-bit words j of a position's head_dim elements, of mix_words(w, t, j)
    -- K then V, [B][Hkv][2] uint32. Pages whose id lies outside the pool
    contribute nothing. Pools are [num_blocks][Hkv][16][head_dim] arrays of
    the dtype's bits (uint16 for bf16, float16, float32)."""
    nb, hkv = k_pool.shape[:2]
    kw = np.ascontiguousarray(k_pool).view(np.uint32).reshape(nb, hkv, 16, -1)
    vw = np.ascontiguousarray(v_pool).view(np.uint32).reshape(nb, hkv, 16, -1)
    nw = kw.shape[-1]
    tables = np.asarray(tables, np.int32)
    b_sz, mbps = tables.shape
    out = np.zeros((b_sz, hkv, 2), np.uint32)
    j = np.arange(nw, dtype=np.uint32)[None, None, :]
    for b in range(b_sz):
        n = int(lens[b])
        if n <= 0 or n > 16 * mbps:
            continue
        npg = (n + 15) // 16
        ids = tables[b, :npg]
        ok = (ids >= 0) & (ids < nb)
        t = np.arange(npg * 16, dtype=np.uint32)
        keep = (t < n) & np.repeat(ok, 16)
        for c, words in ((0, kw), (1, vw)):
            rows = words[np.where(ok, ids, 0)]                      # [npg, Hkv, 16, nw]
            rows = rows.transpose(1, 0, 2, 3).reshape(hkv, npg * 16, nw)
            m = mix_words(rows, t[None, :, None], j)
            m = np.where(keep[None, :, None], m, np.uint32(0))
            out[b, :, c] = (m.sum(axis=(1, 2), dtype=np.uint64) & 0xFFFFFFFF).astype(np.uint32)
    return out


def decode_batch_f32(q: np.ndarray, k: np.ndarray, v: np.ndarray, lens: np.ndarray,
                     scale: float, threads: int = 0) -> np.ndarray:
    """q [B, Hq, d]; k, v [B, Hkv, cap, d] f32; returns [B, Hq, d] f32."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    lens = np.ascontiguousarray(lens, dtype=np.int32)
    b, hq, d = q.shape
    hkv, cap = k.shape[1], k.shape[2]
    out = np.empty_like(q)
    load().orc_decode_batch_f32(_p(q), _p(k), _p(v), _p(lens), b, hq, hkv, cap, d, scale,
                                _p(out), threads)
    return out


def decode_paged_f32(q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray, tables: np.ndarray,
                     lens: np.ndarray, scale: float, threads: int = 0) -> np.ndarray:
    """Decode over a paged pool by first laying each sequence out contiguously
    (the reference's buffer layout) and then running the C restatement."""
    b = q.shape[0]
    hkv, d = k_pool.shape[1], k_pool.shape[3]
    cap = max(int(max(lens)), 1)
    kc = np.zeros((b, hkv, cap, d), dtype=np.float32)
    vc = np.zeros_like(kc)
    for i in range(b):
        n = int(lens[i])
        if n > 0:
            kc[i, :, :n] = paged_to_contiguous(k_pool, tables[i], n).astype(np.float32)
            vc[i, :, :n] = paged_to_contiguous(v_pool, tables[i], n).astype(np.float32)
    return decode_batch_f32(q.astype(np.float32), kc, vc, lens, scale, threads)


def prefill_f32(q: np.ndarray, k: np.ndarray, v: np.ndarray, offset: int, scale: float,
                threads: int = 0) -> np.ndarray:
    """q [Hq, q_len, d]; k, v [Hkv, cap, d]; keys 0..offset+q_len-1 visible."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    hq, ql, d = q.shape
    hkv, cap = k.shape[0], k.shape[1]
    out = np.empty_like(q)
    load().orc_prefill_f32(_p(q), _p(k), _p(v), hq, hkv, cap, ql, offset, d, scale, _p(out),
                           threads)
    return out


def rmsnorm_f32(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, n = x.reshape(-1, x.shape[-1]).shape
    out = np.empty_like(x)
    load().orc_rmsnorm_f32(_p(x), _p(w), _p(out), rows, n, eps)
    return out


def rmsnorm_bf16(x_bits: np.ndarray, w_bits: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    rows, n = x.reshape(-1, x.shape[-1]).shape
    out = np.empty_like(x)
    load().orc_rmsnorm_bf16(_p(x), _p(w), _p(out), rows, n, eps)
    return out


def sumsq_tree(x: np.ndarray, epl: int) -> np.ndarray:
    """orc_sumsq_tree per row of x [..., n] (f32): the sum of squares in the
    order every K-writing RMSNorm follows (packets of epl elements summed in
    order, then a balanced pairwise tree over the packets)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    rows = x.size // n
    out = np.empty(rows, np.float32)
    load().orc_sumsq_tree_rows(_p(x), rows, n, epl, _p(out))
    return out.reshape(x.shape[:-1])


def rmsnorm_f16(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """RmsNorm::forward on f16 storage (qwen2.rs:68-75): f32 arithmetic with
    the sum of squares in the 8-element packet order of orc_sumsq_tree,
    x / norm rounded to f16, then the weight product rounded to f16."""
    xf = np.asarray(x, np.float16).astype(np.float32)
    n = xf.shape[-1]
    ss = sumsq_tree(xf, 8)
    norm = np.sqrt(ss * np.float32(1.0 / n) + np.float32(eps)).astype(np.float32)
    xn = (xf / norm[..., None]).astype(np.float16).astype(np.float32)
    return (xn * np.asarray(w, np.float16).astype(np.float32)).astype(np.float16)


def rope_tables_f32(theta: float, d: int, max_pos: int):
    c = np.empty((max_pos, d // 2), dtype=np.float32)
    s = np.empty_like(c)
    load().orc_rope_tables_f32(theta, d, max_pos, _p(c), _p(s))
    return c, s


def apply_rope_f32(x: np.ndarray, pos: np.ndarray, cos_t: np.ndarray, sin_t: np.ndarray):
    """x [rows, d] (copied), pos [rows]."""
    x = np.array(x, dtype=np.float32, order="C")
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    load().orc_apply_rope_f32(_p(x), _p(pos), _p(np.ascontiguousarray(cos_t, np.float32)),
                              _p(np.ascontiguousarray(sin_t, np.float32)), x.shape[0],
                              x.shape[1])
    return x


def apply_rope_bf16(x_bits: np.ndarray, pos: np.ndarray, cos_bits: np.ndarray,
                    sin_bits: np.ndarray):
    x = np.array(x_bits, dtype=np.uint16, order="C")
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    load().orc_apply_rope_bf16(_p(x), _p(pos), _p(np.ascontiguousarray(cos_bits, np.uint16)),
                               _p(np.ascontiguousarray(sin_bits, np.uint16)), x.shape[0],
                               x.shape[1])
    return x


def decode_step_f32(q, k_new, v_new, k, v, lens, scale, threads=0):
    """Append + decode of one layer on contiguous buffers (timed CPU baseline)."""
    b, hq, d = q.shape
    hkv, cap = k.shape[1], k.shape[2]
    out = np.empty_like(q)
    load().orc_decode_step_f32(_p(q), _p(k_new), _p(v_new), _p(k), _p(v), _p(lens), b, hq, hkv,
                               cap, d, scale, _p(out), threads)
    return out


def max_threads() -> int:
    return load().orc_max_threads()


# ---------------------------------------------------------------------------
# numpy float64 textbook forms
# ---------------------------------------------------------------------------
def softmax_f64(s: np.ndarray, axis: int = -1) -> np.ndarray:
    s = s - np.max(s, axis=axis, keepdims=True)
    e = np.exp(s)
    return e / np.sum(e, axis=axis, keepdims=True)


def decode_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """One sequence: q [Hq, d]; k, v [Hkv, L, d]; query head h uses KV head h // G."""
    hq = q.shape[0]
    hkv = k.shape[0]
    g = hq // hkv
    q = q.astype(np.float64)
    kk = np.repeat(k.astype(np.float64), g, axis=0)  # repeat_kv
    vv = np.repeat(v.astype(np.float64), g, axis=0)
    s = np.einsum("hd,hld->hl", q, kk) * scale
    return np.einsum("hl,hld->hd", softmax_f64(s), vv)


def prefill_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, offset: int, scale: float):
    """q [Hq, q_len, d]; k, v [Hkv, offset+q_len, d]; causal with offset."""
    hq, ql, d = q.shape
    hkv, lk = k.shape[0], k.shape[1]
    g = hq // hkv
    kk = np.repeat(k.astype(np.float64), g, axis=0)
    vv = np.repeat(v.astype(np.float64), g, axis=0)
    s = np.einsum("hid,hjd->hij", q.astype(np.float64), kk) * scale
    i = np.arange(ql)[:, None]
    j = np.arange(lk)[None, :]
    s = np.where(j - offset > i, -np.inf, s)
    return np.einsum("hij,hjd->hid", softmax_f64(s), vv)


def rmsnorm_f64(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = x.astype(np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w.astype(np.float64)


def rope_f64(x: np.ndarray, pos: np.ndarray, theta: float) -> np.ndarray:
    """NeoX rotation in float64: pairs (i, i + d/2) rotated by pos * theta^(-2i/d)."""
    x = x.astype(np.float64)
    d = x.shape[-1]
    half = d // 2
    inv = theta ** (-(2.0 * np.arange(half)) / d)
    ang = np.asarray(pos, dtype=np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    x1, x2 = x[:, :half], x[:, half:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)


# ---------------------------------------------------------------------------
# KVCache (src/cache/kv_cache.rs:15-145), pure Python
# ---------------------------------------------------------------------------
class KVCacheModel:
    def __init__(self, total_blocks: int, block_size: int = 16):
        self.total = total_blocks
        self.block_size = block_size
        self.free = list(range(total_blocks - 1, -1, -1))  # pop() yields 0, 1, 2, ...
        self.allocations: Dict[str, List[int]] = {}

    def blocks_needed(self, tokens: int) -> int:
        return 1 if tokens == 0 else -(-tokens // self.block_size)

    def allocate(self, rid: str, num_tokens: int) -> List[int]:
        needed = self.blocks_needed(num_tokens)
        if needed > len(self.free):
            raise MemoryError(f"Requested {needed} blocks ({num_tokens} tokens), but only "
                              f"{len(self.free)} free blocks remain")
        blocks = [self.free.pop() for _ in range(needed)]
        self.allocations[rid] = list(blocks)
        return blocks

    def allocate_block(self, rid: str) -> int:
        if not self.free:
            raise MemoryError("KV cache pressure: no free blocks remaining for incremental "
                              "allocation")
        b = self.free.pop()
        self.allocations.setdefault(rid, []).append(b)
        return b

    def release(self, rid: str) -> int:
        blocks = self.allocations.pop(rid, None)
        if blocks is None:
            return 0
        self.free.extend(blocks)
        return len(blocks)

    def stats(self):
        free = len(self.free)
        allocated = self.total - free
        util = np.float32(allocated) / np.float32(self.total) if self.total > 0 else np.float32(0)
        fs = set(self.free)
        runs = sum(1 for i in range(self.total) if i in fs and (i == 0 or (i - 1) not in fs))
        frag = (np.float32(runs) - np.float32(1)) / np.float32(free) if (free > 0 and runs > 1) \
            else np.float32(0)

        def r3(x):
            x = np.float32(x) * np.float32(1000.0)
            return np.float32(math.floor(abs(float(x)) + 0.5) * (1 if x >= 0 else -1)) \
                / np.float32(1000.0)
        return (self.total, allocated, free, float(r3(util)), float(r3(min(frag, 1.0))))


# ---------------------------------------------------------------------------
# PrefixCache (src/cache/prefix_cache.rs:58-394), pure Python
# ---------------------------------------------------------------------------
class PrefixCacheModel:
    """Chunk keys, LRU order and the lookup / insert / insert_kv / lookup_kv
    rules of the reference's PrefixCache, with a chunk's KV reduced to a flag
    and an optional logits handle (the memory budget is not modelled: page
    references need no new memory)."""

    def __init__(self, chunk_size: int, max_chunks: int):
        self.cs = chunk_size
        self.max = max_chunks
        self.chunks = {}  # key -> {"kv": bool, "logits": handle or None}
        self.lru = []     # keys, least recently used first
        self.hits = self.misses = self.tokens_saved = self.kv_evictions = 0

    @staticmethod
    def chunk_hashes(tokens, chunk_size):
        """compute_chunk_hashes (:98-124): key_i = sha256(key_{i-1} hex ||
        tokens of chunk i as little-endian u32), hex encoded."""
        import hashlib
        out, prev = [], ""
        for i in range(len(tokens) // chunk_size):
            h = hashlib.sha256()
            if prev:
                h.update(prev.encode())
            for t in tokens[i * chunk_size:(i + 1) * chunk_size]:
                h.update(int(t).to_bytes(4, "little"))
            prev = h.hexdigest()
            out.append(prev)
        return out

    def _touch(self, k):
        self.lru.remove(k)
        self.lru.append(k)

    def _evict_oldest(self):
        k = self.lru.pop(0)
        if self.chunks.pop(k)["kv"]:
            self.kv_evictions += 1

    def _add(self, k, kv, logits):
        while len(self.chunks) >= self.max:
            self._evict_oldest()
        self.chunks[k] = {"kv": kv, "logits": logits}
        self.lru.append(k)

    def lookup(self, tokens):
        m = 0
        for k in self.chunk_hashes(tokens, self.cs):
            if k not in self.chunks:
                break
            m += 1
            self._touch(k)
        return m * self.cs

    def insert(self, tokens):
        if self.max == 0:
            return
        for k in self.chunk_hashes(tokens, self.cs):
            if k not in self.chunks:
                self._add(k, False, None)

    def insert_kv(self, tokens, logits=None):
        if self.max == 0:
            return
        for i, k in enumerate(self.chunk_hashes(tokens, self.cs)):
            offer = logits is not None and (i + 1) * self.cs == len(tokens)
            c = self.chunks.get(k)
            if c is not None and c["kv"] and (not offer or c["logits"] is not None):
                continue
            if c is not None:
                del self.chunks[k]
                self.lru.remove(k)
            self._add(k, True, logits if offer else None)

    def lookup_kv(self, tokens):
        best, best_key = 0, None
        for i, k in enumerate(self.chunk_hashes(tokens, self.cs)):
            if k in self.chunks:
                if self.chunks[k]["kv"]:
                    best, best_key = (i + 1) * self.cs, k
                self._touch(k)
        logits = self.chunks[best_key]["logits"] if best_key and best == len(tokens) else None
        return best, logits

    def record_reuse(self, skipped):
        if skipped == 0:
            self.misses += 1
        else:
            self.hits += 1
            self.tokens_saved += skipped


# ---------------------------------------------------------------------------
# The rest of a batched decode step: ModelForCausalLM::step_decode_batch
# (src/backends/qwen2.rs:628-764), numpy.
#
# Values of every dtype are held as float32 arrays; ``round_to`` rounds a
# float32 result to the tensor dtype (round to nearest even), which is what
# Candle's element-wise ops do on bf16/f16 tensors: each op computes in f32
# (half 2.7.1's bf16/f16 arithmetic converts both operands to f32) and stores
# its result in the tensor dtype. The reference runs f32 on the CPU
# (src/backends/candle.rs:185), where ``round_to`` is the identity.
# The element-wise rules live in candle-core 0.11.0 / candle-nn 0.11.0
# (Cargo.lock), which are not vendored: they are restated from their
# published sources and pinned by closed forms in tests/test_oracle_model.py.
# ---------------------------------------------------------------------------
DTYPES = ("f32", "bf16", "f16")


def round_to(x, dt: str) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    if dt == "f32":
        return x
    if dt == "bf16":
        return round_bf16(x)
    if dt == "f16":
        return x.astype(np.float16).astype(np.float32)
    raise ValueError(dt)


def embedding_ref(ids, table: np.ndarray) -> np.ndarray:
    """candle_nn::Embedding::forward (qwen2.rs:651-652): rows of the table
    by token id. The reference rejects an id outside [0, vocab) with an
    index error; the device op writes a zero row for it, which is what this
    returns."""
    ids = np.asarray(ids, dtype=np.int64)
    out = np.zeros((len(ids), table.shape[1]), dtype=np.float32)
    ok = (ids >= 0) & (ids < table.shape[0])
    out[ok] = table[ids[ok]]
    return out


def rmsnorm_ref(x: np.ndarray, w: np.ndarray, eps: float, dt: str) -> np.ndarray:
    """RmsNorm::forward (qwen2.rs:68-75): in f32, variance = sum(x^2) * (1/n),
    norm = sqrt(variance + eps), x / norm cast to the dtype, then the weight
    product in the dtype."""
    x = np.asarray(x, dtype=np.float32)
    n = x.shape[-1]
    ss = sumsq_tree(x, 4 if dt == "f32" else 8)   # the C oracle's order (orc_sumsq_tree)
    norm = np.sqrt(ss * np.float32(1.0 / n) + np.float32(eps)).astype(np.float32)
    xn = round_to(x / norm[..., None], dt)
    return round_to(xn * np.asarray(w, np.float32), dt)


def add_rmsnorm_ref(x: np.ndarray, residual: np.ndarray, w: np.ndarray, eps: float, dt: str):
    """`xs_mid = residual + attn_proj` then post_attention_layernorm
    (qwen2.rs:748-753), and `xs = xs_mid + mlp_out` then the next layer's
    input_layernorm (:756, :665-667): returns (sum, normed sum)."""
    h = round_to(np.asarray(residual, np.float32) + np.asarray(x, np.float32), dt)
    return h, rmsnorm_ref(h, w, eps, dt)


def silu_ref(g: np.ndarray, dt: str) -> np.ndarray:
    """Activation::Silu, candle-core's unary op: v / (1 + exp(-v)), each of
    exp, the sum and the quotient rounded to the dtype."""
    g = np.asarray(g, np.float32)
    with np.errstate(over="ignore"):
        e = round_to(np.exp(-g), dt)
    den = round_to(np.float32(1.0) + e, dt)
    return round_to(g / den, dt)


def silu_mul_ref(gate: np.ndarray, up: np.ndarray, dt: str) -> np.ndarray:
    """MLP::forward (qwen2.rs:170-175) between the projections:
    act(gate_proj(x)) * up_proj(x), the product rounded."""
    return round_to(silu_ref(gate, dt) * np.asarray(up, np.float32), dt)


def linear_ref(x: np.ndarray, w: np.ndarray, b, dt: str) -> np.ndarray:
    """candle_nn::Linear::forward: x . W^T, the exact product (float64, one
    rounding to the dtype), then + bias rounded again (broadcast_add)."""
    y = round_to(np.asarray(x, np.float64) @ np.asarray(w, np.float64).T, dt)
    if b is not None:
        y = round_to(y + np.asarray(b, np.float32), dt)
    return y


def argmax_ref(logits: np.ndarray) -> np.ndarray:
    """Greedy branch of sample_token (src/backends/candle.rs:737-751):
    Tensor::argmax(0) of the f32 logits, candle-core's CPU index reduction --
    start at index 0 and move to i only when value[i] > the current best, so
    ties keep the first index, a NaN is never taken, and a NaN at index 0 is
    never left. Per row of a [rows, vocab] array."""
    logits = np.atleast_2d(np.asarray(logits, np.float32))
    out = np.zeros(logits.shape[0], dtype=np.int32)
    for r, row in enumerate(logits):
        best, idx = row[0], 0
        for i in range(1, len(row)):
            if row[i] > best:
                best, idx = row[i], i
        out[r] = idx
    return out


def rope_ref(x: np.ndarray, pos, cos_t: np.ndarray, sin_t: np.ndarray, dt: str) -> np.ndarray:
    """Batched RoPE of step_decode_batch (qwen2.rs:701-719): x * cos +
    rotate_half(x) * sin with the tables' rows at each position, both
    products and the sum rounded to the dtype. x [rows, d]; cos_t, sin_t
    [max_pos, d/2] already in the dtype."""
    x = np.asarray(x, np.float32)
    half = x.shape[-1] // 2
    c = np.asarray(cos_t, np.float32)[np.asarray(pos)]
    s = np.asarray(sin_t, np.float32)[np.asarray(pos)]
    c2, s2 = np.concatenate([c, c], -1), np.concatenate([s, s], -1)
    rot = np.concatenate([-x[..., half:], x[..., :half]], -1)
    return round_to(round_to(x * c2, dt) + round_to(rot * s2, dt), dt)


class ModelSpec:
    """Shape of a Qwen2/Qwen3 decoder (the fields of qwen2.rs Config that the
    decode step reads)."""

    def __init__(self, hidden, layers, heads, kv_heads, head_dim, inter, vocab, eps=1e-6,
                 theta=1e6, qk_norm=True, qkv_bias=False, tied=True):
        self.hidden, self.layers, self.heads, self.kv_heads = hidden, layers, heads, kv_heads
        self.head_dim, self.inter, self.vocab, self.eps = head_dim, inter, vocab, eps
        self.theta, self.qk_norm, self.qkv_bias, self.tied = theta, qk_norm, qkv_bias, tied


def random_weights(spec: ModelSpec, rng, dt: str) -> Dict[str, np.ndarray]:
    """Seeded random weights of the architecture, scaled 1/sqrt(fan_in) so
    activations stay O(1), norms 1 + 0.1 N(0,1); values rounded to dt."""
    h, d = spec.hidden, spec.head_dim
    nq, nkv = spec.heads * d, spec.kv_heads * d

    def mat(o, i):
        return round_to(rng.standard_normal((o, i)).astype(np.float32) / np.sqrt(i), dt)

    def vec(n, base, sd):
        return round_to(base + sd * rng.standard_normal(n).astype(np.float32), dt)

    w = {"embed": round_to(rng.standard_normal((spec.vocab, h)).astype(np.float32), dt),
         "norm": vec(h, 1.0, 0.1)}
    w["lm_head"] = w["embed"] if spec.tied else mat(spec.vocab, h)
    for l in range(spec.layers):
        p = f"l{l}."
        w[p + "in_norm"] = vec(h, 1.0, 0.1)
        w[p + "post_norm"] = vec(h, 1.0, 0.1)
        w[p + "q_w"], w[p + "k_w"], w[p + "v_w"] = mat(nq, h), mat(nkv, h), mat(nkv, h)
        if spec.qkv_bias:
            w[p + "q_b"], w[p + "k_b"], w[p + "v_b"] = vec(nq, 0, .1), vec(nkv, 0, .1), \
                vec(nkv, 0, .1)
        if spec.qk_norm:
            w[p + "q_norm"], w[p + "k_norm"] = vec(d, 1.0, 0.1), vec(d, 1.0, 0.1)
        w[p + "o_w"] = mat(h, nq)
        w[p + "gate_w"], w[p + "up_w"] = mat(spec.inter, h), mat(spec.inter, h)
        w[p + "down_w"] = mat(h, spec.inter)
    return w


def model_step_ref(spec: ModelSpec, w: Dict[str, np.ndarray], ids, k_cache, v_cache,
                   cos_t: np.ndarray, sin_t: np.ndarray, dt: str) -> np.ndarray:
    """One batched decode step (step_decode_batch, qwen2.rs:628-764): token
    ids[b] of sequence b at position len(k_cache[l][b]) along axis 1. Appends
    each layer's new K/V rows to k_cache[l][b] / v_cache[l][b] ([Hkv, len, d]
    float32 arrays of dt values, replaced in the lists) and returns the
    logits [B, vocab]. Attention over dt-valued q/K/V is the C restatement in
    f32 with its output rounded once to the dtype."""
    b_sz = len(ids)
    d, hq, hkv = spec.head_dim, spec.heads, spec.kv_heads
    scale = 1.0 / math.sqrt(d)
    pos = np.array([k_cache[0][b].shape[1] for b in range(b_sz)], dtype=np.int64)
    xs = embedding_ref(ids, w["embed"])
    for l in range(spec.layers):
        p = f"l{l}."
        residual = xs
        hn = rmsnorm_ref(xs, w[p + "in_norm"], spec.eps, dt)
        q = linear_ref(hn, w[p + "q_w"], w.get(p + "q_b"), dt).reshape(b_sz, hq, d)
        k = linear_ref(hn, w[p + "k_w"], w.get(p + "k_b"), dt).reshape(b_sz, hkv, d)
        v = linear_ref(hn, w[p + "v_w"], w.get(p + "v_b"), dt).reshape(b_sz, hkv, d)
        if spec.qk_norm:
            q = rmsnorm_ref(q, w[p + "q_norm"], spec.eps, dt)
            k = rmsnorm_ref(k, w[p + "k_norm"], spec.eps, dt)
        attn = np.empty((b_sz, hq, d), dtype=np.float32)
        for b in range(b_sz):
            qb = rope_ref(q[b], np.full(hq, pos[b]), cos_t, sin_t, dt)
            kb = rope_ref(k[b], np.full(hkv, pos[b]), cos_t, sin_t, dt)
            k_cache[l][b] = np.concatenate([k_cache[l][b], kb[:, None]], axis=1)
            v_cache[l][b] = np.concatenate([v_cache[l][b], v[b][:, None]], axis=1)
            n = k_cache[l][b].shape[1]
            attn[b] = decode_batch_f32(qb[None], k_cache[l][b][None], v_cache[l][b][None],
                                       np.array([n], np.int32), scale)[0]
        attn = round_to(attn, dt).reshape(b_sz, hq * d)
        o = linear_ref(attn, w[p + "o_w"], None, dt)
        xs_mid, hn = add_rmsnorm_ref(o, residual, w[p + "post_norm"], spec.eps, dt)
        gate = linear_ref(hn, w[p + "gate_w"], None, dt)
        up = linear_ref(hn, w[p + "up_w"], None, dt)
        mlp = linear_ref(silu_mul_ref(gate, up, dt), w[p + "down_w"], None, dt)
        xs = round_to(xs_mid + mlp, dt)
    xs = rmsnorm_ref(xs, w["norm"], spec.eps, dt)
    return linear_ref(xs, w["lm_head"], None, dt)
