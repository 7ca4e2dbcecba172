"""ctypes binding of librlse_kv.so, the C ABI declared in include/rlse_kv.h.

This is the Python face of the MI355X paged KV-cache hot path. It mirrors the
reference's operator and cache APIs by name and behaviour:

* ``BlockManager`` -- KVCache (src/cache/kv_cache.rs:15-145): ``allocate``,
  ``allocate_block``, ``release``, ``blocks_needed``, ``stats`` with the same
  ids, counts and CachePressure messages, plus ``fork`` for refcounted prefix
  sharing with copy-on-write of a partial block.
* ``KVPool`` -- the physical pool that replaces the per-request contiguous
  candle_nn KvCache buffers (src/backends/qwen2.rs:349-361).
* ``kv_append`` / ``kv_gather`` / ``kv_scatter`` / ``kv_copy_blocks`` --
  Attention::append_kv and get/set_kv_snapshot (qwen2.rs:349-377, 547-574).
* ``paged_gqa_decode`` -- decode_attention_gqa_zero_copy (qwen2.rs:177-203).
* ``rmsnorm`` / ``rope`` / ``qk_norm_rope_append`` -- RmsNorm::forward,
  apply_rotary_emb_qkv and the front half of Attention::forward
  (qwen2.rs:56-142, 291-313).

Device arguments are raw device addresses (ints) or objects with a
``data_ptr()`` method (torch tensors). Every call raises ``RlseError`` when the
library returns a non-zero status; nothing here computes on the CPU. Loading
fails loudly when the shared library has not been built.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

_HERE = os.path.dirname(os.path.abspath(__file__))
# RLSE_KV_LIB names another build of the library (a sanitized one, or one
# built from other sources for a before/after measurement).
LIB_PATH = os.environ.get("RLSE_KV_LIB") or os.path.join(_HERE, "librlse_kv.so")

DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
DTYPE_NAMES = {"f32": DTYPE_F32, "float32": DTYPE_F32, "bf16": DTYPE_BF16,
               "bfloat16": DTYPE_BF16, "f16": DTYPE_F16, "float16": DTYPE_F16}
DTYPE_SIZE = {DTYPE_F32: 4, DTYPE_BF16: 2, DTYPE_F16: 2}

OK = 0
ERR_INVALID_VALUE = 1
ERR_CACHE_PRESSURE = 10001
ERR_UNKNOWN_REQUEST = 10002
ERR_BUFFER_TOO_SMALL = 10003
ERR_TOKEN_LIMIT = 10004
ERR_DEVICE_TIMEOUT = 10005
DECODE_STREAM = 1
WS_ERR_MERGE_TIMEOUT = 1
WS_ERR_LENGTH = 2
WS_ERR_PREFIX = 4
BLOCK_SIZE = 16

# Every extern "C" symbol of include/rlse_kv.h (checked by the CPU tests).
EXPORTED = (
    "rlse_last_error", "rlse_version",
    "rlse_pool_create", "rlse_pool_destroy", "rlse_pool_layer", "rlse_pool_info",
    "rlse_kv_append", "rlse_kv_gather", "rlse_kv_scatter", "rlse_kv_copy_blocks",
    "rlse_decode_workspace_size", "rlse_paged_gqa_decode", "rlse_decode_step",
    "rlse_prefill_workspace_size", "rlse_prefill_attn",
    "rlse_rmsnorm", "rlse_rope_tables", "rlse_rope", "rlse_qk_norm_rope_append",
    "launch_rmsnorm_f32", "launch_rmsnorm_f16", "launch_rmsnorm_bf16",
    "launch_paged_gqa_decode_tiled_f32", "launch_paged_gqa_decode_tiled_f16",
    "launch_paged_gqa_decode_tiled_bf16",
    "rlse_bm_create", "rlse_bm_destroy", "rlse_bm_blocks_needed", "rlse_bm_free_count",
    "rlse_bm_allocate", "rlse_bm_allocate_block", "rlse_bm_release", "rlse_bm_fork",
    "rlse_bm_block_table", "rlse_bm_refcount", "rlse_bm_stats",
    "rlse_pc_create", "rlse_pc_destroy", "rlse_pc_chunk_hashes", "rlse_pc_lookup",
    "rlse_pc_insert", "rlse_pc_insert_kv", "rlse_pc_lookup_kv", "rlse_pc_fork",
    "rlse_pc_reclaim", "rlse_pc_clear", "rlse_pc_record_reuse", "rlse_pc_stats",
    "rlse_pc_reserve_memory",
    "rlse_mb_create", "rlse_mb_destroy", "rlse_mb_stats", "rlse_mb_try_reserve",
    "rlse_mb_release", "rlse_mb_record_rejection", "rlse_bm_attach_budget",
    "rlse_memory_charge",
    "rlse_bm_release_all", "rlse_st_create", "rlse_st_destroy", "rlse_st_reset",
    "rlse_st_prepare", "rlse_st_host", "rlse_st_upload", "rlse_st_mark_uploaded",
    "rlse_embedding", "rlse_add_rmsnorm", "rlse_silu_mul", "rlse_argmax", "rlse_linear",
    "rlse_argmax_workspace_size", "rlse_qkv_proj", "rlse_linear_residual", "rlse_gate_up_silu",
    "rlse_dense_workspace_size", "rlse_dense_pack", "rlse_decode_plan_size", "rlse_decode_plan",
    "rlse_decode_step_planned", "rlse_workspace_check", "rlse_set_merge_wait_ns",
    "rlse_decode_step_noalloc", "rlse_decode_prefix_size", "rlse_decode_plan_cascade",
    "rlse_decode_step_cascade", "rlse_decode_plan_groups", "rlse_decode_step_groups",
    "rlse_kv_checksum", "rlse_kv_checksum_planned",
)


class RlseError(RuntimeError):
    """A non-zero status from librlse_kv; ``status`` holds the code."""

    def __init__(self, status: int, message: str):
        super().__init__(f"rlse status {status}: {message}")
        self.status = status
        self.message = message


class CachePressure(RlseError):
    """RLSE_ERR_CACHE_PRESSURE, the reference's EngineError::CachePressure."""


class TokenLimitExceeded(RlseError):
    """RLSE_ERR_TOKEN_LIMIT, the reference's EngineError::TokenLimitExceeded."""


class DeviceTimeout(RlseError):
    """RLSE_ERR_DEVICE_TIMEOUT: a merge on the device gave up waiting; the
    caller treats it as the reference's BackendError (quarantine,
    src/backends/candle.rs:689-696)."""


class _MemoryStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_longlong) for n in (
        "budget_bytes", "headroom_bytes", "active_kv_reserved_bytes", "execution_reserved_bytes",
        "prefix_retained_bytes", "reserved_bytes", "available_bytes", "peak_reserved_bytes",
        "rejections")]


@dataclass
class MemoryStats:
    """TensorMemoryStats (src/cache/tensor_memory.rs:28-39)."""
    budget_bytes: int
    headroom_bytes: int
    active_kv_reserved_bytes: int
    execution_reserved_bytes: int
    prefix_retained_bytes: int
    reserved_bytes: int
    available_bytes: int
    peak_reserved_bytes: int
    rejections: int


class ModelShape(ctypes.Structure):
    """The Config fields memory_charge reads (src/backends/candle.rs:241-282)."""
    _fields_ = [(n, ctypes.c_int) for n in (
        "num_layers", "num_heads", "num_kv_heads", "head_dim", "hidden_size",
        "intermediate_size", "vocab_size", "dtype_bytes", "context_length", "block_size")]


class _CacheStats(ctypes.Structure):
    _fields_ = [("total_blocks", ctypes.c_int), ("allocated_blocks", ctypes.c_int),
                ("free_blocks", ctypes.c_int), ("utilization", ctypes.c_float),
                ("fragmentation", ctypes.c_float)]


class _PrefixStats(ctypes.Structure):
    _fields_ = [("hits", ctypes.c_longlong), ("misses", ctypes.c_longlong),
                ("tokens_saved", ctypes.c_longlong), ("kv_evictions", ctypes.c_longlong),
                ("chunks", ctypes.c_longlong), ("held_pages", ctypes.c_longlong),
                ("hit_rate", ctypes.c_float)]


@dataclass
class PrefixStats:
    hits: int
    misses: int
    tokens_saved: int
    kv_evictions: int
    chunks: int
    held_pages: int
    hit_rate: float


@dataclass
class CacheStats:
    total_blocks: int
    allocated_blocks: int
    free_blocks: int
    utilization: float
    fragmentation: float


_vp, _i, _f, _d, _ll, _sz = (ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_double,
                             ctypes.c_longlong, ctypes.c_size_t)
_ip = ctypes.POINTER(ctypes.c_int32)
_cp = ctypes.c_char_p

_SIGS = {
    "rlse_last_error": (ctypes.c_char_p, []),
    "rlse_version": (_i, []),
    "rlse_pool_create": (_i, [_i, _i, _i, _i, _i, _i, ctypes.POINTER(_vp)]),
    "rlse_pool_destroy": (_i, [_vp]),
    "rlse_pool_layer": (_i, [_vp, _i, ctypes.POINTER(_vp), ctypes.POINTER(_vp)]),
    "rlse_pool_info": (_i, [_vp, ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_i),
                            ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_ll)]),
    "rlse_kv_append": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "rlse_kv_gather": (_i, [_vp, _vp, _ll, _i, _vp, _i, _vp, _vp, _i, _i, _i, _i, _vp]),
    "rlse_kv_scatter": (_i, [_vp, _vp, _vp, _vp, _ll, _i, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "rlse_kv_copy_blocks": (_i, [_vp, _vp, _ll, _i, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "rlse_decode_workspace_size": (_i, [_i, _i, _i, _i, ctypes.POINTER(_sz)]),
    "rlse_paged_gqa_decode": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f,
                                   _i, _vp, _sz, _vp]),
    "rlse_decode_step": (_i, [_vp, _vp, _vp, _vp, _vp, _f, _vp, _vp, _i, _vp, _vp, _vp, _vp,
                              _vp, _i, _i, _i, _i, _i, _i, _f, _i, _vp, _sz, _vp]),
    "rlse_decode_step_planned": (_i, [_vp, _vp, _vp, _vp, _vp, _f, _vp, _vp, _i, _vp, _vp, _vp, _vp,
                              _vp, _i, _i, _i, _i, _i, _i, _f, _i, _vp, _sz, _vp, _i, _vp]),
    "rlse_decode_prefix_size": (_i, [_i, _i, _i, _i, ctypes.POINTER(_sz)]),
    "rlse_decode_plan_cascade": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "rlse_decode_step_cascade": (_i, [_vp, _vp, _vp, _vp, _vp, _f, _vp, _vp, _i, _vp, _vp, _vp,
                                      _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _i, _vp, _sz, _vp, _i,
                                      _i, _vp, _sz, _vp]),
    "rlse_decode_plan_groups": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "rlse_kv_checksum": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp]),
    "rlse_kv_checksum_planned": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp,
                                      _vp]),
    "rlse_decode_step_groups": (_i, [_vp, _vp, _vp, _vp, _vp, _f, _vp, _vp, _i, _vp, _vp, _vp,
                                     _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _i, _vp, _sz, _vp, _i,
                                     _i, _i, _vp, _sz, _vp]),
    "rlse_prefill_workspace_size": (_i, [_i, _i, _i, _i, _i, ctypes.POINTER(_sz)]),
    "rlse_prefill_attn": (_i, [_vp, _vp, _vp, _vp, _i, _i, _vp, _i, _i, _i, _i, _i, _f, _i, _vp,
                               _sz, _vp]),
    "rlse_rmsnorm": (_i, [_vp, _vp, _vp, _i, _i, _f, _i, _vp]),
    "rlse_rope_tables": (_i, [_d, _i, _i, _i, _vp, _vp]),
    "rlse_rope": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "rlse_qk_norm_rope_append": (_i, [_vp, _vp, _vp, _vp, _vp, _f, _vp, _vp, _i, _vp, _vp, _i,
                                      _vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _i, _vp]),
    "launch_rmsnorm_f32": (_i, [_vp, _vp, _vp, _i, _i, _f]),
    "launch_rmsnorm_f16": (_i, [_vp, _vp, _vp, _i, _i, _f]),
    "launch_rmsnorm_bf16": (_i, [_vp, _vp, _vp, _i, _i, _f]),
    "launch_paged_gqa_decode_tiled_f32": (_i, [_vp] * 6 + [_i] * 4 + [_f]),
    "launch_paged_gqa_decode_tiled_f16": (_i, [_vp] * 6 + [_i] * 4 + [_f]),
    "launch_paged_gqa_decode_tiled_bf16": (_i, [_vp] * 6 + [_i] * 4 + [_f]),
    "rlse_bm_create": (_i, [_i, _i, ctypes.POINTER(_vp)]),
    "rlse_bm_destroy": (_i, [_vp]),
    "rlse_bm_blocks_needed": (_i, [_vp, _ll]),
    "rlse_bm_free_count": (_i, [_vp]),
    "rlse_bm_allocate": (_i, [_vp, _cp, _ll, _ip, _i, ctypes.POINTER(_i)]),
    "rlse_bm_allocate_block": (_i, [_vp, _cp, _ip]),
    "rlse_bm_release": (_i, [_vp, _cp, ctypes.POINTER(_i)]),
    "rlse_bm_fork": (_i, [_vp, _cp, _cp, _ll, _ip, _ip, _i, ctypes.POINTER(_i)]),
    "rlse_bm_block_table": (_i, [_vp, _cp, _ip, _i, ctypes.POINTER(_i)]),
    "rlse_bm_refcount": (_i, [_vp, _i]),
    "rlse_bm_stats": (_i, [_vp, ctypes.POINTER(_CacheStats)]),
    "rlse_pc_create": (_i, [_vp, _i, _i, ctypes.POINTER(_vp)]),
    "rlse_pc_destroy": (_i, [_vp]),
    "rlse_pc_chunk_hashes": (_i, [_vp, _ll, _i, ctypes.c_char_p, _i, ctypes.POINTER(_i)]),
    "rlse_pc_lookup": (_i, [_vp, _vp, _ll, ctypes.POINTER(_ll)]),
    "rlse_pc_insert": (_i, [_vp, _vp, _ll]),
    "rlse_pc_insert_kv": (_i, [_vp, _vp, _ll, _cp, _i, _ll]),
    "rlse_pc_lookup_kv": (_i, [_vp, _vp, _ll, ctypes.POINTER(_ll), ctypes.POINTER(_i),
                               ctypes.POINTER(_ll)]),
    "rlse_pc_fork": (_i, [_vp, _vp, _ll, _ll, _cp, _ip, _ip, _i, ctypes.POINTER(_i)]),
    "rlse_pc_reclaim": (_i, [_vp, _i, ctypes.POINTER(_i)]),
    "rlse_pc_clear": (_i, [_vp]),
    "rlse_pc_record_reuse": (_i, [_vp, _ll]),
    "rlse_pc_stats": (_i, [_vp, ctypes.POINTER(_PrefixStats)]),
    "rlse_pc_reserve_memory": (_i, [_vp, _ll, _ll, _ll, ctypes.POINTER(_ll)]),
    "rlse_mb_create": (_i, [_ll, _ll, ctypes.POINTER(_vp)]),
    "rlse_mb_destroy": (_i, [_vp]),
    "rlse_mb_stats": (_i, [_vp, ctypes.POINTER(_MemoryStats)]),
    "rlse_mb_try_reserve": (_i, [_vp, _ll, _ll, _ll, ctypes.POINTER(_ll)]),
    "rlse_mb_release": (_i, [_vp, _ll]),
    "rlse_mb_record_rejection": (_i, [_vp]),
    "rlse_bm_attach_budget": (_i, [_vp, _vp, _ll]),
    "rlse_memory_charge": (_i, [ctypes.POINTER(ModelShape), _ll, _ll, ctypes.POINTER(_ll),
                                ctypes.POINTER(_ll), ctypes.POINTER(_ll)]),
    "rlse_bm_release_all": (_i, [_vp, ctypes.POINTER(_i)]),
    "rlse_st_create": (_i, [_i, _i, ctypes.POINTER(_vp)]),
    "rlse_st_destroy": (_i, [_vp]),
    "rlse_st_reset": (_i, [_vp]),
    "rlse_st_prepare": (_i, [_vp, _vp, ctypes.POINTER(_cp), ctypes.POINTER(_ll), _i, _ip]),
    "rlse_st_host": (_i, [_vp, ctypes.POINTER(_ip), ctypes.POINTER(_ip), ctypes.POINTER(_i),
                          ctypes.POINTER(_ip), ctypes.POINTER(_i)]),
    "rlse_st_upload": (_i, [_vp, _vp, _vp, _vp]),
    "rlse_st_mark_uploaded": (_i, [_vp]),
    "rlse_embedding": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "rlse_add_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f, _i, _vp]),
    "rlse_silu_mul": (_i, [_vp, _vp, _i, _i, _i, _vp]),
    "rlse_argmax_workspace_size": (_i, [_i, _i, ctypes.POINTER(_sz)]),
    "rlse_argmax": (_i, [_vp, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "rlse_linear": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "rlse_dense_workspace_size": (_i, [_i, _i, _i, ctypes.POINTER(_sz)]),
    "rlse_decode_plan_size": (_i, [ctypes.POINTER(_sz)]),
    "rlse_decode_plan": (_i, [_vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "rlse_qkv_proj": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "rlse_linear_residual": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "rlse_gate_up_silu": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "rlse_dense_pack": (_i, [_vp, _vp, _i, _i, _i, _i, _vp]),
    "rlse_workspace_check": (_i, [_vp, _vp, ctypes.POINTER(ctypes.c_uint)]),
    "rlse_decode_step_noalloc": (_i, [_vp, _vp, _vp, _vp, _vp, _f, _vp, _vp, _i, _vp, _vp, _vp,
                                      _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _i, _vp]),
    "rlse_set_merge_wait_ns": (_i, [ctypes.c_ulonglong]),
}

_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Loads librlse_kv.so (built in tree next to this file); raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; "
            "g.build()' or make -C mini-serve-rs_amd/csrc)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return load().rlse_last_error().decode("utf-8", "replace")


def _check(status: int) -> None:
    if status != OK:
        msg = last_error()
        if status == ERR_CACHE_PRESSURE:
            raise CachePressure(status, msg)
        if status == ERR_TOKEN_LIMIT:
            raise TokenLimitExceeded(status, msg)
        if status == ERR_DEVICE_TIMEOUT:
            raise DeviceTimeout(status, msg)
        raise RlseError(status, msg)


def _ptr(x) -> Optional[int]:
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return int(x.data_ptr())


def _dt(dtype) -> int:
    if isinstance(dtype, int):
        return dtype
    name = str(dtype).replace("torch.", "")
    return DTYPE_NAMES[name]


def _stream(stream) -> Optional[int]:
    if stream is None:
        return None
    if isinstance(stream, int):
        return stream
    return int(stream.cuda_stream)


# --------------------------------------------------------------------------
# Block manager (KVCache successor)
# --------------------------------------------------------------------------
class BlockManager:
    """KVCache (src/cache/kv_cache.rs) over physical pool block ids."""

    def __init__(self, total_blocks: int, block_size: int = BLOCK_SIZE):
        lib = load()
        h = _vp()
        _check(lib.rlse_bm_create(total_blocks, block_size, ctypes.byref(h)))
        self._h = h
        self._lib = lib
        self._total = total_blocks
        self._block_size = block_size

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.rlse_bm_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def block_size(self) -> int:
        return self._block_size

    def total_blocks(self) -> int:
        return self._total

    def free_count(self) -> int:
        return self._lib.rlse_bm_free_count(self._h)

    def allocated_count(self) -> int:
        return self._total - self.free_count()

    def blocks_needed(self, tokens: int) -> int:
        return self._lib.rlse_bm_blocks_needed(self._h, tokens)

    def allocate(self, request_id: str, num_tokens: int) -> List[int]:
        n = self.blocks_needed(num_tokens)
        buf = (ctypes.c_int32 * max(n, 1))()
        got = _i()
        _check(self._lib.rlse_bm_allocate(self._h, request_id.encode(), num_tokens, buf, n,
                                          ctypes.byref(got)))
        return list(buf[:got.value])

    def allocate_block(self, request_id: str) -> int:
        b = ctypes.c_int32()
        _check(self._lib.rlse_bm_allocate_block(self._h, request_id.encode(), ctypes.byref(b)))
        return b.value

    def release(self, request_id: str) -> int:
        n = _i()
        _check(self._lib.rlse_bm_release(self._h, request_id.encode(), ctypes.byref(n)))
        return n.value

    def fork(self, parent_id: str, child_id: str, num_tokens: int) -> List[Tuple[int, int]]:
        src, dst, n = (ctypes.c_int32 * 1)(), (ctypes.c_int32 * 1)(), _i()
        _check(self._lib.rlse_bm_fork(self._h, parent_id.encode(), child_id.encode(),
                                      num_tokens, src, dst, 1, ctypes.byref(n)))
        return [(src[i], dst[i]) for i in range(n.value)]

    def block_table(self, request_id: str) -> List[int]:
        n = _i()
        _check(self._lib.rlse_bm_block_table(self._h, request_id.encode(), None, 0,
                                             ctypes.byref(n)))
        buf = (ctypes.c_int32 * max(n.value, 1))()
        _check(self._lib.rlse_bm_block_table(self._h, request_id.encode(), buf, n.value,
                                             ctypes.byref(n)))
        return list(buf[:n.value])

    def refcount(self, block: int) -> int:
        return self._lib.rlse_bm_refcount(self._h, block)

    def stats(self) -> CacheStats:
        s = _CacheStats()
        _check(self._lib.rlse_bm_stats(self._h, ctypes.byref(s)))
        return CacheStats(s.total_blocks, s.allocated_blocks, s.free_blocks, s.utilization,
                          s.fragmentation)

    def release_all(self) -> int:
        """Releases every request (the KV side of quarantine); returns how many."""
        n = _i()
        _check(self._lib.rlse_bm_release_all(self._h, ctypes.byref(n)))
        return n.value

    def attach_budget(self, budget: Optional["MemoryBudget"], page_bytes: int = 0) -> None:
        """Charges this manager's pages to budget from now on (None: detach)."""
        _check(self._lib.rlse_bm_attach_budget(self._h, budget._h if budget else None,
                                               page_bytes))
        self._budget = budget  # the budget must outlive the attachment


def _tokens(tokens):
    arr = (ctypes.c_uint32 * max(len(tokens), 1))(*[int(t) & 0xffffffff for t in tokens])
    return arr, len(tokens)


class PrefixCache:
    """PrefixCache (src/cache/prefix_cache.rs) over refcounted pages of a
    BlockManager: chained SHA-256 chunk keys and LRU as the reference; a
    chunk with KV holds references on its prefix's pages (no copies)."""

    def __init__(self, bm: BlockManager, chunk_size: int = BLOCK_SIZE, max_chunks: int = 512):
        lib = load()
        h = _vp()
        _check(lib.rlse_pc_create(bm._h, chunk_size, max_chunks, ctypes.byref(h)))
        self._h, self._lib, self._bm = h, lib, bm
        self.chunk_size = chunk_size

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.rlse_pc_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def compute_chunk_hashes(tokens, chunk_size: int) -> List[str]:
        arr, n = _tokens(tokens)
        cnt = _i()
        _check(load().rlse_pc_chunk_hashes(arr, n, chunk_size, None, 0, ctypes.byref(cnt)))
        buf = ctypes.create_string_buffer(65 * max(cnt.value, 1))
        _check(load().rlse_pc_chunk_hashes(arr, n, chunk_size, buf, cnt.value, ctypes.byref(cnt)))
        return [buf.raw[65 * i:65 * i + 64].decode() for i in range(cnt.value)]

    def lookup(self, tokens) -> int:
        arr, n = _tokens(tokens)
        m = _ll()
        _check(self._lib.rlse_pc_lookup(self._h, arr, n, ctypes.byref(m)))
        return m.value

    def insert(self, tokens) -> None:
        arr, n = _tokens(tokens)
        _check(self._lib.rlse_pc_insert(self._h, arr, n))

    def insert_kv(self, tokens, request_id: str, logits_handle: Optional[int] = None) -> None:
        arr, n = _tokens(tokens)
        _check(self._lib.rlse_pc_insert_kv(self._h, arr, n, request_id.encode(),
                                           0 if logits_handle is None else 1,
                                           0 if logits_handle is None else logits_handle))

    def lookup_kv(self, tokens) -> Tuple[int, Optional[int]]:
        """(matched tokens, logits handle or None)."""
        arr, n = _tokens(tokens)
        m, has, handle = _ll(), _i(), _ll()
        _check(self._lib.rlse_pc_lookup_kv(self._h, arr, n, ctypes.byref(m), ctypes.byref(has),
                                           ctypes.byref(handle)))
        return m.value, (handle.value if has.value else None)

    def fork(self, tokens, restore_tokens: int, child_id: str) -> List[Tuple[int, int]]:
        """Restores restore_tokens cached tokens into child_id; returns the
        copy-on-write (src, dst) page pairs for rlse_kv_copy_blocks."""
        arr, n = _tokens(tokens)
        src, dst, cnt = (ctypes.c_int32 * 1)(), (ctypes.c_int32 * 1)(), _i()
        _check(self._lib.rlse_pc_fork(self._h, arr, n, restore_tokens, child_id.encode(), src,
                                      dst, 1, ctypes.byref(cnt)))
        return [(src[i], dst[i]) for i in range(cnt.value)]

    def reclaim(self, min_free_blocks: int) -> int:
        n = _i()
        _check(self._lib.rlse_pc_reclaim(self._h, min_free_blocks, ctypes.byref(n)))
        return n.value

    def clear(self) -> None:
        _check(self._lib.rlse_pc_clear(self._h))

    def record_reuse(self, skipped_tokens: int) -> None:
        _check(self._lib.rlse_pc_record_reuse(self._h, skipped_tokens))

    def stats(self) -> PrefixStats:
        st = _PrefixStats()
        _check(self._lib.rlse_pc_stats(self._h, ctypes.byref(st)))
        return PrefixStats(st.hits, st.misses, st.tokens_saved, st.kv_evictions, st.chunks,
                           st.held_pages, st.hit_rate)

    def reserve_memory(self, active_kv: int = 0, execution: int = 0, prefix: int = 0) -> int:
        """reserve_memory (prefix_cache.rs:229-244) on the block manager's
        budget: evicts LRU chunks until the charge fits; a lease id, or
        CachePressure (one rejection recorded)."""
        lease = _ll()
        _check(self._lib.rlse_pc_reserve_memory(self._h, active_kv, execution, prefix,
                                                ctypes.byref(lease)))
        return lease.value


# --------------------------------------------------------------------------
# Tensor memory budget (TensorMemoryBudget successor, page-based KV charges)
# --------------------------------------------------------------------------
class MemoryBudget:
    """TensorMemoryBudget (src/cache/tensor_memory.rs:41-125). Block
    managers attached with BlockManager.attach_budget charge their pages to
    it; leases cover the other reservations."""

    def __init__(self, budget_bytes: int, headroom_bytes: int):
        lib = load()
        h = _vp()
        _check(lib.rlse_mb_create(budget_bytes, headroom_bytes, ctypes.byref(h)))
        self._h, self._lib = h, lib

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.rlse_mb_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def stats(self) -> MemoryStats:
        st = _MemoryStats()
        _check(self._lib.rlse_mb_stats(self._h, ctypes.byref(st)))
        return MemoryStats(*(getattr(st, f) for f, _ in _MemoryStats._fields_))

    def try_reserve(self, active_kv: int = 0, execution: int = 0,
                    prefix: int = 0) -> Optional[int]:
        """try_reserve (:72-90): a lease id, or None when the charge does not fit."""
        lease = _ll()
        st = self._lib.rlse_mb_try_reserve(self._h, active_kv, execution, prefix,
                                           ctypes.byref(lease))
        if st == ERR_CACHE_PRESSURE:
            return None
        _check(st)
        return lease.value

    def release(self, lease: int) -> None:
        _check(self._lib.rlse_mb_release(self._h, lease))

    def record_rejection(self) -> None:
        _check(self._lib.rlse_mb_record_rejection(self._h))


class StepTables:
    """Per-step block tables (scheduler.rs:422-449 reservation loop + the
    upload of the tables the decode kernels read, sending only changes)."""

    def __init__(self, max_batch: int, max_blocks_per_seq: int):
        lib = load()
        h = _vp()
        _check(lib.rlse_st_create(max_batch, max_blocks_per_seq, ctypes.byref(h)))
        self._h, self._lib = h, lib
        self.max_batch, self.max_blocks_per_seq = max_batch, max_blocks_per_seq

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.rlse_st_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prepare(self, bm: BlockManager, request_ids: Sequence[str],
                next_lens: Sequence[int]) -> List[int]:
        """Grows each request to blocks_needed(next_len) and lays out the rows;
        returns the per-request status (0 OK, else the request left the batch)."""
        n = len(request_ids)
        ids = (_cp * max(n, 1))(*[r.encode() for r in request_ids])
        lens = (_ll * max(n, 1))(*next_lens)
        status = (ctypes.c_int32 * max(n, 1))()
        _check(self._lib.rlse_st_prepare(self._h, bm._h, ids, lens, n, status))
        return list(status[:n])

    def host(self):
        """(tables [max_batch][max_blocks_per_seq], seq_lens [max_batch], batch,
        pending (row, col, page) triples) as numpy copies."""
        import numpy as np
        t, l, p = _ip(), _ip(), _ip()
        b, n = _i(), _i()
        _check(self._lib.rlse_st_host(self._h, ctypes.byref(t), ctypes.byref(l), ctypes.byref(b),
                                      ctypes.byref(p), ctypes.byref(n)))
        tables = np.ctypeslib.as_array(t, (self.max_batch, self.max_blocks_per_seq)).copy()
        lens = np.ctypeslib.as_array(l, (self.max_batch,)).copy()
        pend = (np.ctypeslib.as_array(p, (n.value, 3)).copy() if n.value
                else np.zeros((0, 3), np.int32))
        return tables, lens, b.value, pend

    def upload(self, tables, seq_lens, stream=None) -> None:
        _check(self._lib.rlse_st_upload(self._h, _ptr(tables), _ptr(seq_lens), _stream(stream)))

    def mark_uploaded(self) -> None:
        _check(self._lib.rlse_st_mark_uploaded(self._h))

    def reset(self) -> None:
        _check(self._lib.rlse_st_reset(self._h))


def memory_charge(shape: ModelShape, prompt_tokens: int, max_tokens: int) -> Tuple[int, int, int]:
    """memory_charge (src/backends/candle.rs:241-282) for paged KV:
    (kv_bytes, execution_bytes, page_bytes)."""
    kv, ex, page = _ll(), _ll(), _ll()
    _check(load().rlse_memory_charge(ctypes.byref(shape), prompt_tokens, max_tokens,
                                     ctypes.byref(kv), ctypes.byref(ex), ctypes.byref(page)))
    return kv.value, ex.value, page.value


# --------------------------------------------------------------------------
# Physical pool
# --------------------------------------------------------------------------
class KVPool:
    """Device pool [layers] x {K, V} x [num_blocks][Hkv][16][head_dim]."""

    def __init__(self, num_layers: int, num_blocks: int, num_kv_heads: int, head_dim: int,
                 dtype, block_size: int = BLOCK_SIZE):
        lib = load()
        h = _vp()
        _check(lib.rlse_pool_create(num_layers, num_blocks, num_kv_heads, head_dim, _dt(dtype),
                                    block_size, ctypes.byref(h)))
        self._h = h
        self._lib = lib
        self.num_layers, self.num_blocks = num_layers, num_blocks
        self.num_kv_heads, self.head_dim, self.dtype = num_kv_heads, head_dim, _dt(dtype)
        stride = _ll()
        _check(lib.rlse_pool_info(h, None, None, None, None, None, ctypes.byref(stride)))
        self.layer_stride_elems = stride.value

    def layer(self, layer: int) -> Tuple[int, int]:
        k, v = _vp(), _vp()
        _check(self._lib.rlse_pool_layer(self._h, layer, ctypes.byref(k), ctypes.byref(v)))
        return k.value, v.value

    def close(self) -> None:
        if getattr(self, "_h", None):
            _check(self._lib.rlse_pool_destroy(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# --------------------------------------------------------------------------
# Kernels
# --------------------------------------------------------------------------
def kv_append(k_new, v_new, k_pool, v_pool, block_tables, num_seqs: int, seq_index, positions,
              num_tokens: int, num_kv_heads: int, head_dim: int, max_blocks_per_seq: int,
              num_blocks: int, dtype, stream=None) -> None:
    _check(load().rlse_kv_append(_ptr(k_new), _ptr(v_new), _ptr(k_pool), _ptr(v_pool),
                                 _ptr(block_tables), num_seqs, _ptr(seq_index), _ptr(positions),
                                 num_tokens, num_kv_heads, head_dim, max_blocks_per_seq,
                                 num_blocks, _dt(dtype), _stream(stream)))


def kv_gather(k_pool, v_pool, layer_stride_elems: int, num_layers: int, block_table, length: int,
              k_out, v_out, num_kv_heads: int, head_dim: int, num_blocks: int, dtype,
              stream=None) -> None:
    _check(load().rlse_kv_gather(_ptr(k_pool), _ptr(v_pool), layer_stride_elems, num_layers,
                                 _ptr(block_table), length, _ptr(k_out), _ptr(v_out),
                                 num_kv_heads, head_dim, num_blocks, _dt(dtype), _stream(stream)))


def kv_scatter(k_in, v_in, k_pool, v_pool, layer_stride_elems: int, num_layers: int, block_table,
               start: int, length: int, num_kv_heads: int, head_dim: int, num_blocks: int, dtype,
               stream=None) -> None:
    _check(load().rlse_kv_scatter(_ptr(k_in), _ptr(v_in), _ptr(k_pool), _ptr(v_pool),
                                  layer_stride_elems, num_layers, _ptr(block_table), start,
                                  length, num_kv_heads, head_dim, num_blocks, _dt(dtype),
                                  _stream(stream)))


def kv_copy_blocks(k_pool, v_pool, layer_stride_elems: int, num_layers: int, src_blocks,
                   dst_blocks, num_pairs: int, num_kv_heads: int, head_dim: int,
                   num_blocks: int, dtype, stream=None) -> None:
    _check(load().rlse_kv_copy_blocks(_ptr(k_pool), _ptr(v_pool), layer_stride_elems,
                                      num_layers, _ptr(src_blocks), _ptr(dst_blocks), num_pairs,
                                      num_kv_heads, head_dim, num_blocks, _dt(dtype),
                                      _stream(stream)))


def decode_workspace_size(batch: int, num_heads: int, num_kv_heads: int, head_dim: int) -> int:
    """Bytes of workspace for paged_gqa_decode. A workspace must be zero-filled
    once before its first use (every launch leaves it zero again: the group
    that merges a partial record clears it)."""
    n = _sz()
    _check(load().rlse_decode_workspace_size(batch, num_heads, num_kv_heads, head_dim,
                                             ctypes.byref(n)))
    return n.value


def paged_gqa_decode(q, k_pool, v_pool, block_tables, seq_lens, out, batch: int, num_heads: int,
                     num_kv_heads: int, head_dim: int, max_blocks_per_seq: int, num_blocks: int,
                     scale: float, dtype, workspace=None, workspace_bytes: int = 0,
                     stream=None) -> None:
    _check(load().rlse_paged_gqa_decode(_ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(block_tables),
                                        _ptr(seq_lens), _ptr(out), batch, num_heads,
                                        num_kv_heads, head_dim, max_blocks_per_seq, num_blocks,
                                        scale, _dt(dtype), _ptr(workspace), workspace_bytes,
                                        _stream(stream)))


def decode_step_noalloc(q, k_new, v_new, q_norm_weight, k_norm_weight, eps: float, cos_table,
                        sin_table, max_pos: int, k_pool, v_pool, block_tables, seq_lens, out,
                        batch: int, num_heads: int, num_kv_heads: int, head_dim: int,
                        max_blocks_per_seq: int, num_blocks: int, scale: float, dtype,
                        stream=None) -> None:
    """decode_step without a workspace: the split-K records live in the
    library's static device scratch; nothing is allocated."""
    _check(load().rlse_decode_step_noalloc(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(q_norm_weight), _ptr(k_norm_weight), eps,
        _ptr(cos_table), _ptr(sin_table), max_pos, _ptr(k_pool), _ptr(v_pool),
        _ptr(block_tables), _ptr(seq_lens), _ptr(out), batch, num_heads, num_kv_heads, head_dim,
        max_blocks_per_seq, num_blocks, scale, _dt(dtype), _stream(stream)))


def decode_step(q, k_new, v_new, q_norm_weight, k_norm_weight, eps: float, cos_table, sin_table,
                max_pos: int, k_pool, v_pool, block_tables, seq_lens, out, batch: int,
                num_heads: int, num_kv_heads: int, head_dim: int, max_blocks_per_seq: int,
                num_blocks: int, scale: float, dtype, workspace=None, workspace_bytes: int = 0,
                stream=None) -> None:
    """One layer's fused q/k-norm + RoPE + append + paged decode (new token of
    sequence b at position seq_lens[b] - 1)."""
    _check(load().rlse_decode_step(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(q_norm_weight), _ptr(k_norm_weight), eps,
        _ptr(cos_table), _ptr(sin_table), max_pos, _ptr(k_pool), _ptr(v_pool),
        _ptr(block_tables), _ptr(seq_lens), _ptr(out), batch, num_heads, num_kv_heads, head_dim,
        max_blocks_per_seq, num_blocks, scale, _dt(dtype), _ptr(workspace), workspace_bytes,
        _stream(stream)))


def decode_plan_size() -> int:
    """Bytes of a per-step decode plan (rlse_decode_plan)."""
    n = _sz(0)
    _check(load().rlse_decode_plan_size(ctypes.byref(n)))
    return n.value


def decode_plan(block_tables, seq_lens, batch: int, num_kv_heads: int, max_blocks_per_seq: int,
                num_blocks: int, plan, plan_bytes: int, stream=None) -> None:
    """Builds the per-step plan every layer's decode_step_planned then reads."""
    _check(load().rlse_decode_plan(_ptr(block_tables), _ptr(seq_lens), batch, num_kv_heads,
                                   max_blocks_per_seq, num_blocks, _ptr(plan), plan_bytes,
                                   _stream(stream)))


def decode_step_planned(q, k_new, v_new, q_norm_weight, k_norm_weight, eps: float, cos_table,
                        sin_table, max_pos: int, k_pool, v_pool, block_tables, seq_lens, out,
                        batch: int, num_heads: int, num_kv_heads: int, head_dim: int,
                        max_blocks_per_seq: int, num_blocks: int, scale: float, dtype, plan,
                        workspace=None, workspace_bytes: int = 0, stream=None,
                        stream_pages: bool = False) -> None:
    """decode_step with a plan built by decode_plan from the same tables and
    lengths; the results are the same bit for bit. stream_pages
    (RLSE_DECODE_STREAM): no page is read by more than one row of the batch,
    so pages are read with non-temporal loads."""
    _check(load().rlse_decode_step_planned(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(q_norm_weight), _ptr(k_norm_weight), eps,
        _ptr(cos_table), _ptr(sin_table), max_pos, _ptr(k_pool), _ptr(v_pool),
        _ptr(block_tables), _ptr(seq_lens), _ptr(out), batch, num_heads, num_kv_heads, head_dim,
        max_blocks_per_seq, num_blocks, scale, _dt(dtype), _ptr(workspace), workspace_bytes,
        _ptr(plan), DECODE_STREAM if stream_pages else 0, _stream(stream)))


def decode_prefix_size(batch: int, num_heads: int, head_dim: int, prefix_pages: int) -> int:
    """Bytes of the prefix partials of a cascade step (rlse_decode_prefix_size)."""
    n = _sz(0)
    _check(load().rlse_decode_prefix_size(batch, num_heads, head_dim, prefix_pages,
                                          ctypes.byref(n)))
    return n.value


def decode_plan_cascade(block_tables, seq_lens, batch: int, num_kv_heads: int,
                        max_blocks_per_seq: int, num_blocks: int, prefix_pages: int, plan,
                        plan_bytes: int, stream=None) -> None:
    """decode_plan for a cascade step: every row's page stream starts after
    the first prefix_pages table entries."""
    _check(load().rlse_decode_plan_cascade(_ptr(block_tables), _ptr(seq_lens), batch,
                                           num_kv_heads, max_blocks_per_seq, num_blocks,
                                           prefix_pages, _ptr(plan), plan_bytes, _stream(stream)))


def decode_step_cascade(q, k_new, v_new, q_norm_weight, k_norm_weight, eps: float, cos_table,
                        sin_table, max_pos: int, k_pool, v_pool, block_tables, seq_lens, out,
                        batch: int, num_heads: int, num_kv_heads: int, head_dim: int,
                        max_blocks_per_seq: int, num_blocks: int, scale: float, dtype, plan,
                        prefix_pages: int, prefix_buf, prefix_bytes: int, workspace=None,
                        workspace_bytes: int = 0, stream=None, stream_pages: bool = False) -> None:
    """The shared-prefix (cascade) decode step: the first prefix_pages pages,
    common to every sequence, attended once for the batch, then each
    sequence's own pages, the two softmax states combined per row. plan: from
    decode_plan_cascade with the same prefix_pages, or None."""
    _check(load().rlse_decode_step_cascade(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(q_norm_weight), _ptr(k_norm_weight), eps,
        _ptr(cos_table), _ptr(sin_table), max_pos, _ptr(k_pool), _ptr(v_pool),
        _ptr(block_tables), _ptr(seq_lens), _ptr(out), batch, num_heads, num_kv_heads, head_dim,
        max_blocks_per_seq, num_blocks, scale, _dt(dtype), _ptr(workspace), workspace_bytes,
        _ptr(plan), DECODE_STREAM if stream_pages else 0, prefix_pages, _ptr(prefix_buf),
        prefix_bytes, _stream(stream)))


def kv_checksum(k_pool, v_pool, block_tables, seq_lens, batch: int, num_kv_heads: int,
                head_dim: int, max_blocks_per_seq: int, num_blocks: int, dtype, out,
                stream=None, plan=None) -> None:
    """Adds every (sequence, KV head) row's K and V checksums into out
    (device int32/uint32 [batch][num_kv_heads][2], zero-filled by the caller).
    plan: a decode plan of the same tables and lengths (rlse_kv_checksum_planned:
    each wave's first page requested from it, as a planned decode does)."""
    if plan is None:
        _check(load().rlse_kv_checksum(_ptr(k_pool), _ptr(v_pool), _ptr(block_tables),
                                       _ptr(seq_lens), batch, num_kv_heads, head_dim,
                                       max_blocks_per_seq, num_blocks, _dt(dtype), _ptr(out),
                                       _stream(stream)))
        return
    _check(load().rlse_kv_checksum_planned(_ptr(k_pool), _ptr(v_pool), _ptr(block_tables),
                                           _ptr(seq_lens), batch, num_kv_heads, head_dim,
                                           max_blocks_per_seq, num_blocks, _dt(dtype), _ptr(plan),
                                           _ptr(out), _stream(stream)))


def decode_plan_groups(block_tables, seq_lens, seq_group, group_pages, num_groups: int,
                       batch: int, num_heads: int, num_kv_heads: int, max_blocks_per_seq: int,
                       num_blocks: int, plan, plan_bytes: int, stream=None) -> None:
    """The plan of a cascade step with prefix groups: seq_group (device int32
    [batch], -1 = no shared prefix) and group_pages (device int32
    [num_groups], the leading table entries each group's members share)."""
    _check(load().rlse_decode_plan_groups(_ptr(block_tables), _ptr(seq_lens), _ptr(seq_group),
                                          _ptr(group_pages), num_groups, batch, num_heads,
                                          num_kv_heads, max_blocks_per_seq, num_blocks,
                                          _ptr(plan), plan_bytes, _stream(stream)))


def decode_step_groups(q, k_new, v_new, q_norm_weight, k_norm_weight, eps: float, cos_table,
                       sin_table, max_pos: int, k_pool, v_pool, block_tables, seq_lens, out,
                       batch: int, num_heads: int, num_kv_heads: int, head_dim: int,
                       max_blocks_per_seq: int, num_blocks: int, scale: float, dtype, plan,
                       num_groups: int, max_group_pages: int, prefix_buf, prefix_bytes: int,
                       workspace=None, workspace_bytes: int = 0, stream=None,
                       stream_pages: bool = False) -> None:
    """The cascade step of a mixed batch: each prefix group's shared pages
    attended once for its members, every other page once for its sequence.
    plan: from decode_plan_groups (required); prefix_buf: decode_prefix_size
    bytes with prefix_pages = max_group_pages."""
    _check(load().rlse_decode_step_groups(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(q_norm_weight), _ptr(k_norm_weight), eps,
        _ptr(cos_table), _ptr(sin_table), max_pos, _ptr(k_pool), _ptr(v_pool),
        _ptr(block_tables), _ptr(seq_lens), _ptr(out), batch, num_heads, num_kv_heads, head_dim,
        max_blocks_per_seq, num_blocks, scale, _dt(dtype), _ptr(workspace), workspace_bytes,
        _ptr(plan), DECODE_STREAM if stream_pages else 0, num_groups, max_group_pages,
        _ptr(prefix_buf), prefix_bytes, _stream(stream)))


def prefill_workspace_size(num_tokens: int, ctx_len: int, num_heads: int, num_kv_heads: int,
                           head_dim: int) -> int:
    n = _sz(0)
    _check(load().rlse_prefill_workspace_size(num_tokens, ctx_len, num_heads, num_kv_heads,
                                              head_dim, ctypes.byref(n)))
    return n.value


def prefill_attn(q, k_pool, v_pool, block_table, ctx_len: int, num_tokens: int, out,
                 num_heads: int, num_kv_heads: int, head_dim: int, max_blocks: int,
                 num_blocks: int, scale: float, dtype, workspace=None, workspace_bytes: int = 0,
                 stream=None) -> None:
    """Causal attention of a chunk of num_tokens queries (positions
    ctx_len-num_tokens .. ctx_len-1) over one sequence's paged K/V."""
    _check(load().rlse_prefill_attn(_ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(block_table),
                                    ctx_len, num_tokens, _ptr(out), num_heads, num_kv_heads,
                                    head_dim, max_blocks, num_blocks, scale, _dt(dtype),
                                    _ptr(workspace), workspace_bytes, _stream(stream)))


def rmsnorm(x, weight, out, rows: int, n: int, eps: float, dtype, stream=None) -> None:
    _check(load().rlse_rmsnorm(_ptr(x), _ptr(weight), _ptr(out), rows, n, eps, _dt(dtype),
                               _stream(stream)))


def rope_tables(theta: float, head_dim: int, max_pos: int, dtype):
    """Host cos/sin tables [max_pos][head_dim/2] as raw bytes (bytearray pair)."""
    es = DTYPE_SIZE[_dt(dtype)]
    n = max_pos * (head_dim // 2)
    cos_b = (ctypes.c_char * (n * es))()
    sin_b = (ctypes.c_char * (n * es))()
    _check(load().rlse_rope_tables(theta, head_dim, max_pos, _dt(dtype),
                                   ctypes.cast(cos_b, _vp), ctypes.cast(sin_b, _vp)))
    return bytes(cos_b), bytes(sin_b)


def rope(q, k, cos_table, sin_table, positions, num_tokens: int, num_heads: int,
         num_kv_heads: int, head_dim: int, max_pos: int, dtype, stream=None) -> None:
    _check(load().rlse_rope(_ptr(q), _ptr(k), _ptr(cos_table), _ptr(sin_table), _ptr(positions),
                            num_tokens, num_heads, num_kv_heads, head_dim, max_pos, _dt(dtype),
                            _stream(stream)))


def qk_norm_rope_append(q, k, v, q_norm_weight, k_norm_weight, eps: float, cos_table, sin_table,
                        max_pos: int, positions, block_tables, num_seqs: int, seq_index,
                        num_tokens: int, num_heads: int, num_kv_heads: int, head_dim: int,
                        max_blocks_per_seq: int, num_blocks: int, q_out, k_pool, v_pool, dtype,
                        stream=None) -> None:
    _check(load().rlse_qk_norm_rope_append(
        _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm_weight), _ptr(k_norm_weight), eps,
        _ptr(cos_table), _ptr(sin_table), max_pos, _ptr(positions), _ptr(block_tables),
        num_seqs, _ptr(seq_index), num_tokens, num_heads, num_kv_heads, head_dim,
        max_blocks_per_seq, num_blocks, _ptr(q_out), _ptr(k_pool), _ptr(v_pool), _dt(dtype),
        _stream(stream)))


# --------------------------------------------------------------------------
# The rest of a decode step (step_decode_batch ops around rlse_decode_step)
# --------------------------------------------------------------------------
def embedding(ids, table, out, batch: int, hidden: int, vocab: int, dtype, stream=None) -> None:
    _check(load().rlse_embedding(_ptr(ids), _ptr(table), _ptr(out), batch, hidden, vocab,
                                 _dt(dtype), _stream(stream)))


def add_rmsnorm(x, residual, weight, out, rows: int, n: int, eps: float, dtype,
                stream=None, packed_out: bool = False) -> None:
    """packed_out: out in the packed row order (PACKED_ROWS) the projections
    read with packed_x; out then holds whole 16-row tiles."""
    _check(load().rlse_add_rmsnorm(_ptr(x), _ptr(residual), _ptr(weight), _ptr(out), rows, n,
                                   eps, _dt(dtype) | (PACKED_ROWS if packed_out else 0),
                                   _stream(stream)))


def silu_mul(gate_up, out, rows: int, inter: int, dtype, stream=None) -> None:
    _check(load().rlse_silu_mul(_ptr(gate_up), _ptr(out), rows, inter, _dt(dtype),
                                _stream(stream)))


def argmax_workspace_size(rows: int, vocab: int) -> int:
    n = _sz(0)
    _check(load().rlse_argmax_workspace_size(rows, vocab, ctypes.byref(n)))
    return n.value


def argmax(logits, out, rows: int, vocab: int, dtype, workspace, workspace_bytes: int,
           stream=None) -> None:
    _check(load().rlse_argmax(_ptr(logits), _ptr(out), rows, vocab, _dt(dtype), _ptr(workspace),
                              workspace_bytes, _stream(stream)))


# RLSE_DENSE_PACKED: OR-ed into the dtype of the projection calls, the
# weight is in the tile order dense_pack writes.
DENSE_PACKED = 0x100
# RLSE_PACKED_ROWS: x of a projection (or out of add_rmsnorm) in the packed
# row order of the MFMA kernel's B operands.
PACKED_ROWS = 0x200
# RLSE_PACKED_OUT: gate_up_silu's act written in that order.
PACKED_OUT = 0x400


def _dtp(dtype, packed: bool, packed_x: bool = False) -> int:
    return _dt(dtype) | (DENSE_PACKED if packed else 0) | (PACKED_ROWS if packed_x else 0)


def dense_pack(weight, packed, out_features: int, in_features: int, gate_up_inter: int, dtype,
               stream=None) -> None:
    """rlse_dense_pack: weight [out][in] row-major -> packed (same size) in the
    order the MFMA projections load; gate_up_inter > 0 for the stacked
    gate/up weight of gate_up_silu."""
    _check(load().rlse_dense_pack(_ptr(weight), _ptr(packed), out_features, in_features,
                                  gate_up_inter, _dt(dtype), _stream(stream)))


def linear(x, weight, bias, y, rows: int, out_features: int, in_features: int, dtype,
           stream=None, packed: bool = False, packed_x: bool = False) -> None:
    _check(load().rlse_linear(_ptr(x), _ptr(weight), _ptr(bias), _ptr(y), rows, out_features,
                              in_features, _dtp(dtype, packed, packed_x), _stream(stream)))


def dense_workspace_size(rows: int, out_features: int, in_features: int) -> int:
    """Bytes of workspace for the K split of qkv_proj / linear_residual /
    gate_up_silu (out_features: all outputs of the call, 2*inter for
    gate_up_silu). Zero-fill it once before first use."""
    n = _sz(0)
    _check(load().rlse_dense_workspace_size(rows, out_features, in_features, ctypes.byref(n)))
    return n.value


def _ws(workspace):
    if workspace is None:
        return None, 0
    return _ptr(workspace), int(workspace.numel() * workspace.element_size())


def qkv_proj(x, w_qkv, b_qkv, q, k, v, rows: int, hidden: int, q_features: int,
             kv_features: int, dtype, workspace=None, stream=None, packed: bool = False,
             packed_x: bool = False) -> None:
    wp, wb = _ws(workspace)
    _check(load().rlse_qkv_proj(_ptr(x), _ptr(w_qkv), _ptr(b_qkv), _ptr(q), _ptr(k), _ptr(v),
                                rows, hidden, q_features, kv_features,
                                _dtp(dtype, packed, packed_x), wp, wb, _stream(stream)))


def linear_residual(x, weight, residual, rows: int, out_features: int, in_features: int, dtype,
                    workspace=None, stream=None, packed: bool = False,
                    packed_x: bool = False) -> None:
    wp, wb = _ws(workspace)
    _check(load().rlse_linear_residual(_ptr(x), _ptr(weight), _ptr(residual), rows,
                                       out_features, in_features, _dtp(dtype, packed, packed_x),
                                       wp, wb, _stream(stream)))


def gate_up_silu(x, w_gate_up, act, rows: int, hidden: int, inter: int, dtype, workspace=None,
                 stream=None, packed: bool = False, packed_x: bool = False,
                 packed_out: bool = False) -> None:
    wp, wb = _ws(workspace)
    _check(load().rlse_gate_up_silu(_ptr(x), _ptr(w_gate_up), _ptr(act), rows, hidden, inter,
                                    _dtp(dtype, packed, packed_x) |
                                    (PACKED_OUT if packed_out else 0), wp, wb, _stream(stream)))


# --------------------------------------------------------------------------
# Device-side failures
# --------------------------------------------------------------------------
def workspace_flags(workspace=None, stream=None) -> int:
    """Synchronises the stream, then reads and clears the sticky error flags
    of a decode or projection workspace (None: the library-owned decode
    workspace). Returns them without raising (WS_ERR_* bits)."""
    flags = ctypes.c_uint(0)
    load().rlse_workspace_check(_ptr(workspace), _stream(stream), ctypes.byref(flags))
    return int(flags.value)


def workspace_check(workspace=None, stream=None) -> None:
    """As workspace_flags, raising DeviceTimeout (a merge gave up) or
    TokenLimitExceeded (a length exceeded its block table) when a flag was
    set -- the point where a serving loop turns a device failure into the
    reference's BackendError."""
    flags = ctypes.c_uint(0)
    _check(load().rlse_workspace_check(_ptr(workspace), _stream(stream), ctypes.byref(flags)))


def set_merge_wait_ns(ns: int) -> None:
    """Bound on a cross-workgroup merge's wait for launches queued after the
    call (default 100 ms; 0 gives up at the first miss)."""
    _check(load().rlse_set_merge_wait_ns(int(ns)))
