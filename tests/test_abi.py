"""The C-ABI library loads, exports every symbol include/rlse_kv.h declares and
rejects bad arguments before touching a device (no GPU needed)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rlse_kv.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*([a-z_0-9]+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_and_binding_agree(kv):
    assert _declared_functions() == sorted(kv.EXPORTED)


def test_library_exports_every_declared_symbol(kv):
    out = subprocess.run(["nm", "-D", "--defined-only", kv.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [n for n in _declared_functions() if n not in exported]
    assert not missing, missing


def test_version_and_error_text(kv):
    assert kv.load().rlse_version() >= 100
    rc = kv.load().rlse_pool_create(1, 8, 8, 128, kv.DTYPE_BF16, 8, ctypes.byref(ctypes.c_void_p()))
    assert rc == kv.ERR_INVALID_VALUE
    assert "block_size" in kv.last_error()


@pytest.mark.parametrize("args", [
    # batch 0 (the reference harness's fail-closed check, validate_cuda_kernels.py:120-122)
    dict(batch=0, hq=16, hkv=8, d=128),
    dict(batch=2, hq=15, hkv=8, d=128),   # heads not a multiple of KV heads
    dict(batch=2, hq=16, hkv=8, d=96),    # unsupported head_dim
    dict(batch=2, hq=72, hkv=8, d=128),   # group size 9 > 8
])
def test_decode_rejects_bad_shapes(kv, args):
    lib = kv.load()
    rc = lib.rlse_paged_gqa_decode(1, 1, 1, 1, 1, 1, args["batch"], args["hq"], args["hkv"],
                                   args["d"], 8, 32, 0.088, kv.DTYPE_BF16, None, 0, None)
    assert rc == kv.ERR_INVALID_VALUE


@pytest.mark.parametrize("case", [
    dict(tq=0, L=10, hq=8, hkv=8, d=128, mb=1, dt="bf16"),     # empty chunk
    dict(tq=20, L=10, hq=8, hkv=8, d=128, mb=1, dt="bf16"),    # chunk longer than context
    dict(tq=4, L=40, hq=8, hkv=8, d=128, mb=2, dt="bf16"),     # table too short for ctx_len
    dict(tq=4, L=10, hq=12, hkv=8, d=128, mb=1, dt="bf16"),    # Hq not a multiple of Hkv
    dict(tq=4, L=10, hq=8, hkv=8, d=96, mb=1, dt="bf16"),      # unsupported head_dim
    dict(tq=4, L=10, hq=8, hkv=8, d=128, mb=1, dt=9),          # no such dtype code
])
def test_prefill_rejects_bad_arguments(kv, case):
    lib = kv.load()
    dt = kv.DTYPE_NAMES[case["dt"]] if isinstance(case["dt"], str) else case["dt"]
    rc = lib.rlse_prefill_attn(1, 1, 1, 1, case["L"], case["tq"], 1, case["hq"], case["hkv"],
                               case["d"], case["mb"], 64, 0.088, dt, None, 0, None)
    assert rc == kv.ERR_INVALID_VALUE, kv.last_error()


def test_prototype_launchers_fail_closed(kv):
    lib = kv.load()
    assert lib.launch_rmsnorm_f32(None, None, None, 0, 1024, 1e-6) != 0
    assert lib.launch_paged_gqa_decode_tiled_f32(None, None, None, None, None, None, 0, 16, 8, 8,
                                                 1.0) != 0


def test_movement_rejects_bad_geometry(kv):
    lib = kv.load()
    # head_dim 3 bf16 = 6 bytes per row: not a whole number of 16-byte packets
    assert lib.rlse_kv_append(1, 1, 1, 1, 1, 1, None, 1, 1, 8, 3, 8, 8, kv.DTYPE_BF16,
                              None) == kv.ERR_INVALID_VALUE
    assert lib.rlse_kv_gather(1, 1, 0, 0, 1, 4, 1, 1, 8, 128, 8, kv.DTYPE_BF16,
                              None) == kv.ERR_INVALID_VALUE
    assert lib.rlse_kv_copy_blocks(1, 1, 0, 1, 1, 1, -1, 8, 128, 8, kv.DTYPE_BF16,
                                   None) == kv.ERR_INVALID_VALUE
    assert lib.rlse_rmsnorm(1, 1, 1, 0, 128, 1e-6, kv.DTYPE_F32, None) == kv.ERR_INVALID_VALUE
    # zero-sized work is a no-op that succeeds without a device
    assert lib.rlse_kv_append(1, 1, 1, 1, 1, 0, None, 1, 0, 8, 128, 8, 8, kv.DTYPE_BF16,
                              None) == kv.OK


def test_rope_tables_match_oracle(kv, orc):
    import numpy as np
    cos_b, sin_b = kv.rope_tables(1e6, 128, 700, kv.DTYPE_F32)
    c = np.frombuffer(cos_b, np.float32).reshape(700, 64)
    s = np.frombuffer(sin_b, np.float32).reshape(700, 64)
    oc, os_ = orc.rope_tables_f32(1e6, 128, 700)
    np.testing.assert_array_equal(c, oc)
    np.testing.assert_array_equal(s, os_)
    cb, _ = kv.rope_tables(1e6, 128, 700, kv.DTYPE_BF16)
    np.testing.assert_array_equal(np.frombuffer(cb, np.uint16).reshape(700, 64),
                                  orc.f32_to_bf16_bits(oc))
