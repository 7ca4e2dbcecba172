"""Pool checksums (rlse_kv_checksum, and rlse_kv_checksum_planned with a
decode plan) on the GPU against the oracle's
definition, and the append checked through them at full size.

The checksum of a (sequence, KV head) row is the sum mod 2^32, over its
attended positions and the 32-bit words of each position's elements, of a
mix of word, position and word index (oracle.kv_checksum_ref, pinned against
a brute-force loop in tests/test_oracle.py). Its use here is the reference's
snapshot-bytes check (src/backends/candle.rs:1281-1292) at sizes where
copying the pool back is costly: after a decode step over the benched
Qwen3-0.6B batch (140 MB of K/V in one layer) the pool's sums must equal the
sums of the expected pool -- the old one with each sequence's new row, the
oracle's k_norm + RoPE of the new k and the raw new v, at its position.
Bit-exact throughout.
"""
import math
import os
import sys

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import DEV, build_tables, random_values, to_dev

pytestmark = pytest.mark.gpu

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402  (the bench's own input builders)


def _host_bits(t):
    torch.cuda.synchronize()
    if t.dtype == torch.float32:
        return t.contiguous().cpu().numpy()
    return t.contiguous().view(torch.int16).cpu().numpy().view(
        np.uint16 if t.dtype == torch.bfloat16 else np.float16)


def _device_sums(kv, kp, vp, tables, lens, hkv, d, nb, dtype, reps=1, plan=None):
    """The device sums; plan: None (rlse_kv_checksum), "plan" (a decode plan
    of the same tables and lengths: rlse_kv_checksum_planned) or "zeros" (a
    zero-filled plan buffer, whose stamp is no plain plan's: ignored)."""
    out = torch.zeros((len(lens), hkv, 2), dtype=torch.int32, device=DEV)
    t_dev, l_dev = to_dev(tables), to_dev(np.asarray(lens, np.int32))
    pl = None
    if plan is not None:
        pl = torch.zeros(kv.decode_plan_size(), dtype=torch.uint8, device=DEV)
        if plan == "plan":
            kv.decode_plan(t_dev, l_dev, len(lens), hkv, tables.shape[1], nb, pl, pl.numel())
    for _ in range(reps):
        kv.kv_checksum(kp, vp, t_dev, l_dev, len(lens), hkv, d, tables.shape[1], nb, dtype, out,
                       plan=pl)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("hkv,d", [(8, 128), (2, 64), (1, 128)])
def test_checksums_match_oracle(kv, dtype, hkv, d):
    """Ragged lengths (empty, one token, page edges, long rows), a page id
    outside the pool and a row longer than its table, on shuffled pages; a
    second call adds the same sums again (mod 2^32)."""
    rng = np.random.default_rng(hkv * 100 + d + len(dtype))
    lens = np.array([0, 1, 15, 16, 17, 33, 700, 2049, 300, 64], np.int32)
    mbps = (int(lens.max()) + 15) // 16
    nb = int(sum((int(n) + 15) // 16 for n in lens)) + 5
    tables = build_tables(rng, lens, nb, mbps)
    tables[6, 3] = nb + 7               # a page outside the pool: skipped
    lens = lens.copy()
    lens[9] = 16 * mbps + 1             # longer than its table: no keys
    kp = random_values(rng, (nb, hkv, 16, d), dtype)
    vp = random_values(rng, (nb, hkv, 16, d), dtype)
    want = O.kv_checksum_ref(kp, vp, tables, lens)
    print(f"checksum {dtype} Hkv={hkv} d={d} B={len(lens)}", flush=True)
    got = _device_sums(kv, to_dev(kp, dtype), to_dev(vp, dtype), tables, lens, hkv, d, nb, dtype)
    np.testing.assert_array_equal(got, want)
    twice = _device_sums(kv, to_dev(kp, dtype), to_dev(vp, dtype), tables, lens, hkv, d, nb,
                         dtype, reps=2)
    np.testing.assert_array_equal(twice, (2 * want.astype(np.uint64) & 0xFFFFFFFF).astype(np.uint32))
    # The planned walk (first pages from a decode plan) and a plan of no
    # plain step's shape (ignored) give the same sums.
    for plan in ("plan", "zeros"):
        got = _device_sums(kv, to_dev(kp, dtype), to_dev(vp, dtype), tables, lens, hkv, d, nb,
                           dtype, plan=plan)
        np.testing.assert_array_equal(got, want, err_msg=f"plan={plan}")


def test_full_batch_append_through_checksums(kv):
    """The Qwen3-0.6B bench batch (B=32, cached U[128,2048] + 1, 140 MB of
    K/V): pool sums before a planned streamed decode step equal the oracle's
    of the host copy; after it they equal the oracle's of the expected pool,
    in which only each sequence's new position changed (k_norm + RoPE of its
    new k, its raw new v)."""
    workload = "qwen3"
    hq, hkv, d, _, b, _, _, _ = bench.WORKLOADS[workload]
    w = bench.decode_inputs(workload, 2, DEV, layers=1)
    lens, tables, mbps, nb = w["lens"], w["tables"], w["mbps"], w["num_blocks"]
    kp, vp = w["k_pools"][0], w["v_pools"][0]
    kp0, vp0 = _host_bits(kp), _host_bits(vp)
    print(f"full batch: {w['pages']} pages, {kp.numel() * 4 / 1e6:.0f} MB of K/V", flush=True)
    before = O.kv_checksum_ref(kp0, vp0, tables, lens)
    np.testing.assert_array_equal(_device_sums(kv, kp, vp, tables, lens, hkv, d, nb, "bf16"),
                                  before)
    np.testing.assert_array_equal(
        _device_sums(kv, kp, vp, tables, lens, hkv, d, nb, "bf16", plan="plan"), before)
    t_dev, l_dev = to_dev(tables), to_dev(lens)
    out = torch.empty((b, hq, d), dtype=torch.bfloat16, device=DEV)
    ws = torch.zeros(kv.decode_workspace_size(b, hq, hkv, d), dtype=torch.uint8, device=DEV)
    plan = torch.zeros(kv.decode_plan_size(), dtype=torch.uint8, device=DEV)
    kv.decode_plan(t_dev, l_dev, b, hkv, mbps, nb, plan, plan.numel())
    kv.decode_step_planned(w["q"][0], w["k_new"][0], w["v_new"][0], w["q_norm"][0],
                           w["k_norm"][0], 1e-6, w["cos"], w["sin"], w["max_pos"], kp, vp, t_dev,
                           l_dev, out, b, hq, hkv, d, mbps, nb, 1.0 / math.sqrt(d), "bf16", plan,
                           ws, ws.numel(), stream_pages=True)
    torch.cuda.synchronize()
    assert kv.workspace_flags(ws) == 0
    c_h = np.frombuffer(w["cos_bytes"], np.uint16).reshape(w["max_pos"], d // 2)
    s_h = np.frombuffer(w["sin_bytes"], np.uint16).reshape(w["max_pos"], d // 2)
    knh, vnh, kwh = (_host_bits(x) for x in (w["k_new"][0], w["v_new"][0], w["k_norm"][0]))
    for i in range(b):                  # the expected pool: the new rows at their positions
        pos = int(lens[i]) - 1
        blk, slot = int(tables[i, pos // 16]), pos % 16
        kn = O.rmsnorm_bf16(knh[i], kwh, 1e-6)
        kp0[blk, :, slot] = O.apply_rope_bf16(kn, np.full(hkv, pos, np.int32), c_h, s_h)
        vp0[blk, :, slot] = vnh[i]
    got = _device_sums(kv, kp, vp, tables, lens, hkv, d, nb, "bf16")
    np.testing.assert_array_equal(got, O.kv_checksum_ref(kp0, vp0, tables, lens))
    got = _device_sums(kv, kp, vp, tables, lens, hkv, d, nb, "bf16", plan="plan")
    np.testing.assert_array_equal(got, O.kv_checksum_ref(kp0, vp0, tables, lens))
    print(f"full batch: {b * hkv} rows' K and V sums equal the expected pool's after the append")
