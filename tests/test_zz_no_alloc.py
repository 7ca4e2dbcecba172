"""rlse_decode_step_noalloc: the fused decode step without a workspace (its
split-K records in the library's static device scratch) against
rlse_decode_step with a caller workspace, bit for bit, on two calls in a row
-- the second with a smaller batch, so records of the first call are still
in the scratch when the second runs. No counterpart in the reference; the
step itself restates Attention::forward's decode branch
(src/backends/qwen2.rs:291-328), checked against the oracle elsewhere.
"""
import math

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, build_tables, to_dev

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _case(kv, rng, g, lens, hq, hkv, d):
    lens = np.asarray(lens, np.int32)
    b = len(lens)
    mbps = int(max((int(n) + 15) // 16 for n in lens))
    nb = int(sum((int(n) + 15) // 16 for n in lens)) + 5
    tables = build_tables(rng, lens, nb, mbps)
    kp = torch.randn((nb, hkv, 16, d), generator=g, device=DEV, dtype=BF)
    vp = torch.randn((nb, hkv, 16, d), generator=g, device=DEV, dtype=BF)
    q = torch.randn((b, hq, d), generator=g, device=DEV, dtype=BF)
    kn = torch.randn((b, hkv, d), generator=g, device=DEV, dtype=BF)
    vn = torch.randn((b, hkv, d), generator=g, device=DEV, dtype=BF)
    qw = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(BF)
    kw = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(BF)
    max_pos = mbps * 16
    cos_b, sin_b = kv.rope_tables(1e6, d, max_pos, "bf16")
    c = torch.frombuffer(bytearray(cos_b), dtype=torch.int16).to(DEV).view(BF)
    s = torch.frombuffer(bytearray(sin_b), dtype=torch.int16).to(DEV).view(BF)
    return dict(kp=kp, vp=vp, q=q, kn=kn, vn=vn, qw=qw, kw=kw, c=c, s=s, max_pos=max_pos,
                t=to_dev(tables), l=to_dev(lens), b=b, mbps=mbps, nb=nb)


def _run(kv, x, hq, hkv, d, noalloc, ws=None):
    kp, vp = x["kp"].clone(), x["vp"].clone()
    out = torch.full((x["b"], hq, d), 5.0, dtype=BF, device=DEV)
    args = (x["q"], x["kn"], x["vn"], x["qw"], x["kw"], 1e-6, x["c"], x["s"], x["max_pos"], kp, vp,
            x["t"], x["l"], out, x["b"], hq, hkv, d, x["mbps"], x["nb"], 1.0 / math.sqrt(d),
            "bf16")
    if noalloc:
        kv.decode_step_noalloc(*args)
    else:
        kv.decode_step(*args, ws, ws.numel())
    torch.cuda.synchronize()
    return out, kp, vp


def _same(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (14, 2, 64)])
def test_noalloc_step_equals_workspace_step_on_two_calls(kv, hq, hkv, d):
    rng = np.random.default_rng(hq + d)
    g = torch.Generator(device=DEV)
    g.manual_seed(hq * d)
    big = _case(kv, rng, g, rng.integers(128, 2049, 32) + 1, hq, hkv, d)
    small = _case(kv, rng, g, rng.integers(1, 600, 5) + 1, hq, hkv, d)
    ws = torch.zeros(kv.decode_workspace_size(32, hq, hkv, d), dtype=torch.uint8, device=DEV)
    kv.workspace_flags()   # start from clear flags in the library's own workspaces
    for name, x in (("B=32 U[128,2048]", big), ("B=5 U[1,600]", small)):
        print(f"noalloc Hq={hq} Hkv={hkv} d={d} {name}: workspace step", flush=True)
        want = _run(kv, x, hq, hkv, d, False, ws)
        print(f"noalloc Hq={hq} Hkv={hkv} d={d} {name}: static-scratch step", flush=True)
        got = _run(kv, x, hq, hkv, d, True)
        for a, b_, what in zip(got, want, ("out", "k_pool", "v_pool")):
            assert _same(a, b_), f"{name}: {what} differs"
        assert kv.workspace_flags(ws) == 0
        assert kv.workspace_flags() == 0


def test_noalloc_step_reports_invalid_rows_through_the_library_flags(kv):
    """A row longer than its block table raises RLSE_WS_ERR_LENGTH in the
    static scratch; rlse_workspace_check(NULL) reads and clears it."""
    rng = np.random.default_rng(7)
    g = torch.Generator(device=DEV)
    g.manual_seed(7)
    hq, hkv, d = 16, 8, 128
    x = _case(kv, rng, g, [40, 300, 47], hq, hkv, d)
    lens = np.array([40, 300, x["mbps"] * 16 + 1], np.int32)
    x["l"] = to_dev(lens)
    kv.workspace_flags()
    out, _, _ = _run(kv, x, hq, hkv, d, True)
    assert kv.workspace_flags() == kv.WS_ERR_LENGTH
    assert kv.workspace_flags() == 0
    assert torch.count_nonzero(out[2].float()) == 0
