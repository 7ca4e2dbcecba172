"""The long-context and prefix-fork workloads at their stated full size.

* Qwen3-8B long-context decode: 32 query heads, 8 KV heads, head_dim 128,
  bf16, 128 sequences with U[8192, 32768] cached tokens + 1 appended, on
  shuffled 16-token pages -- the regime where the reference's per-sequence
  decode collapsed historically (docs/benchmarks_and_performance.md:94-99).
  One planned fused step (rlse_decode_step_planned: q/k norm, RoPE, append,
  decode) runs over all 128 sequences; 8 rows (the longest, the shortest and
  six seeded others) are checked with all their heads against the oracle's
  Candle op chain (RmsNorm, apply_rope, KvCache append, zero-copy GQA decode;
  src/backends/qwen2.rs:177-203, 291-328), and the whole batch through
  size-independent properties: a repeated launch gives the same bits and
  raises no device error.
* Qwen3-0.6B prefix-fork decode: 64 sequences forked from one 1024- or
  1030-token prefix (src/cache/prefix_cache.rs:250-345,
  src/backends/candle.rs:437-478), private suffixes U[64, 512], one layer.
  Forked pages (shared by refcount, the partial page copied on write) must
  read back byte for byte as prefix || suffix, the fused decode step over
  them must equal the same step over private copies bit for bit, and the
  shared prefix must be unchanged after the forks' appends
  (src/backends/candle.rs:1281-1292).
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import DEV, TOL, err_report, to_dev

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _bits(t):
    return t.contiguous().view(torch.int16)


def _host_bf16(t):
    torch.cuda.synchronize()
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _rope_dev(kv, d, max_pos):
    cos_b, sin_b = kv.rope_tables(1e6, d, max_pos, "bf16")
    c = np.frombuffer(cos_b, np.uint16).reshape(max_pos, d // 2).copy()
    s = np.frombuffer(sin_b, np.uint16).reshape(max_pos, d // 2).copy()
    return c, s, to_dev(c, "bf16"), to_dev(s, "bf16")


def test_qwen3_8b_long_context_decode_step_full_batch(kv):
    hq, hkv, d, b = 32, 8, 128, 128
    rng = np.random.default_rng(5)
    cached = rng.integers(8192, 32769, b).astype(np.int32)
    lens = cached + 1
    pages = (lens + 15) // 16
    mbps = int(pages.max())
    nb = int(pages.sum()) + 16
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.zeros((b, mbps), np.int32)
    used = 0
    for i in range(b):
        tables[i, :pages[i]] = perm[used:used + pages[i]]
        used += int(pages[i])
    print(f"qwen3-8b decode: B={b} keys {int(lens.min())}..{int(lens.max())} "
          f"pages {nb} ({2 * nb * hkv * 16 * d * 2 / 1e9:.1f} GB K+V)", flush=True)
    g = torch.Generator(device=DEV)
    g.manual_seed(5)
    kp = torch.randn((nb, hkv, 16, d), generator=g, device=DEV, dtype=BF)
    vp = torch.randn((nb, hkv, 16, d), generator=g, device=DEV, dtype=BF)
    q = torch.randn((b, hq, d), generator=g, device=DEV, dtype=BF)
    kn = torch.randn((b, hkv, d), generator=g, device=DEV, dtype=BF)
    vn = torch.randn((b, hkv, d), generator=g, device=DEV, dtype=BF)
    qw = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(BF)
    kw = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(BF)
    max_pos = mbps * 16
    c_h, s_h, c_d, s_d = _rope_dev(kv, d, max_pos)
    t_dev, l_dev = to_dev(tables), to_dev(lens)
    ws = torch.zeros(kv.decode_workspace_size(b, hq, hkv, d), dtype=torch.uint8, device=DEV)
    plan = torch.zeros(kv.decode_plan_size(), dtype=torch.uint8, device=DEV)
    scale = 1.0 / math.sqrt(d)
    outs = []
    for rep in range(2):
        out = torch.full((b, hq, d), 7.0, dtype=BF, device=DEV)
        print(f"qwen3-8b decode: planned fused step, launch {rep}", flush=True)
        kv.decode_plan(t_dev, l_dev, b, hkv, mbps, nb, plan, plan.numel())
        kv.decode_step_planned(q, kn, vn, qw, kw, 1e-6, c_d, s_d, max_pos, kp, vp, t_dev, l_dev,
                               out, b, hq, hkv, d, mbps, nb, scale, "bf16", plan, ws, ws.numel(),
                               stream_pages=rep == 1)
        torch.cuda.synchronize()
        assert kv.workspace_flags(ws) == 0
        outs.append(out)
    # the second launch (streamed pages) re-appends the same token bits at the
    # same positions and gives the first's output
    assert torch.equal(_bits(outs[0]), _bits(outs[1]))

    rows = [int(np.argmax(lens)), int(np.argmin(lens))]
    rows += [int(r) for r in rng.choice(np.setdiff1d(np.arange(b), rows), 6, replace=False)]
    got_all = O.bf16_bits_to_f32(_host_bf16(outs[0]))
    qh, knh, vnh = _host_bf16(q), _host_bf16(kn), _host_bf16(vn)
    qwh, kwh = _host_bf16(qw), _host_bf16(kw)
    worst = 0.0
    for r in rows:
        n = int(lens[r])
        ko = torch.empty((1, hkv, n, d), dtype=BF, device=DEV)
        vo = torch.empty_like(ko)
        kv.kv_gather(kp, vp, 0, 1, t_dev[r], n, ko, vo, hkv, d, nb, "bf16")
        kh, vh = _host_bf16(ko)[0], _host_bf16(vo)[0]
        pos = np.full(hkv, n - 1, np.int32)
        # the appended token: k_norm + RoPE of the raw k (bit-exact), raw v
        k_ref = O.apply_rope_bf16(O.rmsnorm_bf16(knh[r], kwh, 1e-6), pos, c_h, s_h)
        np.testing.assert_array_equal(kh[:, n - 1], k_ref)
        np.testing.assert_array_equal(vh[:, n - 1], vnh[r])
        q_ref = O.apply_rope_bf16(O.rmsnorm_bf16(qh[r], qwh, 1e-6), np.full(hq, n - 1, np.int32),
                                  c_h, s_h)
        want = O.decode_batch_f32(O.bf16_bits_to_f32(q_ref)[None], O.bf16_bits_to_f32(kh)[None],
                                  O.bf16_bits_to_f32(vh)[None], np.array([n], np.int32), scale)
        mx, rel = err_report(got_all[r], want[0])
        worst = max(worst, mx)
        print(f"[qwen3-8b row {r} keys {n}] max_abs={mx:.3e} rel={rel:.3e}", flush=True)
        assert np.isfinite(got_all[r]).all()
        assert mx <= TOL["bf16"], (r, mx)
    print(f"qwen3-8b decode: 8 rows x 32 heads within {worst:.3e} (bar 2e-2)")


@pytest.mark.parametrize("prefix_len", [1024, 1030])
def test_prefix_fork_decode_full_size(kv, prefix_len):
    hq, hkv, d, b = 16, 8, 128, 64
    rng = np.random.default_rng(prefix_len)
    suffix = rng.integers(64, 513, b).astype(np.int32)
    lens = prefix_len + suffix + 1           # keys after this step's append
    priv_pages = int(((lens + 15) // 16).sum())
    nb = priv_pages + 64
    print(f"fork full size: prefix {prefix_len}, B={b}, suffix {int(suffix.min())}.."
          f"{int(suffix.max())}, {nb} pages per layout", flush=True)
    pa = kv.KVPool(1, nb, hkv, d, "bf16")    # forked: shared prefix pages
    pb = kv.KVPool(1, nb, hkv, d, "bf16")    # private copies
    ka, va = pa.layer(0)
    kb, vb = pb.layer(0)
    bma, bmb = kv.BlockManager(nb), kv.BlockManager(nb)
    g = torch.Generator(device=DEV)
    g.manual_seed(prefix_len)
    pk = torch.randn((1, hkv, prefix_len, d), generator=g, device=DEV, dtype=BF)
    pv = torch.randn((1, hkv, prefix_len, d), generator=g, device=DEV, dtype=BF)
    bma.allocate("prefix", prefix_len)
    ptab = to_dev(np.array(bma.block_table("prefix"), np.int32))
    kv.kv_scatter(pk, pv, ka, va, 0, 1, ptab, 0, prefix_len, hkv, d, nb, "bf16")
    src, dst = [], []
    for i in range(b):
        for s_, d_ in bma.fork("prefix", f"r{i}", prefix_len):
            src.append(s_)
            dst.append(d_)
        while len(bma.block_table(f"r{i}")) * 16 < int(lens[i]):
            bma.allocate_block(f"r{i}")
        bmb.allocate(f"r{i}", int(lens[i]))
    assert len(src) == (b if prefix_len % 16 else 0)
    if src:
        kv.kv_copy_blocks(ka, va, 0, 1, to_dev(np.array(src, np.int32)),
                          to_dev(np.array(dst, np.int32)), len(src), hkv, d, nb, "bf16")
    mbps = max(len(bma.block_table(f"r{i}")) for i in range(b))
    ta = np.zeros((b, mbps), np.int32)
    tb = np.zeros((b, mbps), np.int32)
    suffix_kv = []
    for i in range(b):
        a_t, b_t = bma.block_table(f"r{i}"), bmb.block_table(f"r{i}")
        ta[i, :len(a_t)] = a_t
        tb[i, :len(b_t)] = b_t
        n = int(suffix[i])
        sk = torch.randn((1, hkv, n, d), generator=g, device=DEV, dtype=BF)
        sv = torch.randn((1, hkv, n, d), generator=g, device=DEV, dtype=BF)
        suffix_kv.append((sk, sv))
        kv.kv_scatter(sk, sv, ka, va, 0, 1, to_dev(ta[i]), prefix_len, n, hkv, d, nb, "bf16")
        kv.kv_scatter(torch.cat([pk, sk], 2), torch.cat([pv, sv], 2), kb, vb, 0, 1, to_dev(tb[i]),
                      0, prefix_len + n, hkv, d, nb, "bf16")
    torch.cuda.synchronize()
    # forked pages read back as prefix || suffix, byte for byte
    for i in range(b):
        n = prefix_len + int(suffix[i])
        ko = torch.empty((1, hkv, n, d), dtype=BF, device=DEV)
        vo = torch.empty_like(ko)
        kv.kv_gather(ka, va, 0, 1, to_dev(ta[i]), n, ko, vo, hkv, d, nb, "bf16")
        sk, sv = suffix_kv[i]
        assert torch.equal(_bits(ko), _bits(torch.cat([pk, sk], 2))), i
        assert torch.equal(_bits(vo), _bits(torch.cat([pv, sv], 2))), i
    max_pos = mbps * 16
    _, _, c_d, s_d = _rope_dev(kv, d, max_pos)
    q = torch.randn((b, hq, d), generator=g, device=DEV, dtype=BF)
    kn = torch.randn((b, hkv, d), generator=g, device=DEV, dtype=BF)
    vn = torch.randn((b, hkv, d), generator=g, device=DEV, dtype=BF)
    qw = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(BF)
    kw = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(BF)
    l_dev = to_dev(lens.astype(np.int32))
    outs = []
    for (k0, v0), tab in (((ka, va), ta), ((kb, vb), tb)):
        out = torch.empty((b, hq, d), dtype=BF, device=DEV)
        print(f"fork full size: fused decode step, {'forked' if k0 is ka else 'private'}",
              flush=True)
        kv.decode_step(q, kn, vn, qw, kw, 1e-6, c_d, s_d, max_pos, k0, v0, to_dev(tab), l_dev, out,
                       b, hq, hkv, d, mbps, nb, 1.0 / math.sqrt(d), "bf16")
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(_bits(outs[0]), _bits(outs[1]))
    assert kv.workspace_flags() == 0
    # Planned steps over the same inputs (the appended token is rewritten with
    # the same bits): the forked layout shares pages, so they stay cacheable;
    # the private layout streams them (RLSE_DECODE_STREAM). Both give the
    # unplanned output bit for bit.
    plan = torch.zeros(kv.decode_plan_size(), dtype=torch.uint8, device=DEV)
    for (k0, v0), tab, streams in (((ka, va), ta, False), ((kb, vb), tb, True)):
        t_dev = to_dev(tab)
        kv.decode_plan(t_dev, l_dev, b, hkv, mbps, nb, plan, plan.numel())
        out = torch.empty((b, hq, d), dtype=BF, device=DEV)
        print(f"fork full size: planned step, {'private' if streams else 'forked'}", flush=True)
        kv.decode_step_planned(q, kn, vn, qw, kw, 1e-6, c_d, s_d, max_pos, k0, v0, t_dev, l_dev,
                               out, b, hq, hkv, d, mbps, nb, 1.0 / math.sqrt(d), "bf16", plan,
                               stream_pages=streams)
        torch.cuda.synchronize()
        assert torch.equal(_bits(out), _bits(outs[0]))
    # every sequence, its appended token included, reads back identically
    for i in range(b):
        n = int(lens[i])
        got = []
        for (k0, v0), tab in (((ka, va), ta), ((kb, vb), tb)):
            ko = torch.empty((1, hkv, n, d), dtype=BF, device=DEV)
            vo = torch.empty_like(ko)
            kv.kv_gather(k0, v0, 0, 1, to_dev(tab[i]), n, ko, vo, hkv, d, nb, "bf16")
            got.append((ko, vo))
        assert torch.equal(_bits(got[0][0]), _bits(got[1][0])), i
        assert torch.equal(_bits(got[0][1]), _bits(got[1][1])), i
    # the shared prefix is untouched
    ko = torch.empty((1, hkv, prefix_len, d), dtype=BF, device=DEV)
    vo = torch.empty_like(ko)
    kv.kv_gather(ka, va, 0, 1, ptab, prefix_len, ko, vo, hkv, d, nb, "bf16")
    torch.cuda.synchronize()
    assert torch.equal(_bits(ko), _bits(pk)) and torch.equal(_bits(vo), _bits(pv))
    print(f"fork full size: prefix {prefix_len}: forked == private, prefix unchanged")
    pa.close()
    pb.close()
