"""Shared-prefix (cascade) decode step on the GPU.

rlse_decode_step_cascade attends the first prefix_pages pages -- the same
pages in every sequence's block table, as after a prefix fork
(src/cache/prefix_cache.rs:250-345, src/backends/candle.rs:437-478) -- once
for the whole batch and then each sequence's own pages, combining the two
softmax states per row. Its result is decode_attention_gqa_zero_copy
(src/backends/qwen2.rs:177-203) over each sequence's full key range, checked
here against the oracle on the appended pool (bar 2e-2 for bf16/f16, as for
every decode), against rlse_decode_step_planned (the same attention with
another sum order), and for the pool bytes and the error flags.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import DEV, TOL, err_report, to_dev

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _host16(t):
    torch.cuda.synchronize()
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _to_f32(bits, dtype):
    return O.bf16_bits_to_f32(bits) if dtype == "bf16" else bits.view(np.float16).astype(np.float32)


def _fork_batch(rng, b, prefix_pages, suffix_lo, suffix_hi, hkv, d, dtype, seed):
    """A pool in which every sequence's first prefix_pages pages are one
    shared set and the rest are private (shuffled page ids)."""
    suffix = rng.integers(suffix_lo, suffix_hi + 1, b).astype(np.int32)
    lens = (16 * prefix_pages + suffix + 1).astype(np.int32)   # keys after the append
    own = (lens + 15) // 16 - prefix_pages
    nb = prefix_pages + int(own.sum()) + 3
    perm = rng.permutation(nb).astype(np.int32)
    shared = perm[:prefix_pages]
    mbps = int(prefix_pages + own.max())
    tables = np.zeros((b, mbps), np.int32)
    used = prefix_pages
    for i in range(b):
        tables[i, :prefix_pages] = shared
        tables[i, prefix_pages:prefix_pages + own[i]] = perm[used:used + own[i]]
        used += int(own[i])
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    tdt = BF if dtype == "bf16" else torch.float16
    kp = torch.randn((nb, hkv, 16, d), generator=g, device=DEV).to(tdt)
    vp = torch.randn((nb, hkv, 16, d), generator=g, device=DEV).to(tdt)
    return lens, tables, nb, mbps, kp, vp, g, tdt


def _step_inputs(kv, g, tdt, b, hq, hkv, d, mbps, dtype):
    q = torch.randn((b, hq, d), generator=g, device=DEV).to(tdt)
    kn = torch.randn((b, hkv, d), generator=g, device=DEV).to(tdt)
    vn = torch.randn((b, hkv, d), generator=g, device=DEV).to(tdt)
    qw = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(tdt)
    kw = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(tdt)
    max_pos = mbps * 16
    cos_b, sin_b = kv.rope_tables(1e6, d, max_pos, dtype)
    c_h = np.frombuffer(cos_b, np.uint16).reshape(max_pos, d // 2).copy()
    s_h = np.frombuffer(sin_b, np.uint16).reshape(max_pos, d // 2).copy()
    c_d = torch.from_numpy(c_h.view(np.int16)).to(DEV).view(tdt)
    s_d = torch.from_numpy(s_h.view(np.int16)).to(DEV).view(tdt)
    return q, kn, vn, qw, kw, max_pos, c_h, s_h, c_d, s_d


@pytest.mark.parametrize("hq,hkv,d,b,prefix_pages,dtype,suffix_hi", [
    (16, 8, 128, 64, 64, "bf16", 300),  # Qwen3-0.6B fork workload: 1024-token prefix, 64 sequences
    (16, 8, 128, 64, 64, "bf16", 20),   # short suffixes: rows finish inside one wave's range
    (14, 2, 64, 9, 5, "bf16", 300),     # G = 7, a tile of 16 queries cut by the batch end
    (32, 8, 128, 3, 1, "f16", 300),     # G = 4, one shared page, f16
    (8, 8, 64, 2, 17, "bf16", 300),     # G = 1, two slices, waves with unequal page shares
    (16, 8, 128, 2, 130, "bf16", 300),  # eight slices of 17 pages, idle waves in each
])
def test_cascade_step_matches_oracle_and_planned(kv, hq, hkv, d, b, prefix_pages, dtype,
                                                 suffix_hi):
    rng = np.random.default_rng(prefix_pages * 31 + b + suffix_hi)
    lens, tables, nb, mbps, kp, vp, g, tdt = _fork_batch(rng, b, prefix_pages, 0, suffix_hi, hkv,
                                                        d, dtype, seed=prefix_pages + b)
    q, kn, vn, qw, kw, max_pos, c_h, s_h, c_d, s_d = _step_inputs(kv, g, tdt, b, hq, hkv, d,
                                                                  mbps, dtype)
    print(f"cascade: Hq={hq} Hkv={hkv} d={d} B={b} prefix {prefix_pages} pages, keys "
          f"{int(lens.min())}..{int(lens.max())}, {dtype}", flush=True)
    t_dev, l_dev = to_dev(tables), to_dev(lens)
    scale = 1.0 / math.sqrt(d)
    ws = torch.zeros(kv.decode_workspace_size(b, hq, hkv, d), dtype=torch.uint8, device=DEV)
    plan = torch.zeros(kv.decode_plan_size(), dtype=torch.uint8, device=DEV)
    pre = torch.zeros(kv.decode_prefix_size(b, hq, d, prefix_pages), dtype=torch.uint8,
                      device=DEV)
    results = {}
    for name in ("planned", "cascade", "cascade_unplanned", "cascade_stream"):
        kp_i, vp_i = kp.clone(), vp.clone()
        out = torch.full((b, hq, d), 3.0, dtype=tdt, device=DEV)
        args = (q, kn, vn, qw, kw, 1e-6, c_d, s_d, max_pos, kp_i, vp_i, t_dev, l_dev, out, b, hq,
                hkv, d, mbps, nb, scale, dtype)
        if name == "planned":
            kv.decode_plan(t_dev, l_dev, b, hkv, mbps, nb, plan, plan.numel())
            kv.decode_step_planned(*args, plan, ws, ws.numel())
        else:
            p_ = None
            if name != "cascade_unplanned":
                kv.decode_plan_cascade(t_dev, l_dev, b, hkv, mbps, nb, prefix_pages, plan,
                                       plan.numel())
                p_ = plan
            kv.decode_step_cascade(*args, p_, prefix_pages, pre, pre.numel(), ws, ws.numel(),
                                   stream_pages=name == "cascade_stream")
        torch.cuda.synchronize()
        assert kv.workspace_flags(ws) == 0, name
        results[name] = (_host16(out), _host16(kp_i), _host16(vp_i))
    ref_out, ref_k, ref_v = results["planned"]
    for name in ("cascade", "cascade_unplanned", "cascade_stream"):
        out_h, k_h, v_h = results[name]
        # the append is the same bytes; the output differs only by the sum order
        np.testing.assert_array_equal(k_h, ref_k, err_msg=name)
        np.testing.assert_array_equal(v_h, ref_v, err_msg=name)
        mx, rel = err_report(_to_f32(out_h, dtype), _to_f32(ref_out, dtype))
        print(f"[{name} vs planned] max_abs={mx:.3e} rel={rel:.3e}")
        assert mx <= 1e-2, (name, mx)
    # planned and unplanned cascade steps, cacheable or streamed pages: one result
    for name in ("cascade_unplanned", "cascade_stream"):
        np.testing.assert_array_equal(results[name][0], results["cascade"][0], err_msg=name)

    # against the oracle over each row's full key range, on the appended pool
    out_c, k_h, v_h = results["cascade"]
    got = _to_f32(out_c, dtype)
    kf, vf = _to_f32(k_h, dtype), _to_f32(v_h, dtype)
    qh, qwh = _host16(q), _host16(qw)
    rows = sorted(set([0, b - 1, int(np.argmax(lens))] + list(rng.choice(b, min(b, 5), False))))
    worst = 0.0
    for r in rows:
        n = int(lens[r])
        pos = np.full(hq, n - 1, np.int32)
        if dtype == "bf16":
            q_ref = O.bf16_bits_to_f32(O.apply_rope_bf16(O.rmsnorm_bf16(qh[r], qwh, 1e-6), pos,
                                                          c_h, s_h))
        else:
            qn = O.rmsnorm_f16(qh[r].view(np.float16), qwh.view(np.float16), 1e-6)
            q_ref = O.rope_ref(qn.astype(np.float32), pos, c_h.view(np.float16).astype(np.float32),
                               s_h.view(np.float16).astype(np.float32), "f16").astype(np.float32)
        kc = O.paged_to_contiguous(kf, tables[r], n)
        vc = O.paged_to_contiguous(vf, tables[r], n)
        want = O.decode_batch_f32(q_ref[None], kc[None], vc[None], np.array([n], np.int32), scale)
        mx, rel = err_report(got[r], want[0])
        worst = max(worst, mx)
        assert np.isfinite(got[r]).all()
        assert mx <= TOL[dtype], (r, mx)
    print(f"cascade: rows {rows} within {worst:.3e} of the oracle (bar {TOL[dtype]})")


def test_cascade_contract_violations_raise_the_prefix_flag(kv):
    """A sequence whose first prefix_pages table entries are not sequence
    0's, or whose new token lies inside the prefix, breaks the cascade
    contract: the step raises RLSE_WS_ERR_PREFIX (rlse_workspace_check maps
    it to RLSE_ERR_INVALID_VALUE). Host-side limits are errors at the call."""
    hq, hkv, d, b, pp = 16, 8, 128, 4, 3
    rng = np.random.default_rng(77)
    lens, tables, nb, mbps, kp, vp, g, tdt = _fork_batch(rng, b, pp, 20, 60, hkv, d, "bf16", 7)
    q, kn, vn, qw, kw, max_pos, _, _, c_d, s_d = _step_inputs(kv, g, tdt, b, hq, hkv, d, mbps,
                                                              "bf16")
    ws = torch.zeros(kv.decode_workspace_size(b, hq, hkv, d), dtype=torch.uint8, device=DEV)
    pre = torch.zeros(kv.decode_prefix_size(b, hq, d, pp), dtype=torch.uint8, device=DEV)
    out = torch.empty((b, hq, d), dtype=tdt, device=DEV)

    def step(tables_, lens_, prefix_pages=pp, pre_bytes=pre.numel(), dtype="bf16"):
        kv.decode_step_cascade(q, kn, vn, qw, kw, 1e-6, c_d, s_d, max_pos, kp.clone(), vp.clone(),
                               to_dev(tables_), to_dev(lens_), out, b, hq, hkv, d, mbps, nb,
                               1.0 / math.sqrt(d), dtype, None, prefix_pages, pre, pre_bytes, ws,
                               ws.numel())
        torch.cuda.synchronize()
        return kv.workspace_flags(ws)

    assert step(tables, lens) == 0
    bad_t = tables.copy()
    bad_t[2, 1] = tables[2, pp]          # a private page inside sequence 2's prefix
    print("cascade contract: prefix tables differ", flush=True)
    assert step(bad_t, lens) == kv.WS_ERR_PREFIX
    bad_l = lens.copy()
    bad_l[1] = 16 * pp                   # the new token at the prefix's last position
    print("cascade contract: new token inside the prefix", flush=True)
    assert step(tables, bad_l) == kv.WS_ERR_PREFIX
    assert step(tables, lens) == 0       # flags cleared by the check, next step clean
    for kwargs in ({"prefix_pages": mbps + 1}, {"prefix_pages": -1},
                   {"pre_bytes": pre.numel() - 16}, {"dtype": "f32"}):
        with pytest.raises(kv.RlseError):
            step(tables, lens, **kwargs)
    # Planned steps: the plan checks the contract once (its verdict word),
    # the step's prefix launch raises the flag from it.
    plan = torch.zeros(kv.decode_plan_size(), dtype=torch.uint8, device=DEV)

    def planned(tables_, lens_):
        t_dev, l_dev = to_dev(tables_), to_dev(lens_)
        kv.decode_plan_cascade(t_dev, l_dev, b, hkv, mbps, nb, pp, plan, plan.numel())
        kv.decode_step_cascade(q, kn, vn, qw, kw, 1e-6, c_d, s_d, max_pos, kp.clone(), vp.clone(),
                               t_dev, l_dev, out, b, hq, hkv, d, mbps, nb, 1.0 / math.sqrt(d),
                               "bf16", plan, pp, pre, pre.numel(), ws, ws.numel())
        torch.cuda.synchronize()
        return kv.workspace_flags(ws)

    print("cascade contract, planned steps", flush=True)
    assert planned(tables, lens) == 0
    assert planned(bad_t, lens) == kv.WS_ERR_PREFIX
    assert planned(tables, bad_l) == kv.WS_ERR_PREFIX
    assert planned(tables, lens) == 0    # a clean plan after a violating one


def _group_batch(rng, groups, n_unforked, hkv, d, seed):
    """A mixed batch: groups = [(members, shared pages)], each member holding
    its group's shared pages then private ones (suffix U[1, 300] + the new
    token), plus n_unforked sequences with private pages only (U[1, 2000]
    keys); batch positions shuffled so members are scattered."""
    spec = [(g, pp) for g, (n, pp) in enumerate(groups) for _ in range(n)]
    spec += [(-1, 0)] * n_unforked
    order = rng.permutation(len(spec))
    spec = [spec[i] for i in order]
    b = len(spec)
    seq_group = np.array([g for g, _ in spec], np.int32)
    lens = np.array([16 * pp + int(rng.integers(1, 301)) + 1 if g >= 0 else
                     int(rng.integers(1, 2001)) for g, pp in spec], np.int32)
    own = np.array([(int(n) + 15) // 16 - pp for n, (_, pp) in zip(lens, spec)])
    nb = sum(pp for _, pp in groups) + int(own.sum()) + 5
    perm = rng.permutation(nb).astype(np.int32)
    used = 0
    shared = []
    for _, pp in groups:
        shared.append(perm[used:used + pp])
        used += pp
    mbps = int(max((int(n) + 15) // 16 for n in lens))
    tables = np.zeros((b, mbps), np.int32)
    for i, (g, pp) in enumerate(spec):
        if g >= 0:
            tables[i, :pp] = shared[g]
        tables[i, pp:pp + own[i]] = perm[used:used + own[i]]
        used += int(own[i])
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    kp = torch.randn((nb, hkv, 16, d), generator=gen, device=DEV).to(BF)
    vp = torch.randn((nb, hkv, 16, d), generator=gen, device=DEV).to(BF)
    return seq_group, lens, tables, nb, mbps, kp, vp, gen


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (14, 2, 64), (32, 8, 128), (8, 8, 64)])
def test_grouped_cascade_mixed_batch_matches_oracle(kv, hq, hkv, d):
    """Three prefix groups (5, 17 and 64 shared pages: one, two and four
    slices) and unforked sequences, members scattered through the batch, in
    one grouped cascade step (rlse_decode_step_groups, streamed pages): every
    row against the oracle over its full key range, the outputs against the
    planned step's (another sum order) and the pool bytes equal to its. Group
    sizes G = 2, 7, 4 and 1: with G = 7 a member's columns straddle the
    16-column tiles, with G = 1 a tile holds 16 members."""
    rng = np.random.default_rng(91 + hq + d)
    groups = [(5, 5), (9, 17), (20, 64)]
    seq_group, lens, tables, nb, mbps, kp, vp, g = _group_batch(rng, groups, 7, hkv, d, 91)
    b = len(lens)
    q, kn, vn, qw, kw, max_pos, c_h, s_h, c_d, s_d = _step_inputs(kv, g, BF, b, hq, hkv, d, mbps,
                                                                  "bf16")
    print(f"grouped cascade: Hq={hq} Hkv={hkv} d={d} B={b}, groups {groups}, 7 unforked, keys "
          f"{int(lens.min())}..{int(lens.max())}", flush=True)
    t_dev, l_dev = to_dev(tables), to_dev(lens)
    sg_dev = to_dev(seq_group)
    gp = np.array([pp for _, pp in groups], np.int32)
    gp_dev = to_dev(gp)
    max_pages = int(gp.max())
    scale = 1.0 / math.sqrt(d)
    ws = torch.zeros(kv.decode_workspace_size(b, hq, hkv, d), dtype=torch.uint8, device=DEV)
    plan = torch.zeros(kv.decode_plan_size(), dtype=torch.uint8, device=DEV)
    pre = torch.zeros(kv.decode_prefix_size(b, hq, d, max_pages), dtype=torch.uint8, device=DEV)
    res = {}
    for name in ("grouped", "grouped_cacheable", "planned"):
        kp_i, vp_i = kp.clone(), vp.clone()
        out = torch.full((b, hq, d), 3.0, dtype=BF, device=DEV)
        args = (q, kn, vn, qw, kw, 1e-6, c_d, s_d, max_pos, kp_i, vp_i, t_dev, l_dev, out, b, hq,
                hkv, d, mbps, nb, scale, "bf16")
        if name == "planned":
            kv.decode_plan(t_dev, l_dev, b, hkv, mbps, nb, plan, plan.numel())
            kv.decode_step_planned(*args, plan, ws, ws.numel())
        else:
            kv.decode_plan_groups(t_dev, l_dev, sg_dev, gp_dev, len(groups), b, hq, hkv, mbps, nb,
                                  plan, plan.numel())
            kv.decode_step_groups(*args, plan, len(groups), max_pages, pre, pre.numel(), ws,
                                  ws.numel(), stream_pages=name == "grouped")
        torch.cuda.synchronize()
        assert kv.workspace_flags(ws) == 0, name
        res[name] = (_host16(out), _host16(kp_i), _host16(vp_i))
    out_g, k_g, v_g = res["grouped"]
    np.testing.assert_array_equal(res["grouped_cacheable"][0], out_g)  # the cache flag: same bits
    np.testing.assert_array_equal(k_g, res["planned"][1])
    np.testing.assert_array_equal(v_g, res["planned"][2])
    mx, rel = err_report(_to_f32(out_g, "bf16"), _to_f32(res["planned"][0], "bf16"))
    print(f"[grouped vs planned] max_abs={mx:.3e} rel={rel:.3e}")
    assert mx <= 1e-2
    got = _to_f32(out_g, "bf16")
    kf, vf = _to_f32(k_g, "bf16"), _to_f32(v_g, "bf16")
    qh, qwh = _host16(q), _host16(qw)
    worst = {}
    for r in range(b):
        n = int(lens[r])
        pos = np.full(hq, n - 1, np.int32)
        q_ref = O.bf16_bits_to_f32(O.apply_rope_bf16(O.rmsnorm_bf16(qh[r], qwh, 1e-6), pos,
                                                      c_h, s_h))
        kc = O.paged_to_contiguous(kf, tables[r], n)
        vc = O.paged_to_contiguous(vf, tables[r], n)
        want = O.decode_batch_f32(q_ref[None], kc[None], vc[None], np.array([n], np.int32), scale)
        mx, _ = err_report(got[r], want[0])
        key = int(seq_group[r])
        worst[key] = max(worst.get(key, 0.0), mx)
        assert np.isfinite(got[r]).all()
        assert mx <= TOL["bf16"], (r, key, mx)
    print("grouped cascade: worst max_abs per group (-1 = unforked): " +
          ", ".join(f"{k}: {v:.3e}" for k, v in sorted(worst.items())))


def test_grouped_cascade_contract_and_plan_stamp(kv):
    """A member whose shared entries differ from its group's, or a group id
    out of range, raises RLSE_WS_ERR_PREFIX; so does a planned launch given a
    plan built for another step shape (a plain plan for a cascade step, a
    cascade plan of another prefix, a grouped plan of another group size).
    The next correct step is clean."""
    hq, hkv, d = 16, 8, 128
    rng = np.random.default_rng(93)
    groups = [(3, 4), (4, 9)]
    seq_group, lens, tables, nb, mbps, kp, vp, g = _group_batch(rng, groups, 2, hkv, d, 93)
    b = len(lens)
    q, kn, vn, qw, kw, max_pos, _, _, c_d, s_d = _step_inputs(kv, g, BF, b, hq, hkv, d, mbps,
                                                              "bf16")
    ws = torch.zeros(kv.decode_workspace_size(b, hq, hkv, d), dtype=torch.uint8, device=DEV)
    plan = torch.zeros(kv.decode_plan_size(), dtype=torch.uint8, device=DEV)
    pre = torch.zeros(kv.decode_prefix_size(b, hq, d, 9), dtype=torch.uint8, device=DEV)
    out = torch.empty((b, hq, d), dtype=BF, device=DEV)
    gp = to_dev(np.array([4, 9], np.int32))

    def grouped(tables_, sg):
        t_dev, l_dev = to_dev(tables_), to_dev(lens)
        kv.decode_plan_groups(t_dev, l_dev, to_dev(sg), gp, 2, b, hq, hkv, mbps, nb, plan,
                              plan.numel())
        kv.decode_step_groups(q, kn, vn, qw, kw, 1e-6, c_d, s_d, max_pos, kp.clone(), vp.clone(),
                              t_dev, l_dev, out, b, hq, hkv, d, mbps, nb, 1.0 / math.sqrt(d),
                              "bf16", plan, 2, 9, pre, pre.numel(), ws, ws.numel())
        torch.cuda.synchronize()
        return kv.workspace_flags(ws)

    assert grouped(tables, seq_group) == 0
    m = int(np.flatnonzero(seq_group == 1)[1])
    bad_t = tables.copy()
    bad_t[m, 2] = tables[m, 9]                   # a private page inside group 1's shared range
    print("grouped contract: member's shared entries differ", flush=True)
    assert grouped(bad_t, seq_group) == kv.WS_ERR_PREFIX
    bad_g = seq_group.copy()
    bad_g[0] = 5                                 # no group 5
    print("grouped contract: group id out of range", flush=True)
    assert grouped(tables, bad_g) == kv.WS_ERR_PREFIX
    assert grouped(tables, seq_group) == 0
    # a plan of another step shape
    t_dev, l_dev = to_dev(tables), to_dev(lens)
    fork_t = tables.copy()
    fork_t[:, :2] = tables[0, :2]                # two pages shared by the whole batch
    ft_dev = to_dev(fork_t)
    pre2 = torch.zeros(kv.decode_prefix_size(b, hq, d, 2), dtype=torch.uint8, device=DEV)
    for plan_prefix, step_prefix in ((0, 2), (1, 2)):
        print(f"plan stamp: plan for prefix {plan_prefix}, cascade step of prefix {step_prefix}",
              flush=True)
        kv.decode_plan_cascade(ft_dev, l_dev, b, hkv, mbps, nb, plan_prefix, plan, plan.numel())
        kv.decode_step_cascade(q, kn, vn, qw, kw, 1e-6, c_d, s_d, max_pos, kp.clone(), vp.clone(),
                               ft_dev, l_dev, out, b, hq, hkv, d, mbps, nb, 1.0 / math.sqrt(d),
                               "bf16", plan, step_prefix, pre2, pre2.numel(), ws, ws.numel())
        torch.cuda.synchronize()
        assert kv.workspace_flags(ws) == kv.WS_ERR_PREFIX
    print("plan stamp: grouped plan for a plain planned step", flush=True)
    kv.decode_plan_groups(t_dev, l_dev, to_dev(seq_group), gp, 2, b, hq, hkv, mbps, nb, plan,
                          plan.numel())
    kv.decode_step_planned(q, kn, vn, qw, kw, 1e-6, c_d, s_d, max_pos, kp.clone(), vp.clone(),
                           t_dev, l_dev, out, b, hq, hkv, d, mbps, nb, 1.0 / math.sqrt(d), "bf16",
                           plan, ws, ws.numel())
    torch.cuda.synchronize()
    assert kv.workspace_flags(ws) == kv.WS_ERR_PREFIX
    assert grouped(tables, seq_group) == 0
    print("plan stamp: grouped plan of group size 1 for a step of group size 2", flush=True)
    kv.decode_plan_groups(t_dev, l_dev, to_dev(seq_group), gp, 2, b, hkv, hkv, mbps, nb, plan,
                          plan.numel())
    kv.decode_step_groups(q, kn, vn, qw, kw, 1e-6, c_d, s_d, max_pos, kp.clone(), vp.clone(),
                          t_dev, l_dev, out, b, hq, hkv, d, mbps, nb, 1.0 / math.sqrt(d), "bf16",
                          plan, 2, 9, pre, pre.numel(), ws, ws.numel())
    torch.cuda.synchronize()
    assert kv.workspace_flags(ws) == kv.WS_ERR_PREFIX
    assert grouped(tables, seq_group) == 0
    for kwargs in ({"num_groups": 0}, {"num_groups": 65}, {"max_group_pages": 0},
                   {"max_group_pages": mbps + 1}, {"dtype": "f32"}):
        a = dict(num_groups=2, max_group_pages=9, dtype="bf16")
        a.update(kwargs)
        with pytest.raises(kv.RlseError):
            kv.decode_step_groups(q, kn, vn, qw, kw, 1e-6, c_d, s_d, max_pos, kp.clone(),
                                  vp.clone(), t_dev, l_dev, out, b, hq, hkv, d, mbps, nb,
                                  1.0 / math.sqrt(d), a["dtype"], plan, a["num_groups"],
                                  a["max_group_pages"], pre, pre.numel(), ws, ws.numel())
