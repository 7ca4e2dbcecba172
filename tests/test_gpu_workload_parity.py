"""The benched workloads at their own inputs, against the oracle.

The bench times three paths that the other GPU tests reach only at other
sizes; here each runs on exactly the inputs the bench builds (bench.py's
decode_inputs / fork_inputs, default seed 2) or at the benched model shape:

* the planned step with streamed pages (rlse_decode_step_planned with
  RLSE_DECODE_STREAM) -- the default bench line -- on the Qwen3-0.6B batch
  (B=32, cached U[128,2048] + 1) and the Qwen2.5-0.5B batch (B=64, 4096 + 1),
  every row and head against the oracle's Candle op chain (RmsNorm where the
  model has q/k norms, apply_rope, KvCache append, zero-copy GQA decode;
  src/backends/qwen2.rs:177-203, 291-328), and the appended K/V rows bit for
  bit;
* the cascade step (rlse_decode_step_cascade, streamed) on the 1030-token
  prefix fork: 64 sequences sharing 64 full pages, each holding its own
  copy-on-write copy of the partial page and U[64,512] private suffix tokens
  (src/cache/prefix_cache.rs:250-345, src/backends/candle.rs:437-478), rows
  against the oracle over each sequence's full key range, the pool bytes
  against the planned step's and the shared prefix unchanged;
* one DecodeModel.step (step_decode_batch, src/backends/qwen2.rs:628-764) at
  the Qwen3-0.6B and Qwen2.5-0.5B configurations (28/24 layers, vocab
  151936), logits of every row against the oracle's model_step_ref.

Bars: max-abs 2e-2 for bf16 attention outputs; logits relative 2e-2 (max-abs
over max |reference|); the appended rows and the pool bit-exact.
"""
import math
import os
import sys

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import DEV, TOL, err_report, to_dev

pytestmark = pytest.mark.gpu

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402  (the bench's own input builders)

BF = torch.bfloat16
BENCH_SEED = 2   # bench.py's default --seed


def _host16(t):
    torch.cuda.synchronize()
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _q_ref(q_bits, qw_bits, pos, c_h, s_h):
    """Candle's q chain for one sequence [Hq, d]: RmsNorm (when the model
    has q_norm), then apply_rope at position pos, bf16 rounding per op."""
    qn = q_bits if qw_bits is None else O.rmsnorm_bf16(q_bits, qw_bits, 1e-6)
    return O.apply_rope_bf16(qn, np.full(q_bits.shape[0], pos, np.int32), c_h, s_h)


def _gather(kv, k_ptr, v_ptr, table_row, n, hkv, d, nb):
    """Sequence's K and V over its first n positions, [Hkv, n, d] bf16 bits."""
    ko = torch.empty((1, hkv, n, d), dtype=BF, device=DEV)
    vo = torch.empty_like(ko)
    kv.kv_gather(k_ptr, v_ptr, 0, 1, table_row, n, ko, vo, hkv, d, nb, "bf16")
    return _host16(ko)[0], _host16(vo)[0]


@pytest.mark.parametrize("workload", ["qwen3", "qwen25", "qwen25_7b"])
def test_bench_planned_stream_step_matches_oracle(kv, workload):
    hq, hkv, d, _, b, _, _, _ = bench.WORKLOADS[workload]
    w = bench.decode_inputs(workload, BENCH_SEED, DEV, layers=1)
    lens, tables, mbps, nb = w["lens"], w["tables"], w["mbps"], w["num_blocks"]
    print(f"{workload}: B={b}, keys {int(lens.min())}..{int(lens.max())}, {w['pages']} pages, "
          f"q/k norm {w['q_norm'][0] is not None}", flush=True)
    c_h = np.frombuffer(w["cos_bytes"], np.uint16).reshape(w["max_pos"], d // 2)
    s_h = np.frombuffer(w["sin_bytes"], np.uint16).reshape(w["max_pos"], d // 2)
    t_dev, l_dev = to_dev(tables), to_dev(lens)
    kp, vp = w["k_pools"][0], w["v_pools"][0]
    kp0, vp0 = _host16(kp), _host16(vp)          # the pool before the step
    out = torch.full((b, hq, d), 3.0, dtype=BF, device=DEV)
    ws = torch.zeros(kv.decode_workspace_size(b, hq, hkv, d), dtype=torch.uint8, device=DEV)
    plan = torch.zeros(kv.decode_plan_size(), dtype=torch.uint8, device=DEV)
    scale = 1.0 / math.sqrt(d)
    kv.decode_plan(t_dev, l_dev, b, hkv, mbps, nb, plan, plan.numel())
    kv.decode_step_planned(w["q"][0], w["k_new"][0], w["v_new"][0], w["q_norm"][0],
                           w["k_norm"][0], 1e-6, w["cos"], w["sin"], w["max_pos"], kp, vp, t_dev,
                           l_dev, out, b, hq, hkv, d, mbps, nb, scale, "bf16", plan, ws,
                           ws.numel(), stream_pages=True)
    torch.cuda.synchronize()
    assert kv.workspace_flags(ws) == 0
    got = O.bf16_bits_to_f32(_host16(out))
    kp1, vp1 = _host16(kp), _host16(vp)
    qh, knh, vnh = _host16(w["q"][0]), _host16(w["k_new"][0]), _host16(w["v_new"][0])
    qwh = None if w["q_norm"][0] is None else _host16(w["q_norm"][0])
    kwh = None if w["k_norm"][0] is None else _host16(w["k_norm"][0])
    # The pool changed exactly at each sequence's new position: k_norm + RoPE
    # of the new k, the raw new v.
    changed = np.zeros(kp0.shape[:1] + kp0.shape[2:3], bool)   # [block, slot]
    for i in range(b):
        pos = int(lens[i]) - 1
        blk, slot = int(tables[i, pos // 16]), pos % 16
        want_k = _q_ref(knh[i], kwh, pos, c_h, s_h)
        np.testing.assert_array_equal(kp1[blk, :, slot], want_k, err_msg=f"k row {i}")
        np.testing.assert_array_equal(vp1[blk, :, slot], vnh[i], err_msg=f"v row {i}")
        changed[blk, slot] = True
    np.testing.assert_array_equal(kp1[~changed[:, None, :].repeat(hkv, 1)],
                                  kp0[~changed[:, None, :].repeat(hkv, 1)])
    np.testing.assert_array_equal(vp1[~changed[:, None, :].repeat(hkv, 1)],
                                  vp0[~changed[:, None, :].repeat(hkv, 1)])
    del kp0, vp0
    # every row and head against the oracle on the appended pool
    q_ref = np.stack([O.bf16_bits_to_f32(_q_ref(qh[i], qwh, int(lens[i]) - 1, c_h, s_h))
                      for i in range(b)])
    want = O.decode_paged_f32(q_ref, O.bf16_bits_to_f32(kp1), O.bf16_bits_to_f32(vp1), tables,
                              lens, scale)
    mx, rel = err_report(got, want)
    print(f"{workload} planned stream step: all {b} rows x {hq} heads max_abs={mx:.3e} "
          f"rel={rel:.3e} (bar {TOL['bf16']})")
    assert np.isfinite(got).all()
    assert mx <= TOL["bf16"]


def test_cascade_step_fork1030_bench_inputs_match_oracle(kv):
    workload = "qwen3_fork1030"
    hq, hkv, d, _, b, plen, _, _, _ = bench.FORK[workload]
    f = bench.fork_inputs(workload, BENCH_SEED, DEV, layers=1)
    lens, tables, mbps, nb = f["lens"], f["tables"], f["mbps"], f["num_blocks"]
    shared = plen // 16
    assert len(f["cow_pairs"]) == b              # each sequence copied the partial page
    assert (tables[:, :shared] == tables[0, :shared]).all()
    assert len(set(tables[:, shared].tolist())) == b   # the copies are private
    print(f"fork1030: B={b}, {shared} shared pages, keys {int(lens.min())}..{int(lens.max())}",
          flush=True)
    k_ptr, v_ptr = f["pool"].layer(0)
    c_h = np.frombuffer(f["cos_bytes"], np.uint16).reshape(f["max_pos"], d // 2)
    s_h = np.frombuffer(f["sin_bytes"], np.uint16).reshape(f["max_pos"], d // 2)
    t_dev, l_dev = f["tables_dev"], to_dev(lens.astype(np.int32))
    pk0, pv0 = _gather(kv, k_ptr, v_ptr, f["prefix_table"], plen, hkv, d, nb)
    scale = 1.0 / math.sqrt(d)
    ws = torch.zeros(kv.decode_workspace_size(b, hq, hkv, d), dtype=torch.uint8, device=DEV)
    plan = torch.zeros(kv.decode_plan_size(), dtype=torch.uint8, device=DEV)
    pre = torch.zeros(kv.decode_prefix_size(b, hq, d, shared), dtype=torch.uint8, device=DEV)
    args = (f["q"][0], f["k_new"][0], f["v_new"][0], f["q_norm"], f["k_norm"], 1e-6, f["cos"],
            f["sin"], f["max_pos"], k_ptr, v_ptr, t_dev, l_dev)
    outs, seqs = {}, {}
    # the cascade step the bench times, then the planned step over the same
    # inputs (its append rewrites the same bits) for the pool comparison
    for name in ("cascade", "planned"):
        out = torch.full((b, hq, d), 3.0, dtype=BF, device=DEV)
        if name == "cascade":
            kv.decode_plan_cascade(t_dev, l_dev, b, hkv, mbps, nb, shared, plan, plan.numel())
            kv.decode_step_cascade(*args, out, b, hq, hkv, d, mbps, nb, scale, "bf16", plan,
                                   shared, pre, pre.numel(), ws, ws.numel(), stream_pages=True)
        else:
            kv.decode_plan(t_dev, l_dev, b, hkv, mbps, nb, plan, plan.numel())
            kv.decode_step_planned(*args, out, b, hq, hkv, d, mbps, nb, scale, "bf16", plan, ws,
                                   ws.numel())
        torch.cuda.synchronize()
        assert kv.workspace_flags(ws) == 0, name
        outs[name] = O.bf16_bits_to_f32(_host16(out))
        seqs[name] = [_gather(kv, k_ptr, v_ptr, t_dev[i], int(lens[i]), hkv, d, nb)
                      for i in range(b)]
    for i in range(b):       # one pool: both steps appended the same bytes
        np.testing.assert_array_equal(seqs["cascade"][i][0], seqs["planned"][i][0], err_msg=i)
        np.testing.assert_array_equal(seqs["cascade"][i][1], seqs["planned"][i][1], err_msg=i)
    mx, rel = err_report(outs["cascade"], outs["planned"])
    print(f"fork1030 cascade vs planned: max_abs={mx:.3e} rel={rel:.3e}")
    assert mx <= 1e-2
    # the shared prefix is unchanged; every appended row is the oracle's
    pk1, pv1 = _gather(kv, k_ptr, v_ptr, f["prefix_table"], plen, hkv, d, nb)
    np.testing.assert_array_equal(pk1, pk0)
    np.testing.assert_array_equal(pv1, pv0)
    qh, knh, vnh = _host16(f["q"][0]), _host16(f["k_new"][0]), _host16(f["v_new"][0])
    qwh, kwh = _host16(f["q_norm"]), _host16(f["k_norm"])
    for i in range(b):
        pos = int(lens[i]) - 1
        k_i, v_i = seqs["cascade"][i]
        np.testing.assert_array_equal(k_i[:, pos], _q_ref(knh[i], kwh, pos, c_h, s_h), err_msg=i)
        np.testing.assert_array_equal(v_i[:, pos], vnh[i], err_msg=i)
        np.testing.assert_array_equal(k_i[:, :plen], pk0, err_msg=i)   # prefix || suffix
    # rows against the oracle over the full key range (prefix, copied page, suffix)
    rng = np.random.default_rng(11)
    rows = sorted(set([0, b - 1, int(np.argmax(lens)), int(np.argmin(lens))] +
                      [int(x) for x in rng.choice(b, 8, replace=False)]))
    worst = 0.0
    for r in rows:
        n = int(lens[r])
        q_ref = O.bf16_bits_to_f32(_q_ref(qh[r], qwh, n - 1, c_h, s_h))
        k_i, v_i = seqs["cascade"][r]
        want = O.decode_batch_f32(q_ref[None], O.bf16_bits_to_f32(k_i)[None],
                                  O.bf16_bits_to_f32(v_i)[None], np.array([n], np.int32), scale)
        mx, rel = err_report(outs["cascade"][r], want[0])
        worst = max(worst, mx)
        assert np.isfinite(outs["cascade"][r]).all()
        assert mx <= TOL["bf16"], (r, mx)
    print(f"fork1030 cascade: {len(rows)} rows x {hq} heads within {worst:.3e} of the oracle "
          f"(bar {TOL['bf16']})")
    f["pool"].close()


@pytest.mark.timeout(900)
@pytest.mark.parametrize("factory", ["qwen3_0_6b", "qwen2_5_0_5b"])
def test_decode_model_step_at_model_shape_matches_oracle(kv, factory):
    from decode_model import DecodeModel, ModelConfig
    cfg = getattr(ModelConfig, factory)()
    spec = O.ModelSpec(cfg.hidden, cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.inter,
                       cfg.vocab, cfg.eps, cfg.theta, cfg.qk_norm, cfg.qkv_bias, cfg.tied)
    dt = "bf16"
    rng = np.random.default_rng(17)
    print(f"{factory}: drawing weights (hidden {cfg.hidden}, {cfg.layers} layers, vocab "
          f"{cfg.vocab})", flush=True)
    w = O.random_weights(spec, rng, dt)
    ctx = [0, 37, 300, 1100]               # cached tokens per sequence
    b, steps = len(ctx), 2
    mbps = max((n + steps + 15) // 16 for n in ctx) + 1
    nb = b * mbps + 5
    tables = np.zeros((b, mbps), np.int32)
    perm = rng.permutation(nb).astype(np.int32)
    for i in range(b):
        tables[i] = perm[i * mbps:(i + 1) * mbps]
    model = DecodeModel(cfg, w, dt, nb, b, mbps, DEV, stream_pages=True)
    t_dev = torch.from_numpy(tables).to(DEV)
    kc = [[None] * b for _ in range(spec.layers)]
    vc = [[None] * b for _ in range(spec.layers)]
    for i, n in enumerate(ctx):   # cached context: N(0,1) K/V, the same in pool and oracle
        k = O.round_to(rng.standard_normal((spec.layers, spec.kv_heads, n, spec.head_dim)), dt)
        v = O.round_to(rng.standard_normal((spec.layers, spec.kv_heads, n, spec.head_dim)), dt)
        if n:
            model.set_kv(t_dev[i], k, v)
        for layer in range(spec.layers):
            kc[layer][i], vc[layer][i] = k[layer], v[layer]
    cos_t, sin_t = O.rope_tables_f32(spec.theta, spec.head_dim, model.max_pos)
    cos_t, sin_t = O.round_to(cos_t, dt), O.round_to(sin_t, dt)
    ids = np.array(rng.integers(0, spec.vocab, b), np.int32)
    lens = np.array(ctx, np.int32)
    for step in range(steps):
        lens = lens + 1
        print(f"{factory}: step {step}", flush=True)
        logits, nxt = model.step(torch.from_numpy(ids).to(DEV), t_dev,
                                 torch.from_numpy(lens).to(DEV), b)
        torch.cuda.synchronize()
        got = logits.float().cpu().numpy()
        want = O.model_step_ref(spec, w, list(ids), kc, vc, cos_t, sin_t, dt)
        for r in range(b):
            mx, rel = err_report(got[r], want[r])
            print(f"[{factory} step {step} row {r} (cached {ctx[r] + step})] logits "
                  f"max_abs={mx:.3e} rel={rel:.3e}")
            assert np.isfinite(got[r]).all()
            assert rel <= TOL[dt], (step, r, mx, rel)
        g = nxt.cpu().numpy()
        np.testing.assert_array_equal(g, O.argmax_ref(got))
        ids = g.astype(np.int32)     # teacher-forced into the oracle too
    model.close()


def test_grouped_cascade_mixed_bench_inputs_match_oracle(kv):
    """The mixed-batch bench's inputs (bench.py mixed_inputs, one layer):
    sequences forked from 1024-, 512- and 2048-token prefixes and unforked
    ones, scattered through the batch, in one grouped cascade step
    (rlse_decode_step_groups, streamed): rows of every group and unforked
    rows against the oracle over their full key range, outputs against the
    planned step's, the pool bytes equal to its."""
    workload = "qwen3_mixed"
    hq, hkv, d, _, groups, _, _, _, _, _, _ = bench.MIXED[workload]
    f = bench.mixed_inputs(workload, BENCH_SEED, DEV, layers=1)
    lens, tables, mbps, nb = f["lens"], f["tables"], f["mbps"], f["num_blocks"]
    sg, gp = f["seq_group"], f["group_pages"]
    b = len(lens)
    for g in range(len(groups)):   # members share their group's pages
        rows = np.flatnonzero(sg == g)
        assert (tables[rows, :gp[g]] == tables[rows[0], :gp[g]]).all()
    print(f"mixed: B={b}, groups {groups}, keys {int(lens.min())}..{int(lens.max())}", flush=True)
    k_ptr, v_ptr = f["pool"].layer(0)
    c_h = np.frombuffer(f["cos_bytes"], np.uint16).reshape(f["max_pos"], d // 2)
    s_h = np.frombuffer(f["sin_bytes"], np.uint16).reshape(f["max_pos"], d // 2)
    t_dev, l_dev = f["tables_dev"], to_dev(lens)
    scale = 1.0 / math.sqrt(d)
    ws = torch.zeros(kv.decode_workspace_size(b, hq, hkv, d), dtype=torch.uint8, device=DEV)
    plan = torch.zeros(kv.decode_plan_size(), dtype=torch.uint8, device=DEV)
    pre = torch.zeros(kv.decode_prefix_size(b, hq, d, int(gp.max())), dtype=torch.uint8,
                      device=DEV)
    args = (f["q"][0], f["k_new"][0], f["v_new"][0], f["q_norm"], f["k_norm"], 1e-6, f["cos"],
            f["sin"], f["max_pos"], k_ptr, v_ptr, t_dev, l_dev)
    outs, seqs = {}, {}
    for name in ("grouped", "planned"):
        out = torch.full((b, hq, d), 3.0, dtype=BF, device=DEV)
        if name == "grouped":
            kv.decode_plan_groups(t_dev, l_dev, to_dev(sg), to_dev(gp), len(groups), b, hq, hkv,
                                  mbps, nb, plan, plan.numel())
            kv.decode_step_groups(*args, out, b, hq, hkv, d, mbps, nb, scale, "bf16", plan,
                                  len(groups), int(gp.max()), pre, pre.numel(), ws, ws.numel(),
                                  stream_pages=True)
        else:
            kv.decode_plan(t_dev, l_dev, b, hkv, mbps, nb, plan, plan.numel())
            kv.decode_step_planned(*args, out, b, hq, hkv, d, mbps, nb, scale, "bf16", plan, ws,
                                   ws.numel())
        torch.cuda.synchronize()
        assert kv.workspace_flags(ws) == 0, name
        outs[name] = O.bf16_bits_to_f32(_host16(out))
        seqs[name] = [_gather(kv, k_ptr, v_ptr, t_dev[i], int(lens[i]), hkv, d, nb)
                      for i in range(b)]
    for i in range(b):
        np.testing.assert_array_equal(seqs["grouped"][i][0], seqs["planned"][i][0], err_msg=i)
        np.testing.assert_array_equal(seqs["grouped"][i][1], seqs["planned"][i][1], err_msg=i)
    mx, rel = err_report(outs["grouped"], outs["planned"])
    print(f"mixed grouped vs planned: max_abs={mx:.3e} rel={rel:.3e}")
    assert mx <= 1e-2
    qh, qwh = _host16(f["q"][0]), _host16(f["q_norm"])
    rng = np.random.default_rng(13)
    rows = []
    for g in list(range(len(groups))) + [-1]:   # three rows of every group and unforked
        rows += [int(x) for x in rng.choice(np.flatnonzero(sg == g), 3, replace=False)]
    worst = 0.0
    for r in rows:
        n = int(lens[r])
        q_ref = O.bf16_bits_to_f32(_q_ref(qh[r], qwh, n - 1, c_h, s_h))
        k_i, v_i = seqs["grouped"][r]
        want = O.decode_batch_f32(q_ref[None], O.bf16_bits_to_f32(k_i)[None],
                                  O.bf16_bits_to_f32(v_i)[None], np.array([n], np.int32), scale)
        mx, _ = err_report(outs["grouped"][r], want[0])
        worst = max(worst, mx)
        assert np.isfinite(outs["grouped"][r]).all()
        assert mx <= TOL["bf16"], (r, int(sg[r]), mx)
    print(f"mixed grouped: {len(rows)} rows (3 per group and unforked) x {hq} heads within "
          f"{worst:.3e} of the oracle (bar {TOL['bf16']})")
    f["pool"].close()
