"""The rest of the decode step on the GPU against the oracle.

Reference: ModelForCausalLM::step_decode_batch (src/backends/qwen2.rs:628-764)
and the greedy branch of sample_token (src/backends/candle.rs:737-751). Each
device op (rlse_embedding, rlse_add_rmsnorm, rlse_silu_mul, rlse_linear,
rlse_argmax) is checked against its oracle restatement
(oracle/oracle.py ``*_ref``, pinned in test_oracle_model.py), then whole
steps of small Qwen3- and Qwen2-style decoders run through DecodeModel
against model_step_ref.

Bars: embedding, argmax and the residual sums bit-exact; the normalised and
activated values within a few units in the last place of the dtype, as
bounded at each test (the sum of squares runs in another order and exp comes
from another math library); linear and whole-step outputs max-abs 2e-3 (f32)
and 2e-2 (bf16/f16) relative to the largest reference magnitude, the
relative error printed beside the max-abs one.
"""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import DEV, TOL, build_tables, err_report

pytestmark = pytest.mark.gpu

_T = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
ULP = {"f32": 2.0 ** -23, "bf16": 2.0 ** -7, "f16": 2.0 ** -10}


def dev(a, dt):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV).to(_T[dt])


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def rel_check(name, got, want, dt, bar=None):
    mx, rel = err_report(got, want)
    print(f"[{name}] dtype={dt} max_abs={mx:.3e} rel={rel:.3e}")
    assert np.isfinite(got).all()
    assert rel <= (TOL[dt] if bar is None else bar), (name, mx, rel)


@pytest.mark.parametrize("dt", O.DTYPES)
def test_embedding_rows_bit_exact(kv, dt):
    rng = np.random.default_rng(1)
    table = O.round_to(rng.standard_normal((300, 128)), dt)
    ids = np.array([5, 0, 299, -1, 300, 17, 17], np.int32)
    out = torch.full((len(ids), 128), 7.0, dtype=_T[dt], device=DEV)
    kv.embedding(torch.from_numpy(ids).to(DEV), dev(table, dt), out, len(ids), 128, 300, dt)
    np.testing.assert_array_equal(host(out), O.embedding_ref(ids, table))


@pytest.mark.parametrize("dt", O.DTYPES)
@pytest.mark.parametrize("rows,n", [(1, 64), (7, 896), (33, 1024), (5, 4096)])
def test_add_rmsnorm_matches_oracle(kv, dt, rows, n):
    rng = np.random.default_rng(rows * n)
    x = O.round_to(rng.standard_normal((rows, n)), dt)
    r = O.round_to(2 * rng.standard_normal((rows, n)), dt)
    w = O.round_to(1 + 0.1 * rng.standard_normal(n), dt)
    xd, rd, out = dev(x, dt), dev(r, dt), torch.empty((rows, n), dtype=_T[dt], device=DEV)
    kv.add_rmsnorm(xd, rd, dev(w, dt), out, rows, n, 1e-6, dt)
    h_want, o_want = O.add_rmsnorm_ref(x, r, w, 1e-6, dt)
    np.testing.assert_array_equal(host(rd), h_want)           # the rounded sum: exact
    got = host(out)
    # The sum of squares runs in another order: its f32 relative error is at
    # most n * 2^-24, the norm's half that; then two roundings to the dtype
    # (x / norm, then * w) can each move an output by one ulp.
    bound = (n * 2.0 ** -25 + 2 * ULP[dt]) * np.abs(o_want).max()
    mx, rel = err_report(got, o_want)
    print(f"[add_rmsnorm {rows}x{n}] dtype={dt} max_abs={mx:.3e} rel={rel:.3e}")
    assert mx <= bound, (mx, bound)


@pytest.mark.parametrize("dt", O.DTYPES)
def test_silu_mul_matches_oracle(kv, dt):
    rng = np.random.default_rng(3)
    rows, inter = 9, 3072
    gu = O.round_to(4 * rng.standard_normal((rows, 2 * inter)), dt)
    gu[0, :8] = [0, -0.0, 30, -30, 88, -88, 11, -11.5]        # exp overflow edges
    out = torch.empty((rows, inter), dtype=_T[dt], device=DEV)
    kv.silu_mul(dev(gu, dt), out, rows, inter, dt)
    want = O.silu_mul_ref(gu[:, :inter], gu[:, inter:], dt)
    got = host(out)
    diff = np.abs(got.astype(np.float64) - want)
    # exp differs between math libraries by up to about two ulps in f32 and
    # three roundings follow it: four f32 ulps; in bf16/f16 the f32
    # differences can only flip a rounding, by one ulp at each of the steps.
    ulps = 4 if dt == "f32" else 2
    scaled = diff / (ULP[dt] * np.maximum(np.abs(want), 2.0 ** -14))
    worst = np.unravel_index(np.argmax(scaled), scaled.shape)
    print(f"[silu_mul] dtype={dt} max_abs={diff.max():.3e} max_ulps={scaled.max():.2f} "
          f"mismatches={(got != want).sum()}/{got.size} worst: gate={gu[worst]!r} "
          f"up={gu[worst[0], inter + worst[1]]!r} got={got[worst]!r} want={want[worst]!r}")
    assert scaled.max() <= ulps


@pytest.mark.parametrize("dt", O.DTYPES)
@pytest.mark.parametrize("rows,n_out,n_in,bias", [(1, 2048, 1024, False), (32, 3072, 1024, True),
                                                  (33, 896, 4864, False), (64, 1000, 128, True),
                                                  (40, 8192, 256, True),    # two tiles per group
                                                  (17, 64, 48, True)])      # f32: three 16-wide k steps
def test_linear_matches_oracle(kv, dt, rows, n_out, n_in, bias):
    """Decode-shaped products run on the MFMA kernel: bf16/f16 with in % 32,
    f32 (16-element k steps on f32 MFMAs) with in % 16, outputs a multiple of
    16; others (1000 outputs, 48 inputs at 16 bits) go to the library GEMM."""
    rng = np.random.default_rng(rows + n_out)
    x = O.round_to(rng.standard_normal((rows, n_in)), dt)
    w = O.round_to(rng.standard_normal((n_out, n_in)) / np.sqrt(n_in), dt)
    b = O.round_to(rng.standard_normal(n_out), dt) if bias else None
    y = torch.empty((rows, n_out), dtype=_T[dt], device=DEV)
    kv.linear(dev(x, dt), dev(w, dt), None if b is None else dev(b, dt), y, rows, n_out, n_in,
              dt)
    rel_check(f"linear {rows}x{n_out}x{n_in} bias={bias}", host(y), O.linear_ref(x, w, b, dt),
              dt)


@pytest.mark.parametrize("dt", O.DTYPES)
def test_argmax_bit_exact_with_ties_and_nans(kv, dt):
    rng = np.random.default_rng(4)
    vocab = 151936
    rows = O.round_to(rng.standard_normal((12, vocab)), dt)
    rows[1, 1000] = rows[1, 90000] = 50.0                # tie: first index
    rows[2, 0] = np.nan                                  # NaN at 0 wins outright
    rows[3, 5] = np.nan
    rows[3, 77] = 60.0                                   # later NaN never taken
    rows[4] = -np.inf                                    # all -inf: index 0
    rows[5, :] = np.nan
    rows[5, 9] = -np.inf                                 # NaN at 0 again
    rows[6, vocab - 1] = 70.0                            # maximum at the end
    rows[7, 3:] = -np.inf
    rows[7, :3] = [-np.inf, 2.0, 2.0]
    rows[8, 100] = -0.0
    rows[8, 200] = 0.0
    rows[8, :100] = -1.0
    rows[8, 101:] = -1.0
    rows[8, 200] = 0.0                                   # -0 then +0: the first (scan: equal)
    out = torch.full((12,), -5, dtype=torch.int32, device=DEV)
    nbytes = kv.argmax_workspace_size(12, vocab)
    ws = torch.full((nbytes,), 0xAB, dtype=torch.uint8, device=DEV)   # needs no clearing
    kv.argmax(dev(rows, dt), out, 12, vocab, dt, ws, nbytes)
    torch.cuda.synchronize()
    want = O.argmax_ref(rows)
    np.testing.assert_array_equal(out.cpu().numpy(), want)
    assert want[1] == 1000 and want[2] == 0 and want[3] == 77 and want[4] == 0 and \
        want[6] == vocab - 1 and want[7] == 1 and want[8] == 100
    with pytest.raises(kv.RlseError):
        kv.argmax(dev(rows, dt), out, 12, vocab, dt, ws, nbytes - 8)


@pytest.mark.parametrize("vocab", [1, 4095, 4096, 4097, 9000])
def test_argmax_chunk_edges(kv, vocab):
    rng = np.random.default_rng(vocab)
    rows = O.round_to(rng.standard_normal((5, vocab)), "bf16")
    rows[1, vocab - 1] = 9.0
    rows[2, min(4095, vocab - 1)] = 9.0
    rows[3, :] = 1.0
    out = torch.empty(5, dtype=torch.int32, device=DEV)
    nbytes = kv.argmax_workspace_size(5, vocab)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    kv.argmax(dev(rows, "bf16"), out, 5, vocab, "bf16", ws, nbytes)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), O.argmax_ref(rows))


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_argmax_packet_paths_agree(kv, dt):
    """16-bit rows of whole 16-byte packets take the packet-load path; the
    same rows one element into the buffer (not 16-byte aligned) take the
    element path. Both give the scan's answer: ties inside one packet and
    across the lanes of one chunk go to the first index."""
    rng = np.random.default_rng(6)
    vocab, n = 8192, 4
    rows = O.round_to(rng.standard_normal((n, vocab)), dt)
    rows[0, 8 * 37 + 5] = rows[0, 8 * 37 + 2] = 30.0      # tie inside one packet
    rows[1, 8 * 300 + 1] = rows[1, 8 * 12 + 7] = 30.0     # tie across lanes, first is later
    rows[2, 4096 + 3] = rows[2, 4095] = 30.0              # tie across the chunk edge
    rows[3, 7] = np.nan
    rows[3, 8 * 500] = 30.0                               # NaN after index 0: skipped
    want = O.argmax_ref(rows)
    assert list(want) == [8 * 37 + 2, 8 * 12 + 7, 4095, 8 * 500]
    nbytes = kv.argmax_workspace_size(n, vocab)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    flat = torch.empty(n * vocab + 8, dtype=_T[dt], device=DEV)
    for off in (0, 1):                                    # aligned, then misaligned
        view = flat[off:off + n * vocab].view(n, vocab)
        view.copy_(dev(rows, dt))
        out = torch.full((n,), -1, dtype=torch.int32, device=DEV)
        kv.argmax(view, out, n, vocab, dt, ws, nbytes)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), want)


# ------------------------------------------------ fused MFMA projections ---
ROWS = [1, 5, 16, 33, 64, 100]


def _dense_ws(kv, rows, n_out, n_in, use):
    """The K-split workspace (zero-filled, as the contract asks), or None."""
    if not use:
        return None
    n = kv.dense_workspace_size(rows, n_out, n_in)
    return torch.zeros(max(n, 4), dtype=torch.uint8, device=DEV)


def _assert_clean(ws):
    """No device error flag raised; the launch counters all equal (every
    K-split launch advances each of them once)."""
    if ws is not None and ws.numel() > 4:
        import rlse_kv
        assert rlse_kv.workspace_flags(ws) == 0
        ctr = ws.view(torch.int32)[64:64 + DENSE_CTR].cpu().numpy()
        assert (ctr == ctr[0]).all()


DENSE_CTR = 2048   # launch counters of a K-split workspace (512 workgroups x 4 waves)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("hidden,nq,nkv,bias", [(1024, 2048, 1024, False), (896, 896, 128, True),
                                               (256, 512, 128, False)])
def test_qkv_proj_matches_three_linears(kv, dt, rows, hidden, nq, nkv, bias):
    rng = np.random.default_rng(rows * 7 + hidden)
    x = O.round_to(rng.standard_normal((rows, hidden)), dt)
    ws = [O.round_to(rng.standard_normal((n, hidden)) / np.sqrt(hidden), dt)
          for n in (nq, nkv, nkv)]
    bs = [O.round_to(0.1 * rng.standard_normal(n), dt) if bias else None for n in (nq, nkv, nkv)]
    outs = [torch.full((rows, n), 5.0, dtype=_T[dt], device=DEV) for n in (nq, nkv, nkv)]
    wk = _dense_ws(kv, rows, nq + 2 * nkv, hidden, rows % 2 == 1)
    kv.qkv_proj(dev(x, dt), dev(np.concatenate(ws), dt),
                dev(np.concatenate(bs), dt) if bias else None, *outs, rows, hidden, nq, nkv, dt,
                wk)
    _assert_clean(wk)
    for name, o, w_, b_ in zip("qkv", outs, ws, bs):
        rel_check(f"qkv_proj {name} rows={rows}", host(o), O.linear_ref(x, w_, b_, dt), dt)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("n_out,n_in", [(1024, 2048), (1024, 3072), (896, 4864), (64, 160),
                                        (8192, 128), (1024, 256), (2048, 256), (1536, 1024)])
def test_linear_residual_matches_oracle(kv, dt, rows, split, n_out, n_in):
    """(1024, 256) and (2048, 256) split K into slices of one 32-wide step
    per wave (a regression case: the steps past a wave's own once ran under
    an exec mask and fed stale operands into the sums). The split runs
    inside the workgroup, each 16-row tile on its own workgroup row:
    (1024, 256) and (2048, 256) in 2 slices, (1536, 1024) in 3,
    (1024, 2048/3072) in 4, (896, 4864) in 4 of its 5."""
    rng = np.random.default_rng(rows + n_in)
    x = O.round_to(rng.standard_normal((rows, n_in)), dt)
    w = O.round_to(rng.standard_normal((n_out, n_in)) / np.sqrt(n_in), dt)
    r = O.round_to(2 * rng.standard_normal((rows, n_out)), dt)
    rd = dev(r, dt)
    wk = _dense_ws(kv, rows, n_out, n_in, split)
    kv.linear_residual(dev(x, dt), dev(w, dt), rd, rows, n_out, n_in, dt, wk)
    _assert_clean(wk)
    want = O.round_to(r + O.linear_ref(x, w, None, dt), dt)
    rel_check(f"linear_residual rows={rows} {n_out}x{n_in} split={split}", host(rd), want, dt)


# K-split projections over 3072 inputs, 64 output tiles (4 slices):
# "residual" is linear_residual and "qkv" a q/k/v projection of
# 512 + 2 x 256 features (both split inside the workgroup, row tiles on grid
# rows), "gate_up" the SwiGLU projection of 2 x 512 features (the split grid
# and its records). Returns the call's output on the host.
_SPLIT_OUT = {"residual": 1024, "qkv": 1024, "gate_up": 512}


def _split_call(kv, kind, x, w, r0, rows, wk):
    dt = "bf16"
    if kind == "residual":
        r = r0.clone()
        kv.linear_residual(x, w, r, rows, 1024, 3072, dt, wk)
        return host(r)
    if kind == "qkv":
        outs = [torch.empty((rows, n), dtype=torch.bfloat16, device=DEV) for n in (512, 256, 256)]
        kv.qkv_proj(x, w, None, *outs, rows, 3072, 512, 256, dt, wk)
        return np.concatenate([host(o) for o in outs], axis=1)
    act = torch.empty((rows, 512), dtype=torch.bfloat16, device=DEV)
    kv.gate_up_silu(x, w, act, rows, 3072, 512, dt, wk)
    return host(act)


def _split_inputs(rng, rows, dt="bf16"):
    x = dev(O.round_to(rng.standard_normal((rows, 3072)), dt), dt)
    w = dev(O.round_to(rng.standard_normal((1024, 3072)) / np.sqrt(3072), dt), dt)
    r0 = dev(O.round_to(rng.standard_normal((rows, 1024)), dt), dt)
    return x, w, r0


@pytest.mark.parametrize("kind,rows", [("residual", 32), ("residual", 64), ("qkv", 64),
                                       ("gate_up", 64)])
def test_k_split_is_deterministic_and_equals_unsplit_closely(kv, kind, rows):
    """The merged K slices add in slice order: repeated calls give the same
    bits; the split and unsplit sums differ only by rounding order (the
    split inside the workgroup for the residual and q/k/v projections, the
    split grid for SwiGLU)."""
    rng = np.random.default_rng(31)
    dt = "bf16"
    x, w, r0 = _split_inputs(rng, rows)
    wk = _dense_ws(kv, rows, 1024, 3072, True)
    assert wk.numel() > 4                    # this shape splits K
    outs = [_split_call(kv, kind, x, w, r0, rows, wk if use else None)
            for use in (True, True, True, False)]
    np.testing.assert_array_equal(outs[0], outs[1])
    np.testing.assert_array_equal(outs[0], outs[2])
    # SwiGLU rounds gate and up before silu(gate) * up: an ulp of either
    # moves the product by up to a few ulps of the largest output
    bar = (8 if kind == "gate_up" else 2) * ULP[dt]
    assert np.abs(outs[0] - outs[3]).max() <= bar * np.abs(outs[3]).max()
    _assert_clean(wk)
    if kind == "gate_up":
        with pytest.raises(kv.RlseError):    # a workspace too small is refused
            _split_call(kv, kind, x, w, r0, rows, wk[:64])


def test_split_results_do_not_depend_on_the_row_count(kv):
    """A row's outputs are the same bits whatever other rows share the call:
    the residual and q/k/v projections (the split inside the workgroup, one
    row tile per workgroup row) at 32, 33 and 64 rows, and SwiGLU (the split
    grid) at 32 and 33 rows, for 2, 3 and 4 slices of q/k/v."""
    rng = np.random.default_rng(35)
    dt = "bf16"
    for hidden, nq, nkv in ((256, 512, 256), (1024, 1024, 256), (3072, 512, 256)):
        n_out = nq + 2 * nkv
        x = O.round_to(rng.standard_normal((64, hidden)), dt)
        w = dev(O.round_to(rng.standard_normal((n_out, hidden)) / np.sqrt(hidden), dt), dt)
        wk = _dense_ws(kv, 64, n_out, hidden, True)
        got = {}
        for rows in (64, 33, 32):
            outs = [torch.empty((rows, n), dtype=torch.bfloat16, device=DEV) for n in (nq, nkv, nkv)]
            kv.qkv_proj(dev(x[:rows], dt), w, None, *outs, rows, hidden, nq, nkv, dt, wk)
            got[rows] = [host(o) for o in outs]
        _assert_clean(wk)
        print(f"row-count independence: q/k/v {n_out}x{hidden}", flush=True)
        for rows in (64, 33):
            for a, b in zip(got[32], got[rows]):
                np.testing.assert_array_equal(a, b[:32])
    x, w, r0 = _split_inputs(rng, 64)
    wk = _dense_ws(kv, 64, 1024, 3072, True)
    for kind, counts in (("residual", (64, 33, 32)), ("gate_up", (33, 32))):
        got = {rows: _split_call(kv, kind, x[:rows], w, r0[:rows], rows, wk) for rows in counts}
        _assert_clean(wk)
        for rows in counts[:-1]:
            np.testing.assert_array_equal(got[32], got[rows][:32])


@pytest.mark.parametrize("kind,rows", [("residual", 32), ("gate_up", 64)])
def test_k_split_ignores_stale_records_and_reports_timeouts(kv, kind, rows):
    """K-split records carry their launch's epoch: records planted with other
    tags between calls (the previous call's epoch, later ones) are never
    summed. With the merge's wait bound forced to zero from the host, a
    merge that gives up writes NaN and raises RLSE_WS_ERR_MERGE_TIMEOUT;
    every kernel ends normally and the next calls are exact again. (The
    residual projection splits inside the workgroup: no records, nothing to
    time out; the planted records must still never reach the sums. SwiGLU
    takes the split grid.)"""
    rng = np.random.default_rng(32)
    dt = "bf16"
    x, w, r0 = _split_inputs(rng, rows)
    wk = _dense_ws(kv, rows, 1024, 3072, True)

    def call():
        return _split_call(kv, kind, x, w, r0, rows, wk)

    ref = call()
    _assert_clean(wk)
    words = wk.view(torch.int32)
    for rep_ in range(2):
        ep = int(words[64].item()) & 0xFFFFFFFF
        recs = wk[(64 + DENSE_CTR) * 4:].view(torch.int64)
        n = recs.numel()
        tags = rng.choice(np.array([ep, (ep + 2) & 0xFFFFFFFF, ep ^ 0x5A5A], np.uint64), n)
        vals = rng.standard_normal(n).astype(np.float32).view(np.uint32).astype(np.uint64)
        recs.copy_(torch.from_numpy(((tags << np.uint64(32)) | vals).view(np.int64)).to(DEV))
        np.testing.assert_array_equal(call(), ref, err_msg=f"stale records, call {rep_}")
        _assert_clean(wk)
    kv.set_merge_wait_ns(0)
    try:
        got = call()
    finally:
        kv.set_merge_wait_ns(100_000_000)
    flags = kv.workspace_flags(wk)
    bad = np.isnan(got)
    print(f"dense timeout ({kind}): flags={flags} NaN outputs={int(bad.sum())}", flush=True)
    assert bool(flags & kv.WS_ERR_MERGE_TIMEOUT) == bool(bad.any())
    np.testing.assert_array_equal(got[~bad], ref[~bad])
    for rep_ in range(2):
        np.testing.assert_array_equal(call(), ref, err_msg=f"after the timeout, call {rep_}")
        _assert_clean(wk)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("hidden,inter", [(1024, 3072), (896, 4864), (128, 8)])
def test_gate_up_silu_matches_oracle(kv, dt, rows, hidden, inter):
    rng = np.random.default_rng(rows + inter)
    x = O.round_to(rng.standard_normal((rows, hidden)), dt)
    wg = O.round_to(rng.standard_normal((inter, hidden)) / np.sqrt(hidden) * 3, dt)
    wu = O.round_to(rng.standard_normal((inter, hidden)) / np.sqrt(hidden), dt)
    act = torch.full((rows, inter), 7.0, dtype=_T[dt], device=DEV)
    wk = _dense_ws(kv, rows, 2 * inter, hidden, rows != 16)
    kv.gate_up_silu(dev(x, dt), dev(np.concatenate([wg, wu]), dt), act, rows, hidden, inter, dt,
                    wk)
    _assert_clean(wk)
    want = O.silu_mul_ref(O.linear_ref(x, wg, None, dt), O.linear_ref(x, wu, None, dt), dt)
    rel_check(f"gate_up_silu rows={rows} {hidden}->{inter}", host(act), want, dt)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_linear_wide_output_tiles(kv, dt):
    """An lm_head-sized output (4+ thousand 16-feature tiles) takes the
    four-tiles-per-workgroup form; the rows straddle a 16-row tile."""
    rng = np.random.default_rng(21)
    rows, n_out, n_in = 20, 65536 + 64, 256
    x = O.round_to(rng.standard_normal((rows, n_in)), dt)
    w = O.round_to(rng.standard_normal((n_out, n_in)) / np.sqrt(n_in), dt)
    y = torch.empty((rows, n_out), dtype=_T[dt], device=DEV)
    kv.linear(dev(x, dt), dev(w, dt), None, y, rows, n_out, n_in, dt)
    rel_check("linear wide", host(y), O.linear_ref(x, w, None, dt), dt)


def test_fused_projections_reject_bad_shapes(kv):
    x = torch.zeros((4, 96), dtype=torch.bfloat16, device=DEV)
    w = torch.zeros((48, 96), dtype=torch.bfloat16, device=DEV)
    o = torch.zeros((4, 48), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(kv.RlseError):   # in_features not a multiple of 32
        kv.linear_residual(x[:, :80].contiguous(), w[:, :80].contiguous(), o, 4, 48, 80, "bf16")
    with pytest.raises(kv.RlseError):   # f32 has no MFMA form here
        kv.linear_residual(x.float(), w.float(), o.float(), 4, 48, 96, "f32")
    with pytest.raises(kv.RlseError):   # feature counts must be multiples of 16
        kv.qkv_proj(x, w, None, o, o, o, 4, 96, 24, 12, "bf16")
    with pytest.raises(kv.RlseError):   # misaligned input
        kv.gate_up_silu(x.view(-1)[1:].data_ptr(), w, o, 4, 96, 24, "bf16")


# ------------------------------------------------------------ whole steps ---
SPECS = {
    "qwen3": dict(hidden=128, layers=2, heads=4, kv_heads=2, head_dim=64, inter=256,
                  vocab=1000, qk_norm=True, qkv_bias=False, tied=True),
    "qwen2": dict(hidden=128, layers=2, heads=14, kv_heads=2, head_dim=64, inter=192,
                  vocab=700, theta=1e4, qk_norm=False, qkv_bias=True, tied=False),
}


def _setup(kv, arch, dt, ctx_lens, steps, seed, packed=True):
    from decode_model import DecodeModel, ModelConfig
    spec = O.ModelSpec(**SPECS[arch])
    rng = np.random.default_rng(seed)
    w = O.random_weights(spec, rng, dt)
    b = len(ctx_lens)
    mbps = max((n + steps + 15) // 16 for n in ctx_lens) + 1
    nb = b * mbps + 5
    tables = build_tables(rng, [mbps * 16] * b, nb, mbps)
    model = DecodeModel(ModelConfig(**SPECS[arch]), w, dt, nb, b, mbps, packed_weights=packed)
    # cached context: random K/V (already rotated), the same in pool and oracle
    kc = [[None] * b for _ in range(spec.layers)]
    vc = [[None] * b for _ in range(spec.layers)]
    t_dev = torch.from_numpy(tables).to(DEV)
    for i, n in enumerate(ctx_lens):
        k = O.round_to(rng.standard_normal((spec.layers, spec.kv_heads, n, spec.head_dim)), dt)
        v = O.round_to(rng.standard_normal((spec.layers, spec.kv_heads, n, spec.head_dim)), dt)
        if n:
            model.set_kv(t_dev[i], k, v)
        for l in range(spec.layers):
            kc[l][i], vc[l][i] = k[l], v[l]
    cos_t, sin_t = O.rope_tables_f32(spec.theta, spec.head_dim, model.max_pos)
    return spec, w, model, t_dev, kc, vc, O.round_to(cos_t, dt), O.round_to(sin_t, dt), rng


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("arch", ["qwen3", "qwen2"])
def test_decode_steps_match_oracle(kv, arch, dt):
    """Three steps of a 3-sequence batch with ragged cached contexts (0, 17
    and 40 tokens); each step's ids are the GPU's greedy picks of the last
    (teacher-forced into the oracle too). Logits, greedy ids and the K/V the
    steps appended are checked."""
    ctx = [0, 17, 40]
    spec, w, model, t_dev, kc, vc, cos_t, sin_t, rng = _setup(kv, arch, dt, ctx, 3, 5)
    ids = np.array(rng.integers(0, spec.vocab, len(ctx)), np.int32)
    lens = np.array(ctx, np.int32)
    for step in range(3):
        lens = lens + 1
        logits, nxt = model.step(torch.from_numpy(ids).to(DEV), t_dev,
                                 torch.from_numpy(lens).to(DEV), len(ctx))
        want = O.model_step_ref(spec, w, list(ids), kc, vc, cos_t, sin_t, dt)
        got = host(logits)
        rel_check(f"{arch} step {step} logits", got, want, dt)
        g = nxt.cpu().numpy()
        np.testing.assert_array_equal(g, O.argmax_ref(got))   # argmax of its own logits
        # the pick is a maximum of the oracle's logits up to the bar
        top = want.max(1)
        assert (want[np.arange(len(g)), g] >= top - 2 * TOL[dt] * np.abs(want).max()).all()
        ids = g.astype(np.int32)
    for i, n in enumerate(lens):
        k, v = model.get_kv(t_dev[i], int(n))
        for l in range(spec.layers):
            rel_check(f"{arch} K layer {l} seq {i}", host(k[l]), kc[l][i], dt)
            rel_check(f"{arch} V layer {l} seq {i}", host(v[l]), vc[l][i], dt)
    model.close()


def _bits(t):
    torch.cuda.synchronize()
    return t.contiguous().view(torch.int16).cpu().numpy()


def _pack(kv, w, n_out, n_in, pair, dt):
    packed = torch.empty_like(w)
    kv.dense_pack(w, packed, n_out, n_in, pair, dt)
    return packed


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_dense_pack_layout(kv, dt):
    """rlse_dense_pack against the layout restated in numpy: packet
    ((tile * K/32 + s) * 64 + lane) = row tile_rows[lane % 16] of the tile,
    elements 32 s + 8 (lane / 16) .. +8; gate/up tiles take gate rows 8t..8t+7
    and up rows inter + 8t..+7."""
    rng = np.random.default_rng(4)
    for n_out, n_in, pair in ((48, 96, 0), (64, 64, 32)):
        w = O.round_to(rng.standard_normal((n_out, n_in)), dt)
        got = host(_pack(kv, dev(w, dt), n_out, n_in, pair, dt)).reshape(-1, 8)
        tiles = n_out // 16
        if pair:
            order = np.concatenate([np.r_[8 * t:8 * t + 8, pair + 8 * t:pair + 8 * t + 8]
                                    for t in range(tiles)])
        else:
            order = np.arange(n_out)
        want = (w[order].reshape(tiles, 16, n_in // 32, 4, 8)
                .transpose(0, 2, 3, 1, 4).reshape(-1, 8))
        np.testing.assert_array_equal(got, want)


def _pack_rows(x):
    """Rows [rows][K] in the packed row order (RLSE_PACKED_ROWS), padded to
    whole 16-row tiles with zeros: packet (t * K/32 + s) * 64 + r + 16 j =
    row 16 t + r, elements 32 s + 8 j .. +8."""
    rows, k = x.shape
    rt = (rows + 15) // 16
    xp = np.zeros((rt * 16, k), x.dtype)
    xp[:rows] = x
    return xp.reshape(rt, 16, k // 32, 4, 8).transpose(0, 2, 3, 1, 4).reshape(rt * 16, k)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("rows", [3, 32, 40])
def test_add_rmsnorm_packed_rows(kv, dt, rows):
    """add_rmsnorm with packed output writes the row-major result's bits in
    the packed row order (with and without the residual add)."""
    rng = np.random.default_rng(rows)
    n = 1024
    x = O.round_to(rng.standard_normal((rows, n)), dt)
    r = O.round_to(rng.standard_normal((rows, n)), dt)
    w = O.round_to(1 + 0.1 * rng.standard_normal(n), dt)
    for add in (False, True):
        outs = []
        for packed in (False, True):
            rd = dev(r, dt)
            out = torch.zeros(((rows + 15) // 16 * 16, n), dtype=_T[dt], device=DEV)
            kv.add_rmsnorm(dev(x, dt) if add else None, rd, dev(w, dt), out, rows, n, 1e-6, dt,
                           packed_out=packed)
            outs.append(host(out))
        want = _pack_rows(outs[0][:rows])
        np.testing.assert_array_equal(outs[1].reshape(-1)[:want.size], want.reshape(-1))


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("rows", [1, 33, 100])
def test_packed_rows_and_weights_give_identical_results(kv, dt, rows):
    """q/k/v, gate/up and a wide linear reading packed x (and packed
    weights) return the row-major call's bits."""
    rng = np.random.default_rng(rows + 5)
    r = lambda *s: O.round_to(rng.standard_normal(s) / np.sqrt(s[-1]), dt)  # noqa: E731
    hidden, nq, nkv, inter, vocab = 1024, 2048, 1024, 3072, 4096
    x = r(rows, hidden)
    xd, xpk = dev(x, dt), dev(_pack_rows(x), dt)
    wq, bq = dev(r(nq + 2 * nkv, hidden), dt), dev(r(nq + 2 * nkv), dt)
    wg, wl = dev(r(2 * inter, hidden), dt), dev(r(vocab, hidden), dt)
    pq = _pack(kv, wq, nq + 2 * nkv, hidden, 0, dt)
    pg = _pack(kv, wg, 2 * inter, hidden, inter, dt)
    pl = _pack(kv, wl, vocab, hidden, 0, dt)
    res = []
    for packed in (False, True):
        xx = xpk if packed else xd
        outs = [torch.zeros((rows, n), dtype=_T[dt], device=DEV) for n in (nq, nkv, nkv)]
        ws = _dense_ws(kv, rows, nq + 2 * nkv, hidden, True)
        kv.qkv_proj(xx, pq if packed else wq, bq, *outs, rows, hidden, nq, nkv, dt, ws,
                    packed=packed, packed_x=packed)
        act = torch.zeros((rows, inter), dtype=_T[dt], device=DEV)
        kv.gate_up_silu(xx, pg if packed else wg, act, rows, hidden, inter, dt, None,
                        packed=packed, packed_x=packed)
        y = torch.zeros((rows, vocab), dtype=_T[dt], device=DEV)
        if packed:
            kv.linear(xx, pl, None, y, rows, vocab, hidden, dt, packed=True, packed_x=True)
        else:
            for r0 in range(0, rows, 64):
                n = min(64, rows - r0)
                kv.linear(xd[r0:r0 + n], wl, None, y[r0:r0 + n], n, vocab, hidden, dt)
        res.append([_bits(o) for o in outs + [act, y]])
    for a, c in zip(*res):
        np.testing.assert_array_equal(a, c)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("rows", [1, 33, 100])
def test_packed_act_feeds_down_proj(kv, dt, rows):
    """gate_up_silu with packed output writes the row-major act's bits in the
    packed row order; down_proj (K split) reading it packed returns the
    row-major call's bits."""
    rng = np.random.default_rng(rows + 11)
    r = lambda *s: O.round_to(rng.standard_normal(s) / np.sqrt(s[-1]), dt)  # noqa: E731
    hidden, inter = 1024, 3072
    x, w, wd = dev(r(rows, hidden), dt), dev(r(2 * inter, hidden), dt), dev(r(hidden, inter), dt)
    act0 = torch.zeros((rows, inter), dtype=_T[dt], device=DEV)
    kv.gate_up_silu(x, w, act0, rows, hidden, inter, dt)
    act1 = torch.zeros(((rows + 15) // 16 * 16, inter), dtype=_T[dt], device=DEV)
    kv.gate_up_silu(x, w, act1, rows, hidden, inter, dt, packed_out=True)
    want = _pack_rows(host(act0))
    np.testing.assert_array_equal(host(act1).reshape(-1)[:want.size], want.reshape(-1))
    res0 = O.round_to(rng.standard_normal((rows, hidden)), dt)
    ys = []
    for a, packed in ((act0, False), (act1, True)):
        y = dev(res0, dt)
        ws = _dense_ws(kv, rows, hidden, inter, True)
        kv.linear_residual(a, wd, y, rows, hidden, inter, dt, ws, packed_x=packed)
        _assert_clean(ws)
        ys.append(_bits(y))
    np.testing.assert_array_equal(ys[0], ys[1])


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("rows", [1, 33, 100])
def test_packed_weights_give_identical_results(kv, dt, rows):
    """Every projection over packed weights (RLSE_DENSE_PACKED) returns the
    row-major weight's bits: q/k/v with bias, o/down_proj with and without
    the K split, gate/up with SwiGLU, and a wide linear (lm_head-like; more
    than 64 rows take 64-row chunks, as two row-major calls do)."""
    rng = np.random.default_rng(rows)
    r = lambda *s: O.round_to(rng.standard_normal(s) / np.sqrt(s[-1]), dt)  # noqa: E731
    # q/k/v
    hidden, nq, nkv = 896, 896, 128
    x, w, b = dev(r(rows, hidden), dt), dev(r(nq + 2 * nkv, hidden), dt), dev(r(nq + 2 * nkv), dt)
    pk = _pack(kv, w, nq + 2 * nkv, hidden, 0, dt)
    res = []
    for packed, w_ in ((False, w), (True, pk)):
        outs = [torch.zeros((rows, n), dtype=_T[dt], device=DEV) for n in (nq, nkv, nkv)]
        ws = _dense_ws(kv, rows, nq + 2 * nkv, hidden, True)
        kv.qkv_proj(x, w_, b, *outs, rows, hidden, nq, nkv, dt, ws, packed=packed)
        _assert_clean(ws)
        res.append([_bits(o) for o in outs])
    for a, c in zip(*res):
        np.testing.assert_array_equal(a, c)
    # o_proj / down_proj, K split and not
    for n_out, n_in, split in ((1024, 3072, True), (1024, 2048, False), (8192, 128, True)):
        x, w = dev(r(rows, n_in), dt), dev(r(n_out, n_in), dt)
        r0 = r(rows, n_out)
        pk = _pack(kv, w, n_out, n_in, 0, dt)
        res = []
        for packed, w_ in ((False, w), (True, pk)):
            rd = dev(r0, dt)
            ws = _dense_ws(kv, rows, n_out, n_in, split)
            kv.linear_residual(x, w_, rd, rows, n_out, n_in, dt, ws, packed=packed)
            _assert_clean(ws)
            res.append(_bits(rd))
        np.testing.assert_array_equal(res[0], res[1])
    # gate/up + SwiGLU
    hidden, inter = 1024, 3072
    x, w = dev(r(rows, hidden), dt), dev(r(2 * inter, hidden), dt)
    pk = _pack(kv, w, 2 * inter, hidden, inter, dt)
    res = []
    for packed, w_ in ((False, w), (True, pk)):
        act = torch.zeros((rows, inter), dtype=_T[dt], device=DEV)
        ws = _dense_ws(kv, rows, 2 * inter, hidden, True)
        kv.gate_up_silu(x, w_, act, rows, hidden, inter, dt, ws, packed=packed)
        _assert_clean(ws)
        res.append(_bits(act))
    np.testing.assert_array_equal(res[0], res[1])
    # wide linear with bias
    n_out, n_in = 4096, 1024
    x, w, b = dev(r(rows, n_in), dt), dev(r(n_out, n_in), dt), dev(r(n_out), dt)
    pk = _pack(kv, w, n_out, n_in, 0, dt)
    y0 = torch.zeros((rows, n_out), dtype=_T[dt], device=DEV)
    for r0 in range(0, rows, 64):
        n = min(64, rows - r0)
        kv.linear(x[r0:r0 + n], w, b, y0[r0:r0 + n], n, n_out, n_in, dt)
    y1 = torch.zeros_like(y0)
    kv.linear(x, pk, b, y1, rows, n_out, n_in, dt, packed=True)
    np.testing.assert_array_equal(_bits(y0), _bits(y1))


@pytest.mark.parametrize("arch", ["qwen3", "qwen2"])
def test_decode_model_packed_weights_equal_row_major(kv, arch):
    """Three steps of DecodeModel over packed weights and over row-major
    weights (same weights, contexts and ids): logits and greedy ids bit for
    bit."""
    ctx, dt = [0, 17, 40], "bf16"
    runs = []
    for packed in (True, False):
        spec, w, model, t_dev, *_rest, rng = _setup(kv, arch, dt, ctx, 3, 9, packed=packed)
        assert model.packed == packed
        ids = np.array(rng.integers(0, spec.vocab, len(ctx)), np.int32)
        lens = np.array(ctx, np.int32)
        out = []
        for step in range(3):
            lens = lens + 1
            logits, nxt = model.step(torch.from_numpy(ids).to(DEV), t_dev,
                                     torch.from_numpy(lens).to(DEV), len(ctx))
            out.append((_bits(logits), nxt.cpu().numpy().copy()))
            ids = out[-1][1].astype(np.int32)
        model.close()
        runs.append(out)
    for (la, ia), (lb, ib) in zip(*runs):
        np.testing.assert_array_equal(la, lb)
        np.testing.assert_array_equal(ia, ib)


def test_greedy_loop_on_device_with_step_tables(kv):
    """Tokens of one step feed the next without leaving the device; pages
    grow through the block manager and StepTables (scheduler.rs:422-449).
    Eight bf16 steps of four sequences from empty caches, against the oracle
    teacher-forced on the device's picks."""
    from decode_model import DecodeModel, ModelConfig
    dt, arch = "bf16", "qwen3"
    spec = O.ModelSpec(**SPECS[arch])
    rng = np.random.default_rng(9)
    w = O.random_weights(spec, rng, dt)
    b, mbps, nb = 4, 4, 32
    bm = kv.BlockManager(nb)
    st = kv.StepTables(b, mbps)
    model = DecodeModel(ModelConfig(**SPECS[arch]), w, dt, nb, b, mbps)
    tables = torch.full((b, mbps), 0, dtype=torch.int32, device=DEV)
    lens_d = torch.zeros(b, dtype=torch.int32, device=DEV)
    reqs = [f"r{i}" for i in range(b)]
    for r in reqs:
        bm.allocate(r, 1)
    ids_d = torch.from_numpy(np.array(rng.integers(0, spec.vocab, b), np.int32)).to(DEV)
    kc = [[np.zeros((spec.kv_heads, 0, spec.head_dim), np.float32) for _ in range(b)]
          for _ in range(spec.layers)]
    vc = [[np.zeros((spec.kv_heads, 0, spec.head_dim), np.float32) for _ in range(b)]
          for _ in range(spec.layers)]
    cos_t, sin_t = O.rope_tables_f32(spec.theta, spec.head_dim, model.max_pos)
    cos_t, sin_t = O.round_to(cos_t, dt), O.round_to(sin_t, dt)
    stream = torch.cuda.current_stream()
    for step in range(8):
        # sequence i starts with a 9*i-token cached prefix; lengths grow
        # across page boundaries as the steps go
        n = [step + 1 + 9 * i for i in range(b)]
        if step == 0:
            for i, r in enumerate(reqs):
                bm.release(r)
                bm.allocate(r, n[i])
        assert st.prepare(bm, reqs, n) == [0] * b
        st.upload(tables, lens_d, stream)
        if step == 0:
            for i in range(1, b):
                k = O.round_to(rng.standard_normal((spec.layers, spec.kv_heads, 9 * i,
                                                    spec.head_dim)), dt)
                v = O.round_to(rng.standard_normal(k.shape), dt)
                model.set_kv(tables[i], k, v, 0, stream)
                for l in range(spec.layers):
                    kc[l][i], vc[l][i] = k[l], v[l]
        ids = ids_d.cpu().numpy().copy()
        logits, nxt = model.step(ids_d, tables, lens_d, b, stream)
        want = O.model_step_ref(spec, w, list(ids), kc, vc, cos_t, sin_t, dt)
        rel_check(f"greedy step {step}", host(logits), want, dt)
        ids_d = nxt.clone()
    assert bm.free_count() == nb - sum(bm.blocks_needed(step + 1 + 9 * i) for i in range(b))
    model.close()


def test_captured_step_replays_equal_eager_steps(kv):
    """DecodeModel.capture records one step into a HIP graph; five replays
    (each after eager work on the same stream and a synchronisation) give the
    logits, greedy ids and K/V that five eager steps of an identical model
    give, bit for bit, and the fed-back ids drive the next replay."""
    from decode_model import DecodeModel, ModelConfig
    dt, arch = "bf16", "qwen3"
    spec = O.ModelSpec(**SPECS[arch])
    rng = np.random.default_rng(17)
    w = O.random_weights(spec, rng, dt)
    b, mbps, nb = 3, 4, 16
    ctx = [5, 20, 33]
    tables = build_tables(rng, [mbps * 16] * b, nb, mbps)
    eager = DecodeModel(ModelConfig(**SPECS[arch]), w, dt, nb, b, mbps)
    graph = DecodeModel(ModelConfig(**SPECS[arch]), w, dt, nb, b, mbps)
    t_dev = torch.from_numpy(tables).to(DEV)
    for i, n in enumerate(ctx):
        k = O.round_to(rng.standard_normal((spec.layers, spec.kv_heads, n, spec.head_dim)), dt)
        v = O.round_to(rng.standard_normal(k.shape), dt)
        eager.set_kv(t_dev[i], k, v)
        graph.set_kv(t_dev[i], k, v)
    ids = torch.from_numpy(np.array(rng.integers(0, spec.vocab, b), np.int32)).to(DEV)
    graph.tables_in.copy_(t_dev)
    graph.ids_in.copy_(ids)
    graph.capture(b)
    lens = np.array(ctx, np.int32)
    for step in range(5):
        lens = lens + 1
        lens_d = torch.from_numpy(lens).to(DEV)
        le, ne = eager.step(ids, t_dev, lens_d, b)
        le, ne = le.clone(), ne.clone()
        scratch = torch.randn(1 << 20, device=DEV).sum()      # eager work between replays
        torch.cuda.synchronize()
        graph.lens_in.copy_(lens_d)
        lg, ng = graph.replay(b)
        torch.cuda.synchronize()
        assert torch.equal(le, lg), step
        assert torch.equal(ne, ng), step
        assert torch.equal(graph.ids_in, ne)                   # fed back for the next replay
        ids = ne.clone()
        del scratch
    for i, n in enumerate(lens):
        ke, ve = eager.get_kv(t_dev[i], int(n))
        kg, vg = graph.get_kv(t_dev[i], int(n))
        assert torch.equal(ke, kg) and torch.equal(ve, vg)
    eager.close()
    graph.close()


def test_decode_model_check_raises_token_limit(kv):
    """DecodeModel.check reads and clears the step's device error flags. A
    step with a sequence longer than its block table (mbps * 16 tokens)
    writes zeros for that row and raises RLSE_WS_ERR_LENGTH on the device;
    check() turns it into TokenLimitExceeded (the reference's
    EngineError::TokenLimitExceeded), after which the next step is clean."""
    from decode_model import DecodeModel, ModelConfig
    dt, arch = "bf16", "qwen3"
    spec = O.ModelSpec(**SPECS[arch])
    rng = np.random.default_rng(23)
    w = O.random_weights(spec, rng, dt)
    b, mbps, nb = 2, 3, 8
    tables = build_tables(rng, [mbps * 16] * b, nb, mbps)
    model = DecodeModel(ModelConfig(**SPECS[arch]), w, dt, nb, b, mbps)
    t_dev = torch.from_numpy(tables).to(DEV)
    ids = torch.from_numpy(np.array([3, 4], np.int32)).to(DEV)
    model.step(ids, t_dev, torch.from_numpy(np.array([5, 9], np.int32)).to(DEV), b)
    model.check()                                    # a clean step
    model.step(ids, t_dev, torch.from_numpy(np.array([5, mbps * 16 + 1], np.int32)).to(DEV), b)
    with pytest.raises(kv.TokenLimitExceeded):
        model.check()
    model.check()                                    # the flag was cleared
    model.step(ids, t_dev, torch.from_numpy(np.array([6, 10], np.int32)).to(DEV), b)
    model.check()
    model.close()

