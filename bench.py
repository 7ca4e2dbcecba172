"""Benchmark of the paged KV-cache decode step on one MI355X.

Default workload: Qwen3-0.6B-shaped batched decode in bf16 -- 16 query heads,
8 KV heads, head_dim 128, 28 layers, 32 sequences with cached lengths drawn
uniformly from [128, 2048] plus the token appended this step, K/V in 16-token
pages placed by a seeded random permutation (one table shared by all layers,
as one block id spans all layers), a distinct pool per layer. One step runs,
for every layer, one rlse_decode_step launch: q/k RMSNorm + RoPE of the new
token, its K/V append into the pool, and the split-K GQA decode over the
paged pool (--unfused runs rlse_qk_norm_rope_append + rlse_paged_gqa_decode
instead). Inputs are synthetic N(0, 1) values resident in HBM before timing
starts.

Printed: one JSON line with tokens/s (decode tokens of all sequences per
second), the decode kernel's achieved HBM bandwidth against the 8 TB/s peak
(algorithmic bytes per launch / HIP-event time per launch), and the oracle's
CPU time on a bounded sample of the same workload.

  python bench.py [--steps K] [--warmup W] [--workload NAME]

Other attention workloads: qwen25 (Qwen2.5-0.5B, G=7, d=64), qwen25_7b
(Qwen2.5-7B, G=7, d=128), qwen3_8b (long context); prefix forks, mixed
batches, chunked prefill and whole decode steps (see --help).
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mini-serve-rs_amd"))

PEAK_HBM_GBS = 8000.0

WORKLOADS = {
    # name: (Hq, Hkv, d, layers, batch, len_lo, len_hi, description)
    "qwen3": (16, 8, 128, 28, 32, 128, 2048,
              "Qwen3-0.6B batched decode: 16q/8kv heads, d=128, 28 layers, B=32, "
              "cached U[128,2048] + 1 appended, bf16, 16-token pages"),
    "qwen25": (14, 2, 64, 24, 64, 4096, 4096,
               "Qwen2.5-0.5B high-GQA decode: 14q/2kv heads, d=64, 24 layers, B=64, "
               "4096 cached + 1 appended, bf16, 16-token pages"),
    "qwen3_8b": (32, 8, 128, 1, 128, 8192, 32768,
                 "Qwen3-8B long-context decode: 32q/8kv heads, d=128, 1 layer, B=128, "
                 "cached U[8192,32768] + 1 appended, bf16, 16-token pages"),
    "qwen25_7b": (28, 4, 128, 28, 32, 128, 2048,
                  "Qwen2.5-7B batched decode: 28q/4kv heads (G=7), d=128, 28 layers, B=32, "
                  "cached U[128,2048] + 1 appended, bf16, 16-token pages"),
}
METRIC_NAME = {
    "qwen3": "decode-attn HBM GB/s (% of peak) + attn tokens/sec at Qwen3-0.6B shape, 1 GPU",
    "qwen25": "decode-attn HBM GB/s (% of peak) + attn tokens/sec at Qwen2.5-0.5B shape, 1 GPU",
    "qwen3_8b": "decode-attn HBM GB/s (% of peak) + attn tokens/sec at Qwen3-8B long-context "
                "shape, 1 GPU",
    "qwen25_7b": "decode-attn HBM GB/s (% of peak) + attn tokens/sec at Qwen2.5-7B shape, 1 GPU",
}
# Chunked prefill: (Hq, Hkv, d, chunk tokens, cached tokens before the chunk, description)
PREFILL = {
    "qwen3_8b_prefill": (32, 8, 128, 512, 8192, "bf16",
                         "Qwen3-8B chunked prefill: 512-token chunk after 8192 cached tokens, "
                         "32q/8kv heads, d=128, causal, bf16, one layer"),
    "qwen3_8b_prefill_f32": (32, 8, 128, 512, 8192, "f32",
                             "Qwen3-8B chunked prefill in f32 (the reference CPU path's dtype): "
                             "512-token chunk after 8192 cached tokens, 32q/8kv heads, d=128, "
                             "causal, one layer"),
}
PEAK_BF16_TFLOPS = 2500.0  # dense MFMA
PEAK_F32_TFLOPS = 157.3    # dense MFMA, f32 operands
# Prefix fork: (Hq, Hkv, d, layers, batch, prefix tokens, suffix lo, suffix hi, description)
FORK = {
    "qwen3_fork": (16, 8, 128, 28, 64, 1024, 64, 512,
                   "Qwen3-0.6B prefix-fork decode: 64 sequences forked from one 1024-token "
                   "prefix (refcounted pages), private suffixes U[64,512] + 1 appended, 16q/8kv "
                   "heads, d=128, 28 layers, bf16"),
    "qwen3_fork1030": (16, 8, 128, 28, 64, 1030, 64, 512,
                       "Qwen3-0.6B prefix-fork decode: 64 sequences forked from one 1030-token "
                       "prefix (refcounted pages + copy-on-write of the partial page), private "
                       "suffixes U[64,512] + 1 appended, 16q/8kv heads, d=128, 28 layers, bf16"),
}

# Mixed batch: sequences forked from several cached prefixes and unforked
# ones in one decode step: (Hq, Hkv, d, layers, [(members, prefix tokens)],
# unforked, suffix lo, suffix hi, unforked cached lo, hi, description)
MIXED = {
    "qwen3_mixed": (16, 8, 128, 28, [(20, 1024), (20, 512), (8, 2048)], 16, 64, 512, 128, 2048,
                    "Qwen3-0.6B mixed-batch decode: 64 sequences -- 20 forked from a 1024-token "
                    "prefix, 20 from a 512-token one, 8 from a 2048-token one (refcounted "
                    "pages), private suffixes U[64,512] + 1 appended -- and 16 unforked with "
                    "U[128,2048] cached + 1, batch order shuffled, 16q/8kv heads, d=128, 28 "
                    "layers, bf16"),
}

# Whole decode step (every op of step_decode_batch on the device):
# (model config factory name, batch, len_lo, len_hi, description)
E2E = {
    "qwen3_e2e": ("qwen3_0_6b", 32, 128, 2048,
                  "Qwen3-0.6B whole decode step: embedding, 28 layers (RMSNorm, q/k/v/o "
                  "projections, q/k norm + RoPE + append + paged GQA decode, SwiGLU MLP), final "
                  "norm, tied lm_head (151936), greedy argmax; B=32, cached U[128,2048] + 1, "
                  "bf16, 16-token pages, random weights"),
    "qwen25_e2e": ("qwen2_5_0_5b", 64, 4096, 4096,
                   "Qwen2.5-0.5B whole decode step: embedding, 24 layers (q/k/v with bias, "
                   "14q/2kv heads, d=64), SwiGLU MLP (4864), tied lm_head (151936), greedy "
                   "argmax; B=64, 4096 cached + 1, bf16, 16-token pages, random weights"),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="qwen3",
                    choices=sorted(WORKLOADS) + sorted(PREFILL) + sorted(FORK) + sorted(MIXED) +
                    sorted(E2E))
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="wall-clock budget of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--unfused", action="store_true",
                    help="norm/RoPE/append and decode as two launches per layer")
    ap.add_argument("--eager", action="store_true",
                    help="whole-step workloads: launch every op from the host each step "
                         "instead of replaying the step captured as a HIP graph")
    ap.add_argument("--no-cascade", action="store_true",
                    help="fork and mixed workloads: decode every sequence's prefix pages in "
                         "the decode launch (rlse_decode_step_planned) instead of once per "
                         "batch or group (rlse_decode_step_cascade / rlse_decode_step_groups)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of 1 GiB (HBM counter calibration)")
    ap.add_argument("--timeline", action="store_true",
                    help="attention workloads: per-phase timeline of the last decode launch of "
                         "one step, from the measurement build (make -C mini-serve-rs_amd/csrc "
                         "timeline), as one JSON line instead of the bench line")
    return ap.parse_args()


COPY_BYTES = 1 << 30


def copy_calibration():
    """A plain device-to-device copy of COPY_BYTES, three times: reads and
    writes exactly COPY_BYTES per dispatch, so the FETCH_SIZE / WRITE_SIZE
    counters of one dispatch give the counters' scale for HBM bytes."""
    import torch
    dev = torch.device("cuda:0")
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "dispatches": 3}))


def algorithmic_decode_bytes(lens, hq, hkv, d, es, fused, qk_norm=True):
    """HBM bytes one decode launch must move: every attended K and V row once,
    q in and out once, the used block-table entries and the lengths. The fused
    step also reads each sequence's new K/V rows and writes them into the pool
    (2 x B x 2 x Hkv x d elements), reads one cos and one sin row of d/2
    elements per sequence and, when the model has q/k norms, the two RMSNorm
    weights."""
    b = len(lens)
    kv = sum(int(n) * 2 * hkv * d * es for n in lens)
    qo = 2 * b * hq * d * es
    tab = sum(((int(n) + 15) // 16) * 4 for n in lens)
    app = (2 * b * 2 * hkv * d * es + b * d * es + (2 * d * es if qk_norm else 0)) if fused else 0
    return kv + qo + tab + 4 * b + app


def measured_traffic(workload, fused):
    """HBM bytes per launch of the fused decode kernel for this workload, from
    the committed rocprofv3 FETCH_SIZE / WRITE_SIZE counter runs (scaled by the
    copy calibration recorded beside them), or None when none is recorded."""
    if not fused:
        return None, None
    path = os.path.join(ROOT, "profiles", f"decode_step_{workload}_hbm_counters.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        rec = json.load(f)
    return rec["traffic_bytes_per_launch"], os.path.relpath(path, ROOT)


# What every cpu_baseline times: the oracle's scalar C restatement of the
# reference's Candle CPU path (gcc -O2, no fast-math, no contraction,
# sequential dot products; OpenMP over "cores" threads), not Candle itself,
# whose matmuls use the SIMD gemm crate. "nproc" is the host's CPU count.
ORACLE_IMPL = ("scalar C restatement of the reference CPU path (-O2, no SIMD gemm), "
               "OpenMP over 'cores' threads")


def cpu_baseline(args, lens, hq, hkv, d, layers):
    """The oracle (C restatement of the reference's Candle CPU path: contiguous
    per-sequence f32 buffers, KvCache append, per-KV-head matmul / softmax /
    matmul) timed on this host for a bounded number of layer-steps."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    b = len(lens)
    cap = int(max(lens))
    rng = np.random.default_rng(7)
    tile = rng.standard_normal((hkv, 1, d)).astype(np.float32)
    k = np.ascontiguousarray(np.broadcast_to(tile, (b, hkv, cap, d)), dtype=np.float32)
    v = k.copy()
    q = rng.standard_normal((b, hq, d)).astype(np.float32)
    kn = rng.standard_normal((b, hkv, d)).astype(np.float32)
    vn = rng.standard_normal((b, hkv, d)).astype(np.float32)
    lens32 = np.asarray(lens, np.int32)
    threads = O.max_threads()
    scale = 1.0 / math.sqrt(d)
    O.decode_step_f32(q, kn, vn, k, v, lens32, scale, threads)  # warm
    n = 0
    t0 = time.perf_counter()
    while True:
        O.decode_step_f32(q, kn, vn, k, v, lens32, scale, threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= args.cpu_seconds or n >= 200 * layers:
            break
    steps = n / layers
    return {"value": b * steps / el, "unit": "tokens/s", "cores": threads, "kind": "port",
            "nproc": os.cpu_count(), "impl": ORACLE_IMPL,
            "sample": f"{n} layer-steps (append + decode of all {b} sequences, f32, one "
                      f"layer's contiguous buffers reused) in {el:.2f} s = {steps:.2f} "
                      f"decode steps of {layers} layers"}


def prefill_flops(hq, d, tq, offset):
    """Algorithmic FLOPs of one causal chunk: query t attends offset+t+1 keys;
    q.k and p.v are 2*d FLOPs each per (query head, key)."""
    pairs = tq * offset + tq * (tq + 1) // 2
    return 4 * d * hq * pairs


def prefill_bench(args):
    """One step = one rlse_prefill_attn call (its merge launch included) for
    the chunk, inputs resident in HBM; value = algorithmic TFLOP/s."""
    import numpy as np
    import torch

    import rlse_kv as kv

    hq, hkv, d, tq, offset, dt, desc = PREFILL[args.workload]
    peak = PEAK_F32_TFLOPS if dt == "f32" else PEAK_BF16_TFLOPS
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L = offset + tq
    npages = (L + 15) // 16
    nb = npages + 64
    rng = np.random.default_rng(args.seed)
    table = torch.from_numpy(rng.permutation(nb)[:npages].astype(np.int32)).to(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    tdt = torch.float32 if dt == "f32" else torch.bfloat16
    kp = torch.randn((nb, hkv, 16, d), generator=g, device=dev, dtype=tdt)
    vp = torch.randn((nb, hkv, 16, d), generator=g, device=dev, dtype=tdt)
    q = torch.randn((tq, hq, d), generator=g, device=dev, dtype=tdt)
    out = torch.empty_like(q)
    ws_bytes = kv.prefill_workspace_size(tq, L, hq, hkv, d)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    scale = 1.0 / math.sqrt(d)

    def step():
        kv.prefill_attn(q, kp, vp, table, L, tq, out, hq, hkv, d, npages, nb, scale, dt, ws,
                        ws_bytes, stream)

    for _ in range(args.warmup):
        step()
    # Launch duration by HIP events on the launch stream: one pair around
    # the timed calls (no event-record stall between them), / calls.
    n_ev = args.steps
    ev_a, ev_b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev_a.record(stream)
    for _ in range(args.steps):
        step()
    ev_b.record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    avg_ms = ev_a.elapsed_time(ev_b) / n_ev
    flops = prefill_flops(hq, d, tq, offset)
    achieved = flops / (avg_ms * 1e-3) / 1e12
    result = {
        "metric": f"prefill-attn TFLOP/s (% of dense {dt} MFMA peak) at Qwen3-8B chunk, 1 GPU",
        "value": flops * args.steps / elapsed / 1e12, "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": elapsed * 1e3 / args.steps, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": dt,
        "data": "synthetic N(0,1) q/K/V, seeded random page permutation",
        "config": {"workload": desc, "chunk": tq, "cached": offset, "q_heads": hq,
                   "kv_heads": hkv, "head_dim": d, "splits_workspace_bytes": ws_bytes,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": peak,
                     "unit": "TFLOP/s", "frac": achieved / peak, "traffic": None,
                     "kernel": "prefill_kernel + prefill_merge_kernel (rlse_prefill_attn)",
                     "flops_per_launch": flops, "avg_launch_ms": avg_ms,
                     "timed_launches": n_ev},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        result["cpu_baseline"] = prefill_cpu_baseline(args, hq, hkv, d, tq, offset)
    print(json.dumps(result))


def prefill_cpu_baseline(args, hq, hkv, d, tq, offset):
    """The oracle's orc_prefill_f32 (Candle's CPU op order: per query, dot
    products, mask, softmax, weighted V sum; OpenMP over all host threads) on
    the same chunk shape, for a bounded number of KV heads."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    g = hq // hkv
    L = offset + tq
    rng = np.random.default_rng(7)
    q = rng.standard_normal((g, tq, d)).astype(np.float32)
    k = rng.standard_normal((1, L, d)).astype(np.float32)
    v = rng.standard_normal((1, L, d)).astype(np.float32)
    threads = O.max_threads()
    n = 0
    t0 = time.perf_counter()
    while True:
        O.prefill_f32(q, k, v, offset, 1.0 / math.sqrt(d), threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= args.cpu_seconds or n >= hkv:
            break
    flops = prefill_flops(g, d, tq, offset) * n
    return {"value": flops / el / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "nproc": os.cpu_count(), "impl": ORACLE_IMPL,
            "sample": f"{n} KV head(s) of the chunk ({g} query heads each, f32) in {el:.2f} s"}


def fork_inputs(workload, seed, dev, layers=None):
    """Every buffer of a prefix-fork workload, resident on dev. One prefix of
    plen tokens is written into refcounted pages of a pool handle (all layers
    in one allocation, one block id spanning the layers); 64 requests are
    forked from it by the block manager (full pages shared, the trailing
    partial page copied on write, timed as fork_ms), each then growing
    private pages for its suffix of U[lo, hi] cached tokens + the token this
    step appends. Returns the pool, the host and device block tables, the
    lengths (keys after the append), each layer's q / new k / new v, the q/k
    RMSNorm weights and the RoPE tables. layers: how many layers the pool
    holds (default: all of the workload's)."""
    import numpy as np
    import torch
    import rlse_kv as kv
    hq, hkv, d, n_layers, b, plen, lo, hi, _ = FORK[workload]
    layers = n_layers if layers is None else layers
    rng = np.random.default_rng(seed)
    suffix = rng.integers(lo, hi + 1, b).astype(np.int32)
    lens = plen + suffix + 1  # keys after this step's append
    nb = (plen + 15) // 16 + int(sum((int(n) + 15) // 16 - plen // 16 for n in lens)) + 64
    bf = torch.bfloat16
    pool = kv.KVPool(layers, nb, hkv, d, "bf16")
    stride = pool.layer_stride_elems
    k0, v0 = pool.layer(0)
    bm = kv.BlockManager(nb)
    bm.allocate("prefix", plen)
    ptable = torch.tensor(bm.block_table("prefix"), dtype=torch.int32, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    pk = torch.randn((layers, hkv, plen, d), generator=g, device=dev, dtype=bf)
    pv = torch.randn((layers, hkv, plen, d), generator=g, device=dev, dtype=bf)
    kv.kv_scatter(pk, pv, k0, v0, stride, layers, ptable, 0, plen, hkv, d, nb, "bf16")
    del pk, pv
    torch.cuda.synchronize()
    # Fork every request from the prefix (host block manager + one device
    # copy of the partial pages), timed.
    t0 = time.perf_counter()
    src, dst = [], []
    for i in range(b):
        for sp, dp in bm.fork("prefix", f"r{i}", plen):
            src.append(sp)
            dst.append(dp)
    if src:
        kv.kv_copy_blocks(k0, v0, stride, layers, torch.tensor(src, dtype=torch.int32, device=dev),
                          torch.tensor(dst, dtype=torch.int32, device=dev), len(src), hkv, d, nb,
                          "bf16")
    torch.cuda.synchronize()
    fork_ms = (time.perf_counter() - t0) * 1e3
    # Private suffix pages and their cached K/V.
    for i in range(b):
        while len(bm.block_table(f"r{i}")) * 16 < int(lens[i]):
            bm.allocate_block(f"r{i}")
    mbps = max(len(bm.block_table(f"r{i}")) for i in range(b))
    tables = np.zeros((b, mbps), np.int32)
    for i in range(b):
        t = bm.block_table(f"r{i}")
        tables[i, :len(t)] = t
    t_dev = torch.from_numpy(tables).to(dev)
    for i in range(b):
        n = int(suffix[i])
        sk = torch.randn((layers, hkv, n, d), generator=g, device=dev, dtype=bf)
        sv = torch.randn((layers, hkv, n, d), generator=g, device=dev, dtype=bf)
        kv.kv_scatter(sk, sv, k0, v0, stride, layers, t_dev[i], plen, n, hkv, d, nb, "bf16")
    q_in = [torch.randn((b, hq, d), generator=g, device=dev, dtype=bf) for _ in range(layers)]
    k_in = [torch.randn((b, hkv, d), generator=g, device=dev, dtype=bf) for _ in range(layers)]
    v_in = [torch.randn((b, hkv, d), generator=g, device=dev, dtype=bf) for _ in range(layers)]
    qw = (1 + 0.1 * torch.randn(d, generator=g, device=dev)).to(bf)
    kw = (1 + 0.1 * torch.randn(d, generator=g, device=dev)).to(bf)
    max_pos = mbps * 16
    cos_b, sin_b = kv.rope_tables(1e6, d, max_pos, "bf16")
    cos_t = torch.frombuffer(bytearray(cos_b), dtype=torch.int16).to(dev).view(bf)
    sin_t = torch.frombuffer(bytearray(sin_b), dtype=torch.int16).to(dev).view(bf)
    return {"pool": pool, "block_manager": bm, "lens": lens, "suffix": suffix, "tables": tables,
            "tables_dev": t_dev, "prefix_table": ptable, "mbps": mbps, "num_blocks": nb,
            "cow_pairs": src, "fork_ms": fork_ms, "q": q_in, "k_new": k_in, "v_new": v_in,
            "q_norm": qw, "k_norm": kw, "cos": cos_t, "sin": sin_t, "cos_bytes": cos_b,
            "sin_bytes": sin_b, "max_pos": max_pos}


def mixed_inputs(workload, seed, dev, layers=None):
    """Every buffer of a mixed-batch workload, resident on dev: each prefix
    of the workload written into refcounted pages of one pool handle and
    forked to its members by the block manager (full pages shared), the
    unforked sequences with private pages only, every sequence growing
    private pages for its suffix and the token this step appends; the batch
    order is a seeded permutation, so group members are scattered. Returns
    the pool, the tables, the lengths, seq_group (-1 = unforked), the groups'
    shared pages, each layer's q / new k / new v, the q/k RMSNorm weights and
    the RoPE tables."""
    import numpy as np
    import torch
    import rlse_kv as kv
    hq, hkv, d, n_layers, groups, n_free, lo, hi, flo, fhi, _ = MIXED[workload]
    layers = n_layers if layers is None else layers
    rng = np.random.default_rng(seed)
    spec = [(g, plen) for g, (n, plen) in enumerate(groups) for _ in range(n)]
    spec += [(-1, 0)] * n_free
    spec = [spec[i] for i in rng.permutation(len(spec))]
    b = len(spec)
    lens = np.array([plen + int(rng.integers(lo, hi + 1)) + 1 if g >= 0 else
                     int(rng.integers(flo, fhi + 1)) + 1 for g, plen in spec], np.int32)
    nb = sum((plen + 15) // 16 for _, plen in groups) + \
        int(sum((int(n) + 15) // 16 - plen // 16 for n, (_, plen) in zip(lens, spec))) + 64
    bf = torch.bfloat16
    pool = kv.KVPool(layers, nb, hkv, d, "bf16")
    stride = pool.layer_stride_elems
    k0, v0 = pool.layer(0)
    bm = kv.BlockManager(nb)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    for gi, (_, plen) in enumerate(groups):
        bm.allocate(f"prefix{gi}", plen)
        ptable = torch.tensor(bm.block_table(f"prefix{gi}"), dtype=torch.int32, device=dev)
        pk = torch.randn((layers, hkv, plen, d), generator=g, device=dev, dtype=bf)
        pv = torch.randn((layers, hkv, plen, d), generator=g, device=dev, dtype=bf)
        kv.kv_scatter(pk, pv, k0, v0, stride, layers, ptable, 0, plen, hkv, d, nb, "bf16")
        del pk, pv
    src, dst = [], []
    for i, (gi, plen) in enumerate(spec):
        if gi >= 0:
            for sp, dp in bm.fork(f"prefix{gi}", f"r{i}", plen):
                src.append(sp)
                dst.append(dp)
    if src:
        kv.kv_copy_blocks(k0, v0, stride, layers, torch.tensor(src, dtype=torch.int32, device=dev),
                          torch.tensor(dst, dtype=torch.int32, device=dev), len(src), hkv, d, nb,
                          "bf16")
    for i, (gi, plen) in enumerate(spec):
        if gi < 0:
            bm.allocate(f"r{i}", 0)
        while len(bm.block_table(f"r{i}")) * 16 < int(lens[i]):
            bm.allocate_block(f"r{i}")
    mbps = max(len(bm.block_table(f"r{i}")) for i in range(b))
    tables = np.zeros((b, mbps), np.int32)
    for i in range(b):
        t = bm.block_table(f"r{i}")
        tables[i, :len(t)] = t
    t_dev = torch.from_numpy(tables).to(dev)
    for i, (gi, plen) in enumerate(spec):   # private cached tokens (before the new one)
        start = plen if gi >= 0 else 0
        n = int(lens[i]) - 1 - start
        sk = torch.randn((layers, hkv, n, d), generator=g, device=dev, dtype=bf)
        sv = torch.randn((layers, hkv, n, d), generator=g, device=dev, dtype=bf)
        kv.kv_scatter(sk, sv, k0, v0, stride, layers, t_dev[i], start, n, hkv, d, nb, "bf16")
    q_in = [torch.randn((b, hq, d), generator=g, device=dev, dtype=bf) for _ in range(layers)]
    k_in = [torch.randn((b, hkv, d), generator=g, device=dev, dtype=bf) for _ in range(layers)]
    v_in = [torch.randn((b, hkv, d), generator=g, device=dev, dtype=bf) for _ in range(layers)]
    qw = (1 + 0.1 * torch.randn(d, generator=g, device=dev)).to(bf)
    kw = (1 + 0.1 * torch.randn(d, generator=g, device=dev)).to(bf)
    max_pos = mbps * 16
    cos_b, sin_b = kv.rope_tables(1e6, d, max_pos, "bf16")
    cos_t = torch.frombuffer(bytearray(cos_b), dtype=torch.int16).to(dev).view(bf)
    sin_t = torch.frombuffer(bytearray(sin_b), dtype=torch.int16).to(dev).view(bf)
    torch.cuda.synchronize()
    return {"pool": pool, "lens": lens, "tables": tables, "tables_dev": t_dev, "mbps": mbps,
            "num_blocks": nb, "seq_group": np.array([gi for gi, _ in spec], np.int32),
            "group_pages": np.array([plen // 16 for _, plen in groups], np.int32),
            "prefix_tokens": [plen for _, plen in groups], "q": q_in, "k_new": k_in,
            "v_new": v_in, "q_norm": qw, "k_norm": kw, "cos": cos_t, "sin": sin_t,
            "cos_bytes": cos_b, "sin_bytes": sin_b, "max_pos": max_pos}


def mixed_bench(args):
    """Mixed batch: one step = one fused decode step per layer for the whole
    batch (append of the new token + decode): by default the grouped cascade
    step (rlse_decode_step_groups: each group's shared pages attended once
    for its members, every other page streamed), with --no-cascade the
    planned step over every sequence's whole table (shared pages cacheable,
    re-read by every member)."""
    import numpy as np
    import torch

    import rlse_kv as kv

    hq, hkv, d, layers, groups, _, _, _, _, _, desc = MIXED[args.workload]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    f = mixed_inputs(args.workload, args.seed, dev)
    pool, lens, mbps, nb, t_dev = f["pool"], f["lens"], f["mbps"], f["num_blocks"], f["tables_dev"]
    b = len(lens)
    lens_dev = torch.from_numpy(lens).to(dev)
    sg_dev = torch.from_numpy(f["seq_group"]).to(dev)
    gp_dev = torch.from_numpy(f["group_pages"]).to(dev)
    ng, max_pages = len(groups), int(f["group_pages"].max())
    out = torch.empty((b, hq, d), device=dev, dtype=torch.bfloat16)
    ws_bytes = kv.decode_workspace_size(b, hq, hkv, d)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    plan_bytes = kv.decode_plan_size()
    plan = torch.zeros(plan_bytes, dtype=torch.uint8, device=dev)
    pre_bytes = kv.decode_prefix_size(b, hq, d, max_pages)
    pre = torch.zeros(pre_bytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    scale = 1.0 / math.sqrt(d)
    ptrs = [pool.layer(layer) for layer in range(layers)]
    cascade = not args.no_cascade

    def step(evs=None):
        if cascade:
            kv.decode_plan_groups(t_dev, lens_dev, sg_dev, gp_dev, ng, b, hq, hkv, mbps, nb, plan,
                                  plan_bytes, stream)
        else:
            kv.decode_plan(t_dev, lens_dev, b, hkv, mbps, nb, plan, plan_bytes, stream)
        if evs is not None:
            evs[0].record(stream)
        for layer in range(layers):
            a = (f["q"][layer], f["k_new"][layer], f["v_new"][layer], f["q_norm"], f["k_norm"],
                 1e-6, f["cos"], f["sin"], f["max_pos"], ptrs[layer][0], ptrs[layer][1], t_dev,
                 lens_dev, out, b, hq, hkv, d, mbps, nb, scale, "bf16", plan)
            if cascade:
                kv.decode_step_groups(*a, ng, max_pages, pre, pre_bytes, ws, ws_bytes, stream,
                                      stream_pages=True)
            else:
                kv.decode_step_planned(*a, ws, ws_bytes, stream)
        if evs is not None:
            evs[1].record(stream)

    for _ in range(args.warmup):
        step()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e in evs:
        step(e)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    kv.workspace_check(ws)
    avg_ms = float(np.mean([a.elapsed_time(z) for a, z in evs])) / layers
    row = 2 * hkv * d * 2  # K+V bytes of one token
    extra = 2 * b * hq * d * 2 + sum(((int(n) + 15) // 16) * 4 for n in lens) + 4 * b + \
        2 * b * row + b * d * 2 + 2 * d * 2
    shared = sum(f["prefix_tokens"])
    own = int(sum(int(n) - (f["prefix_tokens"][gi] if gi >= 0 else 0)
                  for n, gi in zip(lens, f["seq_group"])))
    compulsory = (shared + own) * row + extra
    logical = int(sum(int(n) for n in lens)) * row + extra
    achieved = compulsory / (avg_ms * 1e-3) / 1e9
    result = {
        "metric": "mixed-batch decode tokens/sec and compulsory HBM GB/s at Qwen3-0.6B shape, "
                  "1 GPU",
        "value": b * args.steps / elapsed, "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": elapsed * 1e3 / args.steps,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic N(0,1) prefix/suffix K/V and q, block-manager page placement",
        "config": {"workload": desc, "batch": b, "layers": layers, "groups": groups,
                   "mean_keys": float(np.mean(lens)), "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": None,
                     "kernel": ("decode_prefix_kernel (groups) + decode_kernel grouped cascade "
                                "step (rlse_decode_step_groups)" if cascade else
                                "decode_kernel planned fused step (rlse_decode_step_planned, "
                                "cacheable pages)"),
                     "bytes_per_launch": compulsory, "logical_bytes_per_launch": logical,
                     "effective_GBps": logical / (avg_ms * 1e-3) / 1e9,
                     "avg_launch_ms": avg_ms, "timed_launches": args.steps * layers},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(args, lens, hq, hkv, d, layers)
    print(json.dumps(result))
    pool.close()


def fork_bench(args):
    """Prefix fork: one prefix held in refcounted pages of a pool handle (all
    layers in one allocation, one block id spanning the layers), 64 requests
    forked from it by the block manager (full pages shared, the trailing
    partial page copied on write), each with a private suffix. The fork runs
    once per request and is timed on its own; one step = one fused decode step
    per layer for the 64 forked sequences (append of the new token + decode
    over shared prefix pages and private suffix pages): by default the
    cascade step (rlse_decode_step_cascade: the shared full pages attended once
    for the batch, then each sequence's own pages, streamed), with
    --no-cascade the planned step over every sequence's whole table (prefix
    pages cacheable, re-read by every row)."""
    import numpy as np
    import torch

    import rlse_kv as kv

    hq, hkv, d, layers, b, plen, lo, hi, desc = FORK[args.workload]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    f = fork_inputs(args.workload, args.seed, dev)
    pool, lens, tables, mbps, nb = f["pool"], f["lens"], f["tables"], f["mbps"], f["num_blocks"]
    src, fork_ms, t_dev = f["cow_pairs"], f["fork_ms"], f["tables_dev"]
    q_in, k_in, v_in, qw, kw = f["q"], f["k_new"], f["v_new"], f["q_norm"], f["k_norm"]
    cos_t, sin_t, max_pos = f["cos"], f["sin"], f["max_pos"]
    bf = torch.bfloat16
    lens_dev = torch.from_numpy(lens.astype(np.int32)).to(dev)
    out = torch.empty((b, hq, d), device=dev, dtype=bf)
    ws_bytes = kv.decode_workspace_size(b, hq, hkv, d)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    plan_bytes = kv.decode_plan_size()
    plan = torch.zeros(plan_bytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    scale = 1.0 / math.sqrt(d)
    ptrs = [pool.layer(layer) for layer in range(layers)]
    cascade = not args.no_cascade
    shared = plen // 16      # full prefix pages, the same in every table
    pre_bytes = kv.decode_prefix_size(b, hq, d, shared)
    pre = torch.zeros(pre_bytes, dtype=torch.uint8, device=dev)

    def step(evs=None):
        # evs: one event pair around the step's back-to-back decode launches.
        if cascade:
            kv.decode_plan_cascade(t_dev, lens_dev, b, hkv, mbps, nb, shared, plan, plan_bytes,
                                   stream)
        else:
            kv.decode_plan(t_dev, lens_dev, b, hkv, mbps, nb, plan, plan_bytes, stream)
        if evs is not None:
            evs[0].record(stream)
        for layer in range(layers):
            if cascade:
                # The shared pages are attended once for the batch; the
                # launch after it reads each page once (streamed).
                kv.decode_step_cascade(q_in[layer], k_in[layer], v_in[layer], qw, kw, 1e-6,
                                       cos_t, sin_t, max_pos, ptrs[layer][0], ptrs[layer][1],
                                       t_dev, lens_dev, out, b, hq, hkv, d, mbps, nb, scale,
                                       "bf16", plan, shared, pre, pre_bytes, ws, ws_bytes,
                                       stream, stream_pages=True)
            else:
                # The prefix pages are read by all b rows: they stay cacheable
                # (no RLSE_DECODE_STREAM), so their re-reads hit the caches.
                kv.decode_step_planned(q_in[layer], k_in[layer], v_in[layer], qw, kw, 1e-6,
                                       cos_t, sin_t, max_pos, ptrs[layer][0], ptrs[layer][1],
                                       t_dev, lens_dev, out, b, hq, hkv, d, mbps, nb, scale,
                                       "bf16", plan, ws, ws_bytes, stream)
        if evs is not None:
            evs[1].record(stream)

    for _ in range(args.warmup):
        step()
    ev_steps = args.steps   # an event pair in every timed step
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(ev_steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e in evs:
        step(e)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    avg_ms = float(np.mean([a.elapsed_time(z) for a, z in evs])) / layers
    row = 2 * hkv * d * 2  # K+V bytes of one token
    extra = 2 * b * hq * d * 2 + sum(((int(n) + 15) // 16) * 4 for n in lens) + 4 * b + \
        2 * b * row + b * d * 2 + 2 * d * 2
    compulsory = plen * row + int(sum(int(n) - plen for n in lens)) * row + extra
    logical = int(sum(int(n) for n in lens)) * row + extra
    # The committed counters are those of the cascade step's three kernels.
    traffic, traffic_src = measured_traffic(args.workload, cascade)
    achieved = compulsory / (avg_ms * 1e-3) / 1e9
    result = {
        "metric": "prefix-fork decode tokens/sec and compulsory HBM GB/s at Qwen3-0.6B shape, "
                  "1 GPU",
        "value": b * args.steps / elapsed, "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": elapsed * 1e3 / args.steps,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic N(0,1) prefix/suffix K/V and q, block-manager page placement",
        "config": {"workload": desc, "batch": b, "layers": layers, "prefix": plen,
                   "cascade_pages": shared if cascade else 0,
                   "mean_keys": float(np.mean(lens)), "fork_ms": fork_ms,
                   "cow_pages_per_layer": len(src), "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": ("decode_prefix_kernel + decode_kernel cascade step "
                                "(rlse_decode_step_cascade, the batch's shared pages attended "
                                "once, the rest streamed)" if cascade else
                                "decode_kernel planned fused step "
                                "(rlse_decode_step_planned, cacheable pages)"),
                     "bytes_per_launch": compulsory, "logical_bytes_per_launch": logical,
                     "effective_GBps": logical / (avg_ms * 1e-3) / 1e9,
                     "avg_launch_ms": avg_ms, "timed_launches": ev_steps * layers},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        # The reference holds every forked sequence in its own contiguous
        # buffers (prefix copied in), so its decode step is the plain one over
        # prefix + suffix keys.
        result["cpu_baseline"] = cpu_baseline(args, lens, hq, hkv, d, layers)
    print(json.dumps(result))
    pool.close()


def e2e_step_bytes(cfg, lens, es):
    """Algorithmic HBM bytes of one whole decode step: every weight read once
    (the projections, the norms, lm_head; the tied embedding is read as
    lm_head and its B gathered rows), each layer's decode-step bytes (K/V of
    every attended position, the appended rows, q in / out, tables), and the
    activations each launch reads and writes."""
    b = len(lens)
    h, d = cfg.hidden, cfg.head_dim
    nq, nkv = cfg.heads * d, cfg.kv_heads * d
    per_layer_w = (h * (nq + 2 * nkv) + nq * h + 2 * cfg.inter * h + cfg.inter * h + 2 * h) * es
    per_layer_w += ((nq + 2 * nkv) * es if cfg.qkv_bias else 0) + (2 * d * es if cfg.qk_norm
                                                                   else 0)
    # activations: q/k/v/o/gate_up/down linears (in + out), two add+norm
    # launches (x, residual read and written, out written), silu_mul
    act = b * es * ((h + nq) + 2 * (h + nkv) + (nq + h) + (h + 2 * cfg.inter) +
                    (cfg.inter + h) + 2 * 4 * h + 3 * cfg.inter)
    attn = algorithmic_decode_bytes(lens, cfg.heads, cfg.kv_heads, d, es, True) - 2 * b * nq * es
    head = cfg.vocab * h * es + b * h * es + b * cfg.vocab * es + b * cfg.vocab * es + 4 * b
    embed = b * (4 + 2 * h * es) + 2 * b * h * es + h * es  # gather, first norm, final norm
    return cfg.layers * (per_layer_w + act + attn) + head + embed


def e2e_bench(args):
    """One step = DecodeModel.step: every op of step_decode_batch for all B
    sequences on one stream, the greedy ids of a step fed as the next step's
    input on the device. Each step appends at the same positions (cached + 1
    keys), as the attention-only workloads do."""
    import numpy as np
    import torch

    import rlse_kv as kv
    from decode_model import DecodeModel, ModelConfig

    factory, b, lo, hi, desc = E2E[args.workload]
    cfg = getattr(ModelConfig, factory)()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    rng = np.random.default_rng(args.seed)
    cached = rng.integers(lo, hi + 1, b).astype(np.int32)
    lens = cached + 1
    mbps = int(max((int(n) + 15) // 16 for n in lens))
    need = int(sum((int(n) + 15) // 16 for n in lens))
    nb = need + 64
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.zeros((b, mbps), np.int32)
    used = 0
    for i, n in enumerate(lens):
        k = (int(n) + 15) // 16
        tables[i, :k] = perm[used:used + k]
        used += k
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    bf = torch.bfloat16
    h, d = cfg.hidden, cfg.head_dim
    nq, nkv = cfg.heads * d, cfg.kv_heads * d

    def mat(o, i):
        return (torch.randn((o, i), generator=g, device=dev) / math.sqrt(i)).to(bf)

    def vec(n, base=1.0, sd=0.1):
        return (base + sd * torch.randn(n, generator=g, device=dev)).to(bf)

    w = {"embed": torch.randn((cfg.vocab, h), generator=g, device=dev).to(bf), "norm": vec(h)}
    for l in range(cfg.layers):
        p = f"l{l}."
        w.update({p + "in_norm": vec(h), p + "post_norm": vec(h), p + "q_w": mat(nq, h),
                  p + "k_w": mat(nkv, h), p + "v_w": mat(nkv, h), p + "o_w": mat(h, nq),
                  p + "gate_w": mat(cfg.inter, h), p + "up_w": mat(cfg.inter, h),
                  p + "down_w": mat(h, cfg.inter)})
        if cfg.qkv_bias:
            w.update({p + "q_b": vec(nq, 0), p + "k_b": vec(nkv, 0), p + "v_b": vec(nkv, 0)})
        if cfg.qk_norm:
            w.update({p + "q_norm": vec(d), p + "k_norm": vec(d)})
    # The table is a permutation: no page is shared, so attention streams.
    model = DecodeModel(cfg, w, "bf16", nb, b, mbps, dev, stream_pages=True)
    del w
    t_dev = torch.from_numpy(tables).to(dev)
    for i, n in enumerate(cached):   # cached context: N(0,1) K/V in every layer
        kc = torch.randn((cfg.layers, cfg.kv_heads, int(n), d), generator=g, device=dev).to(bf)
        vc = torch.randn((cfg.layers, cfg.kv_heads, int(n), d), generator=g, device=dev).to(bf)
        model.set_kv(t_dev[i], kc, vc)
        del kc, vc
    lens_dev = torch.from_numpy(lens).to(dev)
    ids = torch.from_numpy(rng.integers(0, cfg.vocab, b).astype(np.int32)).to(dev)
    stream = torch.cuda.current_stream()
    state = {"ids": ids}
    if not args.eager:
        # The step captured once as a HIP graph over the model's input
        # buffers; each replay feeds its greedy ids to the next.
        model.ids_in[:b].copy_(ids)
        model.tables_in[:b].copy_(t_dev)
        model.lens_in[:b].copy_(lens_dev)
        model.capture(b)

    def step():
        if args.eager:
            _, nxt = model.step(state["ids"], t_dev, lens_dev, b, stream)
            state["ids"] = nxt
        else:
            model.replay(b)

    for _ in range(args.warmup):
        step()
    # Step duration by HIP events on the step's stream: one pair around the
    # timed steps, / steps.
    ev_a, ev_b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev_a.record(stream)
    for _ in range(args.steps):
        step()
    ev_b.record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    step_ms = ev_a.elapsed_time(ev_b) / args.steps
    per_step = e2e_step_bytes(cfg, lens, 2)
    achieved = per_step / (step_ms * 1e-3) / 1e9
    result = {
        "metric": f"whole decode step tokens/sec at {factory} shape, 1 GPU",
        "value": b * args.steps / elapsed, "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": elapsed * 1e3 / args.steps, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: random-init weights of the architecture, N(0,1) cached K/V, "
                "seeded random page permutation",
        "config": {"workload": desc, "batch": b, "layers": cfg.layers,
                   "mean_keys": float(np.mean(lens)), "pages_per_layer": need,
                   "launch": "host calls per op" if args.eager else "HIP graph replay",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS, "traffic": None,
                     "kernel": "whole step (all launches of DecodeModel.step)",
                     "bytes_per_step": per_step, "avg_step_ms": step_ms,
                     "timed_steps": args.steps},
        "cpu_baseline": None,
    }
    model.close()
    if not args.no_cpu:
        result["cpu_baseline"] = e2e_cpu_baseline(args, cfg, cached)
    print(json.dumps(result))


def e2e_cpu_baseline(args, cfg, cached):
    """The oracle's model_step_ref in f32 (the reference CPU path's dtype:
    numpy products, the C restatement of the attention) for one step of a
    bounded subset of the batch's sequences, with the same cached lengths."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    spec = O.ModelSpec(cfg.hidden, cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim,
                       cfg.inter, cfg.vocab, cfg.eps, cfg.theta, cfg.qk_norm, cfg.qkv_bias,
                       cfg.tied)
    rng = np.random.default_rng(7)
    w = O.random_weights(spec, rng, "f32")
    sub = [int(n) for n in cached[:4]]
    tile = rng.standard_normal((cfg.kv_heads, 1, cfg.head_dim)).astype(np.float32)
    kc = [[np.ascontiguousarray(np.broadcast_to(tile, (cfg.kv_heads, n, cfg.head_dim)))
           for n in sub] for _ in range(cfg.layers)]
    vc = [[x.copy() for x in row] for row in kc]
    max_steps = 5
    cos_t, sin_t = O.rope_tables_f32(cfg.theta, cfg.head_dim, max(sub) + max_steps + 1)
    ids = list(rng.integers(0, cfg.vocab, len(sub)))
    steps, t0 = 0, time.perf_counter()
    while True:
        O.model_step_ref(spec, w, ids, kc, vc, cos_t, sin_t, "f32")
        steps += 1
        el = time.perf_counter() - t0
        if el >= args.cpu_seconds or steps >= max_steps:
            break
    return {"value": len(sub) * steps / el, "unit": "tokens/s", "cores": O.max_threads(),
            "nproc": os.cpu_count(), "impl": ORACLE_IMPL,
            "kind": "port",
            "sample": f"{steps} whole step(s) of {len(sub)} of the sequences (cached "
                      f"{sub}), f32, in {el:.2f} s"}


# Whether the model of each attention workload has per-head q_norm / k_norm
# (Qwen3 does; Qwen2.5 does not: Config.q_norm is absent for it,
# src/backends/qwen2.rs:251-260). RoPE applies to every workload.
WORKLOAD_QK_NORM = {"qwen3": True, "qwen25": False, "qwen3_8b": True, "qwen25_7b": False}


def decode_layout(workload, seed):
    """Host side of an attention workload: cached lengths U[lo, hi], keys
    attended = cached + 1 (the token appended this step), and block tables
    drawing each sequence's pages from one seeded random permutation."""
    import numpy as np
    hq, hkv, d, layers, b, lo, hi, _ = WORKLOADS[workload]
    rng = np.random.default_rng(seed)
    cached = rng.integers(lo, hi + 1, b).astype(np.int32)
    lens = cached + 1  # keys attended: cached + the appended token
    mbps = int(max((int(n) + 15) // 16 for n in lens))
    need = int(sum((int(n) + 15) // 16 for n in lens))
    nb = need + 64
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.zeros((b, mbps), np.int32)
    used = 0
    for i, n in enumerate(lens):
        k = (int(n) + 15) // 16
        tables[i, :k] = perm[used:used + k]
        used += k
    return cached, lens, tables, mbps, need, nb


def decode_inputs(workload, seed, dev, layers=None):
    """Every buffer of an attention workload, resident on dev: the layout of
    decode_layout, a distinct N(0,1) K/V pool per layer, each layer's q and
    new-token k/v, q/k RMSNorm weights 1 + 0.1 N(0,1) where the model has
    them (None otherwise) and the bf16 RoPE tables (theta 1e6) for every
    position a table can hold. layers: how many layers to build (default:
    all of the workload's; a layer's buffers are drawn together, layer by
    layer, so the first layers do not depend on it)."""
    import torch
    import rlse_kv as kv
    hq, hkv, d, n_layers, b, _, _, _ = WORKLOADS[workload]
    n_layers = n_layers if layers is None else layers
    cached, lens, tables, mbps, need, nb = decode_layout(workload, seed)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    bf = torch.bfloat16
    k_pools, v_pools, q_in, k_in, v_in, qw, kw = [], [], [], [], [], [], []
    for _ in range(n_layers):   # layer by layer: a layer's draws do not depend on n_layers
        k_pools.append(torch.randn((nb, hkv, 16, d), generator=g, device=dev, dtype=bf))
        v_pools.append(torch.randn((nb, hkv, 16, d), generator=g, device=dev, dtype=bf))
        q_in.append(torch.randn((b, hq, d), generator=g, device=dev, dtype=bf))
        k_in.append(torch.randn((b, hkv, d), generator=g, device=dev, dtype=bf))
        v_in.append(torch.randn((b, hkv, d), generator=g, device=dev, dtype=bf))
        qw.append((1 + 0.1 * torch.randn(d, generator=g, device=dev)).to(bf))
        kw.append((1 + 0.1 * torch.randn(d, generator=g, device=dev)).to(bf))
    if not WORKLOAD_QK_NORM[workload]:
        qw = kw = [None] * n_layers
    max_pos = mbps * 16  # every position the block tables can hold
    cos_b, sin_b = kv.rope_tables(1e6, d, max_pos, "bf16")
    cos_t = torch.frombuffer(bytearray(cos_b), dtype=torch.int16).to(dev).view(bf)
    sin_t = torch.frombuffer(bytearray(sin_b), dtype=torch.int16).to(dev).view(bf)
    return {"cached": cached, "lens": lens, "tables": tables, "mbps": mbps, "pages": need,
            "num_blocks": nb, "k_pools": k_pools, "v_pools": v_pools, "q": q_in, "k_new": k_in,
            "v_new": v_in, "q_norm": qw, "k_norm": kw, "cos": cos_t, "sin": sin_t,
            "cos_bytes": cos_b, "sin_bytes": sin_b, "max_pos": max_pos}


def main():
    args = parse()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the library has no multi-GPU path); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)
    if args.timeline:
        timeline_bench(args)
        return
    if args.workload in PREFILL:
        prefill_bench(args)
        return
    if args.workload in FORK:
        fork_bench(args)
        return
    if args.workload in MIXED:
        mixed_bench(args)
        return
    if args.workload in E2E:
        e2e_bench(args)
        return
    import numpy as np
    import torch

    import rlse_kv as kv

    hq, hkv, d, layers, b, lo, hi, desc = WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    w = decode_inputs(args.workload, args.seed, dev)
    lens, cached, tables, mbps, need, nb = (w["lens"], w["cached"], w["tables"], w["mbps"],
                                            w["pages"], w["num_blocks"])
    k_pools, v_pools, q_in, k_in, v_in = w["k_pools"], w["v_pools"], w["q"], w["k_new"], w["v_new"]
    qw, kw, cos_t, sin_t, max_pos = w["q_norm"], w["k_norm"], w["cos"], w["sin"], w["max_pos"]
    bf = torch.bfloat16
    t_dev = torch.from_numpy(tables).to(dev)
    pos_dev = torch.from_numpy(cached).to(dev)
    lens_dev = torch.from_numpy(lens).to(dev)
    q_rot = torch.empty((b, hq, d), device=dev, dtype=bf)
    out = torch.empty((b, hq, d), device=dev, dtype=bf)
    ws_bytes = kv.decode_workspace_size(b, hq, hkv, d)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)  # zero-filled before first use
    plan_bytes = kv.decode_plan_size()
    plan = torch.zeros(plan_bytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    scale = 1.0 / math.sqrt(d)
    # Decode-kernel duration by HIP events on the launch stream. Fused step:
    # one event pair around each timed step's `layers` back-to-back decode
    # launches (after the plan), recorded in the timed steps themselves; the
    # average per launch includes the gaps between launches but no
    # event-record stall inside a span. Two-launch mode: a pair around every
    # decode launch (the append kernel sits between them), in a second pass
    # so the timed steps carry no event between their launches.
    ev_steps = args.steps if not args.unfused else min(args.steps, 50)
    n_events = ev_steps if not args.unfused else layers * ev_steps
    ev_a = [torch.cuda.Event(enable_timing=True) for _ in range(n_events)]
    ev_b = [torch.cuda.Event(enable_timing=True) for _ in range(n_events)]

    def step(timed_index=None):
        if not args.unfused:
            # One plan per step (the tables and lengths of every layer).
            kv.decode_plan(t_dev, lens_dev, b, hkv, mbps, nb, plan, plan_bytes, stream)
            if timed_index is not None:
                ev_a[timed_index].record(stream)
        for layer in range(layers):
            if args.unfused:
                kv.qk_norm_rope_append(q_in[layer], k_in[layer], v_in[layer], qw[layer],
                                       kw[layer], 1e-6, cos_t, sin_t, max_pos, pos_dev, t_dev, b,
                                       None, b, hq, hkv, d, mbps, nb, q_rot, k_pools[layer],
                                       v_pools[layer], "bf16", stream)
                if timed_index is not None:
                    ev_a[timed_index * layers + layer].record(stream)
            if args.unfused:
                kv.paged_gqa_decode(q_rot, k_pools[layer], v_pools[layer], t_dev, lens_dev, out,
                                    b, hq, hkv, d, mbps, nb, scale, "bf16", ws, ws_bytes, stream)
            else:
                # The table is a permutation: no page is read by two rows, so the
                # pages stream (RLSE_DECODE_STREAM).
                kv.decode_step_planned(q_in[layer], k_in[layer], v_in[layer], qw[layer],
                                       kw[layer], 1e-6, cos_t, sin_t, max_pos, k_pools[layer],
                                       v_pools[layer], t_dev, lens_dev, out, b, hq, hkv, d, mbps,
                                       nb, scale, "bf16", plan, ws, ws_bytes, stream,
                                       stream_pages=True)
            if args.unfused and timed_index is not None:
                ev_b[timed_index * layers + layer].record(stream)
        if not args.unfused and timed_index is not None:
            ev_b[timed_index].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(None if args.unfused else i)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    if args.unfused:
        for i in range(ev_steps):
            step(i)
        torch.cuda.synchronize()
    spans = [a.elapsed_time(e) for a, e in zip(ev_a, ev_b)]
    avg_ms = float(np.mean(spans)) / (layers if not args.unfused else 1)
    per_launch = algorithmic_decode_bytes(lens, hq, hkv, d, 2, not args.unfused,
                                          WORKLOAD_QK_NORM[args.workload])
    achieved = per_launch / (avg_ms * 1e-3) / 1e9
    ms_per_step = elapsed * 1e3 / args.steps
    traffic, traffic_src = measured_traffic(args.workload, not args.unfused)
    result = {
        "metric": METRIC_NAME[args.workload],
        "value": b * args.steps / elapsed,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) K/V/q, seeded random page permutation",
        "config": {"workload": desc, "batch": b, "layers": layers, "q_heads": hq,
                   "kv_heads": hkv, "head_dim": d, "mean_keys": float(np.mean(lens)),
                   "pages_per_layer": need, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS, "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": ("decode_kernel (rlse_paged_gqa_decode)" if args.unfused else
                                "decode_kernel planned fused step (rlse_decode_step_planned, "
                                "streamed pages)"),
                     "bytes_per_launch": per_launch, "avg_launch_ms": avg_ms,
                     "timed_launches": ev_steps * layers,
                     "event_spans": ("one per timed step around its back-to-back decode "
                                     "launches" if not args.unfused else
                                     "one per decode launch, second pass")},
        "cpu_baseline": None,
    }
    result["read_ceiling"] = read_ceiling(kv, k_pools, v_pools, t_dev, lens_dev, lens, hkv, d,
                                          mbps, nb, layers, min(args.steps, 50), stream,
                                          None if args.unfused else plan)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(args, lens, hq, hkv, d, layers)
    print(json.dumps(result))


TIMELINE_POINTS = ["entry", "plan arrived", "first pages requested", "prologue barrier passed",
                   "prologue done", "first page computed", "streaming loop ended",
                   "group barrier passed", "own pieces combined", "records arrived", "finished"]


PREFIX_TIMELINE_POINTS = ["entry", "page ids and query loads issued", "first blocks requested",
                          "queries staged", "first block computed", "loop ended",
                          "waves' states combined", "slice state stored", "finished"]


def _spread(np, x):
    x = x[~np.isnan(x)]
    if not len(x):
        return None
    return {"n": int(len(x)), "min": round(float(x.min()), 2),
            "p10": round(float(np.percentile(x, 10)), 2),
            "median": round(float(np.median(x)), 2),
            "p90": round(float(np.percentile(x, 90)), 2), "max": round(float(x.max()), 2)}


def _decode_timeline(np, stamps, t0):
    """Summary of the decode launch's stamps (TIMELINE_POINTS, four waves a
    workgroup, two workgroups a compute unit), times in us from t0."""
    waves = int(np.nonzero(stamps[:, 0])[0].max()) + 1
    stamps = stamps[:waves]
    groups = waves // 4
    rel = np.where(stamps > 0, (stamps - t0) * 0.01, np.nan)  # us
    slot = (np.arange(waves) // 4) >= groups // 2
    points = {name: {"slot0": _spread(np, rel[~slot, k]), "slot1": _spread(np, rel[slot, k])}
              for k, name in enumerate(TIMELINE_POINTS)}
    P = {name: k for k, name in enumerate(TIMELINE_POINTS)}
    fin, loop_end = P["finished"], P["streaming loop ended"]
    # Phases up to the epilogue's barrier in order, then the epilogue's:
    # waves combining pieces of a row, the merging waves (records of earlier
    # groups), and the waves that publish or write without records.
    pairs = [(k - 1, k, None) for k in range(1, P["group barrier passed"] + 1)]
    merging = ~np.isnan(rel[:, P["records arrived"]])
    combining = ~np.isnan(rel[:, P["own pieces combined"]])
    pairs += [(P["group barrier passed"], P["own pieces combined"], None),
              (P["own pieces combined"], P["records arrived"], "merging waves"),
              (P["records arrived"], fin, "merging waves"),
              (P["own pieces combined"], fin, "publishing or writing waves"),
              (loop_end, fin, None)]
    phases = {}
    for a, b, who in pairs:
        sel = merging if who == "merging waves" else (combining & ~merging if who else
                                                      np.ones(waves, bool))
        name = f"{TIMELINE_POINTS[a]} -> {TIMELINE_POINTS[b]}" + (f" ({who})" if who else "")
        phases[name] = _spread(np, rel[sel, b] - rel[sel, a])
    last = int(np.nanargmax(rel[:, fin]))
    return {"launch_span_us": round(float(np.nanmax(rel[:, fin]) -
                                          np.nanmin(rel[:, P["entry"]])), 2),
            "waves": waves, "workgroups": groups, "points_us": points, "phases_us": phases,
            "last_loop_end_us": round(float(np.nanmax(rel[:, loop_end])), 2),
            "last_finisher": {"wave": last, "workgroup": last // 4, "wave_in_group": last % 4,
                              "points_us": {n: (None if np.isnan(rel[last, k]) else
                                                round(float(rel[last, k]), 2))
                                            for k, n in enumerate(TIMELINE_POINTS)}},
            "finish_by_wave_index": {f"wave{i}": _spread(np, rel[np.arange(waves) % 4 == i, fin])
                                     for i in range(4)}}


def _prefix_timeline(np, stamps):
    """Summary of the cascade prefix launch's stamps (PREFIX_TIMELINE_POINTS,
    eight waves a workgroup; waves without pages have none), times in us
    from the launch's first entry."""
    have = stamps[:, 0] > 0
    waves = int(np.nonzero(have)[0].max()) + 1
    stamps = stamps[:waves]
    t0 = stamps[stamps[:, 0] > 0, 0].min()
    rel = np.where(stamps > 0, (stamps - t0) * 0.01, np.nan)
    n = len(PREFIX_TIMELINE_POINTS)
    points = {name: _spread(np, rel[:, k]) for k, name in enumerate(PREFIX_TIMELINE_POINTS)}
    phases = {}
    for k in range(1, n):
        a = k - 1
        if k == 5:   # waves without blocks have no "first block computed"
            a = 3
            phases[f"{PREFIX_TIMELINE_POINTS[3]} -> {PREFIX_TIMELINE_POINTS[4]}"] = _spread(
                np, rel[:, 4] - rel[:, 3])
            phases[f"{PREFIX_TIMELINE_POINTS[4]} -> {PREFIX_TIMELINE_POINTS[5]}"] = _spread(
                np, rel[:, 5] - rel[:, 4])
            continue
        if k == 4:
            continue
        phases[f"{PREFIX_TIMELINE_POINTS[a]} -> {PREFIX_TIMELINE_POINTS[k]}"] = _spread(
            np, rel[:, k] - rel[:, a])
    last = int(np.nanargmax(rel[:, n - 1]))
    return {"launch_span_us": round(float(np.nanmax(rel[:, n - 1])), 2),
            "waves_with_stamps": int((~np.isnan(rel[:, 0])).sum()),
            "workgroups": (waves + 7) // 8, "points_us": points, "phases_us": phases,
            "last_finisher": {"wave": last, "workgroup": last // 8, "wave_in_group": last % 8,
                              "points_us": {nm: (None if np.isnan(rel[last, k]) else
                                                 round(float(rel[last, k]), 2))
                                            for k, nm in enumerate(PREFIX_TIMELINE_POINTS)}}}


def timeline_bench(args):
    """Per-phase timeline of a decode launch: the measurement build of the
    library (librlse_kv_timeline.so, RLSE_DECODE_TIMELINE) stamps the wall
    clock (100 MHz) in every wave at the points of TIMELINE_POINTS. After
    `warmup` steps of the workload (plan + one planned streamed launch per
    layer, as the bench times them), the stamps are cleared, one more step
    runs, and the last layer's launch is read back: for every point, the
    spread over the waves of each workgroup slot (slot 0: the first
    workgroup dispatched to a compute unit, 1: the second), in us from the
    launch's first entry, and each phase's duration per wave. A prefix-fork
    workload runs its cascade step (plan + prefix launch + decode launch per
    layer) and also reports the prefix launch's points
    (PREFIX_TIMELINE_POINTS), with the decode's times from the same origin
    as the prefix's first entry."""
    import ctypes
    lib = os.path.join(ROOT, "mini-serve-rs_amd", "librlse_kv_timeline.so")
    if not os.path.exists(lib):
        print("bench.py --timeline needs the measurement build: "
              "make -C mini-serve-rs_amd/csrc timeline", file=sys.stderr)
        sys.exit(2)
    if args.workload not in WORKLOADS and args.workload not in FORK:
        print(f"--timeline covers the attention workloads {sorted(WORKLOADS)} and the prefix "
              f"forks {sorted(FORK)}", file=sys.stderr)
        sys.exit(2)
    os.environ["RLSE_KV_LIB"] = lib
    import numpy as np
    import torch
    import rlse_kv as kv
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()
    plan_bytes = kv.decode_plan_size()
    plan = torch.zeros(plan_bytes, dtype=torch.uint8, device=dev)
    fork = args.workload in FORK
    if fork:
        hq, hkv, d, layers, b, plen, _, _, desc = FORK[args.workload]
        f = fork_inputs(args.workload, args.seed, dev)
        t_dev, mbps, nb = f["tables_dev"], f["mbps"], f["num_blocks"]
        lens_dev = torch.from_numpy(f["lens"].astype(np.int32)).to(dev)
        shared = plen // 16
        pre_bytes = kv.decode_prefix_size(b, hq, d, shared)
        pre = torch.zeros(pre_bytes, dtype=torch.uint8, device=dev)
        ptrs = [f["pool"].layer(layer) for layer in range(layers)]
    else:
        hq, hkv, d, layers, b, _, _, desc = WORKLOADS[args.workload]
        w = decode_inputs(args.workload, args.seed, dev)
        t_dev = torch.from_numpy(w["tables"]).to(dev)
        lens_dev = torch.from_numpy(w["lens"]).to(dev)
        mbps, nb = w["mbps"], w["num_blocks"]
    out = torch.empty((b, hq, d), device=dev, dtype=torch.bfloat16)
    ws_bytes = kv.decode_workspace_size(b, hq, hkv, d)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    lib_h = kv.load()
    fn = lib_h.rlse_decode_timeline
    fn.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
    fn.restype = ctypes.c_int

    def step():
        if fork:
            kv.decode_plan_cascade(t_dev, lens_dev, b, hkv, mbps, nb, shared, plan, plan_bytes,
                                   stream)
            for layer in range(layers):
                kv.decode_step_cascade(f["q"][layer], f["k_new"][layer], f["v_new"][layer],
                                       f["q_norm"], f["k_norm"], 1e-6, f["cos"], f["sin"],
                                       f["max_pos"], ptrs[layer][0], ptrs[layer][1], t_dev,
                                       lens_dev, out, b, hq, hkv, d, mbps, nb,
                                       1.0 / math.sqrt(d), "bf16", plan, shared, pre, pre_bytes,
                                       ws, ws_bytes, stream, stream_pages=True)
            return
        kv.decode_plan(t_dev, lens_dev, b, hkv, mbps, nb, plan, plan_bytes, stream)
        for layer in range(layers):
            kv.decode_step_planned(w["q"][layer], w["k_new"][layer], w["v_new"][layer],
                                   w["q_norm"][layer], w["k_norm"][layer], 1e-6, w["cos"],
                                   w["sin"], w["max_pos"], w["k_pools"][layer],
                                   w["v_pools"][layer], t_dev, lens_dev, out, b, hq, hkv, d,
                                   mbps, nb, 1.0 / math.sqrt(d), "bf16", plan, ws, ws_bytes,
                                   stream, stream_pages=True)

    for _ in range(max(args.warmup, 1)):
        step()
    torch.cuda.synchronize()
    n_dec = 8192 * len(TIMELINE_POINTS)
    buf = np.zeros(n_dec + 8192 * len(PREFIX_TIMELINE_POINTS), np.uint64)
    h_stream = ctypes.c_void_p(stream.cuda_stream)
    if fn(None, 0, 1, h_stream) != 0:
        raise RuntimeError("rlse_decode_timeline (clear) failed")
    step()
    torch.cuda.synchronize()
    if fn(buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes, 0, h_stream) != 0:
        raise RuntimeError("rlse_decode_timeline (read) failed")
    dec = buf[:n_dec].reshape(-1, len(TIMELINE_POINTS)).astype(np.int64)
    result = {"timeline": args.workload, "workload": desc}
    t0 = dec[dec[:, 0] > 0, 0].min()
    if fork:
        pst = buf[n_dec:].reshape(-1, len(PREFIX_TIMELINE_POINTS)).astype(np.int64)
        result["prefix"] = _prefix_timeline(np, pst)
        t0 = pst[pst[:, 0] > 0, 0].min()   # the decode's times from the prefix's first entry
    result.update(_decode_timeline(np, dec, t0))
    print(json.dumps(result))


def read_ceiling(kv, k_pools, v_pools, t_dev, lens_dev, lens, hkv, d, mbps, nb, layers, steps,
                 stream, plan=None):
    """The time a launch of the decode's shape needs just to read the
    decode's K/V bytes: rlse_kv_checksum (the decode's grid and page split,
    one page in flight per wave, no other work; with the decode's plan,
    rlse_kv_checksum_planned: each wave's first page requested from the plan,
    as the planned decode does) over every layer's pool with the same tables
    and lengths, timed like the decode (one event pair around a step's
    back-to-back launches). Its sums land in a zero-filled buffer per step
    (the fill outside the event pair)."""
    import numpy as np
    import torch
    b = len(lens)
    out = torch.zeros((b, hkv, 2), dtype=torch.int32, device=t_dev.device)

    def step():
        for layer in range(layers):
            kv.kv_checksum(k_pools[layer], v_pools[layer], t_dev, lens_dev, b, hkv, d, mbps, nb,
                           "bf16", out, stream, plan=plan)

    for _ in range(3):
        step()
    spans = []
    for _ in range(steps):
        out.zero_()
        a, z = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        step()
        z.record(stream)
        spans.append((a, z))
    torch.cuda.synchronize()
    avg_ms = float(np.mean([a.elapsed_time(z) for a, z in spans])) / layers
    kv_bytes = sum(int(n) * 2 * hkv * d * 2 for n in lens)
    read = kv_bytes + sum(((int(n) + 15) // 16) * 4 for n in lens) + 4 * b
    achieved = read / (avg_ms * 1e-3) / 1e9
    return {"kernel": ("checksum_kernel (rlse_kv_checksum%s: the decode's grid and page split, "
                       "one page in flight per wave, nothing else)"
                       % ("_planned, the decode's plan" if plan is not None else "")),
            "bytes_per_launch": read, "avg_launch_ms": avg_ms, "achieved": achieved,
            "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS, "timed_launches": steps * layers}


if __name__ == "__main__":
    main()
