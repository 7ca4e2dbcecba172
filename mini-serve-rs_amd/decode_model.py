"""A whole batched decode step of a Qwen2/Qwen3 decoder on the device.

Host-side mirror of ModelForCausalLM::step_decode_batch
(src/backends/qwen2.rs:628-764) over the paged KV pool: every op of the step
is a C-ABI call into librlse_kv.so on one stream, so the activations, the
logits and the greedy next tokens stay in HBM, and the tokens of one step
feed the next without a host round trip (the reference copies the logits to
the host for sample_token, src/backends/candle.rs:737-751).

Per step, for a batch of B sequences with their new token at position
seq_lens[b] - 1 (bf16 / f16: the projections on the MFMA kernels, fused with
their neighbours):

    x = embed_tokens[ids]                                  rlse_embedding
    h = input_layernorm(x)                                 rlse_add_rmsnorm (no add)
    the step's decode plan (page ids per wave)             rlse_decode_plan
    per layer:
      q, k, v = q/k/v_proj(h)                              rlse_qkv_proj (one launch)
      attn = q/k norm + RoPE + append + paged GQA decode    rlse_decode_step_planned
      x += o_proj(attn)                                    rlse_linear_residual
      h = post_attention_layernorm(x)                      rlse_add_rmsnorm (no add)
      a = silu(gate_proj(h)) * up_proj(h)                  rlse_gate_up_silu
      x += down_proj(a)                                    rlse_linear_residual
      h = next input_layernorm(x) (the final norm last)    rlse_add_rmsnorm (no add)
    logits = lm_head(h); next = argmax(logits)             rlse_linear, rlse_argmax

f32 (a parity dtype, not a performance one) runs the same math as separate
ops: rlse_linear per projection, rlse_add_rmsnorm for the residual adds and
rlse_silu_mul. Each output element is rounded at the same points either way
(the projection, the bias, the residual sum, each step of silu).
"""
from __future__ import annotations

import math
from typing import Dict, Optional

import numpy as np
import torch

import rlse_kv as kv

_TORCH = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


class ModelConfig:
    """The fields of the reference Config (qwen2.rs:10-52) the decode step reads."""

    def __init__(self, hidden, layers, heads, kv_heads, head_dim, inter, vocab, eps=1e-6,
                 theta=1e6, qk_norm=True, qkv_bias=False, tied=True):
        if heads % kv_heads:
            raise ValueError("num_attention_heads must be a multiple of num_key_value_heads")
        self.hidden, self.layers, self.heads, self.kv_heads = hidden, layers, heads, kv_heads
        self.head_dim, self.inter, self.vocab, self.eps = head_dim, inter, vocab, eps
        self.theta, self.qk_norm, self.qkv_bias, self.tied = theta, qk_norm, qkv_bias, tied

    @classmethod
    def from_config(cls, config: dict, tensors=()):
        """The decode step's fields from a config.json dict as the reference
        deserialises it (Config, qwen2.rs:9-54): serde defaults
        tie_word_embeddings true, rope_theta 1e6, rms_norm_eps 1e-6;
        head_dim = the explicit field, else hidden_size / num_attention_heads
        (Config::head_dim, :50-53). `tensors` holds the checkpoint's tensor
        names: q/k/v carry a bias when q_proj has one or attention_bias is
        true (:231-232), and q_norm/k_norm exist when the checkpoint has them
        (:251-260)."""
        heads, hidden = config["num_attention_heads"], config["hidden_size"]
        head_dim = config.get("head_dim")
        if head_dim is None:
            head_dim = hidden // heads
        names = set(tensors)
        has = lambda suffix: any(n.endswith(suffix) for n in names)  # noqa: E731
        return cls(hidden=hidden, layers=config["num_hidden_layers"], heads=heads,
                   kv_heads=config["num_key_value_heads"], head_dim=head_dim,
                   inter=config["intermediate_size"], vocab=config["vocab_size"],
                   eps=config.get("rms_norm_eps", 1e-6), theta=config.get("rope_theta", 1e6),
                   qk_norm=has("self_attn.q_norm.weight"),
                   qkv_bias=has("self_attn.q_proj.bias") or bool(config.get("attention_bias")),
                   tied=config.get("tie_word_embeddings", True))

    @property
    def groups(self) -> int:
        """Query heads per KV head (num_kv_groups, qwen2.rs:227)."""
        return self.heads // self.kv_heads

    @classmethod
    def qwen3_0_6b(cls):
        return cls(hidden=1024, layers=28, heads=16, kv_heads=8, head_dim=128, inter=3072,
                   vocab=151936, eps=1e-6, theta=1e6, qk_norm=True, qkv_bias=False, tied=True)

    @classmethod
    def qwen2_5_0_5b(cls):
        return cls(hidden=896, layers=24, heads=14, kv_heads=2, head_dim=64, inter=4864,
                   vocab=151936, eps=1e-6, theta=1e6, qk_norm=False, qkv_bias=True, tied=True)


def _to_device(a, dtype: str, device) -> torch.Tensor:
    if isinstance(a, torch.Tensor):
        return a.to(device=device, dtype=_TORCH[dtype]).contiguous()
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device).to(
        _TORCH[dtype]).contiguous()


class DecodeModel:
    """Weights, the paged KV pool and the step buffers of one decoder.

    weights: name -> array (numpy float32 holding values of the dtype, or
    torch tensors) with the names embed, norm, lm_head (absent when tied)
    and per layer ``l{i}.`` in_norm, post_norm, q_w, k_w, v_w, [q_b, k_b,
    v_b], [q_norm, k_norm], o_w, gate_w, up_w, down_w; linear weights are
    [out_features][in_features] as in the checkpoints.
    """

    def __init__(self, cfg: ModelConfig, weights: Dict[str, object], dtype: str,
                 num_blocks: int, max_batch: int, max_blocks_per_seq: int, device="cuda:0",
                 stream_pages: bool = False, packed_weights: bool = True):
        if dtype not in _TORCH:
            raise ValueError(f"dtype {dtype!r}")
        # RLSE_DECODE_STREAM for every step: the caller guarantees that no
        # page is read by two sequences (no forked prefixes), so attention
        # reads its pages with non-temporal loads.
        self.stream_pages = stream_pages
        kv.load()
        self.cfg, self.dtype, self.device = cfg, dtype, torch.device(device)
        self.max_batch, self.mbps, self.num_blocks = max_batch, max_blocks_per_seq, num_blocks
        dev = self.device
        up = lambda name: _to_device(weights[name], dtype, dev)  # noqa: E731
        self.embed = up("embed")
        self.norm = up("norm")
        self.lm_head = self.embed if cfg.tied else up("lm_head")
        self.fused = dtype != "f32"
        self.layers = []
        for l in range(cfg.layers):
            p = f"l{l}."
            L = {n: up(p + n) for n in ("in_norm", "post_norm", "o_w", "down_w")}
            L["gate_up_w"] = torch.cat([up(p + "gate_w"), up(p + "up_w")], 0).contiguous()
            qkv = [up(p + n) for n in ("q_w", "k_w", "v_w")]
            bias = [up(p + n) for n in ("q_b", "k_b", "v_b")] if cfg.qkv_bias else None
            if self.fused:
                L["qkv_w"] = torch.cat(qkv, 0).contiguous()
                L["qkv_b"] = torch.cat(bias, 0).contiguous() if bias else None
            else:
                L["q_w"], L["k_w"], L["v_w"] = qkv
                L["q_b"], L["k_b"], L["v_b"] = bias if bias else (None, None, None)
            for n in ("q_norm", "k_norm") if cfg.qk_norm else ():
                L[n] = up(p + n)
            self.layers.append(L)
        # 16-bit steps: the projection weights in the tile order of the MFMA
        # kernel (rlse_dense_pack), bit-identical results with one contiguous
        # KiB per operand load; lm_head too when its shape allows.
        self.packed = self.fused and packed_weights
        self.lm_packed = (self.packed and cfg.vocab % 16 == 0 and cfg.hidden % 32 == 0)
        self.act_packed = self.packed and cfg.inter % 32 == 0
        if self.packed:
            nq, nkv = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
            shapes = {"qkv_w": (nq + 2 * nkv, cfg.hidden, 0), "o_w": (cfg.hidden, nq, 0),
                      "gate_up_w": (2 * cfg.inter, cfg.hidden, cfg.inter),
                      "down_w": (cfg.hidden, cfg.inter, 0)}
            for L in self.layers:
                for n, (rows, cols, pair) in shapes.items():
                    w = torch.empty_like(L[n])
                    kv.dense_pack(L[n], w, rows, cols, pair, dtype)
                    L[n] = w
            if self.lm_packed:
                w = torch.empty_like(self.lm_head)
                kv.dense_pack(self.lm_head, w, cfg.vocab, cfg.hidden, 0, dtype)
                self.lm_head = w
            torch.cuda.synchronize(dev)

        self.pool = kv.KVPool(cfg.layers, num_blocks, cfg.kv_heads, cfg.head_dim, dtype)
        self.max_pos = max_blocks_per_seq * kv.BLOCK_SIZE
        es = kv.DTYPE_SIZE[kv._dt(dtype)]
        cos_b, sin_b = kv.rope_tables(cfg.theta, cfg.head_dim, self.max_pos, dtype)
        self.cos = torch.frombuffer(bytearray(cos_b), dtype=torch.uint8).to(dev)
        self.sin = torch.frombuffer(bytearray(sin_b), dtype=torch.uint8).to(dev)
        assert self.cos.numel() == self.max_pos * cfg.head_dim // 2 * es

        B, t = max_batch, _TORCH[dtype]
        nq, nkv = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
        z = lambda *s: torch.zeros(s, dtype=t, device=dev)  # noqa: E731
        # h (the norms' output, the projections' input) holds whole 16-row
        # tiles: with packed weights it is written in packed row order.
        self.x, self.o = z(B, cfg.hidden), z(B, cfg.hidden)
        self.h = z((B + 15) // 16 * 16, cfg.hidden)
        self.q, self.k, self.v, self.attn = z(B, nq), z(B, nkv), z(B, nkv), z(B, nq)
        self.gu = None if self.fused else z(B, 2 * cfg.inter)
        self.act = z((B + 15) // 16 * 16, cfg.inter)  # whole 16-row tiles (packed rows)
        self.logits = z(B, cfg.vocab)
        self.next_ids = torch.zeros(B, dtype=torch.int32, device=dev)
        self.arg_ws = torch.zeros(max(kv.argmax_workspace_size(B, cfg.vocab), 8),
                                  dtype=torch.uint8, device=dev)
        # One workspace for the K split of every fused projection (they run
        # one after another on the step's stream); zero-filled once, then
        # kept consistent by the kernels (epoch-tagged records).
        dense_ws = max([kv.dense_workspace_size(B, n, k) for n, k in (
            (nq + 2 * nkv, cfg.hidden), (cfg.hidden, nq), (2 * cfg.inter, cfg.hidden),
            (cfg.hidden, cfg.inter))] + [4])
        self.dense_ws = torch.zeros(dense_ws, dtype=torch.uint8, device=dev)
        ws = kv.decode_workspace_size(B, cfg.heads, cfg.kv_heads, cfg.head_dim)
        # Zero once: the decode kernels keep it consistent from then on.
        self.workspace = torch.zeros(max(ws, 1), dtype=torch.uint8, device=dev)
        # The step's decode plan: built once per step, read by every layer.
        self.plan = torch.zeros(kv.decode_plan_size(), dtype=torch.uint8, device=dev)
        self.scale = 1.0 / math.sqrt(cfg.head_dim)
        self.layer_pools = [self.pool.layer(l) for l in range(cfg.layers)]
        # Inputs of captured steps: the graph reads them at these addresses.
        self.ids_in = torch.zeros(B, dtype=torch.int32, device=dev)
        self.tables_in = torch.zeros((B, max_blocks_per_seq), dtype=torch.int32, device=dev)
        self.lens_in = torch.zeros(B, dtype=torch.int32, device=dev)
        self.graphs = {}

    def check(self, stream=None) -> None:
        """Synchronises the stream, then reads and clears the sticky device
        error flags the step's kernels raise: a sequence longer than its
        block table (its rows come out as zeros) raises TokenLimitExceeded,
        a split-K merge that gave up waiting (its rows come out as NaN)
        raises DeviceTimeout -- the device-side failures a step can have,
        surfaced where the reference returns BackendError for a failed step
        (src/backends/candle.rs:689-696). step() and replay() do not check
        on their own (a check synchronises the host with the device): call
        this after the steps whose results are used -- after each eager
        step, or after a run of graph replays."""
        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        # both workspaces are read and cleared, whichever of them raises
        errs = []
        for ws in (self.workspace, self.dense_ws):
            try:
                kv.workspace_check(ws, stream)
            except kv.RlseError as e:
                errs.append(e)
        if errs:
            raise errs[0]

    def close(self) -> None:
        if getattr(self, "pool", None) is not None:
            torch.cuda.synchronize(self.device)
            self.graphs.clear()
            self.pool.close()
            self.pool = None

    # -- captured steps ------------------------------------------------------
    def capture(self, batch: int, feed_back: bool = True) -> None:
        """Records step(ids_in, tables_in, lens_in, batch) into a HIP graph
        (through torch.cuda.CUDAGraph): a replay issues the step's ~200
        launches at once instead of one host call each. With feed_back the
        graph ends by copying the greedy ids into ids_in, so successive
        replays decode greedily on the device alone. No launch of the step
        records a memset: the workspaces need no clearing between launches
        (their records carry a per-launch epoch)."""
        torch.cuda.synchronize(self.device)
        # One eager run first, outside the capture, with every length zero
        # (nothing is appended or attended), then the inputs are restored.
        saved = self.lens_in.clone()
        self.lens_in.zero_()
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self.step(self.ids_in, self.tables_in, self.lens_in, batch)
        torch.cuda.current_stream(self.device).wait_stream(side)
        self.lens_in.copy_(saved)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            _, nxt = self.step(self.ids_in, self.tables_in, self.lens_in, batch)
            if feed_back:
                self.ids_in[:batch].copy_(nxt)
        self.graphs[batch] = g

    def replay(self, batch: int):
        """Runs the step captured for `batch` on the current stream; returns
        views of its logits and greedy ids (as step does)."""
        self.graphs[batch].replay()
        return self.logits[:batch], self.next_ids[:batch]

    # -- KV snapshots (Attention::set_kv_snapshot / get_kv_snapshot) --------
    def set_kv(self, block_table, k, v, start: int = 0, stream=None) -> None:
        """Writes positions start.. of one sequence from contiguous K/V
        [layers][Hkv][len][head_dim] (qwen2.rs:373-377, 547-574)."""
        k, v = _to_device(k, self.dtype, self.device), _to_device(v, self.dtype, self.device)
        length = k.shape[2]
        kp, vp = self.pool.layer(0)
        kv.kv_scatter(k, v, kp, vp, self.pool.layer_stride_elems, self.cfg.layers,
                      block_table, start, length, self.cfg.kv_heads, self.cfg.head_dim,
                      self.num_blocks, self.dtype, stream)

    def get_kv(self, block_table, length: int, stream=None):
        """Contiguous K/V [layers][Hkv][length][head_dim] of one sequence."""
        shape = (self.cfg.layers, self.cfg.kv_heads, length, self.cfg.head_dim)
        k = torch.empty(shape, dtype=_TORCH[self.dtype], device=self.device)
        v = torch.empty_like(k)
        kp, vp = self.pool.layer(0)
        kv.kv_gather(kp, vp, self.pool.layer_stride_elems, self.cfg.layers, block_table, length,
                     k, v, self.cfg.kv_heads, self.cfg.head_dim, self.num_blocks, self.dtype,
                     stream)
        return k, v

    # -- the step ------------------------------------------------------------
    def step(self, ids, block_tables, seq_lens, batch: int, stream=None):
        """One decode step of `batch` sequences: ids int32 [batch] on the
        device; block_tables int32 [batch][max_blocks_per_seq] and seq_lens
        int32 [batch] (length including the new token) on the device. Returns
        views of the logits [batch][vocab] and the greedy next ids [batch]."""
        cfg, dt = self.cfg, self.dtype
        if not 0 < batch <= self.max_batch:
            raise ValueError(f"batch {batch} outside 1..{self.max_batch}")
        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        H, nq, nkv = cfg.hidden, cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
        inter = cfg.inter
        kv.embedding(ids, self.embed, self.x, batch, H, cfg.vocab, dt, stream)
        kv.add_rmsnorm(None, self.x, self.layers[0]["in_norm"], self.h, batch, H, cfg.eps, dt,
                       stream, packed_out=self.packed if cfg.layers else self.lm_packed)
        kv.decode_plan(block_tables, seq_lens, batch, cfg.kv_heads, self.mbps, self.num_blocks,
                       self.plan, self.plan.numel(), stream)
        for l, L in enumerate(self.layers):
            if self.fused:
                kv.qkv_proj(self.h, L["qkv_w"], L["qkv_b"], self.q, self.k, self.v, batch, H, nq,
                            nkv, dt, self.dense_ws, stream, packed=self.packed,
                            packed_x=self.packed)
            else:
                kv.linear(self.h, L["q_w"], L["q_b"], self.q, batch, nq, H, dt, stream)
                kv.linear(self.h, L["k_w"], L["k_b"], self.k, batch, nkv, H, dt, stream)
                kv.linear(self.h, L["v_w"], L["v_b"], self.v, batch, nkv, H, dt, stream)
            kp, vp = self.layer_pools[l]
            kv.decode_step_planned(self.q, self.k, self.v, L.get("q_norm"), L.get("k_norm"),
                                   cfg.eps, self.cos, self.sin, self.max_pos, kp, vp,
                                   block_tables, seq_lens, self.attn, batch, cfg.heads,
                                   cfg.kv_heads, cfg.head_dim, self.mbps, self.num_blocks,
                                   self.scale, dt, self.plan, self.workspace,
                                   self.workspace.numel(), stream,
                                   stream_pages=self.stream_pages)
            nxt = self.layers[l + 1]["in_norm"] if l + 1 < cfg.layers else self.norm
            if self.fused:
                kv.linear_residual(self.attn, L["o_w"], self.x, batch, H, nq, dt, self.dense_ws,
                                   stream, packed=self.packed)
                kv.add_rmsnorm(None, self.x, L["post_norm"], self.h, batch, H, cfg.eps, dt,
                               stream, packed_out=self.packed)
                kv.gate_up_silu(self.h, L["gate_up_w"], self.act, batch, H, inter, dt,
                                self.dense_ws, stream, packed=self.packed, packed_x=self.packed,
                                packed_out=self.act_packed)
                kv.linear_residual(self.act, L["down_w"], self.x, batch, H, inter, dt,
                                   self.dense_ws, stream, packed=self.packed,
                                   packed_x=self.act_packed)
                # lm_head reads the final norm packed only if it runs on the
                # MFMA kernel (vocab a multiple of 16)
                last = l + 1 == cfg.layers
                kv.add_rmsnorm(None, self.x, nxt, self.h, batch, H, cfg.eps, dt, stream,
                               packed_out=self.lm_packed if last else self.packed)
            else:
                kv.linear(self.attn, L["o_w"], None, self.o, batch, H, nq, dt, stream)
                kv.add_rmsnorm(self.o, self.x, L["post_norm"], self.h, batch, H, cfg.eps, dt,
                               stream)
                kv.linear(self.h, L["gate_up_w"], None, self.gu, batch, 2 * inter, H, dt,
                          stream)
                kv.silu_mul(self.gu, self.act, batch, inter, dt, stream)
                kv.linear(self.act, L["down_w"], None, self.o, batch, H, inter, dt, stream)
                kv.add_rmsnorm(self.o, self.x, nxt, self.h, batch, H, cfg.eps, dt, stream)
        kv.linear(self.h, self.lm_head, None, self.logits, batch, cfg.vocab, H, dt, stream,
                  packed=self.lm_packed, packed_x=self.lm_packed)
        kv.argmax(self.logits, self.next_ids, batch, cfg.vocab, dt, self.arg_ws,
                  self.arg_ws.numel(), stream)
        return self.logits[:batch], self.next_ids[:batch]
