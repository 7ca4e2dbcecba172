"""A whole batched decode step of a Qwen2/Qwen3 decoder on the device.

Host-side mirror of ModelForCausalLM::step_decode_batch
(src/backends/qwen2.rs:628-764) over the paged KV pool: every op of the step
is a C-ABI call into librlse_kv.so on one stream, so the activations, the
logits and the greedy next tokens stay in HBM, and the tokens of one step
feed the next without a host round trip (the reference copies the logits to
the host for sample_token, src/backends/candle.rs:737-751).

Per step, for a batch of B sequences with their new token at position
seq_lens[b] - 1:

    x = embed_tokens[ids]                                  rlse_embedding
    h = input_layernorm(x)                                 rlse_rmsnorm (layer 0)
    per layer:
      q, k, v = q/k/v_proj(h)                              rlse_linear x 3
      attn = q/k norm + RoPE + append + paged GQA decode    rlse_decode_step
      x, h = x + o_proj(attn), post_attention_layernorm     rlse_linear, rlse_add_rmsnorm
      a = silu(gate_proj(h)) * up_proj(h)                  rlse_linear (gate|up), rlse_silu_mul
      x, h = x + down_proj(a), next input_layernorm        rlse_linear, rlse_add_rmsnorm
             (the final norm after the last layer)
    logits = lm_head(h); next = argmax(logits)             rlse_linear, rlse_argmax

gate_proj and up_proj run as one product over their stacked weights (each
output element is the same dot product, rounded once). torch is used only to
hold device memory; nothing here computes on the CPU or through torch ops.
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
                 num_blocks: int, max_batch: int, max_blocks_per_seq: int, device="cuda:0"):
        if dtype not in _TORCH:
            raise ValueError(f"dtype {dtype!r}")
        kv.load()
        self.cfg, self.dtype, self.device = cfg, dtype, torch.device(device)
        self.max_batch, self.mbps, self.num_blocks = max_batch, max_blocks_per_seq, num_blocks
        dev = self.device
        up = lambda name: _to_device(weights[name], dtype, dev)  # noqa: E731
        self.embed = up("embed")
        self.norm = up("norm")
        self.lm_head = self.embed if cfg.tied else up("lm_head")
        self.layers = []
        for l in range(cfg.layers):
            p = f"l{l}."
            L = {n: up(p + n) for n in ("in_norm", "post_norm", "q_w", "k_w", "v_w", "o_w",
                                        "down_w")}
            L["gate_up_w"] = torch.cat([up(p + "gate_w"), up(p + "up_w")], 0).contiguous()
            for n in ("q_b", "k_b", "v_b") if cfg.qkv_bias else ():
                L[n] = up(p + n)
            for n in ("q_norm", "k_norm") if cfg.qk_norm else ():
                L[n] = up(p + n)
            self.layers.append(L)

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
        self.x, self.h, self.o = z(B, cfg.hidden), z(B, cfg.hidden), z(B, cfg.hidden)
        self.q, self.k, self.v, self.attn = z(B, nq), z(B, nkv), z(B, nkv), z(B, nq)
        self.gu, self.act = z(B, 2 * cfg.inter), z(B, cfg.inter)
        self.logits = z(B, cfg.vocab)
        self.next_ids = torch.zeros(B, dtype=torch.int32, device=dev)
        ws = kv.decode_workspace_size(B, cfg.heads, cfg.kv_heads, cfg.head_dim)
        # Zero once: every launch of the decode kernel leaves it zero again.
        self.workspace = torch.zeros(max(ws, 1), dtype=torch.uint8, device=dev)
        self.scale = 1.0 / math.sqrt(cfg.head_dim)

    def close(self) -> None:
        if getattr(self, "pool", None) is not None:
            torch.cuda.synchronize(self.device)
            self.pool.close()
            self.pool = None

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
        kv.embedding(ids, self.embed, self.x, batch, H, cfg.vocab, dt, stream)
        kv.rmsnorm(self.x, self.layers[0]["in_norm"], self.h, batch, H, cfg.eps, dt, stream)
        for l, L in enumerate(self.layers):
            kv.linear(self.h, L["q_w"], L.get("q_b"), self.q, batch, nq, H, dt, stream)
            kv.linear(self.h, L["k_w"], L.get("k_b"), self.k, batch, nkv, H, dt, stream)
            kv.linear(self.h, L["v_w"], L.get("v_b"), self.v, batch, nkv, H, dt, stream)
            kp, vp = self.pool.layer(l)
            kv.decode_step(self.q, self.k, self.v, L.get("q_norm"), L.get("k_norm"), cfg.eps,
                           self.cos, self.sin, self.max_pos, kp, vp, block_tables, seq_lens,
                           self.attn, batch, cfg.heads, cfg.kv_heads, cfg.head_dim, self.mbps,
                           self.num_blocks, self.scale, dt, self.workspace,
                           self.workspace.numel(), stream)
            kv.linear(self.attn, L["o_w"], None, self.o, batch, H, nq, dt, stream)
            kv.add_rmsnorm(self.o, self.x, L["post_norm"], self.h, batch, H, cfg.eps, dt, stream)
            kv.linear(self.h, L["gate_up_w"], None, self.gu, batch, 2 * cfg.inter, H, dt,
                      stream)
            kv.silu_mul(self.gu, self.act, batch, cfg.inter, dt, stream)
            kv.linear(self.act, L["down_w"], None, self.o, batch, H, cfg.inter, dt, stream)
            nxt = self.layers[l + 1]["in_norm"] if l + 1 < cfg.layers else self.norm
            kv.add_rmsnorm(self.o, self.x, nxt, self.h, batch, H, cfg.eps, dt, stream)
        kv.linear(self.h, self.lm_head, None, self.logits, batch, cfg.vocab, H, dt, stream)
        kv.argmax(self.logits, self.next_ids, batch, cfg.vocab, dt, stream)
        return self.logits[:batch], self.next_ids[:batch]
