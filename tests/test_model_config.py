"""ModelConfig.from_config against the reference's Config (qwen2.rs:9-54).

The fixtures are the configs the reference's own tests build
(tests/test_pretrained_numerics.rs:74-79, qwen2.rs:787-803) and the two
published model configs the decode step is measured on; each expectation is
what Config::head_dim (:50-53), the bias rule (:231-232) and the q_norm rule
(:251-260) give for it.
"""
import pytest

from decode_model import ModelConfig

QWEN3 = ["model.layers.0.self_attn.q_norm.weight", "model.layers.0.self_attn.k_norm.weight",
         "model.layers.0.self_attn.q_proj.weight"]
QWEN2 = ["model.layers.0.self_attn.q_proj.weight", "model.layers.0.self_attn.q_proj.bias"]


def test_reference_test_configs():
    # test_pretrained_numerics.rs:74-79: explicit head_dim, serde defaults
    c = ModelConfig.from_config({
        "hidden_size": 32, "intermediate_size": 64, "vocab_size": 64, "num_hidden_layers": 2,
        "num_attention_heads": 4, "num_key_value_heads": 2, "max_position_embeddings": 128,
        "head_dim": 8, "hidden_act": "silu", "attention_bias": False})
    assert (c.head_dim, c.groups, c.heads, c.kv_heads) == (8, 2, 4, 2)
    assert c.tied and c.theta == 1e6 and c.eps == 1e-6
    assert not c.qkv_bias and not c.qk_norm
    # qwen2.rs:787-803: head_dim Some(16) with hidden 64 / 4 heads, untied, theta 1e4
    c = ModelConfig.from_config({
        "hidden_size": 64, "intermediate_size": 128, "vocab_size": 100, "num_hidden_layers": 2,
        "num_attention_heads": 4, "num_key_value_heads": 2, "max_position_embeddings": 512,
        "tie_word_embeddings": False, "rope_theta": 10000.0, "rms_norm_eps": 1e-6,
        "hidden_act": "silu", "head_dim": 16, "attention_bias": False})
    assert (c.head_dim, c.groups, c.tied, c.theta) == (16, 2, False, 1e4)


def test_published_model_configs():
    # Qwen3-0.6B: head_dim 128 given explicitly although hidden / heads = 64
    q3 = ModelConfig.from_config({
        "hidden_size": 1024, "intermediate_size": 3072, "vocab_size": 151936,
        "num_hidden_layers": 28, "num_attention_heads": 16, "num_key_value_heads": 8,
        "max_position_embeddings": 40960, "head_dim": 128, "rope_theta": 1000000,
        "rms_norm_eps": 1e-06, "tie_word_embeddings": True, "attention_bias": False,
        "hidden_act": "silu"}, QWEN3)
    ref = ModelConfig.qwen3_0_6b()
    assert vars(q3) == vars(ref)
    assert q3.groups == 2
    # Qwen2.5-0.5B: no head_dim field (896 / 14 = 64), bias from the checkpoint
    q25 = ModelConfig.from_config({
        "hidden_size": 896, "intermediate_size": 4864, "vocab_size": 151936,
        "num_hidden_layers": 24, "num_attention_heads": 14, "num_key_value_heads": 2,
        "max_position_embeddings": 32768, "rope_theta": 1000000.0, "rms_norm_eps": 1e-06,
        "tie_word_embeddings": True, "hidden_act": "silu"}, QWEN2)
    assert vars(q25) == vars(ModelConfig.qwen2_5_0_5b())
    assert q25.groups == 7


def test_bias_and_norm_rules():
    base = {"hidden_size": 128, "intermediate_size": 256, "vocab_size": 10,
            "num_hidden_layers": 1, "num_attention_heads": 4, "num_key_value_heads": 4,
            "max_position_embeddings": 64, "hidden_act": "silu"}
    assert not ModelConfig.from_config(base).qkv_bias                      # absent -> false
    assert not ModelConfig.from_config(dict(base, attention_bias=None)).qkv_bias
    assert ModelConfig.from_config(dict(base, attention_bias=True)).qkv_bias
    assert ModelConfig.from_config(base, QWEN2).qkv_bias                  # from the checkpoint
    assert ModelConfig.from_config(base, QWEN3).qk_norm
    assert not ModelConfig.from_config(base, QWEN2).qk_norm
    assert ModelConfig.from_config(dict(base, head_dim=None)).head_dim == 32
    with pytest.raises(ValueError):                                        # 4 heads over 3
        ModelConfig.from_config(dict(base, num_key_value_heads=3))
