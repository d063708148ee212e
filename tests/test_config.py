"""DecoderConfig mirror vs the reference's own config tests
(crates/esp/src/infer/decoder/config.rs:573-839)."""
import json

import pytest

from esp_amd.config import DecoderConfig, RopeScaling
from esp_amd.errors import InvalidConfig, Unsupported

TINYLLAMA = {
    "architectures": ["LlamaForCausalLM"], "hidden_act": "silu", "hidden_size": 2048,
    "intermediate_size": 5632, "max_position_embeddings": 2048, "model_type": "llama",
    "num_attention_heads": 32, "num_hidden_layers": 22, "num_key_value_heads": 4,
    "rms_norm_eps": 1e-05, "rope_theta": 10000.0, "tie_word_embeddings": False,
    "torch_dtype": "bfloat16", "eos_token_id": 2, "vocab_size": 32000,
}


def parse(d):
    return DecoderConfig.from_json_bytes(json.dumps(d).encode())


def tiny_with(extra):
    base = {"vocab_size": 32, "hidden_size": 8, "intermediate_size": 16,
            "num_hidden_layers": 2, "num_attention_heads": 4, "num_key_value_heads": 2,
            "max_position_embeddings": 16}
    base.update(extra)
    return base


def refused_field(extra):
    with pytest.raises(Unsupported) as e:
        parse(tiny_with(extra))
    return e.value.feature


def test_parses_real_tinyllama_config():
    c = parse(TINYLLAMA)
    assert (c.hidden_size, c.num_hidden_layers, c.kv_heads(), c.head_dim(), c.kv_group_size()) == \
        (2048, 22, 4, 64, 8)
    assert not c.tie_word_embeddings and c.eos_token_id == [2]


def test_eos_list_and_mha_fallback_and_defaults():
    c = parse({"vocab_size": 32, "hidden_size": 8, "intermediate_size": 16,
               "num_hidden_layers": 2, "num_attention_heads": 4, "max_position_embeddings": 16,
               "eos_token_id": [128001, 128008]})
    assert c.eos_token_id == [128001, 128008]
    assert c.kv_heads() == 4 and c.kv_group_size() == 1
    assert c.rms_norm_eps == 1e-5 and c.rope_theta == 10000.0


def test_real_llama_block_fields_are_accepted():
    parse(tiny_with({"architectures": ["LlamaForCausalLM"], "model_type": "llama",
                     "hidden_act": "silu", "rope_scaling": None, "attention_bias": False,
                     "mlp_bias": False, "head_dim": 2, "pretraining_tp": 1,
                     "sliding_window": None}))


def test_foreign_families_refused():
    assert refused_field({"model_type": "gemma2"}) == "config.model_type"
    assert refused_field({"architectures": ["GemmaForCausalLM"]}) == "config.architectures"
    with pytest.raises(Unsupported) as e:
        DecoderConfig.from_json_bytes(b'{"model_type": "llama", "text_config": {"hidden_size": 8}}')
    assert e.value.feature == "config.text_config"
    assert refused_field({"model_type": "qwen3", "architectures": ["LlamaForCausalLM"]}) == \
        "config.architectures"


def test_rope_scaling_validated():
    c = parse(tiny_with({"rope_scaling": {"rope_type": "llama3", "factor": 32.0,
                                          "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                                          "original_max_position_embeddings": 8192}}))
    assert isinstance(c.rope_scaling, RopeScaling) and c.rope_scaling.kind == "llama3"
    assert refused_field({"rope_scaling": {"rope_type": "yarn", "factor": 4}}) == "config.rope_scaling"
    assert refused_field({"rope_scaling": {"rope_type": "llama3", "factor": 4, "low_freq_factor": 4,
                                           "high_freq_factor": 1,
                                           "original_max_position_embeddings": 8192}}) == \
        "config.rope_scaling"
    assert refused_field({"rope_scaling": {"type": "linear", "rope_type": "llama3",
                                           "factor": 2}}) == "config.rope_scaling"
    assert refused_field({"rope_scaling": {"rope_type": "linear", "factor": 0.5}}) == \
        "config.rope_scaling"


def test_partial_rotary_and_width_checks():
    assert refused_field({"partial_rotary_factor": 0.75}) == "config.partial_rotary_factor"
    parse(tiny_with({"partial_rotary_factor": 1.0}))
    assert parse(tiny_with({"head_dim": 4})).query_width() == 16
    with pytest.raises(InvalidConfig):
        parse(tiny_with({"num_key_value_heads": 0}))
    with pytest.raises(InvalidConfig):
        parse(tiny_with({"num_key_value_heads": 3}))


def test_biases_windows_activation_capping_experts():
    assert parse(tiny_with({"attention_bias": True})).output_bias()
    assert refused_field({"mlp_bias": True}) == "config.mlp_bias"
    assert parse(tiny_with({"sliding_window": 8})).layer_window(0) == 8
    parse(tiny_with({"sliding_window": 8, "use_sliding_window": False}))
    assert refused_field({"layer_types": ["mystery", "full_attention"]}) == "config.layer_types"
    assert refused_field({"hidden_act": "gelu"}) == "config.hidden_act"
    assert refused_field({"hidden_activation": "gelu_pytorch_tanh"}) == "config.hidden_activation"
    parse(tiny_with({"hidden_act": "swish"}))
    assert refused_field({"attn_logit_softcapping": 50.0}) == "config.attn_logit_softcapping"
    assert refused_field({"final_logit_softcapping": 30.0}) == "config.final_logit_softcapping"
    for f in ("num_experts", "num_local_experts", "n_routed_experts", "num_experts_per_tok"):
        assert refused_field({f: 8}) == f"config.{f}"


def test_derived_geometry_of_families():
    q2 = parse(tiny_with({"model_type": "qwen2", "use_sliding_window": True, "sliding_window": 3,
                          "max_window_layers": 1}))
    assert q2.qkv_bias() and not q2.output_bias()
    assert q2.layer_window(0) is None and q2.layer_window(1) == 3
    q3 = parse(tiny_with({"model_type": "qwen3"}))
    assert q3.qk_norm()
    moe = parse(tiny_with({"model_type": "qwen2_moe", "num_experts": 4, "num_experts_per_tok": 2,
                           "moe_intermediate_size": 12, "shared_expert_intermediate_size": 20,
                           "decoder_sparse_step": 2, "mlp_only_layers": []}))
    assert [moe.layer_is_moe(i) for i in range(2)] == [False, True]
    with pytest.raises(Unsupported):
        parse(tiny_with({"model_type": "qwen2_moe", "num_experts": 4, "num_experts_per_tok": 5,
                         "moe_intermediate_size": 12, "shared_expert_intermediate_size": 20}))
    mx = DecoderConfig.mixtral_style(vocab_size=32, hidden_size=8, intermediate_size=16,
                                     num_hidden_layers=2, num_attention_heads=4,
                                     max_position_embeddings=16, num_experts=8,
                                     num_experts_per_tok=2, moe_intermediate_size=16)
    assert mx.moe.shared_expert_intermediate_size == 0 and mx.moe.norm_topk_prob
    assert all(mx.layer_is_moe(i) for i in range(2))
