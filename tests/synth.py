"""Seeded synthetic decoder checkpoints for parity tests.

Weights are N(0, std) from a splitmix64 counter stream turned into normals
by Box-Muller (float64, then rounded to f32 or to bf16 with round-to-
nearest-even); each tensor's stream is seeded from the case seed and the
tensor name. RMSNorm gammas are 1 (HF's initialisation; N(0, 0.02) gammas
would make every activation vanish). Prompts are uniform ids from the seed.
"""
from __future__ import annotations

import json
import zlib
from typing import Dict, List, Optional, Tuple

import numpy as np

from esp_amd.config import DecoderConfig
from oracle import st

GAMMA = np.uint64(0x9E3779B97F4A7C15)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def tensor_seed(seed: int, name: str) -> int:
    z = np.array([(seed * 0x100000001B3 + zlib.crc32(name.encode())) & ((1 << 64) - 1)],
                 dtype=np.uint64)
    with np.errstate(over="ignore"):
        return int(_mix(z + GAMMA)[0])


def normal(seed: int, n: int, std: float) -> np.ndarray:
    with np.errstate(over="ignore"):
        p = np.arange((n + 1) // 2, dtype=np.uint64)
        base = np.uint64(seed) + GAMMA * (np.uint64(2) * p)
        x1 = _mix(base + GAMMA)
        x2 = _mix(base + GAMMA + GAMMA)
    u1 = ((x1 >> np.uint64(11)).astype(np.float64) + 1.0) / 9007199254740992.0
    u2 = (x2 >> np.uint64(11)).astype(np.float64) / 9007199254740992.0
    r = np.sqrt(-2.0 * np.log(u1))
    t = 2.0 * np.pi * u2
    out = np.empty(2 * len(p), np.float64)
    out[0::2] = r * np.cos(t)
    out[1::2] = r * np.sin(t)
    return (out[:n] * std).astype(np.float32)


def uniform_ids(seed: int, n: int, vocab: int) -> List[int]:
    with np.errstate(over="ignore"):
        z = _mix(np.uint64(seed) + GAMMA * np.arange(1, n + 1, dtype=np.uint64))
    return [int(v % vocab) for v in z]


def make_tensors(cfg: DecoderConfig, seed: int, fmt: str = "f32", std: float = 0.02,
                 bias_std: float = 0.0, fast: bool = False) -> Dict[str, Tuple[np.ndarray, str]]:
    """HF-named tensors for `cfg` (dense, or qwen2_moe / Mixtral-style experts).

    fast=True draws the same splitmix64 / Box-Muller stream with the CPU
    oracle's OpenMP generator (glibc log/cos/sin instead of numpy's; the f32
    values can differ by an ulp, bf16 roundings almost never): for the
    full-width shapes, whose weights numpy would take minutes to draw."""
    H, F, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    qw, kvw, hd = cfg.query_width(), cfg.kv_heads() * cfg.head_dim(), cfg.head_dim()
    out: Dict[str, Tuple[np.ndarray, str]] = {}

    def put(name, shape, kind="w"):
        n = int(np.prod(shape))
        if kind == "one":
            arr = np.ones(n, np.float32)
        elif kind == "bias":
            arr = normal(tensor_seed(seed, name), n, bias_std) if bias_std else np.zeros(n, np.float32)
        elif fast:
            from oracle import oracle
            raw = oracle.fill_normal(tensor_seed(seed, name), n, std, fmt == "bf16")
            out[name] = (raw.reshape(shape), "BF16" if fmt == "bf16" else "F32")
            return
        else:
            arr = normal(tensor_seed(seed, name), n, std)
        arr = arr.reshape(shape)
        if fmt == "bf16":
            out[name] = (st.bf16_round(arr), "BF16")
        else:
            out[name] = (arr, "F32")

    put("model.embed_tokens.weight", (V, H))
    put("model.norm.weight", (H,), "one")
    if not cfg.tie_word_embeddings:
        put("lm_head.weight", (V, H))
    for l in range(cfg.num_hidden_layers):
        p = f"model.layers.{l}."
        put(p + "input_layernorm.weight", (H,), "one")
        put(p + "post_attention_layernorm.weight", (H,), "one")
        put(p + "self_attn.q_proj.weight", (qw, H))
        put(p + "self_attn.k_proj.weight", (kvw, H))
        put(p + "self_attn.v_proj.weight", (kvw, H))
        put(p + "self_attn.o_proj.weight", (H, qw))
        if cfg.qkv_bias():
            put(p + "self_attn.q_proj.bias", (qw,), "bias")
            put(p + "self_attn.k_proj.bias", (kvw,), "bias")
            put(p + "self_attn.v_proj.bias", (kvw,), "bias")
        if cfg.output_bias():
            put(p + "self_attn.o_proj.bias", (H,), "bias")
        if cfg.qk_norm():
            put(p + "self_attn.q_norm.weight", (hd,), "one")
            put(p + "self_attn.k_norm.weight", (hd,), "one")
        if cfg.layer_is_moe(l):
            m = cfg.moe
            put(p + "mlp.gate.weight", (m.num_experts, H))
            for e in range(m.num_experts):
                ep = p + f"mlp.experts.{e}."
                put(ep + "gate_proj.weight", (m.moe_intermediate_size, H))
                put(ep + "up_proj.weight", (m.moe_intermediate_size, H))
                put(ep + "down_proj.weight", (H, m.moe_intermediate_size))
            if m.shared_expert_intermediate_size:
                fs = m.shared_expert_intermediate_size
                put(p + "mlp.shared_expert_gate.weight", (1, H))
                put(p + "mlp.shared_expert.gate_proj.weight", (fs, H))
                put(p + "mlp.shared_expert.up_proj.weight", (fs, H))
                put(p + "mlp.shared_expert.down_proj.weight", (H, fs))
        else:
            put(p + "mlp.gate_proj.weight", (F, H))
            put(p + "mlp.up_proj.weight", (F, H))
            put(p + "mlp.down_proj.weight", (H, F))
    return out


def llama_config(layers: int, hidden: int, heads: int, kv_heads: int, ffn: int, vocab: int,
                 head_dim: Optional[int] = None, theta: float = 10000.0, max_pos: int = 2048,
                 extra: Optional[dict] = None) -> DecoderConfig:
    raw = {"architectures": ["LlamaForCausalLM"], "model_type": "llama",
           "hidden_size": hidden, "intermediate_size": ffn, "num_hidden_layers": layers,
           "num_attention_heads": heads, "num_key_value_heads": kv_heads,
           "max_position_embeddings": max_pos, "rms_norm_eps": 1e-5, "rope_theta": theta,
           "vocab_size": vocab, "tie_word_embeddings": False, "hidden_act": "silu"}
    if head_dim is not None:
        raw["head_dim"] = head_dim
    if extra:
        raw.update(extra)
    return DecoderConfig.from_json_bytes(json.dumps(raw).encode())


def tiny_llama_case(seed: int, layers: int, hidden: int, heads: int, kv_heads: int, ffn: int,
                    vocab: int, prompt_len: int, fmt: str = "f32", theta: float = 10000.0,
                    max_pos: int = 2048):
    cfg = llama_config(layers, hidden, heads, kv_heads, ffn, vocab, theta=theta, max_pos=max_pos)
    tensors = make_tensors(cfg, seed, fmt)
    blob = st.dump(tensors)
    prompt = uniform_ids(seed ^ 0xABCDEF, prompt_len, vocab)
    return cfg, tensors, blob, prompt


# BASELINE.json configs[0] (C1): tiny llama, fp32, N(0, 0.02), 2 layers,
# hidden 256, 4 heads (hd 64), ffn 688, eps 1e-5, theta 1e4, vocab 1024;
# 32-token prompt then 32 greedy steps.
def c1_case(seed: int = 2026):
    return tiny_llama_case(seed, layers=2, hidden=256, heads=4, kv_heads=4, ffn=688, vocab=1024,
                           prompt_len=32, fmt="f32", theta=10000.0, max_pos=128)
