"""Pins of the CPU oracle beyond the Transformers goldens: published
splitmix64 outputs, the reference's own sampler/mask/RoPE/GQA/cache
invariants, closed forms, and planted mistakes that the goldens must catch."""
import json
import math
import os

import numpy as np
import pytest

from esp_amd.config import DecoderConfig
from esp_amd.sample import Sampler, SplitMix64
from oracle import oracle, st
from tests import synth

ARCH = os.path.join(os.path.dirname(__file__), "golden", "arch")
REF = json.load(open(os.path.join(ARCH, "reference.json")))


def load_case(name):
    cfg = DecoderConfig.from_json_bytes(open(os.path.join(ARCH, name, "config.json"), "rb").read())
    return cfg, st.load(open(os.path.join(ARCH, name, "model.safetensors"), "rb").read())


# ------------------------------------------------------------- splitmix64

def test_splitmix64_published_vectors():
    """Vigna's reference splitmix64 (seed 0): first outputs."""
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    s = 0
    got = []
    for _ in range(4):
        v, s = oracle.splitmix64_next(s)
        got.append(v)
    assert got == want
    py = SplitMix64(0)
    assert [py.next_u64() for _ in range(4)] == want


def test_skip_draws_equals_stepping():
    """sample.rs:64-69"""
    st0 = 12345
    s = st0
    for _ in range(37):
        _, s = oracle.splitmix64_next(s)
    assert oracle.skip_draws(st0, 37) == s
    smp = Sampler(0.8, 0.9, st0)
    smp.skip_draws(37)
    assert smp.rng.state == s


# ---------------------------------------------------------------- sampler
LOGITS = [2.0, -1.0, 2.5, -3.0]


def test_sampler_same_seed_same_stream():
    def stream(seed):
        s, out = seed, []
        for _ in range(32):
            t, s = oracle.sample(LOGITS, 0.8, 0.9, s)
            out.append(t)
        return out
    assert stream(42) == stream(42)


def test_sampler_tiny_top_p_and_low_temperature_are_greedy():
    s = 7
    for _ in range(16):
        t, s = oracle.sample(LOGITS, 1.0, 1e-6, s)
        assert t == 2
    s = 7
    for _ in range(16):
        t, s = oracle.sample(LOGITS, 0.01, None, s)
        assert t == 2


def test_sampler_frequencies_track_distribution():
    s, counts = 1234, [0, 0, 0, 0]
    for _ in range(2000):
        t, s = oracle.sample(LOGITS, 1.0, None, s)
        counts[t] += 1
    assert counts[2] > counts[0] > counts[1] >= counts[3] and counts[2] + counts[0] > 1800


def test_sampler_matches_brute_force_inverse_cdf():
    """Independent restatement of sample.rs:83-121 in float32 numpy."""
    rng = np.random.default_rng(3)
    for trial in range(40):
        row = rng.normal(0, 2, 50).astype(np.float32)
        T, p, seed = np.float32(0.7 + trial % 3 * 0.3), [None, 0.9, 0.5][trial % 3], 99 + trial
        got, _ = oracle.sample(row, float(T), p, seed)
        inv_t = np.float32(1) / T
        w = np.exp((row - row.max()) * inv_t).astype(np.float32)
        order = sorted(range(50), key=lambda i: (-w[i], i))
        ws = [w[i] for i in order]
        keep = 50
        if p is not None:
            total = np.float32(0)
            for x in ws:
                total = np.float32(total + x)
            target = np.float32(total * np.float32(p))
            mass = np.float32(0)
            for k, x in enumerate(ws):
                mass = np.float32(mass + x)
                if mass >= target:
                    keep = k + 1
                    break
        tot = np.float32(0)
        for x in ws[:keep]:
            tot = np.float32(tot + x)
        v, _ = oracle.splitmix64_next(seed)
        u = np.float32(np.float32((v >> 11) / float(1 << 53)) * tot)
        want = order[keep - 1]
        for k in range(keep):
            u = np.float32(u - ws[k])
            if u <= 0:
                want = order[k]
                break
        assert got == want


def test_mask_semantics():
    """constraint.rs:466-494: non-finite never wins; disallowed -> -inf."""
    bits = np.zeros(8, np.uint32)
    bits[0] = (1 << 3) | (1 << 5)
    for bad in (np.nan, np.inf, -np.inf):
        row = np.zeros(256, np.float32)
        row[3] = bad
        row[5] = 2.0
        m, n = oracle.mask(row, bits)
        assert m[3] == -np.inf and n == 1 and oracle.argmax(m) == 5
    row = np.full(256, np.nan, np.float32)
    row[5] = np.inf
    m, n = oracle.mask(row, bits)
    assert n == 0 and np.all(m == -np.inf)
    assert oracle.argmax(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 1  # lowest id on ties


# ------------------------------------------------------------------- RoPE

def test_rope_table_closed_form():
    """attention.rs:491-516 (theta 1e4, hd 4) and the llama3 / linear rules
    of config.rs:158-180 against float64 math."""
    cfg = synth.llama_config(1, 8, 2, 2, 8, 8, head_dim=4, max_pos=8)
    cos, sin = oracle.rope_table(cfg, 8)
    assert abs(cos[1, 0] - math.cos(1.0)) < 1e-6 and abs(sin[1, 1] - math.sin(0.01)) < 1e-6
    assert cos[1, 2] == cos[1, 0] and sin[3, 3] == sin[3, 1]
    lin = synth.llama_config(1, 8, 2, 2, 8, 8, head_dim=4, max_pos=8,
                             extra={"rope_scaling": {"rope_type": "linear", "factor": 4.0}})
    lc, _ = oracle.rope_table(lin, 8)
    assert abs(lc[4, 0] - math.cos(1.0)) < 1e-6
    l3 = synth.llama_config(1, 64, 1, 1, 8, 8, head_dim=64, max_pos=4, theta=500000.0,
                            extra={"rope_scaling": {"rope_type": "llama3", "factor": 8.0,
                                                    "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                                                    "original_max_position_embeddings": 8192}})
    c3, s3 = oracle.rope_table(l3, 4)
    for i in range(32):
        f = 1.0 / 500000.0 ** (2 * i / 64)
        wl = 2 * math.pi / f
        if wl < 8192 / 4:
            g = f
        elif wl > 8192 / 1:
            g = f / 8
        else:
            sm = (8192 / wl - 1) / 3
            g = (1 - sm) * f / 8 + sm * f
        assert abs(s3[1, i] - math.sin(g)) < 2e-6, i


# ---------------------------------------------------- forward invariants

def det_model(kv_heads=2, tied=False):
    cfg = synth.llama_config(2, 32, 4, kv_heads, 48, 40, max_pos=32,
                             extra={"tie_word_embeddings": tied})
    return cfg, synth.make_tensors(cfg, 5, "f32", std=0.2)


def test_cached_blocks_equal_full_recompute():
    """model.rs:725-763"""
    cfg, t = det_model()
    m = oracle.OracleModel(cfg, t)
    tokens = [1, 4, 7, 2, 9, 3]
    _, full = m.forward_last(m.new_cache(), tokens, all_logits=True)
    for block in (1, 2, 3):
        kv = m.new_cache()
        rows = []
        for i in range(0, 6, block):
            _, a = m.forward_last(kv, tokens[i:i + block], all_logits=True)
            rows.append(a)
        assert np.abs(np.concatenate(rows) - full).max() < 1e-5


def test_causal_perturbation_changes_only_last_position():
    """attention.rs:518-562 at model level: change the last token."""
    cfg, t = det_model()
    m = oracle.OracleModel(cfg, t)
    _, a = m.forward_last(m.new_cache(), [3, 1, 4, 1, 5], all_logits=True)
    _, b = m.forward_last(m.new_cache(), [3, 1, 4, 1, 9], all_logits=True)
    assert np.abs(a[:4] - b[:4]).max() == 0.0 and np.abs(a[4] - b[4]).max() > 1e-6


def test_gqa_equals_mha_with_duplicated_kv():
    """attention.rs:575-627: kv head i serves query heads i*group .. (HF rule)."""
    cfg, t = det_model(kv_heads=2)
    mha_cfg = synth.llama_config(2, 32, 4, 4, 48, 40, max_pos=32)
    t2 = dict(t)
    hd = 8
    for l in range(2):
        for nm in ("k_proj", "v_proj"):
            key = f"model.layers.{l}.self_attn.{nm}.weight"
            w = t[key][0].reshape(2, hd, 32)
            t2[key] = (np.repeat(w, 2, axis=0).reshape(4 * hd, 32), "F32")
    a = oracle.OracleModel(cfg, t).forward_last(oracle.OracleModel(cfg, t).new_cache(), [1, 2, 3])
    mm = oracle.OracleModel(mha_cfg, t2)
    b = mm.forward_last(mm.new_cache(), [1, 2, 3])
    assert np.abs(a - b).max() < 1e-5


def test_tied_head_equals_explicit_transposed_embedding():
    """model.rs:787-813"""
    cfg, t = det_model(tied=True)
    untied_cfg, _ = det_model(tied=False)
    t2 = dict(t)
    t2["lm_head.weight"] = t["model.embed_tokens.weight"]
    a = oracle.OracleModel(cfg, t)
    b = oracle.OracleModel(untied_cfg, t2)
    assert np.array_equal(a.forward_last(a.new_cache(), [5, 6]), b.forward_last(b.new_cache(), [5, 6]))


def test_lora_merge_closed_form():
    """lora.rs:93-97: W + (A^T B^T) * scale, HF orientation W + s * B @ A."""
    rng = np.random.default_rng(0)
    base = rng.normal(0, 0.02, (24, 16)).astype(np.float32)
    a = rng.normal(0, 0.02, (4, 16)).astype(np.float32)
    b = rng.normal(0, 0.01, (24, 4)).astype(np.float32)
    merged = np.zeros_like(base)
    keep = []
    oracle.lib().orc_lora_merge(oracle._tensor(base, "F32", keep), a.ctypes.data, b.ctypes.data,
                                24, 16, 4, 2.0, merged.ctypes.data)
    assert np.abs(merged - (base + 2.0 * (b.astype(np.float64) @ a))).max() < 1e-7


def test_moe_routing_ties_go_to_lower_expert():
    """moe.rs:166: equal router probabilities -> lower expert id first. A zero
    router makes all experts tie, so top-2 must be experts 0 and 1: the
    output equals running experts 0 and 1 alone with weight 1/2 each."""
    raw = {"architectures": ["Qwen2MoeForCausalLM"], "model_type": "qwen2_moe", "hidden_size": 16,
           "intermediate_size": 24, "num_hidden_layers": 1, "num_attention_heads": 2,
           "num_key_value_heads": 1, "max_position_embeddings": 16, "vocab_size": 20,
           "num_experts": 4, "num_experts_per_tok": 2, "moe_intermediate_size": 8,
           "shared_expert_intermediate_size": 8, "norm_topk_prob": True}
    cfg = DecoderConfig.from_json_bytes(json.dumps(raw).encode())
    t = synth.make_tensors(cfg, 9, "f32", std=0.3)
    t["model.layers.0.mlp.gate.weight"] = (np.zeros((4, 16), np.float32), "F32")
    full = oracle.OracleModel(cfg, t)
    out = full.forward_last(full.new_cache(), [3, 4])
    t2 = dict(t)
    for e in (2, 3):  # replace experts 2, 3 by copies of 0, 1 -> identical if unused
        for nm in ("gate_proj", "up_proj", "down_proj"):
            t2[f"model.layers.0.mlp.experts.{e}.{nm}.weight"] = \
                t[f"model.layers.0.mlp.experts.{e - 2}.{nm}.weight"]
    alt = oracle.OracleModel(cfg, t2)
    assert np.array_equal(out, alt.forward_last(alt.new_cache(), [3, 4]))
    t3 = dict(t)
    for nm in ("gate_proj", "up_proj", "down_proj"):  # perturb a selected expert -> changes
        w, dt = t[f"model.layers.0.mlp.experts.1.{nm}.weight"]
        t3[f"model.layers.0.mlp.experts.1.{nm}.weight"] = (w * 1.5, dt)
    pert = oracle.OracleModel(cfg, t3)
    assert not np.array_equal(out, pert.forward_last(pert.new_cache(), [3, 4]))


# ------------------------------------------------------- planted mistakes

def golden_error(name, mutate_tensors=None, mutate_rope=None):
    cfg, t = load_case(name)
    row = next(c for c in REF["cases"] if c["name"] == name)
    if mutate_tensors:
        t = mutate_tensors(dict(t))
    m = oracle.OracleModel(cfg, t)
    if mutate_rope:
        mutate_rope(m)
    logits = m.forward_last(m.new_cache(), row["input_ids"])
    return float(np.abs(logits - np.array(row["last_logits"], np.float32)).max())


def test_planted_mistakes_fail_the_goldens():
    """Each plausible slip in the forward moves the golden logits past twice the
    2e-5 gate of architecture_tests.rs:237-248."""
    assert golden_error("llama") < 2e-5

    def neg_sin(m):  # wrong rotation direction
        s = np.ctypeslib.as_array(m.struct.rope_sin, shape=(256 * 8,))
        s *= -1.0
    assert golden_error("llama", mutate_rope=neg_sin) > 4e-5

    def adjacent_pairs(m):  # burn's adjacent-pair rotary instead of split-half
        c = np.ctypeslib.as_array(m.struct.rope_cos, shape=(256, 8))
        c[:] = c[:, [0, 4, 1, 5, 2, 6, 3, 7]]
    assert golden_error("llama", mutate_rope=adjacent_pairs) > 4e-5

    def swap_gate_up(t):  # silu on the wrong side of SwiGLU
        for l in range(2):
            g, u = f"model.layers.{l}.mlp.gate_proj.weight", f"model.layers.{l}.mlp.up_proj.weight"
            t[g], t[u] = t[u], t[g]
        return t
    assert golden_error("llama", mutate_tensors=swap_gate_up) > 4e-5

    def transpose_o(t):  # o_proj applied transposed
        for l in range(2):
            k = f"model.layers.{l}.self_attn.o_proj.weight"
            t[k] = (np.ascontiguousarray(t[k][0].T), t[k][1])
        return t
    assert golden_error("llama", mutate_tensors=transpose_o) > 4e-5

    def drop_bias(t):  # qwen2 q/k/v biases dropped
        for l in range(2):
            for nm in ("q_proj", "k_proj", "v_proj"):
                k = f"model.layers.{l}.self_attn.{nm}.bias"
                t[k] = (np.zeros_like(t[k][0]), t[k][1])
        return t
    assert golden_error("qwen2", mutate_tensors=drop_bias) > 4e-5

    def no_shared_expert(t):
        for l in range(2):
            k = f"model.layers.{l}.mlp.shared_expert.down_proj.weight"
            t[k] = (np.zeros_like(t[k][0]), t[k][1])
        return t
    assert golden_error("qwen2_moe", mutate_tensors=no_shared_expert) > 4e-5
