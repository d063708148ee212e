"""Routed experts through the grouped expert GEMMs: skewed routing (most
rows on one expert, several experts empty) against the oracle in both
weight formats, batched blocks of several sequences, and the router's
refusal reported by the forward (moe.rs:160-171) after the layers ran on
the device without a host round trip."""
from __future__ import annotations

import numpy as np
import pytest

from esp_amd import Backend, DecoderModel
from oracle import oracle, st
from tests import synth

pytestmark = pytest.mark.gpu

QWEN2_MOE = {"model_type": "qwen2_moe", "architectures": ["Qwen2MoeForCausalLM"],
             "num_experts": 12, "num_experts_per_tok": 2, "moe_intermediate_size": 160,
             "shared_expert_intermediate_size": 64, "norm_topk_prob": False,
             "decoder_sparse_step": 1}


def _close(got, want, fmt):
    if fmt == "bf16":
        return np.all(np.abs(got - want) <= 1e-2 + 2e-2 * np.abs(want))
    return np.all(np.abs(got - want) <= 1e-4 * float(np.abs(want).max()))


def _f32(arr, dt):
    return st.bf16_to_f32(arr) if dt == "BF16" else np.array(arr, np.float32, copy=True)


def _back(arr, dt):
    return st.bf16_round(arr) if dt == "BF16" else arr


def _skewed(fmt: str, seed: int):
    cfg = synth.llama_config(2, 256, 4, 2, 256, 700, head_dim=64, max_pos=1400, extra=QWEN2_MOE)
    tensors = synth.make_tensors(cfg, seed, fmt)
    for l in range(cfg.num_hidden_layers):
        name = f"model.layers.{l}.mlp.gate.weight"
        r, dt = tensors[name]
        r = _f32(r, dt)
        r[3] *= 40.0      # expert 3 wins nearly every row
        r[7:] *= 0.01     # experts 7.. almost never chosen
        tensors[name] = (_back(r, dt), dt)
    return cfg, tensors


@pytest.mark.parametrize("fmt", ["f32", "bf16"])
def test_grouped_experts_skewed_routing_match_oracle(fmt):
    cfg, tensors = _skewed(fmt, 61)
    model = DecoderModel.from_bytes(cfg, st.dump(tensors), fmt)
    ref = oracle.OracleModel(cfg, tensors)
    # 1100 rows: the grouped LDS-streamed form (>= 1024 grouped rows); then a
    # 3-row block and single rows over the warm cache
    seed = 62
    prompt = synth.uniform_ids(seed, 1100, cfg.vocab_size)
    kv, rkv = model.new_cache(1, 1200), ref.new_cache(1200)
    got = model.try_forward_cached_last(prompt, kv)
    want = ref.forward_last(rkv, prompt)
    assert _close(got, want, fmt), ("prefill", float(np.abs(got - want).max()), seed)
    for ids in ([5, 6, 7], [oracle.argmax(want)], [11]):
        got = model.try_forward_cached_last(ids, kv)
        want = ref.forward_last(rkv, ids)
        assert _close(got, want, fmt), (ids, float(np.abs(got - want).max()))
    # several sequences of different lengths in one forward == each alone
    kvb = model.new_cache(3, 64)
    blocks = [synth.uniform_ids(70 + i, n, cfg.vocab_size) for i, n in enumerate((9, 1, 30))]
    rows = model.forward_batch(kvb, [0, 1, 2], blocks)
    for i, b in enumerate(blocks):
        rk = ref.new_cache(64)
        assert _close(rows[i], ref.forward_last(rk, b), fmt), i


@pytest.mark.parametrize("fmt", ["f32", "bf16"])
def test_router_failure_is_reported_and_no_position_moves(fmt):
    cfg = synth.llama_config(1, 128, 4, 2, 128, 300, head_dim=32, max_pos=64, extra=QWEN2_MOE)
    tensors = synth.make_tensors(cfg, 5, fmt)
    # every embedding row carries 100 in dim 0, so RMSNorm(h)[0] ~ sqrt(H)
    # for any token, and router row 2 (1e38 there, finite) overflows to inf
    e, edt = tensors["model.embed_tokens.weight"]
    e = _f32(e, edt)
    e[:, 0] = 100.0
    tensors["model.embed_tokens.weight"] = (_back(e, edt), edt)
    name = "model.layers.0.mlp.gate.weight"
    r, dt = tensors[name]
    r = _f32(r, dt)
    r[2] = 0.0
    r[2, 0] = 1e38
    tensors[name] = (_back(r, dt), dt)
    model = DecoderModel.from_bytes(cfg, st.dump(tensors), fmt)
    kv = model.new_cache(1, 64)
    for ids in ([1, 2, 3, 4], [9]):  # grouped prefill, then the single-row decode path
        with pytest.raises(Backend, match="non-finite expert router"):
            model.try_forward_cached_last(ids, kv)
        assert kv.position() == 0
    with pytest.raises(Backend, match="non-finite expert router"):
        model.generate_greedy_device(model.new_cache(1, 64), [1, 2], 4, eos=[])


@pytest.mark.parametrize("n", [40, 300])
def test_router_failure_in_batched_routing_forms(n):
    """The router's refusal through the other routing forms: one block for
    up to 256 rows (40), the grid top-k plus grouping pass above (300)."""
    print(f"router failure rows {n}", flush=True)
    cfg = synth.llama_config(1, 128, 4, 2, 128, 300, head_dim=32, max_pos=512, extra=QWEN2_MOE)
    tensors = synth.make_tensors(cfg, 5, "f32")
    e, edt = tensors["model.embed_tokens.weight"]
    e = _f32(e, edt)
    e[:, 0] = 100.0
    tensors["model.embed_tokens.weight"] = (_back(e, edt), edt)
    name = "model.layers.0.mlp.gate.weight"
    r, dt = tensors[name]
    r = _f32(r, dt)
    r[2] = 0.0
    r[2, 0] = 1e38
    tensors[name] = (_back(r, dt), dt)
    model = DecoderModel.from_bytes(cfg, st.dump(tensors), "f32")
    kv = model.new_cache(1, n + 8)
    with pytest.raises(Backend, match="non-finite expert router"):
        model.try_forward_cached_last(synth.uniform_ids(3, n, cfg.vocab_size), kv)
    assert kv.position() == 0
