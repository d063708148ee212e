"""Host side of the stage seam (esp_amd/stage.py) against the reference's
stage tests (stage.rs:597-680): range assignment, per-layer admission
bytes and the f32 hidden wire."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from esp_amd import InvalidConfig, InvalidRequest
from esp_amd.stage import (LayerRange, StageCapacity, StageAssignment, assign_ranges,
                           decode_hidden, encode_hidden, layer_resident_bytes)
from tests import synth


def _tiny(**extra):
    """decoder/mod.rs:141-164 tiny_config: vocab 32, hidden 8, ffn 16, 2
    layers, 4 heads, 2 kv heads, 16 positions."""
    return synth.llama_config(2, 8, 4, 2, 16, 32, max_pos=16, extra=extra or None)


def test_ranges_honor_runtime_budgets_and_distinct_devices():
    """stage.rs:597-642"""
    a, b = bytes([1]) * 32, bytes([2]) * 32
    devices = [StageCapacity(a, 21), StageCapacity(b, 30)]
    assert assign_ranges([10, 11, 12, 13], devices) == [
        StageAssignment(a, LayerRange(0, 2)), StageAssignment(b, LayerRange(2, 4))]
    with pytest.raises(InvalidConfig):
        assign_ranges([22, 31], devices)
    with pytest.raises(InvalidConfig):
        assign_ranges([1], [devices[0], devices[0]])
    assert layer_resident_bytes(_tiny(), "f32") == 2880
    devices = [StageCapacity(a, 1), StageCapacity(b, 20)]
    assert assign_ranges([10, 10], devices)[0].device == b
    with pytest.raises(InvalidConfig):
        assign_ranges([0, 1], devices)


def test_admission_bytes_closed_forms():
    """weights (q, o: h*qw each; k, v: h*kv each; 3 h*ffn MLP; 2 norms) +
    the whole context's K and V, per format"""
    cfg = synth.llama_config(4, 256, 8, 2, 512, 100, max_pos=64)
    h, qw, kv, f, P = 256, 256, 64, 512, 64
    proj = 2 * h * qw + 2 * h * kv + 3 * h * f
    assert layer_resident_bytes(cfg, "f32") == (proj + 2 * h) * 4 + kv * P * 2 * 4
    assert layer_resident_bytes(cfg, "bf16") == (proj + 2 * h) * 2 + kv * P * 2 * 2
    assert layer_resident_bytes(cfg, "q8-block32") == proj + proj // 32 * 4 + 2 * h * 2 + kv * P * 4
    assert layer_resident_bytes(cfg, "q4-block32") == proj // 2 + proj // 32 * 4 + 2 * h * 2 + kv * P * 4


def test_hybrid_admission_covers_a_dense_mlp_larger_than_the_expert_bank():
    """stage.rs:664-680"""
    dense = synth.llama_config(2, 8, 4, 2, 4096, 32, max_pos=16)
    hybrid = synth.llama_config(2, 8, 4, 2, 4096, 32, max_pos=16, extra={
        "model_type": "qwen2_moe", "architectures": ["Qwen2MoeForCausalLM"], "num_experts": 1,
        "num_experts_per_tok": 1, "moe_intermediate_size": 1,
        "shared_expert_intermediate_size": 1, "decoder_sparse_step": 2})
    assert layer_resident_bytes(hybrid, "f32") >= layer_resident_bytes(dense, "f32")


def test_hidden_wire_refuses_overflow_nonfinite_and_dtype_changes():
    """stage.rs:645-662"""
    data = bytearray(encode_hidden(np.ones((1, 3, 8), np.float32), 112))
    assert decode_hidden(bytes(data), 8, 16, "f32").shape == (3, 8)
    with pytest.raises(InvalidRequest):
        encode_hidden(np.ones((1, 3, 8), np.float32), 111)
    with pytest.raises(InvalidRequest):
        decode_hidden(bytes(data), 4, 16, "f32")
    with pytest.raises(InvalidRequest):
        decode_hidden(bytes(data), 8, 2, "f32")
    data[16:20] = struct.pack("<f", float("nan"))
    with pytest.raises(InvalidRequest):
        decode_hidden(bytes(data), 8, 16, "f32")
    data[16:20] = struct.pack("<f", 0.1234567)
    with pytest.raises(InvalidRequest):
        decode_hidden(bytes(data), 8, 16, "f16")
    assert decode_hidden(bytes(data), 8, 16, "f32")[0, 0] == np.float32(0.1234567)
    data[:8] = struct.pack("<Q", 2 ** 64 - 1)
    with pytest.raises(InvalidRequest):
        decode_hidden(bytes(data), 8, 2 ** 62, "f32")


def test_wire_round_trip_is_exact():
    rng = np.random.default_rng(1)
    h = rng.standard_normal((5, 16)).astype(np.float32)
    out = decode_hidden(encode_hidden(h, 1 << 20), 16, 8)
    assert out.dtype == np.float32 and np.array_equal(out, h)
    assert LayerRange(1, 3).validate(3) is None
    for bad in (LayerRange(2, 2), LayerRange(0, 4)):
        with pytest.raises(InvalidConfig, match="empty or out-of-model stage range"):
            bad.validate(3)
