"""Host side of layer streaming (esp_amd/streaming.py): the verified-layer
cache against the reference's own tests (streaming.rs:322-388), the
options' validation and the checkpoint splitter (checkpoint.rs:47-293)."""
from __future__ import annotations

import numpy as np
import pytest

from esp_amd import InvalidConfig, InvalidWeights
from esp_amd.streaming import (Artifact, FnSource, StreamingOptions, cache_verified_layers,
                               read_header, split_checkpoint, with_expert_reader)
from oracle import st
from tests import synth


def test_immutable_hits_share_the_verified_allocation_and_recheck_limits():
    """streaming.rs:327-345"""
    reads = []

    def read(index, _limit):
        reads.append(index)
        return bytes([index]) * 32

    source = cache_verified_layers(FnSource(read), 64)
    first = source.read_layer_shared(3, 32)
    second = source.read_layer_shared(3, 32)
    assert first is second
    assert source.read_layer(3, 32) == bytes([3]) * 32
    with pytest.raises(InvalidWeights):
        source.read_layer_shared(3, 31)
    assert len(reads) == 1
    stats = source.cache_stats()
    assert stats.hits == 2
    assert stats.retained_capacity_bytes == 32


def test_budget_counts_allocation_capacity_and_does_not_thrash_on_a_sweep():
    """streaming.rs:347-367: index 2 sits in a 128-byte allocation."""
    source = cache_verified_layers(
        FnSource(lambda i, _l: Artifact(bytes([i]) * 32, 128 if i == 2 else 32)), 64)
    for _ in range(3):
        for index in range(4):
            source.read_layer_shared(index, 32)
    stats = source.cache_stats()
    assert stats.entries == 2
    assert stats.retained_capacity_bytes == 64
    assert stats.hits == 4
    assert stats.misses == 8


def test_failed_or_oversized_reads_never_enter_the_cache():
    """streaming.rs:369-388"""
    count = [0]

    def read(_i, _l):
        count[0] += 1
        if count[0] == 1:
            raise InvalidWeights("content hash mismatch")
        if count[0] == 2:
            return bytes(33)
        return bytes([1]) * 32

    source = cache_verified_layers(FnSource(read), 64)
    with pytest.raises(InvalidWeights):
        source.read_layer_shared(0, 32)
    with pytest.raises(InvalidWeights):
        source.read_layer_shared(0, 32)
    assert source.cache_stats().entries == 0
    assert source.read_layer_shared(0, 32) == bytes([1]) * 32
    source.read_layer_shared(0, 32)
    assert count[0] == 3


def test_zero_budget_is_the_source_itself_and_experts_compose():
    src = FnSource(lambda i, _l: bytes(4))
    assert cache_verified_layers(src, 0) is src
    with pytest.raises(InvalidWeights, match="no expert reader"):
        src.read_expert(0, 0, 8)
    both = with_expert_reader(lambda i, _l: bytes([i]), lambda l, e, _x: bytes([l, e]))
    assert both.read_layer(5, 8) == b"\x05" and both.read_expert(2, 3, 8) == b"\x02\x03"


def test_options_validate_and_deny_unknown_fields():
    o = StreamingOptions()
    assert (o.query_chunk, o.max_layer_bytes, o.max_shared_bytes) == (32, 256 << 20, 1 << 30)
    o.validate()
    assert StreamingOptions.from_json(o.to_json()) == o
    for bad in ('{"query_chunk": 1, "max_layer_bytes": 2}',
                '{"query_chunk": 1, "max_layer_bytes": 2, "max_shared_bytes": 3, "x": 4}'):
        with pytest.raises(InvalidConfig):
            StreamingOptions.from_json(bad)
    with pytest.raises(InvalidConfig, match="streaming limits must be positive"):
        StreamingOptions(0, 1, 1).validate()


def test_split_checkpoint_keeps_exact_tensors_per_artifact():
    cfg = synth.llama_config(3, 64, 4, 2, 96, 50, head_dim=16,
                             extra={"model_type": "qwen2", "architectures": ["Qwen2ForCausalLM"]})
    tensors = synth.make_tensors(cfg, 3, "bf16", bias_std=0.1)
    blob = st.dump(tensors)
    shared, layers = split_checkpoint(blob, cfg)
    assert set(read_header(shared)[0]) == {"model.embed_tokens.weight", "model.norm.weight",
                                          "lm_head.weight"}
    for i, art in enumerate(layers):
        got = st.load(art)
        assert set(got) == {n for n in tensors if n.startswith(f"model.layers.{i}.")}
        for n, (arr, dt) in got.items():
            assert dt == tensors[n][1] and np.array_equal(arr, tensors[n][0])
    with pytest.raises(InvalidWeights, match="artifact tensor data exceeds"):
        split_checkpoint(blob, cfg, StreamingOptions(max_layer_bytes=1000))
    t = dict(tensors)
    t["model.layers.0.extra.weight"] = (np.zeros(4, np.float32), "F32")
    with pytest.raises(InvalidWeights, match="tensor names do not match"):
        split_checkpoint(st.dump(t), cfg)


def test_layer_index_round_trip_and_strict_fields():
    from esp_amd.streaming import IndexedSource, LayerArtifact, LayerWeightIndex
    idx = LayerWeightIndex(LayerArtifact("blob-s", 4), (LayerArtifact("b0", 3), LayerArtifact("b1", 5)),
                           StreamingOptions(8, 16, 32))
    raw = idx.to_json()
    assert LayerWeightIndex.from_json(raw) == idx
    bad = dict(raw, extra=1)
    with pytest.raises(InvalidWeights):
        LayerWeightIndex.from_json(bad)
    bad = dict(raw, shared={"blob": "x"})
    with pytest.raises(InvalidWeights):
        LayerWeightIndex.from_json(bad)
    store = {"blob-s": b"ssss", "b0": b"abc", "b1": b"wrong"}
    src = IndexedSource(idx, lambda blob, size: store[blob])
    assert src.shared() == b"ssss" and src.read_layer(0, 16) == b"abc"
    with pytest.raises(InvalidWeights, match="byte limit mismatch"):
        src.read_layer(1, 4)  # declared 5 > limit 4: refused before reading
    store["b1"] = b"1234"
    with pytest.raises(InvalidWeights, match="do not match their reference"):
        src.read_layer(1, 16)
    with pytest.raises(InvalidWeights, match="missing layer artifact 2"):
        src.read_layer(2, 16)


def test_format_qualification_rules():
    """layer_library.rs:61-87: every measure present, finite and consistent;
    unmeasured candidates are not selectable."""
    from esp_amd.streaming import (FormatQualification, FormattedLayerWeightIndex, LayerArtifact,
                                   LayerWeightIndex, PromptDeviation)
    idx = LayerWeightIndex(LayerArtifact("s", 1), (), StreamingOptions())
    p = PromptDeviation("hi", (1, 2), (1, 3), 0.1, 0.5)
    q = FormatQualification("base", "bf16", "q8", (p,), 1, 2, 3, 4, 5, 1.5)
    q.validate()
    f = FormattedLayerWeightIndex(idx, "q8-k32-f32-scale-f16-shared-v1", ("src",), None)
    assert not f.selectable()
    assert FormattedLayerWeightIndex(idx, "bf16", (), q).selectable()
    for bad in (q.__class__(**{**q.__dict__, "prompts": ()}),
                q.__class__(**{**q.__dict__, "elapsed_seconds": float("nan")}),
                q.__class__(**{**q.__dict__, "largest_layer_bytes": 0}),
                q.__class__(**{**q.__dict__, "prompts": (PromptDeviation("hi", (1,), (1,), 0.6, 0.5),)})):
        with pytest.raises(InvalidWeights, match="incomplete or non-finite"):
            bad.validate()
    with pytest.raises(InvalidWeights, match="unknown weight format"):
        FormattedLayerWeightIndex(idx, "int3", (), None)
