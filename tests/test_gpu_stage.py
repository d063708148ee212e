"""Stage chain (stage.rs) on the MI355X: disjoint layer-range stages chained
through the f32 hidden wire give the resident model's logits bit for bit
(the same kernels over the same weights) and the oracle's within the
format's tolerance (stage.rs:531-596: stages == the full layer stack), and
enforce the reference's positions."""
from __future__ import annotations

import numpy as np
import pytest

from esp_amd import DecoderModel, InvalidConfig, InvalidRequest, InvalidWeights
from esp_amd.stage import (DecoderStage, LayerRange, StageChain, StagedModel, decode_hidden,
                           encode_hidden)
from esp_amd.streaming import ArtifactSource, split_checkpoint
from oracle import oracle, st
from tests import synth

pytestmark = pytest.mark.gpu


def _case(art, layers=3, tensors=False):
    cfg = synth.llama_config(layers, 128, 4, 2, 256, 300, head_dim=32)
    t = synth.make_tensors(cfg, 21, art, std=0.05)
    return (cfg, st.dump(t), t) if tensors else (cfg, st.dump(t))


def _close(got, want, fmt):
    if fmt == "bf16":
        return np.all(np.abs(got - want) <= 1e-2 + 2e-2 * np.abs(want))
    return np.all(np.abs(got - want) <= 1e-4 * float(np.abs(want).max()))


@pytest.mark.parametrize("fmt", ["f32", "bf16"])
def test_disjoint_stages_match_the_resident_model(fmt):
    print(f"stages {fmt}", flush=True)
    cfg, blob, tensors = _case(fmt, tensors=True)
    shared, layers = split_checkpoint(blob, cfg)
    src = ArtifactSource(layers)
    first = DecoderStage.from_source(cfg, LayerRange(0, 1), src, fmt=fmt, max_ctx=64)
    last = DecoderStage.from_source(cfg, LayerRange(1, 3), src, fmt=fmt, shared=shared, max_ctx=64)
    staged = StagedModel(cfg, shared, StageChain([first, last]))
    resident = DecoderModel.from_bytes(cfg, blob, fmt)
    ref = oracle.OracleModel(cfg, tensors)
    kv, rkv = resident.new_cache(1, 64), ref.new_cache(64)
    prompt = synth.uniform_ids(3, 9, cfg.vocab_size)
    want = resident.try_forward_cached_last(prompt, kv)
    got = staged.try_forward_cached_last(prompt)
    assert np.array_equal(got, want)
    orc = ref.forward_last(rkv, prompt)
    assert _close(got, orc, fmt), float(np.abs(got - orc).max())
    for _ in range(3):
        t = oracle.argmax(orc)
        want = resident.try_forward_cached_last([t], kv)
        got = staged.try_forward_cached_last([t])
        assert np.array_equal(got, want)
        orc = ref.forward_last(rkv, [t])
        assert _close(got, orc, fmt), float(np.abs(got - orc).max())
    # a restart at 0 rebuilds every stage's cache
    staged.reset()
    assert np.array_equal(staged.try_forward_cached_last(prompt),
                          resident.try_forward_cached_last(prompt, resident.new_cache(1, 64)))


def test_stage_positions_wire_and_ownership():
    cfg, blob = _case("f32")
    shared, layers = split_checkpoint(blob, cfg)
    src = ArtifactSource(layers)
    first = DecoderStage.from_source(cfg, LayerRange(0, 2), src, max_ctx=32)
    x = np.random.default_rng(0).standard_normal((3, cfg.hidden_size)).astype(np.float32) * 0.1
    h0 = first.forward(x, 0)
    assert h0.shape == (3, cfg.hidden_size)
    with pytest.raises(InvalidRequest, match="position mismatch"):
        first.forward(x[:1], 4)
    with pytest.raises(InvalidRequest, match="position mismatch"):
        first.forward(x[:2], 3)  # only single tokens after the prefill
    first.forward(x[:1], 3)
    assert np.array_equal(first.forward(x, 0), h0)  # restart: same rows
    # the wire form of the same call
    wire = first.forward_bytes(encode_hidden(x, 1 << 20), 0, 1 << 20)
    assert np.array_equal(decode_hidden(wire, cfg.hidden_size, 64), h0)
    with pytest.raises(InvalidRequest, match="hidden wire budget"):
        first.forward_bytes(encode_hidden(x, 1 << 20), 0, 64)
    with pytest.raises(InvalidWeights, match="only the final stage may own the output head"):
        DecoderStage.from_source(cfg, LayerRange(0, 2), src, shared=shared)
    with pytest.raises(InvalidConfig, match="empty or out-of-model stage range"):
        DecoderStage.from_source(cfg, LayerRange(1, 4), src)
    with pytest.raises(InvalidConfig, match="contiguous"):
        last = DecoderStage.from_source(cfg, LayerRange(2, 3), src, shared=shared)
        StageChain([DecoderStage.from_source(cfg, LayerRange(0, 1), src), last])


def test_stage_windows_follow_the_global_layer_index():
    """A qwen2 config whose layers from index 1 on use a 4-token sliding
    window (config.rs:467-485): a stage over layers 1..3 must apply the
    windows of global layers 1 and 2, so the chain stays bit-identical to
    the resident model past the window."""
    cfg = synth.llama_config(3, 128, 4, 2, 256, 300, head_dim=32, extra={
        "model_type": "qwen2", "architectures": ["Qwen2ForCausalLM"], "use_sliding_window": True,
        "sliding_window": 4, "max_window_layers": 1})
    assert cfg.layer_window(0) is None and cfg.layer_window(1) == 4
    blob = st.dump(synth.make_tensors(cfg, 23, "bf16", std=0.05, bias_std=0.05))
    shared, layers = split_checkpoint(blob, cfg)
    src = ArtifactSource(layers)
    chain = StageChain([DecoderStage.from_source(cfg, LayerRange(0, 1), src, fmt="bf16", max_ctx=64),
                        DecoderStage.from_source(cfg, LayerRange(1, 3), src, fmt="bf16",
                                                 shared=shared, max_ctx=64)])
    staged = StagedModel(cfg, shared, chain)
    resident = DecoderModel.from_bytes(cfg, blob, "bf16")
    kv = resident.new_cache(1, 64)
    prompt = synth.uniform_ids(5, 20, cfg.vocab_size)
    want = resident.try_forward_cached_last(prompt, kv)
    assert np.array_equal(staged.try_forward_cached_last(prompt), want)
    for t in (7, 8, 9):
        assert np.array_equal(staged.try_forward_cached_last([t]),
                              resident.try_forward_cached_last([t], kv))
