"""Streamed layers (streaming.rs, model.rs:196-415) on the MI355X.

A streamed model runs the same kernels over the same weights as the resident
model loaded from the whole checkpoint, so logits must be bit-identical to
the resident model's (which is itself pinned to the CPU oracle by the parity
tests; one case here checks the oracle too). The refusal cases follow the
reference's layer-library tests (layer_library.rs:556-671): oversized,
corrupted or misnamed layers are refused before a token is committed."""
from __future__ import annotations

import numpy as np
import pytest

from esp_amd import DecoderModel, InvalidConfig, InvalidWeights, Unsupported
from esp_amd.streaming import (ArtifactSource, FnSource, StreamingOptions, cache_verified_layers,
                               pack, read_header, split_checkpoint)
from oracle import oracle, quant, st
from tests import synth

pytestmark = pytest.mark.gpu


def _case(fmt_art="f32", layers=3, extra=None, seed=11, bias_std=0.0):
    cfg = synth.llama_config(layers, 128, 4, 2, 256, 300, head_dim=32, extra=extra)
    tensors = synth.make_tensors(cfg, seed, fmt_art, std=0.05, bias_std=bias_std)
    return cfg, tensors, st.dump(tensors)


def _run(model, prompt, steps):
    """prefill + greedy decode; returns every logits row and the ids"""
    kv = model.new_cache(1, 64)
    rows, ids = [model.try_forward_cached_last(prompt, kv)], []
    for _ in range(steps):
        ids.append(int(np.argmax(rows[-1])))
        rows.append(model.try_forward_cached_last([ids[-1]], kv))
    return rows, ids, kv


CASES = [
    ("f32", "f32", None, 0.0),
    ("bf16", "bf16", None, 0.0),
    ("f32", "bf16", None, 0.0),  # f32 model from bf16 artifacts: widened on the device
    ("bf16", "bf16", {"model_type": "qwen2", "architectures": ["Qwen2ForCausalLM"]}, 0.05),
    ("f32", "f32", {"model_type": "qwen3", "architectures": ["Qwen3ForCausalLM"]}, 0.0),
    # sliding window of 4 on layers 1.. (config.rs:467-485), past the window
    ("bf16", "bf16", {"model_type": "qwen2", "architectures": ["Qwen2ForCausalLM"],
                      "use_sliding_window": True, "sliding_window": 4, "max_window_layers": 1}, 0.0),
]


@pytest.mark.parametrize("fmt,art,extra,bias", CASES)
def test_streamed_matches_resident_bit_exactly(fmt, art, extra, bias):
    print(f"streamed {fmt} from {art} {extra}", flush=True)
    cfg, tensors, blob = _case(art, extra=extra, bias_std=bias)
    shared, layers = split_checkpoint(blob, cfg)
    resident = DecoderModel.from_bytes(cfg, blob, fmt)
    streamed = DecoderModel.from_layer_source(cfg, shared, ArtifactSource(layers),
                                              StreamingOptions(), fmt)
    prompt = synth.uniform_ids(5, 9, cfg.vocab_size)
    want_rows, want_ids, _ = _run(resident, prompt, 6)
    got_rows, got_ids, kv = _run(streamed, prompt, 6)
    for g, w in zip(got_rows, want_rows):
        assert np.array_equal(g, w)
    assert got_ids == want_ids and kv.position() == len(prompt) + 6
    stats = streamed.streaming_stats()
    assert stats.layer_reads == 7 * cfg.num_hidden_layers  # every forward reads every layer
    assert stats.largest_encoded_layer == max(len(b) for b in layers)
    assert stats.device_cache is None
    # device generation: the streamed host loop gives the resident graph's ids
    dev = streamed.generate_greedy_device(streamed.new_cache(1, 64), prompt, 6, eos=[])
    assert dev == resident.generate_greedy_device(resident.new_cache(1, 64), prompt, 6, eos=[])
    if fmt == "f32" and art == "f32" and extra is None:
        ref = oracle.OracleModel(cfg, tensors)
        rkv = ref.new_cache()
        want = ref.forward_last(rkv, prompt)
        assert np.abs(got_rows[0] - want).max() <= 1e-4 * float(np.abs(want).max())


def test_streamed_batch_and_long_prompt_match_resident():
    cfg, _, blob = _case("bf16")
    shared, layers = split_checkpoint(blob, cfg)
    resident = DecoderModel.from_bytes(cfg, blob, "bf16")
    streamed = DecoderModel.from_layer_source(cfg, shared, ArtifactSource(layers), fmt="bf16")
    a = synth.uniform_ids(1, 40, cfg.vocab_size)
    b = synth.uniform_ids(2, 17, cfg.vocab_size)
    out = []
    for m in (resident, streamed):
        kv = m.new_cache(2, 128)
        r1 = m.forward_batch(kv, [0, 1], [a, b])
        r2 = m.forward_batch(kv, [0, 1], [[3], [4]])
        out.append((r1, r2))
    assert np.array_equal(out[0][0], out[1][0]) and np.array_equal(out[0][1], out[1][1])


@pytest.mark.parametrize("bits", [8, 4])
def test_streamed_packed_matches_resident(bits):
    cfg = synth.llama_config(2, 128, 4, 2, 256, 300, head_dim=32)
    tensors = synth.make_tensors(cfg, 7, "f32", std=0.1)
    art = st.dump(quant.convert_artifact(tensors, bits))
    fmt = {8: "q8-block32", 4: "q4-block32"}[bits]
    shared, layers = split_checkpoint(art, cfg)
    resident = DecoderModel.from_bytes(cfg, art, fmt)
    streamed = DecoderModel.from_layer_source(cfg, shared, ArtifactSource(layers), fmt=fmt)
    prompt = synth.uniform_ids(3, 10, cfg.vocab_size)
    for g, w in zip(_run(streamed, prompt, 4)[0], _run(resident, prompt, 4)[0]):
        assert np.array_equal(g, w)


def test_device_layer_cache_counts_and_keeps_results():
    """model.rs:336-362, 560-646: first-fit within the payload budget, at
    most 128 layers; hits and misses per layer read; payload is 4 bytes per
    artifact element."""
    cfg, _, blob = _case("bf16", layers=4)
    shared, layers = split_checkpoint(blob, cfg)
    resident = DecoderModel.from_bytes(cfg, blob, "bf16")
    hdr = read_header(layers[0])[0]
    payload = sum(4 * int(np.prod(h["shape"])) for h in hdr.values())
    streamed = DecoderModel.from_layer_source(cfg, shared, ArtifactSource(layers), fmt="bf16")
    streamed.with_layer_cache(2 * payload + payload // 2)  # room for two layers
    prompt = synth.uniform_ids(8, 12, cfg.vocab_size)
    want = _run(resident, prompt, 3)[0]
    got = _run(streamed, prompt, 3)[0]
    assert all(np.array_equal(g, w) for g, w in zip(got, want))
    s = streamed.streaming_stats()
    dc = s.device_cache
    assert dc.layers == 2 and dc.retained_payload_bytes == 2 * payload
    assert dc.payload_budget_bytes == 2 * payload + payload // 2
    # 4 forwards x 4 layers: layers 0 and 1 miss once then hit
    assert dc.misses == 2 + 4 * 2 and dc.hits == 3 * 2
    assert s.layer_reads == dc.misses
    with pytest.raises(InvalidConfig, match="device layer caching"):
        resident.with_layer_cache(1 << 20)
    resident.with_layer_cache(0)  # budget 0 is accepted everywhere


def test_resident_layers_read_once_and_stop_streaming():
    cfg, _, blob = _case("f32")
    shared, layers = split_checkpoint(blob, cfg)
    reads = []

    def read(i, limit):
        reads.append(i)
        return layers[i]

    m = DecoderModel.from_layer_source(cfg, shared, FnSource(read))
    m.with_resident_layers()
    assert reads == list(range(cfg.num_hidden_layers))
    assert m.streaming_stats() is None
    prompt = synth.uniform_ids(4, 8, cfg.vocab_size)
    resident = DecoderModel.from_bytes(cfg, blob, "f32")
    assert all(np.array_equal(g, w) for g, w in zip(_run(m, prompt, 3)[0], _run(resident, prompt, 3)[0]))
    assert reads == list(range(cfg.num_hidden_layers))


def test_host_verified_cache_feeds_the_device():
    cfg, _, blob = _case("bf16")
    shared, layers = split_checkpoint(blob, cfg)
    src = cache_verified_layers(ArtifactSource(layers), 1 << 30)
    m = DecoderModel.from_layer_source(cfg, shared, src, fmt="bf16")
    _run(m, synth.uniform_ids(4, 8, cfg.vocab_size), 2)
    v = m.streaming_stats().verified_cache
    assert v.misses == cfg.num_hidden_layers and v.hits == 2 * cfg.num_hidden_layers


def test_refusals_commit_nothing():
    """layer_library.rs:583-671: corrupted, oversized and failed layer reads
    are refused before any token or position is committed."""
    cfg, tensors, blob = _case("bf16")
    shared, layers = split_checkpoint(blob, cfg)
    prompt = synth.uniform_ids(6, 8, cfg.vocab_size)

    def model_with(arts, opts=None):
        return DecoderModel.from_layer_source(cfg, shared, ArtifactSource(arts), opts, fmt="bf16")

    # a layer artifact with another layer's names
    bad = list(layers)
    bad[1] = layers[2]
    m = model_with(bad)
    kv = m.new_cache(1, 64)
    with pytest.raises(InvalidWeights, match="layer 1 tensor names do not match"):
        m.try_forward_cached_last(prompt, kv)
    assert kv.position() == 0
    # over the byte limit
    m = model_with(layers, StreamingOptions(max_layer_bytes=len(layers[0]) - 1))
    kv = m.new_cache(1, 64)
    with pytest.raises(InvalidWeights, match="byte limit"):
        m.try_forward_cached_last(prompt, kv)
    assert kv.position() == 0
    # a corrupted header
    bad = list(layers)
    bad[2] = b"\xff" * 16 + layers[2][16:]
    m = model_with(bad)
    with pytest.raises(InvalidWeights, match="layer 2"):
        m.try_forward_cached_last(prompt, m.new_cache(1, 64))
    # a source that fails mid-generation: the source's own error, no position
    calls = []

    def flaky(i, limit):
        calls.append(i)
        if len(calls) > cfg.num_hidden_layers + 1:
            raise InvalidWeights("content hash mismatch")
        return layers[i]

    m = DecoderModel.from_layer_source(cfg, shared, FnSource(flaky), fmt="bf16")
    kv = m.new_cache(1, 64)
    m.try_forward_cached_last(prompt, kv)
    with pytest.raises(InvalidWeights, match="content hash mismatch"):
        m.try_forward_cached_last([1], kv)
    assert kv.position() == len(prompt)
    # a non-finite weight: named, and not kept by the device cache
    t = dict(tensors)
    name = "model.layers.1.mlp.up_proj.weight"
    arr = t[name][0].copy()
    arr.reshape(-1)[77] = np.uint16(0x7f80)  # bf16 +inf
    t[name] = (arr, "BF16")
    _, bad_layers = split_checkpoint(st.dump(t), cfg)
    m = model_with(bad_layers).with_layer_cache(1 << 30)
    kv = m.new_cache(1, 64)
    with pytest.raises(InvalidWeights, match="non-finite weight in " + name.replace(".", r"\.")):
        m.try_forward_cached_last(prompt, kv)
    assert kv.position() == 0
    assert m.streaming_stats().device_cache.layers == cfg.num_hidden_layers - 1


def test_shared_artifact_refusals():
    cfg, tensors, blob = _case("f32")
    shared, layers = split_checkpoint(blob, cfg)
    with pytest.raises(InvalidWeights, match="shared artifact exceeds its byte limit"):
        DecoderModel.from_layer_source(cfg, shared, ArtifactSource(layers),
                                       StreamingOptions(max_shared_bytes=len(shared) - 1))
    hdr, start = read_header(shared)
    extra = [(n, h["dtype"], h["shape"], shared[start + h["data_offsets"][0]:start + h["data_offsets"][1]])
             for n, h in hdr.items()]
    extra.append(("model.layers.0.input_layernorm.weight", "F32", [128], b"\0" * 512))
    with pytest.raises(InvalidWeights, match="unexpected tensor in shared artifact"):
        DecoderModel.from_layer_source(cfg, pack(extra), ArtifactSource(layers))
    with pytest.raises(InvalidConfig, match="streaming limits must be positive"):
        DecoderModel.from_layer_source(cfg, shared, ArtifactSource(layers), StreamingOptions(0))
    moe = synth.llama_config(2, 128, 4, 2, 256, 300, head_dim=32, extra={
        "model_type": "qwen2_moe", "architectures": ["Qwen2MoeForCausalLM"], "num_experts": 4,
        "num_experts_per_tok": 2, "moe_intermediate_size": 64,
        "shared_expert_intermediate_size": 64, "decoder_sparse_step": 1})
    with pytest.raises(Unsupported, match="expert streaming"):
        DecoderModel.from_layer_source(moe, shared, ArtifactSource(layers))


def test_fully_cached_stream_replays_the_decode_graph():
    """Once every layer is in the device cache, greedy generation replays
    the captured step; ids equal the resident model's and the cache counts
    one hit per layer for each forward the reference takes (prefill, then
    one per emitted token before the last; generate.rs:154-168)."""
    cfg, _, blob = _case("bf16")
    L = cfg.num_hidden_layers
    shared, layers = split_checkpoint(blob, cfg)
    resident = DecoderModel.from_bytes(cfg, blob, "bf16")
    m = DecoderModel.from_layer_source(cfg, shared, ArtifactSource(layers), fmt="bf16")
    m.with_layer_cache(1 << 32)
    prompt = synth.uniform_ids(12, 9, cfg.vocab_size)
    want = resident.generate_greedy_device(resident.new_cache(1, 64), prompt, 6, eos=[])
    got = m.generate_greedy_device(m.new_cache(1, 64), prompt, 6, eos=[])
    assert got == want
    s = m.streaming_stats()
    assert s.layer_reads == L and s.device_cache.misses == L and s.device_cache.hits == 5 * L
    # eos = the first id not seen earlier: generation stops before it
    k = next(i for i in range(1, len(want)) if want[i] not in want[:i])
    got = m.generate_greedy_device(m.new_cache(1, 64), prompt, 6, eos=[want[k]])
    assert got == want[:k]
    s = m.streaming_stats()
    assert s.layer_reads == L and s.device_cache.hits == 5 * L + L + k * L
