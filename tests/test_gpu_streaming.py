"""Streamed layers (streaming.rs, model.rs:196-415) on the MI355X.

A streamed model runs the same kernels over the same weights as the resident
model loaded from the whole checkpoint, so logits must be bit-identical to
the resident model's, and every case's logits are checked against the CPU
oracle within the format's tolerance. The refusal cases follow the
reference's layer-library tests (layer_library.rs:556-671): oversized,
corrupted or misnamed layers are refused before a token is committed."""
from __future__ import annotations

import numpy as np
import pytest

from esp_amd import DecoderModel, InvalidConfig, InvalidWeights
from esp_amd.stage import DecoderStage, LayerRange, StageChain, StagedModel
from esp_amd.streaming import (ArtifactSource, FnSource, StreamingOptions, cache_verified_layers,
                               pack, read_header, split_checkpoint, split_experts,
                               with_expert_reader)
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
    # every streamed row against the oracle, teacher-forced on the same ids
    ref = oracle.OracleModel(cfg, tensors)
    rkv = ref.new_cache(64)
    for i, g in enumerate(got_rows):
        want = ref.forward_last(rkv, prompt if i == 0 else [got_ids[i - 1]])
        if fmt == "bf16":
            assert np.all(np.abs(g - want) <= 1e-2 + 2e-2 * np.abs(want)), i
        else:
            assert np.abs(g - want).max() <= 1e-4 * float(np.abs(want).max()), i


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


# ---- routed experts (streaming.rs:26-66, moe.rs:183-243, loader.rs:137-210)

MOE = {"model_type": "qwen2_moe", "architectures": ["Qwen2MoeForCausalLM"], "num_experts": 6,
       "num_experts_per_tok": 2, "moe_intermediate_size": 96,
       "shared_expert_intermediate_size": 64, "norm_topk_prob": False,
       "decoder_sparse_step": 2}  # layers 1 and 3 routed, 0 and 2 dense


def _moe_case(fmt, seed=31):
    cfg = synth.llama_config(4, 128, 4, 2, 256, 300, head_dim=32, max_pos=256, extra=MOE)
    tensors = synth.make_tensors(cfg, seed, fmt, std=0.05)
    blob = st.dump(tensors)
    shared, layers = split_checkpoint(blob, cfg)
    return cfg, tensors, blob, shared, layers, split_experts(blob, cfg)


def _close(got, want, fmt):
    if fmt == "bf16":
        return np.all(np.abs(got - want) <= 1e-2 + 2e-2 * np.abs(want))
    return np.abs(got - want).max() <= 1e-4 * float(np.abs(want).max())


@pytest.mark.parametrize("fmt", ["f32", "bf16"])
def test_streamed_experts_match_oracle_and_count_reads(fmt):
    """Core artifacts per layer, experts read per forward: only the experts
    the router chose, so a single-token forward reads exactly top-k experts
    per routed layer; every logits row within the format's tolerance of the
    oracle (teacher-forced on the streamed ids) and the greedy ids equal to
    the resident model's."""
    cfg, tensors, blob, shared, layers, experts = _moe_case(fmt)
    assert all(f"model.layers.1.mlp.experts.0.up_proj.weight" in read_header(experts[(1, 0)])[0]
               for _ in [0])
    assert "model.layers.1.mlp.gate.weight" in read_header(layers[1])[0]
    streamed = DecoderModel.from_layer_source(cfg, shared, ArtifactSource(layers, experts),
                                              fmt=fmt)
    resident = DecoderModel.from_bytes(cfg, blob, fmt)
    ref = oracle.OracleModel(cfg, tensors)
    prompt = synth.uniform_ids(9, 30, cfg.vocab_size)
    kv, rkv = streamed.new_cache(1, 64), ref.new_cache(64)
    got = streamed.try_forward_cached_last(prompt, kv)
    want = ref.forward_last(rkv, prompt)
    assert _close(got, want, fmt), float(np.abs(got - want).max())
    first = streamed.streaming_stats()
    routed = sum(cfg.layer_is_moe(i) for i in range(cfg.num_hidden_layers))
    assert routed == 2 and 2 * 2 <= first.expert_reads <= 2 * 6
    assert first.largest_encoded_expert == max(len(b) for b in experts.values())
    ids = []
    for step in range(4):
        ids.append(int(np.argmax(got)))
        before = streamed.streaming_stats().expert_reads
        got = streamed.try_forward_cached_last([ids[-1]], kv)
        want = ref.forward_last(rkv, [ids[-1]])
        assert _close(got, want, fmt), (step, float(np.abs(got - want).max()))
        assert streamed.streaming_stats().expert_reads - before == 2 * routed
    # the resident model's greedy ids; the streamed host loop reproduces them
    rk = resident.new_cache(1, 64)
    r = resident.try_forward_cached_last(prompt, rk)
    want_ids = []
    for _ in range(4):
        want_ids.append(int(np.argmax(r)))
        r = resident.try_forward_cached_last([want_ids[-1]], rk)
    assert ids == want_ids
    assert streamed.generate_greedy_device(streamed.new_cache(1, 64), prompt, 4, eos=[]) == ids
    # a device layer cache keeps core blocks; experts are still read per forward
    streamed.with_layer_cache(1 << 30)
    before = streamed.streaming_stats().expert_reads
    _run(streamed, prompt, 2)
    s2 = streamed.streaming_stats()
    assert s2.device_cache.layers == cfg.num_hidden_layers and s2.expert_reads > before


@pytest.mark.parametrize("fmt", ["f32", "bf16"])
def test_resident_experts_read_once_match_the_resident_model(fmt):
    """loader.rs:196-210 ExpertMode::Resident: every layer and every expert
    read once and kept; the model then equals the resident one bit for bit
    and reads nothing more. Stages over routed layers read their experts
    the same way and chain to the same logits."""
    cfg, _, blob, shared, layers, experts = _moe_case(fmt, seed=37)
    reads = []

    def read_expert(layer, expert, limit):
        reads.append((layer, expert))
        return experts[(layer, expert)]

    src = with_expert_reader(lambda i, limit: layers[i], read_expert)
    m = DecoderModel.from_layer_source(cfg, shared, src, fmt=fmt)
    m.with_resident_layers()
    assert sorted(reads) == sorted(experts) and m.streaming_stats() is None
    resident = DecoderModel.from_bytes(cfg, blob, fmt)
    prompt = synth.uniform_ids(4, 20, cfg.vocab_size)
    want = _run(resident, prompt, 3)[0]
    assert all(np.array_equal(g, w) for g, w in zip(_run(m, prompt, 3)[0], want))
    assert len(reads) == len(experts)
    chain = StageChain([DecoderStage.from_source(cfg, LayerRange(0, 2), src, fmt=fmt, max_ctx=64),
                        DecoderStage.from_source(cfg, LayerRange(2, 4), src, fmt=fmt,
                                                 shared=shared, max_ctx=64)])
    staged = StagedModel(cfg, shared, chain)
    got = [staged.try_forward_cached_last(prompt)]
    kv = resident.new_cache(1, 64)
    ref_rows = [resident.try_forward_cached_last(prompt, kv)]
    for t in (5, 6):
        got.append(staged.try_forward_cached_last([t]))
        ref_rows.append(resident.try_forward_cached_last([t], kv))
    assert all(np.array_equal(g, w) for g, w in zip(got, ref_rows))


def test_expert_refusals():
    """moe.rs:210-235, loader.rs:137-168: a source without an expert
    reader, an artifact past the budget, misnamed expert tensors and a
    non-finite expert weight are refused; no position moves."""
    cfg, tensors, blob, shared, layers, experts = _moe_case("f32", seed=41)
    prompt = synth.uniform_ids(2, 6, cfg.vocab_size)
    m = DecoderModel.from_layer_source(cfg, shared, ArtifactSource(layers), fmt="f32")
    kv = m.new_cache(1, 32)
    with pytest.raises(InvalidWeights, match="no expert reader"):
        m.try_forward_cached_last(prompt, kv)
    assert kv.position() == 0
    big = StreamingOptions(max_layer_bytes=max(len(b) for b in layers))
    over = with_expert_reader(lambda i, limit: layers[i],
                              lambda l, e, limit: experts[(l, e)] + b"\0" * (limit + 1))
    m = DecoderModel.from_layer_source(cfg, shared, over, big, fmt="f32")
    with pytest.raises(InvalidWeights, match="expert source exceeded artifact budget"):
        m.try_forward_cached_last(prompt, m.new_cache(1, 32))
    swapped = with_expert_reader(lambda i, limit: layers[i],
                                 lambda l, e, limit: experts[(l, (e + 1) % 6)])
    m = DecoderModel.from_layer_source(cfg, shared, swapped, fmt="f32")
    with pytest.raises(InvalidWeights, match="expert artifact names disagree"):
        m.try_forward_cached_last(prompt, m.new_cache(1, 32))
    # expert 2 of layer 3 carries an inf in up_proj: refused when it is read
    name = "model.layers.3.mlp.experts.2.up_proj.weight"
    hdr, start = read_header(experts[(3, 2)])
    parts = []
    for n, h in hdr.items():
        raw = bytearray(experts[(3, 2)][start + h["data_offsets"][0]:start + h["data_offsets"][1]])
        if n == name:
            raw[0:4] = np.array([np.inf], np.float32).tobytes()
        parts.append((n, h["dtype"], h["shape"], bytes(raw)))
    bad = dict(experts)
    bad[(3, 2)] = pack(parts)
    m = DecoderModel.from_layer_source(cfg, shared, ArtifactSource(layers, bad), fmt="f32")
    with pytest.raises(InvalidWeights, match=f"non-finite weight in {name}"):
        m.with_resident_layers()
