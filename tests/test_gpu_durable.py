"""Durable generation on the device: the checkpointed loop, its pause /
resume, commit-failure and draw-validation rules, numerical recovery from
non-finite scores, and the context-window rule.

Restates crates/esp/tests/durable_generation.rs:23-105 and the provider's
score-fault tests (crates/esp/src/infer/decoder/provider.rs:981-1104) over
seeded synthetic models, with every generated stream also checked against
the CPU oracle's greedy argmax / seeded sampler over its own logits."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from esp_amd import Backend, DecoderModel, InvalidRequest, TokenPicker, generate_ids_with
from esp_amd.generate import try_generate_ids_with
from esp_amd.provider import DecoderProvider, GenerationRequest
from oracle import oracle, st
from tests import synth
from tests.grammar_cases import byte_tokenizer

pytestmark = pytest.mark.gpu

_HIP = None


def _hip():
    global _HIP
    if _HIP is None:
        _HIP = C.CDLL("libamdhip64.so.7")
        _HIP.hipMemsetD32Async.argtypes = [C.c_void_p, C.c_int, C.c_size_t, C.c_void_p]
        _HIP.hipStreamSynchronize.argtypes = [C.c_void_p]
    return _HIP


class FaultyProvider(DecoderProvider):
    """The reference's test build: `score_faults` maps an output index to a
    row of NaN scores that replaces the model's row before the constrained
    choice at that index (provider.rs:70-71, 755-762). The NaNs are written
    over the device logits row, so the library's own flags see them."""

    def __init__(self, *a, **k):
        super().__init__(*a, **k)
        self.score_faults = set()

    def _observe_scores(self, cache, index):
        if index in self.score_faults:
            self.score_faults.discard(index)
            ptr, rows = cache.logits_device()
            assert ptr and rows >= 1
            h = _hip()
            assert h.hipMemsetD32Async(ptr, 0x7FC00000, self.model.config.vocab_size,
                                       cache.stream()) == 0
            assert h.hipStreamSynchronize(cache.stream()) == 0


def _tiny(vocab: int, seed: int, max_pos: int = 128, std: float = 0.2):
    cfg = synth.llama_config(1, 64, 4, 2, 96, vocab, max_pos=max_pos)
    tensors = synth.make_tensors(cfg, seed, "f32", std=std)
    return cfg, tensors, DecoderModel.from_bytes(cfg, st.dump(tensors), "f32")


def _oracle_stream(cfg, tensors, prompt, n, temperature, top_p, seed):
    """The reference's plain loop (generate.rs:134-170) on the oracle."""
    ref = oracle.OracleModel(cfg, tensors)
    kv = ref.new_cache(min(len(prompt) + n, cfg.max_position_embeddings))
    row = ref.forward_last(kv, prompt)
    state = seed
    out = []
    for i in range(n):
        if temperature == 0.0:
            t = oracle.argmax(row)
        else:
            t, state = oracle.sample(row, temperature, top_p, state)
        out.append(t)
        if i + 1 < n:
            row = ref.forward_last(kv, [t])
    return out


def test_every_pause_boundary_rebuilds_the_same_greedy_and_seeded_stream():
    """durable_generation.rs:23-65, plus the stream itself against the oracle."""
    cfg, tensors, model = _tiny(64, 23)
    provider = DecoderProvider(model)
    for temperature in (0.0, 0.85):
        request = GenerationRequest(prompt_ids=[1, 5], max_tokens=8, temperature=temperature,
                                    top_p=0.95, seed=42)
        whole = provider.generate_checkpointed(request)
        assert whole.complete and len(whole.token_ids) == 8
        assert whole.token_ids == _oracle_stream(cfg, tensors, [1, 5], 8, temperature, 0.95, 42)
        for at in range(8):
            n = [0]

            def commit(cp):
                n[0] = len(cp.token_ids)

            paused = provider.generate_checkpointed(request, None, commit, lambda: n[0] >= at)
            assert len(paused.token_ids) == at
            assert paused.draws == (at if temperature > 0.0 else 0)
            assert not paused.complete
            resumed = provider.generate_checkpointed(request, paused)
            assert resumed.token_ids == whole.token_ids, (at, temperature)
            assert resumed.complete
        # a complete checkpoint resumes to itself without a forward
        assert provider.generate_checkpointed(request, whole) == whole


def test_commit_failure_stops_before_another_token_and_bad_draws_are_refused():
    """durable_generation.rs:67-105"""
    _, _, model = _tiny(64, 29)
    provider = DecoderProvider(model)
    calls = [0]
    request = GenerationRequest(prompt_ids=[1], max_tokens=6, temperature=0.8)

    def commit(cp):
        calls[0] = len(cp.token_ids)
        if len(cp.token_ids) == 2:
            raise Backend("disk full")

    with pytest.raises(Backend, match="disk full"):
        provider.generate_checkpointed(request, None, commit)
    assert calls[0] == 2
    cp = provider.generate_checkpointed(request, None, None, lambda: True)
    assert cp.request.seed is not None, "unseeded asks persist their actual seed before a draw"
    cp.draws = 8
    with pytest.raises(InvalidRequest):
        provider.generate_checkpointed(request, cp)
    # the persisted seed replays: resuming the untouched pause gives the same
    # stream as a fresh seeded run
    cp.draws = 0
    resumed = provider.generate_checkpointed(request, cp)
    seeded = GenerationRequest(prompt_ids=[1], max_tokens=6, temperature=0.8, seed=cp.request.seed)
    assert resumed.token_ids == provider.generate_checkpointed(seeded).token_ids
    # a different request against the checkpoint is refused
    with pytest.raises(InvalidRequest, match="differs"):
        provider.generate_checkpointed(GenerationRequest(prompt_ids=[2], max_tokens=6,
                                                         temperature=0.8), cp)


def _ok_grammar():
    return {"kind": "sequence", "items": [
        {"kind": "literal", "value": "{\"ok\":"},
        {"kind": "choice", "alternatives": [{"kind": "literal", "value": "true}"},
                                            {"kind": "literal", "value": "false}"}]}]}


def test_numerical_recovery_preserves_committed_prefix_and_sampling_draws():
    """provider.rs:981-1034: a NaN row at the first model-chosen token is
    recomputed once from the committed prefix; the stream, draws and
    checkpoint equal the fault-free run."""
    _, _, model = _tiny(256, 17)
    tok = byte_tokenizer()
    provider = FaultyProvider(model, tokenizer=tok)
    for temperature in (0.0, 0.7):
        r = GenerationRequest(prompt_ids=[ord("x")], max_tokens=64, temperature=temperature,
                              seed=17, output_grammar=_ok_grammar())
        full = provider.generate_checkpointed(r)
        assert full.complete
        assert bytes(full.token_ids).decode() in ('{"ok":true}', '{"ok":false}')
        provider.score_faults.add(6)
        recovered = provider.generate_checkpointed(r)
        assert recovered == full
        assert not provider.score_faults
    health = provider.score_health()
    assert health.invalid_rows == 2
    assert health.prefix_recomputations == 2
    assert health.failed_recoveries == 0


def test_repeated_numerical_fault_stops_before_a_second_token_decision():
    """provider.rs:1036-1104"""
    _, _, model = _tiny(256, 19)
    tok = byte_tokenizer()
    provider = FaultyProvider(model, tokenizer=tok)
    choice = {"kind": "choice", "alternatives": [{"kind": "literal", "value": "true"},
                                                 {"kind": "literal", "value": "false"}]}
    grammar = {"kind": "sequence", "items": [
        {"kind": "literal", "value": "{\"first\":"}, choice,
        {"kind": "literal", "value": ",\"second\":"}, choice, {"kind": "literal", "value": "}"}]}
    r = GenerationRequest(prompt_ids=[ord("x")], max_tokens=64, output_grammar=grammar)
    full = provider.generate_checkpointed(r)
    text = bytes(full.token_ids).decode()
    second = text.index("\"second\":") + 9
    provider.score_faults.update([9, second])
    last = []

    def commit(cp):
        last.append((list(cp.token_ids), cp.complete))

    with pytest.raises(Backend):
        provider.generate_checkpointed(r, None, commit)
    ids, complete = last[-1]
    assert not complete
    assert ids == full.token_ids[:second]
    assert not provider.score_faults
    health = provider.score_health()
    assert health.invalid_rows == 2
    assert health.prefix_recomputations == 1
    assert health.failed_recoveries == 1


def test_window_rule_early_eos_succeeds_and_overrun_is_refused():
    """generate.rs:134-170 over a cache that would pass the window: the
    reference refuses only the forward that passes max_position_embeddings
    (model.rs:547-556), so an eos before it ends the run normally."""
    cfg, tensors, model = _tiny(64, 31, max_pos=16)
    prompt = [3, 1, 4, 1]
    fits = 16 - len(prompt) + 1  # tokens the fitting forwards yield
    ids = generate_ids_with(model, prompt, fits, [], TokenPicker.greedy())
    assert ids == _oracle_stream(cfg, tensors, prompt, fits, 0.0, None, 0)
    # device loop and host loop: an eos inside the window -> the short list
    eos = ids[5]
    first = ids.index(eos)
    assert generate_ids_with(model, prompt, 100, [eos], TokenPicker.greedy()) == ids[:first]
    seen = []
    assert generate_ids_with(model, prompt, 100, [eos], TokenPicker.greedy(),
                             lambda t: seen.append(t) and False) == ids[:first]
    assert seen == ids[:first]
    # the KV handed in keeps exactly the fed tokens
    kv = model.new_cache(1, 16)
    try_generate_ids_with(model, prompt, 100, [eos], TokenPicker.greedy(), cache=kv)
    assert kv.position() == len(prompt) + first
    kv = model.new_cache(1, 16)
    try_generate_ids_with(model, prompt, 3, [], TokenPicker.greedy(), cache=kv)
    assert kv.position() == len(prompt) + 2
    # no eos before the window ends: the refused forward, on both loops
    with pytest.raises(InvalidRequest, match="context window"):
        generate_ids_with(model, prompt, 100, [], TokenPicker.greedy())
    with pytest.raises(InvalidRequest, match="context window"):
        generate_ids_with(model, prompt, 100, [], TokenPicker.greedy(), lambda t: False)
    # the provider clamps max_new to the window instead (provider.rs:508-516)
    provider = DecoderProvider(model)
    cp = provider.generate_checkpointed(GenerationRequest(prompt_ids=prompt, max_tokens=100))
    assert cp.complete and cp.token_ids == ids[:16 - len(prompt)]
