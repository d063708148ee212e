"""Host rules of the durable provider that run before any device work:
request admission and the window rule (provider.rs:474-517) and the
checkpoint validation of generate_checkpointed (provider.rs:612-705). The
model is a stub holding only a config, so any device call would fail."""
from __future__ import annotations

import math

import pytest

from esp_amd import InvalidRequest, PromptTooLong, Unsupported
from esp_amd.provider import DecoderProvider, GenerationCheckpoint, GenerationRequest
from tests import synth


class _StubModel:
    def __init__(self, max_pos=16, vocab=64):
        self.config = synth.llama_config(1, 64, 4, 2, 96, vocab, max_pos=max_pos)


def _provider():
    return DecoderProvider(_StubModel(), eos_token_ids=[0])


def test_prepare_generation_refusals_and_window():
    p = _provider()
    with pytest.raises(InvalidRequest, match="empty prompt"):
        p.prepare_generation(GenerationRequest(prompt_ids=[], max_tokens=4))
    with pytest.raises(InvalidRequest, match="max_tokens is 0"):
        p.prepare_generation(GenerationRequest(prompt_ids=[1], max_tokens=0))
    for t in (-0.1, math.nan, math.inf):
        with pytest.raises(InvalidRequest, match="temperature must be finite"):
            p.prepare_generation(GenerationRequest(prompt_ids=[1], max_tokens=4, temperature=t))
    with pytest.raises(PromptTooLong) as e:
        p.prepare_generation(GenerationRequest(prompt_ids=list(range(16)), max_tokens=4))
    assert (e.value.length, e.value.limit) == (16, 16)
    ids, max_new, picker = p.prepare_generation(GenerationRequest(prompt_ids=[1, 2, 3, 4],
                                                                  max_tokens=100))
    assert ids == [1, 2, 3, 4] and max_new == 12 and picker.sampler is None
    _, max_new, picker = p.prepare_generation(GenerationRequest(prompt_ids=[1], max_tokens=5,
                                                                temperature=0.5, seed=9))
    assert max_new == 5 and picker.sampler.rng.state == 9


def _cp(request, **kw):
    base = dict(request=request, prompt_ids=list(request.prompt_ids), token_ids=[], draws=0,
                complete=False)
    base.update(kw)
    return GenerationCheckpoint(**base)


def test_checkpoint_validation_before_any_forward():
    p = _provider()
    r = GenerationRequest(prompt_ids=[1, 2], max_tokens=6, temperature=0.8, seed=3)
    with pytest.raises(Unsupported):
        p.generate_checkpointed(GenerationRequest(prompt_ids=[1], max_tokens=2, stop=["x"]))
    other = GenerationRequest(prompt_ids=[1, 2], max_tokens=7, temperature=0.8, seed=3)
    with pytest.raises(InvalidRequest, match="differs"):
        p.generate_checkpointed(other, _cp(r))
    bad = [_cp(r, token_ids=[5, 6], draws=1),             # draws != committed ids
           _cp(r, token_ids=[5, 64], draws=2),            # id outside the vocabulary
           _cp(r, token_ids=[5] * 7, draws=7),            # more ids than max_new
           _cp(r, prompt_ids=[1, 3])]                     # prompt differs
    for cp in bad:
        with pytest.raises(InvalidRequest, match="invalid generation checkpoint"):
            p.generate_checkpointed(r, cp)
    greedy = GenerationRequest(prompt_ids=[1, 2], max_tokens=6)
    with pytest.raises(InvalidRequest, match="invalid generation checkpoint"):
        p.generate_checkpointed(greedy, _cp(greedy, token_ids=[4], draws=1))
    # an unseeded resume takes the checkpoint's seed
    unseeded = GenerationRequest(prompt_ids=[1, 2], max_tokens=6, temperature=0.8)
    done = _cp(r, token_ids=[4, 5], draws=2, complete=True)
    assert p.generate_checkpointed(unseeded, done) == done
    # a complete checkpoint returns without a forward (the stub has none)
    assert p.generate_checkpointed(r, done) == done


def test_paused_resume_commits_before_the_window_check():
    p = _provider()
    r = GenerationRequest(prompt_ids=[1, 2, 3, 4], max_tokens=100)
    cp = _cp(r, token_ids=[9] * 12)
    seen = []
    # stop() at the first boundary: the committed checkpoint comes back as is
    out = p.generate_checkpointed(r, cp, lambda c: seen.append(len(c.token_ids)), lambda: True)
    assert out == cp and seen == [12]
    with pytest.raises(PromptTooLong):
        p.generate_checkpointed(r, cp)
