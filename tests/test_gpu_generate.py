"""The device greedy loop (esp_generate_greedy) against the host-driven loop
of generate.rs:134-170: stopping at eos after about as many forwards as the
reference takes, and any max_new up to UINT32_MAX at the C ABI."""
import numpy as np
import pytest

from esp_amd import DecoderModel, TokenPicker
from esp_amd.generate import try_generate_ids_with
from esp_amd.errors import InvalidRequest
from esp_amd.model import profile_enable, profile_read
from tests import synth

pytestmark = pytest.mark.gpu

U32_MAX = 0xFFFFFFFF


def _host_loop(model, prompt, max_new, eos, max_ctx=None):
    # a per-token callback keeps the host-driven loop (one forward per token)
    cache = model.new_cache(1, max_ctx) if max_ctx else None
    return try_generate_ids_with(model, prompt, max_new, eos, TokenPicker.greedy(),
                                 on_token=lambda _t: False, cache=cache)


def _first_new(ids, lo):
    """Index >= lo of the first id not seen before it (an eos that ends the
    run exactly there)."""
    for i in range(lo, len(ids)):
        if ids[i] not in ids[:i]:
            return i
    return None


def _forwards():
    return profile_read("greedy_forwards")[0]


def test_device_greedy_stops_at_eos():
    """max_new 512 with eos at about step 5: ids equal the host loop's and
    the forwards issued stay within the chunk that holds the eos (chunks of
    4 then 8), not max_new."""
    cfg, _, blob, prompt = synth.tiny_llama_case(41, 2, 128, 4, 2, 192, 512, 12, max_pos=1024)
    model = DecoderModel.from_bytes(cfg, blob, "f32")
    full = _host_loop(model, prompt, 40, [])
    i = _first_new(full, 5)
    assert i is not None and i < 12, full
    eos = full[i]
    want = _host_loop(model, prompt, 512, [eos])
    assert want == full[:i]
    profile_enable("greedy_forwards")
    got = model.generate_greedy_device(model.new_cache(1, 1024), prompt, 512, [eos])
    n = _forwards()
    profile_enable("greedy_forwards", False)
    print("eos index", i, "forwards", n)
    assert got == want
    # the reference runs i forwards; the loop may finish the chunk holding it
    assert i <= n <= 12
    # without eos the loop runs every forward max_new asks for
    profile_enable("greedy_forwards")
    got = model.generate_greedy_device(model.new_cache(1, 1024), prompt, 40, [])
    n = _forwards()
    profile_enable("greedy_forwards", False)
    assert got == full and n == 39


def test_device_greedy_eos_on_first_token():
    """An eos picked from the prefill logits ends the call with no forward."""
    cfg, _, blob, prompt = synth.tiny_llama_case(43, 2, 128, 4, 2, 192, 512, 9)
    model = DecoderModel.from_bytes(cfg, blob, "f32")
    first = _host_loop(model, prompt, 1, [])[0]
    profile_enable("greedy_forwards")
    got = model.generate_greedy_device(model.new_cache(1, 64), prompt, 512, [first])
    n = _forwards()
    profile_enable("greedy_forwards", False)
    assert got == [] and n == 0


def test_device_greedy_max_new_u32_max():
    """max_new = UINT32_MAX (a 'no limit' value at the C ABI) on a small
    window: with an eos inside the window the call succeeds with the host
    loop's ids; without one it fails as the forward past the window does
    (model.rs:547-556), like the host loop."""
    cfg, _, blob, prompt = synth.tiny_llama_case(47, 2, 128, 4, 2, 192, 512, 10, max_pos=1024)
    model = DecoderModel.from_bytes(cfg, blob, "f32")
    window = 24
    full = _host_loop(model, prompt, window - len(prompt) + 1, [], max_ctx=window)
    assert len(full) == window - len(prompt) + 1
    i = _first_new(full, 3)
    assert i is not None, full
    eos = full[i]
    got = model.generate_greedy_device(model.new_cache(1, window), prompt, U32_MAX, [eos])
    assert got == full[:i]
    # no eos: the forward past the window is refused, by both loops
    absent = next(t for t in range(cfg.vocab_size) if t not in full)
    with pytest.raises(InvalidRequest):
        model.generate_greedy_device(model.new_cache(1, window), prompt, U32_MAX, [absent])
    with pytest.raises(InvalidRequest):
        _host_loop(model, prompt, 10 ** 6, [absent], max_ctx=window)
    # the handle still works afterwards
    again = model.generate_greedy_device(model.new_cache(1, window), prompt, U32_MAX, [eos])
    assert again == full[:i]


def test_device_greedy_chunks_match_host_loop_bf16():
    """A bf16 model over 70 steps (chunks 4 + 8 + 16 + 32 + the rest): the
    replayed chunks give the host loop's ids."""
    cfg, _, blob, prompt = synth.tiny_llama_case(53, 2, 256, 4, 2, 320, 700, 20, fmt="bf16",
                                                 max_pos=256)
    model = DecoderModel.from_bytes(cfg, blob, "bf16")
    want = _host_loop(model, prompt, 70, [])
    got = model.generate_greedy_device(model.new_cache(1, 128), prompt, 70, [])
    assert got == want
    assert np.all(np.asarray(got) < cfg.vocab_size)
