"""esp_pick_noalloc (device inputs and outputs, scratch in the library's fixed
device array, no allocation) against esp_pick on the same device logits:
ids, flags and advanced sampler states identical, on two calls in a row
(the second over fewer rows), masked and unmasked, sampled and greedy."""
import ctypes as C

import numpy as np
import pytest

from esp_amd import DecoderModel, Sampler, _lib
from esp_amd.errors import InvalidRequest
from oracle import st
from tests import synth

pytestmark = pytest.mark.gpu

SAMPLER = np.dtype([("temperature", "<f4"), ("top_p", "<f4"), ("state", "<u8")])


def _bits(rng, n, vocab, frac):
    words = (vocab + 31) // 32
    allow = rng.random((n, words * 32)) < frac
    allow[:, vocab:] = False
    allow[np.arange(n), rng.integers(0, vocab, n)] = True
    return np.packbits(allow, axis=1, bitorder="little").view(np.uint32).copy()


def _noalloc(kv, n, bits, smp):
    """One esp_pick_noalloc call with every buffer in device memory."""
    import torch
    dev = torch.device("cuda")
    d_bits = None if bits is None else torch.from_numpy(bits.reshape(-1).view(np.int32)).to(dev)
    d_smp = None if smp is None else torch.from_numpy(smp.view(np.uint8)).to(dev)
    d_ids = torch.full((n,), -1, dtype=torch.int32, device=dev)
    d_flags = torch.full((n,), 0xEE, dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    rc = _lib.load().esp_pick_noalloc(kv._h, n, None if d_bits is None else d_bits.data_ptr(),
                                      None if d_smp is None else d_smp.data_ptr(),
                                      d_ids.data_ptr(), d_flags.data_ptr())
    _lib.check(rc)
    torch.cuda.synchronize()
    states = None if d_smp is None else d_smp.cpu().numpy().view(SAMPLER)["state"].copy()
    return d_ids.cpu().numpy().view(np.uint32), d_flags.cpu().numpy(), states


def _compare(model, kv, n, bits, temps, top_p, seed):
    """esp_pick (host buffers) and esp_pick_noalloc from the same states."""
    samplers = None
    smp = None
    if temps is not None:
        samplers = [None if t <= 0 else Sampler(t, top_p, seed + i) for i, t in enumerate(temps)]
        smp = np.zeros(n, SAMPLER)
        for i, s in enumerate(samplers):
            if s is not None:
                smp[i] = (s.temperature, -1.0 if s.top_p is None else s.top_p, s.rng.state)
            else:
                smp[i] = (0.0, -1.0, 0)
    ids_d, flags_d, states_d = _noalloc(kv, n, bits, smp)
    ids_h, flags_h = model.pick(kv, n, bits, samplers)
    assert np.array_equal(ids_d, ids_h), (ids_d, ids_h)
    assert np.array_equal(flags_d, flags_h)
    if samplers is not None:
        for i, s in enumerate(samplers):
            want = s.rng.state if s is not None else 0
            assert int(states_d[i]) == want, i
    return ids_h


def test_pick_noalloc_matches_pick():
    V = 40000
    cfg = synth.llama_config(1, 64, 4, 2, 96, V)
    tensors = synth.make_tensors(cfg, 77, "f32", std=0.2)
    model = DecoderModel.from_bytes(cfg, st.dump(tensors), "f32")
    rng = np.random.default_rng(3)
    kv = model.new_cache(8, 32)
    # call 1: 8 rows, 60% masks, T 0.8 / top-p 0.9 with two greedy rows
    model.forward_batch(kv, list(range(8)), [synth.uniform_ids(50 + i, 6, V) for i in range(8)])
    print("noalloc: 8 sampled rows", flush=True)
    bits = _bits(rng, 8, V, 0.6)
    _compare(model, kv, 8, bits, [0.8, 0.8, 0.0, 0.8, 0.8, 0.0, 0.8, 0.8], 0.9, 100)
    # call 2: fewer rows (3), unmasked, no nucleus, over a new forward
    model.forward_batch(kv, [0, 1, 2], [[7], [8], [9]])
    print("noalloc: 3 sampled rows", flush=True)
    _compare(model, kv, 3, None, [1.3, 1.3, 1.3], None, 200)
    # greedy masked rows need no sampling scratch
    print("noalloc: greedy masked", flush=True)
    bits = _bits(rng, 3, V, 0.05)
    _compare(model, kv, 3, bits, None, None, 0)
    # a request beyond the fixed scratch is refused, nothing launched
    kv40 = model.new_cache(40, 16)
    model.forward_batch(kv40, list(range(40)), [[i + 1] for i in range(40)])
    smp = np.zeros(40, SAMPLER)
    smp["temperature"], smp["top_p"] = 0.8, -1.0
    with pytest.raises(InvalidRequest, match="above the fixed"):
        _noalloc(kv40, 40, None, smp)
    # the entry point still works after the refusal
    _compare(model, kv40, 4, None, [0.9, 0.9, 0.9, 0.9], 0.5, 300)
