"""Device grammar mask and constrained picking vs the CPU constraint oracle.

Bit-exact: every allowed-token bit the device computes must equal the
oracle's (constraint.rs:274-295), over random walks through each grammar,
for the reference's byte tokenizer, a trained multi-byte BPE and a
Llama-3-sized (128256-entry) synthetic token table."""
from __future__ import annotations

import json
import math
import random

import numpy as np
import pytest

from esp_amd import DecoderModel, InvalidRequest, Sampler, TokenPicker, generate_constrained
from esp_amd.constraint import Constraint, Vocabulary, token_bytes
from oracle import constraint as ref
from oracle import oracle, st
from tests import synth
from tests.grammar_cases import (C, L, Q, S, byte_tokenizer, grammars, llama_sized_table,
                                 trained_bpe)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def byte_tok():
    return byte_tokenizer()


@pytest.fixture(scope="module")
def bpe():
    return trained_bpe(3000)


def bits_of(words) -> np.ndarray:
    return np.asarray(words, np.uint32)


def _compare_walk(grammar, table, vocab, seed, steps):
    rng = random.Random(seed)
    lib = Constraint(grammar, vocab=vocab)
    orc = ref.Constraint(grammar, table)
    for step in range(steps):
        want = bits_of(orc.allowed_bits())
        got = lib.allowed_bits()
        if not np.array_equal(got, want):
            diff = np.nonzero(np.unpackbits((got ^ want).view(np.uint8), bitorder="little"))[0]
            raise AssertionError(f"step {step}: {len(diff)} tokens differ, first "
                                 f"{[(int(i), table[i]) for i in diff[:5]]}")
        assert lib.complete() == orc.complete()
        good = np.nonzero(np.unpackbits(want.view(np.uint8), bitorder="little"))[0]
        if len(good) == 0:
            break
        t = int(good[rng.randrange(len(good))])
        lib.accept(t)
        orc.accept(t)


def test_reference_mask_cases_on_device(byte_tok):
    """constraint.rs:441-494 mask assertions with the device bits."""
    c = Constraint(Q(L("{\"v\":"), S(8), L("}")), byte_tok, 256)
    for i in c.forced(byte_tok):
        c.accept(i)
    row = np.zeros(256, np.float32)
    c.mask(row)
    assert np.isinf(row[10]) and np.isinf(row[34]) and np.isfinite(row[97])
    c = Constraint(C(L("a"), L("b")), byte_tok, 256)
    for bad in (math.nan, math.inf, -math.inf):
        row = np.zeros(256, np.float32)
        row[ord("a")] = bad
        row[ord("b")] = 2.0
        c.mask(row)
        assert row[ord("a")] == -np.inf
        assert oracle.argmax(row) == ord("b")
    row = np.full(256, np.nan, np.float32)
    row[ord("b")] = np.inf
    with pytest.raises(InvalidRequest, match="no finite eligible"):
        c.mask(row)
    assert np.all(row == -np.inf)


# (lane capacity, wave capacity, string-class table): defaults; string
# states walked; every live token walked by its wave; by the block kernel;
# and small capacities that mix all three.
WALKS = [(8, 64, 1), (8, 64, 0), (0, 64, 0), (0, 0, 0), (1, 2, 1)]


def _walk_env(monkeypatch, lane_cap, wave_cap, strclass):
    monkeypatch.setenv("ESP_CMASK_LANE_CAP", str(lane_cap))
    monkeypatch.setenv("ESP_CMASK_WAVE_CAP", str(wave_cap))
    monkeypatch.setenv("ESP_CMASK_STRCLASS", str(strclass))


@pytest.mark.parametrize("lane_cap,wave_cap,strclass", WALKS)
@pytest.mark.parametrize("name", sorted(grammars()))
def test_device_mask_matches_oracle(byte_tok, bpe, name, lane_cap, wave_cap, strclass,
                                    monkeypatch):
    _walk_env(monkeypatch, lane_cap, wave_cap, strclass)
    print(f"grammar {name} walks {lane_cap} {wave_cap} {strclass}", flush=True)
    g = grammars()[name]
    for tok, seed in ((byte_tok, 3), (bpe, 4)):
        n = tok.get_vocab_size()
        table = token_bytes(tok, n + 7)
        _compare_walk(g, table, Vocabulary(table), seed, 24)


@pytest.mark.parametrize("lane_cap,wave_cap,strclass", WALKS)
@pytest.mark.parametrize("name", ["object", "enum64", "optional", "unicode"])
def test_device_mask_llama_sized_vocab(name, lane_cap, wave_cap, strclass, monkeypatch):
    _walk_env(monkeypatch, lane_cap, wave_cap, strclass)
    print(f"grammar {name} V=128256 walks {lane_cap} {wave_cap} {strclass}", flush=True)
    table = llama_sized_table()
    _compare_walk(grammars()[name], table, Vocabulary(table), 9, 4)


def test_wide_frontier_tokens_take_the_block_walk(bpe):
    """64 alternatives alive after a shared prefix (plus the continuation):
    frontiers above the wave capacity go through the block kernel; bits
    still match the oracle."""
    alts = [L(f"pre_fix_{i:02d}_" + "x" * (i % 5)) for i in range(64)]
    g = Q(L("<"), C(*alts), L(">"))
    table = [bytes([b]) for b in range(256)] + [b"pre_fix_", b"_fix_", b"fix_0", b"pre_fix_1",
                                               b"e_fix_3", b"x>", b"xx", b"_x", b"pre", b"_0"]
    _compare_walk(g, table, Vocabulary(table), 5, 30)
    n = bpe.get_vocab_size()
    table = token_bytes(bpe, n)
    _compare_walk(g, table, Vocabulary(table), 6, 30)


def _model(vocab: int, seed: int):
    cfg = synth.llama_config(1, 64, 4, 2, 96, vocab)
    tensors = synth.make_tensors(cfg, seed, "f32", std=0.2)
    return DecoderModel.from_bytes(cfg, st.dump(tensors), "f32")


def test_pick_constrained_matches_oracle(bpe):
    """provider.rs:744-817 on a batch: rows masked by their own constraints
    (one unconstrained), greedy and sampled ids equal to the oracle's."""
    V = bpe.get_vocab_size() + 3
    model = _model(V, 31)
    table = token_bytes(bpe, V)
    vocab = Vocabulary(table)
    names = ["object", "enum64", "optional", None, "unicode"]
    n = len(names)
    lib = [None if k is None else Constraint(grammars()[k], vocab=vocab) for k in names]
    orc = [None if k is None else ref.Constraint(grammars()[k], table) for k in names]
    kv = model.new_cache(n, 64)
    prompts = [synth.uniform_ids(40 + i, 5, V) for i in range(n)]
    logits = model.forward_batch(kv, list(range(n)), prompts, want_logits=True)
    samplers = [Sampler(0.8, 0.9, 500 + i) for i in range(n)]
    for step in range(6):
        greedy, _ = model.pick_constrained(kv, lib)
        states = [s.rng.state for s in samplers]
        sampled, _ = model.pick_constrained(kv, lib, samplers)
        for i in range(n):
            if orc[i] is None:
                row = logits[i]
            else:
                row, cnt = oracle.mask(logits[i], np.asarray(orc[i].allowed_bits(), np.uint32))
                assert cnt > 0
            assert greedy[i] == oracle.argmax(row), (step, i)
            tok, st2 = oracle.sample(row, 0.8, 0.9, states[i])
            assert sampled[i] == tok and samplers[i].rng.state == st2, (step, i)
        for i in range(n):
            if lib[i] is not None:
                lib[i].accept(int(greedy[i]))
                orc[i].accept(int(greedy[i]))
                if orc[i].complete():  # nothing is eligible after the end
                    lib[i] = orc[i] = None
        logits = model.forward_batch(kv, list(range(n)), [[int(t)] for t in greedy],
                                     want_logits=True)


def test_generate_constrained_matches_oracle_loop(byte_tok):
    """The provider's constrained loop on the device vs the same loop run
    with the oracle's mask and forced spans over the device logits."""
    model = _model(256, 17)
    g = Q(L("{\"ok\":"), C(L("true}"), L("false}")))
    for gram in (g, grammars()["object"]):
        c = Constraint(gram, byte_tok, 256)
        ids, done = generate_constrained(model, [1, 2, 3], 40, [], TokenPicker.greedy(), c,
                                         byte_tok)
        assert done
        json.loads(bytes(ids).decode())
        # oracle loop
        o = ref.Constraint(gram, ref.token_table(byte_tok, 256))
        kv = model.new_cache(1, 64)
        logits = model.try_forward_cached_last([1, 2, 3], kv)
        want = []
        while not o.complete():
            forced = o.forced(byte_tok)
            if forced:
                toks = forced
            else:
                row, _ = oracle.mask(logits, np.asarray(o.allowed_bits(), np.uint32))
                toks = [oracle.argmax(row)]
            fed = []
            for t in toks:
                o.accept(t)
                want.append(t)
                fed.append(t)
                if o.complete():
                    break
            if not o.complete():
                logits = model.try_forward_cached_last(fed, kv)
        assert ids == want
    # a limit reached before completion is refused
    c = Constraint(grammars()["object"], byte_tok, 256)
    with pytest.raises(InvalidRequest, match="token limit"):
        generate_constrained(model, [1, 2, 3], 3, [], TokenPicker.greedy(), c, byte_tok)
    # sampled: forced spans skip one draw per token
    c = Constraint(g, byte_tok, 256)
    s = Sampler(0.7, None, 17)
    ids, done = generate_constrained(model, [1, 2, 3], 40, [], TokenPicker.sampled(s), c,
                                     byte_tok)
    assert done and bytes(ids).decode() in ('{"ok":true}', '{"ok":false}')
