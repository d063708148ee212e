"""The library's host-side constraint (compile, accept, complete, forced
bytes) against the CPU oracle, through the C ABI. No GPU is needed: the
device tables are built only when a mask is first requested."""
from __future__ import annotations

import json
import random

import pytest

from esp_amd import InvalidRequest
from esp_amd.constraint import Constraint, Vocabulary, token_bytes
from oracle import constraint as ref
from tests.grammar_cases import C, L, Q, S, byte_tokenizer, grammars, trained_bpe


@pytest.fixture(scope="module")
def byte_tok():
    return byte_tokenizer()


@pytest.fixture(scope="module")
def bpe():
    return trained_bpe(1500)


def test_token_table_matches_oracle(byte_tok, bpe):
    assert token_bytes(byte_tok, 256) == ref.token_table(byte_tok, 256)
    v = bpe.get_vocab_size()
    assert token_bytes(bpe, v + 5) == ref.token_table(bpe, v + 5)
    # the added special token is excluded
    assert token_bytes(bpe, v)[bpe.token_to_id("<|end|>")] == b""


def test_reference_utf8_and_escapes_through_the_library(byte_tok):
    """constraint.rs:406-440 on the library's automaton."""
    vocab = Vocabulary.from_tokenizer(byte_tok, 256)
    c = Constraint(S(32), vocab=vocab)
    for b in "\"café → \\".encode():
        c.accept(b)
    with pytest.raises(InvalidRequest, match="violates"):
        c.accept(ord("x"))
    for b in b'n"':
        c.accept(b)
    assert c.complete()
    with pytest.raises(InvalidRequest):
        c.accept(ord('"'))
    for bad in [b'"\xed\xa0\x80"', b'"\xc0\x80"', b'"a\nb"', b'"\\uD800"', b'""']:
        c = Constraint(S(32), vocab=vocab)
        with pytest.raises(InvalidRequest):
            for b in bad:
                c.accept(b)
    c = Constraint(S(1), vocab=vocab)
    c.accept(34)
    for b in (92, 0xC3):
        with pytest.raises(InvalidRequest):
            c.accept(b)
    c.accept(97)
    with pytest.raises(InvalidRequest):
        c.accept(98)
    c.accept(34)
    assert c.complete()


def test_reference_forced_span(byte_tok):
    """constraint.rs:441-466, the forced and accept halves."""
    c = Constraint(Q(L("{\"v\":"), S(8), L("}")), byte_tok, 256)
    ids = c.forced(byte_tok)
    assert ids == list(b'{"v":"')
    for i in ids:
        c.accept(i)
    assert c.forced(byte_tok) == []
    for b in b'ok"}':
        c.accept(b)
    assert c.complete()
    with pytest.raises(InvalidRequest):
        c.accept(ord("\n"))
    with pytest.raises(InvalidRequest, match="1..4096"):
        Constraint(S(4097), byte_tok, 256)


def test_unsupported_tokens(bpe):
    v = bpe.get_vocab_size()
    c = Constraint(S(8), bpe, v + 3)
    for bad in (bpe.token_to_id("<|end|>"), v + 1, v + 3, 1 << 31):
        with pytest.raises(InvalidRequest, match="unsupported token"):
            c.accept(bad)


def test_non_byte_level_tokenizer_is_refused(byte_tok):
    desc = json.loads(byte_tok.to_str())
    desc["decoder"] = {"type": "Metaspace", "replacement": "_", "prepend_scheme": "always",
                       "split": True}
    import tokenizers
    t = tokenizers.Tokenizer.from_str(json.dumps(desc))
    with pytest.raises(InvalidRequest, match="ByteLevel"):
        Constraint(S(4), t, 256)


@pytest.mark.parametrize("grammar,msg", [
    ({"kind": "literal"}, "missing field `value`"),
    ({"kind": "literal", "value": "a", "items": []}, "unknown field"),
    ({"kind": "literal", "value": "a", "extra": 1}, "unknown field `extra`"),
    ({"kind": "json_string", "max_bytes": -1}, "negative"),
    ({"kind": "json_string", "max_bytes": 2.5}, "floating point"),
    ({"kind": "json_string", "max_bytes": 0}, "1..4096"),
    ({"kind": "choice", "alternatives": []}, "1..64"),
    ({"kind": "choice", "alternatives": [L("a")] * 65}, "1..64"),
    ({"kind": "regex", "value": "a"}, "unknown variant"),
    ({"value": "a"}, "missing field `kind`"),
    ('{"kind":"literal","value":"a","value":"b"}', "duplicate field"),
    ('{"kind":"literal","value":"\\ud800"}', "surrogate"),
    ('{"kind":"literal","value":"a"} x', "trailing"),
    ('[1]', "expected"),
])
def test_grammar_json_errors(byte_tok, grammar, msg):
    vocab = Vocabulary.from_tokenizer(byte_tok, 256)
    with pytest.raises(InvalidRequest, match=msg):
        Constraint(grammar, vocab=vocab)


def test_grammar_bounds_match_oracle(byte_tok):
    vocab = Vocabulary.from_tokenizer(byte_tok, 256)
    deep_ok, deep_bad = L("x"), L("x")
    for _ in range(24):
        deep_ok = Q(deep_ok)
    for _ in range(25):
        deep_bad = Q(deep_bad)
    Constraint(deep_ok, vocab=vocab)
    for g, msg in [(deep_bad, "exceeds its bounds"), (L("a" * 262145), "literals exceed"),
                   (L("a" * 100000), "state bound")]:
        with pytest.raises(InvalidRequest, match=msg):
            Constraint(g, vocab=vocab)
        with pytest.raises(ref.GrammarError, match=msg):
            ref.compile_grammar(g)
    Constraint(L("a" * 99999), vocab=vocab)
    ref.compile_grammar(L("a" * 99999))


def test_escaped_grammar_literals(byte_tok):
    vocab = Vocabulary.from_tokenizer(byte_tok, 256)
    text = '{"kind":"literal","value":"\\"\\\\\\/\\b\\f\\n\\r\\t\\u00e9\\ud83d\\ude00"}'
    c = Constraint(text, vocab=vocab)
    want = "\"\\/\b\f\n\r\té\U0001F600".encode()
    assert c.forced_bytes() == want


def _walk(grammar, vocab_tokens, vocab, seed, steps=40):
    rng = random.Random(seed)
    lib = Constraint(grammar, vocab=vocab)
    orc = ref.Constraint(grammar, vocab_tokens)
    for _ in range(steps):
        assert lib.complete() == orc.complete()
        assert lib.forced_bytes() == orc.forced_bytes()
        ok = orc.allowed()
        good = [i for i, a in enumerate(ok) if a]
        bad = [i for i, a in enumerate(ok) if not a and vocab_tokens[i]]
        for t in rng.sample(bad, min(3, len(bad))):
            with pytest.raises(InvalidRequest):
                lib.accept(t)
        if not good:
            break
        t = rng.choice(good)
        lib.accept(t)
        orc.accept(t)


@pytest.mark.parametrize("name", sorted(grammars()))
def test_random_walks_match_oracle(byte_tok, bpe, name):
    g = grammars()[name]
    for tok, seed in ((byte_tok, 1), (bpe, 2)):
        n = tok.get_vocab_size()
        table = token_bytes(tok, n)
        _walk(g, table, Vocabulary(table), seed)
