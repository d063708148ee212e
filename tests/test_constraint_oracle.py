"""The CPU constraint oracle against the reference's own tests and brute force.

The four tests of constraint.rs:372-494 are restated on the oracle; the
JSON-string automaton is checked exhaustively on short byte strings against
Python's strict UTF-8 decoder and json module, so a wrong range, phase or
bound fails here.
"""
from __future__ import annotations

import itertools
import json
import math

import pytest

from oracle.constraint import Constraint, GrammarError, compile_grammar, token_table
from tests.grammar_cases import C, L, Q, S, byte_tokenizer, grammars, trained_bpe


@pytest.fixture(scope="module")
def tok():
    return byte_tokenizer()


def make(g, tok, v=256):
    return Constraint(g, token_table(tok, v))


def test_byte_tokenizer_table_is_identity(tok):
    t = token_table(tok, 256)
    assert t == [bytes([b]) for b in range(256)]
    assert token_table(tok, 300)[256:] == [b""] * 44


def test_every_accepted_small_string_is_valid_json(tok):
    """constraint.rs:372-404"""
    alphabet = [32, 34, 47, 92, 97, 110, 114, 116, 117, 120, 10, 0xC3, 0xA9, 0xE0, 0xED, 0xA0,
                0x80, 0xF4, 0x8F, 0xBF]
    accepted = 0

    def walk(c, state, raw):
        nonlocal accepted
        if any(c.nodes[p[0]][0] == "end" for p in state):
            value = json.loads(bytes(raw).decode("utf-8"))
            assert isinstance(value, str) and value
            accepted += 1
            return
        for b in alphabet:
            nxt = c.step(state, b)
            if nxt:
                raw.append(b)
                walk(c, nxt, raw)
                raw.pop()

    for mx in range(1, 5):
        c = make(S(mx), tok)
        walk(c, c.active, [])
    assert accepted > 1000


def test_utf8_split_tokens_and_escapes_are_exact_and_bounded(tok):
    """constraint.rs:406-440"""
    c = make(S(32), tok)
    for b in "\"café → \\".encode():
        c.accept(b)
    with pytest.raises(GrammarError):
        c.accept(ord("x"))
    for b in b'n"':
        c.accept(b)
    assert c.complete()
    with pytest.raises(GrammarError):
        c.accept(ord('"'))
    for bad in [b'"\xed\xa0\x80"', b'"\xc0\x80"', b'"a\nb"', b'"\\uD800"', b'""']:
        c = make(S(32), tok)
        with pytest.raises(GrammarError):
            for b in bad:
                c.accept(b)
    c = make(S(1), tok)
    c.accept(34)
    for b in (92, 0xC3):
        with pytest.raises(GrammarError):
            c.accept(b)
    c.accept(97)
    with pytest.raises(GrammarError):
        c.accept(98)
    c.accept(34)
    assert c.complete()


def test_masking_and_forced_spans_refuse_extra_syntax(tok):
    """constraint.rs:441-466"""
    g = Q(L("{\"v\":"), S(8), L("}"))
    c = make(g, tok)
    ids = c.forced(tok)
    assert ids == list(b'{"v":"')
    for i in ids:
        c.accept(i)
    row = [0.0] * 256
    c.mask(row)
    assert math.isinf(row[10]) and math.isinf(row[34]) and math.isfinite(row[97])
    for b in b'ok"}':
        c.accept(b)
    assert c.complete()
    with pytest.raises(GrammarError):
        c.accept(ord("\n"))
    with pytest.raises(GrammarError):
        make(S(4097), tok)


def test_nonfinite_scores_cannot_win_or_create_an_eligible_choice(tok):
    """constraint.rs:467-494"""
    c = make(C(L("a"), L("b")), tok)
    for bad in (math.nan, math.inf, -math.inf):
        row = [0.0] * 256
        row[ord("a")] = bad
        row[ord("b")] = 2.0
        c.mask(row)
        assert row[ord("a")] == -math.inf
        assert max(range(256), key=lambda i: row[i]) == ord("b")
    row = [math.nan] * 256
    row[ord("b")] = math.inf
    with pytest.raises(GrammarError):
        c.mask(row)
    assert all(v == -math.inf for v in row)


# JSON string content the automaton must accept: valid UTF-8, no raw
# control bytes, only the short escapes; `max` counts encoded bytes.


def _string_ok(raw: bytes, mx: int) -> bool:
    if len(raw) < 3 or raw[0] != 0x22 or raw[-1] != 0x22:
        return False
    body = raw[1:-1]
    if not 1 <= len(body) <= mx:
        return False
    try:
        body.decode("utf-8")
    except UnicodeDecodeError:
        return False
    i = 0
    while i < len(body):
        b = body[i]
        if b < 0x20 or b == 0x22:
            return False
        if b == 0x5C:
            if i + 1 >= len(body) or body[i + 1] not in b'"\\/bfnrt':
                return False
            i += 2
            continue
        i += 1
    # every accepted string is valid JSON text for a non-empty string
    assert isinstance(json.loads(raw.decode("utf-8")), str)
    return True


def test_json_string_automaton_matches_brute_force(tok):
    """Every string over a byte alphabet that hits each range edge, up to
    four bytes after the opening quote, walked depth-first from the parent
    state: done-ness must equal the brute-force predicate."""
    alphabet = [0x22, 0x5C, 0x61, 0x6E, 0x75, 0x1F, 0x20, 0x7F, 0xC2, 0xC3, 0xA9, 0xBF, 0x80,
                0xE0, 0xA0, 0xED, 0x9F, 0xF0, 0x90, 0xF4, 0x8F, 0xF5, 0xC1]
    for mx in (1, 2, 3, 4):
        c = make(S(mx), tok)
        checked = 0

        def walk(state, raw):
            nonlocal checked
            done = any(c.nodes[p[0]][0] == "end" for p in state)
            assert done == _string_ok(bytes(raw), mx), (mx, bytes(raw))
            checked += 1
            if len(raw) == 5:
                return
            for b in alphabet:
                nxt = c.step(state, b) if state else []
                raw.append(b)
                walk(nxt, raw)
                raw.pop()

        walk(c.step(c.active, 0x22), [0x22])
        assert checked == sum(23 ** k for k in range(5))


def test_compile_bounds():
    with pytest.raises(GrammarError):
        compile_grammar(S(0))
    with pytest.raises(GrammarError):
        compile_grammar(C())
    with pytest.raises(GrammarError):
        compile_grammar(C(*[L("a")] * 65))
    deep = L("x")
    for _ in range(25):
        deep = Q(deep)
    with pytest.raises(GrammarError):
        compile_grammar(deep)
    ok = L("x")
    for _ in range(24):
        ok = Q(ok)
    compile_grammar(ok)
    with pytest.raises(GrammarError):
        compile_grammar(L("a" * 262145))
    with pytest.raises(GrammarError, match="state bound"):
        compile_grammar(L("a" * 262144))
    nodes, start = compile_grammar(Q(L("ab"), S(3)))
    assert [n[0] for n in nodes] == ["end", "string", "byte", "byte"] and start == 3


def test_forced_stops_at_choice_and_utf8_boundary(tok):
    c = make(Q(L("x"), C(L("éa"), L("éb"))), tok)
    # both alternatives share the two bytes of U+00E9; then a choice
    assert c.forced_bytes() == "xé".encode()
    c = make(Q(L("x"), C(L("é"), L("ê"))), tok)
    # the common lead byte 0xC3 alone is not valid UTF-8 and is cut
    assert c.forced_bytes() == b"x"


def test_trained_bpe_table_and_oracle_mask_consistency():
    t = trained_bpe(800)
    table = token_table(t, t.get_vocab_size())
    assert sum(len(x) > 1 for x in table) > 200
    g = grammars()["object"]
    c = Constraint(g, table)
    ok = c.allowed()
    # allowed tokens are exactly those whose bytes the automaton walks
    for i, data in enumerate(table[:400]):
        assert ok[i] == (bool(data) and bool(c.after(data)))
