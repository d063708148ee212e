"""Tokenizers and grammars shared by the constraint tests (no GPU needed).

byte_tokenizer() is the reference's own test tokenizer (constraint.rs:
352-371): one BPE token per byte, pieces in the GPT-2 byte alphabet, no
merges, ByteLevel decoder. trained_bpe() trains a small ByteLevel BPE on a
synthetic JSON-ish corpus, so tokens span several bytes, split UTF-8
sequences and mix quotes, escapes and literal syntax. llama_sized_table()
is a seeded 128256-entry token byte table of the same kinds of pieces.
"""
from __future__ import annotations

import json
import random
from typing import List

import numpy as np

_TOKENIZERS = None


def _tk():
    global _TOKENIZERS
    if _TOKENIZERS is None:
        import tokenizers
        _TOKENIZERS = tokenizers
    return _TOKENIZERS


def byte_alphabet_pieces() -> List[str]:
    printable = set(range(33, 127)) | set(range(161, 173)) | set(range(174, 256))
    out, n = [], 0
    for b in range(256):
        if b in printable:
            out.append(chr(b))
        else:
            out.append(chr(256 + n))
            n += 1
    return out


def byte_tokenizer():
    vocab = {p: b for b, p in enumerate(byte_alphabet_pieces())}
    desc = {"version": "1.0",
            "decoder": {"type": "ByteLevel", "add_prefix_space": False, "trim_offsets": False,
                        "use_regex": False},
            "model": {"type": "BPE", "vocab": vocab, "merges": []}}
    return _tk().Tokenizer.from_str(json.dumps(desc))


def corpus(n: int = 3000, seed: int = 7) -> List[str]:
    rng = random.Random(seed)
    words = ["value", "name", "ok", "true", "false", "null", "item_", "café", "→",
             "über", "日本", "\U0001F600", "\\n", "\\\"", "\\\\", "id", "x", "  ",
             "{\"", "\":", ",\"", "\"}", "[1,2]", "0.5", "-3", "été"]
    out = []
    for _ in range(n):
        k = rng.randint(2, 12)
        out.append("{\"" + "".join(rng.choice(words) for _ in range(k)) + "\"}")
    return out


def trained_bpe(vocab_size: int = 3000):
    tk = _tk()
    tok = tk.Tokenizer(tk.models.BPE())
    tok.pre_tokenizer = tk.pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)
    tok.decoder = tk.decoders.ByteLevel()
    trainer = tk.trainers.BpeTrainer(vocab_size=vocab_size, show_progress=False,
                                     initial_alphabet=tk.pre_tokenizers.ByteLevel.alphabet(),
                                     special_tokens=["<|end|>"])
    tok.train_from_iterator(corpus(), trainer)
    return tok


def L(v):
    return {"kind": "literal", "value": v}


def S(n):
    return {"kind": "json_string", "max_bytes": n}


def Q(*items):
    return {"kind": "sequence", "items": list(items)}


def C(*alts):
    return {"kind": "choice", "alternatives": list(alts)}


def grammars():
    """Named grammars covering literals, strings, choices with shared
    prefixes (wide frontiers), optional fields (choices with an empty
    alternative, i.e. chains of Splits) and non-ASCII literals."""
    enum64 = C(*[L(f"\"item_{i:02d}\"") for i in range(64)])
    opt = lambda k: C(L(""), Q(L(f",\"{k}\":"), S(6)))  # noqa: E731
    return {
        "object": Q(L("{\"v\":"), S(8), L("}")),
        "bool": Q(L("{\"ok\":"), C(L("true}"), L("false}"))),
        "enum64": Q(L("{\"e\":"), enum64, L("}")),
        "optional": Q(L("{\"a\":1"), opt("b"), opt("c"), opt("d"), L("}")),
        "nested": Q(L("["), C(Q(S(4), C(L(","), L(""))), L("null")), C(S(3), L("true")), L("]")),
        "unicode": Q(L("«café → "), S(12), L(" \U0001F600»")),
        "ambiguous": Q(C(L("ab"), L("a"), L("")), C(L("b\""), S(2)), L("!")),
        "strings": Q(S(1), L(":"), S(4096)),
    }


# the C5-grammar bench's token table (defined with the bench workload)
from bench import llama_sized_table  # noqa: E402,F401
