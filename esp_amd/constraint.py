"""Constrained decoding, mirroring crates/esp/src/infer/decoder/constraint.rs.

The automaton (compile, accept, complete, the forced byte span) runs in the
HIP library's host code and the token mask runs on the device
(`esp_constraint_mask`, `esp_pick_constrained`); this module derives the
token byte table from a `tokenizers.Tokenizer`, tokenises forced spans and
keeps the reference's method names and errors.

Grammars use the serde form of OutputGrammar (provider.rs:55-75): dicts
tagged by "kind". `literal`, `json_string`, `sequence` and `choice` build
them.
"""
from __future__ import annotations

import ctypes as C
import json
from typing import List, Optional, Sequence, Tuple, Union

import numpy as np

from . import _lib
from .errors import InvalidRequest


def literal(value: str) -> dict:
    """OutputGrammar::Literal (provider.rs:62-64)"""
    return {"kind": "literal", "value": value}


def json_string(max_bytes: int) -> dict:
    """OutputGrammar::JsonString (provider.rs:65-69)"""
    return {"kind": "json_string", "max_bytes": max_bytes}


def sequence(items: Sequence[dict]) -> dict:
    """OutputGrammar::Sequence (provider.rs:70-72)"""
    return {"kind": "sequence", "items": list(items)}


def choice(alternatives: Sequence[dict]) -> dict:
    """OutputGrammar::Choice (provider.rs:73-75)"""
    return {"kind": "choice", "alternatives": list(alternatives)}


def _byte_alphabet() -> dict:
    # constraint.rs:125-139: bytes 33..126, 161..172 and 174..255 stand for
    # themselves; every other byte, in increasing order, is written as the
    # scalar 256 + k.
    keep = set(range(33, 127)) | set(range(161, 173)) | set(range(174, 256))
    table = {}
    k = 0
    for b in range(256):
        if b in keep:
            table[chr(b)] = b
        else:
            table[chr(256 + k)] = b
            k += 1
    return table


_ALPHABET = _byte_alphabet()


def token_bytes(tokenizer, vocabulary: int) -> List[bytes]:
    """constraint.rs:114-154: the byte string of every token id below
    `vocabulary`. Added tokens, ids the tokenizer lacks and pieces outside
    the byte alphabet are empty (never allowed)."""
    desc = json.loads(tokenizer.to_str())
    if (desc.get("decoder") or {}).get("type") != "ByteLevel":
        raise InvalidRequest("constrained decoding requires a ByteLevel decoder")
    added = {int(t["id"]) for t in desc.get("added_tokens") or [] if "id" in t}
    out = [b""] * vocabulary
    for piece, tid in tokenizer.get_vocab(with_added_tokens=False).items():
        if tid >= vocabulary or tid in added:
            continue
        raw = [_ALPHABET.get(c) for c in piece]
        if all(b is not None for b in raw):
            out[tid] = bytes(raw)
    return out


class Vocabulary:
    """A token byte table in the library (esp_vocab)."""

    def __init__(self, tokens: Sequence[bytes]):
        self.tokens = [bytes(t) for t in tokens]
        offs = np.zeros(len(self.tokens) + 1, np.uint32)
        offs[1:] = np.cumsum([len(t) for t in self.tokens], dtype=np.uint64)
        blob = np.frombuffer(b"".join(self.tokens) or b"\0", np.uint8)
        h = C.c_void_p()
        _lib.check(_lib.load().esp_vocab_create(
            blob.ctypes.data, offs.ctypes.data_as(C.POINTER(C.c_uint32)), len(self.tokens),
            C.byref(h)))
        self._h = h

    @staticmethod
    def from_tokenizer(tokenizer, vocabulary: int) -> "Vocabulary":
        return Vocabulary(token_bytes(tokenizer, vocabulary))

    def __len__(self) -> int:
        return len(self.tokens)

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.load().esp_vocab_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()


class Constraint:
    """constraint.rs:37-344 `Constraint`.

    `Constraint(grammar, tokenizer, vocabulary)` as the reference's `new`, or
    `Constraint(grammar, vocab=Vocabulary)` to share one token table between
    many requests."""

    def __init__(self, grammar: Union[dict, str], tokenizer=None,
                 vocabulary: Optional[int] = None, vocab: Optional[Vocabulary] = None):
        if vocab is None:
            if tokenizer is None or vocabulary is None:
                raise InvalidRequest("constraint needs a tokenizer and vocabulary size")
            vocab = Vocabulary.from_tokenizer(tokenizer, vocabulary)
        self.vocab = vocab
        text = grammar if isinstance(grammar, str) else json.dumps(grammar)
        raw = text.encode("utf-8")
        h = C.c_void_p()
        _lib.check(_lib.load().esp_constraint_create(vocab._h, raw, len(raw), C.byref(h)))
        self._h = h

    def accept(self, token: int) -> None:
        """constraint.rs:261-273"""
        if not 0 <= token < 1 << 32:
            raise InvalidRequest("constraint encountered an unsupported token")
        _lib.check(_lib.load().esp_constraint_accept(self._h, token))

    def complete(self) -> bool:
        """constraint.rs:256-260"""
        v = C.c_uint8()
        _lib.check(_lib.load().esp_constraint_complete(self._h, C.byref(v)))
        return bool(v.value)

    def allowed_bits(self, stream: Optional[int] = None) -> np.ndarray:
        """The device-computed eligibility bitmask, ceil(V/32) u32 words."""
        words = np.zeros((len(self.vocab) + 31) // 32, np.uint32)
        _lib.check(_lib.load().esp_constraint_mask(
            self._h, stream, None, words.ctypes.data_as(C.POINTER(C.c_uint32))))
        return words

    def mask(self, row: np.ndarray) -> None:
        """constraint.rs:274-295 on a host float32 row, in place: disallowed
        or non-finite scores become -inf; no finite eligible token raises."""
        bits = self.allowed_bits()
        ok = np.unpackbits(bits.view(np.uint8), bitorder="little")[:len(row)].astype(bool)
        if len(ok) < len(row):
            ok = np.concatenate([ok, np.zeros(len(row) - len(ok), bool)])
        keep = ok & np.isfinite(row)
        row[~keep] = -np.inf
        if not keep.any():
            raise InvalidRequest("output grammar has no finite eligible token")

    def forced_bytes(self) -> bytes:
        """constraint.rs:296-318: the unique-byte continuation."""
        buf = (C.c_uint8 * 4096)()
        n = C.c_uint32()
        _lib.check(_lib.load().esp_constraint_forced_bytes(self._h, buf, 4096, C.byref(n)))
        return bytes(buf[:n.value])

    def forced(self, tokenizer) -> List[int]:
        """constraint.rs:296-344: the forced span, canonically tokenised,
        refused unless its tokens' bytes reproduce it exactly."""
        data = self.forced_bytes()
        if not data:
            return []
        try:
            ids = tokenizer.encode(data.decode("utf-8"), add_special_tokens=False).ids
        except Exception as e:  # tokenizer failure -> InvalidRequest
            raise InvalidRequest(str(e)) from None
        toks = self.vocab.tokens
        actual = b"".join(toks[i] if 0 <= i < len(toks) else b"" for i in ids)
        if actual != data:
            raise InvalidRequest("forced grammar span does not round-trip through tokenizer")
        return list(ids)

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.load().esp_constraint_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()


def constraint_handles(constraints: Sequence[Optional[Constraint]]) -> Tuple[C.Array, list]:
    arr = (C.c_void_p * len(constraints))()
    for i, c in enumerate(constraints):
        arr[i] = None if c is None else c._h.value
    return arr, list(constraints)
