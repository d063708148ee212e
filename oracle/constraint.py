"""CPU restatement of esp's byte-grammar constraint (test infrastructure).

THIS IS THE PARITY CHECKER, NOT THE PRODUCT. Only tests/, the smoke check
and bench.py's cpu_baseline leg import it. The product's constraint lives in
esp_amd/csrc/constraint.cpp (host automaton) and k_constraint.hip (device
mask); esp_amd/constraint.py drives them through the C ABI.

Restates crates/esp/src/infer/decoder/constraint.rs:
  compile             constraint.rs:63-113  (nodes, bounds)
  token_table         constraint.rs:114-154 (ByteLevel alphabet inverse)
  close               constraint.rs:158-169
  step                constraint.rs:170-245
  after               constraint.rs:246-255
  complete            constraint.rs:256-260
  accept              constraint.rs:261-273
  mask / allowed      constraint.rs:274-295
  forced              constraint.rs:296-344
Pinned by the reference's own tests (constraint.rs:346-495), restated in
tests/test_constraint_oracle.py, and by a brute-force check of every short
byte string against Python's UTF-8 decoder and json module.

Grammars are the serde form of OutputGrammar (provider.rs:55-75): dicts
tagged by "kind" = literal | json_string | sequence | choice.
"""
from __future__ import annotations

import json
from typing import Dict, List, Optional, Sequence, Tuple

# node kinds (constraint.rs:10-16)
END, BYTE, SPLIT, STRING = "end", "byte", "split", "string"

Position = Tuple[int, int, int, int, int]  # node, used, phase, low, high


class GrammarError(ValueError):
    """InvalidRequest raised while building a constraint."""


def at(node: int) -> Position:
    return (node, 0, 0, 0, 0)


def compile_grammar(grammar: dict) -> Tuple[list, int]:
    """constraint.rs:63-113. Returns (nodes, start)."""
    nodes: list = [(END,)]
    budget = [0]

    def comp(g: dict, nxt: int, depth: int) -> int:
        if depth > 24 or len(nodes) > 100_000 or budget[0] > 262_144:
            raise GrammarError("output grammar exceeds its bounds")
        kind = g["kind"]
        if kind == "literal":
            value = g["value"].encode("utf-8")
            budget[0] += len(value)
            if budget[0] > 262_144:
                raise GrammarError("output grammar literals exceed their bound")
            cur = nxt
            for b in reversed(value):
                nodes.append((BYTE, b, cur))
                cur = len(nodes) - 1
            return cur
        if kind == "json_string":
            mb = g["max_bytes"]
            if not 1 <= mb <= 4096:
                raise GrammarError("JSON string bound must be 1..4096")
            nodes.append((STRING, mb, nxt))
            return len(nodes) - 1
        if kind == "sequence":
            cur = nxt
            for item in reversed(g["items"]):
                cur = comp(item, cur, depth + 1)
            return cur
        if kind == "choice":
            alts = g["alternatives"]
            if not 1 <= len(alts) <= 64:
                raise GrammarError("grammar choice must have 1..64 alternatives")
            ids = [comp(a, nxt, depth + 1) for a in alts]
            nodes.append((SPLIT, ids))
            return len(nodes) - 1
        raise GrammarError(f"unknown grammar kind {kind!r}")

    start = comp(grammar, 0, 0)
    if len(nodes) > 100_000:
        raise GrammarError("compiled output grammar exceeds its state bound")
    return nodes, start


def byte_alphabet_inverse() -> Dict[str, int]:
    """constraint.rs:125-139: the GPT-2 byte alphabet. Printable bytes map to
    themselves; the rest map, in byte order, to scalars 256, 257, ..."""
    printable = set(range(33, 127)) | set(range(161, 173)) | set(range(174, 256))
    inv: Dict[str, int] = {}
    extra = 0
    for b in range(256):
        if b in printable:
            inv[chr(b)] = b
        else:
            inv[chr(256 + extra)] = b
            extra += 1
    return inv


def token_table(tokenizer, vocabulary: int) -> List[bytes]:
    """constraint.rs:114-154 for a `tokenizers.Tokenizer`: the byte string of
    every id below `vocabulary`; added tokens and pieces outside the
    alphabet stay empty."""
    desc = json.loads(tokenizer.to_str())
    if (desc.get("decoder") or {}).get("type") != "ByteLevel":
        raise GrammarError("constrained decoding requires a ByteLevel decoder")
    inv = byte_alphabet_inverse()
    added = {int(t["id"]) for t in (desc.get("added_tokens") or []) if "id" in t}
    tokens = [b""] * vocabulary
    for piece, tid in tokenizer.get_vocab(with_added_tokens=False).items():
        if tid >= vocabulary or tid in added:
            continue
        try:
            tokens[tid] = bytes(inv[c] for c in piece)
        except KeyError:
            pass
    return tokens


class Constraint:
    """The reference's Constraint over a token table."""

    def __init__(self, grammar: dict, tokens: Sequence[bytes]):
        self.nodes, start = compile_grammar(grammar)
        self.tokens = list(tokens)
        self.active = self.close([at(start)])

    def close(self, positions: List[Position]) -> List[Position]:
        """constraint.rs:158-169"""
        out = []
        stack = list(positions)
        while stack:
            p = stack.pop()
            n = self.nodes[p[0]]
            if n[0] == SPLIT:
                stack.extend(at(i) for i in n[1])
            else:
                out.append(p)
        return sorted(set(out))

    def step(self, active: Sequence[Position], byte: int) -> List[Position]:
        """constraint.rs:170-245"""
        out = []
        for p in active:
            node, used, phase, low, high = p
            n = self.nodes[node]
            if n[0] == BYTE:
                if n[1] == byte:
                    out.append(at(n[2]))
                continue
            if n[0] != STRING:
                continue
            mx, nxt = n[1], n[2]
            if phase == 0:
                if byte == 0x22:
                    out.append((node, used, 1, low, high))
                continue
            if phase == 1 and byte == 0x22:
                if used > 0:
                    out.append(at(nxt))
                continue
            if used >= mx:
                continue
            q_used, q_phase, q_low, q_high = used + 1, phase, low, high
            if phase == 1:
                if byte == 0x5C and used + 2 <= mx:
                    q_phase = 2
                elif 0x20 <= byte <= 0x7F and byte not in (0x22, 0x5C):
                    pass
                elif 0xC2 <= byte <= 0xDF and used + 2 <= mx:
                    q_phase, q_low, q_high = 3, 0x80, 0xBF
                elif 0xE0 <= byte <= 0xEF and used + 3 <= mx:
                    q_phase = 4
                    q_low = 0xA0 if byte == 0xE0 else 0x80
                    q_high = 0x9F if byte == 0xED else 0xBF
                elif 0xF0 <= byte <= 0xF4 and used + 4 <= mx:
                    q_phase = 5
                    q_low = 0x90 if byte == 0xF0 else 0x80
                    q_high = 0x8F if byte == 0xF4 else 0xBF
                else:
                    continue
            elif phase == 2:
                if byte not in b'"\\/bfnrt':
                    continue
                q_phase = 1
            elif phase in (3, 4, 5):
                if byte < low or byte > high:
                    continue
                q_phase = 1 if phase == 3 else phase - 1
                q_low, q_high = 0x80, 0xBF
            else:
                continue
            out.append((node, q_used, q_phase, q_low, q_high))
        return self.close(out)

    def after(self, data: bytes, state: Optional[List[Position]] = None) -> List[Position]:
        """constraint.rs:246-255"""
        state = list(self.active if state is None else state)
        for b in data:
            state = self.step(state, b)
            if not state:
                break
        return state

    def complete(self) -> bool:
        """constraint.rs:256-260"""
        return any(self.nodes[p[0]][0] == END for p in self.active)

    def accept(self, token: int) -> None:
        """constraint.rs:261-273"""
        data = self.tokens[token] if 0 <= token < len(self.tokens) else b""
        if not data:
            raise GrammarError("constraint encountered an unsupported token")
        state = self.after(data)
        if not state:
            raise GrammarError("token violates output grammar")
        self.active = state

    def allowed(self) -> List[bool]:
        """The eligibility half of constraint.rs:274-295: token non-empty and
        after(bytes) non-empty. after() of a token is the step of after() of
        its prefix, so prefix states are memoised (same values)."""
        memo: Dict[bytes, Tuple[Position, ...]] = {b"": tuple(self.active)}

        def state_of(data: bytes) -> Tuple[Position, ...]:
            s = memo.get(data)
            if s is None:
                prev = state_of(data[:-1])
                s = tuple(self.step(prev, data[-1])) if prev else ()
                memo[data] = s
            return s

        return [bool(t) and bool(state_of(t)) for t in self.tokens]

    def allowed_bits(self) -> "list[int]":
        """allowed() packed as ceil(V/32) u32 words, bit id%32 of word id/32."""
        ok = self.allowed()
        words = [0] * ((len(ok) + 31) // 32)
        for i, a in enumerate(ok):
            if a:
                words[i >> 5] |= 1 << (i & 31)
        return words

    def mask(self, row: list) -> None:
        """constraint.rs:274-295 on a Python list of floats, in place."""
        ok = self.allowed()
        anyok = False
        for i in range(len(row)):
            allowed = i < len(ok) and ok[i]
            v = row[i]
            finite = v == v and v not in (float("inf"), float("-inf"))
            if not allowed or not finite:
                row[i] = float("-inf")
            else:
                anyok = True
        if not anyok:
            raise GrammarError("output grammar has no finite eligible token")

    def forced_bytes(self) -> bytes:
        """constraint.rs:296-318"""
        state = list(self.active)
        out = bytearray()
        for _ in range(4096):
            if any(self.nodes[p[0]][0] == END for p in state):
                break
            live = [(b, s) for b in range(256) for s in [self.step(state, b)] if s]
            if len(live) != 1:
                break
            out.append(live[0][0])
            state = live[0][1]
        while True:
            try:
                bytes(out).decode("utf-8")
                break
            except UnicodeDecodeError:
                out.pop()
        return bytes(out)

    def forced(self, tokenizer) -> List[int]:
        """constraint.rs:296-344"""
        data = self.forced_bytes()
        if not data:
            return []
        ids = tokenizer.encode(data.decode("utf-8"), add_special_tokens=False).ids
        actual = b"".join(self.tokens[i] if 0 <= i < len(self.tokens) else b"" for i in ids)
        if actual != data:
            raise GrammarError("forced grammar span does not round-trip through tokenizer")
        return list(ids)
