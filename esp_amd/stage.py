"""Layer-range stages and their chain, mirroring esp's stage seam.

crates/esp/src/infer/decoder/stage.rs: ``LayerRange``, ``StageCapacity`` /
``StageAssignment`` / ``assign_ranges`` (contiguous ranges within each
device's layer budget), ``layer_resident_bytes`` (the admission cost of one
layer), the lossless f32 hidden wire (``encode_hidden`` / ``decode_hidden``)
and ``DecoderStage`` (resident weights for one range, its own KV cache and
position rules; the final range may own the output head). A stage's layers
run in libesp_hip.so (``esp_stage_*``); on one GPU every stage of a chain
shares the card, and the wire between them is host memory.
"""
from __future__ import annotations

import ctypes as C
import struct
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np

from . import _lib
from .config import DecoderConfig
from .errors import Backend, InvalidConfig, InvalidRequest, InvalidWeights, Unsupported
from .streaming import LayerSource, SourceBridge, StreamingOptions, read_header

PACKED = {"q8-block32", "q8-k32-f32-scale-f16-shared-v1", "q4-block32",
          "q4-k32-f32-scale-f16-shared-v1"}


@dataclass(frozen=True)
class LayerRange:
    """stage.rs:20-36: layers first..end-1."""

    first: int
    end: int

    def validate(self, layers: int) -> None:
        if self.first >= self.end or self.end > layers:
            raise InvalidConfig("empty or out-of-model stage range")


@dataclass(frozen=True)
class StageCapacity:
    """stage.rs:38-46: layer memory a device offers after the host's
    reservations; device ids are distinct 32-byte identities."""

    device: bytes
    layer_bytes: int


@dataclass(frozen=True)
class StageAssignment:
    device: bytes
    range: LayerRange


def layer_resident_bytes(config: DecoderConfig, fmt: str = "f32") -> int:
    """stage.rs:53-128: runtime weights plus the whole context's K/V of one
    layer (tensor payload, not process memory)."""
    if config.num_attention_heads == 0 or config.kv_heads() == 0 or config.hidden_size == 0:
        raise InvalidConfig("invalid stage head dimensions")
    h = config.hidden_size
    kv = config.kv_heads() * config.head_dim()
    inter = config.intermediate_size
    if config.moe is not None:
        if fmt != "f32":
            raise Unsupported("MoE stage format", "only f32 expert execution is qualified")
        m = config.moe
        bank = h * 3 * (m.num_experts * m.moe_intermediate_size
                        + m.shared_expert_intermediate_size) + h * (m.num_experts + 1)
        dense = any(not config.layer_is_moe(i) for i in range(config.num_hidden_layers))
        mlp = max(bank, h * inter * 3) if dense else bank
    else:
        mlp = h * inter * 3
    projections = h * config.query_width() * 2 + h * kv * 2 + mlp
    scalar = 4 if fmt == "f32" else 2
    extra = ((config.query_width() + 2 * kv) if config.qkv_bias() else 0) \
        + (h if config.output_bias() else 0) + (2 * config.head_dim() if config.qk_norm() else 0)
    if fmt.startswith("q8"):
        weights = projections + projections // 32 * 4 + (2 * h + extra) * scalar
    elif fmt.startswith("q4"):
        weights = projections // 2 + projections // 32 * 4 + (2 * h + extra) * scalar
    else:
        weights = (projections + 2 * h + extra) * scalar
    total = weights + kv * config.max_position_embeddings * 2 * scalar
    if total >= 1 << 64:
        raise InvalidConfig("stage resident payload size overflow")
    return total


def assign_ranges(costs: Sequence[int], devices: Sequence[StageCapacity]) -> List[StageAssignment]:
    """stage.rs:131-172: fill each device in order with the longest
    contiguous run of layers its budget holds; a device that holds none is
    skipped."""
    ids = [d.device for d in devices]
    if not costs or 0 in costs or not devices or len(set(ids)) != len(ids):
        raise InvalidConfig("invalid stage costs or duplicate devices")
    first, out = 0, []
    for d in devices:
        end, left = first, d.layer_bytes
        while end < len(costs) and costs[end] <= left:
            left -= costs[end]
            end += 1
        if end > first:
            out.append(StageAssignment(d.device, LayerRange(first, end)))
            first = end
        if first == len(costs):
            return out
    raise InvalidConfig("available stage memory cannot hold all layers")


def encode_hidden(hidden: np.ndarray, limit: int) -> bytes:
    """stage.rs:191-220: u64 seq, u64 width, then f32 values little-endian;
    every value finite, the whole within ``limit`` bytes."""
    h = np.asarray(hidden, dtype=np.float32)
    if h.ndim == 3:
        if h.shape[0] != 1:
            raise InvalidRequest("hidden wire budget or shape")
        h = h[0]
    seq, width = h.shape
    if seq == 0 or width == 0 or 16 + seq * width * 4 > limit:
        raise InvalidRequest("hidden wire budget or shape")
    if not np.isfinite(h).all():
        raise Backend("nonfinite stage hidden")
    return struct.pack("<QQ", seq, width) + h.astype("<f4").tobytes()


def decode_hidden(data: bytes, width: int, max_seq: int, activation: str = "f32") -> np.ndarray:
    """stage.rs:222-265: the wire back to [seq, width] f32, refusing a wrong
    shape or length, non-finite values, and values not exact in the
    receiving stage's activation dtype ("f32", "bf16" or "f16"; this
    library's stages keep f32 activations in every weight format)."""
    if len(data) < 16:
        raise InvalidRequest("truncated hidden header")
    seq, wire_width = struct.unpack_from("<QQ", data, 0)
    if seq == 0 or seq > max_seq or wire_width != width or 16 + seq * width * 4 != len(data):
        raise InvalidRequest("hidden wire dimensions or length")
    v = np.frombuffer(data, "<f4", offset=16).astype(np.float32).reshape(seq, width)
    if not np.isfinite(v).all():
        raise InvalidRequest("nonfinite hidden values")
    if activation == "bf16":
        exact = (v.view(np.uint32) & 0xFFFF) == 0
    elif activation == "f16":
        exact = v.astype(np.float16).astype(np.float32) == v
    else:
        exact = np.ones_like(v, dtype=bool)
    if not exact.all():
        raise InvalidRequest("hidden values are not exact in the declared activation dtype")
    return v


class StageExecutor:
    """stage.rs:174-187: a synchronous stage seam."""

    def session_id(self) -> Optional[str]:
        return None

    def returns_logits(self) -> bool:
        return False

    def forward(self, hidden: np.ndarray, start: int) -> np.ndarray:
        raise NotImplementedError


class DecoderStage(StageExecutor):
    """stage.rs:280-527 on the MI355X: resident layers of one range."""

    def __init__(self, handle, config: DecoderConfig, rng: LayerRange, fmt: str, head: bool,
                 options: StreamingOptions, bridge: SourceBridge):
        self._h = handle
        self.config = config
        self.range = rng
        self.format = fmt
        self._head = head
        self.options = options
        self._bridge = bridge

    @staticmethod
    def from_source(config: DecoderConfig, rng: LayerRange, source: LayerSource,
                    options: Optional[StreamingOptions] = None, fmt: str = "f32",
                    shared: Optional[bytes] = None, max_ctx: int = 0) -> "DecoderStage":
        """from_source (+ with_output when ``shared`` is given: the final
        range's norm and head from the shared artifact)."""
        from .model import esp_config
        rng.validate(config.num_hidden_layers)
        options = options or StreamingOptions()
        options.validate()
        c, keep = esp_config(config, fmt)
        bridge = SourceBridge(source)
        src = _lib.EspLayerSource(bridge.fn, None, bridge.efn)
        opt = _lib.EspStreamingOptions(options.query_chunk, options.max_layer_bytes,
                                       options.max_shared_bytes)
        buf = (C.c_uint8 * len(shared)).from_buffer_copy(shared) if shared else None
        h = C.c_void_p()
        status = _lib.load().esp_stage_create(C.byref(c), rng.first, rng.end, C.byref(src),
                                              C.byref(opt), buf, len(shared or b""), max_ctx,
                                              C.byref(h))
        err = bridge.take()
        if status and err is not None:
            raise err
        _lib.check(status)
        del keep
        return DecoderStage(h, config, rng, fmt, shared is not None, options, bridge)

    def returns_logits(self) -> bool:
        return self._head

    def forward(self, hidden: np.ndarray, start: int) -> np.ndarray:
        h = np.ascontiguousarray(hidden, dtype=np.float32)
        if h.ndim == 3:
            if h.shape[0] != 1:
                raise InvalidRequest("stage hidden shape, dtype or context")
            h = h[0]
        if h.ndim != 2 or h.shape[1] != self.config.hidden_size:
            raise InvalidRequest("stage hidden shape, dtype or context")
        seq = h.shape[0]
        out = np.empty(self.config.vocab_size if self._head else (seq, self.config.hidden_size),
                       np.float32)
        _lib.check(_lib.load().esp_stage_forward(self._h, h.ctypes.data, seq, start,
                                                 out.ctypes.data))
        return out

    def forward_bytes(self, data: bytes, start: int, limit: int) -> bytes:
        """stage.rs:444-462: the wire in, the wire out (logits of the final
        stage travel as one row)."""
        if len(data) > limit:
            raise InvalidRequest("hidden wire budget")
        hidden = decode_hidden(data, self.config.hidden_size,
                               self.config.max_position_embeddings, "f32")
        out = self.forward(hidden, start)
        return encode_hidden(out.reshape(1, -1) if self._head else out, limit)

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.load().esp_stage_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()


class StageChain(StageExecutor):
    """A host chain of stages over contiguous ranges ending in the stage
    that owns the head, each hand-off through the f32 hidden wire."""

    def __init__(self, stages: Sequence[StageExecutor], wire_limit: int = 1 << 30):
        if not stages or not stages[-1].returns_logits():
            raise InvalidConfig("a complete chain ends with the stage that owns the head")
        ranges = [getattr(s, "range", None) for s in stages]
        if all(r is not None for r in ranges):
            if ranges[0].first != 0 or any(a.end != b.first for a, b in zip(ranges, ranges[1:])):
                raise InvalidConfig("stage ranges must be contiguous from layer 0")
        self.stages = list(stages)
        self.wire_limit = wire_limit

    def returns_logits(self) -> bool:
        return True

    def forward(self, hidden: np.ndarray, start: int) -> np.ndarray:
        wire = encode_hidden(hidden, self.wire_limit)
        for st in self.stages[:-1]:
            width = st.config.hidden_size
            wire = encode_hidden(st.forward(decode_hidden(wire, width, 1 << 62), start),
                                 self.wire_limit)
        last = self.stages[-1]
        return last.forward(decode_hidden(wire, last.config.hidden_size, 1 << 62), start)


def _embedding(shared: bytes, config: DecoderConfig) -> np.ndarray:
    hdr, start = read_header(shared)
    e = hdr.get("model.embed_tokens.weight")
    if e is None or list(e["shape"]) != [config.vocab_size, config.hidden_size]:
        raise InvalidWeights("shared artifact has no embedding of the declared shape")
    b, t = e["data_offsets"]
    raw = np.frombuffer(shared, np.uint8, count=t - b, offset=start + b)
    if e["dtype"] == "F32":
        v = raw.view("<f4").astype(np.float32)
    elif e["dtype"] == "BF16":
        v = (raw.view("<u2").astype(np.uint32) << 16).view(np.float32)
    elif e["dtype"] == "F16":
        v = raw.view("<f2").astype(np.float32)
    else:
        raise InvalidWeights(f"weight format: cannot import {e['dtype']} (model.embed_tokens.weight)")
    if not np.isfinite(v).all():
        raise InvalidWeights("weight format: non-finite weight in model.embed_tokens.weight")
    return v.reshape(config.vocab_size, config.hidden_size)


class StagedModel:
    """model.rs:417-432 with_stages: the embedding and the position stay with
    the host model; a complete chain returns the last position's logits."""

    def __init__(self, config: DecoderConfig, shared: bytes, chain: StageExecutor):
        if not chain.returns_logits():
            raise InvalidConfig("the stage chain must end with the output head")
        self.config = config
        self._embed = _embedding(shared, config)
        self.chain = chain
        self.position = 0

    def reset(self) -> None:
        self.position = 0

    def try_forward_cached_last(self, ids: Sequence[int]) -> np.ndarray:
        ids = [int(i) for i in ids]
        if not ids or self.position + len(ids) > self.config.max_position_embeddings:
            raise InvalidRequest("cached input is empty or exceeds the context window")
        if any(i < 0 or i >= self.config.vocab_size for i in ids):
            raise InvalidRequest("token id outside the vocabulary")
        logits = self.chain.forward(self._embed[ids], self.position)
        if logits.shape != (self.config.vocab_size,):
            raise Backend("final stage returned a different logits shape or dtype")
        self.position += len(ids)
        return logits
