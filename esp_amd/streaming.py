"""Layer sources and artifacts for streamed decoding, mirroring esp's host side.

crates/esp/src/infer/decoder/streaming.rs (``LayerSource``,
``with_expert_reader``, ``cache_verified_layers``, ``StreamingOptions``,
the read statistics) and decoder/checkpoint.rs (splitting a checkpoint into
one shared artifact and one safetensors artifact per layer). The device side
(staging each artifact into HBM, checking it, running the layer) lives in
libesp_hip.so behind ``DecoderModel.from_layer_source``; this module only
moves bytes and enforces the byte limits.
"""
from __future__ import annotations

import ctypes as C
import json
import struct
import threading
from concurrent.futures import ThreadPoolExecutor
from dataclasses import asdict, dataclass
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np

from .config import DecoderConfig
from .errors import Backend, InferError, InvalidConfig, InvalidWeights


@dataclass
class StreamingOptions:
    """streaming.rs:172-202: per-provider limits, all positive."""

    query_chunk: int = 32
    max_layer_bytes: int = 256 * 1024 * 1024
    max_shared_bytes: int = 1024 * 1024 * 1024

    def validate(self) -> None:
        if self.query_chunk <= 0 or self.max_layer_bytes <= 0 or self.max_shared_bytes <= 0:
            raise InvalidConfig("streaming limits must be positive")

    def to_json(self) -> str:
        return json.dumps(asdict(self))

    @staticmethod
    def from_json(text: str) -> "StreamingOptions":
        """serde(deny_unknown_fields): every field present, nothing else."""
        raw = json.loads(text)
        names = {"query_chunk", "max_layer_bytes", "max_shared_bytes"}
        if not isinstance(raw, dict) or set(raw) != names or not all(
                isinstance(raw[k], int) and not isinstance(raw[k], bool) and raw[k] >= 0
                for k in names):
            raise InvalidConfig("streaming options: expected exactly query_chunk, "
                                "max_layer_bytes and max_shared_bytes as unsigned integers")
        return StreamingOptions(**raw)


@dataclass
class LayerCacheStats:
    """streaming.rs:83-91 host allocation accounting of the verified cache."""

    hits: int = 0
    misses: int = 0
    retained_capacity_bytes: int = 0
    entries: int = 0
    capacity_budget_bytes: int = 0


@dataclass
class DeviceLayerCacheStats:
    """streaming.rs:204-220 logical tensor payload kept in HBM."""

    hits: int = 0
    misses: int = 0
    retained_payload_bytes: int = 0
    payload_budget_bytes: int = 0
    layers: int = 0


@dataclass
class StreamingReadStats:
    """streaming.rs:222-238 logical verified artifact reads."""

    layer_reads: int = 0
    encoded_bytes_read: int = 0
    largest_encoded_layer: int = 0
    expert_reads: int = 0
    expert_encoded_bytes_read: int = 0
    largest_encoded_expert: int = 0
    verified_cache: Optional[LayerCacheStats] = None
    device_cache: Optional[DeviceLayerCacheStats] = None


class Artifact(bytes):
    """Artifact bytes that may sit in a larger allocation: ``capacity`` is
    what a verified cache charges against its budget (streaming.rs:129-138
    counts Vec capacity, not length)."""

    capacity: int

    def __new__(cls, data: bytes, capacity: Optional[int] = None):
        obj = super().__new__(cls, data)
        obj.capacity = len(data) if capacity is None else max(capacity, len(data))
        return obj


def _capacity(b) -> int:
    return getattr(b, "capacity", len(b))


class LayerSource:
    """streaming.rs:17-37: a host-owned source of verified standalone layer
    artifacts. ``read_layer`` must check the declared size against ``limit``
    before reading and verify content identity before returning bytes."""

    def read_layer(self, index: int, limit: int) -> bytes:
        raise NotImplementedError

    def read_layer_shared(self, index: int, limit: int) -> bytes:
        return self.read_layer(index, limit)

    def cache_stats(self) -> Optional[LayerCacheStats]:
        return None

    def read_expert(self, layer: int, expert: int, limit: int) -> bytes:
        raise InvalidWeights("layer source has no expert reader")


class FnSource(LayerSource):
    """streaming.rs:177-184: any ``f(index, limit) -> bytes`` is a source."""

    def __init__(self, read: Callable[[int, int], bytes]):
        self._read = read

    def read_layer(self, index: int, limit: int) -> bytes:
        return self._read(index, limit)


def with_expert_reader(layers: Callable[[int, int], bytes],
                       experts: Callable[[int, int, int], bytes]) -> LayerSource:
    """streaming.rs:41-66: compose a layer reader and an expert reader."""

    class _Readers(LayerSource):
        def read_layer(self, index, limit):
            return layers(index, limit)

        def read_expert(self, layer, expert, limit):
            return experts(layer, expert, limit)

    return _Readers()


def cache_verified_layers(source: LayerSource, budget: int) -> LayerSource:
    """streaming.rs:93-170: cache verified immutable artifacts by index.

    First-fit admission, at most 128 entries and ``budget`` bytes of
    allocation capacity; hits return the same object and re-check the
    caller's limit; errors and oversized reads are never cached; experts
    keep the uncached path. ``budget`` 0 returns ``source`` itself."""
    if budget == 0:
        return source

    class _Cached(LayerSource):
        def __init__(self):
            self._lock = threading.Lock()
            self._entries: List[Tuple[int, bytes]] = []
            self._stats = LayerCacheStats(capacity_budget_bytes=budget)

        def read_layer(self, index, limit):
            return bytes(self.read_layer_shared(index, limit))

        def read_layer_shared(self, index, limit):
            with self._lock:
                for key, data in self._entries:
                    if key == index:
                        if len(data) > limit:
                            raise InvalidWeights("cached layer exceeds its byte limit")
                        self._stats.hits += 1
                        return data
                self._stats.misses += 1
                data = source.read_layer_shared(index, limit)
                if len(data) > limit:
                    raise InvalidWeights("layer source exceeded its byte limit")
                cap = _capacity(data)
                st = self._stats
                if len(self._entries) < 128 and cap <= st.capacity_budget_bytes - st.retained_capacity_bytes:
                    st.retained_capacity_bytes += cap
                    self._entries.append((index, data))
                    st.entries = len(self._entries)
                return data

        def read_expert(self, layer, expert, limit):
            return source.read_expert(layer, expert, limit)

        def cache_stats(self):
            with self._lock:
                return LayerCacheStats(**asdict(self._stats))

    return _Cached()


class ArtifactSource(LayerSource):
    """Verified in-memory artifacts (one per layer), the shape of a host
    reader over an artifact index (layer_library.rs:107-140): the declared
    byte size is checked against ``limit`` before the bytes are handed out,
    and against the bytes themselves."""

    def __init__(self, artifacts: Sequence[bytes],
                 experts: Optional[Dict[Tuple[int, int], bytes]] = None):
        self._artifacts = list(artifacts)
        self._experts = experts

    def read_layer(self, index: int, limit: int) -> bytes:
        if index >= len(self._artifacts):
            raise InvalidWeights(f"layer library: missing layer artifact {index}")
        data = self._artifacts[index]
        if len(data) > limit:
            raise InvalidWeights("layer library: layer artifact identity, schema or byte limit "
                                 "mismatch")
        return data

    def read_expert(self, layer: int, expert: int, limit: int) -> bytes:
        if self._experts is None:
            return super().read_expert(layer, expert, limit)
        data = self._experts.get((layer, expert))
        if data is None:
            raise InvalidWeights(f"layer library: missing expert artifact {layer}/{expert}")
        if len(data) > limit:
            raise InvalidWeights("layer library: expert artifact identity, schema or byte limit "
                                 "mismatch")
        return data


# ---- safetensors artifacts (checkpoint.rs:246-292 pack) ----

_ALIGN = {"F64": 8, "I64": 8, "U64": 8, "F32": 4, "I32": 4, "U32": 4, "F16": 2, "BF16": 2,
          "I16": 2, "U16": 2, "I8": 1, "U8": 1, "BOOL": 1}


def read_header(buf) -> Tuple[Dict[str, dict], int]:
    """The safetensors header of ``buf``: tensor entries and the data start."""
    if len(buf) < 8:
        raise InvalidWeights("checkpoint: invalid safetensors header length")
    (n,) = struct.unpack_from("<Q", buf, 0)
    if n > len(buf) - 8 or n > 100_000_000:
        raise InvalidWeights("checkpoint: invalid safetensors header length")
    header = json.loads(bytes(buf[8:8 + n]))
    header.pop("__metadata__", None)
    return header, 8 + n


def pack(entries: Sequence[Tuple[str, str, Sequence[int], bytes]]) -> bytes:
    """Serialize (name, dtype, shape, raw bytes) tensors: data ordered by
    dtype alignment (largest first) then name, header padded with spaces to
    8 bytes, as the safetensors crate writes them."""
    order = sorted(entries, key=lambda e: (-_ALIGN.get(e[1], 1), e[0]))
    header, off, blobs = {}, 0, []
    for name, dt, shape, data in order:
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(data)]}
        off += len(data)
        blobs.append(bytes(data))
    text = json.dumps(header, separators=(",", ":")).encode()
    text += b" " * ((8 - len(text) % 8) % 8)
    return struct.pack("<Q", len(text)) + text + b"".join(blobs)


def layer_tensor_names(config: DecoderConfig) -> List[str]:
    """loader.rs:48-64 per-layer tensors of a dense Llama block."""
    names = ["input_layernorm.weight", "post_attention_layernorm.weight",
             "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
             "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
             "mlp.down_proj.weight"]
    if config.qkv_bias():
        names += ["self_attn.q_proj.bias", "self_attn.k_proj.bias", "self_attn.v_proj.bias"]
    if config.output_bias():
        names.append("self_attn.o_proj.bias")
    if config.qk_norm():
        names += ["self_attn.q_norm.weight", "self_attn.k_norm.weight"]
    return names


def layer_core_tensor_names(config: DecoderConfig, index: int) -> List[str]:
    """loader.rs:66-85: a routed-expert layer's core artifact holds the
    router and the shared expert (when the configuration declares one) in
    place of the dense MLP; its experts are separate artifacts."""
    names = layer_tensor_names(config)
    if config.layer_is_moe(index):
        names = [n for n in names if not n.startswith("mlp.")] + ["mlp.gate.weight"]
        if config.moe.shared_expert_intermediate_size:
            names += ["mlp.shared_expert_gate.weight", "mlp.shared_expert.gate_proj.weight",
                      "mlp.shared_expert.up_proj.weight", "mlp.shared_expert.down_proj.weight"]
    return names


def expert_tensor_names(layer: int, expert: int) -> List[str]:
    """loader.rs:87-91"""
    return [f"model.layers.{layer}.mlp.experts.{expert}.{n}.weight"
            for n in ("gate_proj", "up_proj", "down_proj")]


class CheckpointReader:
    """checkpoint.rs:47-293 over one safetensors checkpoint held in memory:
    the declared names are checked once, then the shared artifact, each
    layer's core artifact and each routed expert's artifact are packed on
    request within a byte limit."""

    def __init__(self, checkpoint: bytes, config: DecoderConfig):
        self._buf = memoryview(checkpoint)
        self._header, self._start = read_header(self._buf)
        self._config = config
        want = {"model.embed_tokens.weight", "model.norm.weight"}
        for i in range(config.num_hidden_layers):
            want |= {f"model.layers.{i}.{s}" for s in layer_core_tensor_names(config, i)}
            if config.layer_is_moe(i):
                for e in range(config.moe.num_experts):
                    want |= set(expert_tensor_names(i, e))
        if not config.tie_word_embeddings or "lm_head.weight" in self._header:
            want.add("lm_head.weight")
        have = {n for n in self._header if not n.endswith(".rotary_emb.inv_freq")}
        if want != have:
            raise InvalidWeights("checkpoint: tensor names do not match the declared Llama block")

    def _pack(self, names: List[str], limit: int) -> bytes:
        total = 0
        for n in names:
            b, e = self._header[n]["data_offsets"]
            total += e - b
        if total > limit:
            raise InvalidWeights("checkpoint: artifact tensor data exceeds configured byte limit")
        entries = []
        for n in names:
            h = self._header[n]
            b, e = h["data_offsets"]
            entries.append((n, h["dtype"], h["shape"], self._buf[self._start + b:self._start + e]))
        out = pack(entries)
        if len(out) > limit:
            raise InvalidWeights("checkpoint: encoded artifact exceeds configured byte limit")
        return out

    def shared_bytes(self, limit: int) -> bytes:
        names = [n for n in ("model.embed_tokens.weight", "model.norm.weight", "lm_head.weight")
                 if n in self._header]
        return self._pack(names, limit)

    def layer_bytes(self, index: int, limit: int) -> bytes:
        return self._pack([f"model.layers.{index}.{s}"
                           for s in layer_core_tensor_names(self._config, index)], limit)

    def expert_bytes(self, layer: int, expert: int, limit: int) -> bytes:
        """checkpoint.rs:231-244"""
        c = self._config
        if (layer >= c.num_hidden_layers or not c.layer_is_moe(layer)
                or expert >= c.moe.num_experts):
            raise InvalidWeights("checkpoint: expert outside the declared sparse layer")
        return self._pack(expert_tensor_names(layer, expert), limit)


def split_checkpoint(checkpoint: bytes, config: DecoderConfig,
                     options: Optional[StreamingOptions] = None) -> Tuple[bytes, List[bytes]]:
    """layer_library.rs:211-266 import without the store: the shared
    artifact and one artifact per layer, each within the options' limits."""
    options = options or StreamingOptions()
    options.validate()
    r = CheckpointReader(checkpoint, config)
    return (r.shared_bytes(options.max_shared_bytes),
            [r.layer_bytes(i, options.max_layer_bytes) for i in range(config.num_hidden_layers)])


def split_experts(checkpoint: bytes, config: DecoderConfig,
                  options: Optional[StreamingOptions] = None) -> Dict[Tuple[int, int], bytes]:
    """One artifact per routed expert, keyed (layer, expert), each within
    the options' layer limit (checkpoint.rs:231-244)."""
    options = options or StreamingOptions()
    options.validate()
    r = CheckpointReader(checkpoint, config)
    return {(i, e): r.expert_bytes(i, e, options.max_layer_bytes)
            for i in range(config.num_hidden_layers) if config.layer_is_moe(i)
            for e in range(config.moe.num_experts)}


# ---- the C callback behind esp_model_load_streamed ----

class SourceBridge:
    """Adapts a LayerSource to esp_layer_read_fn: copies each artifact into
    the library's pinned staging buffer (large ones in parallel slices) and
    keeps the exception a source raised so the caller sees it unchanged."""

    _SLICE = 64 << 20

    def __init__(self, source: LayerSource):
        from . import _lib
        self.source = source
        self.error: Optional[BaseException] = None
        self._pool = ThreadPoolExecutor(8)
        self.fn = _lib.LAYER_READ_FN(self._read)
        self.efn = _lib.EXPERT_READ_FN(self._read_expert)

    def _read(self, user, index, limit, dst, cap, plen):
        return self._fill(lambda: self.source.read_layer_shared(int(index), int(limit)),
                          dst, cap, plen)

    def _read_expert(self, user, layer, expert, limit, dst, cap, plen):
        return self._fill(lambda: self.source.read_expert(int(layer), int(expert), int(limit)),
                          dst, cap, plen)

    def _fill(self, read, dst, cap, plen):
        try:
            data = read()
            n = len(data)
            plen[0] = n
            if n <= cap:
                src = np.frombuffer(data, np.uint8).ctypes.data if n else 0
                if n <= self._SLICE:
                    C.memmove(dst, src, n)
                else:
                    jobs = [self._pool.submit(C.memmove, dst + o, src + o, min(self._SLICE, n - o))
                            for o in range(0, n, self._SLICE)]
                    for j in jobs:
                        j.result()
            return 0
        except InferError as e:
            self.error = e
            return e.code
        except BaseException as e:  # noqa: BLE001 - reported through the status
            self.error = e
            return Backend.code

    def take(self) -> Optional[BaseException]:
        e, self.error = self.error, None
        return e


# ---- esp.layer-weights index objects (layer_library.rs:16-152) ----
# Blob ids come from the reference's content-addressed store (eidetic
# ManifestId, not in this build): they are kept as opaque strings and the
# reader given to IndexedSource verifies content identity.

WEIGHT_FORMATS = ("f32", "f16", "bf16", "q8-k32-f32-scale-f16-shared-v1",
                  "q4-k32-f32-scale-f16-shared-v1")  # weight_format.rs:20-32 serde names


def _strict(raw, names: Sequence[str], what: str) -> dict:
    """serde(deny_unknown_fields) with every field required."""
    if not isinstance(raw, dict) or set(raw) != set(names):
        raise InvalidWeights(f"layer library: {what} fields must be exactly {sorted(names)}")
    return raw


def _uint(v, what: str) -> int:
    if not isinstance(v, int) or isinstance(v, bool) or v < 0:
        raise InvalidWeights(f"layer library: {what} must be an unsigned integer")
    return v


@dataclass(frozen=True)
class LayerArtifact:
    """layer_library.rs:105-140: one verified artifact by blob id and size."""

    blob: str
    byte_size: int

    def to_json(self) -> dict:
        return {"blob": self.blob, "byte_size": self.byte_size}

    @staticmethod
    def from_json(raw) -> "LayerArtifact":
        r = _strict(raw, ("blob", "byte_size"), "artifact")
        if not isinstance(r["blob"], str) or not r["blob"]:
            raise InvalidWeights("layer library: artifact blob must be a non-empty id")
        return LayerArtifact(r["blob"], _uint(r["byte_size"], "byte_size"))


@dataclass(frozen=True)
class LayerWeightIndex:
    """layer_library.rs:140-152 (schema esp.layer-weights/v1): the shared
    artifact, one artifact per layer in order, and the streaming limits."""

    shared: LayerArtifact
    layers: Tuple[LayerArtifact, ...]
    options: StreamingOptions

    def to_json(self) -> dict:
        return {"shared": self.shared.to_json(), "layers": [a.to_json() for a in self.layers],
                "options": asdict(self.options)}

    @staticmethod
    def from_json(raw) -> "LayerWeightIndex":
        r = _strict(raw, ("shared", "layers", "options"), "layer index")
        if not isinstance(r["layers"], list):
            raise InvalidWeights("layer library: layers must be a list")
        opts = StreamingOptions.from_json(json.dumps(r["options"]))
        return LayerWeightIndex(LayerArtifact.from_json(r["shared"]),
                                tuple(LayerArtifact.from_json(a) for a in r["layers"]), opts)


@dataclass(frozen=True)
class PromptDeviation:
    """layer_library.rs:34-45"""

    rendered_prompt: str
    baseline_tokens: Tuple[int, ...]
    format_tokens: Tuple[int, ...]
    logit_rmse: float
    logit_max_abs: float


@dataclass(frozen=True)
class FormatQualification:
    """layer_library.rs:46-88: the measurement a formatted candidate needs
    before a resident may select it."""

    baseline_model: str
    baseline_loader: str
    measured_loader: str
    prompts: Tuple[PromptDeviation, ...]
    encoded_weight_bytes: int
    weight_payload_bytes: int
    streaming_resident_payload_bytes: int
    largest_layer_bytes: int
    logical_stream_bytes: int
    elapsed_seconds: float

    def validate(self) -> None:
        fin = lambda x: isinstance(x, (int, float)) and np.isfinite(x)  # noqa: E731
        bad = (not self.baseline_loader or not self.measured_loader or not self.prompts
               or self.encoded_weight_bytes == 0 or self.weight_payload_bytes == 0
               or self.streaming_resident_payload_bytes == 0 or self.largest_layer_bytes == 0
               or self.logical_stream_bytes == 0 or not fin(self.elapsed_seconds)
               or self.elapsed_seconds <= 0.0)
        for p in self.prompts:
            bad = bad or (not p.rendered_prompt or not p.baseline_tokens or not p.format_tokens
                          or not fin(p.logit_rmse) or p.logit_rmse < 0.0
                          or not fin(p.logit_max_abs) or p.logit_max_abs < p.logit_rmse)
        if bad:
            raise InvalidWeights("layer library: incomplete or non-finite format qualification")


@dataclass(frozen=True)
class FormattedLayerWeightIndex:
    """layer_library.rs:89-103 (schema esp.layer-weights/v2): an explicit
    execution format over exact layer artifacts, with the source artifacts
    and an optional measured qualification."""

    weights: LayerWeightIndex
    format: str
    source_artifacts: Tuple[str, ...]
    qualification: Optional[FormatQualification] = None

    def __post_init__(self):
        if self.format not in WEIGHT_FORMATS:
            raise InvalidWeights(f"layer library: unknown weight format {self.format!r}")

    def selectable(self) -> bool:
        """A candidate cannot be selected by the resident until measured."""
        if self.qualification is None:
            return False
        self.qualification.validate()
        return True


class IndexedSource(LayerSource):
    """Reads a LayerWeightIndex's artifacts through ``read(blob, size)``
    (the host's verified store reader), checking each declared size against
    the caller's limit before reading and the bytes against the declared
    size after (layer_library.rs:115-139)."""

    def __init__(self, index: LayerWeightIndex, read: Callable[[str, int], bytes]):
        self.index = index
        self._read = read

    def _fetch(self, art: LayerArtifact, limit: int) -> bytes:
        if art.byte_size > limit:
            raise InvalidWeights("layer library: layer artifact identity, schema or byte limit "
                                 "mismatch")
        data = self._read(art.blob, art.byte_size)
        if len(data) != art.byte_size:
            raise InvalidWeights("layer library: layer artifact bytes do not match their reference")
        return data

    def shared(self) -> bytes:
        return self._fetch(self.index.shared, self.index.options.max_shared_bytes)

    def read_layer(self, index: int, limit: int) -> bytes:
        if index >= len(self.index.layers):
            raise InvalidWeights(f"layer library: missing layer artifact {index}")
        return self._fetch(self.index.layers[index], limit)
