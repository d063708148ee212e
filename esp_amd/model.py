"""DecoderModel / KvCache over the HIP library, mirroring esp's model seam.

crates/esp/src/infer/decoder/model.rs: `DecoderModel::{from_loaded,
new_cache, try_forward_cached_last}` and `KvCache::position`; loader.rs
`load_decoder_from_bytes`; lora.rs adapters. All compute runs in
libesp_hip.so; this module converts arguments and errors only.
"""
from __future__ import annotations

import ctypes as C
import itertools
from typing import List, Optional, Sequence, Tuple

import numpy as np

from . import _lib
from .config import DecoderConfig
from .errors import InvalidRequest
from .sample import Sampler

# numpy view of esp_sampler (float temperature, float top_p, uint64 state)
_SAMPLER_DT = np.dtype([("temperature", "<f4"), ("top_p", "<f4"), ("state", "<u8")], align=True)
assert _SAMPLER_DT.itemsize == C.sizeof(_lib.EspSampler)

# weight_format.rs:34-49 names (short and versioned)
FORMATS = {"f32": _lib.ESP_FORMAT_F32, "bf16": _lib.ESP_FORMAT_BF16,
           "q8-block32": _lib.ESP_FORMAT_Q8, "q8-k32-f32-scale-f16-shared-v1": _lib.ESP_FORMAT_Q8,
           "q4-block32": _lib.ESP_FORMAT_Q4, "q4-k32-f32-scale-f16-shared-v1": _lib.ESP_FORMAT_Q4}
TARGET_BITS = {"q_proj": 1, "k_proj": 2, "v_proj": 4, "o_proj": 8}


def esp_config(cfg: DecoderConfig, fmt: str = "f32"):
    """DecoderConfig -> (EspConfig struct, keep-alive arrays)."""
    c = _lib.EspConfig()
    c.vocab_size = cfg.vocab_size
    c.hidden_size = cfg.hidden_size
    c.intermediate_size = cfg.intermediate_size
    c.num_hidden_layers = cfg.num_hidden_layers
    c.num_attention_heads = cfg.num_attention_heads
    c.num_key_value_heads = cfg.kv_heads()
    c.head_dim = cfg.head_dim()
    c.max_position_embeddings = cfg.max_position_embeddings
    c.rms_norm_eps = cfg.rms_norm_eps
    c.rope_theta = cfg.rope_theta
    rs = cfg.rope_scaling
    if rs is not None:
        c.rope_scaling = _lib.ESP_ROPE_LINEAR if rs.kind == "linear" else _lib.ESP_ROPE_LLAMA3
        c.rope_factor = rs.factor
        c.rope_low_freq_factor = rs.low_freq_factor
        c.rope_high_freq_factor = rs.high_freq_factor
        c.rope_original_max_position_embeddings = rs.original_max_position_embeddings
    c.tie_word_embeddings = int(cfg.tie_word_embeddings)
    c.qkv_bias = int(cfg.qkv_bias())
    c.output_bias = int(cfg.output_bias())
    c.qk_norm = int(cfg.qk_norm())
    L = cfg.num_hidden_layers
    win = (C.c_uint32 * L)(*[cfg.layer_window(i) or 0 for i in range(L)])
    c.layer_window = C.cast(win, C.POINTER(C.c_uint32))
    moe = (C.c_uint8 * L)(*[int(cfg.layer_is_moe(i)) for i in range(L)])
    c.layer_is_moe = C.cast(moe, C.POINTER(C.c_uint8))
    if cfg.moe is not None:
        c.num_experts = cfg.moe.num_experts
        c.num_experts_per_tok = cfg.moe.num_experts_per_tok
        c.moe_intermediate_size = cfg.moe.moe_intermediate_size
        c.shared_expert_intermediate_size = cfg.moe.shared_expert_intermediate_size
        c.norm_topk_prob = int(cfg.moe.norm_topk_prob)
    c.format = FORMATS[fmt]
    return c, (win, moe)


def _borrow(data) -> Optional[C.c_void_p]:
    """A pointer to `data`'s bytes for the duration of one call, without a
    copy (bytes, bytearray or a writable buffer; the library only reads)."""
    if not data:
        return None
    if isinstance(data, bytes):
        return C.cast(C.c_char_p(data), C.c_void_p)
    return C.c_void_p(C.addressof((C.c_uint8 * len(data)).from_buffer(data)))


class LoraAdapter:
    """One PEFT LoRA adapter (lora.rs:99-217): rank, alpha, selection scale,
    target modules and the adapter safetensors bytes. Applied unmerged."""

    def __init__(self, rank: int, alpha: float, targets: Sequence[str], weights: bytes,
                 selection_scale: float = 1.0):
        for t in targets:
            if t not in TARGET_BITS:
                from .errors import InvalidConfig
                raise InvalidConfig(f"PEFT LoRA target module {t!r} is not supported; expected "
                                    "llama q/k/v/o projections")
        self.rank = rank
        # lora.rs:194: alpha / rank * selection scale, in f32
        a = np.float32(alpha) / np.float32(rank)
        self.scale = float(np.float32(a * np.float32(selection_scale)))
        self.mask = sum(TARGET_BITS[t] for t in set(targets))
        self.weights = bytes(weights)


class KvCache:
    """model.rs:671-681 KvCache for `batch` independent sequences."""

    def __init__(self, model: "DecoderModel", batch: int, max_ctx: int, kv_dtype: str = "f32"):
        """kv_dtype "f32" (default) or "f16" (bf16 weights only: half the
        bytes, outside the bf16 tolerance on deep models; esp_kv_create_ex)."""
        L = _lib.load()
        h = C.c_void_p()
        if kv_dtype not in ("f32", "f16"):
            raise InvalidRequest(f"kv_dtype must be f32 or f16, got {kv_dtype}")
        _lib.check(L.esp_kv_create_ex(model._h, batch, max_ctx, 1 if kv_dtype == "f16" else 0,
                                      C.byref(h)))
        self._h = h
        self.model = model
        self.batch = batch
        self.max_ctx = max_ctx
        self.kv_dtype = kv_dtype

    def position(self, seq: int = 0) -> int:
        p = C.c_uint32()
        _lib.check(_lib.load().esp_kv_position(self._h, seq, C.byref(p)))
        return p.value

    def reset(self, seq: Optional[int] = None) -> None:
        _lib.check(_lib.load().esp_kv_reset(self._h, 0xFFFFFFFF if seq is None else seq))

    def stream(self) -> int:
        s = C.c_void_p()
        _lib.check(_lib.load().esp_kv_stream(self._h, C.byref(s)))
        return s.value or 0

    def logits_device(self) -> Tuple[int, int]:
        """(device address, rows) of the last forward's f32 logits rows."""
        p = C.c_void_p()
        n = C.c_uint32()
        _lib.check(_lib.load().esp_kv_logits(self._h, C.byref(p), C.byref(n)))
        return p.value or 0, n.value

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.load().esp_kv_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()


class DecoderModel:
    """model.rs:151-667 DecoderModel, weights resident in HBM."""

    def __init__(self, handle, config: DecoderConfig, fmt: str):
        self._h = handle
        self.config = config
        self.format = fmt

    @staticmethod
    def from_bytes(config: DecoderConfig, weights: bytes, fmt: str = "f32",
                   adapters: Optional[List[LoraAdapter]] = None) -> "DecoderModel":
        """loader.rs:573-580 load_decoder_from_bytes (+ lora.rs adapters)."""
        L = _lib.load()
        c, keep = esp_config(config, fmt)
        buf = _borrow(weights)
        ads = adapters or []
        arr = (_lib.EspLora * max(1, len(ads)))()
        bufs = []
        for i, a in enumerate(ads):
            b = (C.c_uint8 * len(a.weights)).from_buffer_copy(a.weights)
            bufs.append(b)
            arr[i] = _lib.EspLora(a.rank, a.scale, a.mask, C.cast(b, C.c_void_p), len(a.weights))
        h = C.c_void_p()
        _lib.check(L.esp_model_load(C.byref(c), buf, len(weights), arr, len(ads), C.byref(h)))
        del keep, bufs
        return DecoderModel(h, config, fmt)

    @staticmethod
    def synthetic(config: DecoderConfig, seed: int, std: float = 0.02, fmt: str = "bf16",
                  lora_rank: int = 0, lora_targets: Sequence[str] = (), lora_a_std: float = 0.02,
                  lora_b_std: float = 0.01, lora_scale: float = 1.0) -> "DecoderModel":
        L = _lib.load()
        c, keep = esp_config(config, fmt)
        mask = sum(TARGET_BITS[t] for t in set(lora_targets))
        h = C.c_void_p()
        _lib.check(L.esp_model_create_synthetic(C.byref(c), seed, std, lora_rank, mask, lora_a_std,
                                                lora_b_std, lora_scale, C.byref(h)))
        del keep
        return DecoderModel(h, config, fmt)

    @staticmethod
    def from_layer_source(config: DecoderConfig, shared: bytes, source: "LayerSource",
                          options: Optional["StreamingOptions"] = None,
                          fmt: str = "f32") -> "DecoderModel":
        """provider.rs:370-426 + model.rs:268-312: resident embedding, final
        norm and head from the shared artifact; every forward reads each
        layer through ``source`` and stages it into HBM."""
        from .streaming import SourceBridge, StreamingOptions
        options = options or StreamingOptions()
        options.validate()
        L = _lib.load()
        c, keep = esp_config(config, fmt)
        bridge = SourceBridge(source)
        src = _lib.EspLayerSource(bridge.fn, None, bridge.efn)
        opt = _lib.EspStreamingOptions(options.query_chunk, options.max_layer_bytes,
                                       options.max_shared_bytes)
        buf = (C.c_uint8 * len(shared)).from_buffer_copy(shared) if shared else None
        h = C.c_void_p()
        _lib.check(L.esp_model_load_streamed(C.byref(c), buf, len(shared), C.byref(src),
                                             C.byref(opt), C.byref(h)))
        del keep
        m = DecoderModel(h, config, fmt)
        m._bridge = bridge  # the callback must outlive the handle
        return m

    def with_layer_cache(self, budget: int) -> "DecoderModel":
        """model.rs:336-362: keep a first-fit subset of streamed layers in HBM."""
        _lib.check(_lib.load().esp_model_layer_cache(self._h, budget))
        return self

    def with_resident_layers(self) -> "DecoderModel":
        """model.rs:384-415: read every layer once and keep all of them."""
        self._check(_lib.load().esp_model_resident_layers(self._h))
        return self

    def streaming_stats(self) -> Optional["StreamingReadStats"]:
        """model.rs:314-333: None unless layers stream."""
        from .streaming import DeviceLayerCacheStats, StreamingReadStats
        s = _lib.EspStreamingStats()
        _lib.check(_lib.load().esp_model_streaming_stats(self._h, C.byref(s)))
        if not s.streamed:
            return None
        bridge = getattr(self, "_bridge", None)
        out = StreamingReadStats(layer_reads=s.layer_reads, encoded_bytes_read=s.encoded_bytes_read,
                                 largest_encoded_layer=s.largest_encoded_layer,
                                 verified_cache=bridge.source.cache_stats() if bridge else None,
                                 expert_reads=s.expert_reads,
                                 expert_encoded_bytes_read=s.expert_encoded_bytes_read,
                                 largest_encoded_expert=s.largest_encoded_expert)
        if s.device_cache:
            out.device_cache = DeviceLayerCacheStats(s.cache_hits, s.cache_misses,
                                                     s.retained_payload_bytes,
                                                     s.payload_budget_bytes, s.cached_layers)
        return out

    def _check(self, status: int) -> None:
        """_lib.check, re-raising unchanged what a layer source raised."""
        bridge = getattr(self, "_bridge", None)
        err = bridge.take() if bridge is not None else None
        if status and err is not None:
            raise err
        _lib.check(status)

    def weight_bytes(self) -> int:
        n = C.c_uint64()
        _lib.check(_lib.load().esp_model_weight_bytes(self._h, C.byref(n)))
        return n.value

    def new_cache(self, batch: int = 1, max_ctx: Optional[int] = None,
                  kv_dtype: str = "f32") -> KvCache:
        """model.rs:476-483"""
        return KvCache(self, batch, max_ctx or self.config.max_position_embeddings, kv_dtype)

    def try_forward_cached_last(self, ids: Sequence[int], cache: KvCache,
                                seq: int = 0) -> np.ndarray:
        """model.rs:502-539: logits [vocab] (f32) of the block's last position."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty(self.config.vocab_size, np.float32)
        self._check(_lib.load().esp_forward_last(
            self._h, cache._h, seq, ids.ctypes.data_as(C.POINTER(C.c_int32)), len(ids),
            out.ctypes.data))
        return out

    def forward_batch(self, cache: KvCache, seqs: Sequence[int],
                      blocks: Sequence[Sequence[int]], want_logits: bool = True) -> Optional[np.ndarray]:
        """Several sequences' blocks in one pass; row i = last logits of seqs[i]."""
        seqs_a = np.ascontiguousarray(seqs, dtype=np.uint32)
        lens = np.fromiter(map(len, blocks), dtype=np.uint32, count=len(blocks))
        ids = np.fromiter(itertools.chain.from_iterable(blocks), dtype=np.int32, count=int(lens.sum()))
        out = np.empty((len(seqs_a), self.config.vocab_size), np.float32) if want_logits else None
        self._check(_lib.load().esp_forward_batch(
            self._h, cache._h, len(seqs_a), seqs_a.ctypes.data_as(C.POINTER(C.c_uint32)),
            lens.ctypes.data_as(C.POINTER(C.c_uint32)), ids.ctypes.data_as(C.POINTER(C.c_int32)),
            None if out is None else out.ctypes.data))
        return out

    def pick(self, cache: KvCache, n_rows: int, allowed_bits: Optional[np.ndarray] = None,
             samplers: Optional[List[Optional[Sampler]]] = None) -> Tuple[np.ndarray, np.ndarray]:
        """Token choice over the device-resident logits rows of the last forward
        (generate.rs:30-44, provider.rs:807-816). Updates sampler RNG state."""
        bits = None
        if allowed_bits is not None:
            bits = np.ascontiguousarray(allowed_bits, dtype=np.uint32)
            words = (self.config.vocab_size + 31) // 32
            if bits.size != n_rows * words:
                raise InvalidRequest("allowed bitmask has the wrong size")
        return self._pick(cache, n_rows, samplers, lambda *a: _lib.load().esp_pick(
            cache._h, n_rows, None if bits is None else bits.ctypes.data, *a))

    def pick_constrained(self, cache: KvCache, constraints: Sequence[Optional["Constraint"]],
                         samplers: Optional[List[Optional[Sampler]]] = None, check: bool = True):
        """provider.rs:740-817: pick with each row masked on the device by its
        constraint (None = unconstrained). Constraint states are not advanced.
        Returns (ids, flags); with check=False, (ids, flags, status) and no
        raise, so a caller can read the flags of a refused pick first."""
        from .constraint import constraint_handles
        arr, keep = constraint_handles(constraints)
        return self._pick(cache, len(constraints), samplers, lambda *a: _lib.load()
                          .esp_pick_constrained(cache._h, len(keep), arr, *a), check)

    def _pick(self, cache: KvCache, n_rows: int, samplers, call, check: bool = True):
        ids = np.zeros(n_rows, np.uint32)
        flags = np.zeros(n_rows, np.uint8)
        sarr = sptr = None
        if samplers is not None:
            # esp_sampler rows (temperature, top_p, state) built in one pass
            sarr = np.fromiter(((0.0, -1.0, 0) if s is None else
                                (s.temperature, -1.0 if s.top_p is None else s.top_p, s.rng.state)
                                for s in samplers), dtype=_SAMPLER_DT, count=n_rows)
            sptr = sarr.ctypes.data_as(C.POINTER(_lib.EspSampler))
        status = call(sptr, ids.ctypes.data_as(C.POINTER(C.c_uint32)),
                      flags.ctypes.data_as(C.POINTER(C.c_uint8)))
        if samplers is not None:
            for s, st in zip(samplers, sarr["state"].tolist()):
                if s is not None:
                    s.rng.state = st
        if not check:
            return ids, flags, status
        _lib.check(status)
        return ids, flags

    def generate_greedy_device(self, cache: KvCache, prompt: Sequence[int], max_new: int,
                               eos: Sequence[int], seq: int = 0) -> List[int]:
        """generate.rs:134-170 with the greedy picker, run as a device loop."""
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        e = np.ascontiguousarray(list(eos) or [0], dtype=np.int32)
        window = min(cache.max_ctx, self.config.max_position_embeddings)
        out = np.zeros(max(1, min(max_new, window - len(p) + 1)), np.int32)
        n = C.c_uint32()
        P = C.POINTER(C.c_int32)
        self._check(_lib.load().esp_generate_greedy(
            self._h, cache._h, seq, p.ctypes.data_as(P), len(p), max_new, e.ctypes.data_as(P),
            len(eos), out.ctypes.data_as(P), C.byref(n)))
        return [int(x) for x in out[:n.value]]

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.load().esp_model_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()


def profile_enable(kernel: str, on: bool = True) -> None:
    _lib.check(_lib.load().esp_profile_enable(kernel.encode(), int(on)))


def profile_read(kernel: str) -> Tuple[int, float]:
    n = C.c_uint64()
    ms = C.c_double()
    _lib.check(_lib.load().esp_profile_read(kernel.encode(), C.byref(n), C.byref(ms)))
    return n.value, ms.value
