"""HF `config.json` -> decoder geometry, mirroring esp's `DecoderConfig`.

Restates crates/esp/src/infer/decoder/config.rs: the same accepted families,
the same refusals (by field name, as `Unsupported("config.<field>")`), the
same derived geometry (`kv_heads`, `head_dim`, `query_width`, `qkv_bias`,
`output_bias`, `qk_norm`, `layer_is_moe`, `layer_window`, `kv_group_size`)
and the same RoPE scaling validation. The parsed config is handed to the
HIP library as a flat `esp_config` struct (include/esp_hip.h).
"""
from __future__ import annotations

import json
import math
from dataclasses import dataclass, field
from typing import List, Optional

from .errors import InvalidConfig, Unsupported

SUPPORTED_MODEL_TYPES = ("llama", "mistral", "qwen2", "qwen3", "qwen2_moe")  # config.rs:25
SUPPORTED_ARCHITECTURES = {  # config.rs:28-34, family map config.rs:398-405
    "LlamaForCausalLM": "llama",
    "MistralForCausalLM": "mistral",
    "Qwen2ForCausalLM": "qwen2",
    "Qwen3ForCausalLM": "qwen3",
    "Qwen2MoeForCausalLM": "qwen2_moe",
}


def _unsupported(feature: str, detail: str) -> Unsupported:
    return Unsupported(f"config.{feature}", detail)


def _f32(x: float) -> float:
    """Round a Python float to the nearest f32 (the reference parses into f32)."""
    import struct

    return struct.unpack("<f", struct.pack("<f", float(x)))[0]


@dataclass
class RopeScaling:
    """config.rs:54-181. kind: "linear" | "llama3"."""

    kind: str
    factor: float
    low_freq_factor: float = 0.0
    high_freq_factor: float = 0.0
    original_max_position_embeddings: int = 0

    @staticmethod
    def parse(value) -> "RopeScaling":
        """config.rs:69-156"""
        if not isinstance(value, dict):
            raise _unsupported("rope_scaling", "expected an object")
        kind = value.get("rope_type", value.get("type"))
        if not isinstance(kind, str):
            raise _unsupported("rope_scaling", "missing rope_type")
        if "type" in value and "rope_type" in value and value["type"] != value["rope_type"]:
            raise _unsupported("rope_scaling", "conflicting type and rope_type")

        def number(key: str) -> float:
            n = value.get(key)
            n = _f32(n) if isinstance(n, (int, float)) and not isinstance(n, bool) else math.nan
            if not math.isfinite(n) or n <= 0.0:
                raise _unsupported("rope_scaling", f"{key} must be positive and finite")
            return n

        if kind == "linear":
            allowed = {"type", "rope_type", "factor"}
        elif kind == "llama3":
            allowed = {"type", "rope_type", "factor", "low_freq_factor", "high_freq_factor",
                       "original_max_position_embeddings"}
        else:
            raise _unsupported("rope_scaling", f"{kind!r}; supported: linear, llama3")
        if any(k not in allowed for k in value):
            raise _unsupported("rope_scaling", "unimplemented scaling parameters")
        factor = number("factor")
        if factor < 1.0:
            raise _unsupported("rope_scaling", "factor must be at least one")
        if kind == "linear":
            return RopeScaling("linear", factor)
        low = number("low_freq_factor")
        high = number("high_freq_factor")
        orig = value.get("original_max_position_embeddings")
        if not isinstance(orig, int) or isinstance(orig, bool) or orig <= 0:
            raise _unsupported("rope_scaling", "original context must be a positive integer")
        if high <= low:
            raise _unsupported("rope_scaling",
                               "high frequency factor must exceed low frequency factor")
        return RopeScaling("llama3", factor, low, high, orig)


@dataclass
class MoeConfig:
    """config.rs:37-48. `shared_expert_intermediate_size == 0` (no shared
    expert, Mixtral-style) is only reachable through `DecoderConfig.mixtral_style`;
    JSON configs keep the reference's refusal of 0 (config.rs:547-568)."""

    num_experts: int
    num_experts_per_tok: int
    moe_intermediate_size: int
    shared_expert_intermediate_size: int
    norm_topk_prob: bool = False
    decoder_sparse_step: int = 1
    mlp_only_layers: List[int] = field(default_factory=list)


def _uint(d: dict, key: str, default=None, required=True):
    if key not in d or d[key] is None:
        if required and default is None:
            raise InvalidConfig(f"config.json parse: missing field `{key}`")
        return default
    v = d[key]
    if isinstance(v, bool) or not isinstance(v, int) or v < 0:
        raise InvalidConfig(f"config.json parse: invalid value for `{key}`")
    return v


@dataclass
class DecoderConfig:
    """config.rs:322-363 (HF field names)."""

    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    max_position_embeddings: int
    num_key_value_heads: Optional[int] = None
    head_dim_: Optional[int] = None
    rms_norm_eps: float = 1.0e-5
    rope_theta: float = 10_000.0
    tie_word_embeddings: bool = False
    eos_token_id: List[int] = field(default_factory=list)
    model_type: Optional[str] = None
    attention_bias: bool = False
    sliding_window: Optional[int] = None
    use_sliding_window: Optional[bool] = None
    max_window_layers: Optional[int] = None
    layer_types: Optional[List[str]] = None
    rope_scaling: Optional[RopeScaling] = None
    moe: Optional[MoeConfig] = None

    # ------------------------------------------------------------ parsing
    @staticmethod
    def from_json_bytes(data: bytes) -> "DecoderConfig":
        """config.rs:391-431"""
        try:
            raw = json.loads(data)
        except (ValueError, UnicodeDecodeError) as e:
            raise InvalidConfig(f"config.json parse: {e}") from None
        if not isinstance(raw, dict):
            raise InvalidConfig("config.json parse: expected an object")
        _refuse_foreign(raw)
        eos = raw.get("eos_token_id")
        if eos is None:
            eos_ids: List[int] = []
        elif isinstance(eos, list):
            eos_ids = [int(e) for e in eos]
        else:
            eos_ids = [int(eos)]
        cfg = DecoderConfig(
            vocab_size=_uint(raw, "vocab_size"),
            hidden_size=_uint(raw, "hidden_size"),
            intermediate_size=_uint(raw, "intermediate_size"),
            num_hidden_layers=_uint(raw, "num_hidden_layers"),
            num_attention_heads=_uint(raw, "num_attention_heads"),
            max_position_embeddings=_uint(raw, "max_position_embeddings"),
            num_key_value_heads=_uint(raw, "num_key_value_heads", required=False),
            head_dim_=_uint(raw, "head_dim", required=False),
            rms_norm_eps=float(raw.get("rms_norm_eps", 1.0e-5) if raw.get("rms_norm_eps") is not None else 1.0e-5),
            rope_theta=_f32(raw.get("rope_theta", 10_000.0) if raw.get("rope_theta") is not None else 10_000.0),
            tie_word_embeddings=bool(raw.get("tie_word_embeddings") or False),
            eos_token_id=eos_ids,
            model_type=raw.get("model_type"),
            attention_bias=bool(raw.get("attention_bias") or False),
            sliding_window=_uint(raw, "sliding_window", required=False),
            use_sliding_window=raw.get("use_sliding_window"),
            max_window_layers=_uint(raw, "max_window_layers", required=False),
            layer_types=raw.get("layer_types"),
        )
        for name in raw.get("architectures") or []:
            family = SUPPORTED_ARCHITECTURES[name]
            if cfg.model_type is not None and cfg.model_type != family:
                raise _unsupported("architectures", "architecture and model_type disagree")
            cfg.model_type = family
        if raw.get("rope_scaling") is not None:
            cfg.rope_scaling = RopeScaling.parse(raw["rope_scaling"])
        if cfg.model_type == "qwen2_moe":
            cfg.moe = MoeConfig(
                num_experts=_uint(raw, "num_experts"),
                num_experts_per_tok=_uint(raw, "num_experts_per_tok"),
                moe_intermediate_size=_uint(raw, "moe_intermediate_size"),
                shared_expert_intermediate_size=_uint(raw, "shared_expert_intermediate_size"),
                norm_topk_prob=bool(raw.get("norm_topk_prob") or False),
                decoder_sparse_step=_uint(raw, "decoder_sparse_step", default=1, required=False),
                mlp_only_layers=list(raw.get("mlp_only_layers") or []),
            )
        cfg.validate()
        _refuse_features(raw, cfg)
        return cfg

    @staticmethod
    def mixtral_style(**kw) -> "DecoderConfig":
        """A routed-expert config with no shared expert (Mixtral block:
        softmax over all experts, top-k, renormalised). The reference's
        qwen2_moe path computes the same function when its shared expert is
        zero; this constructor states it directly."""
        moe = MoeConfig(
            num_experts=kw.pop("num_experts"),
            num_experts_per_tok=kw.pop("num_experts_per_tok"),
            moe_intermediate_size=kw.pop("moe_intermediate_size"),
            shared_expert_intermediate_size=0,
            norm_topk_prob=True,
        )
        cfg = DecoderConfig(model_type="qwen2_moe", **kw)
        cfg.moe = moe
        cfg.validate(allow_no_shared_expert=True)
        return cfg

    # ------------------------------------------------------------ geometry
    def kv_heads(self) -> int:  # config.rs:434-436
        return self.num_key_value_heads if self.num_key_value_heads is not None else self.num_attention_heads

    def head_dim(self) -> int:  # config.rs:439-443
        return self.head_dim_ if self.head_dim_ is not None else self.hidden_size // self.num_attention_heads

    def query_width(self) -> int:  # config.rs:445-447
        return self.num_attention_heads * self.head_dim()

    def qkv_bias(self) -> bool:  # config.rs:449-451
        return self.model_type in ("qwen2", "qwen2_moe") or self.attention_bias

    def output_bias(self) -> bool:  # config.rs:453-455
        return self.model_type not in ("qwen2", "qwen2_moe") and self.attention_bias

    def qk_norm(self) -> bool:  # config.rs:457-459
        return self.model_type == "qwen3"

    def layer_is_moe(self, index: int) -> bool:  # config.rs:461-465
        m = self.moe
        return m is not None and index not in m.mlp_only_layers and (index + 1) % m.decoder_sparse_step == 0

    def layer_window(self, index: int) -> Optional[int]:  # config.rs:467-485
        if self.layer_types is not None:
            return self.sliding_window if self.layer_types[index] == "sliding_attention" else None
        if self.use_sliding_window is False:
            return None
        if self.model_type in ("qwen2", "qwen3", "qwen2_moe"):
            mwl = self.max_window_layers if self.max_window_layers is not None else 28
            return self.sliding_window if (self.use_sliding_window is True and index >= mwl) else None
        return self.sliding_window

    def kv_group_size(self) -> int:  # config.rs:488-490
        return self.num_attention_heads // self.kv_heads()

    def validate(self, allow_no_shared_expert: bool = False) -> None:
        """config.rs:492-570"""
        if self.num_attention_heads == 0 or (
                self.head_dim_ is None and self.hidden_size % self.num_attention_heads != 0):
            raise InvalidConfig(f"hidden_size {self.hidden_size} not divisible by "
                                f"num_attention_heads {self.num_attention_heads}")
        if self.kv_heads() == 0 or self.num_attention_heads % self.kv_heads() != 0:
            raise InvalidConfig(f"num_attention_heads {self.num_attention_heads} not divisible by "
                                f"num_key_value_heads {self.kv_heads()}")
        if self.head_dim() == 0 or self.head_dim() % 2 != 0:
            raise InvalidConfig(f"head_dim {self.head_dim()} must be even for rotary encoding")
        if (self.hidden_size == 0 or self.intermediate_size == 0 or self.vocab_size == 0
                or self.num_hidden_layers == 0 or self.max_position_embeddings == 0
                or not math.isfinite(self.rms_norm_eps) or self.rms_norm_eps <= 0.0
                or not math.isfinite(self.rope_theta) or self.rope_theta <= 0.0
                or self.sliding_window == 0):
            raise InvalidConfig("zero, non-finite or overflowing decoder dimensions/settings")
        if self.layer_types is not None and (
                len(self.layer_types) != self.num_hidden_layers
                or any((k != "full_attention" and k != "sliding_attention")
                       or (k == "sliding_attention" and self.sliding_window is None)
                       for k in self.layer_types)):
            raise _unsupported("layer_types", "expected one supported attention type per layer "
                                              "and a window for sliding layers")
        m = self.moe
        if m is not None and (
                m.num_experts == 0 or m.num_experts_per_tok == 0
                or m.num_experts_per_tok > m.num_experts or m.moe_intermediate_size == 0
                or (m.shared_expert_intermediate_size == 0 and not allow_no_shared_expert)
                or m.decoder_sparse_step == 0
                or any(i >= self.num_hidden_layers for i in m.mlp_only_layers)):
            raise _unsupported("experts", "invalid expert count, routing, intermediate size or "
                                          "sparse-layer selection")


def _refuse_foreign(raw: dict) -> None:
    """config.rs:230-263 ArchitectureFields::refuse_foreign"""
    if raw.get("text_config") is not None:
        raise _unsupported("text_config", "multimodal configs nest the language model; only a "
                                          "flat decoder config runs")
    mt = raw.get("model_type")
    if mt is not None and mt not in SUPPORTED_MODEL_TYPES:
        raise _unsupported("model_type", f"{mt!r}; supported: {list(SUPPORTED_MODEL_TYPES)}")
    for a in raw.get("architectures") or []:
        if a not in SUPPORTED_ARCHITECTURES:
            raise _unsupported("architectures",
                               f"{a!r}; supported: {list(SUPPORTED_ARCHITECTURES)}")


def _refuse_features(raw: dict, cfg: DecoderConfig) -> None:
    """config.rs:266-316 ArchitectureFields::refuse_features"""
    for fld in ("hidden_act", "hidden_activation"):
        act = raw.get(fld)
        if act is not None and act not in ("silu", "swish"):
            raise _unsupported(fld, f"{act!r}; only the SiLU-gated MLP is implemented")
    prf = raw.get("partial_rotary_factor")
    if prf is not None and prf != 1.0:
        raise _unsupported("partial_rotary_factor", f"{prf}; RoPE is applied to the full head")
    if raw.get("mlp_bias") is True:
        raise _unsupported("mlp_bias", "MLP projections are bias-free")
    for fld in ("attn_logit_softcapping", "final_logit_softcapping"):
        if raw.get(fld) is not None:
            raise _unsupported(fld, f"{raw[fld]}; logit soft-capping is not implemented")
    for fld in ("num_experts", "num_local_experts", "n_routed_experts", "num_experts_per_tok"):
        if cfg.moe is not None and fld in ("num_experts", "num_experts_per_tok"):
            continue
        n = raw.get(fld)
        if n is not None and n > 0:
            raise _unsupported(fld, f"{n}; mixture-of-experts layers are not implemented")
