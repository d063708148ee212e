"""ctypes binding of include/esp_hip.h (esp_amd/libesp_hip.so).

The library must be present: there is no fallback compute path. A missing
or unloadable library raises immediately.
"""
from __future__ import annotations

import ctypes as C
import os

from .errors import raise_for_status

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libesp_hip.so")

ESP_FORMAT_F32, ESP_FORMAT_BF16, ESP_FORMAT_Q8, ESP_FORMAT_Q4 = 0, 1, 2, 3
ESP_ROPE_NONE, ESP_ROPE_LINEAR, ESP_ROPE_LLAMA3 = 0, 1, 2
ESP_PICK_NONFINITE, ESP_PICK_NO_ELIGIBLE = 1, 2


class EspConfig(C.Structure):
    _fields_ = [
        ("vocab_size", C.c_uint32), ("hidden_size", C.c_uint32),
        ("intermediate_size", C.c_uint32), ("num_hidden_layers", C.c_uint32),
        ("num_attention_heads", C.c_uint32), ("num_key_value_heads", C.c_uint32),
        ("head_dim", C.c_uint32), ("max_position_embeddings", C.c_uint32),
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float),
        ("rope_scaling", C.c_uint32), ("rope_factor", C.c_float),
        ("rope_low_freq_factor", C.c_float), ("rope_high_freq_factor", C.c_float),
        ("rope_original_max_position_embeddings", C.c_uint32),
        ("tie_word_embeddings", C.c_uint32), ("qkv_bias", C.c_uint32),
        ("output_bias", C.c_uint32), ("qk_norm", C.c_uint32),
        ("layer_window", C.POINTER(C.c_uint32)),
        ("num_experts", C.c_uint32), ("num_experts_per_tok", C.c_uint32),
        ("moe_intermediate_size", C.c_uint32), ("shared_expert_intermediate_size", C.c_uint32),
        ("norm_topk_prob", C.c_uint32), ("layer_is_moe", C.POINTER(C.c_uint8)),
        ("format", C.c_uint32),
    ]


class EspLora(C.Structure):
    _fields_ = [("rank", C.c_uint32), ("scale", C.c_float), ("target_mask", C.c_uint32),
                ("safetensors", C.c_void_p), ("safetensors_len", C.c_size_t)]


class EspSampler(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("state", C.c_uint64)]


class EspStreamingOptions(C.Structure):
    _fields_ = [("query_chunk", C.c_uint64), ("max_layer_bytes", C.c_uint64),
                ("max_shared_bytes", C.c_uint64)]


# esp_layer_read_fn(user, index, limit, dst, cap, *len) -> esp_status
LAYER_READ_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, C.c_uint64, C.c_void_p,
                            C.c_uint64, C.POINTER(C.c_uint64))


EXPERT_READ_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint64,
                             C.c_void_p, C.c_uint64, C.POINTER(C.c_uint64))


class EspLayerSource(C.Structure):
    _fields_ = [("read_layer", LAYER_READ_FN), ("user", C.c_void_p),
                ("read_expert", EXPERT_READ_FN)]


class EspStreamingStats(C.Structure):
    _fields_ = [("streamed", C.c_uint32), ("device_cache", C.c_uint32),
                ("layer_reads", C.c_uint64), ("encoded_bytes_read", C.c_uint64),
                ("largest_encoded_layer", C.c_uint64), ("cache_hits", C.c_uint64),
                ("cache_misses", C.c_uint64), ("retained_payload_bytes", C.c_uint64),
                ("payload_budget_bytes", C.c_uint64), ("cached_layers", C.c_uint64),
                ("expert_reads", C.c_uint64), ("expert_encoded_bytes_read", C.c_uint64),
                ("largest_encoded_expert", C.c_uint64)]


_lib = None


def load():
    """Load the HIP library (once). Raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
    L = C.CDLL(LIB_PATH)
    vp, u32, i32 = C.c_void_p, C.c_uint32, C.c_int32
    P = C.POINTER
    sigs = {
        "esp_last_error": (C.c_size_t, [C.c_char_p, C.c_size_t]),
        "esp_version": (C.c_char_p, []),
        "esp_model_load": (C.c_int, [P(EspConfig), vp, C.c_size_t, P(EspLora), u32, P(vp)]),
        "esp_model_create_synthetic": (C.c_int, [P(EspConfig), C.c_uint64, C.c_float, u32, u32,
                                                 C.c_float, C.c_float, C.c_float, P(vp)]),
        "esp_model_destroy": (C.c_int, [vp]),
        "esp_model_weight_bytes": (C.c_int, [vp, P(C.c_uint64)]),
        "esp_kv_create": (C.c_int, [vp, u32, u32, P(vp)]),
        "esp_kv_create_ex": (C.c_int, [vp, u32, u32, u32, P(vp)]),
        "esp_kv_destroy": (C.c_int, [vp]),
        "esp_kv_reset": (C.c_int, [vp, u32]),
        "esp_kv_position": (C.c_int, [vp, u32, P(u32)]),
        "esp_kv_stream": (C.c_int, [vp, P(vp)]),
        "esp_kv_logits": (C.c_int, [vp, P(vp), P(u32)]),
        "esp_forward_last": (C.c_int, [vp, vp, u32, P(i32), u32, vp]),
        "esp_forward_batch": (C.c_int, [vp, vp, u32, P(u32), P(u32), P(i32), vp]),
        "esp_pick": (C.c_int, [vp, u32, vp, P(EspSampler), P(u32), P(C.c_uint8)]),
        "esp_generate_greedy": (C.c_int, [vp, vp, u32, P(i32), u32, u32, P(i32), u32, P(i32),
                                          P(u32)]),
        "esp_pick_constrained": (C.c_int, [vp, u32, P(vp), P(EspSampler), P(u32), P(C.c_uint8)]),
        "esp_pick_noalloc": (C.c_int, [vp, u32, vp, vp, vp, vp]),
        "esp_vocab_create": (C.c_int, [vp, P(u32), u32, P(vp)]),
        "esp_vocab_destroy": (C.c_int, [vp]),
        "esp_constraint_create": (C.c_int, [vp, C.c_char_p, C.c_size_t, P(vp)]),
        "esp_constraint_destroy": (C.c_int, [vp]),
        "esp_constraint_accept": (C.c_int, [vp, u32]),
        "esp_constraint_complete": (C.c_int, [vp, P(C.c_uint8)]),
        "esp_constraint_forced_bytes": (C.c_int, [vp, P(C.c_uint8), u32, P(u32)]),
        "esp_constraint_mask": (C.c_int, [vp, vp, P(u32), P(u32)]),
        "esp_model_load_streamed": (C.c_int, [P(EspConfig), vp, C.c_size_t, P(EspLayerSource),
                                              P(EspStreamingOptions), P(vp)]),
        "esp_model_layer_cache": (C.c_int, [vp, C.c_uint64]),
        "esp_model_resident_layers": (C.c_int, [vp]),
        "esp_model_streaming_stats": (C.c_int, [vp, P(EspStreamingStats)]),
        "esp_stage_create": (C.c_int, [P(EspConfig), u32, u32, P(EspLayerSource),
                                       P(EspStreamingOptions), vp, C.c_size_t, u32, P(vp)]),
        "esp_stage_destroy": (C.c_int, [vp]),
        "esp_stage_forward": (C.c_int, [vp, vp, u32, u32, vp]),
        "esp_profile_enable": (C.c_int, [C.c_char_p, C.c_int]),
        "esp_profile_read": (C.c_int, [C.c_char_p, P(C.c_uint64), P(C.c_double)]),
    }
    for name, (res, args) in sigs.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


EXPORTED = ["esp_last_error", "esp_version", "esp_model_load", "esp_model_create_synthetic",
            "esp_model_destroy", "esp_model_weight_bytes", "esp_kv_create", "esp_kv_create_ex",
            "esp_kv_destroy",
            "esp_kv_reset", "esp_kv_position", "esp_kv_stream", "esp_kv_logits", "esp_forward_last",
            "esp_forward_batch", "esp_pick", "esp_pick_constrained", "esp_pick_noalloc",
            "esp_generate_greedy",
            "esp_vocab_create", "esp_vocab_destroy", "esp_constraint_create",
            "esp_constraint_destroy", "esp_constraint_accept", "esp_constraint_complete",
            "esp_constraint_forced_bytes", "esp_constraint_mask", "esp_model_load_streamed",
            "esp_model_layer_cache", "esp_model_resident_layers", "esp_model_streaming_stats",
            "esp_stage_create", "esp_stage_destroy", "esp_stage_forward",
            "esp_profile_enable", "esp_profile_read"]


def check(status: int) -> None:
    """Raise the InferError subclass for a non-zero esp_status."""
    if status == 0:
        return
    L = load()
    n = L.esp_last_error(None, 0)
    buf = C.create_string_buffer(n + 1)
    L.esp_last_error(buf, n + 1)
    raise_for_status(status, buf.value.decode(errors="replace"))
