"""ctypes wrapper over liboracle.so — the CPU restatement of esp's decoder.

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker. The product (esp_amd/) never
imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Dict, Optional, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

ORC_F32, ORC_BF16 = 0, 1
SLOTS = ["IN_NORM", "Q", "K", "V", "O", "Q_BIAS", "K_BIAS", "V_BIAS", "O_BIAS", "Q_NORM",
         "K_NORM", "POST_NORM", "GATE", "UP", "DOWN", "ROUTER", "SHARED_GATE", "SH_GATE",
         "SH_UP", "SH_DOWN"]
SLOT = {n: i for i, n in enumerate(SLOTS)}


class Tensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("dtype", C.c_int32), ("pad", C.c_int32)]


class Model(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("hidden", "layers", "n_heads", "n_kv_heads", "head_dim",
                                         "ffn", "vocab", "max_pos")] + [
        ("rms_eps", C.c_float)] + [(n, C.c_int32) for n in (
            "qkv_bias", "o_bias", "qk_norm", "n_experts", "top_k", "moe_ffn", "shared_ffn",
            "norm_topk")] + [
        ("layer_is_moe", C.POINTER(C.c_int32)), ("layer_window", C.POINTER(C.c_int32)),
        ("rope_cos", C.POINTER(C.c_float)), ("rope_sin", C.POINTER(C.c_float)),
        ("embed", Tensor), ("final_norm", Tensor), ("lm_head", Tensor),
        ("layer", C.POINTER(Tensor)), ("experts", C.POINTER(Tensor))]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run __graft_entry__.build() first")
        L = C.CDLL(LIB_PATH)
        L.orc_kv_create.restype = C.c_void_p
        L.orc_kv_create.argtypes = [C.POINTER(Model), C.c_int]
        L.orc_kv_destroy.argtypes = [C.c_void_p]
        L.orc_kv_position.argtypes = [C.c_void_p]
        L.orc_kv_fill_synthetic.argtypes = [C.c_void_p, C.c_int, C.c_uint64]
        L.orc_forward_last.argtypes = [C.POINTER(Model), C.c_void_p, C.POINTER(C.c_int32), C.c_int,
                                       C.c_void_p, C.c_void_p]
        L.orc_rope_table.argtypes = [C.c_int, C.c_int, C.c_float, C.c_int, C.c_float, C.c_float,
                                     C.c_float, C.c_int, C.c_void_p, C.c_void_p]
        L.orc_lora_merge.argtypes = [Tensor, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                     C.c_float, C.c_void_p]
        L.orc_argmax.argtypes = [C.c_void_p, C.c_int]
        L.orc_mask.argtypes = [C.c_void_p, C.c_int, C.c_void_p]
        L.orc_splitmix64_next.restype = C.c_uint64
        L.orc_splitmix64_next.argtypes = [C.POINTER(C.c_uint64)]
        L.orc_skip_draws.restype = C.c_uint64
        L.orc_skip_draws.argtypes = [C.c_uint64, C.c_uint64]
        L.orc_sample.argtypes = [C.c_void_p, C.c_int, C.c_float, C.c_float, C.POINTER(C.c_uint64)]
        L.orc_fill_normal.argtypes = [C.c_uint64, C.c_size_t, C.c_float, C.c_int, C.c_void_p]
        L.orc_set_threads.argtypes = [C.c_int]
        _lib = L
    return _lib


def rope_table(cfg, max_pos: Optional[int] = None) -> Tuple[np.ndarray, np.ndarray]:
    """attention.rs:58-95 via the C restatement (glibc powf/cosf/sinf)."""
    mp = max_pos or cfg.max_position_embeddings
    hd = cfg.head_dim()
    cos = np.zeros((mp, hd), np.float32)
    sin = np.zeros((mp, hd), np.float32)
    rs = cfg.rope_scaling
    kind = 0 if rs is None else (1 if rs.kind == "linear" else 2)
    lib().orc_rope_table(mp, hd, cfg.rope_theta, kind, rs.factor if rs else 1.0,
                         rs.low_freq_factor if rs else 0.0, rs.high_freq_factor if rs else 0.0,
                         rs.original_max_position_embeddings if rs else 0,
                         cos.ctypes.data, sin.ctypes.data)
    return cos, sin


def _tensor(arr: Optional[np.ndarray], dt: str, keep: list) -> Tensor:
    if arr is None:
        return Tensor(None, 0, 0)
    arr = np.ascontiguousarray(arr)
    keep.append(arr)
    return Tensor(arr.ctypes.data, ORC_BF16 if dt == "BF16" else ORC_F32, 0)


class OracleModel:
    """Holds numpy weights (f32 or raw bf16) in HF layout plus the C struct."""

    def __init__(self, cfg, tensors: Dict[str, Tuple[np.ndarray, str]],
                 lora: Optional[dict] = None, rope_max_pos: Optional[int] = None):
        self.cfg = cfg
        keep: list = []
        self._keep = keep
        tensors = dict(tensors)
        if lora:
            tensors = apply_lora(cfg, tensors, lora)
        L = cfg.num_hidden_layers
        moe = cfg.moe
        E = moe.num_experts if moe else 0
        layer_arr = (Tensor * (L * len(SLOTS)))()
        ex_arr = (Tensor * max(1, L * E * 3))()
        names = {"IN_NORM": "input_layernorm.weight", "Q": "self_attn.q_proj.weight",
                 "K": "self_attn.k_proj.weight", "V": "self_attn.v_proj.weight",
                 "O": "self_attn.o_proj.weight", "Q_BIAS": "self_attn.q_proj.bias",
                 "K_BIAS": "self_attn.k_proj.bias", "V_BIAS": "self_attn.v_proj.bias",
                 "O_BIAS": "self_attn.o_proj.bias", "Q_NORM": "self_attn.q_norm.weight",
                 "K_NORM": "self_attn.k_norm.weight",
                 "POST_NORM": "post_attention_layernorm.weight", "GATE": "mlp.gate_proj.weight",
                 "UP": "mlp.up_proj.weight", "DOWN": "mlp.down_proj.weight",
                 "ROUTER": "mlp.gate.weight", "SHARED_GATE": "mlp.shared_expert_gate.weight",
                 "SH_GATE": "mlp.shared_expert.gate_proj.weight",
                 "SH_UP": "mlp.shared_expert.up_proj.weight",
                 "SH_DOWN": "mlp.shared_expert.down_proj.weight"}
        for l in range(L):
            for slot, suffix in names.items():
                key = f"model.layers.{l}.{suffix}"
                if key in tensors:
                    arr, dt = tensors[key]
                    layer_arr[l * len(SLOTS) + SLOT[slot]] = _tensor(arr, dt, keep)
            for e in range(E):
                for j, nm in enumerate(("gate_proj", "up_proj", "down_proj")):
                    key = f"model.layers.{l}.mlp.experts.{e}.{nm}.weight"
                    if key in tensors:
                        arr, dt = tensors[key]
                        ex_arr[(l * E + e) * 3 + j] = _tensor(arr, dt, keep)
        keep += [layer_arr, ex_arr]
        is_moe = np.array([int(cfg.layer_is_moe(i)) for i in range(L)], np.int32)
        window = np.array([cfg.layer_window(i) or 0 for i in range(L)], np.int32)
        cos, sin = rope_table(cfg, rope_max_pos)
        keep += [is_moe, window, cos, sin]
        m = Model()
        m.hidden = cfg.hidden_size
        m.layers = L
        m.n_heads = cfg.num_attention_heads
        m.n_kv_heads = cfg.kv_heads()
        m.head_dim = cfg.head_dim()
        m.ffn = cfg.intermediate_size
        m.vocab = cfg.vocab_size
        m.max_pos = cos.shape[0]
        m.rms_eps = cfg.rms_norm_eps
        m.qkv_bias = int(cfg.qkv_bias())
        m.o_bias = int(cfg.output_bias())
        m.qk_norm = int(cfg.qk_norm())
        if moe:
            m.n_experts, m.top_k = moe.num_experts, moe.num_experts_per_tok
            m.moe_ffn, m.shared_ffn = moe.moe_intermediate_size, moe.shared_expert_intermediate_size
            m.norm_topk = int(moe.norm_topk_prob)
        m.layer_is_moe = is_moe.ctypes.data_as(C.POINTER(C.c_int32))
        m.layer_window = window.ctypes.data_as(C.POINTER(C.c_int32))
        m.rope_cos = cos.ctypes.data_as(C.POINTER(C.c_float))
        m.rope_sin = sin.ctypes.data_as(C.POINTER(C.c_float))
        emb, edt = tensors["model.embed_tokens.weight"]
        m.embed = _tensor(emb, edt, keep)
        nrm, ndt = tensors["model.norm.weight"]
        m.final_norm = _tensor(nrm, ndt, keep)
        if "lm_head.weight" in tensors:
            hd_, hdt = tensors["lm_head.weight"]
            m.lm_head = _tensor(hd_, hdt, keep)
        m.layer = C.cast(layer_arr, C.POINTER(Tensor))
        m.experts = C.cast(ex_arr, C.POINTER(Tensor))
        self.struct = m

    def new_cache(self, max_ctx: Optional[int] = None) -> "OracleKv":
        return OracleKv(self, max_ctx or self.struct.max_pos)

    def forward_last(self, kv: "OracleKv", ids, all_logits: bool = False):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.zeros(self.cfg.vocab_size, np.float32)
        allo = np.zeros((len(ids), self.cfg.vocab_size), np.float32) if all_logits else None
        rc = lib().orc_forward_last(C.byref(self.struct), kv.ptr,
                                    ids.ctypes.data_as(C.POINTER(C.c_int32)), len(ids),
                                    out.ctypes.data, None if allo is None else allo.ctypes.data)
        if rc != 0:
            raise RuntimeError(f"oracle forward failed: {rc}")
        return (out, allo) if all_logits else out


class OracleKv:
    def __init__(self, model: OracleModel, max_ctx: int):
        self.model = model
        self.ptr = lib().orc_kv_create(C.byref(model.struct), max_ctx)
        if not self.ptr:
            raise MemoryError("oracle KV allocation failed")

    def position(self) -> int:
        return lib().orc_kv_position(self.ptr)

    def fill_synthetic(self, position: int, seed: int) -> None:
        lib().orc_kv_fill_synthetic(self.ptr, position, seed)

    def __del__(self):
        if getattr(self, "ptr", None):
            lib().orc_kv_destroy(self.ptr)
            self.ptr = None


def apply_lora(cfg, tensors, lora: dict):
    """lora.rs:99-217 merge for each target module: W + (alpha/r*scale)·B·A.
    lora = {"rank", "alpha", "scale", "targets": [...], "tensors": {peft name: (arr, dt)}}."""
    out = dict(tensors)
    r = lora["rank"]
    s = np.float32(np.float32(lora["alpha"]) / np.float32(r) * np.float32(lora.get("scale", 1.0)))
    from .st import bf16_to_f32
    for l in range(cfg.num_hidden_layers):
        for mod in lora["targets"]:
            pre = f"base_model.model.model.layers.{l}.self_attn.{mod}"
            a, adt = lora["tensors"][f"{pre}.lora_A.weight"]
            b, bdt = lora["tensors"][f"{pre}.lora_B.weight"]
            a = bf16_to_f32(a) if adt == "BF16" else np.asarray(a, np.float32)
            b = bf16_to_f32(b) if bdt == "BF16" else np.asarray(b, np.float32)
            key = f"model.layers.{l}.self_attn.{mod}.weight"
            base, bdt0 = tensors[key]
            out_f, in_f = base.shape
            merged = np.zeros((out_f, in_f), np.float32)
            keep = []
            lib().orc_lora_merge(_tensor(base, bdt0, keep), np.ascontiguousarray(a).ctypes.data,
                                 np.ascontiguousarray(b).ctypes.data, out_f, in_f, r, float(s),
                                 merged.ctypes.data)
            out[key] = (merged, "F32")
    return out


def argmax(row) -> int:
    row = np.ascontiguousarray(row, np.float32)
    return lib().orc_argmax(row.ctypes.data, len(row))


def mask(row, bits) -> Tuple[np.ndarray, int]:
    row = np.array(row, np.float32)
    bits = np.ascontiguousarray(bits, np.uint32)
    n = lib().orc_mask(row.ctypes.data, len(row), bits.ctypes.data)
    return row, n


def sample(row, temperature: float, top_p: Optional[float], state: int) -> Tuple[int, int]:
    row = np.ascontiguousarray(row, np.float32)
    st = C.c_uint64(state)
    tok = lib().orc_sample(row.ctypes.data, len(row), temperature,
                           -1.0 if top_p is None else top_p, C.byref(st))
    return tok, st.value


def splitmix64_next(state: int) -> Tuple[int, int]:
    st = C.c_uint64(state)
    v = lib().orc_splitmix64_next(C.byref(st))
    return v, st.value


def skip_draws(state: int, draws: int) -> int:
    return lib().orc_skip_draws(state, draws)


def fill_normal(seed: int, n: int, std: float, bf16: bool) -> np.ndarray:
    out = np.empty(n, np.uint16 if bf16 else np.float32)
    lib().orc_fill_normal(seed, n, std, ORC_BF16 if bf16 else ORC_F32, out.ctypes.data)
    return out


def set_threads(n: int) -> None:
    lib().orc_set_threads(n)
