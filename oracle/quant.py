"""CPU restatement of esp's packed projection formats (test infrastructure).

THIS IS THE PARITY CHECKER, NOT THE PRODUCT. Only tests/ and bench.py's
cpu_baseline leg import it. The product reads packed artifacts in
esp_amd/csrc/runtime.cpp and dequantizes in the decode GEMV
(esp_amd/csrc/decode_dev.hpp) and dequant_k (esp_amd/csrc/k_moe.hip).

Restates crates/esp/src/infer/decoder/weight_format.rs:
  quantize_projection  weight_format.rs:150-183 (per 32-input block of each
                       [out, in] row: scale = peak / max, or 1 for an
                       all-zero block, at least f32::MIN_POSITIVE; q =
                       round-half-away(v / scale) clamped to [-max, max];
                       q4 packs two per byte, the even input in the low
                       nibble; the packed values are followed by the f32
                       scales)
  convert_artifact     weight_format.rs:138-223 (projections = 2-D tensors
                       other than the embedding; every other tensor F16)
  dequantize           weight_format.rs:390-397 (weight = q * scale, f32)
Pinned by the reference's own test (weight_format.rs:338-420: the
((i % 103) - 51) / 40 projection, errors below 0.006 for q8 and 0.1 for
q4) and closed forms in tests/test_quant_oracle.py.
"""
from __future__ import annotations

from typing import Dict, Tuple

import numpy as np

MAX = {8: 127.0, 4: 7.0}
F32_MIN_POSITIVE = np.float32(1.17549435e-38)


def _round_half_away(x: np.ndarray) -> np.ndarray:
    """f32::round: nearest integer, halves away from zero (exact in f32)."""
    a = np.abs(x)
    r = np.floor(a)
    r = r + (a - r >= np.float32(0.5))
    return np.copysign(r, x).astype(np.float32)


def quantize_projection(data: np.ndarray, bits: int) -> bytes:
    """weight_format.rs:150-183: [rows, cols] f32 -> packed values + scales."""
    data = np.ascontiguousarray(data, np.float32)
    rows, cols = data.shape
    if cols % 32:
        raise ValueError(f"projection input width {cols} must be divisible by 32")
    qmax = np.float32(MAX[bits])
    blocks = data.reshape(rows, cols // 32, 32)
    peak = np.abs(blocks).max(axis=2)
    scale = np.where(peak == 0, np.float32(1.0),
                     np.maximum(peak / qmax, F32_MIN_POSITIVE)).astype(np.float32)
    q = _round_half_away(blocks / scale[:, :, None])
    q = np.clip(q, -qmax, qmax).astype(np.int8).reshape(-1)
    if bits == 8:
        packed = q.view(np.uint8)
    else:
        nib = (q.view(np.uint8) & 15).reshape(-1, 2)
        packed = (nib[:, 0] | (nib[:, 1] << 4)).astype(np.uint8)
    return packed.tobytes() + scale.reshape(-1).astype("<f4").tobytes()


def dequantize(buf: bytes, rows: int, cols: int, bits: int) -> np.ndarray:
    """weight = q * scale in f32 ([rows, cols])."""
    n = rows * cols
    vb = n if bits == 8 else n // 2
    raw = np.frombuffer(buf, np.uint8, count=vb)
    scales = np.frombuffer(buf, "<f4", count=n // 32, offset=vb).astype(np.float32)
    if bits == 8:
        q = raw.view(np.int8).astype(np.int32)
    else:
        lo = (raw & 15).astype(np.int32)
        hi = (raw >> 4).astype(np.int32)
        q = np.stack([lo, hi], axis=1).reshape(-1)
        q = np.where(q >= 8, q - 16, q)
    w = q.astype(np.float32) * np.repeat(scales, 32)
    return w.reshape(rows, cols)


def convert_artifact(tensors: Dict[str, Tuple[np.ndarray, str]],
                     bits: int) -> Dict[str, Tuple[np.ndarray, str]]:
    """weight_format.rs:138-223 on oracle.st tensors: projections packed as U8
    byte arrays, everything else F16."""
    out = {}
    for name, (arr, dt) in tensors.items():
        a = np.asarray(arr)
        if dt == "BF16":
            a = (a.astype(np.uint32) << 16).view(np.float32)
        a = a.astype(np.float32)
        if not np.isfinite(a).all():
            raise ValueError("non-finite weight")
        if a.ndim == 2 and name != "model.embed_tokens.weight":
            buf = quantize_projection(a, bits)
            out[name] = (np.frombuffer(buf, np.uint8).copy(), "U8")
        else:
            h = a.astype(np.float16)
            if not np.isfinite(h).all():
                raise ValueError(f"{name}: f16 conversion overflow")
            out[name] = (h, "F16")
    return out


def dequantized_model(tensors: Dict[str, Tuple[np.ndarray, str]],
                      shapes: Dict[str, Tuple[int, int]], bits: int
                      ) -> Dict[str, Tuple[np.ndarray, str]]:
    """The f32 weights a packed artifact stands for: projections dequantized,
    F16 tensors widened."""
    out = {}
    for name, (arr, dt) in tensors.items():
        if dt == "U8":
            rows, cols = shapes[name]
            out[name] = (dequantize(arr.tobytes(), rows, cols, bits), "F32")
        else:
            out[name] = (np.asarray(arr).astype(np.float32), "F32")
    return out
