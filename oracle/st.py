"""Minimal safetensors reader/writer on numpy (test infrastructure).

bf16 tensors are carried as raw uint16 bit patterns with dtype tag "BF16".
Format: u64 LE header length, JSON header {name: {dtype, shape, data_offsets}},
then the byte buffer (https://github.com/huggingface/safetensors, format spec).
"""
from __future__ import annotations

import json
import struct
from typing import Dict, Tuple

import numpy as np

_NP = {"F32": np.float32, "BF16": np.uint16, "F16": np.float16, "I32": np.int32,
       "I64": np.int64, "U8": np.uint8}


def load(data: bytes) -> Dict[str, Tuple[np.ndarray, str]]:
    (n,) = struct.unpack("<Q", data[:8])
    header = json.loads(data[8:8 + n])
    base = 8 + n
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        a, b = meta["data_offsets"]
        dt = meta["dtype"]
        arr = np.frombuffer(data, dtype=_NP[dt], count=(b - a) // np.dtype(_NP[dt]).itemsize,
                            offset=base + a).reshape(meta["shape"])
        out[name] = (arr, dt)
    return out


def dump(tensors: Dict[str, Tuple[np.ndarray, str]]) -> bytes:
    header = {}
    offset = 0
    blobs = []
    for name in sorted(tensors):
        arr, dt = tensors[name]
        arr = np.ascontiguousarray(arr, dtype=_NP[dt])
        raw = arr.tobytes()
        header[name] = {"dtype": dt, "shape": list(arr.shape),
                        "data_offsets": [offset, offset + len(raw)]}
        blobs.append(raw)
        offset += len(raw)
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * ((8 - len(hb) % 8) % 8)
    return struct.pack("<Q", len(hb)) + hb + b"".join(blobs)


def dump_buffer(tensors: Dict[str, Tuple[np.ndarray, str]]) -> bytearray:
    """dump() into one preallocated bytearray (same bytes): each tensor is
    copied once, for multi-GB checkpoints."""
    header = {}
    offset = 0
    for name in sorted(tensors):
        arr, dt = tensors[name]
        nbytes = int(np.prod(arr.shape)) * np.dtype(_NP[dt]).itemsize
        header[name] = {"dtype": dt, "shape": list(arr.shape),
                        "data_offsets": [offset, offset + nbytes]}
        offset += nbytes
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * ((8 - len(hb) % 8) % 8)
    base = 8 + len(hb)
    out = bytearray(base + offset)
    out[:8] = struct.pack("<Q", len(hb))
    out[8:base] = hb
    view = np.frombuffer(out, dtype=np.uint8)
    for name in sorted(tensors):
        arr, dt = tensors[name]
        a, b = header[name]["data_offsets"]
        src = np.ascontiguousarray(arr, dtype=_NP[dt]).reshape(-1).view(np.uint8)
        view[base + a:base + b] = src
    return out


def bf16_round(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits, round-to-nearest-even (half::bf16::from_f32)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
