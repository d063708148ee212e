"""The packed-format restatement (oracle/quant.py) against the reference's
own weight-format test and closed forms."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import quant


def _reference_projection(width: int) -> np.ndarray:
    """weight_format.rs:342-348: element i = ((i % 103) - 51) / 40, row major."""
    i = np.arange(width * width)
    return (((i % 103).astype(np.float32) - 51.0) / 40.0).reshape(width, width).astype(np.float32)


@pytest.mark.parametrize("bits,tol", [(8, 0.006), (4, 0.1)])
def test_reference_projection_error_bound(bits, tol):
    """weight_format.rs:389-408: decoded weights within 0.006 (q8) / 0.1 (q4)."""
    for width in (64, 128):
        data = _reference_projection(width)
        buf = quant.quantize_projection(data, bits)
        n = width * width
        assert len(buf) == n * bits // 8 + n // 32 * 4
        got = quant.dequantize(buf, width, width, bits)
        assert np.abs(got - data).max() < tol


def test_values_on_the_grid_round_trip_exactly():
    rng = np.random.default_rng(3)
    for bits in (8, 4):
        qmax = quant.MAX[bits]
        q = rng.integers(-qmax, qmax + 1, size=(4, 64)).astype(np.float32)
        q[:, ::32] = qmax  # every block reaches its peak: scale = peak / max exactly
        scale = np.float32(0.125)
        data = q * scale
        got = quant.dequantize(quant.quantize_projection(data, bits), 4, 64, bits)
        assert np.array_equal(got, data)


def test_layout_nibbles_scales_and_zero_blocks():
    data = np.zeros((1, 64), np.float32)
    data[0, :32] = np.arange(32, dtype=np.float32) - 16.0  # peak 16
    buf4 = quant.quantize_projection(data, 4)
    # even input in the low nibble: inputs 0, 1 -> q = round(-16/(16/7)) = -7, round(-15*7/16) = -7
    b0 = buf4[0]
    assert b0 & 15 == (-7) & 15 and b0 >> 4 == (-7) & 15
    scales = np.frombuffer(buf4, "<f4", offset=32)
    assert scales[0] == np.float32(16.0) / np.float32(7.0)
    assert scales[1] == 1.0  # all-zero block
    assert not any(buf4[16:32])
    buf8 = quant.quantize_projection(data, 8)
    q = np.frombuffer(buf8, np.int8, count=64)
    assert q[0] == -127 and q[16] == 0 and q[31] == round(15 * 127 / 16)
    # halves round away from zero: 0.5 * scale -> 1
    half = np.zeros((1, 32), np.float32)
    half[0, 0] = 127.0
    half[0, 1] = 0.5
    half[0, 2] = -0.5
    q = np.frombuffer(quant.quantize_projection(half, 8), np.int8, count=32)
    assert q[1] == 1 and q[2] == -1


def test_tiny_blocks_keep_a_positive_scale():
    data = np.zeros((1, 32), np.float32)
    data[0, 5] = np.float32(1e-45)  # the smallest subnormal
    buf = quant.quantize_projection(data, 8)
    s = np.frombuffer(buf, "<f4", offset=32)[0]
    assert s == quant.F32_MIN_POSITIVE and np.isfinite(s) and s > 0


def test_convert_artifact_packs_projections_only():
    t = {"model.embed_tokens.weight": (np.ones((4, 32), np.float32), "F32"),
         "model.layers.0.self_attn.q_proj.weight": (np.ones((32, 32), np.float32), "F32"),
         "model.norm.weight": (np.ones(32, np.float32), "F32")}
    out = quant.convert_artifact(t, 8)
    assert out["model.embed_tokens.weight"][1] == "F16"
    assert out["model.norm.weight"][1] == "F16"
    arr, dt = out["model.layers.0.self_attn.q_proj.weight"]
    assert dt == "U8" and arr.shape == (32 * 32 + 32 * 4,)
    with pytest.raises(ValueError):
        quant.quantize_projection(np.ones((2, 33), np.float32), 8)
