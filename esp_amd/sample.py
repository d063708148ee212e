"""Sampler state, mirroring crates/esp/src/infer/decoder/sample.rs.

The draw itself (temperature softmax, nucleus cut, inverse-CDF walk) runs
on the device inside `esp_pick`; the host keeps the splitmix64 state so
that seeded streams, `skip_draws` and checkpoint resumption behave exactly
as the reference's `Sampler` (sample.rs:56-122).
"""
from __future__ import annotations

import os
from typing import Optional

GOLDEN_GAMMA = 0x9E3779B97F4A7C15
MASK64 = (1 << 64) - 1


class SplitMix64:
    """sample.rs:21-52"""

    def __init__(self, seed: int):
        self.state = seed & MASK64

    @staticmethod
    def from_entropy() -> "tuple[SplitMix64, int]":
        seed = int.from_bytes(os.urandom(8), "little")
        return SplitMix64(seed), seed

    def next_u64(self) -> int:
        self.state = (self.state + GOLDEN_GAMMA) & MASK64
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
        return z ^ (z >> 31)

    def next_f64(self) -> float:
        return (self.next_u64() >> 11) / float(1 << 53)


class Sampler:
    """sample.rs:56-122: temperature + optional nucleus sampler with its own RNG."""

    def __init__(self, temperature: float, top_p: Optional[float], seed: int):
        if not temperature > 0.0:
            raise ValueError("temperature must be positive (greedy is a separate picker)")
        self.temperature = float(temperature)
        self.top_p = top_p
        self.rng = SplitMix64(seed)

    def skip_draws(self, draws: int) -> None:
        """sample.rs:64-69: advance exactly `draws` splitmix64 steps in O(1)."""
        self.rng.state = (self.rng.state + GOLDEN_GAMMA * draws) & MASK64
