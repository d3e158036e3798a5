"""Token sampling with the draw on the host and the selection on the device.

``Sampler`` mirrors Sampler (Sources/AlpacaCore/Runtime/Sampler.swift:43-55):
validated parameters (SamplingParameters.validate, :21-25) and its own
SplitMix64 stream (:29-40), from which each non-greedy sample draws one
uniform double the way Swift's Double.random(in: 0..<1) does (the low 53 bits
of a 64-bit word times 2^-53).  The selection itself (top-k, temperature
softmax in double, top-p, the inverse-CDF draw) runs on the device over the
session's logits (ahip_session_sample) or over given logits (ahip_op_sample),
so sampling a decode step does not copy its logits to the host.
"""
from __future__ import annotations

import math
import os


class SplitMix64:
    """SplitMix64 (Sampler.swift:29-40)."""

    MASK = (1 << 64) - 1

    def __init__(self, seed: int):
        self.state = seed & self.MASK

    def next(self) -> int:
        self.state = (self.state + 0x9E3779B97F4A7C15) & self.MASK
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & self.MASK
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & self.MASK
        return z ^ (z >> 31)

    def uniform(self) -> float:
        """Double.random(in: 0..<1, using:) for Double's 53 significand bits."""
        return (self.next() & ((1 << 53) - 1)) * 2.0**-53


class Sampler:
    """Sampler(SamplingParameters): temperature 0 is greedy; top_k 0 and
    top_p 1 disable their filters; seed None draws a fresh seed."""

    def __init__(self, temperature: float = 0.8, top_k: int = 0, top_p: float = 1.0, seed: int | None = None):
        if not (math.isfinite(temperature) and temperature >= 0):
            raise ValueError("temperature must be finite and >= 0")
        if top_k < 0:
            raise ValueError("topK must be >= 0")
        if not (0 < top_p <= 1):
            raise ValueError("topP must be in (0, 1]")
        self.temperature, self.top_k, self.top_p = float(temperature), int(top_k), float(top_p)
        self.rng = SplitMix64(int.from_bytes(os.urandom(8), "little") if seed is None else seed)

    def _draw(self) -> float:
        return 0.0 if self.temperature == 0 else self.rng.uniform()

    def sample(self, session) -> int:
        """The next token from a session's last forward/decode logits (on the device)."""
        return session.sample(self.temperature, self.top_k, self.top_p, self._draw())

    def sample_logits(self, ops, logits) -> int:
        """The same over host logits (HIPOps.sample)."""
        return ops.sample(logits, self.temperature, self.top_k, self.top_p, self._draw())
