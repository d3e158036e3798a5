"""The device sampler (kernels_sample.hip: Sampler.sample, Sampler.swift:57-93)
against the oracle's restatement of it, draw for draw.

Given the same logits, parameters and draw u, the device must return the
oracle's token.  Where top-k or top-p applies the device accumulates its sums
in the reference's order, so the only source of a difference is a last-bit
difference of exp; without them (and for the top-p total without top-k) the
sums are associated by chunks.  Draws within 1e-12 of a boundary between two
tokens, where either effect could flip the choice, are skipped; the number
skipped is printed and must stay a small fraction.  The reference's own
SamplerTests.swift assertions are then run through the device path, and the
session entry point is held to the op-level one on a model's logits.
"""
import zlib

import numpy as np
import pytest

import oracle.oracle as orc
from alpaca_amd import synth
from alpaca_amd._lib import InvalidArgument
from alpaca_amd.model import HIPLlamaModel
from alpaca_amd.sampling import Sampler
from tests.test_gpu_model import built

pytestmark = pytest.mark.gpu

LOGITS = [1.0, 3.0, 2.0, -1.0, 3.0, 0.5]


def logit_cases():
    rng = np.random.default_rng(5)
    big = (rng.standard_normal(49152) * 3).astype(np.float32)  # C1 vocabulary
    flat = (rng.standard_normal(5000) * 0.05).astype(np.float32)  # huge nuclei: many windows
    ties = np.round(rng.standard_normal(3000) * 2).astype(np.float32)  # few distinct values
    zeros = np.zeros(300, np.float32)
    zeros[::2] = -0.0  # -0 and +0 compare equal: ties by index
    zeros[7] = 1.0
    extreme = np.array([1e30, 0, -1e30, 3e38, -3e38], np.float32)
    return {"six": np.array(LOGITS, np.float32), "vocab": big, "flat": flat, "ties": ties, "zeros": zeros,
            "extreme": extreme}


PARAMS = [(1.0, 0, 1.0), (0.5, 0, 1.0), (2.0, 0, 1.0), (1.0, 1, 1.0), (1.0, 2, 1.0), (0.8, 40, 1.0),
          (1.0, 1000, 1.0), (1.0, 1500, 1.0), (1.2, 3000, 1.0), (1.0, 0, 0.3), (1.0, 0, 0.9), (0.7, 0, 0.999),
          (1.0, 50, 0.9), (2.0, 3000, 0.95), (0.0, 0, 1.0)]


@pytest.mark.parametrize("name", list(logit_cases()))
def test_device_sampler_matches_oracle(hip_ops, name):
    l = logit_cases()[name]
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    checked = skipped = 0
    for t, k, p in PARAMS:
        for u in rng.random(12):
            want = orc.sample(l, t, k, p, u)
            if t > 0 and (orc.sample(l, t, k, p, max(u - 1e-12, 0.0)) != want
                          or orc.sample(l, t, k, p, min(u + 1e-12, 1 - 2**-53)) != want):
                skipped += 1
                continue
            got = hip_ops.sample(l, t, k, p, u)
            assert got == want, f"{name} t={t} k={k} p={p} u={u!r}: device {got}, oracle {want}"
            checked += 1
    print(f"[metrics] sampler {name}: {checked} draws identical to the oracle, {skipped} boundary draws skipped")
    assert skipped <= checked // 20


def test_device_sampler_edges(hip_ops):
    rng = np.random.default_rng(9)
    l = rng.standard_normal(100).astype(np.float32)
    for t, k, p in PARAMS:
        if t == 0:
            continue
        assert hip_ops.sample(l, t, k, p, 0.0) == orc.sample(l, t, k, p, 0.0)  # first candidate
        top = 1 - 2**-53
        assert hip_ops.sample(l, t, k, p, top) == orc.sample(l, t, k, p, top)  # last kept candidate
    assert hip_ops.sample([5.0], 1.0, 0, 1.0, 0.5) == 0
    assert hip_ops.sample(np.full(64, -np.inf, np.float32), 1.0, 0, 1.0, 0.5) == orc.sample(
        np.full(64, -np.inf, np.float32), 1.0, 0, 1.0, 0.5)


def test_device_sampler_reference_assertions(hip_ops):
    """SamplerTests.swift through the device: greedy tie rule, seeds, softmax
    frequencies (20,000 draws, 0.015), top-k and top-p supports."""
    ops = hip_ops

    def draws(n=20_000, **p):
        s = Sampler(**p)
        out = {}
        for _ in range(n):
            t = s.sample_logits(ops, LOGITS)
            out[t] = out.get(t, 0) + 1
        return out

    assert Sampler(temperature=0).sample_logits(ops, LOGITS) == 1
    a, b, c = Sampler(temperature=1, seed=42), Sampler(temperature=1, seed=42), Sampler(temperature=1, seed=43)
    sa = [a.sample_logits(ops, LOGITS) for _ in range(200)]
    assert sa == [b.sample_logits(ops, LOGITS) for _ in range(200)]
    assert sa != [c.sample_logits(ops, LOGITS) for _ in range(200)]
    for temperature in (0.5, 1.0, 2.0):
        counts = draws(temperature=temperature, seed=7)
        w = np.exp(np.array(LOGITS, np.float64) / temperature)
        for i, p in enumerate(w / w.sum()):
            assert abs(counts.get(i, 0) / 20_000 - p) < 0.015, (temperature, i)
    counts = draws(temperature=1, top_k=2, seed=1)
    assert set(counts) == {1, 4} and abs(counts[1] / 20_000 - 0.5) < 0.015
    assert set(draws(temperature=5, top_k=1, seed=1)) == {1}
    assert set(draws(temperature=1, top_p=0.3, seed=3)) == {1}
    assert set(draws(temperature=1, top_p=0.6, seed=3)) == {1, 4}
    assert set(draws(temperature=1, top_p=0.8, seed=3)) == {1, 2, 4}
    assert Sampler(temperature=0.1, seed=1).sample_logits(ops, [1e30, 0, -1e30]) == 0
    # the host sampler's stream is the oracle's (same SplitMix64 and uniform)
    s, o = Sampler(temperature=1, seed=11), orc.Sampler(temperature=1, seed=11)
    assert [s.rng.uniform() for _ in range(50)] == [o.draw() for _ in range(50)]


def test_device_sampler_rejects_bad_input(hip_ops):
    for t, k, p in [(-1.0, 0, 1.0), (float("nan"), 0, 1.0), (1.0, -1, 1.0), (1.0, 0, 0.0), (1.0, 0, 1.5)]:
        with pytest.raises(InvalidArgument):
            hip_ops.sample(LOGITS, t, k, p, 0.5)
    with pytest.raises(InvalidArgument):
        hip_ops.sample(LOGITS, 1.0, 0, 1.0, 1.0)  # u must be < 1
    with pytest.raises(InvalidArgument):
        hip_ops.sample([], 0.0, 0, 1.0, 0.5)
    for t in (0.0, 1.0):
        with pytest.raises(InvalidArgument, match="NaN"):
            hip_ops.sample([1.0, float("nan")], t, 0, 1.0, 0.5)


def test_session_sampling_reads_the_last_logits(hip_ctx, hip_ops):
    spec = synth.TINY
    model = HIPLlamaModel(hip_ctx, spec.config, built(spec))
    s = model.make_session(capacity=64)
    with pytest.raises(InvalidArgument, match="no logits"):
        s.sample(1.0, 0, 1.0, 0.5)
    logits = s.forward(synth.prompt_tokens(spec, 20))
    rng = np.random.default_rng(3)
    for t, k, p in [(1.0, 0, 1.0), (0.8, 40, 0.95), (0.0, 0, 1.0), (1.5, 0, 0.9)]:
        for u in rng.random(4):
            assert s.sample(t, k, p, u) == hip_ops.sample(logits, t, k, p, u)
    logits = s.decode(int(np.argmax(logits)))  # the persistent decode kernel's logits
    for u in rng.random(4):
        assert s.sample(0.9, 20, 0.9, u) == hip_ops.sample(logits, 0.9, 20, 0.9, u)
    s.decode_greedy(5, 3, lambda t: True)
    with pytest.raises(InvalidArgument, match="no logits"):
        s.sample(1.0, 0, 1.0, 0.5)
    # a sampled generation: host RNG, device selection, one token per step
    sampler = Sampler(temperature=0.9, top_k=50, top_p=0.95, seed=1)
    s.reset()
    s.forward(synth.prompt_tokens(spec, 10))
    toks = []
    for _ in range(8):
        toks.append(sampler.sample(s))
        s.decode(toks[-1])
    assert all(0 <= t < spec.config.vocab_size for t in toks)
