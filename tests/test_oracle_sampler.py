"""The oracle's sampler (oracle/alpaca_oracle.c orc_sample / orc_uniform53)
against the reference's Tests/AlpacaCoreTests/SamplerTests.swift, case by
case with the same logits, seeds, draw counts and tolerances, plus a check of
the inverse-CDF draw against interval boundaries computed independently
(numpy cumulative sums of the sorted, filtered distribution).

The token stream of a seed also depends on how Swift turns a SplitMix64 word
into Double.random (orc_uniform53 restates the standard library; it cannot be
run here), so these tests pin the distribution and the draw given u, not the
exact stream of a Swift seed.
"""
import numpy as np
import pytest

import oracle.oracle as orc

LOGITS = [1.0, 3.0, 2.0, -1.0, 3.0, 0.5]


def draws(n=20_000, **p):
    s = orc.Sampler(**p)
    counts = {}
    for _ in range(n):
        t = s.sample(LOGITS)
        counts[t] = counts.get(t, 0) + 1
    return counts


def test_greedy_picks_first_maximum():
    assert orc.Sampler(temperature=0).sample(LOGITS) == 1  # tie between 1 and 4: lowest index


def test_seeded_sampling_is_reproducible_and_seeds_differ():
    a, b, c = orc.Sampler(temperature=1, seed=42), orc.Sampler(temperature=1, seed=42), orc.Sampler(temperature=1, seed=43)
    sa = [a.sample(LOGITS) for _ in range(200)]
    assert sa == [b.sample(LOGITS) for _ in range(200)]
    assert sa != [c.sample(LOGITS) for _ in range(200)]


@pytest.mark.parametrize("temperature", [0.5, 1.0, 2.0])
def test_temperature_distribution_matches_softmax(temperature):
    counts = draws(temperature=temperature, seed=7)
    w = np.exp(np.array(LOGITS, np.float64) / temperature)
    for i, p in enumerate(w / w.sum()):
        assert abs(counts.get(i, 0) / 20_000 - p) < 0.015, (temperature, i)


def test_top_k_restricts_support_and_renormalises():
    counts = draws(temperature=1, top_k=2, seed=1)
    assert set(counts) == {1, 4}  # the two tied maxima
    assert abs(counts[1] / 20_000 - 0.5) < 0.015
    assert set(draws(temperature=5, top_k=1, seed=1)) == {1}


def test_top_p_keeps_smallest_nucleus():
    # softmax(T=1): tokens 1, 4 ~ 0.389 each, token 2 ~ 0.143 -> cumulative 0.389, 0.778, 0.921
    assert set(draws(temperature=1, top_p=0.3, seed=3)) == {1}
    assert set(draws(temperature=1, top_p=0.6, seed=3)) == {1, 4}
    assert set(draws(temperature=1, top_p=0.8, seed=3)) == {1, 2, 4}
    assert set(draws(temperature=1, top_p=1.0, seed=3)) == set(range(6))


def test_invalid_inputs_are_rejected():
    for bad in [dict(temperature=-1), dict(temperature=float("nan")), dict(top_k=-1), dict(top_p=0),
                dict(top_p=1.5)]:
        with pytest.raises(ValueError):
            orc.Sampler(**bad)
    s = orc.Sampler(temperature=0)
    with pytest.raises(ValueError):
        s.sample([])
    with pytest.raises(ValueError):
        s.sample([1, float("nan")])
    with pytest.raises(ValueError):
        orc.Sampler(temperature=1).sample([1, float("nan")])


def test_extreme_logits_do_not_overflow():
    assert orc.Sampler(temperature=0.1, seed=1).sample([1e30, 0, -1e30]) == 0


def interval_token(logits, temperature, top_k, top_p, u):
    """The draw by boundaries: order, filter and normalise with numpy, then
    the token whose cumulative interval holds u."""
    l = np.asarray(logits, np.float32)
    n = l.size
    k = min(top_k, n) if top_k > 0 else n
    order = np.arange(n)
    if k < n or top_p < 1:
        order = np.lexsort((np.arange(n), -l.astype(np.float64)))[:k]
    p = np.exp((l[order].astype(np.float64) - l[order].max()) / temperature)
    if top_p < 1:
        c = np.cumsum(p / p.sum())
        keep = int(np.argmax(c >= top_p)) + 1 if (c >= top_p).any() else len(p)
        order, p = order[:keep], p[:keep]
    edges = np.cumsum(p) / p.sum()
    return int(order[min(int(np.searchsorted(edges, u, side="right")), len(order) - 1)])


@pytest.mark.parametrize("case", range(12))
def test_draw_given_u_matches_interval_boundaries(case):
    rng = np.random.default_rng(case)
    n = [6, 50, 1000, 5000][case % 4]
    l = rng.standard_normal(n).astype(np.float32) * [0.5, 2, 5][case % 3]
    l[rng.integers(0, n, n // 10)] = l[0]  # ties
    t, k, p = [(1.0, 0, 1.0), (0.7, 40, 1.0), (1.3, 0, 0.9), (0.5, 200, 0.8)][case % 4]
    for u in rng.random(200):
        # skip draws within 1e-9 of an interval edge, where the two summation orders may disagree
        want = interval_token(l, t, k, p, u)
        if interval_token(l, t, k, p, min(u + 1e-9, 1 - 1e-16)) != want or interval_token(l, t, k, p, max(u - 1e-9, 0)) != want:
            continue
        assert orc.sample(l, t, k, p, u) == want


def test_uniform53_is_the_low_53_bits():
    st = orc.C.c_uint64(5)
    w = orc.lib().orc_splitmix_next(orc.C.byref(orc.C.c_uint64(5)))
    assert orc.lib().orc_uniform53(orc.C.byref(st)) == (w & ((1 << 53) - 1)) * 2.0**-53
