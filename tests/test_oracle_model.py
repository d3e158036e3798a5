"""Pins the oracle's Llama forward and KV cache to the reference's tiny_llama.json.

Mirrors Tests/AlpacaCoreTests/TransformerTests.swift: float64 Hugging Face
logits at every position (atol 2e-5), greedy agreement, incremental decode and
split prefill equal to one-shot, cache bounds, reset and failed-forward rules.
"""
import numpy as np
import pytest

import oracle.oracle as orc
from tests.helpers import assert_close, metrics, tiny_llama_case

VARIANTS = [(n, g) for n in ("gqa_untied", "mha_tied") for g in (False, True)]


def _model(name, gguf):
    cfg, w, tokens, logits = tiny_llama_case(name, gguf)
    return cfg, orc.OracleModel(cfg, w), w, tokens, logits


@pytest.mark.parametrize("name,gguf", VARIANTS)
def test_prefill_logits_match_float64(name, gguf):  # TransformerTests.swift:44-60
    cfg, m, _, tokens, ref = _model(name, gguf)
    kv = orc.OracleKV(cfg, cfg["context"])
    got = orc.forward(m, kv, tokens, all_logits=True)
    assert got.shape == (tokens.size, cfg["vocab"])
    assert_close(got, ref, 2e-5, 0, f"prefill {name} gguf={gguf}")
    r = ref.reshape(tokens.size, -1)
    for p in range(tokens.size):
        assert int(np.argmax(got[p])) == int(np.argmax(r[p]))


@pytest.mark.parametrize("name,gguf", VARIANTS)
def test_incremental_decode_matches_uncached(name, gguf):  # TransformerTests.swift:61-80
    cfg, m, _, tokens, ref = _model(name, gguf)
    kv = orc.OracleKV(cfg, cfg["context"])
    steps = np.stack([orc.forward(m, kv, [t]) for t in tokens])
    assert_close(steps, ref, 2e-5, 0, f"incremental {name}")
    split = orc.OracleKV(cfg, cfg["context"])
    first = orc.forward(m, split, tokens[:4], all_logits=True)
    second = orc.forward(m, split, tokens[4:], all_logits=True)
    full = orc.forward(m, orc.OracleKV(cfg, cfg["context"]), tokens, all_logits=True)
    assert metrics(np.concatenate([first, second]), full)["max_abs"] < 5e-6
    assert kv.length == tokens.size


def test_cache_bounds_and_reset():  # TransformerTests.swift:82-99
    cfg, m, _, tokens, _ = _model("gqa_untied", True)
    kv = orc.OracleKV(cfg, 8)
    orc.forward(m, kv, tokens)
    with pytest.raises(ValueError):
        orc.forward(m, kv, [1, 2])
    assert kv.length == 7, "failed forward must not advance the cache"
    orc.forward(m, kv, [1])
    with pytest.raises(ValueError):
        orc.forward(m, kv, [1])
    kv.reset()
    a = orc.forward(m, kv, tokens)
    b = orc.forward(m, orc.OracleKV(cfg, 8), tokens)
    assert np.array_equal(a, b)
    with pytest.raises(ValueError):
        orc.forward(m, kv, [])
    with pytest.raises(IndexError):
        orc.forward(m, orc.OracleKV(cfg, 64), [64])


def test_f16_rounded_cache_stays_close():
    """KVCache.roundsToFloat16 (KVCache.swift:18-20): logits move by f16 rounding only."""
    cfg, m, _, tokens, ref = _model("gqa_untied", True)
    kv = orc.OracleKV(cfg, 16, rounds_f16=True)
    got = orc.forward(m, kv, tokens, all_logits=True)
    mm = metrics(got, ref)
    assert mm["max_abs"] < 5e-3 and mm["max_abs"] > 0
    k = kv.keys(0)[: tokens.size]
    assert np.array_equal(k, k.astype(np.float16).astype(np.float32))
