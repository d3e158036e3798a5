"""Shared test helpers: fixture loading, tolerance checks and error metrics.

`assert_close` follows the reference's assertClose (Tests/AlpacaCoreTests/
Support.swift:24-34): |a - e| <= atol + rtol * |e| element-wise.  `metrics`
follows ErrorMetrics (Sources/AlpacaCore/Runtime/ErrorMetrics.swift:7-36).
"""
import base64
import json
import os
from contextlib import contextmanager

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_cache = {}


def fixture(name: str) -> dict:
    if name not in _cache:
        with open(os.path.join(GOLDEN, name + ".json")) as f:
            _cache[name] = json.load(f)
    return _cache[name]


@contextmanager
def env(**kv):
    """Sets environment variables (None: unsets one) for the duration of a
    with-block (the HIP library reads its ALPACA_HIP_* switches when a session
    is created)."""
    old = {k: os.environ.get(k) for k in kv}
    for k, v in kv.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = str(v)
    try:
        yield
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def b64(s: str) -> np.ndarray:
    return np.frombuffer(base64.b64decode(s), dtype=np.uint8).copy()


def metrics(actual, expected) -> dict:
    a = np.asarray(actual, dtype=np.float64).ravel()
    e = np.asarray(expected, dtype=np.float64).ravel()
    assert a.size == e.size, f"length mismatch {a.size} vs {e.size}"
    d = np.abs(a - e)
    peak = float(np.abs(e).max()) if e.size else 0.0
    mx = float(d.max()) if d.size else 0.0
    return {
        "count": int(a.size),
        "max_abs": mx,
        "mean_abs": float(d.mean()) if d.size else 0.0,
        "rms": float(np.sqrt((d * d).mean())) if d.size else 0.0,
        "max_rel_peak": mx / peak if peak > 0 else mx,
    }


def assert_close(actual, expected, atol: float, rtol: float = 0.0, label: str = ""):
    a = np.asarray(actual, dtype=np.float64).ravel()
    e = np.asarray(expected, dtype=np.float64).ravel()
    assert a.size == e.size, f"{label}: length {a.size} vs {e.size}"
    m = metrics(a, e)
    print(f"[metrics] {label}: n={m['count']} maxAbs={m['max_abs']:.3e} meanAbs={m['mean_abs']:.3e} "
          f"maxRel(peak)={m['max_rel_peak']:.3e} (atol={atol} rtol={rtol})")
    bad = np.abs(a - e) > atol + rtol * np.abs(e)
    bad |= np.isnan(a) != np.isnan(e)
    if bad.any():
        i = int(np.argmax(bad))
        raise AssertionError(f"{label}[{i}]: {a[i]} vs {e[i]} exceeds atol {atol} rtol {rtol}")
    return m


def splitmix_uniform(seed: int, n: int) -> np.ndarray:
    """KernelTests.swift:102-114 SplitMix.nextFloat(): uniform in [-1, 1), as float32.

    next() is a pure function of the step index, so the sequence is computed
    vectorised: state_i = seed + (i + 1) * gamma (mod 2^64)."""
    gamma = np.uint64(0x9E3779B97F4A7C15)
    with np.errstate(over="ignore"):
        s = np.uint64(seed) + (np.arange(1, n + 1, dtype=np.uint64) * gamma)
        z = s
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    u = (z >> np.uint64(11)).astype(np.float64) / float(1 << 53)
    return (u.astype(np.float32) * np.float32(2) - np.float32(1)).astype(np.float32)


def tiny_llama_case(name: str, gguf: bool):
    """Config and weights of one tiny_llama.json variant (TransformerTests.swift:18-37)."""
    import oracle.oracle as orc
    c = fixture("tiny_llama")[name]
    cc = c["config"]
    cfg = dict(vocab=cc["vocab"], hidden=cc["hidden"], layers=cc["layers"], heads=cc["heads"],
               kv_heads=cc["kvHeads"], head_dim=cc["headDim"], ffn=cc["ffn"], context=cc["context"],
               eps=cc["eps"], theta=cc["theta"], interleaved=gguf, tied=cc["tied"])
    w = c["weights_gguf" if gguf else "weights_hf"]
    weights = {}
    for n, e in w.items():
        arr = np.asarray(e["data"], dtype=np.float32).reshape(e["shape"])
        weights[n] = (orc.F32, arr)
    return cfg, weights, np.asarray(c["tokens"], dtype=np.int32), np.asarray(c["logits"], dtype=np.float64)
