"""Whole-model parity of the HIP session against the CPU oracle.

Follows Tests/AlpacaIntegrationTests/MetalRealModelTests.swift (GPU vs CPU
across chunks and reset, greedy chain vs synchronous decoding, early stop,
capacity) and TransformerTests.swift (tiny models), on synthetic weights and
on the reference's tiny_llama.json fixture.

Tolerances: the C1 north-star test holds logits within 2e-3 absolute + 1e-3
relative of the oracle and greedy ids identical.  The exact configuration
(float32 GEMMs, f32 KV) is held to 1e-4 everywhere.  Other fast-path cases
(f16 MFMA operands) use the reference's own fast-path bound: max |error| /
max |logit| <= 3e-3 (MetalRealModelTests.swift, NUMERICAL_VALIDATION.md
"peak-relative 3e-3"), plus greedy agreement.  With an f16 KV cache the oracle
rounds its cache rows through f16 as well (KVCache.roundsToFloat16).
"""
import numpy as np
import pytest

import oracle.oracle as orc
from alpaca_amd import synth
from alpaca_amd.model import HIPLlamaModel, LlamaConfig
from alpaca_amd.tensor import F16, F32, Q4_0, Q8_0, QTensor, encode
from tests.helpers import assert_close, metrics, tiny_llama_case

pytestmark = pytest.mark.gpu


def oracle_cfg(c: LlamaConfig) -> dict:
    return dict(vocab=c.vocab_size, hidden=c.hidden_size, layers=c.layer_count, heads=c.head_count,
                kv_heads=c.kv_head_count, head_dim=c.head_dim, ffn=c.feed_forward_size, context=c.context_length,
                eps=c.rms_norm_eps, theta=c.rope_theta, interleaved=c.rope_interleaved)


def oracle_model(spec_cfg: LlamaConfig, weights: dict):
    w = {n: (t.dtype, t.data) for n, t in weights.items()}
    return orc.OracleModel(oracle_cfg(spec_cfg), w)


_models = {}


def built(spec):
    key = repr(spec)  # the whole spec: two specs may share a name across test files
    if key not in _models:
        _models[key] = synth.build_weights(spec)
    return _models[key]


def gpu_model(ctx, spec):
    return HIPLlamaModel(ctx, spec.config, built(spec))


def check(g, e, kv, prec, label):
    """exact with an f32 cache: 1e-4; exact and the two-term fast path (the
    default): the BASELINE bar 2e-3 + 1e-3 relative; one f16 term per
    activation (fast-f16): the reference's fast-path bound, 3e-3 of the logit
    peak (MetalRealModelTests.swift)."""
    if prec == "exact" and kv == "f32":
        assert_close(g, e, 1e-4, 0.0, label)
    elif prec in ("exact", "fast"):
        assert_close(g, e, 2e-3, 1e-3, label)
    else:
        m = metrics(g, e)
        print(f"[metrics] {label}: {m}")
        assert m["max_rel_peak"] <= 3e-3, label
    assert int(np.argmax(g)) == int(np.argmax(e)), label


TINY_SPECS = [synth.TINY, synth.with_dtype(synth.TINY, Q4_0), synth.with_dtype(synth.TINY, F16)]


@pytest.mark.parametrize("spec", TINY_SPECS, ids=lambda s: s.name)
@pytest.mark.parametrize("kv,prec", [("f32", "exact"), ("f16", "exact"), ("f16", "fast"), ("f32", "fast"),
                                     ("f16", "fast-f16")])
def test_tiny_prefill_and_decode_match_oracle(hip_ctx, spec, kv, prec):
    c = spec.config
    model = gpu_model(hip_ctx, spec)
    om = oracle_model(c, built(spec))
    prompt = synth.prompt_tokens(spec, 40)
    s = model.make_session(capacity=128, max_batch=512, kv_precision=kv, gemm_precision=prec)
    okv = orc.OracleKV(oracle_cfg(c), 128, rounds_f16=(kv == "f16"))
    g = s.forward(prompt)
    e = orc.forward(om, okv, prompt)
    check(g, e, kv, prec, f"{spec.name} {kv}/{prec} prefill")
    tok = orc.argmax(e)
    for step in range(6):
        g = s.decode(tok)
        e = orc.forward(om, okv, [tok])
        check(g, e, kv, prec, f"{spec.name} {kv}/{prec} decode {step}")
        tok = orc.argmax(e)
    assert s.length == 46


@pytest.mark.parametrize("prec", ["exact", "fast", "fast-f16"])
def test_split_half_rope_layout_matches_oracle(hip_ctx, prec):
    """Hugging Face split-half RoPE (ropeInterleaved = false): q/k rows are
    re-paired at upload; logits must still match the oracle's split-half rotation."""
    from dataclasses import replace
    spec = replace(synth.TINY, config=replace(synth.TINY.config, rope_interleaved=False), name="tiny-hf")
    c = spec.config
    w = built(synth.TINY)
    model = HIPLlamaModel(hip_ctx, c, w)
    om = oracle_model(c, w)
    prompt = synth.prompt_tokens(spec, 33)
    kv = "f32" if prec == "exact" else "f16"
    s = model.make_session(capacity=64, kv_precision=kv, gemm_precision=prec)
    okv = orc.OracleKV(oracle_cfg(c), 64, rounds_f16=(kv == "f16"))
    check(s.forward(prompt), orc.forward(om, okv, prompt), kv, prec, f"split-half prefill {prec}")
    for t in (5, 17, 900):
        check(s.decode(t), orc.forward(om, okv, [t]), kv, prec, f"split-half decode {prec}")


def test_profiled_greedy_equals_graph_greedy(hip_ctx):
    """The greedy chain replays a captured HIP graph; with profiling on it launches the
    same kernels eagerly.  Both must emit the same tokens, and stages must be reported."""
    spec = synth.TINY
    model = gpu_model(hip_ctx, spec)
    prompt = synth.prompt_tokens(spec, 50)
    out = []
    for prof in (False, True, False):
        s = model.make_session(capacity=256)
        s.profiling_enabled = prof
        first = int(np.argmax(s.forward(prompt)))
        got = []
        s.decode_greedy(first, 60, lambda t: got.append(t) or True)
        out.append(got)
        if prof:
            st = s.last_profile
            assert st["attention"].dispatches == 60 * spec.config.layer_count
            assert "sample" in st and st["qkv (fused norm)"].seconds > 0
    assert out[0] == out[1] == out[2]


def test_chunked_prefill_equals_single_pass_and_reset_is_deterministic(hip_ctx):
    spec = synth.TINY
    model = gpu_model(hip_ctx, spec)
    prompt = synth.prompt_tokens(spec, 90)
    one = model.make_session(capacity=128, max_batch=512, kv_precision="f32", gemm_precision="exact")
    chunked = model.make_session(capacity=128, max_batch=32, kv_precision="f32", gemm_precision="exact")
    a = one.forward(prompt)
    b = chunked.forward(prompt)
    assert metrics(a, b)["max_abs"] < 1e-5
    one.reset()
    again = one.forward(prompt)
    assert np.array_equal(again, a), "reset must reproduce the first run bit-for-bit"
    # incremental = one-shot
    inc = model.make_session(capacity=128, max_batch=512, kv_precision="f32", gemm_precision="exact")
    inc.forward(prompt[:50])
    for t in prompt[50:-1]:
        inc.decode(int(t))
    last = inc.decode(int(prompt[-1]))
    assert metrics(last, a)["max_abs"] < 1e-4


def test_session_errors_leave_length_unchanged(hip_ctx):
    from alpaca_amd import _lib as L
    spec = synth.TINY
    model = gpu_model(hip_ctx, spec)
    s = model.make_session(capacity=16)
    s.forward([1, 2, 3])
    with pytest.raises(L.InvalidArgument):
        s.forward([])
    with pytest.raises(L.InvalidArgument):
        s.forward([spec.config.vocab_size])
    with pytest.raises(L.InvalidArgument):
        s.forward([-1])
    with pytest.raises(L.InvalidArgument):
        s.forward(list(range(14)))
    assert s.length == 3
    s.forward(list(range(13)))
    assert s.length == 16
    with pytest.raises(L.InvalidArgument):
        s.decode(1)
    assert s.capacity == 16


def test_greedy_chain_matches_synchronous_decoding(hip_ctx):  # MetalRealModelTests.swift:81-122
    from alpaca_amd import _lib as L
    spec = synth.TINY
    model = gpu_model(hip_ctx, spec)
    prompt = synth.prompt_tokens(spec, 24)
    sync = model.make_session(capacity=128)
    logits = sync.forward(prompt)
    expected = []
    for _ in range(40):
        t = int(np.argmax(logits))
        expected.append(t)
        logits = sync.forward([t])
    chain = model.make_session(capacity=128)
    first = int(np.argmax(chain.forward(prompt)))
    assert first == expected[0]
    got = []
    fed = chain.decode_greedy(first, 39, lambda t: got.append(t) or True)
    assert [first] + got == expected
    assert fed == 39 and chain.length == 24 + 39
    stop = model.make_session(capacity=128)
    stop.forward(prompt)
    seen = []
    fed2 = stop.decode_greedy(first, 30, lambda t: (seen.append(t), len(seen) < 5)[1])
    assert seen == expected[1:6] and fed2 == 5 and stop.length == 24 + 5
    assert int(np.argmax(stop.forward([expected[5]]))) == expected[6]
    tight = model.make_session(capacity=24 + 3)
    tight.forward(prompt)
    n = []
    assert tight.decode_greedy(first, 100, lambda t: n.append(t) or True) == 3
    assert len(n) == 3 and tight.length == 27
    assert tight.decode_greedy(first, 5, lambda t: True) == 0
    with pytest.raises(L.InvalidArgument):
        tight.decode_greedy(spec.config.vocab_size + 5, 1, lambda t: True)


def _tiny_llama_weights(name, gguf, dtype):
    cfg, w, tokens, ref = tiny_llama_case(name, gguf)
    c = LlamaConfig(cfg["vocab"], cfg["hidden"], cfg["layers"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"],
                    cfg["ffn"], cfg["context"], cfg["eps"], cfg["theta"], gguf)
    q = {}
    for n, (_, arr) in w.items():
        a = np.asarray(arr, np.float32)
        q[n] = encode(a.reshape(1, -1) if a.ndim == 1 else a, F32 if n.endswith("norm") else dtype)
    return c, q, tokens, ref


@pytest.mark.parametrize("name,gguf", [("gqa_untied", True), ("gqa_untied", False), ("mha_tied", True),
                                       ("mha_tied", False)])
def test_tiny_llama_fixture_on_gpu(hip_ctx, name, gguf):
    """tiny_llama.json (head_dim 8 is below the GPU kernels' 32-multiple, as on Metal) is rejected;
    the same weights widened are not needed: the fixture pins the oracle, the oracle pins the GPU."""
    from alpaca_amd import _lib as L
    c, q, tokens, ref = _tiny_llama_weights(name, gguf, F16)
    with pytest.raises(L.Unsupported):
        HIPLlamaModel(hip_ctx, c, q)


def test_c1_prefill_and_greedy_tokens_identical_to_oracle(hip_ctx):
    """C1 (135M-shape Q8_0): 128-token prompt then 16 greedy tokens, default GPU
    configuration (fast prefill, f16 KV) vs the oracle with an f16-rounded cache."""
    spec = synth.C1
    c = spec.config
    w = built(spec)
    model = HIPLlamaModel(hip_ctx, c, w)
    om = oracle_model(c, w)
    prompt = synth.prompt_tokens(spec, 128)
    okv = orc.OracleKV(oracle_cfg(c), 256, rounds_f16=True)
    e = orc.forward(om, okv, prompt)
    s = model.make_session(capacity=256)
    g = s.forward(prompt)
    m = assert_close(g, e, 2e-3, 1e-3, "C1 prefill logits")
    expected = [orc.argmax(e)]
    margins = []
    for _ in range(15):
        srt = np.sort(e)
        margins.append(float(srt[-1] - srt[-2]))
        e = orc.forward(om, okv, [expected[-1]])
        expected.append(orc.argmax(e))
    got = []
    first = int(np.argmax(g))
    assert first == expected[0]
    s.decode_greedy(first, 15, lambda t: got.append(t) or True)
    print(f"[metrics] C1 greedy oracle {expected} gpu {[first] + got} min top-2 margin {min(margins):.3e}")
    assert [first] + got == expected
