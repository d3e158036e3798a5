"""The multi-kernel decode step at a large model's layer shape.

C5's layer (hidden 2048, FFN 8192, 32 query / 32 KV heads of 64 dims) with two
layers and a 2,048-token vocabulary: with Q8_0 weights every projection and
the logits are at least 4 MB, so each takes the streamed GEMV with its
prologue or epilogue (the RMSNorm prologue, RoPE and the KV-cache append on the
QKV rows, SwiGLU, the residual add), the split-K attention partials are merged
by their own kernel in front of Wo, and the split-K decode attention runs with
its K and V rows loaded up front (Q4_0 and F16 cover the other formats, where
the smaller or wider matrices keep the one-tile-per-workgroup GEMV).

Held to the CPU oracle (LlamaCPUModel.forward, LlamaCPUModel.swift:24-61)
after an exact-mode prefill, within the BASELINE bound (2e-3 absolute + 1e-3
relative) with the same greedy token; to the one-tile-per-workgroup GEMV
(ALPACA_HIP_GEMV_STREAM=0) and to the persistent decode kernel within 1e-4 of
the logit peak (float32 summation order); and the greedy chain (the captured
graph with the position read on the device) to step-by-step decode.
"""
from dataclasses import replace

import numpy as np
import pytest

import oracle.oracle as orc
from alpaca_amd import synth
from alpaca_amd.model import HIPLlamaModel
from alpaca_amd.tensor import F16, Q4_0
from tests.helpers import assert_close, env, metrics
from tests.test_gpu_model import built, oracle_cfg, oracle_model

pytestmark = pytest.mark.gpu

C5_SHAPE = replace(synth.C5, config=replace(synth.C5.config, layer_count=2, vocab_size=2048, context_length=1024),
                   name="c5-shape-2l")
SPECS = [C5_SHAPE, synth.with_dtype(C5_SHAPE, Q4_0), synth.with_dtype(C5_SHAPE, F16)]


@pytest.mark.parametrize("spec", SPECS, ids=lambda s: s.name)
def test_large_shape_multi_kernel_decode(hip_ctx, spec):
    c = spec.config
    w = built(spec)
    model = HIPLlamaModel(hip_ctx, c, w)
    om = oracle_model(c, w)
    prompt = synth.prompt_tokens(spec, 20)
    with env(ALPACA_HIP_PERSISTENT_DECODE=0):
        multi = model.make_session(capacity=96, gemm_precision="exact")
    with env(ALPACA_HIP_PERSISTENT_DECODE=0, ALPACA_HIP_GEMV_STREAM=0):
        plain = model.make_session(capacity=96, gemm_precision="exact")
    with env(ALPACA_HIP_PERSISTENT_DECODE=2):
        pers = model.make_session(capacity=96, gemm_precision="exact")
    okv = orc.OracleKV(oracle_cfg(c), 96, rounds_f16=True)
    e = orc.forward(om, okv, prompt)
    for s in (multi, plain, pers):
        s.forward(prompt)
    tok = orc.argmax(e)
    for step in range(6):
        g = multi.decode(tok)
        with env(ALPACA_HIP_GEMV_STREAM=0):
            g_plain = plain.decode(tok)
        g_pers = pers.decode(tok)
        e = orc.forward(om, okv, [tok])
        m_plain, m_pers = metrics(g, g_plain), metrics(g, g_pers)
        print(f"[metrics] {spec.name} step {step}: vs one-tile GEMV {m_plain['max_rel_peak']:.2e}, "
              f"vs persistent {m_pers['max_rel_peak']:.2e}")
        assert m_plain["max_rel_peak"] <= 1e-4, step
        assert m_pers["max_rel_peak"] <= 1e-4, step
        assert_close(g, e, 2e-3, 1e-3, f"{spec.name} multi-kernel decode step {step}")
        assert int(np.argmax(g)) == int(np.argmax(e))
        tok = orc.argmax(e)
    # A default session takes the multi-kernel step where every projection of a
    # layer streams (Q8_0 here; the Q4_0 Wo is under 4 MB and the F16 down rows are
    # past the streamed kernel's 512 chunks, so those keep the persistent kernel):
    # a profiled decode leaves persistent-launch stamps only on that kernel.
    default = model.make_session(capacity=96, gemm_precision="exact")
    default.forward(prompt)
    for sess, persistent in ((default, spec.dtype != synth.C5.dtype), (multi, False), (pers, True)):
        sess.profiling_enabled = True
        sess.decode(tok)
        stamps, _ = sess.decode_timeline
        assert (stamps.size > 0) == persistent


def test_large_shape_greedy_chain_matches_stepwise(hip_ctx):
    """The greedy chain through the captured graph of the multi-kernel step
    (the default at this Q8_0 layer shape; positions read on the device,
    attention splits of 64 positions at this capacity) emits the tokens of
    step-by-step decode + host arg-max, across split boundaries."""
    spec = C5_SHAPE
    model = HIPLlamaModel(hip_ctx, spec.config, built(spec))
    prompt = synth.prompt_tokens(spec, 40)
    a = model.make_session(capacity=200)
    b = model.make_session(capacity=200)
    first = int(np.argmax(a.forward(prompt)))
    got = []
    fed = a.decode_greedy(first, 120, lambda t: got.append(t) or True)
    assert fed == 120 and a.length == 160
    tok = int(np.argmax(b.forward(prompt)))
    assert tok == first
    want = []
    for _ in range(120):
        tok = int(np.argmax(b.decode(tok)))
        want.append(tok)
    assert got == want
