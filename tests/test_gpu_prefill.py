"""The fast prefill's fused QKV epilogue: RoPE and the KV-cache append done by
the QKV GEMM (GEMM_QKV_ROPE) instead of a separate kernel over an f32 q/k/v
buffer.  The epilogue evaluates the rotation in the unfused kernel's order on
the same float32 accumulators, so a fused session and an unfused one
(ALPACA_HIP_FUSE_QKV_ROPE=0, read at session creation) must agree bit for bit:
the prefill logits (which read q through attention) and the decode steps after
it (which read the cached k/v rows), across two chunks so the second starts at
a non-zero position.

The prefill weight cache (MetalLlamaModel.buildPrefillCache, MetalLlamaModel.
swift:97-120): a model created with it prefills exactly as a model whose layer
projections are f16(d*q), and its exact prefill and decode are those of the
model without the cache.
"""
from dataclasses import replace

import numpy as np
import pytest

from alpaca_amd import synth
from alpaca_amd.model import HIPLlamaModel
from alpaca_amd.tensor import F16, Q4_0
from tests.helpers import env
from tests.test_gpu_model import built

pytestmark = pytest.mark.gpu

SPECS = [
    synth.TINY,
    synth.with_dtype(synth.TINY, F16),
    replace(synth.TINY, config=replace(synth.TINY.config, head_dim=128), name="tiny-hd128"),
    # C4's layer shape (hidden 960, 15/5 heads, Q4_0) with 2 layers: N = 1600 leaves a partial tile
    replace(synth.C4, config=replace(synth.C4.config, layer_count=2, vocab_size=2048, context_length=512),
            name="c4-shape-2l"),
]


@pytest.mark.parametrize("prec", ["fast", "fast-f16"])
@pytest.mark.parametrize("spec", SPECS, ids=lambda s: s.name)
def test_fused_qkv_rope_is_bit_identical_to_unfused(hip_ctx, spec, prec):
    model = HIPLlamaModel(hip_ctx, spec.config, built(spec))
    prompt = synth.prompt_tokens(spec, 150)
    with env(ALPACA_HIP_FUSE_QKV_ROPE=0):
        ref = model.make_session(capacity=200, gemm_precision=prec)
    fused = model.make_session(capacity=200, gemm_precision=prec)
    for chunk in (prompt[:70], prompt[70:]):  # the second chunk starts at position 70
        a, b = fused.forward(chunk), ref.forward(chunk)
        assert np.array_equal(a, b), f"prefill logits differ: max |d| {np.abs(a - b).max():.3e}"
    tok = int(np.argmax(a))
    for step in range(3):
        a, b = fused.decode(tok), ref.decode(tok)
        assert np.array_equal(a, b), f"decode step {step} differs: max |d| {np.abs(a - b).max():.3e}"
        tok = int(np.argmax(a))


C4_LONG = replace(synth.C4, config=replace(synth.C4.config, layer_count=2, vocab_size=2048, context_length=4352),
                  name="c4-shape-2l-4096")


def test_fused_qkv_rope_with_large_tiles(hip_ctx):
    """A 4096-token chunk at C4's layer shape: the QKV GEMM (N = 1600) runs the
    RoPE epilogue (and the head-dim-64 RoPE staging) on whichever tile the
    grid rule picks.  Fused and unfused sessions agree bit for bit, and so do
    the tile families forced through ALPACA_HIP_GEMM_TILE (read at every
    launch: 64x64, 128x64, 128x128 and 128x256), since each output
    accumulates the same blocks in the same order."""
    spec = C4_LONG
    model = HIPLlamaModel(hip_ctx, spec.config, built(spec))
    prompt = synth.prompt_tokens(spec, 4096)
    with env(ALPACA_HIP_FUSE_QKV_ROPE=0):
        ref = model.make_session(capacity=4200, max_batch=4096, gemm_precision="fast")
    fused = model.make_session(capacity=4200, max_batch=4096, gemm_precision="fast")
    a, b = fused.forward(prompt), ref.forward(prompt)
    assert np.array_equal(a, b), f"prefill logits differ: max |d| {np.abs(a - b).max():.3e}"
    tok = int(np.argmax(a))
    for step in range(2):
        x, y = fused.decode(tok), ref.decode(tok)
        assert np.array_equal(x, y), f"decode step {step} differs: max |d| {np.abs(x - y).max():.3e}"
        tok = int(np.argmax(x))
    for tile in ("64x64", "128x64", "128x128", "128x256"):
        fused.reset()
        with env(ALPACA_HIP_GEMM_TILE=tile):
            t = fused.forward(prompt)
        assert np.array_equal(t, a), f"tile {tile}: prefill logits differ: max |d| {np.abs(t - a).max():.3e}"


HD128_1K = replace(synth.TINY, config=replace(synth.TINY.config, head_count=4, kv_head_count=1, head_dim=128,
                                              context_length=1100), name="tiny-hd128-g4-1k")


@pytest.mark.parametrize("prec", ["fast", "fast-f16"])
@pytest.mark.parametrize("spec", [HD128_1K, C4_LONG], ids=lambda s: s.name)
def test_fused_qkv_rope_under_each_forced_tile(hip_ctx, spec, prec):
    """Fused and unfused sessions agree bit for bit under every tile family
    forced alike for both, including the two-K-set 64x64 tile, whose RoPE
    table copy (32 KB at head dim 128) is larger than one K set's
    single-term stage buffers and so overlaps the buffer through which the
    second set hands its accumulators to the first."""
    model = HIPLlamaModel(hip_ctx, spec.config, built(spec))
    prompt = synth.prompt_tokens(spec, 1024)
    with env(ALPACA_HIP_FUSE_QKV_ROPE=0):
        ref = model.make_session(capacity=1100, max_batch=1024, gemm_precision=prec)
    fused = model.make_session(capacity=1100, max_batch=1024, gemm_precision=prec)
    for tile in ("64x64", "64x64k2", "128x64", "128x128"):
        fused.reset()
        ref.reset()
        with env(ALPACA_HIP_GEMM_TILE=tile, ALPACA_HIP_PREFILL_STREAMS=1):
            a, b = fused.forward(prompt), ref.forward(prompt)
        assert np.array_equal(a, b), f"{spec.name} {prec} tile {tile}: max |d| {np.abs(a - b).max():.3e}"
        tok = int(np.argmax(a))
        x, y = fused.decode(tok), ref.decode(tok)
        assert np.array_equal(x, y), f"{spec.name} {prec} tile {tile}: decode max |d| {np.abs(x - y).max():.3e}"
    model.close()


# ------------------------------------------------------------------ two-stream prefill

C1_2L = replace(synth.C1, config=replace(synth.C1.config, layer_count=2, context_length=4352), name="c1-shape-2l")


@pytest.mark.parametrize("prec,rows", [("fast", "all"), ("fast", "last"), ("fast-f16", "last")])
@pytest.mark.parametrize("spec", [C1_2L, C4_LONG, synth.with_dtype(replace(C1_2L, name="c1-shape-2l-f16"), F16)],
                         ids=lambda s: s.name)
def test_two_stream_prefill_matches_one_stream(hip_ctx, spec, prec, rows):
    """A fast prefill chunk of at least 1,536 tokens whose QKV GEMM grid is at
    most two rounds of 128x64 tiles runs as two halves on two
    streams (the second half's attention of each layer waits for the first
    half's K/V rows).  Every row goes through the same arithmetic as in one
    stream, but a half's smaller grids may take other tiles: the GEMM's
    two-K-set 64x64 tiles and the flash kernel's other key-range split each
    change the float32 summation order.  With every row's activations in two
    f16 terms (ALPACA_HIP_LO_ROWS=all) that order is all that differs, so the
    logits and the decode steps that read the cache agree with
    ALPACA_HIP_PREFILL_STREAMS=1 (read per call) to 1e-5 of the logit peak.
    By default only the QKV input and the rows from the last row rounded down
    to a multiple of 256 (the same rows in both runs: the split point is a
    multiple of 256) take two terms, and past 256 rows the returned row is
    computed in float32 where its launch allows it (the flash launch's wave-sets
    and the GEMM sizes can differ for a half); a float32 value that differs in its last
    bit can then round to the neighbouring f16 (2^-11 relative) in the one-term
    rows, so the runs agree to 2.5e-4 of the peak, and each is held to the
    CPU oracle at full size by the C1P workload test.  (One-term activations
    throughout, fast-f16, never take the two-K-set tiles, and agree to 1e-5.)
    Cases: a 1600-token
    chunk (halves of 768 and 832 rows, just past the 1,536-token threshold),
    one 3100-token chunk (uneven halves), then a 4300-token prompt over chunks
    of 3200 (a split chunk, then a short one at position 3200)."""
    tol = 1e-5 if rows == "all" or prec == "fast-f16" else 2.5e-4
    model = HIPLlamaModel(hip_ctx, spec.config, built(spec))
    prompt = synth.prompt_tokens(spec, 4300)
    for n in (1600, 3100, 4300):
        out = {}
        for streams in ("1", "2"):
            with env(ALPACA_HIP_LO_ROWS=rows):
                s = model.make_session(capacity=4352, max_batch=3200, gemm_precision=prec)
            with env(ALPACA_HIP_PREFILL_STREAMS=streams):
                g = s.forward(prompt[:n])
            tok = int(np.argmax(g))
            steps = [g]
            for _ in range(2):
                steps.append(s.decode(tok))
                tok = int(np.argmax(steps[-1]))
            out[streams] = steps
            s.close()
        for k, (a, b) in enumerate(zip(out["1"], out["2"])):
            d = float(np.abs(a - b).max())
            print(f"[metrics] {spec.name} {prec} rows={rows} n={n} step {k}: two streams vs one max |d| {d:.2e} "
                  f"({d / float(np.abs(a).max()):.2e} of the peak)")
            assert d <= tol * float(np.abs(a).max()), f"{spec.name} {prec} {rows} n={n} step {k}: max |d| {d:.3e}"
            assert int(np.argmax(a)) == int(np.argmax(b))
    model.close()


# ------------------------------------------------------------------ float32 last row

@pytest.mark.parametrize("spec", [C1_2L, C4_LONG], ids=lambda s: s.name)
def test_float32_last_row_matches_two_term_tail(hip_ctx, spec):
    """The row a prefill returns (its last), past the first 256 rows of a call:
    - attention: where the flash launch runs two wave-sets (head dim 64, small
      grids) the row is computed in float32 by workgroups of its own (key
      splits merged by the last one to arrive, a counter per head) and the
      other rows take one f16 term of Q and P; ALPACA_HIP_EXACT_LAST_ROW=0 (read
      at session creation) keeps both second terms on the row's query block;
    - Wo, gate/up and down: over 2,048 rows and more, GEMMs of at least 2M
      weights cover the other rows with one term and the row is a float32 GEMV
      over its two f16 terms; ALPACA_HIP_LAST_ROW_GEMV (a mask, read per call:
      0 none, 7 all three) forces the choice, and with 0 the tail rows from the
      last rounded down to 256 take their second terms in the GEMMs.
    Every form approximates the same float32 row: the logits agree with the
    all-second-terms form to 2.5e-4 of the peak (the tail's other rows round
    differently) with the same greedy token, over one attention split (300
    tokens), several (1000), a two-stream chunk (3100) and a second chunk at
    position 1200.  A repeated prefill on the same session is bit-identical
    (the counters return to zero, the merge order is fixed), and a 100-token
    call, below 256 rows, keeps the second terms (bit-identical to them).
    Each default path is held to the CPU oracle at full size by the workload
    tests."""
    model = HIPLlamaModel(hip_ctx, spec.config, built(spec))
    prompt = synth.prompt_tokens(spec, 3100)
    a = model.make_session(capacity=3200, max_batch=3200)
    with env(ALPACA_HIP_EXACT_LAST_ROW=0):
        b = model.make_session(capacity=3200, max_batch=3200)

    def run(s, mask):
        s.reset()
        p0 = 0
        with env(ALPACA_HIP_LAST_ROW_GEMV=mask):
            for n in chunks:
                g = s.forward(prompt[p0:p0 + n])
                p0 += n
        return g

    for chunks in ([100], [300], [1000], [3100], [1200, 500]):
        ref = run(b, "0")  # second terms on the tail, no float32 row
        forms = {"default": run(a, None), "all GEMVs": run(a, "7"), "attention only": run(a, "0"),
                 "GEMVs only": run(b, None)}
        assert np.array_equal(forms["default"], run(a, None)), f"{spec.name} {chunks}: repeated prefill differs"
        for name, g in forms.items():
            if chunks == [100]:
                assert np.array_equal(g, ref), f"{spec.name} {name}: a 100-token prefill left the second terms"
                continue
            d = float(np.abs(g - ref).max())
            print(f"[metrics] {spec.name} chunks {chunks} {name}: float32 last row vs second terms max |d| {d:.2e} "
                  f"({d / float(np.abs(ref).max()):.2e} of the peak)")
            assert d <= 2.5e-4 * float(np.abs(ref).max()), f"{spec.name} {chunks} {name}: max |d| {d:.3e}"
            assert int(np.argmax(g)) == int(np.argmax(ref))
    a.close()
    b.close()
    model.close()


# ------------------------------------------------------------------ prefill weight cache

LAYER_MATS = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")


def half_layers(weights: dict) -> dict:
    """The weights with every layer projection replaced by f16(d*q) (numpy)."""
    import oracle.oracle as orc
    from alpaca_amd.tensor import QTensor

    out = dict(weights)
    for name, t in weights.items():
        if name.split(".")[-1] in LAYER_MATS:
            v = orc.dequantize(t.dtype, t.data, t.rows * t.cols).astype(np.float16)
            out[name] = QTensor(F16, t.rows, t.cols, v)
    return out


@pytest.mark.parametrize("spec", [synth.TINY, synth.with_dtype(synth.TINY, Q4_0)], ids=lambda s: s.name)
def test_prefill_weight_cache_is_the_f16_model(hip_ctx, spec):
    """A model built with the prefill weight cache prefills (fast path) exactly as a
    model whose layer projections are the numpy f16 values of d*q: the cache holds
    f16(d*q) and the fast GEMMs read it.  Decode and the exact prefill do not use it."""
    w = built(spec)
    c = spec.config
    cached = HIPLlamaModel(hip_ctx, c, w, prefill_weight_cache=True)
    plain = HIPLlamaModel(hip_ctx, c, w)
    ref = HIPLlamaModel(hip_ctx, c, half_layers(w))
    per_layer = sum(w[f"blk.0.{m}"].rows * w[f"blk.0.{m}"].cols for m in LAYER_MATS)
    assert cached.prefill_cache_bytes == 2 * per_layer * c.layer_count and plain.prefill_cache_bytes == 0
    prompt = synth.prompt_tokens(spec, 100)
    a = cached.make_session(capacity=160, gemm_precision="fast").forward(prompt)
    b = ref.make_session(capacity=160, gemm_precision="fast").forward(prompt)
    assert np.array_equal(a, b)
    # past 256 rows, with the returned row's float32 GEMVs forced on (they read the cache too)
    long_prompt = synth.prompt_tokens(spec, 300)
    with env(ALPACA_HIP_LAST_ROW_GEMV=7):
        a = cached.make_session(capacity=320, gemm_precision="fast").forward(long_prompt)
        b = ref.make_session(capacity=320, gemm_precision="fast").forward(long_prompt)
    assert np.array_equal(a, b)
    # exact prefill and decode read the quantised weights
    s1, s2 = cached.make_session(capacity=160, gemm_precision="exact"), plain.make_session(capacity=160,
                                                                                          gemm_precision="exact")
    assert np.array_equal(s1.forward(prompt), s2.forward(prompt))
    for tok in (3, 17):
        assert np.array_equal(s1.decode(tok), s2.decode(tok))


def test_prefill_weight_cache_skips_f16_layers(hip_ctx):
    spec = synth.with_dtype(synth.TINY, F16)
    m = HIPLlamaModel(hip_ctx, spec.config, built(spec), prefill_weight_cache=True)
    assert m.prefill_cache_bytes == 0
