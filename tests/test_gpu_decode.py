"""The persistent single-token decode kernel (one launch per token).

Sessions pick it for single-token forward calls and the greedy chain when the
model allows it; ALPACA_HIP_PERSISTENT_DECODE=0 (read at session creation)
selects the multi-kernel path instead.  These tests hold the persistent path
to the multi-kernel path and to the CPU oracle
(LlamaCPUModel.forward, LlamaCPUModel.swift:24-61) and check the greedy chain
semantics of MetalLlamaSession.decodeGreedy (MetalLlamaModel.swift:228-270).

Tolerances: against the oracle, the BASELINE bound (2e-3 absolute + 1e-3
relative), after an exact-mode prefill (float32 GEMMs) so that the bound
measures the decode step; between the two GPU paths, which compute the same float32
products in a different summation order, 1e-4 of the logit peak.
"""
from dataclasses import replace

import numpy as np
import pytest

import oracle.oracle as orc
from alpaca_amd import synth
from alpaca_amd._lib import HIPError
from alpaca_amd.model import HIPLlamaModel
from alpaca_amd.tensor import F16, Q4_0
from tests.helpers import assert_close, env, metrics
from tests.test_gpu_model import built, oracle_cfg, oracle_model

pytestmark = pytest.mark.gpu


def shaped(name, **kw):
    return replace(synth.TINY, config=replace(synth.TINY.config, **kw), name=name)


# query heads per KV head 1, 2, 4 and 8 at head dim 64; 2 and 4 at head dim 128
HD128_G4 = shaped("tiny-hd128-g4", head_count=4, kv_head_count=1, head_dim=128)
SPECS = [synth.TINY, synth.with_dtype(synth.TINY, Q4_0), synth.with_dtype(synth.TINY, F16),
         shaped("tiny-g4", head_count=8, kv_head_count=2), shaped("tiny-mha", head_count=4, kv_head_count=4),
         shaped("tiny-g8", head_count=8, kv_head_count=1),
         shaped("tiny-hd128-g2", head_count=2, kv_head_count=1, head_dim=128), HD128_G4]


@pytest.mark.parametrize("spec", SPECS, ids=lambda s: s.name)
def test_persistent_decode_matches_multi_kernel_and_oracle(hip_ctx, spec):
    c = spec.config
    w = built(spec)
    model = HIPLlamaModel(hip_ctx, c, w)
    om = oracle_model(c, w)
    prompt = synth.prompt_tokens(spec, 37)
    # exact prefill (float32 GEMMs) so the oracle comparison isolates the decode step
    with env(ALPACA_HIP_PERSISTENT_DECODE=0):
        ref = model.make_session(capacity=160, gemm_precision="exact")
    fast = model.make_session(capacity=160, gemm_precision="exact")
    okv = orc.OracleKV(oracle_cfg(c), 160, rounds_f16=True)
    e = orc.forward(om, okv, prompt)
    ref.forward(prompt)
    fast.forward(prompt)
    tok = orc.argmax(e)
    for step in range(12):
        g_ref = ref.decode(tok)
        g = fast.decode(tok)
        e = orc.forward(om, okv, [tok])
        m = metrics(g, g_ref)
        print(f"[metrics] {spec.name} step {step} persistent vs multi-kernel: {m}")
        assert m["max_rel_peak"] <= 1e-4, step
        assert_close(g, e, 2e-3, 1e-3, f"{spec.name} persistent decode step {step}")
        assert int(np.argmax(g)) == int(np.argmax(e))
        tok = orc.argmax(e)
    assert fast.length == ref.length == 37 + 12


# C4's layer shape (hidden 960, FFN 2560, 15 query / 5 KV heads, Q4_0) with 2 layers.
C4_SHAPE = replace(synth.C4, config=replace(synth.C4.config, layer_count=2, vocab_size=2048, context_length=512),
                   name="c4-shape-2l")


@pytest.mark.parametrize("wgs", [128, 200, 256, 512])
def test_persistent_decode_row_shares_at_c4_shape(hip_ctx, wgs):
    """Grids whose row shares make the waves of a workgroup end a phase at
    different times: at 128 workgroups each takes 20 gate/up rows, so wave 0
    runs a second pass alone while the other waves already wait for the down
    input; at 256, wave 3 has no gate/up rows at all.  The next phase's wait
    must not overwrite the LDS input row under the waves still reading it
    (that race moved logits by up to 15% of their peak, varying run to run).
    The persistent path is held to the multi-kernel path, step by step."""
    spec = C4_SHAPE
    model = HIPLlamaModel(hip_ctx, spec.config, built(spec))
    prompt = synth.prompt_tokens(spec, 300)
    with env(ALPACA_HIP_PERSISTENT_DECODE=0):
        ref = model.make_session(capacity=320, gemm_precision="exact")
    with env(ALPACA_HIP_DECODE_WGS=wgs):
        fast = model.make_session(capacity=320, gemm_precision="exact")
    ref.forward(prompt)
    fast.forward(prompt)
    worst = 0.0
    for step in range(10):
        tok = int(prompt[step])
        m = metrics(fast.decode(tok), ref.decode(tok))
        worst = max(worst, m["max_rel_peak"])
    print(f"[metrics] {spec.name} {wgs} workgroups: worst persistent vs multi-kernel peak-rel {worst:.2e}")
    assert worst <= 1e-4


@pytest.mark.parametrize("spec", [synth.TINY, HD128_G4], ids=lambda s: s.name)
def test_persistent_decode_across_attention_split_boundaries(hip_ctx, spec):
    """Contexts on both sides of every split length (64..256 positions per
    split) and of the capacity: the split-K partials and their merge must
    cover exactly positions 0..pos."""
    c = spec.config
    w = built(spec)
    model = HIPLlamaModel(hip_ctx, c, w)
    om = oracle_model(c, w)
    cap = c.context_length  # 1024
    prompt = synth.prompt_tokens(spec, cap)
    s = model.make_session(capacity=cap, max_batch=512, gemm_precision="exact")
    okv = orc.OracleKV(oracle_cfg(c), cap, rounds_f16=True)
    for p in (1, 63, 64, 65, 127, 128, 129, 255, 256, 257, 511, 640, 1023, cap):
        s.reset()
        okv.reset()
        if p > 1:
            s.forward(prompt[: p - 1])
            orc.forward(om, okv, prompt[: p - 1])
        g = s.decode(int(prompt[p - 1]))
        e = orc.forward(om, okv, [int(prompt[p - 1])])
        assert_close(g, e, 2e-3, 1e-3, f"decode at context {p}")
        assert s.length == p


def test_persistent_greedy_chain_matches_stepwise_decode(hip_ctx):
    """decodeGreedy through the persistent kernel emits the tokens that
    step-by-step decode + host arg-max produce, stops early when emit returns
    False (length = tokens fed) and stops at capacity."""
    spec = synth.TINY
    c = spec.config
    model = HIPLlamaModel(hip_ctx, c, built(spec))
    prompt = synth.prompt_tokens(spec, 30)
    a = model.make_session(capacity=100)
    first = int(np.argmax(a.forward(prompt)))
    got = []
    fed = a.decode_greedy(first, 50, lambda t: got.append(t) or True, depth=4)
    assert fed == 50 and a.length == 80
    b = model.make_session(capacity=100)
    tok = int(np.argmax(b.forward(prompt)))
    want = []
    for _ in range(50):
        tok = int(np.argmax(b.decode(tok)))
        want.append(tok)
    assert got == want
    # early stop after 5 tokens: 5 fed
    cs = model.make_session(capacity=100)
    cs.forward(prompt)
    seen = []
    fed = cs.decode_greedy(first, 50, lambda t: seen.append(t) or len(seen) < 5, depth=3)
    assert fed == 5 and cs.length == 35 and seen == want[:5]
    # capacity: 100 - 30 = 70 steps at most
    d = model.make_session(capacity=100)
    d.forward(prompt)
    fed = d.decode_greedy(first, 500, lambda t: True, depth=2)
    assert fed == 70 and d.length == 100


def test_cooperative_launch_mode_matches_default(hip_ctx):
    """ALPACA_HIP_DECODE_COOPERATIVE=1 (read at session creation) launches the
    same kernel with hipLaunchCooperativeKernel instead of an ordinary launch:
    single-token logits and greedy tokens are bit-identical to the default."""
    spec = synth.TINY
    model = HIPLlamaModel(hip_ctx, spec.config, built(spec))
    prompt = synth.prompt_tokens(spec, 30)
    with env(ALPACA_HIP_DECODE_COOPERATIVE=1):
        coop = model.make_session(capacity=100)
    plain = model.make_session(capacity=100)
    firsts = [int(np.argmax(s.forward(prompt))) for s in (coop, plain)]
    assert firsts[0] == firsts[1]
    la, lb = coop.decode(firsts[0]), plain.decode(firsts[0])
    assert np.array_equal(la, lb)
    ta, tb = [], []
    coop.decode_greedy(int(np.argmax(la)), 24, lambda t: ta.append(t) or True)
    plain.decode_greedy(int(np.argmax(lb)), 24, lambda t: tb.append(t) or True)
    assert ta == tb and len(ta) == 24


def test_persistent_decode_abort_is_reported_and_session_recovers(hip_ctx):
    """A launch that aborts (a wait timed out, or a workgroup gave up) makes every
    workgroup leave through the shared abort word.  Forced from the host
    (ALPACA_HIP_DECODE_ABORT_LAYER: workgroup 0 raises the abort at layer 1 and
    stops, so the others wait for rows it never publishes), the call fails
    without advancing the session, the greedy chain reports it too, and the
    exchange words are reset so that later launches succeed."""
    spec = synth.TINY
    c = spec.config
    model = HIPLlamaModel(hip_ctx, c, built(spec))
    prompt = synth.prompt_tokens(spec, 20)
    with env(ALPACA_HIP_DECODE_ABORT_LAYER=1):
        s = model.make_session(capacity=64)
    s.forward(prompt)
    for _ in range(2):
        with pytest.raises(HIPError, match="aborted"):
            s.decode(7)
        assert s.length == 20
    with pytest.raises(HIPError, match="aborted"):
        s.decode_greedy(7, 5, lambda t: True)
    assert s.length == 20
    ok = model.make_session(capacity=64)
    ok.forward(prompt)
    with env(ALPACA_HIP_PERSISTENT_DECODE=0):
        ref = model.make_session(capacity=64)
    ref.forward(prompt)
    m = metrics(ok.decode(7), ref.decode(7))
    assert m["max_rel_peak"] <= 1e-4


@pytest.mark.parametrize("spec", [synth.TINY, HD128_G4], ids=lambda s: s.name)
def test_persistent_decode_multi_item_attention(hip_ctx, spec):
    """More attention items than workgroups: each workgroup runs the item loop
    of the attention phase several times, loading the next item's K rows into
    registers and DMAing its V rows into the LDS buffer the current item has
    just finished with.  Small grids (ALPACA_HIP_DECODE_WGS 4, 8, 16) and
    item targets (ALPACA_HIP_DECODE_ITEMS 8, 24, 96) give 1-8 items per
    workgroup with splits of 64, 128 and 256 positions; contexts sit on both
    sides of those split lengths, including splits that hold only the current
    position.  Each decode is held to the oracle (2e-3 + 1e-3) and to the
    multi-kernel path (1e-4 of the logit peak).  Reference: the split-boundary
    sweep of KernelTests.swift:123-144."""
    c = spec.config
    w = built(spec)
    model = HIPLlamaModel(hip_ctx, c, w)
    om = oracle_model(c, w)
    cap = c.context_length  # 1024
    prompt = synth.prompt_tokens(spec, cap)
    contexts = (1, 65, 128, 129, 256, 257, 385, 512, 513, 769, 1023, cap)
    with env(ALPACA_HIP_PERSISTENT_DECODE=0):
        ref = model.make_session(capacity=cap, max_batch=512, gemm_precision="exact")
    okv = orc.OracleKV(oracle_cfg(c), cap, rounds_f16=True)
    want = {}
    for p in contexts:
        ref.reset()
        okv.reset()
        if p > 1:
            ref.forward(prompt[: p - 1])
            orc.forward(om, okv, prompt[: p - 1])
        want[p] = (ref.decode(int(prompt[p - 1])), orc.forward(om, okv, [int(prompt[p - 1])]))
    ref.close()
    worst = 0.0
    for wgs in (4, 8, 16):
        for items in (8, 24, 96):
            with env(ALPACA_HIP_DECODE_WGS=wgs, ALPACA_HIP_DECODE_ITEMS=items):
                s = model.make_session(capacity=cap, max_batch=512, gemm_precision="exact")
            for p in contexts:
                s.reset()
                if p > 1:
                    s.forward(prompt[: p - 1])
                g = s.decode(int(prompt[p - 1]))
                r, e = want[p]
                m = metrics(g, r)
                worst = max(worst, m["max_rel_peak"])
                assert m["max_rel_peak"] <= 1e-4, (wgs, items, p, m)
                assert_close(g, e, 2e-3, 1e-3, f"{spec.name} wgs {wgs} items {items} context {p}")
                assert s.length == p
            s.close()
    print(f"[metrics] {spec.name} multi-item attention: worst persistent vs multi-kernel peak-rel {worst:.2e}")


# Output rows per workgroup: a tiny layer shape with a 12,000-entry vocabulary
# (48 rows per workgroup at 256 workgroups), and C1's 49,152-entry vocabulary
# over two C1 layers (192 rows per workgroup, more than LDS can stage).
BIG_VOCAB = [shaped("tiny-v12k", vocab_size=12000),
             synth.with_dtype(shaped("tiny-v12k-q4", vocab_size=12000), Q4_0),
             synth.with_dtype(shaped("tiny-v12k-f16", vocab_size=12000), F16),
             replace(synth.C1, config=replace(synth.C1.config, layer_count=2, context_length=512), name="c1-2l")]


@pytest.mark.parametrize("spec", BIG_VOCAB, ids=lambda s: s.name)
def test_persistent_decode_staged_logit_rows(hip_ctx, spec):
    """The logits phase stages the leading rows of each workgroup's output
    share in LDS by DMA (ALPACA_HIP_DECODE_LOGIT_STAGE_ROWS, read at session
    creation, caps how many) and streams the rest through registers.  Both
    paths form a row's sum with the same lane mapping, chunk order and lane
    reduction, so the logits and greedy ids must be bit-identical whatever the
    split: none staged, one, an odd count, as many as fit (a cap above the
    share), and the default (as many as fit where that is at least half the
    share, else none)."""
    c = spec.config
    model = HIPLlamaModel(hip_ctx, c, built(spec))
    prompt = synth.prompt_tokens(spec, 29)
    runs = {}
    for cap in ("0", "1", "7", "100000", None):
        with env(ALPACA_HIP_DECODE_LOGIT_STAGE_ROWS=cap):
            s = model.make_session(capacity=96)
        tok = int(np.argmax(s.forward(prompt)))
        out = []
        for _ in range(3):
            g = s.decode(tok)
            out.append(g)
            tok = int(np.argmax(g))
        chain = []
        s.decode_greedy(tok, 6, lambda t: chain.append(t) or True)
        runs[cap] = (out, chain)
        s.close()
    ref_out, ref_chain = runs["0"]
    for cap, (out, chain) in runs.items():
        for step, (a, b) in enumerate(zip(out, ref_out)):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), \
                f"{spec.name} stage rows {cap}: step {step} logits differ (max |d| {np.abs(a - b).max():.3e})"
        assert chain == ref_chain, f"{spec.name} stage rows {cap}: greedy {chain} != {ref_chain}"
    model.close()
