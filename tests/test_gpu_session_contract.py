"""The session threading contract of MetalLlamaSession
(Sources/AlpacaMetal/Backend/MetalLlamaModel.swift) through the C ABI:

  * a second call on a session that is already executing fails with BUSY
    (:235 for decodeGreedy, :275 for forward) and changes nothing; the call in
    progress finishes normally;
  * distinct sessions of one model may run at the same time, each on its own
    stream (:170-172, :214-215), and give the results they give alone
    (Tests/AlpacaIntegrationTests/PublicAPITests.swift:87-99).  Their
    persistent decode launches are ordered on the device (each needs every
    CU), so concurrent greedy chains interleave launch by launch.
"""
import threading

import numpy as np
import pytest

from alpaca_amd import synth
from alpaca_amd._lib import Busy
from alpaca_amd.model import HIPLlamaModel
from tests.test_gpu_model import built

pytestmark = pytest.mark.gpu


def test_reentrant_calls_from_emit_are_busy(hip_ctx):
    spec = synth.TINY
    model = HIPLlamaModel(hip_ctx, spec.config, built(spec))
    prompt = synth.prompt_tokens(spec, 24)
    s = model.make_session(capacity=128)
    first = int(np.argmax(s.forward(prompt)))
    seen, refused = [], []

    def emit(tok):
        seen.append(tok)
        if len(seen) == 3:
            for name, call in (("forward", lambda: s.forward([tok])), ("decode", lambda: s.decode(tok)),
                               ("decode_greedy", lambda: s.decode_greedy(tok, 2, lambda t: True)),
                               ("reset", s.reset), ("sample", lambda: s.sample(0.7, 40, 0.9, 0.5))):
                with pytest.raises(Busy):
                    call()
                refused.append(name)
        return True

    fed = s.decode_greedy(first, 10, emit)
    assert refused == ["forward", "decode", "decode_greedy", "reset", "sample"]
    assert fed == 10 and s.length == 34 and len(seen) == 10
    # the chain was not disturbed: the same tokens as an undisturbed session
    t = model.make_session(capacity=128)
    t.forward(prompt)
    want = []
    t.decode_greedy(first, 10, lambda x: want.append(x) or True)
    assert seen == want


@pytest.mark.parametrize("persistent", [1, 0], ids=["persistent", "multi-kernel"])
def test_concurrent_sessions_equal_their_solo_runs(hip_ctx, persistent):
    from tests.helpers import env
    spec = synth.TINY
    model = HIPLlamaModel(hip_ctx, spec.config, built(spec))
    prompts = [synth.prompt_tokens(spec, 40 + 17 * i)[::-1].copy() for i in range(3)]

    def run(session, prompt, out):
        logits = session.forward(prompt)
        toks = []
        session.decode_greedy(int(np.argmax(logits)), 60, lambda t: toks.append(t) or True)
        out.append((logits, toks, session.decode(toks[-1])))

    with env(ALPACA_HIP_PERSISTENT_DECODE=persistent):
        solo = []
        for p in prompts:
            run(model.make_session(capacity=160), p, solo)
        sessions = [model.make_session(capacity=160) for _ in prompts]
    outs = [[] for _ in prompts]
    errs = []

    def worker(i):
        try:
            run(sessions[i], prompts[i], outs[i])
        except BaseException as e:  # noqa: BLE001 - reported below
            errs.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(prompts))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errs, errs
    for i, ((l0, t0, d0), got) in enumerate(zip(solo, outs)):
        l1, t1, d1 = got[0]
        assert np.array_equal(l0, l1), f"session {i}: prefill logits differ"
        assert t0 == t1, f"session {i}: greedy tokens differ"
        assert np.array_equal(d0, d1), f"session {i}: decode logits differ"


def test_model_outlives_its_sessions(hip_ctx):
    """A model destroyed while a session still uses it stays alive until that
    session is destroyed (MetalLlamaSession keeps its MetalLlamaModel), and no
    HIP error from the teardown leaks into later calls."""
    spec = synth.TINY
    model = HIPLlamaModel(hip_ctx, spec.config, built(spec))
    prompt = synth.prompt_tokens(spec, 20)
    s = model.make_session(capacity=64)
    want = s.forward(prompt)
    s.reset()
    model.close()  # the session still holds the model
    assert np.array_equal(s.forward(prompt), want)
    s.close()      # the model goes with it
    other = HIPLlamaModel(hip_ctx, spec.config, built(spec))
    t = other.make_session(capacity=64)
    assert np.array_equal(t.forward(prompt), want)
