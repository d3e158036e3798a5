"""The committed synthetic goldens (tests/golden/synthetic_goldens.json,
written by tests/golden/make_synthetic_goldens.py) against this tree.

CPU side: the seeded inputs still hash to the recorded SHA-256 (so the GPU
tests compare like with like), and the oracle reproduces its recorded C1 and
C2 outputs bit for bit (it is deterministic at any thread count).
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle.oracle as orc
from alpaca_amd import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "synthetic_goldens.json")


def golden() -> dict:
    with open(GOLDEN) as f:
        return json.load(f)


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).view(np.uint8).tobytes())
    return h.hexdigest()


def oracle_cfg(c) -> dict:
    return dict(vocab=c.vocab_size, hidden=c.hidden_size, layers=c.layer_count, heads=c.head_count,
                kv_heads=c.kv_head_count, head_dim=c.head_dim, ffn=c.feed_forward_size, context=c.context_length,
                eps=c.rms_norm_eps, theta=c.rope_theta, interleaved=c.rope_interleaved)


@pytest.mark.parametrize("key,spec", [("C1", synth.C1), ("C4", synth.C4)])
def test_model_inputs_match_golden_hashes(key, spec):
    g = golden()["models"][key]
    w = synth.build_weights(spec)
    assert sha(*[w[n].data for n in synth.tensor_names(spec)]) == g["weights_sha256"]
    assert sha(synth.prompt_tokens(spec, g["prompt_len"]).astype(np.int32)) == g["prompt_sha256"]


def test_isolated_inputs_match_golden_hashes():
    g = golden()
    for case in g["c2"]:
        x, w = synth.c2_gemm_case(case["n"], case["k"])
        assert sha(x) == case["x_sha256"] and sha(w.data) == case["w_sha256"]
    q, k, v = synth.c3_attention_case()
    assert (sha(q), sha(k), sha(v)) == (g["c3"]["q_sha256"], g["c3"]["k_sha256"], g["c3"]["v_sha256"])


def test_oracle_reproduces_c1_golden():
    g = golden()["models"]["C1"]
    spec, c = synth.C1, synth.C1.config
    w = synth.build_weights(spec)
    om = orc.OracleModel(oracle_cfg(c), {n: (t.dtype, t.data) for n, t in w.items()})
    kv = orc.OracleKV(oracle_cfg(c), g["prompt_len"] + 4, rounds_f16=True)
    logits = orc.forward(om, kv, synth.prompt_tokens(spec, g["prompt_len"]))
    assert logits[:16].tolist() == g["prefill_logits_head"]
    assert logits[-16:].tolist() == g["prefill_logits_tail"]
    ids = [orc.argmax(logits)]
    for _ in range(3):
        ids.append(orc.argmax(orc.forward(om, kv, [ids[-1]])))
    assert ids == g["greedy_ids"][:4]


def test_oracle_reproduces_c2_golden():
    for case in golden()["c2"]:
        x, w = synth.c2_gemm_case(case["n"], case["k"])
        assert sha(orc.linear(x, w.dtype, w.data, case["n"])) == case["y_sha256"]


WORKLOADS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "workload_goldens.npz")


@pytest.mark.parametrize("key,spec,base", [("C1L", synth.C1, "C1"), ("C4W", synth.C4, "C4"), ("C5W", synth.C5, "C5")])
def test_workload_goldens_describe_the_benched_inputs(key, spec, base):
    """workload_goldens.npz (make_synthetic_goldens.py --workloads): the same
    weights as the model goldens of the config, the bench's prompt (the
    config's prompt stream, cut at the recorded length), one greedy id and
    top-2 margin per step and full 49,152-logit rows for the prefill, steps
    1-8 and the last step."""
    import json
    with np.load(WORKLOADS) as z:
        if key + "_meta" not in z.files:
            pytest.skip(f"{key} not computed")
        meta = json.loads(str(z[key + "_meta"]))
        ids, margins, steps, logits = (z[key + s] for s in ("_ids", "_margins", "_logit_steps", "_logits"))
    n, g = meta["prompt_len"], meta["greedy_steps"]
    assert meta["weights_sha256"] == golden()["models"][base]["weights_sha256"]
    assert sha(synth.prompt_tokens(spec, n).astype(np.int32)) == meta["prompt_sha256"]
    assert ids.shape == (g + 1,) and margins.shape == (g + 1,) and (margins >= 0).all()
    assert steps.tolist() == [0] + list(range(1, 9)) + [g]
    assert logits.shape == (len(steps), spec.config.vocab_size) and logits.dtype == np.float32
    assert np.isfinite(logits).all()
    # each kept row's arg-max is the recorded greedy id of its step
    assert [int(np.argmax(r)) for r in logits] == [int(ids[s]) for s in steps]
