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
