"""Writes synthetic_goldens.json: the CPU oracle's results on the seeded
synthetic workloads of the benchmark configurations.

    python tests/golden/make_synthetic_goldens.py [--threads N]

The oracle (oracle/, a C restatement of AlpacaCore's CPU path) is pinned to
the reference's own fixtures by tests/test_oracle_*.py; this file freezes its
outputs on larger inputs so GPU runs can be checked without re-running it:

  * C1 (135M-shape Q8_0, seed 0): 128-token prompt, then 16 greedy steps.
  * C4 (360M-shape Q4_0, seed 3): a 2048-token prompt, then 16 greedy steps.
  * C5 (1.7B-shape Q8_0, seed 4), shortened so the CPU oracle finishes in
    minutes: a 256-token prompt, then 8 greedy steps.
  * C2 (seed 1): the two isolated Q8_0 GEMMs, M = 2048.
  * C3 (seed 2): causal GQA attention over T = 4096 after RoPE, and the
    decode query at position 2047 over the L = 2048 visible cache rows.

With --workloads it writes workload_goldens.npz instead: the model workloads
exactly as bench.py times them, with full logit vectors (float32):

  * C1L: C1 decode at context 2048: a 2045-token prompt, then 131 greedy
    steps (3 that bring the context to 2048, then 128 timed ones);
  * C4W: C4's 2048-token prompt, then 256 greedy steps (context 2048-2303);
  * C5W: C5's 4096-token prompt, then 256 greedy steps (context 4096-4351);
  * C1P: C1's 4096-token prompt (the benched prefill, split over two streams
    on the GPU), then 8 greedy steps.

Per case: the greedy ids and top-2 margins of every step, and the full
logits of the prefill (step 0) and of greedy steps 1-8 and the last one.
The C5W prefill takes the oracle about half an hour on 8 cores.

Model cases use an f16-rounded KV cache (the GPU default).  Recorded: SHA-256
of the inputs (weights in GGUF block bytes, prompt ids), first and last 16
logits of the prefill and of the last greedy step, the greedy ids and each
step's top-2 margin; for the isolated cases the SHA-256 of the float32 output
and a strided sample of it.
"""
import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle.oracle as orc  # noqa: E402
from alpaca_amd import synth  # noqa: E402

MODEL_CASES = [("C1", synth.C1, 128, 16), ("C4", synth.C4, 2048, 16), ("C5", synth.C5, 256, 8)]
SAMPLE_STRIDE = 997


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).view(np.uint8).tobytes())
    return h.hexdigest()


def weights_sha(spec, w) -> str:
    return sha(*[w[name].data for name in synth.tensor_names(spec)])


def top2(logits) -> float:
    s = np.sort(logits.astype(np.float64))
    return float(s[-1] - s[-2])


def oracle_cfg(c) -> dict:
    return dict(vocab=c.vocab_size, hidden=c.hidden_size, layers=c.layer_count, heads=c.head_count,
                kv_heads=c.kv_head_count, head_dim=c.head_dim, ffn=c.feed_forward_size, context=c.context_length,
                eps=c.rms_norm_eps, theta=c.rope_theta, interleaved=c.rope_interleaved)


def model_case(spec, n_prompt, n_greedy) -> dict:
    c = spec.config
    w = synth.build_weights(spec)
    om = orc.OracleModel(oracle_cfg(c), {n: (t.dtype, t.data) for n, t in w.items()})
    prompt = synth.prompt_tokens(spec, n_prompt)
    kv = orc.OracleKV(oracle_cfg(c), n_prompt + n_greedy + 1, rounds_f16=True)
    logits = orc.forward(om, kv, prompt)
    out = {"spec": spec.name, "seed": spec.seed, "prompt_len": n_prompt, "greedy_steps": n_greedy,
           "kv": "f16-rounded", "weights_sha256": weights_sha(spec, w), "prompt_sha256": sha(prompt.astype(np.int32)),
           "prefill_logits_head": logits[:16].tolist(), "prefill_logits_tail": logits[-16:].tolist(),
           "prefill_logits_peak": float(np.abs(logits).max())}
    ids, margins = [int(orc.argmax(logits))], [top2(logits)]
    for _ in range(n_greedy - 1):
        logits = orc.forward(om, kv, [ids[-1]])
        ids.append(int(orc.argmax(logits)))
        margins.append(top2(logits))
    out.update({"greedy_ids": ids, "greedy_top2_margins": margins,
                "last_step_logits_head": logits[:16].tolist(), "last_step_logits_tail": logits[-16:].tolist()})
    return out


def sample(a) -> list:
    return a.ravel()[::SAMPLE_STRIDE].astype(np.float64).tolist()


def c2_cases() -> list:
    out = []
    for n, k in [(1536, 576), (576, 1536)]:
        x, w = synth.c2_gemm_case(n, k)
        y = orc.linear(x, w.dtype, w.data, n)
        out.append({"n": n, "k": k, "m": x.shape[0], "x_sha256": sha(x), "w_sha256": sha(w.data),
                    "y_sha256": sha(y), "y_sample_stride": SAMPLE_STRIDE, "y_sample": sample(y)})
    return out


def c3_case() -> dict:
    q, k, v = synth.c3_attention_case()
    theta = 1e5
    qr = orc.rope(q.astype(np.float32), 0, theta, True)
    kr = orc.rope(k.astype(np.float32), 0, theta, True)
    k16 = kr.astype(np.float16).astype(np.float32)  # the cache holds f16 rows
    v32 = v.astype(np.float32)
    o = orc.attention(qr, k16, v32, 0)
    # decode: the query of position 2047 over rows 0..2047 (L = 2048 visible) of the same cache
    od = orc.attention(qr[2047:2048], k16[:2048], v32[:2048], 2047)
    return {"tokens": q.shape[0], "heads": q.shape[1], "kv_heads": k.shape[1], "head_dim": q.shape[2],
            "theta": theta, "q_sha256": sha(q), "k_sha256": sha(k), "v_sha256": sha(v),
            "out_sample_stride": SAMPLE_STRIDE, "out_sample": sample(o),
            "decode_position": 2047, "decode_visible_rows": 2048,
            "decode_out": od.ravel().astype(np.float64).tolist()}


# (key, spec, prompt length, greedy steps): the decode workloads bench.py times
WORKLOAD_CASES = [("C1L", synth.C1, 2045, 131), ("C4W", synth.C4, 2048, 256), ("C5W", synth.C5, 4096, 256),
                  ("C1P", synth.C1, 4096, 8)]
FULL_LOGIT_STEPS = 8  # greedy steps 1..8 (and the last) keep their full logits


def workload_case(key, spec, n_prompt, n_greedy, log) -> dict:
    c = spec.config
    t0 = time.time()
    w = synth.build_weights(spec)
    om = orc.OracleModel(oracle_cfg(c), {n: (t.dtype, t.data) for n, t in w.items()})
    prompt = synth.prompt_tokens(spec, n_prompt)
    kv = orc.OracleKV(oracle_cfg(c), n_prompt + n_greedy + 1, rounds_f16=True)
    logits = orc.forward(om, kv, prompt)
    log(f"{key}: prefill of {n_prompt} tokens in {time.time() - t0:.0f} s")
    keep_steps = [0] + list(range(1, FULL_LOGIT_STEPS + 1)) + [n_greedy]
    kept = {0: logits.astype(np.float32)}
    ids, margins = [int(orc.argmax(logits))], [top2(logits)]
    # step i (1-based) feeds greedy id i-1 at position n_prompt + i - 1
    for i in range(1, n_greedy + 1):
        logits = orc.forward(om, kv, [ids[-1]])
        if i in keep_steps:
            kept[i] = logits.astype(np.float32)
        ids.append(int(orc.argmax(logits)))
        margins.append(top2(logits))
        if i % 32 == 0:
            log(f"{key}: {i} greedy steps, {time.time() - t0:.0f} s")
    # ids[k] / margins[k] (k = 0..n_greedy): arg-max and top-2 margin of step
    # k's logits (step 0 = the prefill); decode_greedy(ids[0], n_greedy) emits
    # ids[1..n_greedy]
    steps = sorted(kept)
    return {f"{key}_ids": np.asarray(ids, np.int32), f"{key}_margins": np.asarray(margins, np.float64),
            f"{key}_logit_steps": np.asarray(steps, np.int32),
            f"{key}_logits": np.stack([kept[i] for i in steps]).astype(np.float32),
            f"{key}_meta": np.array(json.dumps({
                "spec": spec.name, "seed": spec.seed, "prompt_len": n_prompt, "greedy_steps": n_greedy,
                "kv": "f16-rounded", "weights_sha256": weights_sha(spec, w),
                "prompt_sha256": sha(prompt.astype(np.int32))}))}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    ap.add_argument("--out", default=None)
    ap.add_argument("--workloads", action="store_true", help="write workload_goldens.npz (long)")
    ap.add_argument("--cases", default=",".join(k for k, *_ in WORKLOAD_CASES),
                    help="workload cases to compute (with --workloads)")
    a = ap.parse_args()
    orc.build()
    orc.set_threads(a.threads)

    def log(msg):
        print(msg, flush=True)

    if a.workloads:
        out = a.out or os.path.join(HERE, "workload_goldens.npz")
        arrays = {}
        if os.path.exists(out):  # keep cases computed earlier
            with np.load(out) as z:
                arrays = {k: z[k] for k in z.files}
        for key, spec, n_prompt, n_greedy in WORKLOAD_CASES:
            if key not in a.cases.split(","):
                continue
            arrays.update(workload_case(key, spec, n_prompt, n_greedy, log))
            np.savez_compressed(out, **arrays)
            log(f"{key}: greedy {arrays[key + '_ids'][:12].tolist()}..., wrote {out}")
        return
    a.out = a.out or os.path.join(HERE, "synthetic_goldens.json")
    res = {"generator": "tests/golden/make_synthetic_goldens.py", "oracle": "oracle/alpaca_oracle.c", "models": {}}
    for key, spec, n_prompt, n_greedy in MODEL_CASES:
        t0 = time.time()
        res["models"][key] = model_case(spec, n_prompt, n_greedy)
        print(f"{key}: {time.time() - t0:.1f} s, greedy {res['models'][key]['greedy_ids']}", flush=True)
    t0 = time.time()
    res["c2"] = c2_cases()
    print(f"C2: {time.time() - t0:.1f} s", flush=True)
    t0 = time.time()
    res["c3"] = c3_case()
    print(f"C3: {time.time() - t0:.1f} s", flush=True)
    with open(a.out, "w") as f:
        json.dump(res, f, indent=1)
    print(f"wrote {a.out}")


if __name__ == "__main__":
    main()
