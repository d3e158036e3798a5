#!/usr/bin/env python3
"""Benchmark of the Llama forward hot path on one MI355X.

Workload (BASELINE.json metric "prefill tok/s @4096, decode tok/s @2048 ctx
(Q8_0)"): the 135M-shaped Q8_0 decoder (config C1: 30 layers, hidden 576,
9/3 heads, head_dim 64, FFN 1536, vocab 49152, tied embeddings), random-init
synthetic weights.

  * value: decode tok/s at context 2048.  A step is one greedy decode token
    through the GPU-resident chain (MetalLlamaSession.decodeGreedy semantics):
    the session is prefilled to 2048 - warmup positions, `warmup` untimed
    steps bring it to 2048, then exactly `steps` steps are timed.
  * prefill_tok_s: 4096-token prompt / wall time of forward (median of runs).
  * roofline: the dominant decode kernel (by total time), from HIP events the
    session records on its own stream around each stage in a profiled pass
    over the same decode steps; achieved = algorithmic bytes per launch /
    mean launch time, against 8 TB/s.
  * roofline_prefill: the dominant prefill GEMM, algorithmic FLOPs per launch
    / mean launch time, against 2.5 PFLOP/s dense fp16.
  * cpu_baseline: the C oracle (restatement of AlpacaCore's CPU path) on the
    host cores: decode steps at context 2048 (the oracle's cache is filled
    with synthetic rows, since prefilling 2048 positions on the CPU would take
    minutes).

Prints one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
METRIC = "prefill tok/s @4096, decode tok/s @2048 ctx (Q8_0); % of HBM/MFMA peak"
DECODE_CTX = 2048
PREFILL_TOKENS = 4096


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def q8_bytes(rows: int, cols: int) -> int:
    return rows * cols // 32 * 34


def decode_stage_bytes(c, ctx_len: float) -> dict:
    """Algorithmic HBM bytes per launch of each decode stage (one token)."""
    H, QW, KW, F, V = c.hidden_size, c.query_width, c.kv_width, c.feed_forward_size, c.vocab_size
    return {
        "qkv (fused norm)": q8_bytes(QW + 2 * KW, H) + 4 * (2 * H + QW + 2 * KW),
        "rope + kv store": 4 * (QW + 2 * KW) * 2 + 2 * 2 * KW,
        "attention": 2 * 2 * ctx_len * KW + 4 * (QW + 2 * KW) + 4 * QW,
        "attn out projection (+residual)": q8_bytes(H, QW) + 4 * (QW + 2 * H),
        "ffn gate+up+silu (fused norm)": 2 * q8_bytes(F, H) + 4 * (2 * H + F),
        "ffn down (+residual)": q8_bytes(H, F) + 4 * (F + 2 * H),
        "final norm + logits": q8_bytes(V, H) + 4 * (2 * H + V),
        "embed": H // 32 * 34 + 4 * H,
        "sample": 4 * V,
    }


def prefill_stage_flops(c, T: int) -> dict:
    H, QW, KW, F, hd, nh = c.hidden_size, c.query_width, c.kv_width, c.feed_forward_size, c.head_dim, c.head_count
    return {
        "qkv projections": 2 * T * (QW + 2 * KW) * H,
        "attn out projection (+residual)": 2 * T * H * QW,
        "ffn gate+up+silu": 2 * T * 2 * F * H,
        "ffn down (+residual)": 2 * T * H * F,
        "attention": 2 * hd * nh * T * (T + 1),  # QK^T and PV over the causal triangle
    }


def stage_table(profile: dict, units: dict, scale: float, unit: str) -> dict:
    out = {}
    for label, st in profile.items():
        avg = st.seconds / max(st.dispatches, 1)
        row = {"total_ms": round(st.seconds * 1e3, 4), "launches": st.dispatches, "avg_us": round(avg * 1e6, 3)}
        if label in units and avg > 0:
            row[f"achieved_{unit}"] = round(units[label] / avg / scale, 2)
        out[label] = row
    return out


def cpu_baseline(weights, spec, budget_s: float = 12.0) -> dict:
    import numpy as np

    import oracle.oracle as orc
    c = spec.config
    cfg = dict(vocab=c.vocab_size, hidden=c.hidden_size, layers=c.layer_count, heads=c.head_count,
               kv_heads=c.kv_head_count, head_dim=c.head_dim, ffn=c.feed_forward_size, context=c.context_length,
               eps=c.rms_norm_eps, theta=c.rope_theta, interleaved=c.rope_interleaved)
    om = orc.OracleModel(cfg, {n: (t.dtype, t.data) for n, t in weights.items()})
    threads = min(16, os.cpu_count() or 1)
    orc.set_threads(threads)
    kv = orc.OracleKV(cfg, DECODE_CTX + 64)
    kv.fill(DECODE_CTX - 1, seed=7)
    tok = 1
    steps, t0 = 0, time.perf_counter()
    while True:
        logits = orc.forward(om, kv, [tok])
        tok = int(np.argmax(logits))
        steps += 1
        el = time.perf_counter() - t0
        if (el > budget_s and steps >= 2) or steps >= 64:
            break
    return {"value": round(steps / el, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"C1 decode, {steps} greedy steps starting at ctx {DECODE_CTX} (oracle KV cache filled with "
                      f"synthetic rows), oracle threaded over 16-row chunks of each linear as AlpacaCore"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--depth", type=int, default=3, help="greedy-chain steps queued ahead (reference default 3)")
    ap.add_argument("--prefill-runs", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-profile", action="store_true")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures the single-GPU hot path only: this build runs on one GPU "
              "(sharding is described in DESIGN.md, not implemented); run with --gpus 1.", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0 or args.warmup >= DECODE_CTX:
        print("need steps >= 1 and 0 <= warmup < 2048", file=sys.stderr)
        return 2

    import numpy as np

    from alpaca_amd import synth
    from alpaca_amd.model import HIPContext, HIPLlamaModel

    spec = synth.C1
    c = spec.config
    t0 = time.perf_counter()
    weights = synth.build_weights(spec)
    log(f"synthetic C1 weights built in {time.perf_counter() - t0:.1f}s")
    ctx = HIPContext(0)
    model = HIPLlamaModel(ctx, c, weights)
    log(f"model resident: {model.weight_bytes / 1e6:.1f} MB")
    prompt = synth.prompt_tokens(spec, PREFILL_TOKENS)

    # ---------------------------------------------------------------- decode
    cap = DECODE_CTX + args.steps + 16
    s = model.make_session(capacity=cap, max_batch=PREFILL_TOKENS)
    first = int(np.argmax(s.forward(prompt[: DECODE_CTX - args.warmup])))
    toks = []
    if args.warmup:
        s.decode_greedy(first, args.warmup, lambda t: toks.append(t) or True, depth=args.depth)
        first = toks[-1]
    assert s.length == DECODE_CTX, s.length
    log(f"decode: context {s.length}, timing {args.steps} steps")
    timed = []
    t0 = time.perf_counter()
    fed = s.decode_greedy(first, args.steps, lambda t: timed.append(t) or True, depth=args.depth)
    el = time.perf_counter() - t0
    assert fed == args.steps
    decode_tok_s = args.steps / el
    log(f"decode: {decode_tok_s:.1f} tok/s ({el / args.steps * 1e3:.3f} ms/token)")

    # ---------------------------------------------------------------- prefill
    p = model.make_session(capacity=PREFILL_TOKENS, max_batch=PREFILL_TOKENS)
    p.forward(prompt)
    p.reset()
    walls, gpus = [], []
    for _ in range(max(1, args.prefill_runs)):
        t0 = time.perf_counter()
        p.forward(prompt)
        walls.append(time.perf_counter() - t0)
        gpus.append(p.last_gpu_seconds)
        p.reset()
    prefill_tok_s = PREFILL_TOKENS / float(np.median(walls))
    log(f"prefill 4096: {prefill_tok_s:.0f} tok/s (median wall {np.median(walls) * 1e3:.2f} ms, "
        f"GPU {np.median(gpus) * 1e3:.2f} ms)")

    # ---------------------------------------------------------------- stage profiles
    roof, roof_p, stages_d, stages_p = None, None, {}, {}
    if not args.no_profile:
        s2 = model.make_session(capacity=cap, max_batch=PREFILL_TOKENS)
        t2 = int(np.argmax(s2.forward(prompt[:DECODE_CTX])))
        s2.profiling_enabled = True
        s2.decode_greedy(t2, args.steps, lambda t: True, depth=args.depth)
        prof = s2.last_profile
        units = decode_stage_bytes(c, DECODE_CTX + args.steps / 2)
        stages_d = stage_table(prof, units, 1e9, "GBs")
        dom = max((k for k in prof if k in units), key=lambda k: prof[k].seconds)
        avg = prof[dom].seconds / prof[dom].dispatches
        achieved = units[dom] / avg / 1e9
        roof = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "bytes_per_launch": int(units[dom]), "avg_launch_us": round(avg * 1e6, 3)}
        p.profiling_enabled = True
        p.forward(prompt)
        profp = p.last_profile
        p.reset()
        fl = prefill_stage_flops(c, PREFILL_TOKENS)
        stages_p = stage_table(profp, fl, 1e12, "TFLOPs")
        domp = max((k for k in profp if k in fl and k != "attention"), key=lambda k: profp[k].seconds)
        avgp = profp[domp].seconds / profp[domp].dispatches
        ach = fl[domp] / avgp / 1e12
        roof_p = {"bound": "mfma", "kernel": domp, "achieved": round(ach, 2), "peak": MFMA_F16_PEAK_TFLOPS,
                  "unit": "TFLOP/s", "frac": round(ach / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None,
                  "flops_per_launch": int(fl[domp]), "avg_launch_us": round(avgp * 1e6, 3)}
        gemm_s = sum(profp[k].seconds for k in profp if k in fl and k != "attention")
        gemm_f = sum(fl[k] * profp[k].dispatches for k in profp if k in fl and k != "attention")
        roof_p["all_prefill_gemms_frac"] = round(gemm_f / gemm_s / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)
        log(f"decode dominant stage: {dom} {achieved:.0f} GB/s; prefill dominant GEMM: {domp} {ach:.1f} TFLOP/s")

    # ---------------------------------------------------------------- CPU baseline
    cpu = None
    if not args.no_cpu_baseline:
        log("CPU oracle baseline ...")
        cpu = cpu_baseline(weights, spec)
        log(f"CPU oracle: {cpu['value']} tok/s on {cpu['cores']} threads")

    line = {
        "metric": METRIC, "value": round(decode_tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(el / args.steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32 (q8_0 weights, f32 accumulate)",
        "data": "synthetic (random-init weights N(0,0.02) quantised to Q8_0, uniform random token ids)",
        "config": {"workload": "C1 135M-shape Q8_0 Llama: greedy decode at context 2048 (value); "
                               "4096-token prefill (prefill_tok_s)",
                   "layers": c.layer_count, "hidden": c.hidden_size, "heads": f"{c.head_count}/{c.kv_head_count}",
                   "head_dim": c.head_dim, "ffn": c.feed_forward_size, "vocab": c.vocab_size,
                   "kv_cache": "f16", "prefill_precision": "fast (f16 MFMA, f32 accumulate)",
                   "greedy_depth": args.depth},
        "prefill_tok_s": round(prefill_tok_s, 1),
        "decode_ms_per_token": round(el / args.steps * 1e3, 4),
        "roofline": roof, "roofline_prefill": roof_p, "cpu_baseline": cpu,
        "stages_decode": stages_d, "stages_prefill": stages_p,
        "reference_m5": {"prefill_tok_s_4096": 24069, "decode_tok_s_ctx2048": 456,
                         "note": "Apple M5, real SmolLM2-135M Q8_0 (BASELINE.md); context only"},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
