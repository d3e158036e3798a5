#!/usr/bin/env python3
"""Benchmark of the Llama forward hot path on one MI355X.

Workload (BASELINE.json metric "prefill tok/s @4096, decode tok/s @2048 ctx
(Q8_0); % of HBM/MFMA peak"): the 135M-shaped Q8_0 decoder (config C1: 30
layers, hidden 576, 9/3 heads, head_dim 64, FFN 1536, vocab 49152, tied
embeddings), random-init synthetic weights, all resident in HBM.

  * value: decode tok/s at context 2048.  A step is one greedy decode token
    through the GPU-resident chain (MetalLlamaSession.decodeGreedy semantics,
    MetalLlamaModel.swift:228-270): the session is prefilled to
    2048 - warmup positions, `warmup` untimed steps bring it to 2048, then
    exactly `steps` steps are timed by the wall clock around decode_greedy.
    Each step is one launch of the persistent decode kernel.
  * roofline (decode): that kernel.  Algorithmic bytes per launch = bytes one
    token must move (every projection in Q8_0 at 34 B per 32 weights, the tied
    output matrix, the norm gains, the f16 KV rows read at the mean timed
    context and the row written), divided by the mean launch duration measured
    with HIP events the session records on its own stream around the timed
    steps; peak 8 TB/s.
  * prefill_tok_s: 4096-token prompt / median wall time of forward.
  * roofline_prefill: the dominant prefill GEMM (MFMA, f16 operands, f32
    accumulate): algorithmic FLOPs per launch / mean launch time from the
    session's per-stage HIP events; peak 2.5 PFLOP/s dense fp16.  issued_frac
    counts the MFMA work issued: the QKV GEMM takes its activations as two f16
    terms on every row (twice the multiply-adds), the other GEMMs on the
    prompt's last 256 rows only.
  * prefill_mfma_frac: the whole 4096-token prefill (projections + causal
    attention, algorithmic FLOPs) over its wall time, against the same peak.
  * prefill_weight_cache: the same prefill on a model created with the
    prefill weight cache (MetalLlamaModel.buildPrefillCache, f16 copies of the
    layer projections, as `--prefill-cache` in the reference CLI): tok/s and
    the gate+up GEMM's rate.  Reported beside prefill_tok_s, not instead of it.
  * other_configs: decode and prefill of configs C4 (360M-shape Q4_0, decode
    at context 2048) and C5 (1.7B-shape Q8_0, decode at 4096, 4096-token
    prefill) with their fractions of the HBM and MFMA rooflines; reported
    beside the C1 value, not instead of it.
  * cpu_baseline: the C oracle (restatement of AlpacaCore's CPU path, threaded
    over 16-row chunks of each linear as CPUOps does with concurrentPerform) on
    every host core this process may run on (capped by OMP_NUM_THREADS when
    set: the GPU box's CPU share): `value` is decode tok/s at context 2048 (the
    oracle's cache is filled with synthetic rows, since prefilling 2048
    positions on the CPU would take minutes), beside the reference's own
    CPU-runnable case (a 128-token prompt, then 16
    greedy tokens) as prefill and decode tok/s; nproc and the CPU model are
    recorded.
  * kernels: isolated-kernel figures on device-resident inputs (ahip_dev_*):
    the decode GEMV's GB/s per matrix shape (C1's projections and logits, the
    C4 and C5 FFN matrices), warm (Infinity-Cache resident) and cold (cycling
    over copies larger than the cache); C2's two isolated GEMMs' MFMA
    fraction; C3's flash attention (T = 4096) and decode attention (one query
    over 2048 rows).  decode_cache_check: a C1 decode launch's GPU time with the
    previous token's data in the 256 MB Infinity Cache and after evicting it.
    --kernels-only prints just the kernel figures (for kernel traces).
  * roofline.traffic: HBM bytes per decode launch from the committed counter
    summary (profiles/c1_decode_hbm_counters.md), used only when the summary
    was measured on the decode kernel's current sources (it records a hash of
    them; see --counter-summary), else null with the reason.

--decode-only and --prefill-only (with --config C1/C4/C5) run only the timed
decode steps or only --prefill-runs 4096-token prefills, for rocprofv3 counter
passes and kernel traces.

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


def q8_bytes(rows: int, cols: int, block: int = 34) -> int:
    """Bytes of a rows x cols matrix in 32-weight blocks of `block` bytes (Q8_0 34, Q4_0 18)."""
    return rows * cols // 32 * block


def decode_token_bytes(c, ctx_len: float, block: int = 34) -> float:
    """Algorithmic HBM bytes of one decode token at context ctx_len."""
    H, QW, KW, F, V, L = c.hidden_size, c.query_width, c.kv_width, c.feed_forward_size, c.vocab_size, c.layer_count
    b = block
    proj = L * (q8_bytes(QW + 2 * KW, H, b) + q8_bytes(H, QW, b) + 2 * q8_bytes(F, H, b) + q8_bytes(H, F, b))
    return proj + q8_bytes(V, H, b) + (2 * L + 1) * H * 4 + 2 * L * ctx_len * KW * 2 + 2 * L * KW * 2


def decode_phase_bytes(c, ctx_len: float) -> dict:
    """Algorithmic bytes of each phase of one layer (weights or KV rows it must read)."""
    H, QW, KW, F = c.hidden_size, c.query_width, c.kv_width, c.feed_forward_size
    return {
        "qkv (fused norm)": q8_bytes(QW + 2 * KW, H) + 4 * H,
        "attention": 2 * 2 * ctx_len * KW,
        "attn out projection (+residual)": q8_bytes(H, QW),
        "ffn gate+up+silu (fused norm)": 2 * q8_bytes(F, H) + 4 * H,
        "ffn down (+residual)": q8_bytes(H, F),
        "final norm + logits": q8_bytes(c.vocab_size, H) + 4 * H,
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


def other_config(ctx, spec, ctx_len: int, prefill_tokens: int, steps: int = 64, profile: bool = True) -> dict:
    """Decode at ctx_len and a prefill of prefill_tokens on another BASELINE config
    (random-init weights of its shape): tok/s and the fraction of the roofline.
    With profile, one more (profiled, one-stream) prefill gives each GEMM's and
    the attention's algorithmic TFLOP/s and fraction of the f16 MFMA peak."""
    import numpy as np

    from alpaca_amd import synth
    from alpaca_amd.model import HIPLlamaModel
    from alpaca_amd.tensor import Q4_0
    c = spec.config
    model = HIPLlamaModel(ctx, c, synth.build_weights(spec))
    prompt = synth.prompt_tokens(spec, max(ctx_len, prefill_tokens))
    s = model.make_session(capacity=ctx_len + steps + 16, max_batch=4096)
    first = int(np.argmax(s.forward(prompt[:ctx_len])))
    t0 = time.perf_counter()
    s.decode_greedy(first, steps, lambda t: True)
    el = time.perf_counter() - t0
    launch = s.last_gpu_seconds / steps
    tok_bytes = decode_token_bytes(c, ctx_len + (steps - 1) / 2 + 1, 18 if spec.dtype == Q4_0 else 34)
    # which decode step the session took: a profiled single-token decode leaves
    # persistent-launch stamps only on the persistent kernel
    s.profiling_enabled = True
    s.decode(first)
    persistent = s.decode_timeline[0].size > 0
    s.close()
    p = model.make_session(capacity=prefill_tokens, max_batch=4096)
    for _ in range(2):
        p.forward(prompt[:prefill_tokens])
        p.reset()
    walls = []
    for _ in range(5):
        t0 = time.perf_counter()
        p.forward(prompt[:prefill_tokens])
        walls.append(time.perf_counter() - t0)
        p.reset()
    wall = float(np.median(walls))
    # the stage FLOPs are per layer
    fl = prefill_stage_flops(c, prefill_tokens)
    flops = c.layer_count * sum(fl.values()) + 2 * c.vocab_size * c.hidden_size
    stages = None
    if profile:
        p.profiling_enabled = True
        p.forward(prompt[:prefill_tokens])
        prof = p.last_profile
        p.reset()
        stages = {}
        for label, st in prof.items():
            if label in fl and st.dispatches:
                avg = st.seconds / st.dispatches
                stages[label] = {"avg_us": round(avg * 1e6, 2), "TFLOPs": round(fl[label] / avg / 1e12, 1),
                                 "frac": round(fl[label] / avg / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}
    p.close()
    model.close()
    return {"decode_ctx": ctx_len, "decode_tok_s": round(steps / el, 1), "decode_avg_step_us": round(launch * 1e6, 1),
            "decode_path": ("persistent decode kernel, one launch per token" if persistent else
                            "multi-kernel step in one HIP graph per token (streamed GEMVs, split-K attention, merge)"),
            "decode_hbm_frac": round(tok_bytes / launch / 1e9 / HBM_PEAK_GBS, 4),
            "prefill_tokens": prefill_tokens, "prefill_tok_s": round(prefill_tokens / wall, 1),
            "prefill_mfma_frac": round(flops / wall / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
            "prefill_note": "wall clock of forward, GEMMs + causal attention + last-token logits",
            "prefill_stages": stages,
            "prefill_stages_note": ("one profiled one-stream prefill; frac = algorithmic 2*M*N*K (attention: "
                                    "causal QK^T + PV) per launch / launch time / 2.5 PFLOP/s; the QKV GEMM "
                                    "issues twice that MFMA work (two-term input on every row), the others about "
                                    "that (two terms on the last 256 rows)") if stages else None}


class DevBuffers:
    """Device buffers through the C ABI's thin shim (ahip_malloc / ahip_memcpy_htod), freed together."""

    def __init__(self, ctx):
        self.ctx, self.ptrs = ctx, []

    def put(self, arr) -> "object":
        import ctypes as C

        from alpaca_amd import _lib as L
        p = C.c_void_p()
        L.check(L.lib().ahip_malloc(self.ctx.handle, max(int(arr.nbytes), 4), C.byref(p)))
        self.ptrs.append(p)
        L.check(L.lib().ahip_memcpy_htod(self.ctx.handle, p, arr.ctypes.data, arr.nbytes))
        return p

    def empty(self, nbytes: int):
        import ctypes as C

        from alpaca_amd import _lib as L
        p = C.c_void_p()
        L.check(L.lib().ahip_malloc(self.ctx.handle, max(int(nbytes), 4), C.byref(p)))
        self.ptrs.append(p)
        return p

    def close(self) -> None:
        from alpaca_amd import _lib as L
        for p in self.ptrs:
            L.lib().ahip_free(self.ctx.handle, p)
        self.ptrs = []


# Decode GEMV shapes (rows, cols, format) whose kernel-level rate is reported:
# C1's projections and tied logits, C4's FFN matrix and C5's FFN matrix.
GEMV_SHAPES = (("C1 qkv", 960, 576, "q8_0"), ("C1 wo", 576, 576, "q8_0"), ("C1 gate (or up)", 1536, 576, "q8_0"),
               ("C1 down", 576, 1536, "q8_0"), ("C1 logits", 49152, 576, "q8_0"),
               ("C4 gate (or up)", 2560, 960, "q4_0"), ("C5 gate (or up)", 8192, 2048, "q8_0"),
               ("C5 down", 2048, 8192, "q8_0"))
MALL_BYTES = 256 << 20  # MI355X Infinity Cache


def kernel_figures(ctx, iters: int = 200) -> dict:
    """Isolated-kernel figures on device-resident inputs, timed with HIP events
    around back-to-back launches (ahip_dev_*): the decode GEMV per matrix shape
    warm (one matrix, which stays in the 256 MB Infinity Cache once read) and
    cold (launches cycle over copies totalling more than twice that cache, so
    each streams from HBM); C2's two isolated GEMMs; C3's flash attention and
    decode attention."""
    import ctypes as C

    import numpy as np

    from alpaca_amd import _lib as L
    from alpaca_amd import synth
    from alpaca_amd.tensor import Q4_0, Q8_0, encode
    lib = L.lib()
    bufs = DevBuffers(ctx)
    out = {"timing": f"HIP events around {iters} back-to-back launches on the context stream (ahip_dev_*)"}
    try:
        rows = []
        for name, n, k, fmt in GEMV_SHAPES:
            dt = Q8_0 if fmt == "q8_0" else Q4_0
            w = encode(synth.normal(synth.tensor_seed(9, n + k), n * k, 0.02).reshape(n, k), dt)
            wbytes = n * k // 32 * (34 if fmt == "q8_0" else 18)
            moved = wbytes + 4 * k + 4 * n
            copies = max(1, -(-2 * MALL_BYTES // wbytes))
            handles = []
            for _ in range(copies):
                h = C.c_void_p()
                L.check(lib.ahip_dev_pack_weight(ctx.handle, dt, w.data.ctypes.data, n, k, C.byref(h)))
                handles.append(h)
            dx = bufs.put(synth.normal(synth.tensor_seed(9, 7), k, 1.0))
            dy = bufs.empty(4 * n)
            warm, cold = C.c_double(), C.c_double()
            arr = (C.c_void_p * copies)(*[h.value for h in handles])
            L.check(lib.ahip_dev_gemv_cycle(ctx.handle, arr, 1, dx, dy, 20, C.byref(warm)))  # untimed warm-up
            L.check(lib.ahip_dev_gemv_cycle(ctx.handle, arr, 1, dx, dy, iters, C.byref(warm)))
            L.check(lib.ahip_dev_gemv_cycle(ctx.handle, arr, copies, dx, dy, max(iters, 2 * copies), C.byref(cold)))
            for h in handles:
                lib.ahip_dev_weight_free(ctx.handle, h)
            rows.append({"matrix": name, "shape": f"{n}x{k} {fmt}", "bytes": moved,
                         "warm_us": round(warm.value * 1e6, 3), "warm_GBs": round(moved / warm.value / 1e9, 1),
                         "cold_us": round(cold.value * 1e6, 3), "cold_GBs": round(moved / cold.value / 1e9, 1),
                         "cold_hbm_frac": round(moved / cold.value / 1e9 / HBM_PEAK_GBS, 4), "cold_copies": copies})
        out["gemv"] = rows
        out["gemv_note"] = ("gemv_kernel (the multi-kernel decode's GEMV; the persistent decode kernel runs the same "
                            "per-chunk dot products inside its phases): bytes = quantised weights + f32 input + f32 "
                            "output; warm repeats one matrix (Infinity Cache resident once read), cold cycles over "
                            "copies totalling over 512 MB; hbm_frac against 8 TB/s")
        # C2: the two isolated Q8_0 GEMMs (M = 2048), fp32 A and C
        gem = []
        for n, k in ((1536, 576), (576, 1536)):
            x, w = synth.c2_gemm_case(n, k)
            m = x.shape[0]
            h = C.c_void_p()
            L.check(lib.ahip_dev_pack_weight(ctx.handle, w.dtype, w.data.ctypes.data, n, k, C.byref(h)))
            dx, dy = bufs.put(np.ascontiguousarray(x)), bufs.empty(4 * m * n)
            flops = 2 * m * n * k
            row = {"shape": f"M={m} N={n} K={k} q8_0", "flops": flops}
            for prec, code, issued in (("fast", L.GEMM_FAST, 2), ("fast_f16", L.GEMM_FAST_F16, 1),
                                       ("exact", L.GEMM_EXACT, 1)):
                t = C.c_double()
                L.check(lib.ahip_dev_gemm(ctx.handle, h, dx, m, dy, code, 5, C.byref(t)))
                L.check(lib.ahip_dev_gemm(ctx.handle, h, dx, m, dy, code, 50, C.byref(t)))
                tf = flops / t.value / 1e12
                row[prec] = {"us": round(t.value * 1e6, 2), "TFLOPs": round(tf, 1),
                             "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                             "issued_frac": round(issued * tf / MFMA_F16_PEAK_TFLOPS, 4)}
            lib.ahip_dev_weight_free(ctx.handle, h)
            gem.append(row)
        out["c2_gemm"] = gem
        out["c2_note"] = ("frac = 2*M*N*K / time / 2.5 PFLOP/s dense f16; issued_frac counts the MFMA work issued "
                          "(fast: two activation terms on every row, twice the algorithmic; exact is SIMT float32)")
        # C3: causal GQA flash attention at T = 4096 (one f16 term for Q and P, as the
        # prefill's query blocks before the last row's), and decode of one query over 2048 rows
        q, kk, v = synth.c3_attention_case()
        T, H, KVH, hd = q.shape[0], q.shape[1], kk.shape[1], q.shape[2]
        dq, dk, dv = bufs.put(np.ascontiguousarray(q)), bufs.put(np.ascontiguousarray(kk)), bufs.put(np.ascontiguousarray(v))
        do = bufs.empty(4 * T * H * hd)
        t = C.c_double()
        L.check(lib.ahip_dev_attention(ctx.handle, dq, dk, dv, T, H, KVH, hd, 0, do, 3, C.byref(t)))
        L.check(lib.ahip_dev_attention(ctx.handle, dq, dk, dv, T, H, KVH, hd, 0, do, 30, C.byref(t)))
        af = 2 * hd * H * T * (T + 1)
        out["c3_prefill_attention"] = {"us": round(t.value * 1e6, 2), "flops": af,
                                       "TFLOPs": round(af / t.value / 1e12, 1),
                                       "frac": round(af / t.value / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                                       "kernel": "flash_attn_kernel, one f16 term for Q and P"}
        L_vis = 2048
        kc = np.ascontiguousarray(kk.transpose(1, 0, 2))  # [kv_heads][capacity][hd]
        vc = np.ascontiguousarray(v.transpose(1, 0, 2))
        dkc, dvc = bufs.put(kc), bufs.put(vc)
        dq1 = bufs.put(np.ascontiguousarray(q[L_vis - 1].astype(np.float32)))
        do1 = bufs.empty(4 * H * hd)
        L.check(lib.ahip_dev_attention_decode(ctx.handle, dq1, dkc, dvc, T, L_vis, H, KVH, hd, do1, 20, C.byref(t)))
        L.check(lib.ahip_dev_attention_decode(ctx.handle, dq1, dkc, dvc, T, L_vis, H, KVH, hd, do1, iters, C.byref(t)))
        ab = 2 * L_vis * KVH * hd * 2
        out["c3_decode_attention"] = {"us": round(t.value * 1e6, 3), "bytes": ab,
                                      "GBs": round(ab / t.value / 1e9, 1),
                                      "hbm_frac": round(ab / t.value / 1e9 / HBM_PEAK_GBS, 4),
                                      "kernel": "attn_decode_split_kernel + attn_merge_kernel (one query, "
                                                "2048 visible f16 rows of 3 KV heads)"}
    finally:
        bufs.close()
    return out


def mall_check(ctx, session, token: int, steps: int = 24) -> dict:
    """Whether the Infinity Cache serves a C1 decode token's 190 MB: the
    persistent launch's GPU time (HIP events of the call) with the previous
    token's data left in the cache, against the same launch after 1 GiB of
    device writes evicted it."""
    import ctypes as C

    import numpy as np

    from alpaca_amd import _lib as L
    bufs = DevBuffers(ctx)
    try:
        ev = bufs.empty(1 << 30)
        warm, cold = [], []
        for i in range(steps):
            if i % 2:
                L.check(L.lib().ahip_memset(ctx.handle, ev, i & 0xFF, 1 << 30))
            logits = session.decode(token)
            (cold if i % 2 else warm).append(session.last_gpu_seconds)
            token = int(np.argmax(logits))
        w, c = float(np.median(warm[1:])), float(np.median(cold[1:]))
        return {"warm_us": round(w * 1e6, 1), "after_eviction_us": round(c * 1e6, 1), "ratio": round(c / w, 3),
                "note": "decode() GPU time per launch; 'after eviction' follows 1 GiB of device writes (4x the "
                        "256 MB Infinity Cache)"}
    finally:
        bufs.close()


def stage_table(profile: dict, units: dict, scale: float, unit: str, per: int = 1) -> dict:
    out = {}
    for label, st in profile.items():
        avg = st.seconds / max(st.dispatches, 1)
        row = {"total_ms": round(st.seconds * 1e3 / per, 4), "count": st.dispatches // per,
               "avg_us": round(avg * 1e6, 3)}
        if label in units and avg > 0:
            row[f"achieved_{unit}"] = round(units[label] / avg / scale, 2)
        out[label] = row
    return out


DECODE_SOURCES = ("alpaca_amd/csrc/kernels_decode.hip", "alpaca_amd/csrc/gemv_chunks.h", "alpaca_amd/csrc/common.h",
                  "alpaca_amd/csrc/runtime.cpp")


# The sources that decide the prefill GEMMs' memory traffic: the kernels (tile
# choice included) and the shared header.
GEMM_SOURCES = ("alpaca_amd/csrc/kernels_gemm.hip", "alpaca_amd/csrc/common.h")


def source_hash(root: str, sources=DECODE_SOURCES) -> str:
    """sha256 (first 16 hex digits) of the sources that decide a kernel's
    memory traffic (for the decode kernel: its kernel file, the shared headers
    and the host side that sets its launch: items, workgroups, exchange
    layout)."""
    import hashlib
    h = hashlib.sha256()
    for rel in sources:
        with open(os.path.join(root, rel), "rb") as f:
            h.update(rel.encode() + b"\0" + f.read())
    return h.hexdigest()[:16]


def measured_traffic(root: str, rel: str = "profiles/c1_decode_hbm_counters.md", sources=DECODE_SOURCES,
                     label: str = "Decode"):
    """(HBM bytes per launch, source note) from a committed rocprofv3 counter
    summary, or (None, reason) when it is missing or was measured on other
    sources than this tree's."""
    import re
    try:
        with open(os.path.join(root, rel)) as f:
            text = f.read()
    except OSError:
        return None, f"{rel} missing"
    m = re.search(r"Traffic per launch[^:]*:\s*([0-9.]+)\s*MB", text)
    h = re.search(label + r" source hash:\s*([0-9a-f]+)", text)
    cur = source_hash(root, sources)
    if not m or not h:
        return None, f"{rel} has no traffic figure or source hash"
    if h.group(1) != cur:
        return None, f"stale: {rel} was measured on {label.lower()} sources {h.group(1)}, this tree has {cur}"
    return float(m.group(1)) * 1e6, f"{rel} (rocprofv3 FETCH_SIZE and WRITE_SIZE runs, scaled by a copy; sources {cur})"


def counter_summary(dirs: dict, kernel: str, gemm: bool = False) -> int:
    """Markdown summary of rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of
    `kernel` and of the calibration copy, with the source hash bench.py checks."""
    import glob
    import sqlite3

    def values(d: str, name: str, counter: str):
        out = []
        for db in glob.glob(os.path.join(d, "**", "*results.db"), recursive=True):
            con = sqlite3.connect(db)
            rows = con.execute("select kernel_name, counter_name, value from counters_collection").fetchall()
            out += [v for k, c, v in rows if name in k and c == counter]
        return out

    cf, cw = values(dirs["copy_fetch"], "copyBuffer", "FETCH_SIZE"), values(dirs["copy_write"], "copyBuffer", "WRITE_SIZE")
    if kernel in ("decode-step-kernels", "prefill-kernels"):
        return counter_table(dirs, cf, cw, values, prefill=kernel == "prefill-kernels")
    kf, kw = values(dirs["fetch"], kernel, "FETCH_SIZE"), values(dirs["write"], kernel, "WRITE_SIZE")
    if not (cf and cw and kf and kw):
        print("missing counter rows", file=sys.stderr)
        return 1
    copy_kib = 256 * 1024
    sf, sw = copy_kib / max(cf), copy_kib / max(cw)
    mf, mw = sum(kf) / len(kf), sum(kw) / len(kw)
    traffic = (mf * sf + mw * sw) * 1024 / 1e6
    root = os.path.dirname(os.path.abspath(__file__))
    print(f"Calibration: a 256 MiB device-to-device copy reads FETCH_SIZE = {max(cf):,.0f} KiB and "
          f"WRITE_SIZE = {max(cw):,.0f} KiB: FETCH_SIZE is scaled by {sf:.2f}, WRITE_SIZE by {sw:.2f}.\n")
    print(f"| counter | dispatches of {kernel} | mean KiB / dispatch | min | max | scaled MB / dispatch |")
    print("|---|---:|---:|---:|---:|---:|")
    for name, v, sc in (("FETCH_SIZE", kf, sf), ("WRITE_SIZE", kw, sw)):
        print(f"| {name} | {len(v)} | {sum(v) / len(v):.1f} | {min(v):.1f} | {max(v):.1f} | "
              f"{sum(v) / len(v) * sc * 1024 / 1e6:.1f} |")
    label, src = ("GEMM", GEMM_SOURCES) if gemm else ("Decode", DECODE_SOURCES)
    print(f"\nTraffic per launch: {traffic:.1f} MB\n\n{label} source hash: {source_hash(root, src)}")
    return 0


def counter_table(dirs: dict, cf: list, cw: list, values, prefill: bool = False) -> int:
    """Per-kernel HBM bytes: every kernel of a multi-kernel decode run
    (--counter-kernel decode-step-kernels) with its dispatches and scaled
    FETCH_SIZE / WRITE_SIZE per dispatch, and the sum per decode step (one
    arg-max dispatch per step); or every GEMM, attention and RMSNorm kernel of
    a prefill run (--counter-kernel prefill-kernels), per dispatch."""
    import glob
    import re
    import sqlite3

    def per_kernel(d: str, counter: str) -> dict:
        out = {}
        for db in glob.glob(os.path.join(d, "**", "*results.db"), recursive=True):
            con = sqlite3.connect(db)
            for k, c, v in con.execute("select kernel_name, counter_name, value from counters_collection"):
                if c == counter:
                    out.setdefault(re.sub(r"\(anonymous namespace\)::", "", k), []).append(v)
        return out

    if not (cf and cw):
        print("missing calibration rows", file=sys.stderr)
        return 1
    sf, sw = 256 * 1024 / max(cf), 256 * 1024 / max(cw)
    f, w = per_kernel(dirs["fetch"], "FETCH_SIZE"), per_kernel(dirs["write"], "WRITE_SIZE")
    kinds = ("dgemm_kernel", "flash_attn", "rmsnorm_rows") if prefill else \
        ("gemv", "attn_decode", "attn_merge", "argmax", "embed")
    names = [k for k in f if k in w and any(t in k for t in kinds)]
    if not prefill:
        # the prompt's last-row GEMVs (input form 3, two f16 terms) belong to the prefill
        names = [k for k in names if not re.search(r"gemv(_stream)?_kernel<[^>]*, 3>", k)]
    steps = 1 if prefill else max((len(f[k]) for k in names if "argmax" in k), default=0)
    if not names or not steps:
        print("missing kernel rows", file=sys.stderr)
        return 1
    print(f"Calibration: a 256 MiB device-to-device copy reads FETCH_SIZE = {max(cf):,.0f} KiB and "
          f"WRITE_SIZE = {max(cw):,.0f} KiB: FETCH_SIZE is scaled by {sf:.2f}, WRITE_SIZE by {sw:.2f}.\n")
    print("| kernel | dispatches | fetch MB / dispatch | write MB / dispatch | " +
          ("MB / dispatch |" if prefill else "MB per decode step |"))
    print("|---|---:|---:|---:|---:|")
    total = 0.0
    for k in sorted(names, key=lambda k: -sum(f[k]) * sf):
        mf, mw = sum(f[k]) / len(f[k]) * sf * 1024 / 1e6, sum(w[k]) / len(w[k]) * sw * 1024 / 1e6
        per_step = (sum(f[k]) * sf + sum(w[k]) * sw) * 1024 / 1e6 / steps
        total += per_step
        print(f"| `{k[:90]}` | {len(f[k])} | {mf:.2f} | {mw:.3f} | {mf + mw if prefill else per_step:.1f} |")
    if not prefill:
        print(f"\nDecode steps (arg-max dispatches): {steps}; traffic per decode step: {total:.1f} MB")
    return 0


def library_gemm(iters: int = 50) -> list:
    """torch.matmul on f16 operands (hipBLASLt / rocBLAS) at the M = 4096 prefill GEMM shapes of C1 and
    C5 (N counts gate and up together), f16 out, no epilogue: what a plain library f16 GEMM reaches at
    these shapes, beside the quantised two-term kernels of this library (HIP events around `iters`
    back-to-back launches after five untimed ones)."""
    import torch
    shapes = (("C1 qkv", 960, 576), ("C1 wo", 576, 576), ("C1 gate+up", 3072, 576), ("C1 down", 576, 1536),
              ("C5 qkv", 6144, 2048), ("C5 wo", 2048, 2048), ("C5 gate+up", 16384, 2048), ("C5 down", 2048, 8192))
    out = []
    m = PREFILL_TOKENS
    for name, n, k in shapes:
        a = torch.randn(m, k, device="cuda", dtype=torch.float16)
        b = torch.randn(k, n, device="cuda", dtype=torch.float16)
        for _ in range(5):
            c = a @ b
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(iters):
            c = a @ b
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / iters * 1e3
        tf = 2 * m * n * k / us / 1e6
        out.append({"gemm": name, "shape": f"M={m} N={n} K={k} f16", "us": round(us, 2), "TFLOPs": round(tf, 1),
                    "frac": round(tf / 2500, 4)})
        del a, b, c
    return out


def cpu_info() -> dict:
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS")
    threads = min(avail, int(cap)) if cap and cap.isdigit() and int(cap) > 0 else avail
    return {"nproc": os.cpu_count(), "affinity_cores": avail, "threads": threads, "cpu_model": model}


def cpu_baseline(weights, spec, budget_s: float = 12.0) -> dict:
    import numpy as np

    from alpaca_amd import synth
    import oracle.oracle as orc
    c = spec.config
    cfg = dict(vocab=c.vocab_size, hidden=c.hidden_size, layers=c.layer_count, heads=c.head_count,
               kv_heads=c.kv_head_count, head_dim=c.head_dim, ffn=c.feed_forward_size, context=c.context_length,
               eps=c.rms_norm_eps, theta=c.rope_theta, interleaved=c.rope_interleaved)
    om = orc.OracleModel(cfg, {n: (t.dtype, t.data) for n, t in weights.items()})
    info = cpu_info()
    orc.set_threads(info["threads"])
    # the reference's CPU-runnable case: 128-token prompt, then 16 greedy tokens
    kv0 = orc.OracleKV(cfg, 256)
    prompt = synth.prompt_tokens(spec, 128)
    t0 = time.perf_counter()
    tok = int(np.argmax(orc.forward(om, kv0, prompt)))
    pre_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    for _ in range(16):
        tok = int(np.argmax(orc.forward(om, kv0, [tok])))
    dec128_s = time.perf_counter() - t0
    # the headline point: decode at context 2048
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
    return {"value": round(steps / el, 3), "unit": "tok/s", "cores": info["threads"], "kind": "port",
            "sample": f"C1 decode, {steps} greedy steps starting at ctx {DECODE_CTX} (oracle KV cache filled with "
                      f"synthetic rows), oracle threaded over 16-row chunks of each linear as AlpacaCore",
            "prefill_128_tok_s": round(128 / pre_s, 2), "decode_after_128_tok_s": round(16 / dec128_s, 3),
            "nproc": info["nproc"], "affinity_cores": info["affinity_cores"], "cpu_model": info["cpu_model"]}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--depth", type=int, default=3, help="greedy-chain steps queued ahead (reference default 3)")
    ap.add_argument("--prefill-runs", type=int, default=9, help="timed 4096-token prefills (median; after two untimed)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-profile", action="store_true")
    ap.add_argument("--no-weight-cache", action="store_true", help="skip the prefill-weight-cache measurement")
    ap.add_argument("--no-other-configs", action="store_true", help="skip the C4 / C5 decode and prefill lines")
    ap.add_argument("--config", choices=("C1", "C4", "C5"), default="C1",
                    help="model config of a --decode-only run (default C1, the headline)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the timed decode steps (for counter passes of the decode kernel)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only --prefill-runs unprofiled 4096-token prefills of --config (for counter passes and "
                         "traces of the prefill kernels)")
    ap.add_argument("--no-kernels", action="store_true", help="skip the isolated-kernel figures and the cache check")
    ap.add_argument("--kernels-only", action="store_true",
                    help="only the isolated-kernel figures (GEMV per shape, C2 GEMMs, C3 attention), for traces")
    ap.add_argument("--library-gemm", action="store_true",
                    help="only torch's f16 GEMM (the ROCm BLAS libraries) at the prefill GEMM shapes of C1 and C5: "
                         "a reference for what a plain f16 GEMM reaches at those shapes")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only a device-to-device copy of 256 MiB, the reference the HBM byte counters are scaled by")
    ap.add_argument("--counter-summary", nargs=4, metavar=("FETCH_DIR", "WRITE_DIR", "COPY_FETCH_DIR", "COPY_WRITE_DIR"),
                    help="print the markdown summary of rocprofv3 --pmc output directories (no GPU use)")
    ap.add_argument("--counter-kernel", default="decode_step_kernel")
    ap.add_argument("--counter-gemm", action="store_true",
                    help="the summarised kernel is a prefill GEMM: record the GEMM sources' hash")
    args = ap.parse_args()
    if args.counter_summary:
        fd, wd, cfd, cwd = args.counter_summary
        return counter_summary({"fetch": fd, "write": wd, "copy_fetch": cfd, "copy_write": cwd}, args.counter_kernel,
                               args.counter_gemm)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures the single-GPU hot path only: this build runs on one GPU "
              "(sharding over several GPUs is not implemented); run with --gpus 1.", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0 or args.warmup >= DECODE_CTX:
        print("need steps >= 1 and 0 <= warmup < 2048", file=sys.stderr)
        return 2

    if args.calibrate_copy:
        import torch
        a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        log("copied 256 MiB device to device")
        return 0

    import numpy as np

    from alpaca_amd import synth
    from alpaca_amd.model import HIPContext, HIPLlamaModel

    if args.library_gemm:
        print(json.dumps({"library_f16_gemm": library_gemm()}), flush=True)
        return 0
    if args.kernels_only:
        kctx = HIPContext(0)
        print(json.dumps({"kernels": kernel_figures(kctx)}), flush=True)
        kctx.close()
        return 0

    # --config picks another BASELINE config for a --decode-only run (counter passes of its decode)
    spec = {"C1": synth.C1, "C4": synth.C4, "C5": synth.C5}[args.config]
    decode_ctx = {"C1": DECODE_CTX, "C4": 2048, "C5": 4096}[args.config]
    block = 18 if args.config == "C4" else 34
    if args.config != "C1" and not (args.decode_only or args.prefill_only):
        log("--config other than C1 is for --decode-only and --prefill-only runs")
        return 2
    c = spec.config
    t0 = time.perf_counter()
    weights = synth.build_weights(spec)
    log(f"synthetic {args.config} weights built in {time.perf_counter() - t0:.1f}s")
    ctx = HIPContext(0)
    model = HIPLlamaModel(ctx, c, weights)
    log(f"model resident: {model.weight_bytes / 1e6:.1f} MB")
    prompt = synth.prompt_tokens(spec, PREFILL_TOKENS)
    if args.prefill_only:
        p = model.make_session(capacity=PREFILL_TOKENS, max_batch=PREFILL_TOKENS)
        for _ in range(2):
            p.forward(prompt)
            p.reset()
        walls = []
        for _ in range(max(1, args.prefill_runs)):
            t0 = time.perf_counter()
            p.forward(prompt)
            walls.append(time.perf_counter() - t0)
            p.reset()
        print(json.dumps({"config": args.config, "prefill_tokens": PREFILL_TOKENS,
                          "prefill_tok_s": round(PREFILL_TOKENS / float(np.median(walls)), 1)}), flush=True)
        p.close()
        model.close()
        ctx.close()
        return 0

    # ---------------------------------------------------------------- decode
    cap = decode_ctx + args.steps + 16
    s = model.make_session(capacity=cap, max_batch=PREFILL_TOKENS)
    first = int(np.argmax(s.forward(prompt[: decode_ctx - args.warmup])))
    toks = []
    if args.warmup:
        s.decode_greedy(first, args.warmup, lambda t: toks.append(t) or True, depth=args.depth)
        first = toks[-1]
    assert s.length == decode_ctx, s.length
    log(f"decode: context {s.length}, timing {args.steps} steps")
    timed = []
    t0 = time.perf_counter()
    fed = s.decode_greedy(first, args.steps, lambda t: timed.append(t) or True, depth=args.depth)
    el = time.perf_counter() - t0
    gpu_s = s.last_gpu_seconds
    assert fed == args.steps
    decode_tok_s = args.steps / el
    avg_launch = gpu_s / args.steps
    mean_ctx = decode_ctx + (args.steps - 1) / 2 + 1
    tok_bytes = decode_token_bytes(c, mean_ctx, block)
    achieved = tok_bytes / avg_launch / 1e9
    traffic, traffic_note = (measured_traffic(os.path.dirname(os.path.abspath(__file__))) if args.config == "C1"
                             else (None, "counters are summarised for C1 only"))
    mode = "cooperative" if os.environ.get("ALPACA_HIP_DECODE_COOPERATIVE", "0") not in ("", "0") else "ordinary"
    roof = {"bound": "hbm", "kernel": f"decode_step_kernel (persistent, one {mode} launch per token)",
            "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 5),
            "traffic": traffic, "traffic_source": traffic_note,
            "bytes_per_launch": int(tok_bytes), "avg_launch_us": round(avg_launch * 1e6, 3),
            "timing": "HIP events on the session stream around the timed steps, divided by the steps"}
    log(f"decode: {decode_tok_s:.1f} tok/s ({el / args.steps * 1e3:.3f} ms/token wall, "
        f"{avg_launch * 1e6:.1f} us/launch GPU, {achieved:.0f} GB/s algorithmic)")
    if args.decode_only:
        print(json.dumps({"config": args.config, "decode_ctx": decode_ctx, "decode_tok_s": round(decode_tok_s, 2),
                          "roofline": roof}), flush=True)
        s.close()
        model.close()
        ctx.close()
        return 0

    # ---------------------------------------------------------------- prefill
    p = model.make_session(capacity=PREFILL_TOKENS, max_batch=PREFILL_TOKENS)
    for _ in range(2):
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
    roof_p, stages_d, stages_p = None, {}, {}
    if not args.no_profile:
        prof_steps = min(args.steps, 32)
        s2 = model.make_session(capacity=cap, max_batch=PREFILL_TOKENS)
        t2 = int(np.argmax(s2.forward(prompt[:DECODE_CTX])))
        s2.profiling_enabled = True
        s2.decode_greedy(t2, prof_steps, lambda t: True, depth=args.depth)
        stages_d = stage_table(s2.last_profile, decode_phase_bytes(c, DECODE_CTX + prof_steps / 2), 1e9, "GBs",
                               per=prof_steps)
        p.profiling_enabled = True
        p.forward(prompt)
        profp = p.last_profile
        p.reset()
        fl = prefill_stage_flops(c, PREFILL_TOKENS)
        stages_p = stage_table(profp, fl, 1e12, "TFLOPs")
        domp = max((k for k in profp if k in fl and k != "attention"), key=lambda k: profp[k].seconds)
        avgp = profp[domp].seconds / profp[domp].dispatches
        ach = fl[domp] / avgp / 1e12
        ptraffic, ptraffic_note = (None, "counters are summarised for the gate+up+silu GEMM only")
        if domp == "ffn gate+up+silu":
            ptraffic, ptraffic_note = measured_traffic(os.path.dirname(os.path.abspath(__file__)),
                                                       "profiles/c1_prefill_hbm_counters.md", GEMM_SOURCES,
                                                       "GEMM")
        roof_p = {"bound": "mfma", "kernel": domp, "achieved": round(ach, 2), "peak": MFMA_F16_PEAK_TFLOPS,
                  "unit": "TFLOP/s", "frac": round(ach / MFMA_F16_PEAK_TFLOPS, 4), "traffic": ptraffic,
                  "traffic_source": ptraffic_note,
                  "flops_per_launch": int(fl[domp]), "avg_launch_us": round(avgp * 1e6, 3)}
        gemm_s = sum(profp[k].seconds for k in profp if k in fl and k != "attention")
        gemm_f = sum(fl[k] * profp[k].dispatches for k in profp if k in fl and k != "attention")
        roof_p["all_prefill_gemms_frac"] = round(gemm_f / gemm_s / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)
        # MFMA work issued per algorithmic multiply-add: the QKV input enters as two f16 terms on
        # every row, the other GEMMs' inputs on the last 256 rows of the prompt only.
        issue = lambda k: 2.0 if k == "qkv projections" else 1.0 + 256 / PREFILL_TOKENS  # noqa: E731
        roof_p["issued_frac"] = round(issue(domp) * roof_p["frac"], 4)
        gemm_fi = sum(issue(k) * fl[k] * profp[k].dispatches for k in profp if k in fl and k != "attention")
        roof_p["all_prefill_gemms_issued_frac"] = round(gemm_fi / gemm_s / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)
        roof_p["note"] = ("frac counts 2*M*N*K algorithmic FLOPs per GEMM; issued_frac the MFMA work issued (the QKV "
                          "GEMM takes two f16 activation terms on every row, the others on the last 256 rows), "
                          "both against 2.5 PFLOP/s dense f16")
        log(f"prefill dominant GEMM: {domp} {ach:.1f} TFLOP/s")

    # ---------------------------------------------------------------- prefill with the weight cache
    wcache = None
    if not args.no_weight_cache:
        cm = HIPLlamaModel(ctx, c, weights, prefill_weight_cache=True)
        cp = cm.make_session(capacity=PREFILL_TOKENS, max_batch=PREFILL_TOKENS)
        for _ in range(2):
            cp.forward(prompt)
            cp.reset()
        cw = []
        for _ in range(max(1, args.prefill_runs)):
            t0 = time.perf_counter()
            cp.forward(prompt)
            cw.append(time.perf_counter() - t0)
            cp.reset()
        wcache = {"prefill_tok_s": round(PREFILL_TOKENS / float(np.median(cw)), 1),
                  "cache_bytes": cm.prefill_cache_bytes}
        if not args.no_profile:
            cp.profiling_enabled = True
            cp.forward(prompt)
            pr = cp.last_profile
            cp.reset()
            k = "ffn gate+up+silu"
            if k in pr:
                avg = pr[k].seconds / pr[k].dispatches
                wcache["gate_up_TFLOPs"] = round(prefill_stage_flops(c, PREFILL_TOKENS)[k] / avg / 1e12, 2)
        log(f"prefill 4096 with the weight cache: {wcache['prefill_tok_s']:.0f} tok/s")
        cp.close()
        cm.close()

    # ---------------------------------------------------------------- other BASELINE configs
    others = None
    if not args.no_other_configs:
        others = {}
        for key, sp, ctx_len, pre in (("C4 360M-shape Q4_0", synth.C4, 2048, 2048),
                                      ("C5 1.7B-shape Q8_0", synth.C5, 4096, 4096)):
            others[key] = other_config(ctx, sp, ctx_len, pre, profile=not args.no_profile)
            log(f"{key}: decode {others[key]['decode_tok_s']} tok/s at ctx {ctx_len} "
                f"({100 * others[key]['decode_hbm_frac']:.1f}% of HBM), prefill {others[key]['prefill_tok_s']} tok/s")

    # ---------------------------------------------------------------- isolated kernels, cache check
    kernels, mall = None, None
    if not args.no_kernels:
        kernels = kernel_figures(ctx)
        for r in kernels["gemv"]:
            log(f"gemv {r['matrix']} {r['shape']}: warm {r['warm_GBs']} GB/s, cold {r['cold_GBs']} GB/s "
                f"({100 * r['cold_hbm_frac']:.1f}% of HBM)")
        for r in kernels["c2_gemm"]:
            log(f"C2 {r['shape']}: fast {r['fast']['TFLOPs']} TFLOP/s ({100 * r['fast']['frac']:.1f}%), "
                f"fast-f16 {r['fast_f16']['TFLOPs']}")
        log(f"C3 flash {kernels['c3_prefill_attention']['TFLOPs']} TFLOP/s, decode attention "
            f"{kernels['c3_decode_attention']['GBs']} GB/s")
        ms = model.make_session(capacity=DECODE_CTX + 64, max_batch=PREFILL_TOKENS)
        mt = int(np.argmax(ms.forward(prompt[:DECODE_CTX])))
        mall = mall_check(ctx, ms, mt)
        ms.close()
        log(f"decode launch {mall['warm_us']} us warm, {mall['after_eviction_us']} us after evicting the cache")

    # ---------------------------------------------------------------- CPU baseline
    cpu = None
    if not args.no_cpu_baseline:
        log("CPU oracle baseline ...")
        cpu = cpu_baseline(weights, spec)
        log(f"CPU oracle: {cpu['value']} tok/s decode at ctx {DECODE_CTX}, 128-token prefill "
            f"{cpu['prefill_128_tok_s']} tok/s, decode after it {cpu['decode_after_128_tok_s']} tok/s, on "
            f"{cpu['cores']} threads ({cpu['cpu_model']}, nproc {cpu['nproc']})")

    line = {
        "metric": METRIC, "value": round(decode_tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(el / args.steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32 (q8_0 weights, f32 accumulate)",
        "data": "synthetic (random-init weights N(0,0.02) quantised to Q8_0, uniform random token ids)",
        "config": {"workload": "C1 135M-shape Q8_0 Llama: greedy decode at context 2048 (value); "
                               "4096-token prefill (prefill_tok_s)",
                   "layers": c.layer_count, "hidden": c.hidden_size, "heads": f"{c.head_count}/{c.kv_head_count}",
                   "head_dim": c.head_dim, "ffn": c.feed_forward_size, "vocab": c.vocab_size,
                   "kv_cache": "f16",
                   "prefill_precision": "fast: f16 MFMA with exact integer quants, per-block f32 scaling and f32 "
                                        "accumulation; activations as two f16 terms (hi + lo) for the QKV input "
                                        "and on the prompt's last 256 rows, one term elsewhere",
                   "greedy_depth": args.depth},
        "prefill_tok_s": round(prefill_tok_s, 1),
        "prefill_mfma_frac": round(c.layer_count * sum(prefill_stage_flops(c, PREFILL_TOKENS).values()) *
                                   prefill_tok_s / PREFILL_TOKENS / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
        "prefill_weight_cache": wcache,
        "other_configs": others,
        "decode_ms_per_token": round(el / args.steps * 1e3, 4),
        "roofline": roof, "roofline_prefill": roof_p, "cpu_baseline": cpu,
        "stages_decode_per_token": stages_d, "stages_prefill": stages_p,
        "kernels": kernels, "decode_cache_check": mall,
        "reference_m5": {"prefill_tok_s_4096": 24069, "decode_tok_s_ctx2048": 456,
                         "note": "Apple M5, real SmolLM2-135M Q8_0 (BASELINE.md); context only"},
    }
    print(json.dumps(line), flush=True)
    for h in (s, p):
        h.close()
    if not args.no_profile:
        s2.close()
    model.close()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
