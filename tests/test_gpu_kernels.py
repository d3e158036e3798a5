"""HIP kernels vs the CPU oracle, through the C ABI (HIPOps = MetalOps mirror).

Shapes and tolerances follow Tests/AlpacaMetalTests/KernelTests.swift.  Where
this backend's arithmetic matches the CPU reference operation for operation
(dequantisation, embedding, RoPE with the double-precision table, the exact
float32 GEMM), the check is bit-for-bit.
"""
import numpy as np
import pytest

import oracle.oracle as orc
from alpaca_amd.tensor import F16, Q4_0, Q8_0, encode
from tests.helpers import assert_close, b64, env, fixture, metrics, splitmix_uniform

pytestmark = pytest.mark.gpu

FORMATS = [("f16", F16), ("q8_0", Q8_0), ("q4_0", Q4_0)]


def rand(shape, seed, scale=1.0):
    n = int(np.prod(shape))
    return (splitmix_uniform(seed, n) * np.float32(scale)).reshape(shape)


def test_elementwise(hip_ops):  # KernelTests.swift:37-43
    a, b = rand((7, 37), 1, 3), rand((7, 37), 2, 3)
    assert_close(hip_ops.add(a, b), orc.add(a, b), 1e-6, 1e-6, "add")
    assert_close(hip_ops.mul(a, b), orc.mul(a, b), 1e-6, 1e-6, "mul")
    assert_close(hip_ops.silu(a), orc.silu(a), 1e-6, 1e-5, "silu")
    assert_close(hip_ops.silu_mul(a, b), orc.mul(orc.silu(a), b), 1e-5, 1e-5, "silu*mul")


# 30 (not a multiple of 4) and 4096 (past the register-resident row) take the
# block-per-row kernel, the rest the wave-per-row one; 9 rows leave a partial block.
@pytest.mark.parametrize("dim", [30, 32, 576, 960, 1536, 2048, 4096])
def test_rmsnorm(hip_ops, dim):  # KernelTests.swift:45-50
    x, w = rand((9, dim), 3, 2), rand((dim,), 4)
    assert_close(hip_ops.rms_norm(x, w, 1e-5), orc.rmsnorm(x, w, 1e-5), 1e-5, 1e-5, f"rmsnorm {dim}")


@pytest.mark.parametrize("k,n", [(64, 10), (576, 193), (1536, 576)])
@pytest.mark.parametrize("name,dt", FORMATS)
def test_linear_all_formats_and_batch_sizes(hip_ops, k, n, name, dt):  # KernelTests.swift:52-66
    w32 = rand((n, k), 5, 0.3)
    w = encode(w32, dt)
    for t in [1, 3, 8, 11, 16, 33, 70]:
        x = rand((t, k), 6 + t)
        cpu = orc.linear(x, dt, w.data, n)
        gpu = hip_ops.linear(x, w, "exact")
        assert_close(gpu, cpu, 2e-4, 1e-4, f"linear {name} K={k} N={n} T={t}")
        if t > 1:
            # exact GEMM: same per-block float32 order as CPUOps.dot -> identical bits
            assert np.array_equal(gpu.view(np.uint32), cpu.view(np.uint32)), f"exact GEMM bits {name} T={t}"


@pytest.mark.parametrize("k,n", [(64, 10), (576, 193), (1536, 576), (576, 1536)])
@pytest.mark.parametrize("name,dt", FORMATS)
def test_fast_gemm_within_analytic_bound(hip_ops, k, n, name, dt):  # KernelTests.swift:179-217
    """One f16 term per activation: |err| <= 2^-10 * sum_k |x_k w_k| + 1e-5
    element-wise (the reference's fast-path bound); two terms (the default):
    within the exact GEMM's tolerance."""
    w32 = rand((n, k), k * 31 + n, 0.3)
    w = encode(w32, dt)
    wd = orc.dequantize(dt, w.data, n * k).reshape(n, k).astype(np.float64)
    worst = 0.0
    worst_tt = 0.0
    for t in [16, 32, 33, 70, 130, 300]:
        x = rand((t, k), 1000 + t)
        cpu = orc.linear(x, dt, w.data, n).astype(np.float64)
        bound = np.abs(x.astype(np.float64)) @ np.abs(wd).T / 1024 + 1e-5
        # one f16 term per activation (the reference's fast path)
        err = np.abs(hip_ops.linear(x, w, "fast-f16").astype(np.float64) - cpu)
        worst = max(worst, float((err / bound).max()))
        assert (err <= bound).all(), f"fast-f16 GEMM {name} K={k} N={n} T={t}: worst ratio {(err / bound).max()}"
        # two terms (the default): float32-grade inputs, so within the exact GEMM's 2e-4 + 1e-4 |y|
        err = np.abs(hip_ops.linear(x, w, "fast").astype(np.float64) - cpu)
        worst_tt = max(worst_tt, float((err / (2e-4 + 1e-4 * np.abs(cpu))).max()))
        assert (err <= 2e-4 + 1e-4 * np.abs(cpu)).all(), f"fast GEMM {name} K={k} N={n} T={t}"
    print(f"[metrics] fast GEMM {name} K={k} N={n}: worst error / bound = {worst:.3f} (one term), "
          f"{worst_tt:.3f} of 2e-4 + 1e-4 |y| (two terms)")


@pytest.mark.parametrize("k,n", [(64, 10), (96, 40), (576, 193), (256, 300)])
@pytest.mark.parametrize("name,dt", FORMATS)
def test_fast_gemm_weights_enter_exactly(hip_ops, k, n, name, dt):
    """The f16 MFMA GEMM takes the integer quants exactly (f16 holds them) and
    scales each 32-weight block's float32 result by its d.

    With the identity as activations every output is one weight times 1.0 plus
    exact zeros, so Y = W^T must equal the float32 dequantisation bit for bit
    (d * q is exact in float32): a wrong nibble order, block index, scale row or
    LDS swizzle changes a value.  K = 96 takes the register-staged kernel, the
    others the LDS-DMA one.
    """
    w = encode(rand((n, k), 17 * k + n, 0.3), dt)
    deq = orc.dequantize(dt, w.data, n * k).reshape(n, k)
    gpu = hip_ops.linear(np.eye(k, dtype=np.float32), w, "fast")
    assert gpu.shape == (k, n)
    bad = np.argwhere(gpu != deq.T)
    assert bad.size == 0, f"{name} K={k} N={n}: {len(bad)} weights differ, first at (k, n) = {bad[0]}"


@pytest.mark.parametrize("name,dt", FORMATS)
def test_gemm_tile_families_agree_at_large_grids(hip_ops, name, dt):
    """M = 4096, K = 576, N = 1600 (C4's QKV width over a 4096-token prompt):
    800 tiles of 128x64 are more than one round of resident workgroups, so the
    default takes 128x128 tiles.  Every tile family (ALPACA_HIP_GEMM_TILE,
    read per launch) accumulates each output over the same 32-weight blocks in
    the same order, so the store, residual and SwiGLU epilogues must agree bit
    for bit across 64x64, 128x64, 128x128, 128x256 and 256-row tiles.  The
    default (two f16 activation terms) is held to the exact GEMM's tolerance
    2e-4 + 1e-4 |y| against the oracle on every output of the three
    epilogues, and one-hot activation rows pin the weight path of every tile
    (Y[m] = W[:, m mod K] exactly)."""
    m, k, n = 4096, 576, 1600
    w = encode(rand((n, k), 4242 + dt, 0.3), dt)
    wu = encode(rand((n, k), 4343 + dt, 0.3), dt)
    x = rand((m, k), 4244)
    res = rand((m, n), 4245, 5)
    onehot = np.zeros((m, k), np.float32)
    onehot[np.arange(m), np.arange(m) % k] = 1.0
    deq = orc.dequantize(dt, w.data, n * k).reshape(n, k)
    outs = {}
    for tile in (None, "128x64", "128x128", "256", "128x256", "64x64"):
        with env(ALPACA_HIP_GEMM_TILE=tile):
            outs[tile] = (hip_ops.linear(x, w, "fast"), hip_ops.linear_add(x, w, res, "fast"),
                          hip_ops.gate_up_silu(x, w, wu, "fast"))
            ident = hip_ops.linear(onehot, w, "fast")
        bad = np.argwhere(ident != deq.T[np.arange(m) % k])
        assert bad.size == 0, f"{name} tile {tile}: {len(bad)} weights differ, first at (m, n) = {bad[0]}"
    # The tile order (row groups of ALPACA_HIP_GEMM_GROUP row blocks, 3 leaving
    # a partial last group) moves tiles between workgroups, not their sums.
    for tile, group in ((None, "3"), (None, "4"), ("64x64", "3"), ("128x256", "5")):
        with env(ALPACA_HIP_GEMM_TILE=tile, ALPACA_HIP_GEMM_GROUP=group):
            outs[(tile, group)] = (hip_ops.linear(x, w, "fast"), hip_ops.linear_add(x, w, res, "fast"),
                                   hip_ops.gate_up_silu(x, w, wu, "fast"))
    for tile in ("128x64", "128x128", "256", "128x256", "64x64", (None, "3"), (None, "4"), ("64x64", "3"),
                 ("128x256", "5")):
        for i, what in enumerate(("store", "residual", "swiglu")):
            a, b = outs[tile][i], outs[None][i]
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{name} {what}: tile {tile} != default"
    # Two K sets per 64x64 tile sum each output's blocks in two partial sums:
    # equal to the others to float32 rounding, and exact on one-hot rows.
    with env(ALPACA_HIP_GEMM_TILE="64x64k2"):
        k2 = (hip_ops.linear(x, w, "fast"), hip_ops.linear_add(x, w, res, "fast"), hip_ops.gate_up_silu(x, w, wu, "fast"))
        ident = hip_ops.linear(onehot, w, "fast")
    assert np.array_equal(ident, deq.T[np.arange(m) % k]), f"{name}: two K sets, one-hot rows"
    for i, what in enumerate(("store", "residual", "swiglu")):
        a, b = k2[i], outs[None][i]
        assert np.abs(a - b).max() <= 1e-5 * max(1.0, float(np.abs(b).max())), f"{name} {what}: two K sets"
    y = orc.linear(x, dt, w.data, n)
    u = orc.linear(x, dt, wu.data, n)
    cpu = {"store": y, "residual": orc.add(res, y), "swiglu": orc.mul(orc.silu(y), u)}
    for i, what in enumerate(("store", "residual", "swiglu")):
        e = cpu[what].astype(np.float64)
        err = np.abs(outs[None][i].astype(np.float64) - e)
        tol = 2e-4 + 1e-4 * np.abs(e)
        print(f"[metrics] fast GEMM {name} {what} M={m} K={k} N={n}: max |err| {err.max():.3e}, "
              f"worst error / (2e-4 + 1e-4|y|) = {(err / tol).max():.4f}")
        assert (err <= tol).all(), f"{name} {what}: worst error / tolerance {(err / tol).max():.3f}"


@pytest.mark.parametrize("name,dt", FORMATS)
def test_gemm_row_groups_by_default_on_large_weights(hip_ops, name, dt):
    """Weights of 4 MiB and more (4096x1024 in Q8_0, 4.5 MB; 4096x2048 in Q4_0, 4.7 MB; 2048x1024
    in F16, 4.2 MB, the prefill weight cache's format) take the
    tile order in row groups of four row blocks by default; it moves tiles between workgroups, not
    their sums, so the store, residual and SwiGLU epilogues equal the row-by-row order
    (ALPACA_HIP_GEMM_GROUP=0) bit for bit, and the default stays within the exact GEMM's
    tolerance 2e-4 + 1e-4 |y| of the oracle, over M = 1100 rows (a partial last row block and a
    partial last group)."""
    m = 1100
    n, k = {Q8_0: (4096, 1024), Q4_0: (4096, 2048), F16: (2048, 1024)}[dt]
    w = encode(rand((n, k), 6161 + dt, 0.3), dt)
    wu = encode(rand((n, k), 6262 + dt, 0.3), dt)
    x = rand((m, k), 6363)
    res = rand((m, n), 6464, 5)
    outs = {}
    for group in (None, "0"):
        with env(ALPACA_HIP_GEMM_GROUP=group):
            outs[group] = (hip_ops.linear(x, w, "fast"), hip_ops.linear_add(x, w, res, "fast"),
                           hip_ops.gate_up_silu(x, w, wu, "fast"))
    y = orc.linear(x, dt, w.data, n)
    u = orc.linear(x, dt, wu.data, n)
    cpu = (y, orc.add(res, y), orc.mul(orc.silu(y), u))
    for i, what in enumerate(("store", "residual", "swiglu")):
        a, b = outs[None][i], outs["0"][i]
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{name} {what}: row groups != row by row"
        e = cpu[i].astype(np.float64)
        err = np.abs(a.astype(np.float64) - e)
        tol = 2e-4 + 1e-4 * np.abs(e)
        print(f"[metrics] row-group GEMM {name} {what} M={m} K={k} N={n}: worst error / tol {(err / tol).max():.4f}")
        assert (err <= tol).all(), f"{name} {what}: worst error / tolerance {(err / tol).max():.3f}"


def test_fused_gate_up_silu(hip_ops):  # KernelTests.swift:219-244
    k, n = 576, 200
    for t in [1, 3, 16, 40, 100]:
        x = rand((t, k), 77 + t)
        g32, u32 = rand((n, k), 78, 0.3), rand((n, k), 79, 0.3)
        for name, dt in FORMATS:
            wg, wu = encode(g32, dt), encode(u32, dt)
            cpu = orc.mul(orc.silu(orc.linear(x, dt, wg.data, n)), orc.linear(x, dt, wu.data, n))
            for prec in ("exact", "fast"):
                gpu = hip_ops.gate_up_silu(x, wg, wu, prec)
                m = metrics(gpu, cpu)
                print(f"[metrics] gate+up+silu T={t} {name} {prec}: {m}")
                if prec == "exact" or t < 16:
                    assert m["max_abs"] < 1e-3
                else:
                    assert m["max_rel_peak"] < 3e-3


def test_fused_residual_projection(hip_ops):  # KernelTests.swift:246-267
    k, n = 576, 576
    for t in [1, 5, 8, 31, 40, 100]:
        x, res = rand((t, k), 200 + t), rand((t, n), 300 + t, 5)
        for name, dt in FORMATS:
            w = encode(rand((n, k), 400, 0.3), dt)
            cpu = orc.add(res, orc.linear(x, dt, w.data, n))
            for prec in ("exact", "fast"):
                gpu = hip_ops.linear_add(x, w, res, prec)
                bound = 2e-4 if prec == "exact" or t < 16 else 2e-2
                assert metrics(gpu, cpu)["max_abs"] < bound, f"linear+residual {name} {prec} T={t}"


@pytest.mark.parametrize("start,theta", [(0, 10000.0), (7, 100000.0), (1500, 100000.0)])
def test_rope_bit_exact(hip_ops, start, theta):  # KernelTests.swift:68-74
    x = rand((4, 9, 64), 9)
    for inter in (True, False):
        gpu, cpu = hip_ops.rope(x, start, theta, inter), orc.rope(x, start, theta, inter)
        assert np.array_equal(gpu.view(np.uint32), cpu.view(np.uint32)), f"rope start={start} interleaved={inter}"


def _f16(a):
    return a.astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("tokens,start,heads,kv,hd", [(1, 0, 4, 2, 64), (1, 100, 9, 3, 64), (5, 0, 9, 3, 64),
                                                      (7, 20, 8, 2, 128), (3, 1, 6, 6, 32)])
def test_attention_causal_gqa(hip_ops, tokens, start, heads, kv, hd):  # KernelTests.swift:76-88
    cap = start + tokens + 3
    q, k, v = rand((tokens, heads, hd), 11), rand((cap, kv, hd), 12), rand((cap, kv, hd), 13)
    cpu16 = orc.attention(q, _f16(k), _f16(v), start)
    assert_close(hip_ops.attention(q, k, v, start, "f16"), cpu16, 2e-5, 1e-4, f"attention f16-KV T={tokens}")
    cpu32 = orc.attention(q, k, v, start)
    assert_close(hip_ops.attention(q, k, v, start, "f32"), cpu32, 2e-6, 1e-5, f"attention f32-KV T={tokens}")


SPLIT_CASES = [(0, 9, 3, 64), (1, 9, 3, 64), (7, 9, 3, 64), (255, 9, 3, 64), (256, 9, 3, 64), (257, 9, 3, 64),
               (511, 9, 3, 64), (1000, 9, 3, 64), (2047, 9, 3, 64), (300, 8, 2, 128), (700, 8, 8, 64),
               (90, 32, 4, 128), (500, 4, 1, 64), (4095, 15, 5, 64),
               # splits past 256 positions: 512-thread workgroups (the 1.7B shape's 32 KV heads
               # at 4,176 positions: 288-position splits; two heads per KV head, head dim 128;
               # 384- and 448-position splits)
               (4175, 32, 32, 64), (9000, 32, 16, 128), (5999, 64, 32, 64), (6999, 32, 32, 64)]


@pytest.mark.parametrize("start,heads,kv,hd", SPLIT_CASES)
def test_split_decode_attention(hip_ops, start, heads, kv, hd):  # KernelTests.swift:123-144
    cap = start + 1
    q = rand((1, heads, hd), start * 7 + heads)
    k = rand((cap, kv, hd), start * 7 + heads + 1)
    v = rand((cap, kv, hd), start * 7 + heads + 2)
    cpu = orc.attention(q, _f16(k), _f16(v), start)
    gpu = hip_ops.attention(q, k, v, start, "f16")
    m = metrics(gpu, cpu)
    print(f"[metrics] split decode attention ctx={cap} H={heads}/{kv} hd={hd}: {m}")
    assert m["max_abs"] < 2e-6


TILED = [(8, 0, 9, 3, 64), (31, 0, 9, 3, 64), (32, 0, 9, 3, 64), (33, 0, 9, 3, 64), (100, 0, 9, 3, 64),
         (64, 200, 9, 3, 64), (45, 7, 8, 2, 128), (128, 128, 4, 4, 128), (17, 3, 6, 3, 64), (200, 0, 8, 2, 64),
         (16, 0, 9, 3, 64), (300, 40, 15, 5, 64), (1024, 0, 9, 3, 64), (515, 77, 8, 2, 128),
         (1536, 0, 32, 8, 64), (2048, 0, 32, 8, 64)]  # 768 workgroups: two wave-sets; 1,024: one


@pytest.mark.parametrize("t,start,heads,kv,hd", TILED)
def test_flash_attention(hip_ops, t, start, heads, kv, hd):  # KernelTests.swift:146-170
    """f16 Q / P / V on MFMA: <= 1.5e-3 against float64-accurate CPU on the same f16 K/V."""
    cap = start + t
    q, k, v = rand((t, heads, hd), t * 131 + start), rand((cap, kv, hd), t * 131 + start + 1), \
        rand((cap, kv, hd), t * 131 + start + 2)
    cpu = orc.attention(q, _f16(k), _f16(v), start)
    for prec in ("exact", "fast"):
        gpu = hip_ops.attention(q, k, v, start, "f16", prec)
        m = metrics(gpu, cpu)
        print(f"[metrics] attention {prec} T={t} start={start} H={heads}/{kv} hd={hd}: {m}")
        assert np.isfinite(gpu).all()
        assert m["max_abs"] < 1.5e-3


SET_CASES = [(8, 0, 9, 3), (17, 3, 6, 3), (100, 0, 9, 3), (64, 200, 9, 3), (300, 40, 15, 5), (1024, 0, 9, 3),
             (64, 2000, 9, 3), (1536, 0, 32, 8)]


@pytest.mark.parametrize("t,start,heads,kv", SET_CASES)
def test_flash_attention_wave_sets(hip_ops, t, start, heads, kv):
    """Head dim 64 with one and two wave-sets per workgroup
    (ALPACA_HIP_FLASH_SETS, read per launch): two sets split each query
    block's key blocks into consecutive ranges and merge them at the end, so
    both counts are held to the CPU at 1.5e-3 and to each other at 2e-6 (the
    merge changes the float32 summation order only).  Covers a set with no
    key block (8 and 17 tokens: one block), ragged ranges (start 2000: 33
    blocks) and grids past one round."""
    hd = 64
    cap = start + t
    q, k, v = rand((t, heads, hd), t * 17 + start), rand((cap, kv, hd), t * 17 + start + 1), \
        rand((cap, kv, hd), t * 17 + start + 2)
    cpu = orc.attention(q, _f16(k), _f16(v), start)
    out = {}
    for sets in ("1", "2"):
        with env(ALPACA_HIP_FLASH_SETS=sets):
            out[sets] = hip_ops.attention(q, k, v, start, "f16", "fast")
        m = metrics(out[sets], cpu)
        print(f"[metrics] attention sets={sets} T={t} start={start} H={heads}/{kv}: {m}")
        assert np.isfinite(out[sets]).all()
        assert m["max_abs"] < 1.5e-3
    for sets in ("2",):
        assert np.abs(out[sets] - out["1"]).max() <= 2e-6, f"sets={sets}"


@pytest.mark.parametrize("name,dt", FORMATS)
def test_embedding_all_formats(hip_ops, name, dt):  # KernelTests.swift:90-99
    table = rand((50, 96), 21)
    t = encode(table, dt)
    tokens = [0, 49, 7, 7]
    cpu = orc.embed(tokens, dt, t.data, 50, 96)
    gpu = hip_ops.embed(tokens, t)
    assert np.array_equal(gpu.view(np.uint32), cpu.view(np.uint32))
    with pytest.raises(ValueError):
        hip_ops.embed([50], t)


@pytest.mark.parametrize("name", ["q8_0", "q4_0"])
def test_dequantize_bit_exact_against_gguf(hip_ops, name):
    c = fixture("ops")[name]
    dt = Q8_0 if name == "q8_0" else Q4_0
    from alpaca_amd.tensor import QTensor
    t = QTensor(dt, c["n"], c["k"], b64(c["blocks"]))
    gpu = hip_ops.dequantize(t).ravel()
    assert np.array_equal(gpu.astype(np.float64), np.asarray(c["dequantized"], np.float64))
    big = encode(rand((64, 4096), 33, 2.0), dt)
    assert np.array_equal(hip_ops.dequantize(big).ravel(), orc.dequantize(dt, big.data, 64 * 4096))


def test_argmax_rules(hip_ops):
    assert hip_ops.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert hip_ops.argmax([np.nan, 1.0, np.nan, 5.0, 5.0]) == 3  # NaN never wins
    assert hip_ops.argmax([np.nan, np.nan]) == 0
    assert hip_ops.argmax([-np.inf, -np.inf, -1.0]) == 2
    v = rand((49152,), 5)
    v[31337] = 10.0
    v[40000] = 10.0
    assert hip_ops.argmax(v) == 31337 == orc.argmax(v)


@pytest.mark.parametrize("name,dt", FORMATS)
def test_gemm_second_term_from_a_row_on(hip_ops, name, dt):
    """The prefill takes the activations' second term only on a call's last
    rows: a one-term kernel whose tiles from row lo_row0 on (a multiple of
    256) make a second pass over K with the second term as A
    (ALPACA_HIP_OP_LO_ROW0, read per call).  Rows before lo_row0 are the
    one-term (fast-f16) GEMM's bit for bit, as the same one-term tiles compute
    them (SwiGLU's f16 output to its second term); rows from lo_row0 on are
    within the two-term GEMM's tolerance
    2e-4 + 1e-4 |y| of the oracle, in the store, residual and SwiGLU
    epilogues, at M = 4096 (the C1 and C4 prompt length) and one 256-row
    tail, at M = 1000 with a partial last tile."""
    k, n = 576, 1600
    w = encode(rand((n, k), 5151 + dt, 0.3), dt)
    wu = encode(rand((n, k), 5252 + dt, 0.3), dt)
    for m, lo_row0 in ((4096, 3840), (4096, 256), (1000, 768)):
        x = rand((m, k), 5353 + m)
        res = rand((m, n), 5454, 5)
        one = (hip_ops.linear(x, w, "fast-f16"), hip_ops.linear_add(x, w, res, "fast-f16"),
               hip_ops.gate_up_silu(x, w, wu, "fast-f16"))
        with env(ALPACA_HIP_OP_LO_ROW0=lo_row0):
            tail = (hip_ops.linear(x, w, "fast"), hip_ops.linear_add(x, w, res, "fast"),
                    hip_ops.gate_up_silu(x, w, wu, "fast"))
        # row groups of the tile order (3 row blocks: a partial last group) before the tail tiles
        with env(ALPACA_HIP_OP_LO_ROW0=lo_row0, ALPACA_HIP_GEMM_GROUP=3):
            grouped = (hip_ops.linear(x, w, "fast"), hip_ops.linear_add(x, w, res, "fast"),
                       hip_ops.gate_up_silu(x, w, wu, "fast"))
        for i, what in enumerate(("store", "residual", "swiglu")):
            assert np.array_equal(grouped[i].view(np.uint32), tail[i].view(np.uint32)), \
                f"{name} {what} m={m}: row groups of 3 change the result"
        y = orc.linear(x, dt, w.data, n)
        u = orc.linear(x, dt, wu.data, n)
        cpu = (y, orc.add(res, y), orc.mul(orc.silu(y), u))
        for i, what in enumerate(("store", "residual", "swiglu")):
            a, b = tail[i][:lo_row0], one[i][:lo_row0]
            if what == "swiglu":
                # the two-term op returns hi + lo of its f16 output, hi being the one-term op's
                # value and |lo| at most half the ulp of the binade [2^e, 2^(e+1)) that |hi|
                # starts (a power of two rounds from above too), or 2^-24 where hi is
                # subnormal and lo a multiple of 2^-24
                e = np.frexp(np.abs(b.astype(np.float64)))[1] - 1
                half = np.maximum(np.ldexp(0.5, e - 10), 2.0 ** -24)
                d = np.abs(a.astype(np.float64) - b)
                assert (d <= half).all(), f"{name} {what} m={m}: one-term rows differ by {(d / half).max():.2f} half-ulps"
                continue
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{name} {what} m={m}: one-term rows differ"
            e = cpu[i][lo_row0:].astype(np.float64)
            err = np.abs(tail[i][lo_row0:].astype(np.float64) - e)
            tol = 2e-4 + 1e-4 * np.abs(e)
            print(f"[metrics] {name} {what} m={m} rows {lo_row0}..: worst error / (2e-4 + 1e-4|y|) "
                  f"{(err / tol).max():.4f}")
            assert (err <= tol).all(), f"{name} {what} m={m}: two-term rows off by {(err / tol).max():.3f} of tol"


@pytest.mark.parametrize("n,k,name,dt", [(49152, 576, "q8_0", Q8_0), (8192, 2048, "q8_0", Q8_0),
                                         (2048, 8192, "q8_0", Q8_0), (12288, 960, "q4_0", Q4_0),
                                         (4100, 1024, "f16", F16)])
def test_stream_gemv(hip_ops, n, k, name, dt):
    """Matrices of at least 4 MB take the streamed GEMV (the C1 logits, the
    C5 FFN matrices, a Q4_0 and an F16 one with a partial last tile): within
    the exact GEMV's 2e-4 + 1e-4 |y| of the oracle, for the store, residual
    and SwiGLU epilogues, and equal to the one-tile-per-workgroup kernel
    (ALPACA_HIP_GEMV_STREAM=0, read per launch) to float32 rounding (both sum
    each lane's chunks in order, then across lanes)."""
    w = encode(rand((n, k), 6161 + n, 0.05), dt)
    wu = encode(rand((n, k), 6262 + n, 0.05), dt)
    x = rand((1, k), 6363 + k)
    res = rand((1, n), 6464, 3)
    y = orc.linear(x, dt, w.data, n)
    u = orc.linear(x, dt, wu.data, n)
    outs = (hip_ops.linear(x, w, "exact"), hip_ops.linear_add(x, w, res, "exact"), hip_ops.gate_up_silu(x, w, wu, "exact"))
    with env(ALPACA_HIP_GEMV_STREAM=0):
        other = (hip_ops.linear(x, w, "exact"), hip_ops.linear_add(x, w, res, "exact"),
                 hip_ops.gate_up_silu(x, w, wu, "exact"))
    for i, (what, e) in enumerate((("store", y), ("residual", orc.add(res, y)),
                                   ("swiglu", orc.mul(orc.silu(y), u)))):
        assert_close(outs[i], e, 2e-4, 1e-4, f"streamed gemv {name} {n}x{k} {what}")
        d = np.abs(outs[i].astype(np.float64) - other[i])
        assert d.max() <= 1e-5 * max(1.0, float(np.abs(other[i]).max())), f"{what}: streamed vs other kernel {d.max():.3e}"
