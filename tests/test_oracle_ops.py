"""Pins the CPU oracle to the reference's own fixtures and to closed forms.

Mirrors Tests/AlpacaCoreTests/OperationTests.swift (same fixture, same
tolerances) and adds checks that the fixtures leave open: exhaustive f16
conversion, SplitMix64 published vectors, Q4_0 nibble order, RoPE norm
preservation, the argmax tie and NaN rules, and brute-force attention.
"""
import numpy as np
import pytest

import oracle.oracle as orc
from tests.helpers import assert_close, b64, fixture

ops = fixture("ops")


def test_add_mul():  # OperationTests.swift:15-22
    a, m = ops["add"], ops["mul"]
    assert_close(orc.add(a["a"], a["b"]), a["expected"], 2e-7, 1e-6, "add")
    assert_close(orc.mul(m["a"], m["b"]), m["expected"], 2e-7, 1e-6, "mul")


def test_silu():  # OperationTests.swift:24-27
    c = ops["silu"]
    assert_close(orc.silu(c["x"]), c["expected"], 1e-6, 1e-6, "silu")


def test_matmul():  # OperationTests.swift:29-33
    c = ops["matmul"]
    a = np.asarray(c["a"], np.float32).reshape(c["m"], c["k"])
    b = np.asarray(c["b"], np.float32).reshape(c["k"], c["n"])
    assert_close(orc.matmul(a, b), c["expected"], 2e-6, 1e-5, "matmul")


def test_linear_f32_f16():  # OperationTests.swift:35-46
    c = ops["linear"]
    x = np.asarray(c["x"], np.float32).reshape(c["m"], c["k"])
    w = np.asarray(c["w"], np.float32).reshape(c["n"], c["k"])
    assert_close(orc.linear(x, orc.F32, w, c["n"]), c["expected"], 5e-6, 1e-5, "linear f32")
    wh = orc.encode(w, orc.F16)
    assert_close(orc.linear(x, orc.F16, wh, c["n"]), c["expected_f16"], 5e-6, 1e-5, "linear f16")
    assert_close(orc.linear(x[:1], orc.F32, w, c["n"]), c["expected"][: c["n"]], 5e-6, 1e-5, "matvec f32")


def test_rmsnorm():  # OperationTests.swift:48-53
    c = ops["rmsnorm"]
    x = np.asarray(c["x"], np.float32).reshape(c["shape"])
    assert_close(orc.rmsnorm(x, c["w"], c["eps"]), c["expected"], 2e-6, 2e-6, "rmsnorm")


def test_softmax():  # OperationTests.swift:55-61
    c = ops["softmax"]
    x = np.asarray(c["x"], np.float32).reshape(c["shape"])
    r = orc.softmax(x)
    assert_close(r, c["expected"], 1e-6, 1e-5, "softmax")
    np.testing.assert_allclose(r.reshape(-1, c["shape"][-1]).sum(1), 1.0, atol=1e-6)


def test_rope_both_conventions():  # OperationTests.swift:63-70
    c = ops["rope"]
    x = np.asarray(c["x"], np.float32).reshape(c["shape"])
    assert_close(orc.rope(x, c["start"], c["theta"], True), c["expected_interleaved"], 2e-6, 0, "rope interleaved")
    assert_close(orc.rope(x, c["start"], c["theta"], False), c["expected_split"], 2e-6, 0, "rope split")


def test_causal_gqa_attention():  # OperationTests.swift:72-86
    c = ops["attention"]
    t, h, kv, hd, cap = c["tokens"], c["heads"], c["kvHeads"], c["headDim"], c["capacity"]
    q = np.asarray(c["q"], np.float32).reshape(t, h, hd)
    k = np.asarray(c["k"], np.float32).reshape(cap, kv, hd)
    v = np.asarray(c["v"], np.float32).reshape(cap, kv, hd)
    s = orc.attention_scores(q, k, c["length"], c["start"])
    for hh in range(h):
        for tt in range(t):
            for p in range(c["length"]):
                assert (s[hh, tt, p] == -np.inf) == (p > c["start"] + tt)
    out = orc.attention_apply(orc.softmax(s), v)
    assert_close(out, c["expected"], 3e-6, 1e-5, "attention")
    assert_close(orc.attention(q, k, v, c["start"], c["length"]), c["expected"], 3e-6, 1e-5, "attention fused")


@pytest.mark.parametrize("name", ["q8_0", "q4_0"])
def test_quantized_formats_against_gguf(name):  # OperationTests.swift:88-108
    c = ops[name]
    dt = orc.DTYPES[name]
    raw = b64(c["blocks"])
    k, n, m = c["k"], c["n"], c["m"]
    assert raw.size == n * k // 32 * orc.BLOCK_BYTES[dt]
    deq = orc.dequantize(dt, raw, n * k)
    # dequantisation is exact: products of an f16 scale and a small integer
    assert np.array_equal(deq.astype(np.float64), np.asarray(c["dequantized"], np.float64)), f"{name} dequant"
    x = np.asarray(c["x"], np.float32).reshape(m, k)
    assert_close(orc.linear(x, dt, raw, n), c["expected"], 2e-5, 1e-5, f"{name} linear")
    mine = orc.quantize(c["original"], dt)
    assert mine.tobytes() == raw.tobytes(), f"{name} quantiser differs from gguf reference"


def test_embedding():  # OperationTests.swift:110-116
    c = ops["embedding"]
    table = np.asarray(c["table"], np.float32).reshape(c["vocab"], c["dim"])
    out = orc.embed(c["tokens"], orc.F32, table, c["vocab"], c["dim"])
    assert np.array_equal(out.ravel().astype(np.float64), np.asarray(c["expected"], np.float64))
    with pytest.raises(IndexError):
        orc.embed([12], orc.F32, table, c["vocab"], c["dim"])
    with pytest.raises(IndexError):
        orc.embed([-1], orc.F32, table, c["vocab"], c["dim"])


# ---------------------------------------------------------------- closed forms


def test_half_conversion_exhaustive():
    """Every binary16 value converts exactly; float->half is round-to-nearest-even."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    mine = np.array([orc.half_to_float(int(b)) for b in bits], np.float32)
    finite = ~np.isnan(ref)
    assert np.array_equal(mine[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.isnan(mine[~finite]).all()
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
        # halfway cases between adjacent halves: ties must go to even
        (ref[finite & (np.abs(ref) < 60000)].astype(np.float64)
         + np.spacing(ref[finite & (np.abs(ref) < 60000)]).astype(np.float64) / 2).astype(np.float32),
        np.array([65504, 65519, 65520, 1e9, -1e9, 6e-8, 2.9e-8, 3e-8, 0.0, -0.0], np.float32),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref_h = vals.astype(np.float16).view(np.uint16)
    mine_h = np.array([orc.float_to_half(float(v)) for v in vals], np.uint16)
    assert np.array_equal(mine_h, ref_h)


def test_splitmix64_published_vectors():
    """SplitMix64 (Vigna) with seed 0 starts 0xe220a8397b1dcdaf, 0x6e789e6aa1b965f4, ..."""
    g = orc.SplitMix64(0)
    assert [g.next() for _ in range(3)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_q4_0_nibble_order_closed_form():
    """Byte j: low nibble -> element j, high nibble -> element j+16; value = d*(nib-8)."""
    d = np.float16(0.5).view(np.uint16)
    qs = np.array([(j & 0xF) | (((15 - j) & 0xF) << 4) for j in range(16)], np.uint8)
    block = np.concatenate([np.frombuffer(np.uint16(d).tobytes(), np.uint8), qs])
    out = orc.dequantize(orc.Q4_0, block, 32)
    expect = np.array([0.5 * (j - 8) for j in range(16)] + [0.5 * ((15 - j) - 8) for j in range(16)], np.float32)
    assert np.array_equal(out, expect)
    q8 = np.concatenate([np.frombuffer(np.uint16(d).tobytes(), np.uint8), np.arange(-16, 16, dtype=np.int8).view(np.uint8)])
    assert np.array_equal(orc.dequantize(orc.Q8_0, q8, 32), 0.5 * np.arange(-16, 16, dtype=np.float32))


def test_quantize_round_trip_bounds():
    """|dequant(quant(v)) - v| <= d/2 (Q8_0) and <= d (Q4_0, clamp at nibble 15), plus the
    f16 rounding of the stored scale (<= 127 * 2^-11 * d)."""
    rng = np.random.default_rng(3)
    v = rng.standard_normal(32 * 64).astype(np.float32)
    for dt, lim in ((orc.Q8_0, 0.5), (orc.Q4_0, 1.0)):
        raw = orc.quantize(v, dt)
        back = orc.dequantize(dt, raw, v.size)
        bb = orc.BLOCK_BYTES[dt]
        d = np.array([abs(orc.half_to_float(int(raw[b * bb]) | (int(raw[b * bb + 1]) << 8))) for b in range(64)])
        err = np.abs(back - v).reshape(64, 32).max(1)
        assert (err <= (lim + 127 * 2.0 ** -11) * d + 1e-7).all()


def test_rope_preserves_pair_norms_and_position_zero_is_identity():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 4, 16)).astype(np.float32)
    assert np.array_equal(orc.rope(x[:1], 0, 1e4, True), x[:1])
    for inter in (True, False):
        y = orc.rope(x, 100, 1e5, inter)
        if inter:
            nx = np.hypot(x[..., 0::2], x[..., 1::2]); ny = np.hypot(y[..., 0::2], y[..., 1::2])
        else:
            nx = np.hypot(x[..., :8], x[..., 8:]); ny = np.hypot(y[..., :8], y[..., 8:])
        np.testing.assert_allclose(ny, nx, rtol=1e-6, atol=1e-6)
    # pair 0 rotates by exactly `position` radians (freq = theta^0 = 1)
    y = orc.rope(x, 5, 1e4, True)
    c, s = np.cos(5.0), np.sin(5.0)
    np.testing.assert_allclose(y[0, :, 0], x[0, :, 0] * c - x[0, :, 1] * s, rtol=1e-6, atol=1e-6)


def test_attention_brute_force_float64():
    """Attention against a float64 brute force with GQA grouping and causal start offset."""
    rng = np.random.default_rng(2)
    t, h, kv, hd, start = 4, 6, 2, 16, 3
    q = rng.standard_normal((t, h, hd)).astype(np.float32)
    k = rng.standard_normal((start + t, kv, hd)).astype(np.float32)
    v = rng.standard_normal((start + t, kv, hd)).astype(np.float32)
    out = orc.attention(q, k, v, start)
    ref = np.zeros((t, h, hd))
    for tt in range(t):
        for hh in range(h):
            g = hh // (h // kv)
            s = (k[: start + tt + 1, g].astype(np.float64) @ q[tt, hh].astype(np.float64)) / np.sqrt(hd)
            p = np.exp(s - s.max()); p /= p.sum()
            ref[tt, hh] = p @ v[: start + tt + 1, g]
    assert_close(out, ref, 2e-6, 1e-5, "attention brute force")


def test_argmax_ties_and_nan():  # Sampler.swift:100-108, SamplerTests.swift:17-20
    assert orc.argmax([1, 3, 3, 2]) == 1
    assert orc.argmax([-np.inf, -np.inf]) == 0
    assert orc.argmax([0.5]) == 0
    with pytest.raises(ValueError):
        orc.argmax([1.0, np.nan, 2.0])


def test_linear_matches_dequantized_float64():
    """Quantised linear equals float64 x . dequant(W)^T up to f32 accumulation, for all formats."""
    rng = np.random.default_rng(4)
    k, n, m = 256, 19, 3
    w = (rng.standard_normal((n, k)) * 0.3).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    for dt in (orc.F32, orc.F16, orc.Q8_0, orc.Q4_0):
        raw = orc.encode(w, dt)
        deq = orc.dequantize(dt, raw, n * k).reshape(n, k).astype(np.float64)
        assert_close(orc.linear(x, dt, raw, n), x.astype(np.float64) @ deq.T, 2e-5, 1e-5, f"linear dt={dt}")
