"""ahip_attention_decode_noalloc: the single-query split-K attention of
ahip_op_attention on device buffers with its split partials in a fixed device
array (no allocation).  Held to ahip_op_attention (the entry point whose
kernels it shares) bit for bit on two calls in a row, the second smaller than
the first, so a stale partial left in the shared array by the first call
would show; and a shape past the array's size is refused."""
import ctypes as C

import numpy as np
import pytest

from alpaca_amd import _lib as L
from alpaca_amd.ops import HIPOps

pytestmark = pytest.mark.gpu


def splitmix_normal(seed, n):
    rng = np.random.default_rng(seed)
    return rng.standard_normal(n).astype(np.float32)


def device(ctx, arr):
    p = C.c_void_p()
    L.check(L.lib().ahip_malloc(ctx, arr.nbytes, C.byref(p)))
    L.check(L.lib().ahip_memcpy_htod(ctx, p, arr.ctypes.data, arr.nbytes))
    return p


def run_noalloc(hip_ctx, q, k, v, length, kv_precision):
    """q [heads, hd]; k/v [capacity, kv_heads, hd] float32 (as ahip_op_attention takes them)."""
    lib, ctx = L.lib(), hip_ctx.handle
    cap, kvh, hd = k.shape
    heads = q.shape[0]
    dt = np.float16 if kv_precision == L.KV_F16 else np.float32
    # the session cache layout [kv_heads][capacity][hd]
    kc = np.ascontiguousarray(k.transpose(1, 0, 2)).astype(dt)
    vc = np.ascontiguousarray(v.transpose(1, 0, 2)).astype(dt)
    dq, dk, dv = device(ctx, np.ascontiguousarray(q)), device(ctx, kc), device(ctx, vc)
    dout = C.c_void_p()
    out = np.empty(heads * hd, np.float32)
    try:
        L.check(lib.ahip_malloc(ctx, out.nbytes, C.byref(dout)))
        L.check(lib.ahip_attention_decode_noalloc(ctx, dq, dk, dv, kv_precision, cap, heads, kvh, hd, length, dout,
                                                  None))
        L.check(lib.ahip_synchronize(ctx))
        L.check(lib.ahip_memcpy_dtoh(ctx, out.ctypes.data, dout, out.nbytes))
    finally:
        for p in (dq, dk, dv, dout):
            lib.ahip_free(ctx, p)
    return out.reshape(heads, hd)


@pytest.mark.parametrize("kv", ["f16", "f32"])
def test_noalloc_decode_attention_matches_op_attention(hip_ctx, kv):
    ops = HIPOps(hip_ctx)
    kvp = L.KV_F16 if kv == "f16" else L.KV_F32
    # two calls in a row, the second with a smaller input (fewer heads, a shorter context)
    for i, (cap, heads, kvh, hd, length) in enumerate([(4200, 32, 8, 128, 4100), (700, 9, 3, 64, 513)]):
        q = splitmix_normal(10 * i + 1, heads * hd).reshape(heads, hd)
        k = splitmix_normal(10 * i + 2, cap * kvh * hd).reshape(cap, kvh, hd)
        v = splitmix_normal(10 * i + 3, cap * kvh * hd).reshape(cap, kvh, hd)
        got = run_noalloc(hip_ctx, q, k, v, length, kvp)
        # ahip_op_attention: one query at position length - 1 over rows 0..length-1
        want = ops.attention(q.reshape(1, heads, hd), k, v, length - 1, kv).reshape(heads, hd)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
            f"call {i}: max |d| {np.abs(got - want).max():.3e}"


def test_noalloc_refuses_shapes_past_its_scratch(hip_ctx):
    lib, ctx = L.lib(), hip_ctx.handle
    p = C.c_void_p()
    L.check(lib.ahip_malloc(ctx, 1 << 20, C.byref(p)))
    try:
        # 256 heads x 32 splits (of 256 positions) x 130 floats > the 2.5 MiB array: refused before any launch
        rc = lib.ahip_attention_decode_noalloc(ctx, p, p, p, L.KV_F16, 8192, 256, 32, 128, 8192, p, None)
        assert rc == L.INVALID_ARGUMENT
        assert b"scratch" in lib.ahip_last_error()
        # length past the capacity
        assert lib.ahip_attention_decode_noalloc(ctx, p, p, p, L.KV_F16, 100, 8, 8, 64, 101, p, None) == \
            L.INVALID_ARGUMENT
    finally:
        lib.ahip_free(ctx, p)
