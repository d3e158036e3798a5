"""The thin HIP shim of the C ABI (the surface a Swift C target wraps:
streams, events, pinned host memory, asynchronous copies, code-object modules
and their launch), exercised end to end on the device with the library's own
test code object (alpaca_amd/shim_kernels.hsaco).  Error statuses follow
MetalError: a missing kernel is AHIP_ERR_MISSING_KERNEL (missingFunction), an
unreadable code object AHIP_ERR_MODULE_LOAD (shaderCompilation)."""
import ctypes as C

import numpy as np
import pytest

from alpaca_amd import _lib as L

pytestmark = pytest.mark.gpu


def ok(rc):
    L.check(rc)


def test_stream_event_copy_and_module_launch(hip_ctx):
    lib, ctx = L.lib(), hip_ctx.handle
    n = 100_003  # not a multiple of the block
    x = (np.arange(n, dtype=np.float32) * np.float32(0.25)) - np.float32(7.0)
    y = np.cos(np.arange(n, dtype=np.float32)).astype(np.float32)
    nbytes = n * 4
    st, e0, e1, mod = C.c_void_p(), C.c_void_p(), C.c_void_p(), C.c_void_p()
    hx, hy, dx, dy, dz = (C.c_void_p() for _ in range(5))
    ok(lib.ahip_stream_create(ctx, C.byref(st)))
    ok(lib.ahip_event_create(ctx, C.byref(e0)))
    ok(lib.ahip_event_create(ctx, C.byref(e1)))
    for h in (hx, hy):
        ok(lib.ahip_host_alloc(ctx, nbytes, C.byref(h)))
    for d in (dx, dy, dz):
        ok(lib.ahip_malloc(ctx, nbytes, C.byref(d)))
    try:
        C.memmove(hx, x.ctypes.data, nbytes)
        C.memmove(hy, y.ctypes.data, nbytes)
        ok(lib.ahip_memcpy_htod_async(dx, hx, nbytes, st))
        ok(lib.ahip_memcpy_htod_async(dy, hy, nbytes, st))
        ok(lib.ahip_module_load(ctx, L.SHIM_CODE_OBJECT.encode(), C.byref(mod)))
        found = C.c_int(-1)
        ok(lib.ahip_module_has_kernel(mod, b"ahip_shim_axpy", C.byref(found)))
        assert found.value == 1
        ok(lib.ahip_module_has_kernel(mod, b"no_such_kernel", C.byref(found)))
        assert found.value == 0
        # y = 2 x + y: a power-of-two scale keeps the product exact, so fused and
        # unfused evaluation agree with numpy bit for bit
        a, cnt = C.c_float(2.0), C.c_int(n)
        args = (C.c_void_p * 4)(*(C.cast(C.pointer(v), C.c_void_p) for v in (a, dx, dy, cnt)))
        grid = (C.c_uint32 * 3)((n + 255) // 256, 1, 1)
        block = (C.c_uint32 * 3)(256, 1, 1)
        ok(lib.ahip_event_record(e0, st))
        ok(lib.ahip_module_launch(mod, b"ahip_shim_axpy", grid, block, 0, st, args))
        ok(lib.ahip_event_record(e1, st))
        ok(lib.ahip_memcpy_dtod_async(dz, dy, nbytes, st))
        ok(lib.ahip_memcpy_dtoh_async(hy, dz, nbytes, st))
        ok(lib.ahip_stream_synchronize(st))
        ok(lib.ahip_event_synchronize(e1))
        ms = C.c_float(-1)
        ok(lib.ahip_event_elapsed_ms(e0, e1, C.byref(ms)))
        assert 0.0 <= ms.value < 1000.0
        got = np.frombuffer((C.c_char * nbytes).from_address(hy.value), dtype=np.float32).copy()
        assert np.array_equal(got, np.float32(2.0) * x + y)
        # a second kernel of the module, ordered after an event on another stream
        st2 = C.c_void_p()
        ok(lib.ahip_stream_create(ctx, C.byref(st2)))
        ok(lib.ahip_event_record(e0, st))
        ok(lib.ahip_stream_wait_event(st2, e0))
        val = C.c_uint32(0xA1CA9A)
        fargs = (C.c_void_p * 3)(*(C.cast(C.pointer(v), C.c_void_p) for v in (dz, val, cnt)))
        ok(lib.ahip_module_launch(mod, b"ahip_shim_fill_u32", grid, block, 0, st2, fargs))
        ok(lib.ahip_memcpy_dtoh_async(hx, dz, nbytes, st2))
        ok(lib.ahip_stream_synchronize(st2))
        filled = np.frombuffer((C.c_char * nbytes).from_address(hx.value), dtype=np.uint32)
        assert (filled == 0xA1CA9A).all()
        ok(lib.ahip_stream_destroy(st2))
        # error statuses
        assert lib.ahip_module_launch(mod, b"no_such_kernel", grid, block, 0, st, args) == L.MISSING_KERNEL
        bad_grid = (C.c_uint32 * 3)(0, 1, 1)
        assert lib.ahip_module_launch(mod, b"ahip_shim_axpy", bad_grid, block, 0, st, args) == L.INVALID_ARGUMENT
        m2 = C.c_void_p()
        assert lib.ahip_module_load(ctx, b"/nonexistent/code.hsaco", C.byref(m2)) == L.MODULE_LOAD
        # the same code object from memory
        image = open(L.SHIM_CODE_OBJECT, "rb").read()
        buf = C.create_string_buffer(image, len(image))
        ok(lib.ahip_module_load_data(ctx, buf, C.byref(m2)))
        ok(lib.ahip_module_has_kernel(m2, b"ahip_shim_fill_u32", C.byref(found)))
        assert found.value == 1
        ok(lib.ahip_module_unload(m2))
        # the failures above leave no stale HIP error behind: the library's own
        # launches (which read the last HIP error) still succeed
        assert lib.ahip_module_load(ctx, b"/nonexistent/code.hsaco", C.byref(m2)) == L.MODULE_LOAD
        from alpaca_amd.ops import HIPOps
        a = np.arange(1000, dtype=np.float32)
        assert np.array_equal(HIPOps(hip_ctx).add(a, a), a + a)
    finally:
        if mod:
            lib.ahip_module_unload(mod)
        for d in (dx, dy, dz):
            lib.ahip_free(ctx, d)
        for h in (hx, hy):
            lib.ahip_host_free(ctx, h)
        lib.ahip_event_destroy(e0)
        lib.ahip_event_destroy(e1)
        lib.ahip_stream_destroy(st)
