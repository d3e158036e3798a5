"""ctypes binding of libalpaca_hip.so (include/alpaca_hip.h).

The library is loaded from this package directory.  There is no fallback: a
missing library, or one that fails to load, raises ``BackendUnavailable``.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libalpaca_hip.so")
# the shim's test code object (ahip_module_load)
SHIM_CODE_OBJECT = os.path.join(HERE, "shim_kernels.hsaco")

OK, NO_DEVICE, MODULE_LOAD, MISSING_KERNEL, ALLOC, COMMAND_FAILED, UNSUPPORTED, INVALID_ARGUMENT, BUSY, GGUF = range(10)
F32, F16, Q8_0, Q4_0 = 0, 1, 2, 3
KV_F16, KV_F32 = 0, 1
GEMM_EXACT, GEMM_FAST, GEMM_FAST_F16 = 0, 1, 2

STATUS_NAMES = {
    NO_DEVICE: "no device", MODULE_LOAD: "module load", MISSING_KERNEL: "missing kernel", ALLOC: "allocation",
    COMMAND_FAILED: "command failed", UNSUPPORTED: "unsupported", INVALID_ARGUMENT: "invalid argument", BUSY: "busy",
    GGUF: "gguf",
}
# GGUFError cases (ahip_gguf_error), Sources/AlpacaModels/GGUF/GGUFError.swift:5-19.
GGUF_KINDS = {1: "cannotOpen", 2: "invalidMagic", 3: "unsupportedVersion", 4: "bigEndianNotSupported", 5: "truncated",
              6: "malformed", 7: "limitExceeded", 8: "unsupportedTensorType", 9: "duplicateTensor",
              10: "missingMetadata", 11: "missingTensor", 12: "unsupportedModel", 13: "tensorOutOfRange",
              14: "tensorsOverlap"}


class BackendUnavailable(RuntimeError):
    """The HIP library is missing or cannot be loaded."""


class HIPError(RuntimeError):
    """A non-zero ahip_status (MetalError in the reference)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {message}")
        self.code = code


class InvalidArgument(HIPError, ValueError):
    pass


class GGUFError(HIPError):
    """AHIP_ERR_GGUF; ``kind`` names the GGUFError case (GGUF_KINDS)."""

    def __init__(self, code: int, message: str, kind: str):
        super().__init__(code, message)
        self.kind = kind


class Unsupported(HIPError):
    pass


class Busy(HIPError):
    pass


class LlamaConfigC(C.Structure):
    _fields_ = [
        ("vocab_size", C.c_int32), ("hidden_size", C.c_int32), ("layer_count", C.c_int32),
        ("head_count", C.c_int32), ("kv_head_count", C.c_int32), ("head_dim", C.c_int32),
        ("feed_forward_size", C.c_int32), ("context_length", C.c_int32),
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float), ("rope_interleaved", C.c_int32),
    ]


class TensorDescC(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_int32), ("rows", C.c_int64), ("cols", C.c_int64),
                ("data", C.c_void_p), ("bytes", C.c_int64)]


class GGUFTensorC(C.Structure):
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_int32), ("dims", C.c_int64 * 4), ("type", C.c_uint32),
                ("file_offset", C.c_int64), ("byte_count", C.c_int64), ("data", C.c_void_p)]


class LoadReportC(C.Structure):
    _fields_ = [("mapped_weight_bytes", C.c_int64), ("converted_weight_bytes", C.c_int64),
                ("converted_tensors", C.c_int32), ("notes", C.c_char * 2048)]


class StageC(C.Structure):
    _fields_ = [("label", C.c_char * 48), ("seconds", C.c_double), ("dispatches", C.c_int32)]


EMIT_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int32)

vp, fp, ip, dp = C.c_void_p, C.POINTER(C.c_float), C.POINTER(C.c_int32), C.POINTER(C.c_double)
i64, i64p, i = C.c_int64, C.POINTER(C.c_int64), C.c_int

SIGNATURES = {
    "ahip_last_error": (C.c_char_p, []),
    "ahip_device_count": (i, [C.POINTER(C.c_int)]),
    "ahip_version": (C.c_char_p, []),
    "ahip_context_create": (i, [i, C.POINTER(vp)]),
    "ahip_context_destroy": (i, [vp]),
    "ahip_model_create": (i, [vp, C.POINTER(LlamaConfigC), C.POINTER(TensorDescC), i, i, C.POINTER(vp)]),
    "ahip_model_destroy": (i, [vp]),
    "ahip_model_weight_bytes": (i, [vp, i64p]),
    "ahip_model_prefill_cache_bytes": (i, [vp, i64p]),
    "ahip_session_byte_count": (i, [C.POINTER(LlamaConfigC), i, i, i, i64p]),
    "ahip_gguf_last_error_kind": (i, []),
    "ahip_gguf_open": (i, [C.c_char_p, C.POINTER(vp)]),
    "ahip_gguf_open_memory": (i, [vp, i64, C.POINTER(vp)]),
    "ahip_gguf_close": (i, [vp]),
    "ahip_gguf_header": (i, [vp, C.POINTER(C.c_uint32), i64p, i64p, i64p]),
    "ahip_gguf_meta_count": (i, [vp, C.POINTER(C.c_int)]),
    "ahip_gguf_meta_key": (i, [vp, i, C.POINTER(C.c_char_p), C.POINTER(C.c_uint32)]),
    "ahip_gguf_meta_int": (i, [vp, C.c_char_p, i64, i64p]),
    "ahip_gguf_meta_uint": (i, [vp, C.c_char_p, i64, C.POINTER(C.c_uint64)]),
    "ahip_gguf_meta_float": (i, [vp, C.c_char_p, i64, dp]),
    "ahip_gguf_meta_bool": (i, [vp, C.c_char_p, i64, C.POINTER(C.c_int)]),
    "ahip_gguf_meta_string": (i, [vp, C.c_char_p, i64, C.POINTER(C.c_void_p), i64p]),
    "ahip_gguf_meta_array": (i, [vp, C.c_char_p, C.POINTER(C.c_uint32), i64p]),
    "ahip_gguf_tensor_count": (i, [vp, C.POINTER(C.c_int)]),
    "ahip_gguf_tensor_at": (i, [vp, i, C.POINTER(GGUFTensorC)]),
    "ahip_gguf_find_tensor": (i, [vp, C.c_char_p, C.POINTER(C.c_int)]),
    "ahip_gguf_llama_config": (i, [vp, C.POINTER(LlamaConfigC)]),
    "ahip_model_load_gguf": (i, [vp, vp, i, C.POINTER(vp), C.POINTER(LlamaConfigC), C.POINTER(LoadReportC)]),
    "ahip_session_create": (i, [vp, i, i, i, i, C.POINTER(vp)]),
    "ahip_session_destroy": (i, [vp]),
    "ahip_session_forward": (i, [vp, ip, i, C.POINTER(fp)]),
    "ahip_session_decode": (i, [vp, C.c_int32, C.POINTER(fp)]),
    "ahip_session_decode_greedy": (i, [vp, C.c_int32, i, i, EMIT_FN, vp, C.POINTER(C.c_int)]),
    "ahip_session_reset": (i, [vp]),
    "ahip_session_length": (i, [vp, C.POINTER(C.c_int)]),
    "ahip_session_capacity": (i, [vp, C.POINTER(C.c_int)]),
    "ahip_session_last_gpu_seconds": (i, [vp, dp]),
    "ahip_session_last_encode_seconds": (i, [vp, dp]),
    "ahip_session_set_profiling": (i, [vp, i]),
    "ahip_session_profile": (i, [vp, C.POINTER(StageC), i, C.POINTER(C.c_int)]),
    "ahip_session_decode_timeline": (i, [vp, C.POINTER(C.c_uint64), i64, i64p, C.POINTER(C.c_int), dp]),
    "ahip_op_add": (i, [vp, fp, fp, i64, fp]),
    "ahip_op_mul": (i, [vp, fp, fp, i64, fp]),
    "ahip_op_silu": (i, [vp, fp, i64, fp]),
    "ahip_op_silu_mul": (i, [vp, fp, fp, i64, fp]),
    "ahip_op_rmsnorm": (i, [vp, fp, fp, i, i, C.c_float, fp]),
    "ahip_op_linear": (i, [vp, fp, i, i, i, vp, i, i, fp]),
    "ahip_op_linear_add": (i, [vp, fp, i, i, i, vp, i, i, fp]),
    "ahip_op_gate_up_silu": (i, [vp, fp, i, i, i, vp, vp, i, i, fp]),
    "ahip_op_rope": (i, [vp, fp, i, i, i, i, C.c_float, i]),
    "ahip_op_attention": (i, [vp, fp, i, i, i, fp, fp, i, i, i, i, i, fp]),
    "ahip_op_embed": (i, [vp, ip, i, i, vp, i, i, fp]),
    "ahip_op_dequantize": (i, [vp, i, vp, i64, fp]),
    "ahip_op_argmax": (i, [vp, fp, i, ip]),
    "ahip_op_sample": (i, [vp, fp, i, C.c_float, i, C.c_float, C.c_double, ip]),
    "ahip_session_sample": (i, [vp, C.c_float, i, C.c_float, C.c_double, ip]),
    "ahip_attention_decode_noalloc": (i, [vp, vp, vp, vp, i, i, i, i, i, i, vp, vp]),
    "ahip_quantize": (i, [i, fp, i64, vp]),
    "ahip_synth_uniform": (i, [C.c_uint64, C.c_uint64, i64, C.c_float, C.c_float, fp]),
    "ahip_synth_normal": (i, [C.c_uint64, C.c_uint64, i64, C.c_float, fp]),
    "ahip_synth_ints": (i, [C.c_uint64, C.c_uint64, i64, C.c_uint64, i64, ip]),
    "ahip_malloc": (i, [vp, i64, C.POINTER(vp)]),
    "ahip_free": (i, [vp, vp]),
    "ahip_memcpy_htod": (i, [vp, vp, vp, i64]),
    "ahip_memcpy_dtoh": (i, [vp, vp, vp, i64]),
    "ahip_memset": (i, [vp, vp, i, i64]),
    "ahip_synchronize": (i, [vp]),
    "ahip_stream_create": (i, [vp, C.POINTER(vp)]),
    "ahip_stream_destroy": (i, [vp]),
    "ahip_stream_synchronize": (i, [vp]),
    "ahip_stream_wait_event": (i, [vp, vp]),
    "ahip_event_create": (i, [vp, C.POINTER(vp)]),
    "ahip_event_destroy": (i, [vp]),
    "ahip_event_record": (i, [vp, vp]),
    "ahip_event_synchronize": (i, [vp]),
    "ahip_event_elapsed_ms": (i, [vp, vp, fp]),
    "ahip_host_alloc": (i, [vp, i64, C.POINTER(vp)]),
    "ahip_host_free": (i, [vp, vp]),
    "ahip_memcpy_htod_async": (i, [vp, vp, i64, vp]),
    "ahip_memcpy_dtoh_async": (i, [vp, vp, i64, vp]),
    "ahip_memcpy_dtod_async": (i, [vp, vp, i64, vp]),
    "ahip_module_load": (i, [vp, C.c_char_p, C.POINTER(vp)]),
    "ahip_module_load_data": (i, [vp, vp, C.POINTER(vp)]),
    "ahip_module_unload": (i, [vp]),
    "ahip_module_has_kernel": (i, [vp, C.c_char_p, C.POINTER(C.c_int)]),
    "ahip_module_launch": (i, [vp, C.c_char_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.c_uint32, vp,
                               C.POINTER(vp)]),
    "ahip_dev_pack_weight": (i, [vp, i, vp, i, i, C.POINTER(vp)]),
    "ahip_dev_weight_free": (i, [vp, vp]),
    "ahip_dev_gemv": (i, [vp, vp, vp, vp, i, dp]),
    "ahip_dev_gemm": (i, [vp, vp, vp, i, vp, i, i, dp]),
    "ahip_dev_attention": (i, [vp, vp, vp, vp, i, i, i, i, i, vp, i, dp]),
    "ahip_dev_gemv_cycle": (i, [vp, C.POINTER(vp), i, vp, vp, i, dp]),
    "ahip_dev_attention_decode": (i, [vp, vp, vp, vp, i, i, i, i, i, vp, i, dp]),
}

_lib = None


def lib():
    """The loaded library; raises BackendUnavailable when it is absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise BackendUnavailable(f"{LIB_PATH} is missing: build it with `python -m alpaca_amd.build`")
        try:
            L = C.CDLL(LIB_PATH)
        except OSError as e:
            raise BackendUnavailable(f"cannot load {LIB_PATH}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc == OK:
        return
    msg = lib().ahip_last_error().decode(errors="replace")
    if rc == INVALID_ARGUMENT:
        raise InvalidArgument(rc, msg)
    if rc == UNSUPPORTED:
        raise Unsupported(rc, msg)
    if rc == BUSY:
        raise Busy(rc, msg)
    if rc == GGUF:
        raise GGUFError(rc, msg, GGUF_KINDS.get(lib().ahip_gguf_last_error_kind(), "unknown"))
    raise HIPError(rc, msg)
