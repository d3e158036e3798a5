"""Host-side mirror of the reference's GPU model/session API over the C ABI.

``HIPLlamaModel`` / ``HIPLlamaSession`` follow ``MetalLlamaModel`` /
``MetalLlamaSession`` (Sources/AlpacaMetal/Backend/MetalLlamaModel.swift) and
the ``InferenceSession`` protocol (Sources/Alpaca/LanguageModel.swift:317-328):
same method names (snake_case), argument meaning and error behaviour.
"""
from __future__ import annotations

import atexit
import ctypes as C
import weakref
from dataclasses import dataclass, field

import numpy as np

from . import _lib as L
from .tensor import QTensor

# Handles still open when the interpreter exits are closed by an atexit hook
# (sessions, then models, then contexts), which runs at the start of
# interpreter finalization, while the library and the HIP runtime are intact.
# Left to finalizers at module teardown they may not be released at all, and
# the HIP runtime then frees the session's streams, events and mapped host
# words in its own exit handlers, after an attached profiler (rocprofv3) has
# finalized the API tables it intercepts.
_LIVE: "weakref.WeakSet" = weakref.WeakSet()


def close_all() -> None:
    """Closes every session, model and context still open, in that order."""
    for kind in ("session", "model", "context"):
        for obj in list(_LIVE):
            if getattr(obj, "_kind", None) == kind:
                obj.close()


atexit.register(close_all)


class HIPContext:
    """MetalContext equivalent: binds one HIP device (MetalContext.swift:37-126)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        L.check(L.lib().ahip_context_create(device, C.byref(h)))
        self.handle = h
        self.device = device
        self._kind = "context"
        _LIVE.add(self)

    @staticmethod
    def is_available() -> bool:
        n = C.c_int(0)
        L.check(L.lib().ahip_device_count(C.byref(n)))
        return n.value > 0

    def close(self) -> None:
        if getattr(self, "handle", None):
            L.lib().ahip_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()


@dataclass
class LlamaConfig:
    """LlamaConfig.swift:8-20."""
    vocab_size: int
    hidden_size: int
    layer_count: int
    head_count: int
    kv_head_count: int
    head_dim: int
    feed_forward_size: int
    context_length: int
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    rope_interleaved: bool = True

    @property
    def query_width(self) -> int:
        return self.head_count * self.head_dim

    @property
    def kv_width(self) -> int:
        return self.kv_head_count * self.head_dim

    def to_c(self) -> L.LlamaConfigC:
        return L.LlamaConfigC(self.vocab_size, self.hidden_size, self.layer_count, self.head_count,
                              self.kv_head_count, self.head_dim, self.feed_forward_size, self.context_length,
                              self.rms_norm_eps, self.rope_theta, 1 if self.rope_interleaved else 0)


KV = {"f16": L.KV_F16, "f32": L.KV_F32}
GEMM = {"exact": L.GEMM_EXACT, "fast": L.GEMM_FAST, "fast-f16": L.GEMM_FAST_F16}


class HIPLlamaModel:
    """Weights resident in HBM, shared read-only by any number of sessions.

    ``weights`` maps GGUF tensor names (LlamaLoader.swift) to ``QTensor``; a
    missing "output" means tied embeddings.  Host buffers may be dropped after
    construction: the model owns its HBM copies."""

    def __init__(self, context: HIPContext, config: LlamaConfig, weights: dict, prefill_weight_cache: bool = False):
        self.context = context
        self.config = config
        names, descs = [], []
        for name, t in weights.items():
            assert isinstance(t, QTensor), name
            nb = name.encode()
            names.append(nb)
            descs.append(L.TensorDescC(nb, t.dtype, t.rows, t.cols, t.data.ctypes.data, t.data.nbytes))
        arr = (L.TensorDescC * len(descs))(*descs)
        h = C.c_void_p()
        cfg = config.to_c()
        L.check(L.lib().ahip_model_create(context.handle, C.byref(cfg), arr, len(descs),
                                          1 if prefill_weight_cache else 0, C.byref(h)))
        self.handle = h
        self._kind = "model"
        _LIVE.add(self)

    @property
    def weight_bytes(self) -> int:
        v = C.c_int64()
        L.check(L.lib().ahip_model_weight_bytes(self.handle, C.byref(v)))
        return v.value

    @property
    def prefill_cache_bytes(self) -> int:
        """Bytes of the f16 prefill weight copies (MetalLlamaModel.prefillCacheBytes)."""
        v = C.c_int64()
        L.check(L.lib().ahip_model_prefill_cache_bytes(self.handle, C.byref(v)))
        return v.value

    @staticmethod
    def session_byte_count(config: LlamaConfig, capacity: int, max_batch: int, kv_precision: str = "f16") -> int:
        v = C.c_int64()
        cfg = config.to_c()
        L.check(L.lib().ahip_session_byte_count(C.byref(cfg), capacity, max_batch, KV[kv_precision], C.byref(v)))
        return v.value

    def make_session(self, capacity: int | None = None, max_batch: int = 512, kv_precision: str = "f16",
                     gemm_precision: str = "fast") -> "HIPLlamaSession":
        cap = self.config.context_length if capacity is None else capacity
        return HIPLlamaSession(self, cap, max_batch, kv_precision, gemm_precision)

    def close(self) -> None:
        if getattr(self, "handle", None):
            L.lib().ahip_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()


@dataclass
class StageTime:
    seconds: float
    dispatches: int


class HIPLlamaSession:
    """One generation's state: KV cache, scratch and its own HIP stream."""

    def __init__(self, model: HIPLlamaModel, capacity: int, max_batch: int, kv_precision: str, gemm_precision: str):
        self.model = model
        self.kv_precision = kv_precision
        self.gemm_precision = gemm_precision
        h = C.c_void_p()
        L.check(L.lib().ahip_session_create(model.handle, capacity, max_batch, KV[kv_precision],
                                            GEMM[gemm_precision], C.byref(h)))
        self.handle = h
        self._kind = "session"
        _LIVE.add(self)
        self.gpu_seconds = 0.0  # accumulated, as MetalSessionAdapter.gpuSeconds

    # -- InferenceSession ---------------------------------------------------
    def forward(self, tokens) -> np.ndarray:
        """Appends tokens and returns the last position's logits (a copy)."""
        tok = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).ravel())
        p = L.fp()
        L.check(L.lib().ahip_session_forward(self.handle, tok.ctypes.data_as(L.ip), tok.size, C.byref(p)))
        self.gpu_seconds += self.last_gpu_seconds
        return np.ctypeslib.as_array(p, shape=(self.model.config.vocab_size,)).copy()

    def decode(self, token: int) -> np.ndarray:
        p = L.fp()
        L.check(L.lib().ahip_session_decode(self.handle, int(token), C.byref(p)))
        self.gpu_seconds += self.last_gpu_seconds
        return np.ctypeslib.as_array(p, shape=(self.model.config.vocab_size,)).copy()

    def decode_greedy(self, start_token: int, max_steps: int, emit, depth: int = 3) -> int:
        """GPU-resident greedy chain; ``emit(token) -> bool`` (False stops)."""
        err = []

        def cb(_user, token):
            try:
                return 1 if emit(int(token)) else 0
            except BaseException as e:  # noqa: BLE001 - re-raised below
                err.append(e)
                return 0

        fn = L.EMIT_FN(cb)
        fed = C.c_int(0)
        rc = L.lib().ahip_session_decode_greedy(self.handle, int(start_token), int(max_steps), int(depth), fn, None,
                                                C.byref(fed))
        self.gpu_seconds += self.last_gpu_seconds
        if err:
            raise err[0]
        L.check(rc)
        return fed.value

    def sample(self, temperature: float, top_k: int = 0, top_p: float = 1.0, u: float = 0.0) -> int:
        """Samples the last forward/decode logits on the device (ahip_session_sample)."""
        r = C.c_int32()
        L.check(L.lib().ahip_session_sample(self.handle, temperature, top_k, top_p, u, C.byref(r)))
        return r.value

    def reset(self) -> None:
        L.check(L.lib().ahip_session_reset(self.handle))
        self.gpu_seconds = 0.0

    # -- properties ---------------------------------------------------------
    def _int(self, fn) -> int:
        v = C.c_int()
        L.check(fn(self.handle, C.byref(v)))
        return v.value

    def _dbl(self, fn) -> float:
        v = C.c_double()
        L.check(fn(self.handle, C.byref(v)))
        return v.value

    @property
    def length(self) -> int:
        return self._int(L.lib().ahip_session_length)

    @property
    def capacity(self) -> int:
        return self._int(L.lib().ahip_session_capacity)

    @property
    def last_gpu_seconds(self) -> float:
        return self._dbl(L.lib().ahip_session_last_gpu_seconds)

    @property
    def last_encode_seconds(self) -> float:
        return self._dbl(L.lib().ahip_session_last_encode_seconds)

    @property
    def profiling_enabled(self) -> bool:
        return getattr(self, "_profiling", False)

    @profiling_enabled.setter
    def profiling_enabled(self, on: bool) -> None:
        L.check(L.lib().ahip_session_set_profiling(self.handle, 1 if on else 0))
        self._profiling = bool(on)

    @property
    def last_profile(self) -> dict:
        n = C.c_int()
        L.check(L.lib().ahip_session_profile(self.handle, None, 0, C.byref(n)))
        arr = (L.StageC * max(n.value, 1))()
        L.check(L.lib().ahip_session_profile(self.handle, arr, n.value, C.byref(n)))
        return {arr[k].label.decode(): StageTime(arr[k].seconds, arr[k].dispatches) for k in range(n.value)}

    @property
    def decode_timeline(self):
        """Raw stamps of the last profiled single-token persistent launch:
        (array [points, workgroups] of wall-clock ticks, seconds per tick)."""
        n, wg, tick = C.c_int64(), C.c_int(), C.c_double()
        L.check(L.lib().ahip_session_decode_timeline(self.handle, None, 0, C.byref(n), C.byref(wg), C.byref(tick)))
        buf = (C.c_uint64 * max(n.value, 1))()
        L.check(L.lib().ahip_session_decode_timeline(self.handle, buf, n.value, C.byref(n), C.byref(wg),
                                                     C.byref(tick)))
        arr = np.frombuffer(buf, dtype=np.uint64, count=n.value).copy()
        return (arr.reshape(-1, wg.value) if wg.value else arr), tick.value

    def close(self) -> None:
        if getattr(self, "handle", None):
            L.lib().ahip_session_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()
