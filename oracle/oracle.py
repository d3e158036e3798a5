"""ctypes wrapper over the CPU oracle (oracle/alpaca_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of bench.py, and never by the product package
``alpaca_amd``.  Each function mirrors one function of the reference's Swift
CPU backend (Sources/AlpacaCore) -- see the citations in alpaca_oracle.c.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

F32, F16, Q8_0, Q4_0 = 0, 1, 2, 3
DTYPES = {"f32": F32, "f16": F16, "q8_0": Q8_0, "q4_0": Q4_0}
BLOCK_ELEMS = {F32: 1, F16: 1, Q8_0: 32, Q4_0: 32}
BLOCK_BYTES = {F32: 4, F16: 2, Q8_0: 34, Q4_0: 18}


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, fp, ip, i64 = C.c_void_p, C.POINTER(C.c_float), C.POINTER(C.c_int32), C.c_int64
        sig = {
            "orc_half_to_float": (C.c_float, [C.c_uint16]),
            "orc_float_to_half": (C.c_uint16, [C.c_float]),
            "orc_splitmix_next": (C.c_uint64, [C.POINTER(C.c_uint64)]),
            "orc_dequantize": (None, [C.c_int, vp, i64, fp]),
            "orc_quantize": (C.c_int, [C.c_int, fp, i64, vp]),
            "orc_dot": (C.c_float, [C.c_int, vp, fp, C.c_int]),
            "orc_set_threads": (None, [C.c_int]),
            "orc_get_threads": (C.c_int, []),
            "orc_linear": (None, [fp, C.c_int, C.c_int, C.c_int, vp, C.c_int, fp]),
            "orc_matmul": (None, [fp, fp, C.c_int, C.c_int, C.c_int, fp]),
            "orc_add": (None, [fp, fp, i64, fp]),
            "orc_mul": (None, [fp, fp, i64, fp]),
            "orc_silu": (None, [fp, i64, fp]),
            "orc_rmsnorm": (None, [fp, fp, C.c_int, C.c_int, C.c_float, fp]),
            "orc_softmax": (None, [fp, i64, C.c_int]),
            "orc_rope": (None, [fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int]),
            "orc_attention_scores": (None, [fp, C.c_int, C.c_int, C.c_int, fp, C.c_int, C.c_int, C.c_int, fp]),
            "orc_attention_apply": (None, [fp, C.c_int, C.c_int, C.c_int, fp, C.c_int, C.c_int, fp]),
            "orc_attention": (None, [fp, C.c_int, C.c_int, C.c_int, fp, fp, C.c_int, C.c_int, C.c_int, fp, fp]),
            "orc_embed": (C.c_int, [ip, C.c_int, C.c_int, vp, C.c_int, C.c_int, fp]),
            "orc_argmax": (C.c_int, [fp, C.c_int]),
            "orc_uniform53": (C.c_double, [C.POINTER(C.c_uint64)]),
            "orc_sample": (C.c_int, [fp, C.c_int, C.c_float, C.c_int, C.c_float, C.c_double]),
            "orc_model_create": (vp, [vp, C.c_int, C.c_int, C.c_int, vp, vp, fp]),
            "orc_model_set_layer": (None, [vp, C.c_int, fp, vp, vp, vp, vp, fp, vp, vp, vp]),
            "orc_model_destroy": (None, [vp]),
            "orc_kv_create": (vp, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
            "orc_kv_destroy": (None, [vp]),
            "orc_kv_length": (C.c_int, [vp]),
            "orc_kv_reset": (None, [vp]),
            "orc_kv_fill": (C.c_int, [vp, C.c_int, C.c_uint64]),
            "orc_kv_keys": (fp, [vp, C.c_int]),
            "orc_kv_values": (fp, [vp, C.c_int]),
            "orc_forward": (C.c_int, [vp, vp, ip, C.c_int, C.c_int, fp]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _v(a: np.ndarray):
    assert a.flags.c_contiguous
    return C.c_void_p(a.ctypes.data)


def f32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


# ------------------------------------------------------------------ scalars

def half_to_float(h: int) -> float:
    return lib().orc_half_to_float(h)


def float_to_half(f: float) -> int:
    return lib().orc_float_to_half(f)


class SplitMix64:
    """Sampler.swift:30-40 through the oracle."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(seed)

    def next(self) -> int:
        return lib().orc_splitmix_next(C.byref(self.state))


# ------------------------------------------------------------------ ops

def row_bytes(dtype: int, cols: int) -> int:
    return cols // BLOCK_ELEMS[dtype] * BLOCK_BYTES[dtype]


def dequantize(dtype: int, raw: np.ndarray, elements: int) -> np.ndarray:
    out = np.empty(elements, np.float32)
    lib().orc_dequantize(dtype, _v(np.ascontiguousarray(raw)), elements, _f(out))
    return out


def quantize(values, dtype: int) -> np.ndarray:
    v = f32(values).ravel()
    out = np.empty(v.size // 32 * BLOCK_BYTES[dtype], np.uint8)
    rc = lib().orc_quantize(dtype, _f(v), v.size, _v(out))
    if rc != 0:
        raise ValueError("quantize: bad dtype or count")
    return out


def encode(values, dtype: int) -> np.ndarray:
    """Raw bytes of `values` stored as `dtype` (f32/f16 by IEEE conversion)."""
    v = f32(values)
    if dtype == F32:
        return v.view(np.uint8).ravel().copy()
    if dtype == F16:
        return v.astype(np.float16).view(np.uint8).ravel().copy()
    return quantize(v, dtype)


def linear(x, dtype: int, w: np.ndarray, n: int) -> np.ndarray:
    x = f32(x)
    m, k = x.shape
    out = np.empty((m, n), np.float32)
    lib().orc_linear(_f(x), m, k, dtype, _v(np.ascontiguousarray(w)), n, _f(out))
    return out


def matmul(a, b) -> np.ndarray:
    a, b = f32(a), f32(b)
    out = np.empty((a.shape[0], b.shape[1]), np.float32)
    lib().orc_matmul(_f(a), _f(b), a.shape[0], a.shape[1], b.shape[1], _f(out))
    return out


def add(a, b):
    a, b = f32(a), f32(b)
    out = np.empty_like(a)
    lib().orc_add(_f(a), _f(b), a.size, _f(out))
    return out


def mul(a, b):
    a, b = f32(a), f32(b)
    out = np.empty_like(a)
    lib().orc_mul(_f(a), _f(b), a.size, _f(out))
    return out


def silu(x):
    x = f32(x)
    out = np.empty_like(x)
    lib().orc_silu(_f(x), x.size, _f(out))
    return out


def rmsnorm(x, w, eps: float):
    x, w = f32(x), f32(w)
    d = x.shape[-1]
    out = np.empty_like(x)
    lib().orc_rmsnorm(_f(x), _f(w), x.size // d, d, eps, _f(out))
    return out


def softmax(x):
    v = f32(x).copy()
    d = v.shape[-1]
    lib().orc_softmax(_f(v), v.size // d, d)
    return v


def rope(x, start: int, theta: float, interleaved: bool = True):
    v = f32(x).copy()
    t, h, hd = v.shape
    lib().orc_rope(_f(v), t, h, hd, start, theta, 1 if interleaved else 0)
    return v


def attention_scores(q, keys, length: int, start: int):
    q, keys = f32(q), f32(keys)
    t, h, hd = q.shape
    out = np.empty((h, t, length), np.float32)
    lib().orc_attention_scores(_f(q), t, h, hd, _f(keys), keys.shape[1], length, start, _f(out))
    return out


def attention_apply(probs, values):
    probs, values = f32(probs), f32(values)
    h, t, length = probs.shape
    hd = values.shape[2]
    out = np.empty((t, h, hd), np.float32)
    lib().orc_attention_apply(_f(probs), h, t, length, _f(values), values.shape[1], hd, _f(out))
    return out


def attention(q, keys, values, start: int, length: int | None = None):
    """softmax(scores) applied to values; [tokens, heads, hd]."""
    q, keys, values = f32(q), f32(keys), f32(values)
    t, h, hd = q.shape
    if length is None:
        length = start + t
    scratch = np.empty(h * t * length, np.float32)
    out = np.empty((t, h, hd), np.float32)
    lib().orc_attention(_f(q), t, h, hd, _f(keys), _f(values), keys.shape[1], length, start, _f(scratch), _f(out))
    return out


def embed(tokens, dtype: int, table: np.ndarray, vocab: int, dim: int):
    tok = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
    out = np.empty((tok.size, dim), np.float32)
    rc = lib().orc_embed(tok.ctypes.data_as(C.POINTER(C.c_int32)), tok.size, dtype, _v(np.ascontiguousarray(table)),
                         vocab, dim, _f(out))
    if rc != 0:
        raise IndexError("token id outside vocabulary")
    return out


def argmax(logits) -> int:
    v = f32(logits)
    r = lib().orc_argmax(_f(v), v.size)
    if r < 0:
        raise ValueError("logits contain NaN")
    return r


def sample(logits, temperature: float, top_k: int, top_p: float, u: float) -> int:
    """Sampler.sample (Sampler.swift:57-93) for a given draw u in [0, 1)."""
    v = f32(logits)
    if v.size == 0:
        raise ValueError("cannot sample from empty logits")
    r = lib().orc_sample(_f(v), v.size, temperature, top_k, top_p, u)
    if r < 0:
        raise ValueError("logits contain NaN")
    return r


class Sampler:
    """Sampler (Sampler.swift:43-55): validated parameters and a SplitMix64
    stream; each sample() draws one uniform (orc_uniform53) unless greedy."""

    def __init__(self, temperature: float = 0.8, top_k: int = 0, top_p: float = 1.0, seed: int = 0):
        if not (np.isfinite(temperature) and temperature >= 0):
            raise ValueError("temperature must be finite and >= 0")
        if top_k < 0:
            raise ValueError("topK must be >= 0")
        if not (0 < top_p <= 1):
            raise ValueError("topP must be in (0, 1]")
        self.temperature, self.top_k, self.top_p = float(temperature), int(top_k), float(top_p)
        self.state = C.c_uint64(seed)

    def draw(self) -> float:
        return lib().orc_uniform53(C.byref(self.state))

    def sample(self, logits) -> int:
        if len(logits) == 0:
            raise ValueError("cannot sample from empty logits")  # checked before greedy, Sampler.swift:60
        if self.temperature == 0:
            return argmax(logits)
        return sample(logits, self.temperature, self.top_k, self.top_p, self.draw())


def set_threads(n: int) -> None:
    lib().orc_set_threads(n)


def get_threads() -> int:
    return lib().orc_get_threads()


# ------------------------------------------------------------------ model

class Config(C.Structure):
    """LlamaConfig.swift:8-20 (same field order as the C struct)."""
    _fields_ = [
        ("vocab_size", C.c_int32), ("hidden_size", C.c_int32), ("layer_count", C.c_int32),
        ("head_count", C.c_int32), ("kv_head_count", C.c_int32), ("head_dim", C.c_int32),
        ("feed_forward_size", C.c_int32), ("context_length", C.c_int32),
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float), ("rope_interleaved", C.c_int32),
    ]


class OracleModel:
    """LlamaCPUModel over host weights.

    `weights` maps GGUF tensor names (LlamaLoader.swift) to (dtype, raw bytes
    as uint8 array).  Norms must be f32.  Buffers are kept alive here.
    """

    def __init__(self, cfg: dict, weights: dict):
        self.cfg = dict(cfg)
        c = Config(cfg["vocab"], cfg["hidden"], cfg["layers"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"],
                   cfg["ffn"], cfg["context"], cfg["eps"], cfg["theta"], 1 if cfg.get("interleaved", True) else 0)
        self._c = c
        self._keep = weights
        dt = weights["blk.0.attn_q"][0]
        emb_dt, emb = weights["token_embd"]
        out = weights.get("output")
        onorm = np.ascontiguousarray(weights["output_norm"][1].view(np.float32))
        self._onorm = onorm
        self.h = lib().orc_model_create(C.byref(c), dt, emb_dt, out[0] if out else emb_dt, _v(emb),
                                        _v(out[1]) if out else None, _f(onorm))
        self._norms = []
        for i in range(cfg["layers"]):
            g = lambda n: weights[f"blk.{i}.{n}"][1]
            an = np.ascontiguousarray(g("attn_norm").view(np.float32))
            fn = np.ascontiguousarray(g("ffn_norm").view(np.float32))
            self._norms += [an, fn]
            for n in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"):
                assert weights[f"blk.{i}.{n}"][0] == dt, "oracle model needs one projection dtype"
            lib().orc_model_set_layer(self.h, i, _f(an), _v(g("attn_q")), _v(g("attn_k")), _v(g("attn_v")),
                                      _v(g("attn_output")), _f(fn), _v(g("ffn_gate")), _v(g("ffn_up")),
                                      _v(g("ffn_down")))

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_model_destroy(self.h)
            self.h = None


class OracleKV:
    """KVCache.swift over the oracle."""

    def __init__(self, cfg: dict, capacity: int, rounds_f16: bool = False):
        self.h = lib().orc_kv_create(cfg["layers"], capacity, cfg["kv_heads"], cfg["head_dim"], 1 if rounds_f16 else 0)
        self.capacity = capacity
        self.shape = (capacity, cfg["kv_heads"], cfg["head_dim"])

    @property
    def length(self) -> int:
        return lib().orc_kv_length(self.h)

    def reset(self) -> None:
        lib().orc_kv_reset(self.h)

    def fill(self, length: int, seed: int = 0) -> None:
        """Benchmark helper: `length` synthetic valid rows (no prefill needed)."""
        if lib().orc_kv_fill(self.h, length, seed) != 0:
            raise ValueError("fill length exceeds capacity")

    def keys(self, layer: int) -> np.ndarray:
        p = lib().orc_kv_keys(self.h, layer)
        return np.ctypeslib.as_array(p, shape=self.shape).copy()

    def values(self, layer: int) -> np.ndarray:
        p = lib().orc_kv_values(self.h, layer)
        return np.ctypeslib.as_array(p, shape=self.shape).copy()

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_kv_destroy(self.h)
            self.h = None


def forward(model: OracleModel, kv: OracleKV, tokens, all_logits: bool = False) -> np.ndarray:
    tok = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
    v = model.cfg["vocab"]
    out = np.empty((tok.size if all_logits else 1, v), np.float32)
    rc = lib().orc_forward(model.h, kv.h, tok.ctypes.data_as(C.POINTER(C.c_int32)), tok.size,
                           1 if all_logits else 0, _f(out))
    if rc == -1:
        raise ValueError("forward: empty input or cache geometry mismatch")
    if rc == -2:
        raise ValueError("forward: context exhausted")
    if rc == -3:
        raise IndexError("forward: token id outside vocabulary")
    return out if all_logits else out[0]
