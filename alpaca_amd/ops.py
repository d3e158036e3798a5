"""Tensor-in / tensor-out GPU kernels: the MetalOps mirror.

``HIPOps`` follows ``MetalOps`` (Sources/AlpacaMetal/Backend/MetalOps.swift:
11-219): each call uploads its operands, runs the same kernels the session
uses and returns a float32 numpy array.  Weights are ``QTensor``.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib as L
from .model import GEMM, KV, HIPContext
from .tensor import QTensor


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def _fp(a: np.ndarray):
    return a.ctypes.data_as(L.fp)


class HIPOps:
    def __init__(self, context: HIPContext):
        self.context = context
        self.h = context.handle

    def _binary(self, fn, a, b=None):
        a = _f32(a)
        out = np.empty_like(a)
        if b is None:
            L.check(fn(self.h, _fp(a), a.size, _fp(out)))
        else:
            b = _f32(b)
            if a.shape != b.shape:
                raise L.InvalidArgument(L.INVALID_ARGUMENT, f"shape mismatch {a.shape} vs {b.shape}")
            L.check(fn(self.h, _fp(a), _fp(b), a.size, _fp(out)))
        return out

    def add(self, a, b):
        return self._binary(L.lib().ahip_op_add, a, b)

    def mul(self, a, b):
        return self._binary(L.lib().ahip_op_mul, a, b)

    def silu(self, x):
        return self._binary(L.lib().ahip_op_silu, x)

    def silu_mul(self, gate, up):
        return self._binary(L.lib().ahip_op_silu_mul, gate, up)

    def rms_norm(self, x, weight, eps: float):
        x, w = _f32(x), _f32(weight)
        d = x.shape[-1]
        if w.shape != (d,):
            raise L.InvalidArgument(L.INVALID_ARGUMENT, "rmsNorm weight shape")
        out = np.empty_like(x)
        L.check(L.lib().ahip_op_rmsnorm(self.h, _fp(x), _fp(w), x.size // d, d, eps, _fp(out)))
        return out

    def linear(self, x, weight: QTensor, precision: str = "exact"):
        x = _f32(x)
        m, k = x.shape
        if k != weight.cols:
            raise L.InvalidArgument(L.INVALID_ARGUMENT, f"linear shapes {x.shape} / {weight.shape}")
        y = np.empty((m, weight.rows), np.float32)
        L.check(L.lib().ahip_op_linear(self.h, _fp(x), m, k, weight.dtype, weight.data.ctypes.data, weight.rows,
                                       GEMM[precision], _fp(y)))
        return y

    def linear_add(self, x, weight: QTensor, residual, precision: str = "exact"):
        x = _f32(x)
        m, k = x.shape
        res = _f32(residual).copy()
        if k != weight.cols or res.shape != (m, weight.rows):
            raise L.InvalidArgument(L.INVALID_ARGUMENT, "linearAdd shapes")
        L.check(L.lib().ahip_op_linear_add(self.h, _fp(x), m, k, weight.dtype, weight.data.ctypes.data, weight.rows,
                                           GEMM[precision], _fp(res)))
        return res

    def gate_up_silu(self, x, gate: QTensor, up: QTensor, precision: str = "exact"):
        x = _f32(x)
        m, k = x.shape
        if gate.shape != up.shape or gate.dtype != up.dtype or gate.cols != k:
            raise L.InvalidArgument(L.INVALID_ARGUMENT, "gateUpSilu shapes/dtypes")
        out = np.empty((m, gate.rows), np.float32)
        L.check(L.lib().ahip_op_gate_up_silu(self.h, _fp(x), m, k, gate.dtype, gate.data.ctypes.data,
                                             up.data.ctypes.data, gate.rows, GEMM[precision], _fp(out)))
        return out

    def rope(self, x, start_position: int, theta: float, interleaved: bool = True):
        v = _f32(x).copy()
        if v.ndim != 3 or v.shape[2] % 2:
            raise L.InvalidArgument(L.INVALID_ARGUMENT, f"rope shape {v.shape}")
        t, h, hd = v.shape
        L.check(L.lib().ahip_op_rope(self.h, _fp(v), t, h, hd, start_position, theta, 1 if interleaved else 0))
        return v

    def attention(self, q, keys, values, start_position: int, kv: str = "f16", precision: str = "exact"):
        """q [tokens, heads, hd]; keys/values [capacity, kv_heads, hd] -> [tokens, heads, hd]."""
        q, k, v = _f32(q), _f32(keys), _f32(values)
        if q.ndim != 3 or k.shape != v.shape or k.ndim != 3 or k.shape[2] != q.shape[2] or q.shape[1] % k.shape[1]:
            raise L.InvalidArgument(L.INVALID_ARGUMENT, f"attention shapes q {q.shape} k {k.shape}")
        t, h, hd = q.shape
        out = np.empty_like(q)
        L.check(L.lib().ahip_op_attention(self.h, _fp(q), t, h, hd, _fp(k), _fp(v), k.shape[0], k.shape[1],
                                          start_position, KV[kv], GEMM[precision], _fp(out)))
        return out

    def embed(self, tokens, table: QTensor):
        tok = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        out = np.empty((tok.size, table.cols), np.float32)
        L.check(L.lib().ahip_op_embed(self.h, tok.ctypes.data_as(L.ip), tok.size, table.dtype,
                                      table.data.ctypes.data, table.rows, table.cols, _fp(out)))
        return out

    def dequantize(self, t: QTensor):
        out = np.empty((t.rows, t.cols), np.float32)
        L.check(L.lib().ahip_op_dequantize(self.h, t.dtype, t.data.ctypes.data, t.rows * t.cols, _fp(out)))
        return out

    def sample(self, logits, temperature: float, top_k: int, top_p: float, u: float) -> int:
        """Sampler.sample (Sampler.swift:57-93) on the device for a draw u in [0, 1)."""
        v = _f32(logits).ravel()
        r = C.c_int32()
        L.check(L.lib().ahip_op_sample(self.h, _fp(v), v.size, temperature, top_k, top_p, u, C.byref(r)))
        return r.value

    def argmax(self, logits) -> int:
        v = _f32(logits).ravel()
        r = C.c_int32()
        L.check(L.lib().ahip_op_argmax(self.h, _fp(v), v.size, C.byref(r)))
        return r.value
