"""Weight tensors in GGUF on-disk formats (DType.swift:8-56) and conversions.

``QTensor`` holds raw bytes of a [rows, cols] tensor in F32 / F16 / Q8_0 /
Q4_0.  Quantisation goes through the library's ``ahip_quantize``
(Quantization.swift:39-73).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib as L

F32, F16, Q8_0, Q4_0 = L.F32, L.F16, L.Q8_0, L.Q4_0
NAMES = {F32: "f32", F16: "f16", Q8_0: "q8_0", Q4_0: "q4_0"}
BY_NAME = {v: k for k, v in NAMES.items()}
BLOCK_ELEMS = {F32: 1, F16: 1, Q8_0: 32, Q4_0: 32}
BLOCK_BYTES = {F32: 4, F16: 2, Q8_0: 34, Q4_0: 18}


def dtype_of(d) -> int:
    return BY_NAME[d] if isinstance(d, str) else int(d)


def byte_count(dtype: int, elements: int) -> int:
    return elements // BLOCK_ELEMS[dtype] * BLOCK_BYTES[dtype]


@dataclass
class QTensor:
    dtype: int
    rows: int
    cols: int
    data: np.ndarray  # uint8, contiguous

    def __post_init__(self):
        self.data = np.ascontiguousarray(self.data).view(np.uint8).ravel()
        if self.data.nbytes != byte_count(self.dtype, self.rows * self.cols):
            raise ValueError("byte count does not match shape and dtype")

    @property
    def shape(self):
        return (self.rows, self.cols)


def quantize(values: np.ndarray, dtype) -> np.ndarray:
    """Raw Q8_0 / Q4_0 blocks of float32 values (count a multiple of 32)."""
    dt = dtype_of(dtype)
    v = np.ascontiguousarray(np.asarray(values, dtype=np.float32).ravel())
    out = np.empty(byte_count(dt, v.size), np.uint8)
    L.check(L.lib().ahip_quantize(dt, v.ctypes.data_as(L.fp), v.size, out.ctypes.data))
    return out


def encode(values: np.ndarray, dtype) -> QTensor:
    """[rows, cols] float32 values stored as `dtype`."""
    dt = dtype_of(dtype)
    v = np.asarray(values, dtype=np.float32)
    if v.ndim == 1:
        v = v.reshape(1, -1)
    rows, cols = v.shape
    if dt == F32:
        raw = np.ascontiguousarray(v).view(np.uint8)
    elif dt == F16:
        raw = np.ascontiguousarray(v.astype(np.float16)).view(np.uint8)
    else:
        raw = quantize(v, dt)
    return QTensor(dt, rows, cols, raw)
