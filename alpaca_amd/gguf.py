"""GGUF model files: the library's C++ reader and Llama loader through the C
ABI, and a writer for synthetic models.

``GGUFFile`` mirrors GGUFFile (Sources/AlpacaModels/GGUF/GGUFFile.swift): a
read-only mapping validated without trusting any length field; a rejected file
raises ``GGUFError`` whose ``kind`` names the reference's GGUFError case.
``load_llama`` mirrors LlamaLoader.load (Sources/AlpacaModels/Llama/
LlamaLoader.swift:29-104) followed by model creation: the model's tensors go
from the mapping to HBM once.

``GGUFWriter`` writes GGUF v2/v3 containers on its own (it shares no code with
the reader, so a writer mistake cannot hide a reader mistake), in the manner of
the reference's test builder (Tests/AlpacaModelTests/GGUFBuilder.swift:7-61);
``write_llama`` lays out a Llama model under the tensor names and metadata keys
LlamaLoader reads.
"""
from __future__ import annotations

import ctypes as C
import struct
from dataclasses import dataclass, field

import numpy as np

from . import _lib as L
from .model import HIPContext, HIPLlamaModel, LlamaConfig
from .tensor import F16, F32, Q4_0, Q8_0, QTensor

# GGUF metadata value types
U8, I8, U16, I16, U32, I32, F32_T, BOOL, STRING, ARRAY, U64, I64, F64_T = range(13)
# GGML tensor types (GGMLType, GGUFTypes.swift:8-12)
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q4_1, GGML_Q8_0, GGML_BF16 = 0, 1, 2, 3, 8, 30
GGML_OF_DTYPE = {F32: GGML_F32, F16: GGML_F16, Q8_0: GGML_Q8_0, Q4_0: GGML_Q4_0}
DTYPE_OF_GGML = {v: k for k, v in GGML_OF_DTYPE.items()}


@dataclass(frozen=True)
class TensorInfo:
    """GGUFTensorInfo (GGUFTypes.swift:72-84); dims fastest-first."""
    name: str
    dims: tuple
    type: int
    file_offset: int
    byte_count: int

    @property
    def shape(self) -> tuple:
        return tuple(reversed(self.dims))


@dataclass
class LoadReport:
    """LoadReport (LlamaLoader.swift:8-16)."""
    mapped_weight_bytes: int = 0
    converted_weight_bytes: int = 0
    notes: list = field(default_factory=list)


class GGUFFile:
    """A validated GGUF container held by the library (mapping or private copy)."""

    def __init__(self, path: str | None = None, data: bytes | None = None):
        if (path is None) == (data is None):
            raise ValueError("give exactly one of path and data")
        h = C.c_void_p()
        if path is not None:
            L.check(L.lib().ahip_gguf_open(str(path).encode(), C.byref(h)))
        else:
            buf = C.create_string_buffer(bytes(data), len(data)) if data else None
            L.check(L.lib().ahip_gguf_open_memory(buf, len(data), C.byref(h)))
        self.handle = h
        ver, al, off, size = C.c_uint32(), C.c_int64(), C.c_int64(), C.c_int64()
        L.check(L.lib().ahip_gguf_header(h, C.byref(ver), C.byref(al), C.byref(off), C.byref(size)))
        self.version, self.alignment, self.data_offset, self.file_size = ver.value, al.value, off.value, size.value
        self.metadata = self._read_metadata()
        n = C.c_int()
        L.check(L.lib().ahip_gguf_tensor_count(h, C.byref(n)))
        self.tensors = []
        self._ptr = {}
        for k in range(n.value):
            t = L.GGUFTensorC()
            L.check(L.lib().ahip_gguf_tensor_at(h, k, C.byref(t)))
            info = TensorInfo(t.name.decode(errors="replace"), tuple(t.dims[: t.n_dims]), t.type, t.file_offset,
                              t.byte_count)
            self.tensors.append(info)
            self._ptr[info.name] = t.data
        self._by_name = {t.name: t for t in self.tensors}

    # -- metadata
    def _value(self, key: bytes, type_id: int, index: int):
        lib, h = L.lib(), self.handle
        if type_id in (U8, U16, U32, U64):
            v = C.c_uint64()
            L.check(lib.ahip_gguf_meta_uint(h, key, index, C.byref(v)))
            return v.value
        if type_id in (I8, I16, I32, I64):
            v = C.c_int64()
            L.check(lib.ahip_gguf_meta_int(h, key, index, C.byref(v)))
            return v.value
        if type_id in (F32_T, F64_T):
            v = C.c_double()
            L.check(lib.ahip_gguf_meta_float(h, key, index, C.byref(v)))
            return v.value
        if type_id == BOOL:
            v = C.c_int()
            L.check(lib.ahip_gguf_meta_bool(h, key, index, C.byref(v)))
            return bool(v.value)
        if type_id == STRING:
            p, n = C.c_void_p(), C.c_int64()
            L.check(lib.ahip_gguf_meta_string(h, key, index, C.byref(p), C.byref(n)))
            return C.string_at(p, n.value).decode(errors="replace") if n.value else ""
        return None  # arrays nested inside arrays are validated but not exposed

    def _read_metadata(self) -> dict:
        lib, h = L.lib(), self.handle
        n = C.c_int()
        L.check(lib.ahip_gguf_meta_count(h, C.byref(n)))
        out, self.metadata_types = {}, {}
        for k in range(n.value):
            key, t = C.c_char_p(), C.c_uint32()
            L.check(lib.ahip_gguf_meta_key(h, k, C.byref(key), C.byref(t)))
            name = key.value.decode(errors="replace")
            self.metadata_types[name] = t.value
            if t.value == ARRAY:
                et, cnt = C.c_uint32(), C.c_int64()
                L.check(lib.ahip_gguf_meta_array(h, key.value, C.byref(et), C.byref(cnt)))
                out[name] = [self._value(key.value, et.value, j) for j in range(cnt.value)]
            else:
                out[name] = self._value(key.value, t.value, -1)
        return out

    def string(self, key: str):
        v = self.metadata.get(key)
        return v if isinstance(v, str) else None

    def int(self, key: str):
        v = self.metadata.get(key)
        return v if isinstance(v, int) and not isinstance(v, bool) else None

    def double(self, key: str):
        v = self.metadata.get(key)
        return float(v) if isinstance(v, (int, float)) and not isinstance(v, bool) else None

    # -- tensors
    def info(self, name: str) -> TensorInfo | None:
        return self._by_name.get(name)

    def raw_bytes(self, name: str) -> np.ndarray:
        """A copy of a tensor's bytes in its on-disk type (GGUFFile.rawBytes)."""
        info = self._by_name.get(name)
        if info is None:
            idx = C.c_int()
            L.check(L.lib().ahip_gguf_find_tensor(self.handle, name.encode(), C.byref(idx)))
        return np.frombuffer(C.string_at(self._ptr[name], info.byte_count), np.uint8).copy()

    def tensor(self, name: str) -> QTensor:
        """A natively supported tensor (F32, F16, Q8_0, Q4_0) as rows x cols (GGUFFile.tensor(named:))."""
        raw = self.raw_bytes(name)
        info = self._by_name[name]
        if info.type not in DTYPE_OF_GGML:
            raise L.GGUFError(L.GGUF, f"tensor '{name}' uses unsupported GGML type id {info.type}", "unsupportedTensorType")
        rows = int(np.prod(info.dims[1:])) if len(info.dims) > 1 else 1
        return QTensor(DTYPE_OF_GGML[info.type], rows, info.dims[0], raw)

    def llama_config(self) -> LlamaConfig:
        """LlamaLoader.load's configuration (LlamaLoader.swift:36-72)."""
        c = L.LlamaConfigC()
        L.check(L.lib().ahip_gguf_llama_config(self.handle, C.byref(c)))
        return _config_of(c)

    def close(self) -> None:
        if getattr(self, "handle", None):
            L.lib().ahip_gguf_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()


def _config_of(c: L.LlamaConfigC) -> LlamaConfig:
    return LlamaConfig(vocab_size=c.vocab_size, hidden_size=c.hidden_size, layer_count=c.layer_count,
                       head_count=c.head_count, kv_head_count=c.kv_head_count, head_dim=c.head_dim,
                       feed_forward_size=c.feed_forward_size, context_length=c.context_length,
                       rms_norm_eps=c.rms_norm_eps, rope_theta=c.rope_theta, rope_interleaved=bool(c.rope_interleaved))


def load_llama(context: HIPContext, source, prefill_weight_cache: bool = False):
    """LlamaLoader.load + MetalLlamaModel.init: (model, config, report) from a
    GGUF path or an open GGUFFile."""
    f = source if isinstance(source, GGUFFile) else GGUFFile(source)
    h, cfg, rep = C.c_void_p(), L.LlamaConfigC(), L.LoadReportC()
    L.check(L.lib().ahip_model_load_gguf(context.handle, f.handle, 1 if prefill_weight_cache else 0, C.byref(h),
                                         C.byref(cfg), C.byref(rep)))
    model = HIPLlamaModel.__new__(HIPLlamaModel)
    model.context, model.config, model.handle = context, _config_of(cfg), h
    notes = [n for n in rep.notes.decode(errors="replace").split("\n") if n]
    return model, model.config, LoadReport(rep.mapped_weight_bytes, rep.converted_weight_bytes, notes)


# ------------------------------------------------------------------ writer

class GGUFWriter:
    """Builds a GGUF container: header, metadata, tensor directory, aligned data.

    ``metadata`` holds (key, type id, value) with value a Python scalar, or for
    ARRAY a pair (element type id, list).  ``tensors`` holds dicts with name,
    dims (fastest first), type (GGML id), data (bytes) and an optional
    ``offset`` overriding the computed one (for malformed test files)."""

    def __init__(self, version: int = 3, alignment: int = 32):
        self.version = version
        self.alignment = alignment
        self.metadata = []
        self.tensors = []

    @staticmethod
    def _string(s) -> bytes:
        b = s.encode() if isinstance(s, str) else bytes(s)
        return struct.pack("<Q", len(b)) + b

    @classmethod
    def encode_value(cls, type_id: int, v) -> bytes:
        fmt = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32_T: "<f", U64: "<Q", I64: "<q",
               F64_T: "<d"}
        if type_id in fmt:
            return struct.pack(fmt[type_id], v)
        if type_id == BOOL:
            return struct.pack("<B", 1 if v else 0)
        if type_id == STRING:
            return cls._string(v)
        if type_id == ARRAY:
            et, items = v
            return struct.pack("<IQ", et, len(items)) + b"".join(cls.encode_value(et, x) for x in items)
        raise ValueError(f"unknown metadata type {type_id}")

    def add(self, key: str, type_id: int, value) -> "GGUFWriter":
        self.metadata.append((key, type_id, value))
        return self

    def add_tensor(self, name: str, dims, ggml_type: int, data: bytes, offset: int | None = None) -> "GGUFWriter":
        self.tensors.append({"name": name, "dims": list(dims), "type": ggml_type, "data": bytes(data), "offset": offset})
        return self

    def build(self) -> bytes:
        md = list(self.metadata)
        if self.alignment != 32:
            md.append(("general.alignment", U32, self.alignment))
        out = bytearray(b"GGUF" + struct.pack("<IQQ", self.version, len(self.tensors), len(md)))
        for key, t, v in md:
            out += self._string(key) + struct.pack("<I", t) + self.encode_value(t, v)
        payload = bytearray()
        for t in self.tensors:
            off = len(payload) if t["offset"] is None else t["offset"]
            out += self._string(t["name"]) + struct.pack("<I", len(t["dims"]))
            out += b"".join(struct.pack("<Q", d) for d in t["dims"])
            out += struct.pack("<IQ", t["type"], off)
            payload += t["data"]
            payload += bytes((-len(payload)) % self.alignment)
        out += bytes((-len(out)) % self.alignment)
        return bytes(out + payload)


def write_llama(path, config: LlamaConfig, weights: dict, name: str = "synthetic llama", version: int = 3,
                alignment: int = 32, extra_metadata=(), q4_1: dict | None = None) -> None:
    """Writes a Llama model under LlamaLoader's names and keys.

    ``weights`` maps the library's tensor names ("token_embd", "blk.N.attn_q",
    ...) to QTensor in the interleaved RoPE layout GGUF uses; a missing
    "output" means tied embeddings.  ``q4_1`` maps names to raw Q4_1 block
    bytes written instead (the loader expands them to F16)."""
    if not config.rope_interleaved:
        raise ValueError("GGUF Llama weights use interleaved RoPE pairs")
    w = GGUFWriter(version, alignment)
    w.add("general.architecture", STRING, "llama").add("general.name", STRING, name)
    for key, t, v in [("llama.context_length", U32, config.context_length),
                      ("llama.embedding_length", U32, config.hidden_size),
                      ("llama.block_count", U32, config.layer_count),
                      ("llama.feed_forward_length", U32, config.feed_forward_size),
                      ("llama.attention.head_count", U32, config.head_count),
                      ("llama.attention.head_count_kv", U32, config.kv_head_count),
                      ("llama.attention.key_length", U32, config.head_dim),
                      ("llama.attention.value_length", U32, config.head_dim),
                      ("llama.rope.dimension_count", U32, config.head_dim),
                      ("llama.attention.layer_norm_rms_epsilon", F32_T, config.rms_norm_eps),
                      ("llama.rope.freq_base", F32_T, config.rope_theta)]:
        w.add(key, t, v)
    for key, t, v in extra_metadata:
        w.add(key, t, v)
    q4_1 = q4_1 or {}
    for tname, t in weights.items():
        dims = [t.cols] if t.rows == 1 and tname.endswith("norm") else [t.cols, t.rows]
        if tname in q4_1:
            w.add_tensor(tname + ".weight", dims, GGML_Q4_1, q4_1[tname])
        else:
            w.add_tensor(tname + ".weight", dims, GGML_OF_DTYPE[t.dtype], t.data.tobytes())
    with open(path, "wb") as f:
        f.write(w.build())


def q4_1_blocks(values: np.ndarray) -> bytes:
    """Raw Q4_1 blocks of float32 values (count a multiple of 32): per block
    f16 d = (max - min) / 15, f16 m = min, nibbles round((v - m) / d), low
    nibble element j, high nibble element j + 16.  Used to make Q4_1 test
    tensors; the loader's expansion, not this encoder, is what is tested."""
    v = np.asarray(values, np.float32).reshape(-1, 32)
    lo, hi = v.min(1), v.max(1)
    d = ((hi - lo) / 15).astype(np.float16)
    m = lo.astype(np.float16)
    df, mf = d.astype(np.float32)[:, None], m.astype(np.float32)[:, None]
    q = np.clip(np.rint(np.divide(v - mf, df, out=np.zeros_like(v), where=df != 0)), 0, 15).astype(np.uint8)
    out = np.empty((v.shape[0], 20), np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = m.view(np.uint8).reshape(-1, 2)
    out[:, 4:] = q[:, :16] | (q[:, 16:] << 4)
    return out.tobytes()


def expand_q4_1(raw: bytes) -> np.ndarray:
    """Float16 values of Q4_1 blocks as the reference expands them:
    Float16(d * Float(q) + m) with float32 arithmetic (LlamaLoader.swift:110-124)."""
    b = np.frombuffer(raw, np.uint8).reshape(-1, 20)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    m = b[:, 2:4].copy().view(np.float16).astype(np.float32)
    q = np.concatenate([b[:, 4:] & 15, b[:, 4:] >> 4], axis=1).astype(np.float32)
    prod = (d * q).astype(np.float32)  # rounded to float32 before the add (no fused multiply-add)
    return (prod + m).astype(np.float32).astype(np.float16).ravel()
