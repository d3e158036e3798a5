"""The GGUF reader (alpaca_amd/csrc/gguf.cpp through the C ABI), on the CPU.

Follows Tests/AlpacaModelTests/GGUFParserTests.swift case by case: the same
well-formed sample, the same header, metadata and tensor-record mutations with
the GGUFError case each must raise, every truncation, the missing file, and
20,000 seeded mutations (SplitMix64, seed 0xA17ACA) after which the parser
must either reject the file or return tensors that lie inside it.  Files are
made by alpaca_amd.gguf.GGUFWriter, which shares no code with the reader.
The Llama configuration rules follow LlamaLoader.swift:36-72.
"""
import struct

import numpy as np
import pytest

from alpaca_amd import gguf, synth
from alpaca_amd._lib import GGUFError
from alpaca_amd.gguf import (ARRAY, BOOL, F32_T, F64_T, I8, I16, I32, I64, STRING, U8, U16, U32, U64, GGUFFile,
                             GGUFWriter)
from alpaca_amd.tensor import Q8_0


def f32_tensor(w: GGUFWriter, name, dims, values, offset=None):
    return w.add_tensor(name, dims, gguf.GGML_F32, np.asarray(values, np.float32).tobytes(), offset)


def sample() -> GGUFWriter:
    w = GGUFWriter()
    for key, t, v in [("general.architecture", STRING, "llama"), ("n.u8", U8, 200), ("n.i8", I8, -5),
                      ("n.u16", U16, 65000), ("n.i16", I16, -300), ("n.u32", U32, 4_000_000_000), ("n.i32", I32, -7),
                      ("n.f32", F32_T, 1.5), ("n.bool", BOOL, True), ("n.u64", U64, 1 << 40),
                      ("n.i64", I64, -(1 << 40)), ("n.f64", F64_T, 2.25),
                      ("arr.str", ARRAY, (STRING, ["a", "bc"])), ("arr.u32", ARRAY, (U32, [1, 2, 3]))]:
        w.add(key, t, v)
    f32_tensor(w, "a", [4, 2], np.arange(1, 9))
    f32_tensor(w, "b", [3], [9, 10, 11])
    return w


def kind_of(data: bytes) -> str:
    with pytest.raises(GGUFError) as e:
        GGUFFile(data=data)
    return e.value.kind


def patch(data: bytes, at: int, new: bytes) -> bytes:
    return data[:at] + new + data[at + len(new):]


def test_parses_well_formed_file():
    f = GGUFFile(data=sample().build())
    assert f.version == 3
    assert f.string("general.architecture") == "llama"
    m = f.metadata
    assert (m["n.u8"], m["n.i8"], m["n.u16"], m["n.i16"]) == (200, -5, 65000, -300)
    assert (m["n.u32"], m["n.i32"], m["n.u64"], m["n.i64"]) == (4_000_000_000, -7, 1 << 40, -(1 << 40))
    assert (m["n.f32"], m["n.f64"], m["n.bool"]) == (1.5, 2.25, True)
    assert m["arr.str"] == ["a", "bc"] and m["arr.u32"] == [1, 2, 3]
    assert len(f.tensors) == 2
    # GGUF dims are fastest-first: dims [4, 2] is a row-major [2, 4] tensor
    a = f.tensor("a")
    assert f.info("a").shape == (2, 4) and (a.rows, a.cols) == (2, 4)
    assert np.frombuffer(a.data.tobytes(), np.float32).tolist() == list(range(1, 9))
    assert np.frombuffer(f.tensor("b").data.tobytes(), np.float32).tolist() == [9, 10, 11]
    with pytest.raises(GGUFError) as e:
        f.tensor("missing")
    assert e.value.kind == "missingTensor"


def test_custom_alignment():
    w = sample()
    w.alignment = 64
    f = GGUFFile(data=w.build())
    assert f.alignment == 64 and f.data_offset % 64 == 0
    assert np.frombuffer(f.tensor("b").data.tobytes(), np.float32).tolist() == [9, 10, 11]


def test_rejects_bad_headers():
    d = sample().build()
    assert kind_of(b"") == "invalidMagic"
    assert kind_of(b"GGML" + d[4:]) == "invalidMagic"
    for v in (0, 1, 4, 99):
        w = sample()
        w.version = v
        assert kind_of(w.build()) == "unsupportedVersion", v
    assert kind_of(patch(d, 4, bytes([0, 0, 0, 3]))) == "bigEndianNotSupported"


def test_every_truncation_is_rejected_cleanly():
    full = sample().build()
    f = GGUFFile(data=full)
    required = max(t.file_offset + t.byte_count for t in f.tensors)
    # every prefix that cuts into the header, directory or any tensor's bytes is rejected
    for n in range(required):
        with pytest.raises(GGUFError):
            GGUFFile(data=full[:n])
    GGUFFile(data=full)


def test_rejects_malformed_metadata_and_tensors():
    d = sample().build()
    # huge declared counts or lengths fail on size checks before any allocation
    assert kind_of(patch(d, 8, struct.pack("<Q", 2**64 - 1))) == "limitExceeded"  # tensor count
    assert kind_of(patch(d, 16, struct.pack("<Q", 1 << 40))) == "limitExceeded"    # metadata count
    assert kind_of(patch(d, 16, struct.pack("<Q", 60_000))) == "truncated"         # beyond the file
    w = GGUFWriter().add("k", ARRAY, (U32, [1]))
    b = w.build()
    key_end = 24 + 8 + 1 + 4 + 4  # header, key length and byte, value type, element type
    assert kind_of(patch(b, key_end, struct.pack("<Q", 1 << 23))) == "truncated"
    assert kind_of(patch(b, key_end, struct.pack("<Q", 2**64 - 1))) == "limitExceeded"
    b = GGUFWriter().add("k", STRING, "x").build()
    assert kind_of(patch(b, 37, struct.pack("<Q", 2**64 - 1))) == "limitExceeded"  # string length
    assert kind_of(GGUFWriter().add("k", BOOL, True).add("k", BOOL, False).build()) == "malformed"
    assert kind_of(GGUFWriter().add("general.alignment", U32, 48).build()) == "malformed"
    b = GGUFWriter().add("flag", BOOL, True).build()
    at = b.rindex(b"\x01")
    assert kind_of(patch(b, at, b"\x02")) == "malformed"  # a bool that is neither 0 nor 1
    raw = GGUFWriter().add("k", U8, 1).build()
    assert kind_of(patch(raw, 24 + 8 + 1, struct.pack("<I", 13))) == "malformed"  # unknown value type
    nested = GGUFWriter().add("k", ARRAY, (ARRAY, [(U8, [1])]))
    GGUFFile(data=nested.build())  # two levels: accepted
    deep = GGUFWriter().add("k", ARRAY, (ARRAY, [(ARRAY, [(U8, [1])])]))
    assert kind_of(deep.build()) == "limitExceeded"


def one(**mut) -> bytes:
    w = GGUFWriter()
    t = {"name": "w", "dims": [8], "type": gguf.GGML_F32, "data": np.ones(8, np.float32).tobytes(), "offset": None}
    t.update(mut)
    w.add_tensor(t["name"], t["dims"], t["type"], t["data"], t["offset"])
    return w.build()


def test_rejects_invalid_tensor_records():
    assert kind_of(one(dims=[0])) == "malformed"
    assert kind_of(one(dims=[])) == "malformed"
    assert kind_of(one(dims=[1, 1, 1, 1, 8])) == "malformed"
    assert kind_of(one(dims=[1 << 62, 1 << 62])) == "malformed"
    assert kind_of(one(dims=[2**64 - 1])) == "malformed"
    with pytest.raises(GGUFError) as e:
        GGUFFile(data=one(type=99))
    assert e.value.kind == "unsupportedTensorType" and "99" in str(e.value) and "'w'" in str(e.value)
    assert kind_of(one(type=gguf.GGML_Q8_0)) == "malformed"  # row of 8 is not a multiple of 32
    assert kind_of(one(offset=1 << 40)) == "tensorOutOfRange"
    assert kind_of(one(offset=2**64 - 32)) == "tensorOutOfRange"
    assert kind_of(one(offset=5)) == "malformed"
    assert kind_of(one(dims=[1 << 20])) == "tensorOutOfRange"
    w = GGUFWriter()
    f32_tensor(w, "w", [4], [1, 2, 3, 4])
    f32_tensor(w, "w", [4], [1, 2, 3, 4])
    with pytest.raises(GGUFError) as e:
        GGUFFile(data=w.build())
    assert e.value.kind == "duplicateTensor" and "'w'" in str(e.value)
    w = GGUFWriter()
    f32_tensor(w, "x", [16], np.zeros(16), offset=0)
    f32_tensor(w, "y", [16], np.zeros(16), offset=32)  # x occupies bytes 0..64, y starts at 32
    assert kind_of(w.build()) == "tensorsOverlap"


def test_missing_file_reports_clean_error(tmp_path):
    with pytest.raises(GGUFError) as e:
        GGUFFile(str(tmp_path / "nonexistent" / "model.gguf"))
    assert e.value.kind == "cannotOpen"
    empty = tmp_path / "empty.gguf"
    empty.write_bytes(b"")
    with pytest.raises(GGUFError) as e:
        GGUFFile(str(empty))
    assert e.value.kind == "truncated"


def test_mapped_file_matches_memory_image(tmp_path):
    data = sample().build()
    p = tmp_path / "s.gguf"
    p.write_bytes(data)
    a, b = GGUFFile(str(p)), GGUFFile(data=data)
    assert a.metadata == b.metadata and a.tensors == b.tensors and a.file_size == len(data)
    assert a.raw_bytes("a").tobytes() == b.raw_bytes("a").tobytes()


class SplitMix64:
    """Sampler.swift:30-40 / GGUFParserTests.swift:177-188."""

    def __init__(self, seed: int):
        self.state = seed

    def next(self) -> int:
        m = (1 << 64) - 1
        self.state = (self.state + 0x9E3779B97F4A7C15) & m
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
        return z ^ (z >> 31)


def test_mutation_fuzzing():
    """Random byte writes, bit flips, truncations and insertions: the reader
    either raises GGUFError or returns a file whose tensors all lie inside it."""
    base = sample().build()
    rng = SplitMix64(0xA17ACA)
    accepted = rejected = 0
    for _ in range(20_000):
        d = bytearray(base)
        for _ in range(1 + rng.next() % 4):
            op = rng.next() % 4
            if op == 0:
                d[rng.next() % len(d)] = rng.next() & 0xFF
            elif op == 1:
                d[rng.next() % len(d)] ^= 1 << (rng.next() % 8)
            elif op == 2:
                d = d[: rng.next() % (len(d) + 1)]
            else:
                at = rng.next() % (len(d) + 1)
                d[at:at] = bytes([rng.next() & 0xFF])
            if not d:
                d = bytearray(b"\0")
        try:
            f = GGUFFile(data=bytes(d))
        except GGUFError:
            rejected += 1
            continue
        accepted += 1
        for t in f.tensors:
            assert t.file_offset + t.byte_count <= f.file_size
            f.raw_bytes(t.name).sum()
            if t.type == gguf.GGML_F32:
                f.tensor(t.name)
        f.close()
    print(f"[fuzz] 20000 mutated files: {accepted} accepted (tensor ranges in bounds), {rejected} rejected")
    assert accepted + rejected == 20_000 and rejected > 0


# ------------------------------------------------------------------ Llama configuration

TINY = synth.TINY


def llama_bytes(tmp_path, config=None, weights=None, drop=(), extra=(), name="m.gguf", **kw):
    config = config or TINY.config
    weights = dict(weights or synth.build_weights(TINY))
    for n in drop:
        weights.pop(n)
    p = tmp_path / name
    gguf.write_llama(str(p), config, weights, extra_metadata=extra, **kw)
    return p


def rewrite_meta(path, drop_keys=(), replace=None):
    """The file at `path` with metadata keys dropped or replaced (same tensors)."""
    f = GGUFFile(str(path))
    w = GGUFWriter(f.version, f.alignment)
    for k, v in f.metadata.items():
        if k in drop_keys or k == "general.alignment":
            continue
        t = f.metadata_types[k]
        if replace and k in replace:
            t, v = replace[k]
        if t == ARRAY:
            continue
        w.add(k, t, v)
    for k, (t, v) in (replace or {}).items():
        if k not in f.metadata:
            w.add(k, t, v)
    for t in f.tensors:
        w.add_tensor(t.name, t.dims, t.type, f.raw_bytes(t.name).tobytes())
    path.write_bytes(w.build())
    return path


def cfg(c) -> tuple:
    """A LlamaConfig's fields with the floats as float32 (GGUF stores them as F32)."""
    return (c.vocab_size, c.hidden_size, c.layer_count, c.head_count, c.kv_head_count, c.head_dim,
            c.feed_forward_size, c.context_length, np.float32(c.rms_norm_eps), np.float32(c.rope_theta),
            bool(c.rope_interleaved))


def config_kind(path) -> str:
    with pytest.raises(GGUFError) as e:
        GGUFFile(str(path)).llama_config()
    return e.value.kind


def test_llama_config_round_trip(tmp_path):
    f = GGUFFile(str(llama_bytes(tmp_path)))
    assert cfg(f.llama_config()) == cfg(TINY.config)
    w = synth.build_weights(TINY)
    for name in ("token_embd", "blk.0.attn_q", "blk.2.ffn_down", "output_norm"):
        t = f.tensor(name + ".weight")
        assert (t.dtype, t.rows, t.cols) == (w[name].dtype, w[name].rows, w[name].cols)
        assert t.data.tobytes() == w[name].data.tobytes()


def test_llama_config_defaults(tmp_path):
    p = rewrite_meta(llama_bytes(tmp_path), drop_keys={
        "llama.attention.key_length", "llama.attention.value_length", "llama.rope.dimension_count",
        "llama.attention.head_count_kv", "llama.attention.layer_norm_rms_epsilon", "llama.rope.freq_base"})
    c = GGUFFile(str(p)).llama_config()
    # head_dim = hidden / heads, kv heads = heads, eps 1e-5, theta 10000 (LlamaLoader.swift:45, :58-62)
    assert c.head_dim == TINY.config.hidden_size // TINY.config.head_count
    assert c.kv_head_count == c.head_count
    assert c.rms_norm_eps == np.float32(1e-5) and c.rope_theta == 10000.0 and c.rope_interleaved


@pytest.mark.parametrize("case,want", [
    ({"general.architecture": (STRING, "gpt2")}, "unsupportedModel"),
    ({"llama.rope.scaling.type": (STRING, "linear")}, "unsupportedModel"),
    ({"llama.expert_count": (U32, 8)}, "unsupportedModel"),
    ({"llama.attention.value_length": (U32, 32)}, "unsupportedModel"),
    ({"llama.rope.dimension_count": (U32, 32)}, "unsupportedModel"),
    ({"llama.attention.head_count": (U32, 0)}, "malformed"),
    ({"llama.block_count": (STRING, "3")}, "missingMetadata"),
    ({"llama.attention.key_length": (U32, 48)}, "unsupportedModel"),  # fails the kernels' head_dim rule
])
def test_llama_config_refusals(tmp_path, case, want):
    assert config_kind(rewrite_meta(llama_bytes(tmp_path), replace=case)) == want


def test_llama_config_accepts_rope_scaling_none_and_no_experts(tmp_path):
    p = rewrite_meta(llama_bytes(tmp_path), replace={"llama.rope.scaling.type": (STRING, "none"),
                                                     "llama.expert_count": (U32, 0)})
    assert cfg(GGUFFile(str(p)).llama_config()) == cfg(TINY.config)


@pytest.mark.parametrize("key", ["llama.block_count", "llama.context_length", "llama.feed_forward_length",
                                 "llama.embedding_length", "llama.attention.head_count"])
def test_llama_config_requires_keys(tmp_path, key):
    assert config_kind(rewrite_meta(llama_bytes(tmp_path), drop_keys={key})) == "missingMetadata"


def test_llama_config_requires_2d_embedding(tmp_path):
    assert config_kind(llama_bytes(tmp_path, drop=("token_embd",))) == "missingTensor"
    f = GGUFFile(str(llama_bytes(tmp_path)))
    w = GGUFWriter()
    for k, v in f.metadata.items():
        w.add(k, f.metadata_types[k], v)
    for t in f.tensors:
        dims = [t.dims[0] * t.dims[1]] if t.name == "token_embd.weight" else t.dims
        w.add_tensor(t.name, dims, t.type, f.raw_bytes(t.name).tobytes())
    p = tmp_path / "flat.gguf"
    p.write_bytes(w.build())
    assert config_kind(p) == "malformed"


def test_q4_1_expansion_reference_values():
    """The Python expansion used as the GPU test's reference, on hand-made blocks:
    value = f16(f32(d*q) + m) (LlamaLoader.swift:106-125)."""
    d, m = np.float16(0.5), np.float16(-1.25)
    blk = bytearray(np.array([d, m], np.float16).tobytes()) + bytes((j & 15) | ((15 - (j & 15)) << 4) for j in range(16))
    out = gguf.expand_q4_1(bytes(blk)).astype(np.float32)
    want = [0.5 * (j & 15) - 1.25 for j in range(16)] + [0.5 * (15 - (j & 15)) - 1.25 for j in range(16)]
    assert out.tolist() == want
    # encoder round trip stays within half a step
    v = np.linspace(-1, 1, 64, dtype=np.float32)
    back = gguf.expand_q4_1(gguf.q4_1_blocks(v)).astype(np.float32)
    assert np.abs(back - v).max() <= (2 / 15) / 2 + 2e-3


def test_writer_quant_tensor_bytes_round_trip(tmp_path):
    w = synth.build_weights(TINY)
    f = GGUFFile(str(llama_bytes(tmp_path)))
    t = f.tensor("blk.1.attn_v.weight")
    assert t.dtype == Q8_0 and t.data.tobytes() == w["blk.1.attn_v"].data.tobytes()
