"""Synthetic workloads of the benchmark configurations (C1-C5) and small
variants for tests.  No checkpoints or datasets are used: weights are
random-init of the named architecture.

Generator (recorded so any implementation reproduces the bytes):
  * RNG: SplitMix64 (Sampler.swift:30-40), element i of a stream taken from
    the state after i+1 steps; see ahip_synth_* in include/alpaca_hip.h.
  * Tensor k of a model (order: token_embd, then per layer attn_norm, attn_q,
    attn_k, attn_v, attn_output, ffn_norm, ffn_gate, ffn_up, ffn_down, then
    output_norm, then output when untied) uses seed  model_seed*1000003 + k + 1.
  * Projections and embeddings: N(0, 0.02) (Box-Muller in double), quantised
    with the reference quantiser to the config's format.
  * Norm gains: 1.0 (the Hugging Face initialisation; the configs leave the
    norm initialisation open).
  * Prompt token ids: uniform next() % vocab from seed model_seed*1000003 + 999999.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, replace

import numpy as np

from . import _lib as L
from .model import LlamaConfig
from .tensor import F16, F32, Q4_0, Q8_0, QTensor, encode

LAYER_TENSORS = ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm", "ffn_gate", "ffn_up",
                 "ffn_down")


@dataclass(frozen=True)
class ModelSpec:
    name: str
    config: LlamaConfig
    dtype: int
    seed: int
    tied: bool = True
    std: float = 0.02


def _cfg(vocab, hidden, layers, heads, kv, ffn, context, hd=64, theta=1e5):
    return LlamaConfig(vocab_size=vocab, hidden_size=hidden, layer_count=layers, head_count=heads, kv_head_count=kv,
                       head_dim=hd, feed_forward_size=ffn, context_length=context, rms_norm_eps=1e-5,
                       rope_theta=theta, rope_interleaved=True)


# BASELINE.json configs.  Context lengths are the longest position a
# workload reaches, rounded up.
C1 = ModelSpec("C1-135M-Q8_0", _cfg(49152, 576, 30, 9, 3, 1536, 8192), Q8_0, seed=0)
C4 = ModelSpec("C4-360M-Q4_0", _cfg(49152, 960, 32, 15, 5, 2560, 4096), Q4_0, seed=3)
C5 = ModelSpec("C5-1.7B-Q8_0", _cfg(49152, 2048, 24, 32, 32, 8192, 4608), Q8_0, seed=4)
# Small variants with the same structure, for parity tests the oracle runs in seconds.
TINY = ModelSpec("tiny-Q8_0", _cfg(1000, 256, 3, 4, 2, 512, 1024), Q8_0, seed=11, std=0.1)
SPECS = {s.name: s for s in (C1, C4, C5, TINY)}


def with_dtype(spec: ModelSpec, dtype: int) -> ModelSpec:
    return replace(spec, dtype=dtype, name=f"{spec.name.split('-')[0]}-{dtype}")


def tensor_seed(model_seed: int, index: int) -> int:
    return (model_seed * 1000003 + index + 1) & 0xFFFFFFFFFFFFFFFF


def normal(seed: int, n: int, std: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    L.check(L.lib().ahip_synth_normal(seed, 0, n, std, out.ctypes.data_as(L.fp)))
    return out


def uniform(seed: int, n: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    L.check(L.lib().ahip_synth_uniform(seed, 0, n, lo, hi, out.ctypes.data_as(L.fp)))
    return out


def ints(seed: int, n: int, range_: int, bias: int = 0) -> np.ndarray:
    out = np.empty(n, np.int32)
    L.check(L.lib().ahip_synth_ints(seed, 0, n, range_, bias, out.ctypes.data_as(L.ip)))
    return out


def tensor_names(spec: ModelSpec) -> list:
    names = ["token_embd"]
    for i in range(spec.config.layer_count):
        names += [f"blk.{i}.{t}" for t in LAYER_TENSORS]
    names.append("output_norm")
    if not spec.tied:
        names.append("output")
    return names


def tensor_shape(spec: ModelSpec, name: str):
    c = spec.config
    H, QW, KW, F, V = c.hidden_size, c.query_width, c.kv_width, c.feed_forward_size, c.vocab_size
    short = name.split(".")[-1]
    return {"token_embd": (V, H), "output": (V, H), "output_norm": (1, H), "attn_norm": (1, H),
            "ffn_norm": (1, H), "attn_q": (QW, H), "attn_k": (KW, H), "attn_v": (KW, H),
            "attn_output": (H, QW), "ffn_gate": (F, H), "ffn_up": (F, H), "ffn_down": (H, F)}[short]


def build_weights(spec: ModelSpec) -> dict:
    """GGUF-named QTensors of a random-init model in the spec's format."""
    out = {}
    for k, name in enumerate(tensor_names(spec)):
        rows, cols = tensor_shape(spec, name)
        if name.endswith("norm"):
            out[name] = encode(np.ones((1, cols), np.float32), F32)
        else:
            v = normal(tensor_seed(spec.seed, k), rows * cols, spec.std).reshape(rows, cols)
            out[name] = encode(v, spec.dtype)
    return out


def prompt_tokens(spec: ModelSpec, n: int) -> np.ndarray:
    return ints(tensor_seed(spec.seed, 999998), n, spec.config.vocab_size)


# ------------------------------------------------------------------ isolated workloads

def c2_gemm_case(n: int, k: int, m: int = 2048, seed: int = 1):
    """C2: X f32 N(0,1) [m, k]; W Q8_0 [n, k] with q uniform in [-127, 127] and
    d = f16(|N(0, 0.02)| / 127).  Returns (x, QTensor)."""
    x = normal(tensor_seed(seed, 0), m * k, 1.0).reshape(m, k)
    q = ints(tensor_seed(seed, 1), n * k, 255, -127).astype(np.int8).reshape(n * k // 32, 32)
    d = (np.abs(normal(tensor_seed(seed, 2), n * k // 32, 0.02)) / np.float32(127)).astype(np.float16)
    raw = np.empty((n * k // 32, 34), np.uint8)
    raw[:, :2] = d.view(np.uint8).reshape(-1, 2)
    raw[:, 2:] = q.view(np.uint8)
    return x, QTensor(Q8_0, n, k, raw.ravel())


def c3_attention_case(tokens: int = 4096, heads: int = 9, kv_heads: int = 3, hd: int = 64, seed: int = 2):
    """C3: Q [T, 9, 64], K/V [T, 3, 64] f16 N(0,1); RoPE (theta 1e5) is
    applied to Q and K by the caller at positions 0..T-1."""
    q = normal(tensor_seed(seed, 0), tokens * heads * hd, 1.0).astype(np.float16).reshape(tokens, heads, hd)
    k = normal(tensor_seed(seed, 1), tokens * kv_heads * hd, 1.0).astype(np.float16).reshape(tokens, kv_heads, hd)
    v = normal(tensor_seed(seed, 2), tokens * kv_heads * hd, 1.0).astype(np.float16).reshape(tokens, kv_heads, hd)
    return q, k, v
