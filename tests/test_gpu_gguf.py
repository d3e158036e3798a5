"""Models loaded from GGUF files (ahip_model_load_gguf: LlamaLoader.load then
model creation) against the same weights handed over in memory.

The loader copies each tensor from the file mapping to HBM in its on-disk
format, so a loaded model must produce logits bit for bit equal to the
in-memory model's, prefill and decode alike.  Q4_1 tensors are expanded to F16
at load (LlamaLoader.swift:106-125: f16(d*q + m) in float32); the loaded model
must equal an in-memory model given the F16 values of that formula, computed in
numpy, and the load report must list each expanded tensor.  The stacked
q/k/v projection and the gate/up pair run as one matrix each here, so their
members must share a format: a file that expands only some of them is refused
as unsupported.
"""
from dataclasses import replace

import numpy as np
import pytest

from alpaca_amd import gguf, synth
from alpaca_amd._lib import GGUFError, Unsupported
from alpaca_amd.model import HIPLlamaModel
from alpaca_amd.tensor import F16, Q4_0, QTensor
from tests.test_gpu_model import built

pytestmark = pytest.mark.gpu

SPECS = [synth.TINY, synth.with_dtype(synth.TINY, Q4_0), synth.with_dtype(synth.TINY, F16),
         replace(synth.TINY, tied=False, name="tiny-untied")]


def logits_of(model, spec):
    s = model.make_session(capacity=64, gemm_precision="fast")
    a = s.forward(synth.prompt_tokens(spec, 20))
    b = s.decode(int(np.argmax(a)))
    e = model.make_session(capacity=64, gemm_precision="exact")
    c = e.forward(synth.prompt_tokens(spec, 20))
    return a, b, c


@pytest.mark.parametrize("spec", SPECS, ids=lambda s: s.name)
def test_loaded_model_equals_in_memory_model(hip_ctx, tmp_path, spec):
    w = built(spec)
    path = tmp_path / f"{spec.name}.gguf"
    gguf.write_llama(str(path), spec.config, w)
    model, config, report = gguf.load_llama(hip_ctx, str(path))
    assert config == replace(spec.config, rms_norm_eps=config.rms_norm_eps)  # eps travels as f32
    assert report.mapped_weight_bytes == sum(t.data.nbytes for t in w.values()) and report.converted_weight_bytes == 0
    ref = HIPLlamaModel(hip_ctx, config, w)
    for got, want in zip(logits_of(model, spec), logits_of(ref, spec)):
        assert np.array_equal(got, want)


def test_q4_1_tensors_are_expanded_to_f16(hip_ctx, tmp_path):
    spec = synth.TINY
    w = dict(built(spec))
    names = ["blk.0.attn_output", "blk.2.ffn_down"]
    raw, ref_w = {}, dict(w)
    for n in names:
        t = w[n]
        vals = synth.normal(synth.tensor_seed(spec.seed, 777 + len(raw)), t.rows * t.cols, spec.std)
        raw[n] = gguf.q4_1_blocks(vals)
        ref_w[n] = QTensor(F16, t.rows, t.cols, gguf.expand_q4_1(raw[n]))
    path = tmp_path / "q41.gguf"
    gguf.write_llama(str(path), spec.config, w, q4_1=raw)
    model, config, report = gguf.load_llama(hip_ctx, str(path))
    assert report.converted_weight_bytes == sum(ref_w[n].data.nbytes for n in names)
    assert len(report.notes) == 2 and all("Q4_1 expanded to F16" in x for x in report.notes)
    ref = HIPLlamaModel(hip_ctx, config, ref_w)
    for got, want in zip(logits_of(model, spec), logits_of(ref, spec)):
        assert np.array_equal(got, want)


def test_mixed_formats_in_a_stacked_group_are_refused(hip_ctx, tmp_path):
    spec = synth.TINY
    w = built(spec)
    t = w["blk.1.attn_k"]
    raw = {"blk.1.attn_k": gguf.q4_1_blocks(synth.normal(3, t.rows * t.cols, spec.std))}
    path = tmp_path / "mixed.gguf"
    gguf.write_llama(str(path), spec.config, w, q4_1=raw)
    with pytest.raises(Unsupported, match="share one format"):
        gguf.load_llama(hip_ctx, str(path))


def test_loader_refuses_incomplete_models(hip_ctx, tmp_path):
    spec = synth.TINY
    w = dict(built(spec))
    w.pop("blk.1.ffn_down")
    path = tmp_path / "missing.gguf"
    gguf.write_llama(str(path), spec.config, w)
    with pytest.raises(GGUFError) as e:
        gguf.load_llama(hip_ctx, str(path))
    assert e.value.kind == "missingTensor" and "blk.1.ffn_down.weight" in str(e.value)
    w = dict(built(spec))
    w["blk.0.attn_norm"] = QTensor(F16, 1, spec.config.hidden_size,
                                   np.ones(spec.config.hidden_size, np.float16).view(np.uint8))
    path = tmp_path / "f16norm.gguf"
    gguf.write_llama(str(path), spec.config, w)
    with pytest.raises(GGUFError) as e:
        gguf.load_llama(hip_ctx, str(path))
    assert e.value.kind == "unsupportedModel" and "expected F32" in str(e.value)
