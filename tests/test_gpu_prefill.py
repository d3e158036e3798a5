"""The fast prefill's fused QKV epilogue: RoPE and the KV-cache append done by
the QKV GEMM (GEMM_QKV_ROPE) instead of a separate kernel over an f32 q/k/v
buffer.  The epilogue evaluates the rotation in the unfused kernel's order on
the same float32 accumulators, so a fused session and an unfused one
(ALPACA_HIP_FUSE_QKV_ROPE=0, read at session creation) must agree bit for bit:
the prefill logits (which read q through attention) and the decode steps after
it (which read the cached k/v rows), across two chunks so the second starts at
a non-zero position.
"""
from dataclasses import replace

import numpy as np
import pytest

from alpaca_amd import synth
from alpaca_amd.model import HIPLlamaModel
from alpaca_amd.tensor import F16, Q4_0
from tests.helpers import env
from tests.test_gpu_model import built

pytestmark = pytest.mark.gpu

SPECS = [
    synth.TINY,
    synth.with_dtype(synth.TINY, F16),
    replace(synth.TINY, config=replace(synth.TINY.config, head_dim=128), name="tiny-hd128"),
    # C4's layer shape (hidden 960, 15/5 heads, Q4_0) with 2 layers: N = 1600 leaves a partial tile
    replace(synth.C4, config=replace(synth.C4.config, layer_count=2, vocab_size=2048, context_length=512),
            name="c4-shape-2l"),
]


@pytest.mark.parametrize("spec", SPECS, ids=lambda s: s.name)
def test_fused_qkv_rope_is_bit_identical_to_unfused(hip_ctx, spec):
    model = HIPLlamaModel(hip_ctx, spec.config, built(spec))
    prompt = synth.prompt_tokens(spec, 150)
    with env(ALPACA_HIP_FUSE_QKV_ROPE=0):
        ref = model.make_session(capacity=200, gemm_precision="fast")
    fused = model.make_session(capacity=200, gemm_precision="fast")
    for chunk in (prompt[:70], prompt[70:]):  # the second chunk starts at position 70
        a, b = fused.forward(chunk), ref.forward(chunk)
        assert np.array_equal(a, b), f"prefill logits differ: max |d| {np.abs(a - b).max():.3e}"
    tok = int(np.argmax(a))
    for step in range(3):
        a, b = fused.decode(tok), ref.decode(tok)
        assert np.array_equal(a, b), f"decode step {step} differs: max |d| {np.abs(a - b).max():.3e}"
        tok = int(np.argmax(a))
