"""Exported ONNX models end to end on the GPU: read by the protobuf-free
reader, optionally optimized by the pass pipeline, run by the executor, and
compared with the logits torch computed for the same models and inputs
(tests/golden/make_onnx_fixtures.py). The unoptimized graphs exercise the
generic ops (decomposed LayerNorm and GELU, unfused attention with
Transpose / batched MatMul / Softmax, the mask arithmetic); the optimized
ones the fused kernels. Tolerance 1e-4 on the logits."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from inferc_amd import rt

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _run_model(ctx, name, optimize, sets):
    g = rt.Graph.from_onnx(GOLDEN / f"{name}.onnx")
    counts = g.optimize() if optimize else None
    ex = rt.Executor(ctx, g)
    io = np.load(GOLDEN / f"{name}_io.npz")
    for tag in sets:
        feeds = {"input_ids": io[f"ids_{tag}"], "attention_mask": io[f"mask_{tag}"]}
        ref = io[f"logits_{tag}"]
        outs = [ex.run(feeds, ["logits"])["logits"] for _ in range(3)]  # eager, capture, replay
        err = float(np.max(np.abs(outs[0] - ref)))
        print(f"{name} optimize={optimize} set={tag}: max|dlogit| {err:.3e}")
        assert outs[0].shape == ref.shape
        assert err <= 1e-4
        for o in outs[1:]:
            np.testing.assert_array_equal(o, outs[0])
    return counts, ex


@pytest.mark.parametrize("optimize", [False, True])
def test_exported_distilbert(ctx, optimize):
    counts, ex = _run_model(ctx, "distilbert_tiny", optimize, ["a", "b"])
    if optimize:
        assert counts["recognize_attention_additive"] == 2


@pytest.mark.parametrize("optimize", [False, True])
def test_exported_gpt2(ctx, optimize):
    _run_model(ctx, "gpt2_tiny", optimize, ["a", "b"])
