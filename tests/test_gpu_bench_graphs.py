"""The executor graphs bench.py times for BASELINE configs 2 and 3, run the
way the bench runs them (device inputs; eager, then captured, then replayed)
and checked against the CPU oracle at max-abs-diff <= 1e-4:

- config 2: FusedMatMulAddGELU -> MatMul -> Add -> FusedLayerNorm (the
  MatMul + Add fold into one GEMM epilogue), M in {128, 1024, 4096};
  fused_matmul_add_gelu.cc:13-80, matmul.cc:63-159, activation.cc:103-150;
- config 3: FusedQKV -> FusedAttention with a bool graph-input padding mask,
  B = 32, S in {128, 512}; attention.cc:32-141.

Executor dispatch: src/runtime/executor.cc:206-233."""
from __future__ import annotations

import numpy as np
import pytest

import bench
import oracle as O
from inferc_amd import graphs, rt

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _runs(ctx, g, inputs: dict, out: str, n: int = 3):
    """Outputs of n runs of one executor: eager, captured, replayed."""
    ex = rt.Executor(ctx, g)
    keep = bench.device_inputs(ctx, ex, inputs)
    got = []
    for _ in range(n):
        ex.run_async()
        got.append(ex.output(out))
    del keep
    ex.close()
    return got


@pytest.mark.parametrize("M", [128, 1024, 4096])
def test_config2_ffn_ln_graph_vs_oracle(ctx, M):
    g, x = bench.ffn_ln_graph(M)
    seed, n = 3, graphs.normal
    w1, b1 = n(seed, "w1", (768, 3072)), n(seed, "b1", (3072,))
    w2, b2 = n(seed, "w2", (3072, 768)), n(seed, "b2", (768,))
    f = O.fused_matmul_add_gelu(x, w1, b1)
    y = O.matmul(f, w2) + b2
    ref = O.layernorm(y, np.ones(768, np.float32), np.zeros(768, np.float32), 1e-12)
    runs = _runs(ctx, g, {"x": x}, "out")
    for i, got in enumerate(runs):
        d = float(np.max(np.abs(got - ref)))
        assert d <= TOL, f"run {i}: max|d| = {d:.3e}"
    np.testing.assert_array_equal(runs[1], runs[2])


@pytest.mark.parametrize("S", [128, 512])
def test_config3_qkv_mha_graph_vs_oracle(ctx, S):
    g, x, mask, lens = bench.qkv_mha_graph(S)
    seed = 4
    w = {nm: graphs.normal(seed, nm, (768, 768)) for nm in ("wq", "wk", "wv")}
    b = {nm: graphs.normal(seed, nm, (768,)) for nm in ("bq", "bk", "bv")}
    q, k, v = O.fused_qkv(x, w["wq"], b["bq"], w["wk"], b["bk"], w["wv"], b["bv"])
    ref = O.fused_attention(q, k, v, mask, 64, graphs.FILL_MIN)
    assert lens.min() >= 16 and lens.max() <= S
    runs = _runs(ctx, g, {"x": x, "mask": mask}, "ctx")
    for i, got in enumerate(runs):
        d = float(np.max(np.abs(got - ref)))
        assert d <= TOL, f"run {i}: max|d| = {d:.3e}"
    np.testing.assert_array_equal(runs[1], runs[2])
