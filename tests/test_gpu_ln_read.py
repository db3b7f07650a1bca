"""LayerNorms applied by their readers (executor): a FusedGemmEpilogue
writes the row statistics of its output h, and the GEMMs that read the
LayerNorm of h (A of FusedQKV, FusedMatMulAddGELU or FusedGemmEpilogue, the
residual of a FusedGemmEpilogue) normalize h as they read it, so the LayerNorm kernel does
not run. That holds while every product takes the small-M path (M <= 512);
above it the LayerNorm kernel runs as before. Both against a float64
statement of the unfused graph (src/kernels/activation.cc:103-150 for the
LayerNorm, fused_matmul_add_gelu.cc for the GELU epilogue), 1e-4."""
from __future__ import annotations

import math

import numpy as np
import pytest

from inferc_amd import rt

pytestmark = pytest.mark.gpu

H, F = 128, 512


def _w(rng, *shape, std=0.05):
    return (rng.standard_normal(shape) * std).astype(np.float32)


def _graph(rng):
    """out-proj(+x0) -> LN1 -> {QKV, FFN-up -> FFN-down(+LN1), a plain
    projection} -> LN2 -> out-proj(+LN2) -> LN3. LN1 and LN2 are read by GEMMs
    only; LN3 is an output and stays a kernel."""
    g = rt.Graph()
    p = {}
    for nm, shape in [("wo", (H, H)), ("bo", (H,)), ("wq", (H, H)), ("bq", (H,)),
                      ("wk", (H, H)), ("bk", (H,)), ("wv", (H, H)), ("bv", (H,)),
                      ("w1", (H, F)), ("c1", (F,)), ("w2", (F, H)), ("c2", (H,)),
                      ("wo2", (H, H)), ("bo2", (H,)), ("wz", (H, 2 * H)), ("bz", (2 * H,))]:
        p[nm] = _w(rng, *shape)
    for i in (1, 2, 3):
        p[f"g{i}"] = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        p[f"b{i}"] = (0.1 * rng.standard_normal(H)).astype(np.float32)
    for nm, v in p.items():
        g.add_initializer(nm, v)
    g.add_node("FusedGemmEpilogue", ["a", "wo", "bo", "x0"], ["h1"])
    g.add_node("FusedLayerNorm", ["h1", "g1", "b1"], ["x1"], epsilon=1e-12)
    g.add_node("FusedQKV", ["x1", "wq", "bq", "wk", "bk", "wv", "bv"], ["q", "k", "v"])
    g.add_node("FusedMatMulAddGELU", ["x1", "w1", "c1"], ["f"])
    g.add_node("FusedGemmEpilogue", ["x1", "wz", "bz"], ["z"])
    g.add_node("FusedGemmEpilogue", ["f", "w2", "c2", "x1"], ["h2"])
    g.add_node("FusedLayerNorm", ["h2", "g2", "b2"], ["x2"], epsilon=1e-5)
    g.add_node("FusedGemmEpilogue", ["a2", "wo2", "bo2", "x2"], ["h3"])
    g.add_node("FusedLayerNorm", ["h3", "g3", "b3"], ["x3"], epsilon=1e-5)
    for o in ("q", "k", "v", "z", "x3"):
        g.add_output(o)
    return g, p


def _ln(x, g, b, eps):
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * g + b


def _reference(p, x0, a, a2):
    d = {k: v.astype(np.float64) for k, v in p.items()}
    erf = np.vectorize(math.erf)
    h1 = a @ d["wo"] + d["bo"] + x0
    x1 = _ln(h1, d["g1"], d["b1"], 1e-12)
    q, k, v = (x1 @ d["w" + t] + d["b" + t] for t in "qkv")
    z = x1 @ d["wz"] + d["bz"]
    u = x1 @ d["w1"] + d["c1"]
    f = 0.5 * u * (1.0 + erf(u / math.sqrt(2.0)))
    h2 = f @ d["w2"] + d["c2"] + x1
    x2 = _ln(h2, d["g2"], d["b2"], 1e-5)
    h3 = a2 @ d["wo2"] + d["bo2"] + x2
    return {"q": q, "k": k, "v": v, "z": z, "x3": _ln(h3, d["g3"], d["b3"], 1e-5)}


@pytest.mark.parametrize("M", [1, 7, 128, 512, 600])
def test_layernorm_read_by_gemms(ctx, M):
    rng = np.random.default_rng(31 + M)
    g, p = _graph(rng)
    ex = rt.Executor(ctx, g)
    feeds = {"x0": rng.standard_normal((M, H)).astype(np.float32),
             "a": rng.standard_normal((M, H)).astype(np.float32),
             "a2": rng.standard_normal((M, H)).astype(np.float32)}
    # shift the rows off zero mean so the statistics carry real offsets
    feeds["x0"] += np.float32(3.0)
    ref = _reference(p, *(feeds[k].astype(np.float64) for k in ("x0", "a", "a2")))
    names = ["q", "k", "v", "z", "x3"]
    runs = [ex.run(feeds, names) for _ in range(3)]  # eager, capture, replay
    for nm in names:
        err = float(np.max(np.abs(runs[0][nm] - ref[nm])))
        print(f"M={M} {nm}: max|d| {err:.2e}")
        assert err <= 1e-4, nm
        for r in runs[1:]:
            np.testing.assert_array_equal(r[nm], runs[0][nm])


def test_two_layernorms_of_one_input_stay_kernels(ctx):
    """Two LayerNorms (different gamma/beta) of one GEMM output, each read by
    a GEMM: both are computed by the LayerNorm kernel."""
    rng = np.random.default_rng(5)
    M = 32
    p = {"wo": _w(rng, H, H), "bo": _w(rng, H), "w1": _w(rng, H, F), "c1": _w(rng, F),
         "wz": _w(rng, H, H), "bz": _w(rng, H)}
    for i in (1, 2):
        p[f"g{i}"] = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        p[f"b{i}"] = (0.1 * rng.standard_normal(H)).astype(np.float32)
    g = rt.Graph()
    for nm, v in p.items():
        g.add_initializer(nm, v)
    g.add_node("FusedGemmEpilogue", ["a", "wo", "bo", "x0"], ["h"])
    g.add_node("FusedLayerNorm", ["h", "g1", "b1"], ["x1"], epsilon=1e-5)
    g.add_node("FusedLayerNorm", ["h", "g2", "b2"], ["x2"], epsilon=1e-5)
    g.add_node("FusedMatMulAddGELU", ["x1", "w1", "c1"], ["f"])
    g.add_node("FusedGemmEpilogue", ["x2", "wz", "bz"], ["z"])
    g.add_output("f")
    g.add_output("z")
    feeds = {"x0": rng.standard_normal((M, H)).astype(np.float32),
             "a": rng.standard_normal((M, H)).astype(np.float32)}
    d = {k: v.astype(np.float64) for k, v in p.items()}
    h = feeds["a"].astype(np.float64) @ d["wo"] + d["bo"] + feeds["x0"]
    u = _ln(h, d["g1"], d["b1"], 1e-5) @ d["w1"] + d["c1"]
    erf = np.vectorize(math.erf)
    ref = {"f": 0.5 * u * (1.0 + erf(u / math.sqrt(2.0))),
           "z": _ln(h, d["g2"], d["b2"], 1e-5) @ d["wz"] + d["bz"]}
    ex = rt.Executor(ctx, g)
    for _ in range(3):
        got = ex.run(feeds, ["f", "z"])
        for nm in ("f", "z"):
            assert float(np.max(np.abs(got[nm] - ref[nm]))) <= 1e-4, nm
