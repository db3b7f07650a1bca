"""Executor host logic without a GPU (dry-run executor): shape inference over
the fused encoder graph, integer shape plumbing, peephole fusion counts, and
the reference's error behaviour for unsupported ops / missing tensors
(src/runtime/executor.cc:104-110,340-343)."""
from __future__ import annotations

import numpy as np
import pytest

from inferc_amd import graphs
from inferc_amd import lib as L
from inferc_amd.rt import Executor, Graph


@pytest.fixture(scope="module", autouse=True)
def _lib():
    if not L.library_path().exists():
        from inferc_amd.build import build

        build()


def test_encoder_graph_shapes_and_fusion():
    cfg = graphs.small_encoder_cfg()
    g = graphs.encoder_graph(cfg, graphs.encoder_weights(cfg, 3))
    n_nodes = len(g.op_types)
    ex = Executor.dry(g)
    # per layer the two MatMul->Add->Add chains fold into one GEMM each,
    # Gemm->Relu folds once, the embedding Add joins its LayerNorm and the
    # last LayerNorm moves behind the CLS Gather into the head Gemm:
    # 4 nodes removed per layer + 3
    assert ex.node_count() == n_nodes - 4 * cfg["layers"] - 3
    ids, mask = graphs.encoder_inputs(cfg, 3, 21)
    ex.set_input("input_ids", ids)
    ex.set_input("attention_mask", mask)
    ex.run_async()
    assert ex.output_shape("logits") == ((3, 2), np.dtype(np.float32))


def test_shape_plumbing_ops():
    g = Graph()
    g.add_initializer("one", np.array(1, np.int64))
    g.add_initializer("zero", np.array(0, np.int64))
    g.add_node("Shape", ["x"], ["s"])
    g.add_node("Gather", ["s", "one"], ["n"], axis=0)
    g.add_node("Range", ["zero", "n", "one"], ["r"])
    g.add_node("Unsqueeze", ["r"], ["r2"], axes=[0, 2])
    g.add_node("Reshape", ["x", "s"], ["x2"])
    g.add_node("Squeeze", ["r2"], ["r3"], axes=[0])
    for o in ("s", "n", "r", "r2", "x2", "r3"):
        g.add_output(o)
    ex = Executor.dry(g)
    ex.set_input("x", np.zeros((4, 9, 2), np.float32))
    ex.run_async()
    assert ex.output_shape("s")[0] == (3,)
    assert ex.output_shape("n")[0] == ()
    assert ex.output_shape("r")[0] == (9,)
    assert ex.output_shape("r2")[0] == (1, 9, 1)
    assert ex.output_shape("r3")[0] == (9, 1)
    assert ex.output_shape("x2")[0] == (4, 9, 2)


def test_matmul_batched_and_broadcast_shapes():
    g = Graph()
    g.add_initializer("w", np.zeros((5, 7), np.float32))
    g.add_node("MatMul", ["a", "w"], ["y"])
    g.add_node("MatMul", ["a", "b"], ["z"])
    g.add_output("y")
    g.add_output("z")
    ex = Executor.dry(g)
    ex.set_input("a", np.zeros((2, 3, 4, 5), np.float32))
    ex.set_input("b", np.zeros((2, 3, 5, 6), np.float32))
    ex.run_async()
    assert ex.output_shape("y")[0] == (2, 3, 4, 7)
    assert ex.output_shape("z")[0] == (2, 3, 4, 6)


def test_errors_follow_the_reference():
    g = Graph()
    g.add_node("NonZero", ["x"], ["y"])
    ex = Executor.dry(g)
    ex.set_input("x", np.ones(3, np.float32))
    with pytest.raises(RuntimeError, match="unsupported op 'NonZero'") as e:
        ex.run_async()
    assert e.value.code == L.ERR_UNSUPPORTED
    g2 = Graph()
    g2.add_node("Relu", ["missing"], ["y"])
    ex2 = Executor.dry(g2)
    with pytest.raises(RuntimeError, match="missing tensor 'missing'") as e:
        ex2.run_async()
    assert e.value.code == L.ERR_STATE
    g3 = Graph()
    g3.add_initializer("w", np.zeros((4, 3), np.float32))
    g3.add_node("FusedMatMulAddGELU", ["x", "w", "b"], ["y"])
    g3.add_initializer("b", np.zeros(3, np.float32))
    ex3 = Executor.dry(g3)
    ex3.set_input("x", np.zeros((2, 5), np.float32))
    with pytest.raises(RuntimeError, match="K mismatch"):
        ex3.run_async()


def test_peephole_keeps_shared_intermediates():
    """A MatMul output read twice must not be folded into its Add."""
    g = Graph()
    g.add_initializer("w", np.zeros((4, 4), np.float32))
    g.add_initializer("b", np.zeros(4, np.float32))
    g.add_node("MatMul", ["x", "w"], ["m"])
    g.add_node("Add", ["m", "b"], ["y"])
    g.add_node("Relu", ["m"], ["z"])
    g.add_output("y")
    g.add_output("z")
    ex = Executor.dry(g)
    assert ex.node_count() == 3


def test_peephole_folds_add_into_layernorm_with_broadcast():
    """Add(x[B,S,H], p[1,S,H]) -> LayerNorm becomes one LayerNorm whose
    residual repeats over the batch; a sum that is read twice stays an Add."""
    def graph(sum_is_output: bool) -> Graph:
        g = Graph()
        g.add_initializer("gamma", np.ones(8, np.float32))
        g.add_initializer("beta", np.zeros(8, np.float32))
        g.add_node("Add", ["x", "p"], ["s"])
        g.add_node("FusedLayerNorm", ["s", "gamma", "beta"], ["y"], epsilon=1e-12)
        g.add_output("y")
        if sum_is_output:
            g.add_output("s")
        return g

    ex = Executor.dry(graph(False))
    assert ex.node_count() == 1
    ex.set_input("x", np.zeros((3, 5, 8), np.float32))
    ex.set_input("p", np.zeros((1, 5, 8), np.float32))
    ex.run_async()
    assert ex.output_shape("y") == ((3, 5, 8), np.dtype(np.float32))
    assert Executor.dry(graph(True)).node_count() == 2


# (data shape, Gather axis, constant indices): the Gather feeds the Gemm
# directly with a 2-D result. Rows: the encoder head's CLS select; a scalar
# select on the feature axis (K = S != H); a feature-axis permutation whose
# count equals H (the case a blind fold would get silently wrong); a row select.
LN_GATHER_CASES = [((2, 5, 8), 1, 0), ((2, 5, 8), -1, 3), ((6, 8), 1, [3, 1, 2, 7, 0, 4, 6, 5]),
                   ((6, 8), 0, [4, 0, 2])]


@pytest.mark.parametrize("shape,axis,idx", LN_GATHER_CASES)
def test_layernorm_gather_gemm_peephole_respects_axis(shape, axis, idx):
    """LayerNorm -> Gather(constant) -> Gemm(transB): the executor moves the
    LayerNorm into the Gemm only where the two commute (a Gather that keeps
    whole feature rows); a feature-axis Gather applies it itself, so planning
    a K != H product does not fail on the LayerNorm's scale size."""
    H = shape[-1]
    sel = np.take(np.zeros(shape), np.asarray(idx), axis=axis)
    g = Graph()
    g.add_initializer("g", np.ones(H, np.float32))
    g.add_initializer("b", np.zeros(H, np.float32))
    g.add_initializer("ix", np.asarray(idx, np.int64))
    g.add_initializer("W", np.zeros((3, sel.shape[1]), np.float32))
    g.add_node("FusedLayerNorm", ["x", "g", "b"], ["xn"], epsilon=1e-5)
    g.add_node("Gather", ["xn", "ix"], ["sel"], axis=axis)
    g.add_node("Gemm", ["sel", "W"], ["y"], transB=1)
    g.add_output("y")
    ex = Executor.dry(g)
    assert ex.node_count() == 2  # the LayerNorm moved (the Gather may take it back)
    ex.set_input("x", np.zeros(shape, np.float32))
    ex.run_async()
    assert ex.output_shape("y") == ((sel.shape[0], 3), np.dtype(np.float32))
