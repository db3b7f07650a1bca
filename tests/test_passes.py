"""Fusion passes on the graph IR (no GPU): the reference's pass tests
(tests/passes_test.cc:59-337) ported case by case, the attention / QKV /
tanh-GELU matchers it has no unit tests for (src/ir/passes/
recognize_attention.cc, recognize_gelu.cc:165-296) on graphs in the exported
patterns those passes document, the additive-mask attention form, and the
whole pipeline on the exported fixture models."""
from __future__ import annotations

from collections import Counter
from pathlib import Path

import numpy as np
import pytest

from inferc_amd import lib as L
from inferc_amd.rt import PASSES, Graph

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    if not L.library_path().exists():
        from inferc_amd.build import build

        build()


def f32(v):
    return np.array(v, np.float32)


def ops(g: Graph) -> list[str]:
    return [n["op"] for n in g.to_dict()["nodes"]]


def node_of(g: Graph, op: str) -> dict:
    found = [n for n in g.to_dict()["nodes"] if n["op"] == op]
    assert len(found) == 1, found
    return found[0]


# ---------------------------------------------------------------- RecognizeGelu

def gelu_graph(sqrt2=1.41421356, const_first=False, extra_sink=False) -> Graph:
    g = Graph()
    g.add_constant("c_sqrt2", f32(sqrt2))
    g.add_constant("c_one", f32(1.0))
    g.add_constant("c_half", f32(0.5))
    g.add_node("Div", ["X", "c_sqrt2"], ["div_out"])
    g.add_node("Erf", ["div_out"], ["erf_out"])
    g.add_node("Add", ["c_one", "erf_out"] if const_first else ["erf_out", "c_one"], ["plus_one"])
    g.add_node("Mul", ["X", "plus_one"], ["mul1_out"])
    g.add_node("Mul", ["c_half", "mul1_out"] if const_first else ["mul1_out", "c_half"], ["Y"])
    if extra_sink:
        g.add_node("Identity", ["div_out"], ["sink"])
    g.add_output("Y")
    return g


def test_gelu_folds_exact_erf_chain():
    g = gelu_graph()
    assert g.run_pass("recognize_gelu") == 1
    d = g.to_dict()["nodes"]
    assert len(d) == 1
    assert d[0]["op"] == "Gelu" and d[0]["inputs"] == ["X"] and d[0]["outputs"] == ["Y"]


def test_gelu_add_operand_order_tolerant():
    g = gelu_graph(const_first=True)
    assert g.run_pass("recognize_gelu") == 1
    assert ops(g) == ["Gelu"]


def test_gelu_bails_on_wrong_constant():
    g = gelu_graph(sqrt2=1.5)
    assert g.run_pass("recognize_gelu") == 0
    assert len(ops(g)) == 8


def test_gelu_bails_on_extra_consumer():
    g = gelu_graph(extra_sink=True)
    assert g.run_pass("recognize_gelu") == 0


def test_gelu_keeps_a_constant_that_something_else_reads():
    g = gelu_graph()
    g.add_node("Add", ["Y", "c_one"], ["Z"])  # c_one has a reader outside the chain
    assert g.run_pass("recognize_gelu") == 1
    assert ops(g) == ["Constant", "Gelu", "Add"]


# ---------------------------------------------------------- FuseMatMulAddGelu

def mm_add_gelu(bias_first=False) -> Graph:
    g = Graph()
    g.add_node("MatMul", ["X", "W"], ["mm_out"])
    g.add_node("Add", ["B", "mm_out"] if bias_first else ["mm_out", "B"], ["add_out"])
    g.add_node("Gelu", ["add_out"], ["Y"])
    g.add_output("Y")
    return g


def test_fuse_matmul_add_gelu_simple_triplet():
    g = mm_add_gelu()
    assert g.run_pass("fuse_matmul_add_gelu") == 1
    (n,) = g.to_dict()["nodes"]
    assert n["op"] == "FusedMatMulAddGELU" and n["domain"] == "inferc"
    assert n["inputs"] == ["X", "W", "B"] and n["outputs"] == ["Y"]


def test_fuse_matmul_add_gelu_bias_operand_order():
    g = mm_add_gelu(bias_first=True)
    assert g.run_pass("fuse_matmul_add_gelu") == 1
    assert g.to_dict()["nodes"][0]["inputs"][2] == "B"


def test_fuse_matmul_add_gelu_bails_on_extra_consumer():
    g = mm_add_gelu()
    g.add_output("mm_out")
    assert g.run_pass("fuse_matmul_add_gelu") == 0
    g.add_node("Identity", ["mm_out"], ["sink"])
    assert g.run_pass("fuse_matmul_add_gelu") == 0


def test_fuse_matmul_add_gelu_no_match_without_gelu():
    g = Graph()
    g.add_node("MatMul", ["X", "W"], ["mm_out"])
    g.add_node("Add", ["mm_out", "B"], ["add_out"])
    g.add_output("add_out")
    assert g.run_pass("fuse_matmul_add_gelu") == 0
    assert "FusedMatMulAddGELU" not in ops(g)


# ------------------------------------------------------- FoldConstantTranspose

def test_fold_constant_transpose():
    g = Graph()
    g.add_initializer("W", f32([[1, 2, 3], [4, 5, 6]]))
    g.add_node("Transpose", ["W"], ["Wt"], perm=[1, 0])
    g.add_node("Identity", ["Wt"], ["Wt_consumer"])
    g.add_output("Wt_consumer")
    assert g.run_pass("fold_constant_transpose") == 1
    assert ops(g) == ["Identity"]
    np.testing.assert_array_equal(g.initializer("Wt"), f32([[1, 4], [2, 5], [3, 6]]))
    np.testing.assert_array_equal(g.initializer("W"), f32([[1, 2, 3], [4, 5, 6]]))


def test_fold_constant_transpose_rank3_and_default_perm():
    a = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    g = Graph()
    g.add_initializer("A", a)
    g.add_node("Transpose", ["A"], ["At"], perm=[2, 0, 1])
    g.add_node("Transpose", ["A"], ["Ar"])  # no perm: reverse the axes
    g.add_node("Add", ["At", "At"], ["s1"])
    g.add_node("Add", ["Ar", "Ar"], ["s2"])
    g.add_output("s1")
    g.add_output("s2")
    assert g.run_pass("fold_constant_transpose") == 2
    np.testing.assert_array_equal(g.initializer("At"), a.transpose(2, 0, 1))
    np.testing.assert_array_equal(g.initializer("Ar"), a.transpose())


def test_fold_constant_transpose_skips_activation_and_graph_output():
    g1 = Graph()
    g1.add_node("Transpose", ["A"], ["At"], perm=[1, 0])
    g1.add_node("Identity", ["At"], ["At_sink"])
    g1.add_output("At_sink")
    assert g1.run_pass("fold_constant_transpose") == 0
    assert ops(g1).count("Transpose") == 1
    g2 = Graph()
    g2.add_initializer("W", f32([[1, 2], [3, 4]]))
    g2.add_node("Transpose", ["W"], ["Wt"], perm=[1, 0])
    g2.add_output("Wt")
    assert g2.run_pass("fold_constant_transpose") == 0
    assert ops(g2) == ["Transpose"]


# ---------------------------------------------------------- RecognizeLayerNorm

def layernorm_graph(eps: float, use_pow: bool, gamma_init: bool = True) -> Graph:
    g = Graph()
    if gamma_init:
        g.add_initializer("gamma", f32([1, 1, 1, 1]))
    g.add_initializer("beta", f32([0, 0, 0, 0]))
    g.add_node("ReduceMean", ["X"], ["mean"])
    g.add_node("Sub", ["X", "mean"], ["d"])
    if use_pow:
        g.add_constant("two", f32(2.0))
        g.add_node("Pow", ["d", "two"], ["sq"])
    else:
        g.add_node("Mul", ["d", "d"], ["sq"])
    g.add_node("ReduceMean", ["sq"], ["var"])
    g.add_constant("eps", f32(eps))
    g.add_node("Add", ["var", "eps"], ["veps"])
    g.add_node("Sqrt", ["veps"], ["std"])
    g.add_node("Div", ["d", "std"], ["norm"])
    g.add_node("Mul", ["norm", "gamma"], ["sc"])
    g.add_node("Add", ["sc", "beta"], ["Y"])
    g.add_output("Y")
    return g


def test_layernorm_folds_pow_variant():
    g = layernorm_graph(1e-5, use_pow=True)
    before = len(ops(g))
    assert g.run_pass("recognize_layernorm") == 1
    after = ops(g)
    assert after == ["FusedLayerNorm"] and len(after) < before
    n = node_of(g, "FusedLayerNorm")
    assert n["domain"] == "inferc" and n["inputs"] == ["X", "gamma", "beta"]
    assert n["outputs"] == ["Y"]
    assert abs(float(n["attrs"]["epsilon"]) - 1e-5) <= 1e-9
    assert np.float32(float(n["attrs"]["epsilon"])) == np.float32(1e-5)


def test_layernorm_folds_mul_variant():
    g = layernorm_graph(1e-12, use_pow=False)
    assert g.run_pass("recognize_layernorm") == 1
    assert ops(g).count("FusedLayerNorm") == 1


def test_layernorm_no_match_if_gamma_not_initializer():
    g = layernorm_graph(1e-5, use_pow=True, gamma_init=False)
    g.add_input("gamma", np.float32, [4])
    assert g.run_pass("recognize_layernorm") == 0
    assert "FusedLayerNorm" not in ops(g)


def test_layernorm_rejects_out_of_range_epsilon():
    assert layernorm_graph(0.5, use_pow=True).run_pass("recognize_layernorm") == 0


# ---------------------------------------------------------- RecognizeGeluTanh

def gelu_tanh_graph(coef=0.044715) -> Graph:
    """0.5x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 x^3))) as GPT-2 exports it
    (recognize_gelu.h:24-33)."""
    g = Graph()
    g.add_constant("c_half", f32(0.5))
    g.add_node("Mul", ["X", "c_half"], ["halfx"])
    g.add_constant("c_three", f32(3.0))
    g.add_node("Pow", ["X", "c_three"], ["cube"])
    g.add_constant("c_coef", f32(coef))
    g.add_node("Mul", ["cube", "c_coef"], ["m1"])
    g.add_node("Add", ["X", "m1"], ["inner"])
    g.add_constant("c_s", f32(0.7978845608))
    g.add_node("Mul", ["inner", "c_s"], ["m2"])
    g.add_node("Tanh", ["m2"], ["t"])
    g.add_constant("c_one", f32(1.0))
    g.add_node("Add", ["t", "c_one"], ["a1"])
    g.add_node("Mul", ["halfx", "a1"], ["Y"])
    g.add_output("Y")
    return g


def test_gelu_tanh_folds_gpt2_chain():
    g = gelu_tanh_graph()
    assert g.run_pass("recognize_gelu_tanh") == 1
    (n,) = g.to_dict()["nodes"]
    assert n["op"] == "GeluTanh" and n["domain"] == "inferc"
    assert n["inputs"] == ["X"] and n["outputs"] == ["Y"]


def test_gelu_tanh_bails_on_wrong_coefficient():
    g = gelu_tanh_graph(coef=0.05)
    assert g.run_pass("recognize_gelu_tanh") == 0
    assert len(ops(g)) == 13


# ------------------------------------------- RecognizeAttention + FuseQKV

def _proj(g: Graph, p: str, x: str, H: int, rng) -> None:
    g.add_initializer(f"W{p}", rng.standard_normal((H, H)).astype(np.float32))
    g.add_initializer(f"b{p}", rng.standard_normal(H).astype(np.float32))
    g.add_node("MatMul", [x, f"W{p}"], [f"{p}_mm"])
    g.add_node("Add", [f"b{p}", f"{p}_mm"], [f"{p}p"])
    g.add_node("Reshape", [f"{p}p", "shape4"], [f"{p}_r"])


def where_attention_graph(H=64, heads=4, shared_x=True) -> Graph:
    """The BERT block the reference's matcher documents
    (recognize_attention.h:9-22): Div(Qt, sqrt d) -> MatMul(., Kt) ->
    Where(mask, fill, .) -> Softmax -> MatMul(., Vt) -> Transpose -> Reshape,
    the mask broadcast by Cast(Expand(cond, Shape(scores)))."""
    rng = np.random.default_rng(4)
    g = Graph()
    g.add_initializer("shape4", np.array([0, 0, heads, H // heads], np.int64))
    g.add_initializer("shape3", np.array([0, 0, H], np.int64))
    for p in "qkv":
        _proj(g, p, "X" if shared_x or p != "v" else "X2", H, rng)
    g.add_node("Transpose", ["q_r"], ["qt"], perm=[0, 2, 1, 3])
    g.add_node("Transpose", ["k_r"], ["kt"], perm=[0, 2, 3, 1])
    g.add_node("Transpose", ["v_r"], ["vt"], perm=[0, 2, 1, 3])
    g.add_constant("c_scale", f32(np.sqrt(H // heads)))
    g.add_node("Div", ["qt", "c_scale"], ["qs"])
    g.add_node("MatMul", ["qs", "kt"], ["scores"])
    g.add_node("Shape", ["scores"], ["sshape"])
    g.add_node("Expand", ["cond", "sshape"], ["cond_e"])
    g.add_node("Cast", ["cond_e"], ["cond_b"], to=9)
    g.add_constant("c_fill", f32(-3.4028234663852886e38))
    g.add_node("Where", ["cond_b", "c_fill", "scores"], ["masked"])
    g.add_node("Softmax", ["masked"], ["probs"], axis=-1)
    g.add_node("MatMul", ["probs", "vt"], ["ctx4"])
    g.add_node("Transpose", ["ctx4"], ["ctxt"], perm=[0, 2, 1, 3])
    g.add_node("Reshape", ["ctxt", "shape3"], ["ctx"])
    g.add_output("ctx")
    return g


def test_recognize_attention_then_qkv():
    g = where_attention_graph()
    assert g.run_pass("recognize_attention") == 1
    fa = node_of(g, "FusedAttention")
    assert fa["domain"] == "inferc"
    # Cast and Expand are peeled: the kernel broadcasts the [B,1,1,S] mask
    assert fa["inputs"] == ["qp", "kp", "vp", "cond"]
    assert fa["outputs"] == ["ctx"]
    assert fa["attrs"]["head_dim"] == "16"
    assert np.float32(float(fa["attrs"]["fill"])) == np.float32(-3.4028234663852886e38)
    for gone in ("Softmax", "Where", "Div", "Transpose", "Cast", "Expand", "Shape"):
        assert gone not in ops(g), gone
    assert g.run_pass("fuse_qkv_projection") == 1
    qkv = node_of(g, "FusedQKV")
    assert qkv["inputs"] == ["X", "Wq", "bq", "Wk", "bk", "Wv", "bv"]
    assert qkv["outputs"] == ["qp", "kp", "vp"]
    assert "MatMul" not in ops(g)
    # the fused QKV comes before the attention that reads it
    assert ops(g).index("FusedQKV") < ops(g).index("FusedAttention")


def test_qkv_needs_a_shared_input():
    g = where_attention_graph(shared_x=False)
    assert g.run_pass("recognize_attention") == 1
    assert g.run_pass("fuse_qkv_projection") == 0


def additive_attention_graph(keep_if_true=True, scale_op="Mul", H=64, heads=4) -> Graph:
    """The block as current transformers exports export it: Mul(MatMul(Qt, Kt),
    1/sqrt d) + Where(keep, 0, fill) -> Softmax (the fixture model's form)."""
    rng = np.random.default_rng(5)
    dh = H // heads
    g = Graph()
    g.add_initializer("shape4", np.array([0, 0, heads, dh], np.int64))
    g.add_initializer("shape3", np.array([0, 0, H], np.int64))
    for p in "qkv":
        _proj(g, p, "X", H, rng)
    g.add_node("Transpose", ["q_r"], ["qt"], perm=[0, 2, 1, 3])
    g.add_node("Transpose", ["k_r"], ["kt"], perm=[0, 2, 3, 1])
    g.add_node("Transpose", ["v_r"], ["vt"], perm=[0, 2, 1, 3])
    g.add_node("MatMul", ["qt", "kt"], ["scores"])
    if scale_op == "Mul":
        g.add_constant("c_scale", f32(1.0 / np.sqrt(dh)))
    else:
        g.add_constant("c_scale", f32(np.sqrt(dh)))
    g.add_node(scale_op, ["scores", "c_scale"], ["scaled"])
    g.add_constant("c0", f32(0.0))
    g.add_constant("cmin", f32(-3.4028234663852886e38))
    g.add_node("Where", ["cond", "c0", "cmin"] if keep_if_true else ["cond", "cmin", "c0"],
               ["maskf"])
    g.add_node("Add", ["scaled", "maskf"], ["biased"])
    g.add_node("Softmax", ["biased"], ["probs"], axis=-1)
    g.add_node("MatMul", ["probs", "vt"], ["ctx4"])
    g.add_node("Transpose", ["ctx4"], ["ctxt"], perm=[0, 2, 1, 3])
    g.add_node("Reshape", ["ctxt", "shape3"], ["ctx"])
    g.add_output("ctx")
    return g


@pytest.mark.parametrize("keep_if_true", [True, False])
@pytest.mark.parametrize("scale_op", ["Mul", "Div"])
def test_additive_attention(keep_if_true, scale_op):
    g = additive_attention_graph(keep_if_true, scale_op)
    assert g.run_pass("recognize_attention") == 0  # not the reference's form
    assert g.run_pass("recognize_attention_additive") == 1
    fa = node_of(g, "FusedAttention")
    assert fa["attrs"]["head_dim"] == "16"
    assert fa["inputs"][:3] == ["qp", "kp", "vp"]
    if keep_if_true:
        nt = node_of(g, "Not")
        assert nt["inputs"] == ["cond"] and fa["inputs"][3] == nt["outputs"][0]
        assert ops(g).index("Not") < ops(g).index("FusedAttention")
    else:
        assert fa["inputs"][3] == "cond" and "Not" not in ops(g)
    assert "Softmax" not in ops(g)
    assert g.run_pass("fuse_qkv_projection") == 1


def test_additive_attention_checks_the_head_split():
    g = additive_attention_graph()
    d = g.to_dict()
    # same graph with K transposed the wrong way round: no fusion
    g2 = Graph()
    g2.add_initializer("shape4", np.array([0, 0, 4, 16], np.int64))
    for n in d["nodes"]:
        attrs = {k: [int(x) for x in v.split(",")] if k == "perm" else v
                 for k, v in n["attrs"].items()}
        if n["outputs"] == ["kt"]:
            attrs["perm"] = [0, 2, 1, 3]
        if n["op"] == "Constant":
            val = {"c_scale": 0.25, "c0": 0.0, "cmin": -3.4028234663852886e38}[n["outputs"][0]]
            g2.add_constant(n["outputs"][0], f32(val))
        else:
            g2.add_node(n["op"], n["inputs"], n["outputs"], name=n["name"], **attrs)
    g2.add_output("ctx")
    assert g2.run_pass("recognize_attention_additive") == 0


# ------------------------------------------------------------- the pipeline

def test_unknown_pass_is_an_error():
    with pytest.raises(RuntimeError, match="unknown pass"):
        Graph().run_pass("no_such_pass")


@pytest.mark.parametrize("name,layers", [("distilbert_tiny", 2)])
def test_pipeline_on_exported_distilbert(name, layers):
    """Per transformer block: one attention, one QKV, two LayerNorms, one
    erf-GELU folded into one FusedMatMulAddGELU; plus the embedding
    LayerNorm (SESSIONS-style counts: L, L, 2L+1, L, L)."""
    g = Graph.from_onnx(GOLDEN / f"{name}.onnx")
    before = Counter(g.op_types)
    counts = g.optimize()
    assert list(counts) == list(PASSES)
    assert counts == {"fold_constant_transpose": 0, "recognize_attention": 0,
                      "recognize_attention_additive": layers, "fuse_qkv_projection": layers,
                      "recognize_layernorm": 2 * layers + 1, "recognize_gelu": layers,
                      "recognize_gelu_tanh": 0, "fuse_matmul_add_gelu": layers}
    after = Counter(g.op_types)
    for gone in ("Softmax", "Erf", "Sqrt", "ReduceMean", "Transpose"):
        assert after[gone] == 0, gone
    assert after["FusedAttention"] == layers and after["FusedQKV"] == layers
    assert after["MatMul"] == before["MatMul"] - 3 * layers - 2 * layers - layers
    # a second run finds nothing more
    assert sum(g.optimize().values()) == 0


def test_pipeline_on_exported_gpt2():
    """GPT-2's causal attention (left unfused by the reference,
    SESSIONS.md:557) folds through the additive-mask form: the context's
    Reshape target is computed by Shape nodes on the merged heads, which go
    with it; LayerNorm (2 per block + final) and the tanh GELU fold."""
    g = Graph.from_onnx(GOLDEN / "gpt2_tiny.onnx")
    counts = g.optimize()
    assert counts["recognize_attention_additive"] == 2
    assert counts["recognize_layernorm"] == 5 and counts["recognize_gelu_tanh"] == 2
    assert counts["recognize_gelu"] == 0 and counts["fuse_matmul_add_gelu"] == 0
    c = Counter(g.op_types)
    assert c["Tanh"] == 0 and c["Softmax"] == 0 and c["FusedAttention"] == 2
    names = {t for n in g.to_dict()["nodes"] for t in n["inputs"] + n["outputs"]}
    produced = {t for n in g.to_dict()["nodes"] for t in n["outputs"]}
    inits = {i["name"] for i in g.to_dict()["initializers"]}
    # nothing reads a tensor that no node, initializer or input provides
    for n in g.to_dict()["nodes"]:
        for t in n["inputs"]:
            assert t in produced or t in inits or t in ("input_ids", "attention_mask") or t == "", t
    assert names


def test_pipeline_on_exported_gpt2_with_past():
    """The with-past decoder: each layer's Concat(past, new) -> attention
    becomes one FusedAttentionPast producing the present.* outputs."""
    g = Graph.from_onnx(GOLDEN / "gpt2_tiny_past.onnx")
    counts = g.optimize()
    assert counts["recognize_attention_additive"] == 2
    assert counts["recognize_layernorm"] == 5 and counts["recognize_gelu_tanh"] == 2
    fused = [n for n in g.to_dict()["nodes"] if n["op"] == "FusedAttentionPast"]
    assert len(fused) == 2
    for layer, n in enumerate(fused):
        assert n["outputs"][1:] == [f"present.{layer}.key", f"present.{layer}.value"]
        assert n["attrs"]["head_dim"] == "16"
    assert "Concat" not in [n["op"] for n in g.to_dict()["nodes"]
                            if any(o.startswith("present.") for o in n["outputs"])]


def test_pipeline_on_gpt2_small_structure_export():
    """The GPT-2-small with-past export (structure only, parameters as graph
    inputs) with seeded weights bound: every parameter input is placed, the
    pipeline folds one attention-with-past per layer, 2 LayerNorms per layer
    plus the final one, one tanh-GELU per layer, and the planned step writes
    logits [1, 1, vocab] and presents of the grown cache."""
    from inferc_amd import graphs
    from inferc_amd.rt import Executor

    cfg = graphs.GPT2_SMALL
    g = Graph.from_onnx(Path(__file__).resolve().parent / "golden" /
                        "gpt2_small_past_noparams.onnx")
    graphs.gpt2_bind_weights(g, cfg, graphs.gpt2_weights(cfg, 2))
    c = g.optimize()
    assert c["recognize_attention_additive"] == 12
    assert c["recognize_layernorm"] == 25
    assert c["recognize_gelu_tanh"] == 12
    ex = Executor.dry(g)
    ex.set_input("input_ids", np.array([[5]], np.int64))
    ex.set_input("attention_mask", np.ones((1, 33), np.int64))
    for l in range(12):
        for kv in ("key", "value"):
            ex.set_input(f"past_key_values.{l}.{kv}", np.zeros((1, 12, 32, 64), np.float32))
    ex.run_async()
    assert ex.output_shape("logits") == ((1, 1, 50257), np.dtype(np.float32))
    assert ex.output_shape("present.11.value") == ((1, 12, 33, 64), np.dtype(np.float32))


def test_gpt2_weights_read_back_from_the_exported_graph():
    """graphs.gpt2_weights_from_graph (the weights `inferc decode --native /
    --int4` hands the native decoder) returns exactly the weights bound into
    the GPT-2-small structure export, in gpt2_weights' order, and the config
    of BASELINE config 4 (heads from the past inputs, eps from the fused
    LayerNorms)."""
    from inferc_amd import graphs

    cfg = graphs.GPT2_SMALL
    w = graphs.gpt2_weights(cfg, 2)
    g = Graph.from_onnx(Path(__file__).resolve().parent / "golden" /
                        "gpt2_small_past_noparams.onnx")
    graphs.gpt2_bind_weights(g, cfg, w)
    with pytest.raises(ValueError):
        graphs.gpt2_weights_from_graph(Graph())
    assert g.run_pass("recognize_layernorm") == 25
    got_cfg, got = graphs.gpt2_weights_from_graph(g)
    assert {k: v for k, v in got_cfg.items() if k != "eps"} == \
        {k: v for k, v in cfg.items() if k != "eps"}
    assert np.float32(got_cfg["eps"]) == np.float32(cfg["eps"])
    assert len(got) == len(w)
    for a, b in zip(got, w):
        np.testing.assert_array_equal(a, b)


def test_decode_plan_on_exported_gpt2():
    """inferc_executor_set_decode_position's plan on the GPT-2-small with-past
    export: the values computed from the past inputs and the attention mask
    reach only the attention nodes' past/mask inputs and the position
    embedding's Gather, so decode mode is accepted; a graph output computed
    from the mask's length is refused."""
    from inferc_amd import graphs
    from inferc_amd.rt import Executor

    cfg = graphs.GPT2_SMALL
    path = Path(__file__).resolve().parent / "golden" / "gpt2_small_past_noparams.onnx"
    g = Graph.from_onnx(path)
    graphs.gpt2_bind_weights(g, cfg, graphs.gpt2_weights(cfg, 2))
    g.optimize()
    ex = Executor.dry(g)
    ex.set_decode_position(33, "attention_mask")
    ex.set_input("input_ids", np.array([[5]], np.int64))
    ex.set_input("attention_mask", np.ones((1, 1), np.int64))
    for l in range(12):
        for kv in ("key", "value"):
            ex.set_input(f"past_key_values.{l}.{kv}", np.zeros((1, 12, 0, 64), np.float32))
    ex.run_async()
    assert ex.output_shape("logits") == ((1, 1, 50257), np.dtype(np.float32))
    # an output that depends on the past length: refused
    g2 = Graph.from_onnx(path)
    graphs.gpt2_bind_weights(g2, cfg, graphs.gpt2_weights(cfg, 2))
    g2.optimize()
    g2.add_node("Shape", ["attention_mask"], ["mask_shape"])
    g2.add_output("mask_shape")
    ex2 = Executor.dry(g2)
    with pytest.raises(RuntimeError, match="depends on the past length"):
        ex2.set_decode_position(33, "attention_mask")
