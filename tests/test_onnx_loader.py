"""The protobuf-free ONNX reader (no GPU): the reference's loader tests
(tests/loader_test.cc:10-92) on models serialized by tests/pbwire.py, the
ONNX -> IR conversion (src/frontend/onnx_to_ir.cc:33-144) for every
initializer encoding and attribute type, malformed input, and the exported
fixture models read by both this reader and the independent test decoder."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from inferc_amd import lib as L
from inferc_amd import rt
from tests import pbwire as W

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    if not L.library_path().exists():
        from inferc_amd.build import build

        build()


def tiny_relu_model() -> bytes:
    """MakeTinyModel (loader_test.cc:13-45): one Relu, x[2,3] -> y[2,3]."""
    g = W.graph("tiny", nodes=[W.node("Relu", ["x"], ["y"])],
                inputs=[W.value_info("x", W.FLOAT, [2, 3])],
                outputs=[W.value_info("y", W.FLOAT, [2, 3])])
    return W.model(g, ir_version=7, producer="inferc-test", producer_version="0", opset=14)


def test_summary_preserves_fields():
    s = rt.onnx_summary(tiny_relu_model())
    assert s["ir_version"] == 7
    assert s["opset_version"] == 14
    assert s["opset_domain"] == "ai.onnx"
    assert s["graph_name"] == "tiny"
    assert s["node_count"] == 1
    assert s["op_type_counts"] == {"Relu": 1}
    assert s["producer_name"] == "inferc-test" and s["producer_version"] == "0"
    assert len(s["inputs"]) == 1 and s["inputs"][0]["name"] == "x"
    assert s["inputs"][0]["dtype"] == W.FLOAT and s["inputs"][0]["shape"] == [2, 3]
    assert [o["name"] for o in s["outputs"]] == ["y"]


def test_print_summary_text_and_empty_model():
    t = rt.onnx_summary(tiny_relu_model(), text=True)
    lines = t.splitlines()
    assert lines[0] == "Model: tiny"
    assert "  Opset:             ai.onnx v14" in lines
    assert any(ln.startswith("  x ") and ln.rstrip().endswith("float32   [2, 3]") for ln in lines)
    assert "Nodes: 1" in lines
    assert lines[-1] == "Initializers: 0  (0.00 MB)"
    empty = rt.onnx_summary(b"", text=True)  # an empty ModelProto summarises
    assert empty.startswith("Model: ") and "Nodes: 0" in empty
    with pytest.raises(RuntimeError, match="model has no graph"):
        rt.Graph.from_onnx(b"")


def test_element_bytes_known_types():
    import ctypes as C
    lib = L.load_library()
    got = {}
    for dt in (1, 7, 3, 10, 8, 9, 11, 16, 99):
        n = C.c_int64()
        L.check(lib.inferc_onnx_element_bytes(dt, C.byref(n)))
        got[dt] = n.value
    assert got == {1: 4, 7: 8, 3: 1, 10: 2, 8: 0, 9: 1, 11: 8, 16: 2, 99: 0}


def test_symbolic_dims_and_initializer_inputs():
    w = np.arange(6, dtype=np.float32).reshape(2, 3)
    g = W.graph("m", nodes=[W.node("MatMul", ["x", "w"], ["y"])], inits=[W.tensor("w", w)],
                inputs=[W.value_info("x", W.FLOAT, ["batch", 2]),
                        W.value_info("w", W.FLOAT, [2, 3])],
                outputs=[W.value_info("y", W.FLOAT, ["batch", 3])])
    m = W.model(g)
    s = rt.onnx_summary(m)
    # the initializer listed as an input is not a runtime input (onnx_loader.cc:152-168)
    assert [i["name"] for i in s["inputs"]] == ["x"]
    assert s["inputs"][0]["shape"] == [-1, 2] and s["inputs"][0]["dim_param"] == ["batch", ""]
    assert s["initializer_count"] == 1 and s["initializer_total_bytes"] == 24
    assert "  x                   float32   [batch, 2]" in rt.onnx_summary(m, text=True)
    d = rt.Graph.from_onnx(m).to_dict()
    assert [i["name"] for i in d["inputs"]] == ["x"] and d["inputs"][0]["shape"] == [-1, 2]
    assert d["outputs"] == ["y"]


@pytest.mark.parametrize("typed,packed", [(False, True), (True, True), (True, False)])
def test_initializer_encodings(typed, packed):
    """raw_data, packed typed fields and one-record-per-value typed fields all
    give the same bytes (onnx_to_ir.cc:33-83)."""
    rng = np.random.default_rng(3)
    arrs = {"f": rng.standard_normal((3, 4)).astype(np.float32),
            "i64": np.array([-5, 0, 7, 1 << 40, -(1 << 40)], np.int64),
            "i32": np.array([[-3, 2], [1 << 30, -(1 << 30)]], np.int32),
            "s": np.array(2.5, np.float32)}
    inits = [W.tensor(k, a, typed=typed, packed=packed) for k, a in arrs.items()]
    g = W.graph("enc", nodes=[W.node("Identity", ["f"], ["y"])], inits=inits,
                outputs=[W.value_info("y", W.FLOAT, [3, 4])])
    gr = rt.Graph.from_onnx(W.model(g))
    for k, a in arrs.items():
        got = gr.initializer(k)
        assert got.dtype == a.dtype and got.shape == a.shape
        np.testing.assert_array_equal(got, a)


def test_attribute_types_and_constant_tensor():
    c = W.tensor("", np.array([1.5], np.float32))
    nodes = [
        W.node("Constant", [], ["c"], name="k", attrs=[W.attr_tensor("value", c)]),
        W.node("Custom", ["c"], ["y"], name="n", domain="my.domain",
               attrs=[W.attr_int("i", -7), W.attr_float("f", 0.1), W.attr_ints("is", [1, -2, 3]),
                      W.attr_floats("fs", [0.5, -1.25]), W.attr_string("s", "mode")]),
    ]
    d = rt.Graph.from_onnx(W.model(W.graph("a", nodes=nodes))).to_dict()
    k, n = d["nodes"]
    assert k["op"] == "Constant" and k["tensor_attrs"]["value"] == {"dtype": 1, "shape": [1]}
    assert n["domain"] == "my.domain"
    assert n["attrs"]["i"] == "-7" and n["attrs"]["is"] == "1,-2,3"
    assert np.float32(float(n["attrs"]["f"])) == np.float32(0.1)  # exact float32
    assert n["attrs"]["fs"] == "0.5,-1.25" and n["attrs"]["s"] == "mode"


def test_malformed_input_fails_cleanly():
    good = tiny_relu_model()
    for bad in (good[:-1], good[:5], b"\x0a\xff\xff\xff\xff\x0f", b"\x08", b"\x0f\x00",
                b"\x00\x01"):
        with pytest.raises(RuntimeError, match="malformed protobuf"):
            rt.Graph.from_onnx(bad)
    # every truncation and many single-byte corruptions either load or raise
    rng = np.random.default_rng(0)
    for cut in range(len(good)):
        try:
            rt.Graph.from_onnx(good[:cut])
        except RuntimeError:
            pass
    for _ in range(300):
        b = bytearray(good)
        b[int(rng.integers(len(b)))] = int(rng.integers(256))
        try:
            rt.Graph.from_onnx(bytes(b))
        except RuntimeError:
            pass


def test_external_data_and_raw_size_mismatch_are_errors():
    t = W.tensor("w", np.zeros(4, np.float32)) + W.f_varint(14, 1)
    with pytest.raises(RuntimeError, match="external data"):
        rt.Graph.from_onnx(W.model(W.graph("e", inits=[t])))
    t2 = W.tensor("w", np.zeros(4, np.float32), dims=[5])
    with pytest.raises(RuntimeError, match="raw_data size"):
        rt.Graph.from_onnx(W.model(W.graph("e", inits=[t2])))


def test_load_from_file(tmp_path):
    p = tmp_path / "tiny.onnx"
    p.write_bytes(tiny_relu_model())
    assert rt.Graph.from_onnx(p).op_types == ["Relu"]
    with pytest.raises(RuntimeError, match="cannot open"):
        rt.Graph.from_onnx(tmp_path / "missing.onnx")


@pytest.mark.parametrize("name", ["distilbert_tiny", "gpt2_tiny"])
def test_exported_fixture_read_by_both_decoders(name):
    """Models exported by torch.onnx from transformers (tests/golden/
    make_onnx_fixtures.py): the reader's summary agrees with the test decoder
    on node count, op types, initializer count and bytes."""
    data = (GOLDEN / f"{name}.onnx").read_bytes()
    ref = W.decode_graph(data)
    s = rt.onnx_summary(data)
    assert s["node_count"] == ref["node_count"]
    counts: dict[str, int] = {}
    for op in ref["ops"]:
        counts[op] = counts.get(op, 0) + 1
    assert s["op_type_counts"] == counts
    assert s["initializer_count"] == ref["initializer_count"]
    assert s["initializer_total_bytes"] == ref["initializer_total_bytes"]
    g = rt.Graph.from_onnx(data)
    assert g.op_types == ref["ops"]
    assert s["producer_name"] == "pytorch" and s["opset_version"] == 13
