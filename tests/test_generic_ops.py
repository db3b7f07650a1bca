"""The executor's generic ops (Sub/Mul/Div/Pow, comparisons, logic, Where,
unary math, Cast, Expand, Transpose, Slice, ReduceMean, typed Gather,
ConstantOfShape) against numpy, in both of their forms: folded on the host
when every input is a constant (CPU, dry-run executor), and as device kernels
when the inputs are graph inputs (GPU). Semantics follow the ONNX operator
definitions the reference executor implements (src/runtime/executor.cc:
226-339): numpy broadcasting, Cast truncating toward zero and mapping
nonzero to true, Slice clamping per the ONNX rules."""
from __future__ import annotations

import numpy as np
import pytest

from inferc_amd import lib as L
from inferc_amd.rt import Executor, Graph

rng = np.random.default_rng(17)


def _f(*shape):
    return rng.standard_normal(shape).astype(np.float32)


def _i(*shape, lo=-9, hi=9):
    return rng.integers(lo, hi, shape).astype(np.int64)


def _b(*shape):
    return rng.integers(0, 2, shape).astype(np.bool_)


def _slice_ref(x, starts, ends, axes, steps):
    sl = [slice(None)] * x.ndim
    for s, e, a, st in zip(starts, ends, axes, steps):
        sl[a] = slice(s, e, st)
    return x[tuple(sl)]


# name -> (op, inputs, attrs, numpy reference, tensor-attr)
CASES = {
    "sub_bcast": ("Sub", [_f(2, 3, 4), _f(3, 1)], {}, lambda a, b: a - b),
    "mul_mid_bcast": ("Mul", [_f(2, 1, 5, 4), _f(2, 3, 1, 4)], {}, lambda a, b: a * b),
    "div": ("Div", [_f(4, 5), _f(5) + 3.0], {}, lambda a, b: a / b),
    "pow_int_exp": ("Pow", [_f(3, 4), np.array(2, np.int64)], {},
                    lambda a, b: np.power(a, np.float32(2))),
    "pow3": ("Pow", [_f(3, 4), np.array(3.0, np.float32)], {}, lambda a, b: a ** 3),
    "add_i64": ("Add", [_i(2, 3), _i(3)], {}, lambda a, b: a + b),
    "mul_i64": ("Mul", [_i(4), _i(1)], {}, lambda a, b: a * b),
    "less": ("Less", [_f(3, 4), _f(4)], {}, np.less),
    "le_i64": ("LessOrEqual", [_i(5, 1), _i(1, 6)], {}, np.less_equal),
    "ge": ("GreaterOrEqual", [_i(2, 3), _i(3)], {}, np.greater_equal),
    "gt": ("Greater", [_f(6), _f(6)], {}, np.greater),
    "eq_f32": ("Equal", [np.array([1, 2, 3], np.float32), np.array([1, 0, 3], np.float32)], {},
               np.equal),
    "eq_bcast": ("Equal", [_i(1, 4, lo=0, hi=3), _i(3, 1, lo=0, hi=3)], {}, np.equal),
    "and": ("And", [_b(2, 1, 5), _b(1, 3, 5)], {}, np.logical_and),
    "or": ("Or", [_b(4, 2), _b(2)], {}, np.logical_or),
    "xor": ("Xor", [_b(3, 3), _b(3, 3)], {}, np.logical_xor),
    "not": ("Not", [_b(2, 7)], {}, np.logical_not),
    "sqrt": ("Sqrt", [np.abs(_f(3, 5))], {}, np.sqrt),
    "erf": ("Erf", [_f(40)], {}, None),
    "tanh": ("Tanh", [_f(2, 9)], {}, np.tanh),
    "neg_i64": ("Neg", [_i(5)], {}, np.negative),
    "abs": ("Abs", [_f(8)], {}, np.abs),
    "exp": ("Exp", [_f(8)], {}, np.exp),
    "reciprocal": ("Reciprocal", [_f(8) + 4.0], {}, lambda a: np.float32(1) / a),
    "sigmoid": ("Sigmoid", [_f(8)], {}, lambda a: 1 / (1 + np.exp(-a))),
    "cast_f2i": ("Cast", [np.array([-2.7, -0.5, 0.5, 2.9, 7.0], np.float32)], {"to": 7},
                 lambda a: np.trunc(a).astype(np.int64)),
    "cast_i2b": ("Cast", [np.array([0, 3, -1, 0], np.int64)], {"to": 9},
                 lambda a: a != 0),
    "cast_b2f": ("Cast", [_b(6)], {"to": 1}, lambda a: a.astype(np.float32)),
    "cast_i2f": ("Cast", [_i(3, 2)], {"to": 1}, lambda a: a.astype(np.float32)),
    "where": ("Where", [_b(2, 1, 4), _f(3, 4), _f(2, 3, 1)], {}, np.where),
    "where_i64": ("Where", [_b(5), _i(5), np.array(-1, np.int64)], {}, np.where),
    "expand": ("Expand", [_f(3, 1), np.array([2, 1, 4], np.int64)], {},
               lambda a, s: np.broadcast_to(a, (2, 3, 4))),
    "expand_bool": ("Expand", [_b(1, 1, 1, 5), np.array([2, 1, 5, 5], np.int64)], {},
                    lambda a, s: np.broadcast_to(a, (2, 1, 5, 5))),
    "transpose4": ("Transpose", [_f(2, 3, 4, 5)], {"perm": [0, 2, 3, 1]},
                   lambda a: a.transpose(0, 2, 3, 1)),
    "transpose_default": ("Transpose", [_i(2, 3, 4)], {}, lambda a: a.transpose()),
    "slice": ("Slice", [_f(5, 6), np.array([1, -4], np.int64), np.array([4, 100], np.int64)], {},
              lambda x, s, e: _slice_ref(x, [1, -4], [4, 100], [0, 1], [1, 1])),
    "slice_axes_steps": ("Slice", [_f(4, 7, 3), np.array([-1, 0], np.int64),
                                   np.array([-100, 7], np.int64), np.array([1, 0], np.int64),
                                   np.array([-2, 3], np.int64)], {},
                         lambda x, *r: _slice_ref(x, [-1, 0], [-100, 7], [1, 0], [-2, 3])),
    "slice_i64": ("Slice", [_i(1, 64), np.array([0], np.int64), np.array([9], np.int64),
                            np.array([1], np.int64)], {},
                  lambda x, *r: x[:, 0:9]),
    "reduce_last": ("ReduceMean", [_f(3, 4, 8)], {"axes": [-1]},
                    lambda a: a.mean(-1, keepdims=True)),
    "reduce_mid_nokeep": ("ReduceMean", [_f(3, 4, 5)], {"axes": [1], "keepdims": 0},
                          lambda a: a.mean(1)),
    "reduce_all": ("ReduceMean", [_f(2, 3)], {}, lambda a: a.mean(keepdims=True)),
    "gather_i64_axis1": ("Gather", [_i(3, 5), np.array([4, 0, -1], np.int64)], {"axis": 1},
                         lambda a, i: np.take(a, i, axis=1)),
    "gather_bool": ("Gather", [_b(12), np.array([[0, 3], [11, 2]], np.int64)], {},
                    lambda a, i: a[i]),
}


def _build(op, arrays, attrs, as_constants):
    g = Graph()
    names = []
    for k, a in enumerate(arrays):
        nm = f"in{k}"
        if as_constants or (op in ("Expand", "Slice", "Pow") and k > 0) or \
                (op == "Gather" and k == 1):
            g.add_constant(nm, a)
        names.append(nm)
    g.add_node(op, names, ["y"], **attrs)
    g.add_output("y")
    return g


def _check(out, ref, name):
    assert out.shape == ref.shape, name
    if np.asarray(ref).dtype == np.bool_:
        np.testing.assert_array_equal(out.astype(np.bool_), ref)
    elif np.issubdtype(np.asarray(ref).dtype, np.integer):
        np.testing.assert_array_equal(out, ref)
    else:
        np.testing.assert_allclose(out, ref, rtol=2e-6, atol=2e-6)


def _ref(name):
    op, arrays, attrs, f = CASES[name]
    if name == "erf":
        import math
        return np.array([math.erf(float(v)) for v in arrays[0]], np.float32)
    return np.asarray(f(*arrays))


@pytest.fixture(scope="module", autouse=True)
def _lib():
    if not L.library_path().exists():
        from inferc_amd.build import build

        build()


@pytest.mark.parametrize("name", sorted(CASES))
def test_generic_op_folded_on_host(name):
    op, arrays, attrs, _ = CASES[name]
    ex = Executor.dry(_build(op, arrays, attrs, as_constants=True))
    ex.run_async()
    _check(ex.output("y"), _ref(name), name)


def test_constant_of_shape_and_unsupported_mix():
    g = Graph()
    g.add_constant("s", np.array([2, 3], np.int64))
    g.add_node("ConstantOfShape", ["s"], ["z"])
    g.add_node("ConstantOfShape", ["s"], ["o"])
    g.add_tensor_attr("value", np.array([7], np.int64))
    g.add_output("z")
    g.add_output("o")
    ex = Executor.dry(g)
    ex.run_async()
    np.testing.assert_array_equal(ex.output("z"), np.zeros((2, 3), np.float32))
    np.testing.assert_array_equal(ex.output("o"), np.full((2, 3), 7, np.int64))
    g2 = Graph()
    g2.add_constant("a", np.ones(3, np.float32))
    g2.add_constant("b", np.ones(3, np.int64))
    g2.add_node("Sub", ["a", "b"], ["y"])
    g2.add_output("y")
    with pytest.raises(RuntimeError, match="operand types differ"):
        Executor.dry(g2).run_async()


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_generic_op_device_kernel(ctx, name):
    """The same cases with the data operands as device-resident graph inputs
    (the shape-like operands of Expand/Slice/Pow-exponent/Gather-indices
    stay constants), so the device kernels run."""
    op, arrays, attrs, _ = CASES[name]
    g = _build(op, arrays, attrs, as_constants=False)
    ex = Executor(ctx, g)
    feeds = {}
    for k, a in enumerate(arrays):
        if not ((op in ("Expand", "Slice", "Pow") and k > 0) or (op == "Gather" and k == 1)):
            feeds[f"in{k}"] = a
    out = ex.run(feeds, ["y"])["y"]
    _check(out, _ref(name), name)
