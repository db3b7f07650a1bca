"""The executor's one-row GEMV route (the M == 1 sgemv of
src/kernels/matmul.cc:207-216 behind rt::SetGemvDecodeEnabled, :56-61):
the transposed weight copies it reads, the context switch that turns it off
(`inferc decode --no-gemv`), and a fed input that shadows an initializer of
the same name; and when a recorded run may be replayed."""
from __future__ import annotations

import numpy as np
import pytest

from inferc_amd import rt

pytestmark = pytest.mark.gpu

K, N = 768, 1000


def _matmul_graph(w: np.ndarray, shadow: bool = False) -> rt.Graph:
    g = rt.Graph()
    g.add_input("x", np.float32, [1, K])
    g.add_initializer("W", w)
    if shadow:
        g.add_input("W", np.float32, [K, N])
    g.add_node("MatMul", ["x", "W"], ["y"])
    g.add_output("y")
    return g


def _ref(x, w):
    return (x.astype(np.float64) @ w.astype(np.float64)).astype(np.float32)


def test_one_row_matmul_reads_a_transposed_copy(ctx):
    rng = np.random.default_rng(7)
    w = rng.standard_normal((K, N)).astype(np.float32) * 0.02
    x = rng.standard_normal((1, K)).astype(np.float32)
    assert ctx.gemv_decode_enabled()
    ex = rt.Executor(ctx, _matmul_graph(w))
    for _ in range(3):  # eager, captured, replayed
        y = ex.run({"x": x}, ["y"])["y"]
        np.testing.assert_allclose(y, _ref(x, w), rtol=1e-4, atol=1e-5)
    b = ex.device_bytes()
    assert b["initializers"] == K * N * 4 and b["transposed_copies"] == K * N * 4
    ex.close()


def test_gemv_route_switched_off_makes_no_copy(ctx):
    rng = np.random.default_rng(8)
    w = rng.standard_normal((K, N)).astype(np.float32) * 0.02
    x = rng.standard_normal((1, K)).astype(np.float32)
    ctx.set_gemv_decode(False)
    try:
        assert not ctx.gemv_decode_enabled()
        ex = rt.Executor(ctx, _matmul_graph(w))
        for _ in range(3):
            y = ex.run({"x": x}, ["y"])["y"]
            np.testing.assert_allclose(y, _ref(x, w), rtol=1e-4, atol=1e-5)
        assert ex.device_bytes()["transposed_copies"] == 0
        # switched back on: the executor plans the route again and replays it
        ctx.set_gemv_decode(True)
        for _ in range(3):
            y = ex.run({"x": x}, ["y"])["y"]
            np.testing.assert_allclose(y, _ref(x, w), rtol=1e-4, atol=1e-5)
        assert ex.device_bytes()["transposed_copies"] == K * N * 4
        ex.close()
    finally:
        ctx.set_gemv_decode(True)


def test_fed_input_shadowing_an_initializer(ctx):
    """A graph input fed under an initializer's name is what every reader
    sees, the one-row product included: it must not read the transposed copy
    of the initializer's data."""
    rng = np.random.default_rng(9)
    w_init = rng.standard_normal((K, N)).astype(np.float32) * 0.02
    w_fed = rng.standard_normal((K, N)).astype(np.float32)
    x = rng.standard_normal((1, K)).astype(np.float32)
    ex = rt.Executor(ctx, _matmul_graph(w_init, shadow=True))
    for _ in range(3):
        y = ex.run({"x": x, "W": w_fed}, ["y"])["y"]
        np.testing.assert_allclose(y, _ref(x, w_fed), rtol=1e-4, atol=1e-4)
    assert ex.device_bytes()["transposed_copies"] == 0
    ex.close()


def test_recording_not_replayed_after_its_uploaded_constant_changed(ctx):
    """y = x * float(S) for x [1, S]: the scalar is host shape math that the
    Mul kernel reads from an uploaded device copy. The longer length runs
    first, so both lengths share the input and output buffers and their
    recordings differ only in that constant's bytes: after the other length
    uploads its value, a recording must be planned again, not replayed."""
    g = rt.Graph()
    g.add_initializer("one", np.array(1, np.int64))
    g.add_node("Shape", ["x"], ["s"])
    g.add_node("Gather", ["s", "one"], ["n"], axis=0)
    g.add_node("Cast", ["n"], ["nf"], to=1)
    g.add_node("Mul", ["x", "nf"], ["y"])
    g.add_output("y")
    ex = rt.Executor(ctx, g)
    rng = np.random.default_rng(11)
    xs = {S: rng.standard_normal((1, S)).astype(np.float32) for S in (8, 6)}
    for S in (8, 8, 8, 6, 6, 6, 8, 8, 8, 6, 8, 6, 6):
        y = ex.run({"x": xs[S]}, ["y"])["y"]
        np.testing.assert_array_equal(y, xs[S] * np.float32(S), err_msg=f"S={S}")
    ex.close()
