"""The allocation-free GEMM entry point (inferc_hip_gemm_f32_noalloc) against
inferc_hip_gemm_f32, through the C-ABI. The shapes take the split-K path,
whose partial sums live in the static scratch array instead of the context
workspace: two calls in a row, the second on a smaller product (so stale
partials of the first would show), each bit-identical to the regular entry
point (same kernels, same split) and within 1e-4 of a float64 statement."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from inferc_amd import lib as L
from inferc_amd.rt import Tensor

pytestmark = pytest.mark.gpu

# (transA, M, N, K): split-K with 16 splits (M > 512, the small-M kernel
# cannot take it), then a smaller one with 16, then transA with 23 splits
SHAPES = [(0, 600, 256, 4096), (0, 520, 128, 2048), (1, 100, 200, 3000)]


def _gemm(ctx, fn, ta, M, N, K, A, B, C_, R):
    Y = Tensor.empty(ctx, (M, N))
    lda = M if ta else K
    rc = getattr(ctx._lib, fn)(ctx.handle, ta, 0, M, N, K, C.c_float(0.5), A.ptr, lda, B.ptr, N,
                               C.c_float(1.0), C_.ptr, L.C_ROW, 0, R.ptr, N, L.ACT_GELU_ERF,
                               Y.ptr, N)
    L.check(rc)
    return Y.numpy()


def _case(ctx, ta, M, N, K, seed):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    c = rng.standard_normal(N).astype(np.float32)
    r = rng.standard_normal((M, N)).astype(np.float32)
    d = [Tensor.from_numpy(ctx, x) for x in (a, b, c, r)]
    a64 = a.T.astype(np.float64) if ta else a.astype(np.float64)
    v = 0.5 * (a64 @ b.astype(np.float64)) + c + r
    from math import erf
    ref = v * 0.5 * (1.0 + np.vectorize(erf)(v / np.sqrt(2.0)))
    return d, ref


def test_gemm_noalloc_matches_gemm_two_calls(ctx):
    for i, (ta, M, N, K) in enumerate(SHAPES):
        (A, B, C_, R), ref = _case(ctx, ta, M, N, K, 50 + i)
        got = _gemm(ctx, "inferc_hip_gemm_f32_noalloc", ta, M, N, K, A, B, C_, R)
        want = _gemm(ctx, "inferc_hip_gemm_f32", ta, M, N, K, A, B, C_, R)
        np.testing.assert_array_equal(got, want)
        err = float(np.max(np.abs(got - ref)))
        assert err <= 1e-4 * max(1.0, float(np.abs(ref).max())), (ta, M, N, K, err)
    # again, now that the scratch holds the last call's partials
    (A, B, C_, R), ref = _case(ctx, *SHAPES[1], 60)
    got = _gemm(ctx, "inferc_hip_gemm_f32_noalloc", *SHAPES[1], A, B, C_, R)
    np.testing.assert_array_equal(got, _gemm(ctx, "inferc_hip_gemm_f32", *SHAPES[1], A, B, C_, R))


def test_gemm_noalloc_small_m_path_and_errors(ctx):
    """Shapes that need no partial sums (the small-M kernel, the one-row
    GEMV) run unchanged; bad arguments fail before any launch."""
    for ta, M, N, K in [(0, 128, 3072, 768), (0, 1, 768, 768)]:
        (A, B, C_, R), _ = _case(ctx, ta, M, N, K, 70 + M)
        got = _gemm(ctx, "inferc_hip_gemm_f32_noalloc", ta, M, N, K, A, B, C_, R)
        np.testing.assert_array_equal(got, _gemm(ctx, "inferc_hip_gemm_f32", ta, M, N, K,
                                                 A, B, C_, R))
    rc = ctx._lib.inferc_hip_gemm_f32_noalloc(ctx.handle, 0, 0, 4, 4, 4, C.c_float(1.0), None, 4,
                                              None, 4, C.c_float(0.0), None, 0, 0, None, 0, 0,
                                              None, 4)
    assert rc == L.ERR_ARG
