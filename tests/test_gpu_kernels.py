"""GPU parity of every hot-path kernel against the CPU oracle, through the
C-ABI (inferc_amd.rt). fp32 results are compared at the tolerance the
reference's tests use or tighter (1e-4 scaled by the result magnitude);
integer/byte work (int4 unpack, argmax, gather, split/concat) bit-exactly."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from inferc_amd import graphs, lib as L, rt
from inferc_amd.rt import Tensor
from tests import ref64
from tests.conftest import load_golden

pytestmark = pytest.mark.gpu
KAT = load_golden("kernels_kat.json")["cases"]


def T(ctx, a, dtype=np.float32):
    return Tensor.from_numpy(ctx, np.asarray(a, dtype))


def close(got, ref, tol=1e-4):
    ref = np.asarray(ref, np.float64)
    scale = max(1.0, float(np.abs(ref).max()) if ref.size else 1.0)
    np.testing.assert_allclose(np.asarray(got, np.float64), ref, rtol=0, atol=tol * scale)


def rnd(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


# ------------------------------------------------------------------- KATs

def test_kat_matmul_and_gemm(ctx):
    c = KAT["matmul_basic_2d"]
    close(rt.MatMul(T(ctx, c["a"]), T(ctx, c["b"])).numpy(), c["expect"], 1e-6)
    for name in ("gemm_bias_added", "gemv_notransb", "gemv_transb", "gemv_alpha_beta"):
        c = KAT[name]
        out = rt.Gemm(T(ctx, c["a"]), T(ctx, c["b"]),
                      None if c.get("bias") is None else T(ctx, c["bias"]),
                      c.get("alpha", 1.0), c.get("beta", 1.0), False, c.get("trans_b", False))
        close(out.numpy(), c["expect"], 1e-6)


def test_kat_batched_matmul(ctx):
    a = np.arange(1, 13, dtype=np.float32).reshape(2, 2, 3)
    b = np.arange(1, 13, dtype=np.float32).reshape(3, 4)
    out = rt.MatMul(T(ctx, a), T(ctx, b)).numpy()
    assert out.shape == (2, 2, 4)
    np.testing.assert_array_equal(out[0, 0, :2], [38, 44])
    close(out, O.matmul(a, b), 1e-6)


@pytest.mark.parametrize("name", ["attention_single_head", "attention_mask_zeros_out_key"])
def test_kat_attention(ctx, name):
    c = KAT[name]
    m = None if c["mask"] is None else T(ctx, np.array(c["mask"], np.uint8), np.uint8)
    out = rt.FusedAttention(T(ctx, c["q"]), T(ctx, c["k"]), T(ctx, c["v"]), m, c["head_dim"],
                            c["fill"]).numpy()
    np.testing.assert_allclose(out, c["expect"], atol=c["tol"])


def test_kat_pointwise(ctx):
    c = KAT["gelu_known_values"]
    np.testing.assert_allclose(rt.Gelu(T(ctx, c["x"])).numpy(), c["expect"], atol=c["tol"])
    c = KAT["gelu_tanh_formula"]
    np.testing.assert_allclose(rt.GeluTanh(T(ctx, c["x"])).numpy(), c["expect"], atol=c["tol"])
    c = KAT["softmax_stable"]
    y = rt.Softmax(T(ctx, c["x"])).numpy()
    assert np.all(np.isfinite(y)) and abs(y.sum() - 1.0) < c["sum_tol"]
    x = np.arange(12, dtype=np.float32).reshape(2, 3, 2)
    close(rt.Softmax(T(ctx, x), 1).numpy(), O.softmax(x, 1), 1e-6)
    c = KAT["layernorm_mean0_var1"]
    y = rt.LayerNorm(T(ctx, c["x"]), T(ctx, np.ones(4)), T(ctx, np.zeros(4)), c["eps"]).numpy()
    np.testing.assert_allclose(y.mean(-1), 0, atol=c["mean_tol"])
    np.testing.assert_allclose(y.var(-1), 1, atol=c["var_tol"])


@pytest.mark.parametrize("shape,axis", [((3, 1), -1), ((5, 7), -1), ((4, 1000), -1),
                                        ((2, 50257), -1), ((2, 12, 128, 128), -1),
                                        ((3, 5, 6), 1), ((7, 4, 3), 0), ((2, 3, 4, 5), -2)])
def test_softmax_vs_float64_and_oracle(ctx, shape, axis):
    """Softmax (activation.cc:52-101) over every axis position of rank 2-4
    shapes, rows of 1 to 50257 entries (the LM head's), scores offset by up
    to 1e3 (the max subtraction keeps them finite): within 1e-6 of float64
    and within 1e-4 of the oracle (whose serial float32 sum over a 50257-entry
    row is itself off by up to ~1e-4 relative), rows summing to 1."""
    rng = np.random.default_rng(sum(shape) + axis)
    x = (rng.standard_normal(shape) * 4 + rng.uniform(-1e3, 1e3)).astype(np.float32)
    got = rt.Softmax(T(ctx, x), axis).numpy()
    close(got, ref64.softmax(x, axis), 1e-6)
    close(got, O.softmax(x, axis))
    np.testing.assert_allclose(got.astype(np.float64).sum(axis), 1.0, atol=1e-5)


def test_softmax_masked_and_degenerate_rows(ctx):
    """Rows as attention masks leave them: -inf scores get exactly 0 and a
    single finite score exactly 1; equal scores give the uniform row; scores
    near the float32 maximum stay finite; a row of -inf only is NaN
    throughout, as the reference's exp(-inf - (-inf)) makes it."""
    ninf = -np.inf
    x = np.array([[0.5, ninf, ninf, ninf],
                  [ninf, 2.0, ninf, 1.0],
                  [3.0, 3.0, 3.0, 3.0],
                  [3.0e38, 3.0e38, -3.0e38, 0.0],
                  [ninf, ninf, ninf, ninf]], np.float32)
    got = rt.Softmax(T(ctx, x)).numpy()
    ref = O.softmax(x)
    np.testing.assert_array_equal(got[0], [1.0, 0.0, 0.0, 0.0])
    assert got[1, 0] == 0.0 and got[1, 2] == 0.0
    close(got[1], ref64.softmax(np.array([-np.inf, 2.0, -np.inf, 1.0])), 1e-6)
    np.testing.assert_allclose(got[2], 0.25, rtol=0, atol=1e-7)
    np.testing.assert_allclose(got[3], [0.5, 0.5, 0.0, 0.0], rtol=0, atol=1e-7)
    assert np.all(np.isnan(got[4])) and np.all(np.isnan(ref[4]))
    np.testing.assert_allclose(got[:4], ref[:4], rtol=0, atol=1e-7)


def test_kat_gather_split_concat_exact(ctx):
    for name in ("gather_rows", "gather_matrix_indices"):
        c = KAT[name]
        out = rt.Gather(T(ctx, c["data"]), T(ctx, c["idx"], np.int64)).numpy()
        np.testing.assert_array_equal(out, c["expect"])
    with pytest.raises(RuntimeError, match="out of range"):
        rt.Gather(T(ctx, np.ones((4, 3))), T(ctx, [4], np.int64))
    for name in ("split_even_axis0", "split_uneven_axis1", "split_three_way_qkv"):
        c = KAT[name]
        parts = rt.Split(T(ctx, c["x"]), c["axis"], c["sizes"])
        for p, e in zip(parts, c["expect"]):
            np.testing.assert_array_equal(p.numpy(), e)
        np.testing.assert_array_equal(rt.Concat(parts, c["axis"]).numpy(), c["x"])


# ---------------------------------------------------------------- GEMM

GEMM_SHAPES = [(1, 1, 1), (3, 5, 7), (64, 64, 32), (65, 63, 33), (128, 768, 768),
               (128, 3072, 768), (200, 300, 130), (4096, 768, 64), (33, 2304, 768)]


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_vs_oracle(ctx, M, N, K, ta, tb):
    A = rnd((K, M) if ta else (M, K), M * 7 + K)
    B = rnd((N, K) if tb else (K, N), N * 3 + K, 0.05)
    got = rt.Gemm(T(ctx, A), T(ctx, B), trans_a=ta, trans_b=tb).numpy()
    close(got, O.sgemm(A, B, ta, tb))


@pytest.mark.parametrize("act", [L.ACT_NONE, L.ACT_GELU_ERF, L.ACT_GELU_TANH, L.ACT_RELU])
def test_gemm_epilogues(ctx, act):
    M, N, K = 130, 770, 96
    A, B = rnd((M, K), 1), rnd((K, N), 2, 0.1)
    bias, res = rnd(N, 3), rnd((M, N), 4)
    got = rt.Gemm(T(ctx, A), T(ctx, B), T(ctx, bias), 1.0, 1.0, residual=T(ctx, res),
                  act=act).numpy()
    v = (A.astype(np.float64) @ B + bias) + res
    ref = {L.ACT_NONE: v, L.ACT_GELU_ERF: ref64.gelu_erf(v), L.ACT_GELU_TANH: ref64.gelu_tanh(v),
           L.ACT_RELU: np.maximum(v, 0)}[act]
    close(got, ref)


@pytest.mark.parametrize("M,N,K,tb", [(100, 2304, 200, False), (128, 3072, 768, False),
                                       (77, 2352, 52, True)])
def test_gemm_small_m_48_wide_tiles(ctx, M, N, K, tb):
    """Small-M products whose N is a multiple of 48 with enough tiles take
    the 32x48 K-split kernel: partial row tiles, K not a multiple of the
    per-wave k-groups, B plain and transposed."""
    A = rnd((M, K), 94 + M)
    B = rnd((N, K) if tb else (K, N), 95 + K, 0.05)
    bias, res = rnd(N, 96), rnd((M, N), 97)
    got = rt.Gemm(T(ctx, A), T(ctx, B), T(ctx, bias), 1.0, 1.0, trans_b=tb, residual=T(ctx, res),
                  act=L.ACT_GELU_ERF).numpy()
    Bd = (B.T if tb else B).astype(np.float64)
    close(got, ref64.gelu_erf((A.astype(np.float64) @ Bd + bias) + res))


@pytest.mark.parametrize("N,K", [(2, 768), (768, 768), (50, 3072), (33, 100)])
def test_gemm_single_row_transb_epilogues(ctx, N, K):
    """M=1 with B^T takes the GEMV route (matmul.cc:207-216); bias, residual and
    activation must match the GEMM epilogue."""
    A, B = rnd((1, K), 90 + N), rnd((N, K), 91 + K, 0.05)
    bias, res = rnd(N, 92), rnd((1, N), 93)
    for act in (L.ACT_NONE, L.ACT_RELU, L.ACT_GELU_TANH):
        got = rt.Gemm(T(ctx, A), T(ctx, B), T(ctx, bias), 1.0, 1.0, trans_b=True,
                      residual=T(ctx, res), act=act).numpy()
        v = (A.astype(np.float64) @ B.T.astype(np.float64) + bias) + res
        ref = {L.ACT_NONE: v, L.ACT_RELU: np.maximum(v, 0), L.ACT_GELU_TANH: ref64.gelu_tanh(v)}[act]
        close(got, ref)


# Large-M products on the tiled kernel, with edge tiles (M, N not multiples
# of the tile) and partial last K panels: 128x96 tiles (N % 96 == 0), 128x128
# (N % 96 != 0, >= 3 tiles per CU), 128x64 (1-3 tiles per CU).
@pytest.mark.parametrize("M,N,K", [(4000, 768, 768), (4000, 3072, 100), (4032, 768, 45),
                                   (4000, 3136, 96), (2000, 2000, 130)])
@pytest.mark.parametrize("act", [L.ACT_NONE, L.ACT_GELU_ERF])
def test_gemm_large_m_edge_tiles(ctx, M, N, K, act):
    A, B = rnd((M, K), M + K), rnd((K, N), N + K, 0.05)
    bias, res = rnd(N, 3 + N), rnd((M, N), 4 + M)
    got = rt.Gemm(T(ctx, A), T(ctx, B), T(ctx, bias), 1.0, 1.0, residual=T(ctx, res),
                  act=act).numpy()
    v = (A.astype(np.float64) @ B + bias) + res
    close(got, ref64.gelu_erf(v) if act == L.ACT_GELU_ERF else v)


@pytest.mark.parametrize("M,N,K", [(4000, 768, 70), (4096, 768, 64)])
def test_gemm_large_m_c_kinds_alpha_beta(ctx, M, N, K):
    A, B = rnd((M, K), 15), rnd((K, N), 16, 0.1)
    for C in (rnd(N, 17), rnd((M, N), 18), np.array([1.5], np.float32)):
        got = rt.Gemm(T(ctx, A), T(ctx, B), T(ctx, C), alpha=0.75, beta=-2.0).numpy()
        close(got, 0.75 * (A.astype(np.float64) @ B) + -2.0 * np.broadcast_to(
            C.astype(np.float64), (M, N)))


def test_gemm_c_kinds_alpha_beta(ctx):
    A, B = rnd((37, 29), 5), rnd((29, 41), 6)
    for C in (rnd(41, 7), rnd((37, 41), 8), np.array([1.5], np.float32)):
        got = rt.Gemm(T(ctx, A), T(ctx, B), T(ctx, C), alpha=0.75, beta=-2.0).numpy()
        close(got, O.gemm(A, B, C, alpha=0.75, beta=-2.0))


@pytest.mark.parametrize("M,N,K", [(128, 768, 3072), (100, 768, 2048), (160, 768, 3072),
                                   (256, 768, 4096), (128, 768, 2000)])
@pytest.mark.parametrize("act", [L.ACT_NONE, L.ACT_GELU_ERF])
def test_gemm_small_m_long_k(ctx, M, N, K, act):
    """Small-M products with a long K (the b=1 FFN-down and its neighbours:
    ragged M, K not a multiple of the waves' ring) with bias, residual and
    activation, against float64, deterministic over repeats."""
    A, B = rnd((M, K), 21 + M), rnd((K, N), 22 + K, 0.03)
    bias, res = rnd(N, 23), rnd((M, N), 24)
    a, b, c, r = T(ctx, A), T(ctx, B), T(ctx, bias), T(ctx, res)
    got = rt.Gemm(a, b, c, 1.0, 1.0, residual=r, act=act).numpy()
    v = (A.astype(np.float64) @ B + bias) + res
    close(got, ref64.gelu_erf(v) if act == L.ACT_GELU_ERF else v)
    for _ in range(2):
        np.testing.assert_array_equal(rt.Gemm(a, b, c, 1.0, 1.0, residual=r, act=act).numpy(), got)


def test_gemm_deterministic(ctx):
    A, B = rnd((128, 768), 9), rnd((768, 3072), 10, 0.02)
    a, b = T(ctx, A), T(ctx, B)
    first = rt.Gemm(a, b).numpy()
    for _ in range(2):
        np.testing.assert_array_equal(rt.Gemm(a, b).numpy(), first)


def test_gemm_k_split_over_blocks_interleaved(ctx):
    """Long-K small-M products whose K is also split over two blocks per
    tile (the b=1 FFN-down shape and a ragged neighbour), launched
    interleaved many times: each tile's arrival counter must be back at zero
    after every launch, so every repeat gives the first result's bits, and
    that result matches float64."""
    cases = []
    for M, seed in ((128, 31), (160, 32), (256, 33)):
        A, B = rnd((M, 3072), seed), rnd((3072, 768), seed + 10, 0.03)
        bias, res = rnd(768, seed + 20), rnd((M, 768), seed + 30)
        args = (T(ctx, A), T(ctx, B), T(ctx, bias))
        r = T(ctx, res)
        got = rt.Gemm(*args, 1.0, 1.0, residual=r).numpy()
        close(got, (A.astype(np.float64) @ B + bias) + res)
        cases.append((args, r, got))
    for _ in range(8):
        for args, r, first in cases:
            np.testing.assert_array_equal(rt.Gemm(*args, 1.0, 1.0, residual=r).numpy(), first)


@pytest.mark.parametrize("M", [128, 1024, 4096])
def test_config2_ffn_gelu_then_layernorm(ctx, M):
    """GELU_erf(X W1 + b1) -> W2 + b2 -> LayerNorm(eps 1e-12)."""
    X = rnd((M, 768), 11)
    W1, b1 = rnd((768, 3072), 12, 0.02), rnd(3072, 13, 0.02)
    W2, b2 = rnd((3072, 768), 14, 0.02), rnd(768, 15, 0.02)
    g, bt = np.ones(768, np.float32), np.zeros(768, np.float32)
    f = rt.FusedMatMulAddGELU(T(ctx, X), T(ctx, W1), T(ctx, b1))
    y2 = rt.Gemm(f, T(ctx, W2), T(ctx, b2))
    y = rt.LayerNorm(y2, T(ctx, g), T(ctx, bt), 1e-12).numpy()
    f_ref = O.fused_matmul_add_gelu(X, W1, b1)
    close(f.numpy(), f_ref)
    ref = O.layernorm(O.gemm(f_ref, W2, b2), g, bt, 1e-12)
    close(y, ref)


# ------------------------------------------------------------ attention

@pytest.mark.parametrize("B,S", [(1, 1), (1, 5), (2, 33), (1, 128), (3, 130), (2, 257)])
def test_attention_vs_oracle(ctx, B, S):
    H, hd = 128, 64
    q, k, v = rnd((B, S, H), 20 + S), rnd((B, S, H), 21 + S), rnd((B, S, H), 22 + S)
    got = rt.FusedAttention(T(ctx, q), T(ctx, k), T(ctx, v), None, hd, -3e38).numpy()
    close(got, O.fused_attention(q, k, v, None, hd, -3e38))


def test_attention_padding_masks_and_fully_masked_row(ctx):
    B, S, H, hd = 4, 96, 128, 64
    q, k, v = rnd((B, S, H), 30), rnd((B, S, H), 31), rnd((B, S, H), 32)
    mask = np.zeros((B, 1, 1, S), np.uint8)
    mask[0, ..., 17:] = 1          # padding tail
    mask[1, ..., :40] = 1          # leading masked keys
    mask[2, ..., :] = 1            # every key masked: uniform average of V
    fill = graphs.FILL_MIN
    got = rt.FusedAttention(T(ctx, q), T(ctx, k), T(ctx, v), T(ctx, mask, np.uint8), hd,
                            fill).numpy()
    close(got, O.fused_attention(q, k, v, mask, hd, fill))
    close(got[2], np.broadcast_to(v[2].mean(0), (S, H)))


def test_attention_general_mask_and_generic_head_dim(ctx):
    B, S, H = 2, 40, 96
    rng = np.random.default_rng(33)
    q, k, v = rnd((B, S, H), 34), rnd((B, S, H), 35), rnd((B, S, H), 36)
    for hd in (64 if H % 64 == 0 else 32, 32, 8):
        nH = H // hd
        m4 = (rng.random((B, nH, S, S)) < 0.3).astype(np.uint8)
        got = rt.FusedAttention(T(ctx, q), T(ctx, k), T(ctx, v), T(ctx, m4, np.uint8), hd,
                                -1e30).numpy()
        close(got, O.fused_attention(q, k, v, m4, hd, -1e30))


@pytest.mark.parametrize("shape", [(1, 1, 70, 70), (2, 2, 70, 70), (2, 1, 1, 70)])
def test_attention_small_grid_masks_head_dim_64(ctx, shape):
    """Small grids (the 16-query kernel) at head_dim 64 with a per-query mask
    ([B or 1, nH or 1, S, S]: one mask byte per score) and a key-only mask
    ([B, 1, 1, S]: one byte per key, shared across the wave by a ballot),
    S = 70 (a ragged last key tile and query block), a few rows fully
    masked, against the oracle."""
    B, S, H, hd = 2, 70, 128, 64
    rng = np.random.default_rng(37)
    q, k, v = rnd((B, S, H), 38), rnd((B, S, H), 39), rnd((B, S, H), 40)
    m = (rng.random(shape) < 0.3).astype(np.uint8)
    if shape[2] == S:
        m[..., 5, :] = 1             # a fully masked query row
    else:
        m[..., 60:] = 1              # a masked tail of keys
    fill = graphs.FILL_MIN
    got = rt.FusedAttention(T(ctx, q), T(ctx, k), T(ctx, v), T(ctx, m, np.uint8), hd,
                            fill).numpy()
    close(got, O.fused_attention(q, k, v, m, hd, fill))


@pytest.mark.parametrize("S", [128, 512])
def test_config3_qkv_plus_mha(ctx, S):
    """fused QKV projection + MHA, B=32, valid length U[16,S]."""
    B, H = 32, 768
    rng = np.random.default_rng(40 + S)
    X = rnd((B, S, H), 41)
    ws = [rnd((H, H), 42 + i, 0.02) if i % 2 == 0 else rnd(H, 42 + i, 0.02) for i in range(6)]
    lens = rng.integers(16, S + 1, size=B)
    mask = (np.arange(S)[None, :] >= lens[:, None]).astype(np.uint8).reshape(B, 1, 1, S)
    q, k, v = rt.FusedQKVProjection(T(ctx, X), *[T(ctx, w) for w in ws])
    got = rt.FusedAttention(q, k, v, T(ctx, mask, np.uint8), 64, graphs.FILL_MIN).numpy()
    qr, kr, vr = O.fused_qkv(X, *ws)
    close(q.numpy(), qr)
    close(v.numpy(), vr)
    close(got, O.fused_attention(qr, kr, vr, mask, 64, graphs.FILL_MIN))


# ------------------------------------------------------ LN / pointwise

@pytest.mark.parametrize("rows,feat", [(1, 768), (128, 768), (7, 100), (3, 2000)])
@pytest.mark.parametrize("eps", [1e-12, 1e-5])
def test_layernorm_vs_oracle(ctx, rows, feat, eps):
    x = rnd((rows, feat), rows + feat, 3.0) + 1.0
    g, b = rnd(feat, 50), rnd(feat, 51)
    close(rt.LayerNorm(T(ctx, x), T(ctx, g), T(ctx, b), eps).numpy(), O.layernorm(x, g, b, eps))
    r = rnd((rows, feat), 52)
    close(rt.LayerNorm(T(ctx, x), T(ctx, g), T(ctx, b), eps, residual=T(ctx, r)).numpy(),
          O.layernorm(x + r, g, b, eps))


def test_activations_and_add(ctx):
    x = np.linspace(-8, 8, 40001).astype(np.float32)
    close(rt.Gelu(T(ctx, x)).numpy(), O.gelu(x), 1e-6)
    close(rt.GeluTanh(T(ctx, x)).numpy(), O.gelu_tanh(x), 1e-6)
    np.testing.assert_array_equal(rt.Relu(T(ctx, x)).numpy(), np.maximum(x, 0))
    a, row = rnd((5, 7, 9), 60), rnd(9, 61)
    np.testing.assert_array_equal(rt.Add(T(ctx, a), T(ctx, row)).numpy(), a + row)
    np.testing.assert_array_equal(rt.Add(T(ctx, row), T(ctx, a)).numpy(), a + row)


def test_argmax_exact(ctx):
    rng = np.random.default_rng(70)
    for n in (1, 7, 50257, 1 << 20):
        x = rng.standard_normal(n).astype(np.float32)
        assert rt.Argmax(T(ctx, x)) == O.argmax(x)
    y = np.full(50257, -2.0, np.float32)
    y[[123, 40000, 50256]] = 9.0
    assert rt.Argmax(T(ctx, y)) == 123
    z = np.full(300, -np.inf, np.float32)
    assert rt.Argmax(T(ctx, z)) == 0


# ------------------------------------------------------------ GEMV

@pytest.mark.parametrize("N,K", [(5, 7), (2304, 768), (768, 3072), (3072, 768), (50257, 768)])
def test_gemv_vs_oracle(ctx, N, K):
    W, x = rnd((N, K), N, 0.02), rnd(K, K)
    close(rt.Gemv(T(ctx, W), T(ctx, x)).numpy(), O.sgemv_rows(W, x))
    bias, res = rnd(N, 80), rnd(N, 81)
    g, b = rnd(K, 82) + 1.0, rnd(K, 83)
    got = rt.Gemv(T(ctx, W), T(ctx, x), T(ctx, bias), T(ctx, res), L.ACT_GELU_TANH,
                  ln=(T(ctx, g), T(ctx, b), 1e-5)).numpy()
    xn = O.layernorm(x[None], g, b, 1e-5)[0]
    ref = O.gelu_tanh((O.sgemv_rows(W, xn) + bias) + res)
    close(got, ref)


# ------------------------------------------------------------- int4

def test_int4_reference_fixture(ctx):
    g = load_golden("int4_fixture.json")
    N, K = g["N"], g["K"]
    W = np.frombuffer(bytes.fromhex(g["W_hex"]), np.uint8).reshape(N, K // 2)
    x = np.array(g["x"], np.float32)
    s = np.array(g["scales"], np.float32)
    y = rt.Int4Gemv(T(ctx, W, np.uint8), T(ctx, s), T(ctx, x), K).numpy()[0]
    np.testing.assert_allclose(y, g["y_per_row"], atol=g["tol"])
    yt = rt.Int4Gemv(T(ctx, W, np.uint8), T(ctx, np.full(N, g["scale"], np.float32)),
                     T(ctx, x), K).numpy()[0]
    np.testing.assert_allclose(yt, g["y_per_tensor"], atol=g["tol"])


@pytest.mark.parametrize("N,K", [(16, 256), (2304, 768), (768, 3072), (50257, 768), (7, 30)])
def test_int4_unpack_bit_exact(ctx, N, K):
    W, s = graphs.int4_weights(N, K, 90, "unpack")
    got = rt.Int4Unpack(T(ctx, W, np.uint8), T(ctx, s), K).numpy()
    np.testing.assert_array_equal(got.view(np.uint32), O.int4_unpack(W, s, K).view(np.uint32))


def _int4_close(got, W, s, x, K):
    """|d| <= 1e-4 * max(|y_ref|, sum_k |w_k x_k| * 2^-10) per element, and
    plain relative error reported by the assertion message."""
    ref = O.int4_gemv_per_row(W, s, x, K)
    deq = ref64.int4_deq(W, s, K).astype(np.float64)
    mag = np.abs(x.astype(np.float64)) @ np.abs(deq).T
    bound = 1e-4 * np.maximum(np.abs(ref), mag * 2.0 ** -10)
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= bound), f"max err {err.max():.3e}, max rel {np.max(err / (np.abs(ref) + 1e-30)):.3e}"


@pytest.mark.parametrize("N,K", [(2304, 768), (768, 3072), (50257, 768), (33, 64), (9, 30)])
@pytest.mark.parametrize("B", [1, 8])
def test_int4_gemv_vs_oracle(ctx, N, K, B):
    W, s = graphs.int4_weights(N, K, 91, "gemv")
    x = rnd((B, K), 92)
    got = rt.Int4Gemv(T(ctx, W, np.uint8), T(ctx, s), T(ctx, x), K).numpy()
    _int4_close(got, W, s, x, K)


def test_int4_grouped_full_gpt2_volume(ctx):
    """BASELINE config 5 shapes in one launch: all 49 GPT-2-small matrices."""
    mats = []
    host = []
    for i, (N, K) in enumerate(graphs.int4_matrices()):
        W, s = graphs.int4_weights(N, K, 93, f"m{i}")
        x = rnd((1, K), 200 + i)
        y = Tensor.empty(ctx, (1, N))
        mats.append((T(ctx, W, np.uint8), T(ctx, s), T(ctx, x), y, K))
        host.append((W, s, x, K))
    rt.int4_gemv_grouped(ctx, mats, 1)
    for (Wd, sd, xd, y, K), (W, s, x, _) in zip(mats, host):
        if W.shape[0] > 5000:
            # LM head: check a slice of rows exactly against the oracle
            _int4_close(y.numpy()[:, :4096], W[:4096], s[:4096], x, K)
        else:
            _int4_close(y.numpy(), W, s, x, K)


@pytest.mark.parametrize("scale", [1e-30, 1.0, 1e30])
def test_int4_gemv_batches_and_x_scale(ctx, scale):
    """Five batches (a pass of four plus one) and x spanning 60 decades: the
    fixed-point exponent is chosen per batch from max|x|."""
    N, K, B = 300, 768, 5
    W, s = graphs.int4_weights(N, K, 98, "scale")
    x = (rnd((B, K), 99) * np.float32(scale)).astype(np.float32)
    x[3] *= np.float32(1e-3)  # batches of different magnitude in one pass
    got = rt.Int4Gemv(T(ctx, W, np.uint8), T(ctx, s), T(ctx, x), K).numpy()
    assert np.all(np.isfinite(got))
    _int4_close(got, W, s, x, K)


def test_int4_gemv_nan_propagates(ctx):
    N, K = 64, 768
    W, s = graphs.int4_weights(N, K, 100, "nan")
    x = rnd((2, K), 101)
    x[1, 17] = np.nan
    got = rt.Int4Gemv(T(ctx, W, np.uint8), T(ctx, s), T(ctx, x), K).numpy()
    assert np.all(np.isnan(got[1]))
    _int4_close(got[:1], W, s, x[:1], K)


def test_int4_reference_stand_in_shape(ctx):
    """The reference's own benchmark matrix, N=60000 x K=2048 (int4_gemv_amx.cc:550),
    batch 1; rows checked on a slice to keep the float64 bound cheap."""
    N, K = 60000, 2048
    W, s = graphs.int4_weights(N, K, 96, "standin")
    x = rnd((1, K), 97)
    got = rt.Int4Gemv(T(ctx, W, np.uint8), T(ctx, s), T(ctx, x), K).numpy()
    for lo in (0, N - 4096):
        _int4_close(got[:, lo:lo + 4096], W[lo:lo + 4096], s[lo:lo + 4096], x, K)


@pytest.mark.parametrize("N,K", [(1, 768), (7, 768), (65, 768), (97, 768), (1, 3072),
                                 (5, 3072), (19, 3072), (40, 1536), (130, 512), (8193, 768),
                                 (8231, 768)])
def test_int4_gemv_batch1_run_edges(ctx, N, K):
    """Batch 1, row counts that end a wave's run early (fewer rows than one
    chunk, a partial last chunk, a partial last run, whole runs of waves that
    only round a matrix up to a block), the 15 KB runs of K = 768 matrices
    over 8192 rows, and the row lengths that take the looped form (K = 1536,
    512)."""
    W, s = graphs.int4_weights(N, K, 102, "edges")
    x = rnd((1, K), 103)
    got = rt.Int4Gemv(T(ctx, W, np.uint8), T(ctx, s), T(ctx, x), K).numpy()
    _int4_close(got, W, s, x, K)


@pytest.mark.parametrize("N,K,B", [(37, 1536, 3), (100, 3072, 2), (17, 768, 6), (1000, 768, 8),
                                   (5, 3072, 7), (130, 1536, 5)])
def test_int4_gemv_multi_batch_shapes(ctx, N, K, B):
    """Several batches (one and two column groups of four), rows split over
    2 or 4 waves (K = 1536, 3072) and tiles that end past the last row."""
    W, s = graphs.int4_weights(N, K, 104, "multi")
    x = rnd((B, K), 105)
    got = rt.Int4Gemv(T(ctx, W, np.uint8), T(ctx, s), T(ctx, x), K).numpy()
    _int4_close(got, W, s, x, K)


@pytest.mark.parametrize("B", [1, 8])
def test_int4_deterministic(ctx, B):
    W, s = graphs.int4_weights(3072, 768, 94, "det")
    x = rnd((B, 768), 95)
    a, b, c = T(ctx, W, np.uint8), T(ctx, s), T(ctx, x)
    first = rt.Int4Gemv(a, b, c, 768).numpy()
    np.testing.assert_array_equal(rt.Int4Gemv(a, b, c, 768).numpy(), first)


# ------------------------------------------------------ decode attention

def test_kv_append_attend_vs_numpy(ctx):
    nH, D, T_ = 12, 64, 160
    rng = np.random.default_rng(100)
    kc = np.zeros((nH, T_, D), np.float32)
    vc = np.zeros((nH, T_, D), np.float32)
    kc[:, :40] = rng.standard_normal((nH, 40, D))
    vc[:, :40] = rng.standard_normal((nH, 40, D))
    kcd, vcd = T(ctx, kc), T(ctx, vc)
    for pos in (40, 41, 42):
        q, kn, vn = (rng.standard_normal(nH * D).astype(np.float32) for _ in range(3))
        out = rt.KvAppendAttend(T(ctx, q), T(ctx, kn), T(ctx, vn), kcd, vcd,
                                T(ctx, [pos], np.int64), nH, D, T_).numpy()
        kc[:, pos] = kn.reshape(nH, D)
        vc[:, pos] = vn.reshape(nH, D)
        t = pos + 1
        s = np.einsum("hd,htd->ht", q.reshape(nH, D).astype(np.float64), kc[:, :t]) / 8.0
        p = ref64.softmax(s)
        ref = np.einsum("ht,htd->hd", p, vc[:, :t]).ravel()
        close(out, ref)
        np.testing.assert_array_equal(kcd.numpy()[:, pos], kn.reshape(nH, D))
        np.testing.assert_array_equal(vcd.numpy()[:, pos], vn.reshape(nH, D))


@pytest.mark.parametrize("pos", [0, 31, 255, 256, 299])
def test_kv_append_attend_ignores_rows_past_pos(ctx, pos):
    """Cache rows at and past pos hold NaN/Inf (the kernel reads its first
    key chunk before the position, clamped to the cache, not to pos): the
    output depends on rows [0, pos) of the cache and the new row only. T=300
    spans two rounds of key chunks (8 waves x 32 keys)."""
    nH, D, T_ = 12, 64, 300
    rng = np.random.default_rng(200 + pos)
    kc = rng.standard_normal((nH, T_, D)).astype(np.float32)
    vc = rng.standard_normal((nH, T_, D)).astype(np.float32)
    kc[:, pos:, ::2], kc[:, pos:, 1::2] = np.nan, np.inf
    vc[:, pos:, ::2], vc[:, pos:, 1::2] = -np.inf, np.nan
    q, kn, vn = (rng.standard_normal(nH * D).astype(np.float32) for _ in range(3))
    kcd, vcd = T(ctx, kc), T(ctx, vc)
    out = rt.KvAppendAttend(T(ctx, q), T(ctx, kn), T(ctx, vn), kcd, vcd,
                            T(ctx, [pos], np.int64), nH, D, T_).numpy()
    kc[:, pos] = kn.reshape(nH, D)
    vc[:, pos] = vn.reshape(nH, D)
    t = pos + 1
    s = np.einsum("hd,htd->ht", q.reshape(nH, D).astype(np.float64), kc[:, :t]) / 8.0
    ref = np.einsum("ht,htd->hd", ref64.softmax(s), vc[:, :t]).ravel()
    assert np.isfinite(out).all()
    close(out, ref)
    np.testing.assert_array_equal(kcd.numpy()[:, pos], kn.reshape(nH, D))
    np.testing.assert_array_equal(vcd.numpy()[:, pos], vn.reshape(nH, D))
