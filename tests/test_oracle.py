"""Pins the CPU oracle (CPU only, no GPU).

Each oracle function is checked against (a) the known-answer vectors of the
reference's own tests (tests/golden/kernels_kat.json, from kernels_test.cc),
(b) the closed-form fixtures of int4_gemv_amx.cc and amx_gemm_test.cc
(tests/golden/*_fixture.json), and (c) float64 statements of the mathematics
(tests/ref64.py) on small random shapes, plus invariants (softmax rows sum to
1, LN mean 0 / var 1, masked keys get zero weight, incremental decode equals
full recompute). The last tests plant mistakes in copies of oracle outputs to
show that the checks used would catch them.
"""
from __future__ import annotations

import hashlib
import math

import numpy as np
import pytest

import oracle as O
from inferc_amd import graphs
from tests import ref64
from tests.conftest import load_golden

KAT = load_golden("kernels_kat.json")["cases"]


def f32(x):
    return np.asarray(x, np.float32)


# ------------------------------------------------------- reference KATs

def test_kat_matmul_basic():
    c = KAT["matmul_basic_2d"]
    np.testing.assert_allclose(O.matmul(f32(c["a"]), f32(c["b"])), c["expect"], atol=c["tol"])


def test_kat_matmul_batched_broadcast():
    c = KAT["matmul_batched_broadcast"]
    a = np.arange(1, 13, dtype=np.float32).reshape(c["a_shape"])
    b = np.arange(1, 13, dtype=np.float32).reshape(c["b_shape"])
    out = O.matmul(a, b)
    assert out.shape == (2, 2, 4)
    np.testing.assert_allclose(out[0, 0, :2], c["expect_first_row_prefix"], atol=c["tol"])
    np.testing.assert_allclose(out, a.astype(np.float64) @ b, atol=1e-4)


@pytest.mark.parametrize("name", ["gemm_bias_added", "gemv_notransb", "gemv_transb",
                                  "gemv_alpha_beta"])
def test_kat_gemm(name):
    c = KAT[name]
    out = O.gemm(f32(c["a"]), f32(c["b"]), None if c.get("bias") is None else f32(c["bias"]),
                 alpha=c.get("alpha", 1.0), beta=c.get("beta", 1.0),
                 trans_b=c.get("trans_b", False))
    np.testing.assert_allclose(out, c["expect"], atol=c["tol"])


@pytest.mark.parametrize("name", ["attention_single_head", "attention_mask_zeros_out_key"])
def test_kat_attention(name):
    c = KAT[name]
    out = O.fused_attention(f32(c["q"]), f32(c["k"]), f32(c["v"]),
                            None if c["mask"] is None else np.array(c["mask"], np.uint8),
                            c["head_dim"], c["fill"])
    np.testing.assert_allclose(out, c["expect"], atol=c["tol"])


def test_kat_gelu_and_tanh():
    c = KAT["gelu_known_values"]
    np.testing.assert_allclose(O.gelu(f32(c["x"])), c["expect"], atol=c["tol"])
    c = KAT["gelu_tanh_formula"]
    np.testing.assert_allclose(O.gelu_tanh(f32(c["x"])), c["expect"], atol=c["tol"])


def test_kat_softmax_stable():
    c = KAT["softmax_stable"]
    y = O.softmax(f32(c["x"]))
    assert np.all(np.isfinite(y))
    assert abs(float(y.sum()) - 1.0) < c["sum_tol"]
    assert y[0, 3] > y[0, 2] and y[0, 3] > y[0, 1]


def test_softmax_axis_mid_dim():  # kernels_test.cc:327-341
    x = np.arange(12, dtype=np.float32).reshape(2, 3, 2)
    y = O.softmax(x, 1)
    np.testing.assert_allclose(y.sum(1), 1.0, atol=1e-5)
    np.testing.assert_allclose(y, ref64.softmax(x, 1), atol=1e-6)


def test_kat_layernorm():
    c = KAT["layernorm_mean0_var1"]
    y = O.layernorm(f32(c["x"]), np.ones(4, np.float32), np.zeros(4, np.float32), c["eps"])
    np.testing.assert_allclose(y.mean(-1), 0.0, atol=c["mean_tol"])
    np.testing.assert_allclose(((y - y.mean(-1, keepdims=True)) ** 2).mean(-1), 1.0,
                               atol=c["var_tol"])


@pytest.mark.parametrize("name", ["gather_rows", "gather_matrix_indices"])
def test_kat_gather(name):
    c = KAT[name]
    out = O.gather_rows(f32(c["data"]), np.array(c["idx"], np.int64))
    np.testing.assert_array_equal(out, c["expect"])


def test_gather_negative_and_out_of_range():
    t = np.arange(12, dtype=np.float32).reshape(4, 3)
    np.testing.assert_array_equal(O.gather_rows(t, np.array([-1])), t[[3]])
    with pytest.raises(RuntimeError):
        O.gather_rows(t, np.array([4]))


@pytest.mark.parametrize("name", ["split_even_axis0", "split_uneven_axis1",
                                  "split_three_way_qkv"])
def test_kat_split(name):
    c = KAT[name]
    parts = O.split(f32(c["x"]), c["axis"], c["sizes"])
    for p, e in zip(parts, c["expect"]):
        np.testing.assert_array_equal(p, e)
    np.testing.assert_array_equal(O.concat(parts, c["axis"]), c["x"])


def test_kat_concat():
    c = KAT["concat_axis0"]
    np.testing.assert_array_equal(O.concat([f32(p) for p in c["parts"]], c["axis"]), c["expect"])


@pytest.mark.parametrize("name", ["add_row_broadcast", "add_no_broadcast", "add_scalar"])
def test_kat_add_broadcast(name):
    c = KAT[name]
    y = O.add_bcast(f32(c["a"]), f32(c["b"])).ravel()
    for i, v in c["expect_at"]:
        assert abs(y[i] - v) <= c["tol"], (name, i, y[i], v)


def test_kat_add_parallel_rows():
    # kernels_test.cc:196-216 input: a[i] = i - 192 over [4, 96], a row of 2.0.
    c = KAT["add_parallel_rows"]
    n = int(np.prod(c["a_shape"]))
    a = (np.arange(n, dtype=np.float32) - 192.0).reshape(c["a_shape"])
    b = np.full((1, c["a_shape"][1]), c["b_value"], np.float32)
    np.testing.assert_array_equal(O.add_bcast(a, b), a + np.float32(c["b_value"]))
    # A per-row bias (not a repeat of one row) must not pass for the row broadcast.
    col = np.arange(c["a_shape"][1], dtype=np.float32)
    y = O.add_bcast(a, col[None, :])
    np.testing.assert_array_equal(y[3], a[3] + col)


# --------------------------------------------------- closed-form fixtures

def test_gemm_fixture_sin_cos():
    g = load_golden("gemm_fixture.json")
    M, N, K = g["M"], g["N"], g["K"]
    A = np.sin(0.1 * np.arange(M * K)).astype(np.float32).reshape(M, K)
    B = np.cos(0.07 * np.arange(K * N)).astype(np.float32).reshape(K, N)
    np.testing.assert_allclose(O.sgemm(A, B), np.array(g["C"]).reshape(M, N), atol=1e-5)


def _int4_fixture():
    g = load_golden("int4_fixture.json")
    N, K = g["N"], g["K"]
    W = np.frombuffer(bytes.fromhex(g["W_hex"]), np.uint8).reshape(N, K // 2)
    assert np.array_equal(W.ravel(), [(i * 31) & 0xFF for i in range(N * K // 2)])
    x = np.array(g["x"], np.float32)
    np.testing.assert_array_equal(x, np.sin(0.07 * np.arange(K)).astype(np.float32))
    return g, N, K, W, x, np.array(g["scales"], np.float32)


def test_int4_fixture_per_row_and_per_tensor():
    g, N, K, W, x, scales = _int4_fixture()
    y = O.int4_gemv_per_row(W, scales, x, K)[0]
    np.testing.assert_allclose(y, g["y_per_row"], rtol=0, atol=1e-6)
    yt = O.int4_gemv_per_tensor(W, g["scale"], x, N, K)
    np.testing.assert_allclose(yt, g["y_per_tensor"], rtol=0, atol=1e-6)
    # fp32-accumulating baseline variant stays within the fixture tolerance
    y32 = O.int4_gemv_f32acc(W, scales, x, K)[0]
    np.testing.assert_allclose(y32, g["y_per_row"], atol=g["tol"])


def test_int4_unpack_bit_exact():
    g, N, K, W, x, scales = _int4_fixture()
    deq = O.int4_unpack(W, scales, K)
    assert hashlib.sha256(deq.tobytes()).hexdigest() == g["dequant_per_row_bits_sha"]
    # nibble rule by hand on byte 0: (0*31)&0xff = 0 -> q=-8 for k=0 and k=1
    assert deq[0, 0] == np.float32(scales[0]) * np.float32(-8)
    b1 = (1 * 31) & 0xFF  # byte 1 holds k=2 (low nibble) and k=3 (high nibble)
    assert deq[0, 2] == np.float32(scales[0]) * np.float32((b1 & 0xF) - 8)
    assert deq[0, 3] == np.float32(scales[0]) * np.float32((b1 >> 4) - 8)
    np.testing.assert_array_equal(deq, ref64.int4_deq(W, scales, K))


def test_int4_random_batched_vs_float64():
    W, s = graphs.int4_weights(96, 320, 5, "t")
    x = np.random.default_rng(0).standard_normal((3, 320)).astype(np.float32)
    y = O.int4_gemv_per_row(W, s, x, 320)
    ref = x.astype(np.float64) @ ref64.int4_deq(W, s, 320).astype(np.float64).T
    np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-6)


# ------------------------------------------------------ float64 statements

def test_sgemm_transposes_vs_float64():
    rng = np.random.default_rng(1)
    for ta in (False, True):
        for tb in (False, True):
            A = rng.standard_normal((37, 19) if ta else (19, 37)).astype(np.float32)
            B = rng.standard_normal((53, 37) if tb else (37, 53)).astype(np.float32)
            ref = (A.T if ta else A).astype(np.float64) @ (B.T if tb else B)
            np.testing.assert_allclose(O.sgemm(A, B, ta, tb), ref, atol=1e-4)


def test_gemm_c_kinds_vs_float64():
    rng = np.random.default_rng(2)
    A = rng.standard_normal((5, 7)).astype(np.float32)
    B = rng.standard_normal((7, 3)).astype(np.float32)
    for C in (rng.standard_normal(3), rng.standard_normal((5, 3)), np.array([2.5])):
        C = C.astype(np.float32)
        ref = 1.5 * (A.astype(np.float64) @ B) + 0.25 * np.broadcast_to(C, (5, 3))
        np.testing.assert_allclose(O.gemm(A, B, C, alpha=1.5, beta=0.25), ref, atol=1e-5)


def test_fused_ffn_and_qkv_vs_float64():
    rng = np.random.default_rng(3)
    X = rng.standard_normal((9, 16)).astype(np.float32)
    W = (rng.standard_normal((16, 24)) * 0.3).astype(np.float32)
    b = rng.standard_normal(24).astype(np.float32)
    np.testing.assert_allclose(O.fused_matmul_add_gelu(X, W, b),
                               ref64.gelu_erf(X.astype(np.float64) @ W + b), atol=1e-5)
    ws = [rng.standard_normal(s).astype(np.float32) for s in [(16, 8), 8] * 3]
    q, k, v = O.fused_qkv(X, *ws)
    for o, (w, bb) in zip((q, k, v), zip(ws[0::2], ws[1::2])):
        np.testing.assert_allclose(o, X.astype(np.float64) @ w + bb, atol=1e-5)


@pytest.mark.parametrize("fill", [-1e30, float(np.finfo(np.float32).min)])
def test_attention_vs_float64_with_masks(fill):
    rng = np.random.default_rng(4)
    B, S, hd, nH = 3, 11, 8, 2
    q, k, v = (rng.standard_normal((B, S, hd * nH)).astype(np.float32) for _ in range(3))
    # key padding [B,1,1,S], one row fully masked (reference: uniform weights)
    mask = np.zeros((B, 1, 1, S), np.uint8)
    mask[0, 0, 0, 7:] = 1
    mask[2, 0, 0, :] = 1
    out = O.fused_attention(q, k, v, mask, hd, fill)
    np.testing.assert_allclose(out, ref64.attention(q, k, v, hd, mask, fill), atol=1e-5)
    # fully-masked batch row = mean of V over all keys
    np.testing.assert_allclose(out[2], np.broadcast_to(v[2].mean(0), (S, hd * nH)), atol=1e-5)
    # per-(b,h,i,j) mask
    m4 = (rng.random((B, nH, S, S)) < 0.3).astype(np.uint8)
    m4[..., 0] = 0
    np.testing.assert_allclose(O.fused_attention(q, k, v, m4, hd, fill),
                               ref64.attention(q, k, v, hd, m4, fill), atol=1e-5)


def test_layernorm_and_activations_vs_float64():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((7, 300)) * 3 + 1).astype(np.float32)
    g = rng.standard_normal(300).astype(np.float32)
    b = rng.standard_normal(300).astype(np.float32)
    for eps in (1e-12, 1e-5):
        np.testing.assert_allclose(O.layernorm(x, g, b, eps), ref64.layernorm(x, g, b, eps),
                                   atol=2e-5)
    z = np.linspace(-6, 6, 1001).astype(np.float32)
    np.testing.assert_allclose(O.gelu(z), ref64.gelu_erf(z), atol=2e-6)
    np.testing.assert_allclose(O.gelu_tanh(z), ref64.gelu_tanh(z), atol=2e-6)


def test_argmax_first_max_wins():
    x = np.array([1.0, 3.0, 2.0, 3.0, -1.0], np.float32)
    assert O.argmax(x) == 1
    assert O.argmax(np.zeros(17, np.float32)) == 0
    y = np.full(1000, -5.0, np.float32)
    y[[400, 999]] = 7.0
    assert O.argmax(y) == 400


def test_sgemv_rows_vs_float64():
    rng = np.random.default_rng(6)
    W = rng.standard_normal((33, 70)).astype(np.float32)
    x = rng.standard_normal(70).astype(np.float32)
    np.testing.assert_allclose(O.sgemv_rows(W, x), W.astype(np.float64) @ x, atol=1e-4)


# ------------------------------------------------------------ model level

def test_encoder_vs_float64_small_ragged():
    cfg = graphs.small_encoder_cfg()
    w = graphs.encoder_weights(cfg, seed=11)
    ids, mask = graphs.encoder_inputs(cfg, 3, 40, ragged=True)
    np.testing.assert_allclose(O.encoder_forward(cfg, w, ids, mask),
                               ref64.encoder(cfg, w, ids, mask), atol=1e-5)


def test_gpt2_forward_vs_float64_small():
    cfg = graphs.small_gpt2_cfg()
    w = graphs.gpt2_weights(cfg, seed=12)
    ids = graphs.gpt2_prompt(cfg, 20)
    np.testing.assert_allclose(O.gpt2_forward(cfg, w, ids), ref64.gpt2_logits(cfg, w, ids),
                               atol=1e-4)


def test_gpt2_incremental_decode_equals_full_recompute():
    """KV-cache invariant: each greedily generated token equals the argmax of
    a full-sequence forward over prompt + tokens so far."""
    cfg = graphs.small_gpt2_cfg()
    w = graphs.gpt2_weights(cfg, seed=13)
    prompt = graphs.gpt2_prompt(cfg, 8)
    toks, last_logits, margins = O.gpt2_generate(cfg, w, prompt, 12)
    seq = list(prompt)
    for t in toks:
        logits = O.gpt2_forward(cfg, w, np.array(seq, np.int64))[-1]
        assert O.argmax(logits) == t
        seq.append(int(t))
    full = O.gpt2_forward(cfg, w, np.array(seq[:-1], np.int64))[-1]
    np.testing.assert_allclose(last_logits, full, atol=1e-4)
    assert np.all(margins >= 0)


# ------------------------------------------------- planted mistakes (CPU)

def test_planted_mistakes_are_caught():
    """Plausible bugs planted in copies of oracle outputs fail the checks
    above: a transposed operand, a dropped bias, a swapped nibble order and
    a missing 1/sqrt(d) scale."""
    rng = np.random.default_rng(7)
    A = rng.standard_normal((6, 6)).astype(np.float32)
    B = rng.standard_normal((6, 6)).astype(np.float32)
    good = A.astype(np.float64) @ B
    assert not np.allclose(O.sgemm(A, B, False, True), good, atol=1e-4)  # transposed B
    b = rng.standard_normal(6).astype(np.float32)
    assert not np.allclose(O.gemm(A, B, None), good + b, atol=1e-4)       # dropped bias
    g, N, K, W, x, scales = _int4_fixture()
    swapped = ((W & 0xF) << 4 | (W >> 4)).astype(np.uint8)                # nibble order
    assert not np.array_equal(O.int4_unpack(swapped, scales, K), ref64.int4_deq(W, scales, K))
    q = rng.standard_normal((1, 5, 8)).astype(np.float32)
    unscaled = O.fused_attention(q * math.sqrt(8), q, q, None, 8, -1e30)  # scale dropped
    assert not np.allclose(unscaled, ref64.attention(q, q, q, 8), atol=1e-4)
