"""The host int4 quantiser behind inferc_gpt2_use_int4 (no GPU): per-row
symmetric scale s_r = max|w_r| / 7, q = clamp(rint(w / s_r), -8, 7), packed
two per byte in the reference's layout (bench/amx/int4_gemv_amx.cc:249-250,
264-267: low nibble = even k, nibble = q + 8)."""
from __future__ import annotations

import numpy as np
import pytest

from inferc_amd import graphs, rt


def _weights(seed: int, N: int, K: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w[1] = 0.0                                     # all-zero row
    w[2] *= np.float32(1e-30)                      # tiny magnitudes
    w[3] *= np.float32(1e30)                       # huge magnitudes
    w[4, ::2] = np.float32(0.5)                    # exact half steps of the scale
    w[4, 1::2] = np.float32(-3.5)
    return w


@pytest.mark.parametrize("N,K", [(8, 2), (9, 64), (33, 768)])
def test_quantize_matches_numpy_statement(N, K):
    w = _weights(N * 7 + K, N, K)
    packed, s, deq = rt.int4_quantize_rows(w)
    q, s_ref = graphs.int4_quantize_rows_np(w)
    np.testing.assert_array_equal(s, s_ref)
    nib = (q.astype(np.int16) + 8).astype(np.uint8)
    np.testing.assert_array_equal(packed, nib[:, 0::2] | (nib[:, 1::2] << 4))
    np.testing.assert_array_equal(deq, (s_ref[:, None] * q.astype(np.float32)).astype(np.float32))


def test_quantize_error_and_range_properties():
    w = _weights(5, 16, 128)
    packed, s, deq = rt.int4_quantize_rows(w)
    lo, hi = (packed & 15).astype(np.int16) - 8, (packed >> 4).astype(np.int16) - 8
    q = np.empty(w.shape, np.int16)
    q[:, 0::2], q[:, 1::2] = lo, hi
    # symmetric: -8 is never produced, the largest magnitude maps to +-7
    assert q.min() >= -7 and q.max() <= 7
    for r in range(w.shape[0]):
        if s[r] > 0:
            assert np.abs(q[r]).max() == 7
    # rounding to nearest: |w - s q| <= s/2 (plus the rounding of w / s)
    err = np.abs(w.astype(np.float64) - s[:, None].astype(np.float64) * q)
    assert np.all(err <= s[:, None].astype(np.float64) * (0.5 + 1e-6))
    assert np.all(deq[1] == 0) and s[1] == 0


def test_quantize_planted_nibble_swap_is_caught():
    """A packing with the nibble order swapped (odd k in the low nibble)
    must not pass the equality above."""
    w = _weights(11, 6, 16)
    packed, _, _ = rt.int4_quantize_rows(w)
    q, _ = graphs.int4_quantize_rows_np(w)
    nib = (q.astype(np.int16) + 8).astype(np.uint8)
    swapped = nib[:, 1::2] | (nib[:, 0::2] << 4)
    assert not np.array_equal(packed, swapped)


def test_quantize_rejects_odd_k():
    with pytest.raises(RuntimeError, match="K must be even"):
        rt.int4_quantize_rows(np.zeros((2, 3), np.float32))
