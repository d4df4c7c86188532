"""Pins of the oracle's layer arithmetic (linear_forward, lora_h, DoRA calibration).

Each check is independent of the formula it tests: brute-force loops with exact
(math.fsum) sums, one-hot activations, hand-built inputs whose single and double
roundings differ, and closed-form hand matrices.  A dropped DoRA term, a
transposed operand, a wrong rounding point or a wrong norm axis fails one of them.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import wlq_oracle as O


def _f16(a):
    return np.asarray(a, dtype=np.float16)


def _brute(x, W0, H=None, B=None, gamma=None, s=1.0, double_round=False):
    """Explicit loops, exact sums (math.fsum), one rounding at each reference point."""
    M, K = x.shape
    N = W0.shape[0]
    y = np.empty((M, N), dtype=np.float16)
    for i in range(M):
        for n in range(N):
            acc = math.fsum(float(x[i, k]) * float(W0[n, k]) for k in range(K))
            if H is not None:
                if double_round:
                    acc = float(np.float16(acc))
                lo = math.fsum(float(H[i, j]) * float(B[n, j]) for j in range(B.shape[1]))
                acc = (acc + s * lo) * float(gamma[n])
            y[i, n] = np.float16(acc)
    return y


@pytest.mark.parametrize("M", [1, 3, 16, 17])
def test_linear_forward_matches_loops(M):
    rng = np.random.default_rng(M)
    N, K, r = 5, 7, 3
    x = _f16(rng.standard_normal((M, K)))
    W0 = _f16(rng.standard_normal((N, K)) * 0.1)
    A = _f16(rng.standard_normal((r, K)) * 0.1)
    B = _f16(rng.standard_normal((N, r)) * 0.1)
    g = _f16(rng.uniform(0.9, 1.1, N))
    H = O.lora_h(x, A)
    y = O.linear_forward(x, W0, H, B, g, s=0.5)
    ref = _brute(x, W0, H, B, g, s=0.5, double_round=M >= 16)
    # fp64 accumulation vs exact fsum: equal except for a last-bit tie, which these inputs avoid
    assert np.array_equal(y.view(np.uint16), ref.view(np.uint16))
    # without DoRA: fp16(x W0^T) for every M
    assert np.array_equal(O.linear_forward(x, W0).view(np.uint16), _brute(x, W0).view(np.uint16))


def test_one_hot_rows_return_weight_columns():
    rng = np.random.default_rng(1)
    N, K = 6, 9
    W0 = _f16(rng.standard_normal((N, K)))
    x = np.eye(K, dtype=np.float16)
    y = O.linear_forward(x, W0)
    assert np.array_equal(y.view(np.uint16), W0.T.copy().view(np.uint16))


def test_rounding_points_single_vs_double():
    # x . W0 = 1 + 2^-11 + 2^-13 exactly; DoRA term -2^-12; gamma 1.
    # single rounding: fp16(1 + 2^-11 - 2^-13) = 1;  double: fp16(fp16(...) - 2^-12) = 1 + 2^-10
    W0 = _f16([[1.0, 2.0 ** -11, 2.0 ** -13]])
    B = _f16([[-(2.0 ** -12)]])
    g = _f16([1.0])
    for M, expect in ((1, 1.0), (15, 1.0), (16, 1.0 + 2.0 ** -10), (40, 1.0 + 2.0 ** -10)):
        x = np.ones((M, 3), dtype=np.float16)
        H = np.ones((M, 1), dtype=np.float32)
        y = O.linear_forward(x, W0, H, B, g, s=1.0)
        assert np.all(y.astype(np.float64) == expect), (M, y[0])
    # forcing the rounding point overrides the M rule
    x = np.ones((1, 3), dtype=np.float16)
    y = O.linear_forward(x, W0, np.ones((1, 1), np.float32), B, g, round_gemm_output=True)
    assert float(y[0, 0]) == 1.0 + 2.0 ** -10


def test_zero_adapter_equals_plain_product():
    rng = np.random.default_rng(2)
    for M in (1, 20):
        x = _f16(rng.standard_normal((M, 8)))
        W0 = _f16(rng.standard_normal((4, 8)))
        H = rng.standard_normal((M, 2)).astype(np.float32)
        y0 = O.linear_forward(x, W0)
        y1 = O.linear_forward(x, W0, H, np.zeros((4, 2), np.float16), np.ones(4, np.float16))
        assert np.array_equal(y0.view(np.uint16), y1.view(np.uint16))
        # r = 0 disables the epilogue even with gamma != 1
        y2 = O.linear_forward(x, W0, np.zeros((M, 0), np.float32), np.zeros((4, 0), np.float16),
                              np.full(4, 2.0, np.float16))
        assert np.array_equal(y0.view(np.uint16), y2.view(np.uint16))


def test_linearity_in_x():
    # small integers: every sum below is exact in fp16 and fp64
    rng = np.random.default_rng(3)
    x1 = _f16(rng.integers(-3, 4, (2, 6)))
    x2 = _f16(rng.integers(-3, 4, (2, 6)))
    W0 = _f16(rng.integers(-4, 5, (3, 6)) / 8.0)
    y1 = O.linear_forward(x1, W0, return_f64=True)
    y2 = O.linear_forward(x2, W0, return_f64=True)
    y12 = O.linear_forward(_f16(x1.astype(np.float32) + x2.astype(np.float32)), W0, return_f64=True)
    assert np.array_equal(y12, y1 + y2)


def test_lora_h_rounds_exact_sum_to_fp16():
    # x . A^T = 1 + 2^-11 + 2^-20 exactly -> fp16 rounds up to 1 + 2^-10 (above the tie)
    x = _f16([[1.0, 1.0, 1.0]])
    A = _f16([[1.0, 2.0 ** -11, 2.0 ** -20]])
    H = O.lora_h(x, A)
    assert H.dtype == np.float32 and float(H[0, 0]) == 1.0 + 2.0 ** -10
    # a transposed operand would change the shape
    A2 = _f16(np.arange(6).reshape(2, 3))
    assert O.lora_h(_f16(np.ones((4, 3))), A2).shape == (4, 2)


def test_dora_gamma_hand_cases():
    W0 = _f16([[3.0, 4.0], [0.0, 2.0]])
    A = np.zeros((1, 2))
    B = np.zeros((2, 1))
    # m defaults to ||W0||_row: gamma = 1 with a zero adapter
    assert np.all(O.dora_gamma(W0, A, B, 1.0) == np.float16(1.0))
    # m given: gamma = m / ||W0||
    assert list(O.dora_gamma(W0, A, B, 1.0, m=np.array([10.0, 1.0])).astype(float)) == [2.0, 0.5]
    # V = W0 + s B A: row 0 = [3, 0] + [0, 4] -> norm 5; m = ||W0 row|| = 3 -> 0.6
    W1 = _f16([[3.0, 0.0]])
    g = O.dora_gamma(W1, np.array([[0.0, 1.0]]), np.array([[2.0]]), 2.0)
    assert g[0] == np.float16(0.6)
    # a zero row: the norm floor 1e-12 keeps gamma finite (0 / 1e-12 = 0)
    g0 = O.dora_gamma(_f16([[0.0, 0.0]]), np.zeros((1, 2)), np.zeros((1, 1)), 1.0)
    assert g0[0] == 0.0


def test_merge_dora_block_diagonal():
    A1, A2 = np.ones((2, 5)), 2 * np.ones((3, 5))
    B1, B2 = np.full((4, 2), 3.0), np.full((6, 3), 4.0)
    A, B, m = O.merge_dora([A1, A2], [B1, B2], [np.ones(4), np.ones(6)])
    assert A.shape == (5, 5) and np.array_equal(A[:2], A1) and np.array_equal(A[2:], A2)
    assert B.shape == (10, 5)
    assert np.all(B[:4, :2] == 3) and np.all(B[4:, 2:] == 4) and np.all(B[:4, 2:] == 0) and np.all(B[4:, :2] == 0)
    assert m.shape == (10,)
    # B A of the merge = the stacked per-projection products
    assert np.array_equal(B @ A, np.concatenate([B1 @ A1, B2 @ A2]))
    assert O.merge_dora([A1, A2], [B1, B2], [np.ones(4), None])[2] is None


def test_lora_scale():
    assert O.lora_scale(None, 16) == 1.0
    assert O.lora_scale(32, 16) == 2.0
    assert O.lora_scale(8.0, 16) == 0.5


def test_apply_bias_dtype_and_shape():
    rng = np.random.default_rng(4)
    W0 = _f16(rng.standard_normal((3, 4)))
    x = rng.standard_normal((2, 5, 4)).astype(np.float32)
    bias = np.array([1.0, -2.0, 0.5], np.float32)
    y = O.apply(x, W0, bias=bias, out_dtype=np.float32)
    assert y.shape == (2, 5, 3) and y.dtype == np.float32
    ref = O.linear_forward(x.reshape(-1, 4).astype(np.float16), W0).astype(np.float32) + bias
    assert np.array_equal(y.reshape(-1, 3), ref)
