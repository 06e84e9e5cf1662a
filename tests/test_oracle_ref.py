"""Oracle restatement vs the reference's bwpp_cpu_ref.c compiled unchanged
(oracle/_ref): bit-identical on random shapes, strides and special values.
Skipped where oracle/_ref was not built."""
import numpy as np
import pytest

from conftest import assert_bits_equal

SHAPES = [(1, 1), (3, 7), (16, 64), (33, 129), (5, 1000)]


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (4, 4, 4), (13, 31, 7), (37, 53, 61), (64, 96, 128)])
@pytest.mark.parametrize("silu,add", [(0, 0), (1, 1), (0, 1), (1, 0)])
def test_matmul_vs_ref(oracle, ref, M, N, K, silu, add):
    rng = np.random.default_rng(M * 1000 + N * 10 + K)
    a = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    b = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    bias = rng.uniform(-1, 1, N).astype(np.float32)
    assert_bits_equal(oracle.matmul(a, b, bias, silu, add), ref.matmul(a, b, bias, silu, add))


def test_matmul_strided_vs_ref(oracle, ref):
    rng = np.random.default_rng(7)
    A = rng.normal(size=(20, 40)).astype(np.float32)
    B = rng.normal(size=(30, 50)).astype(np.float32)
    a, b = A[:, :25], B[:25, :33]
    assert_bits_equal(oracle.matmul(a, b), ref.matmul(a, b))


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_softmax_rmsnorm_vs_ref(oracle, ref, rows, cols):
    rng = np.random.default_rng(rows * 7919 + cols)
    x = rng.normal(0, 3, (rows, cols)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    b = rng.normal(0, 0.1, cols).astype(np.float32)
    assert_bits_equal(oracle.softmax(x), ref.softmax(x), "softmax")
    for gg, bb in ((None, None), (g, None), (g, b), (None, b)):
        assert_bits_equal(oracle.rmsnorm(x, gg, bb, 1e-6), ref.rmsnorm(x, gg, bb, 1e-6), "rmsnorm")


def test_strided_rows_vs_ref(oracle, ref):
    rng = np.random.default_rng(3)
    X = rng.normal(size=(9, 70)).astype(np.float32)
    x = X[:, :61]
    assert_bits_equal(oracle.softmax(x), ref.softmax(x))
    assert_bits_equal(oracle.rmsnorm(x, None, None, 1e-5), ref.rmsnorm(x, None, None, 1e-5))


@pytest.mark.parametrize("M,N,K,D", [(1, 1, 1, 1), (2, 3, 4, 5), (17, 33, 16, 8), (64, 80, 32, 48)])
def test_attention_vs_ref(oracle, ref, M, N, K, D):
    rng = np.random.default_rng(M + N + K + D)
    q = rng.normal(size=(M, K)).astype(np.float32)
    k = rng.normal(size=(N, K)).astype(np.float32)
    v = rng.normal(size=(N, D)).astype(np.float32)
    assert_bits_equal(oracle.attention(q, k, v), ref.attention(q, k, v))


@pytest.mark.parametrize("axis", [0, 1])
def test_reduce_max_mask_grad_vs_ref(oracle, ref, axis):
    rng = np.random.default_rng(11 + axis)
    x = rng.integers(-3, 3, (23, 17)).astype(np.float32)
    x[4] = np.nan
    x[:, 5] = -np.inf
    x[7, 3] = np.inf
    dy = rng.normal(size=17 if axis == 0 else 23).astype(np.float32)
    m = oracle.reduce_max_mask(x, axis)
    assert_bits_equal(m, ref.reduce_max_mask(x, axis))
    assert_bits_equal(oracle.reduce_max_grad_mask(m, dy, axis), ref.reduce_max_grad_mask(m, dy, axis))


def test_softmax_special_values_vs_ref(oracle, ref):
    x = np.array([[np.inf, np.inf, 1], [np.nan, np.nan, np.nan], [-np.inf, 0, np.inf],
                  [1e30, -1e30, 0], [-0.0, 0.0, -0.0]], np.float32)
    assert_bits_equal(oracle.softmax(x), ref.softmax(x))
    assert_bits_equal(oracle.rmsnorm(x, None, None, 1e-5), ref.rmsnorm(x, None, None, 1e-5))
