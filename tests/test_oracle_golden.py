"""The oracle reproduces the reference's outputs bit for bit.

Golden vectors come from the reference's runtime/cpu/bwpp_cpu_ref.c compiled
as is (tests/golden/make_golden.py); the fixtures include the reference
tests' own ramp inputs.  Also the reference tests' known answers and
invariants (runtime/cpu/test_matmul.c, test_norm.c, test_reduce_max.c).
"""
import numpy as np
import pytest

from conftest import assert_bits_equal


def cases(golden, prefix):
    names = sorted({k.split("/")[0] for k in golden if k.startswith(prefix)})
    assert names, prefix
    return names


def test_matmul_golden(golden, oracle):
    for name in cases(golden, "matmul_"):
        g = lambda k: golden[f"{name}/{k}"]
        c = oracle.matmul(g("a"), g("b"), g("bias"), apply_silu=bool(g("silu")),
                          apply_bias=bool(g("add")))
        assert_bits_equal(c, g("c"), name)


def test_softmax_golden(golden, oracle):
    for name in ("softmax_ramp", "softmax_seed", "softmax_special"):
        assert_bits_equal(oracle.softmax(golden[f"{name}/x"]), golden[f"{name}/y"], name)
    xf = golden["softmax_ld/xfull"]
    cols = int(golden["softmax_ld/cols"])
    y = oracle.softmax(xf[:, :cols])
    assert_bits_equal(y, golden["softmax_ld/yfull"][:, :cols], "softmax_ld")


def test_rmsnorm_golden(golden, oracle):
    for name in cases(golden, "rmsnorm_"):
        g = lambda k: golden.get(f"{name}/{k}")
        y = oracle.rmsnorm(g("x"), g("gamma"), g("beta"), float(g("eps")))
        assert_bits_equal(y, g("y"), name)


def test_attention_golden(golden, oracle):
    for name in cases(golden, "attention_"):
        g = lambda k: golden[f"{name}/{k}"]
        assert_bits_equal(oracle.attention(g("q"), g("k"), g("v")), g("o"), name)
        # batched restatement at scale 1, unmasked, is the same function
        q, k, v = (g(t)[None, None] for t in "qkv")
        assert_bits_equal(oracle.attention_bh(q, k, v, 1.0, False)[0, 0], g("o"), name + "_bh")


def test_reduce_max_mask_grad_golden(golden, oracle):
    for name in cases(golden, "rmax_"):
        g = lambda k: golden[f"{name}/{k}"]
        axis = 0 if name.endswith("axis0") else 1
        m = oracle.reduce_max_mask(g("x"), axis)
        assert_bits_equal(m, g("mask"), name + "/mask")
        assert_bits_equal(oracle.reduce_max_grad_mask(m, g("dy"), axis), g("dx"), name + "/dx")


def _ramp(rows, cols, scale):
    i = np.arange(rows * cols, dtype=np.uint32) + np.uint32(1)
    return (i.astype(np.float32) * np.float32(scale)).reshape(rows, cols)


@pytest.mark.parametrize("ep_add,ep_silu,expect", [(0, 0, "24.720001"), (1, 1, "21.514381")])
def test_matmul_checksum_known_answer(oracle, ep_add, ep_silu, expect):
    """runtime/cpu/test_matmul.c:76-101 prints these checksums for
    examples/matmul.bwpp and examples/matmul_add_silu.bwpp."""
    a = _ramp(4, 4, 0.1)
    b = _ramp(4, 4, 0.05)
    bias = np.array([0.01 * (i + 1) if ep_add else 0.0 for i in range(4)], np.float32)
    c = oracle.matmul(a, b, bias, apply_silu=bool(ep_silu), apply_bias=bool(ep_add))
    s = np.float32(0.0)
    for v in c.ravel():
        s = np.float32(s + v)
    assert f"{float(s):.6f}" == expect


def test_norm_invariants(oracle):
    """runtime/cpu/test_norm.c:37,51: softmax rows sum to 1 (1e-3); RMSNorm
    with gamma = 1 has unit RMS (1e-2)."""
    x = _ramp(2, 4, 0.1)
    y = oracle.softmax(x)
    assert np.all(np.abs(y.sum(axis=1) - 1.0) <= 1e-3)
    z = oracle.rmsnorm(x, np.ones(4, np.float32), None, 1e-5)
    assert np.all(np.abs(np.sqrt((z.astype(np.float64) ** 2).mean(axis=1)) - 1.0) <= 1e-2)


def test_reduce_max_known_answer(oracle):
    """runtime/cpu/test_reduce_max.c:13-55: x[r][c] = r*cols + c, axis 1 ->
    one-hot at the last column; grad dy[r] = r + 1 routed there."""
    x = np.arange(6, dtype=np.float32).reshape(2, 3)
    m = oracle.reduce_max_mask(x, 1)
    assert np.array_equal(m, np.array([[0, 0, 1], [0, 0, 1]], np.float32))
    dx = oracle.reduce_max_grad_mask(m, np.array([1, 2], np.float32), 1)
    assert np.array_equal(dx, np.array([[0, 0, 1], [0, 0, 2]], np.float32))
