"""The CPU plan executor (oracle/plan_cpu.py), which checks plans run on the
GPU and times config 5's CPU baseline: it must reproduce float64 autograd of
the block the plan was lowered from (a textbook reference of the whole
graph), and the oracle's
transposed-operand matmuls it relies on must be bit-identical to the plain
matmul on explicitly transposed copies (the reordered loops keep each
output's k-order fp32 sum)."""
import numpy as np
import pytest

from bwpp import plan
from conftest import rel_max_err
from oracle.plan_cpu import CpuPlan, PlanTextError


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("M,N,K", [(37, 29, 53), (5, 130, 7), (1, 1, 1)])
def test_transposed_matmul_bit_identical(oracle, ta, tb, M, N, K):
    rng = np.random.default_rng(M * 100 + N)
    a = rng.normal(size=(M, K)).astype(np.float32)
    b = rng.normal(size=(K, N)).astype(np.float32)
    bias = rng.normal(size=N).astype(np.float32)
    want = oracle.matmul(a, b, bias, apply_silu=True, apply_bias=True)
    A = np.ascontiguousarray(a.T) if ta else a
    B = np.ascontiguousarray(b.T) if tb else b
    got = oracle.matmul(A, B, bias, apply_silu=True, apply_bias=True, trans_a=ta, trans_b=tb)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("BATCH,T,D,H,HEADS", [(2, 16, 64, 128, 1), (1, 40, 96, 192, 3)])
def test_cpu_plan_matches_float64_autograd(BATCH, T, D, H, HEADS):
    """The lowered training plan of tiny_model's block, run op by op on the
    oracle, against float64 autograd of the same program."""
    from blockref import block_inputs, block_reference, grad_shapes
    text = plan.load_text("block_train", BATCH=BATCH, T=T, D=D, H=H, HEADS=HEADS)
    t = block_inputs(BATCH, T, D, H, seed=T)
    cp = CpuPlan(text)
    for k, v in t.items():
        cp.bind(k, v)
    cp.run()
    out, loss, grads = block_reference(t, BATCH, T, D, H, HEADS)
    assert rel_max_err(cp.get("out"), out) <= 1e-5
    assert abs(float(cp.get("loss")[0, 0]) - loss) <= 1e-5 * abs(loss)
    for name, shape in grad_shapes(BATCH, T, D, H).items():
        assert rel_max_err(cp.get(name).reshape(shape), grads[name]) <= 1e-5, name


def test_cpu_plan_rejects_bad_text():
    with pytest.raises(PlanTextError):
        CpuPlan("bwpp.plan 2\n")
    with pytest.raises(PlanTextError):
        CpuPlan("bwpp.plan 1\nvalue x f32 [Q] input\n")
    cp = CpuPlan("bwpp.plan 1\ndim N 4\nvalue x f32 [N] input\nvalue y f32 [N] output\nop silu out=y in=x\n")
    with pytest.raises(PlanTextError):
        cp.bind("x", np.zeros(3, np.float32))
    with pytest.raises(PlanTextError):
        cp.bind("y", np.zeros(4, np.float32))
