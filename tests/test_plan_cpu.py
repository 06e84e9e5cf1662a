"""The CPU plan executor (oracle/plan_cpu.py), which checks plans run on the
GPU and times config 5's CPU baseline: it must reproduce float64 autograd of
the same block (a textbook reference of the whole graph), and the oracle's
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


def _block_inputs(B, T, D, F, seed):
    from bwpp import synth
    w = lambda shape, st: synth.normal(shape, seed, st, 0.0, 0.02)
    return {"x": synth.normal((B * T, D), seed, 0), "g1": synth.uniform((D,), seed, 1, 0.5, 1.5),
            "wqkv": w((D, 3 * D), 2), "wo": w((D, D), 3), "g2": synth.uniform((D,), seed, 4, 0.5, 1.5),
            "w1": w((D, F), 5), "w2": w((F, D), 6)}


def _torch_block(t, B, T, D, H, F):
    import torch
    p = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True) for k, v in t.items()}
    rms = lambda a, g: a / torch.sqrt((a * a).mean(dim=1, keepdim=True) + 1e-5) * g
    n1 = rms(p["x"], p["g1"])
    qkv = n1 @ p["wqkv"]
    dh = D // H
    heads = lambda m: m.reshape(B, T, H, dh).permute(0, 2, 1, 3)
    q, k, v = heads(qkv[:, :D]), heads(qkv[:, D:2 * D]), heads(qkv[:, 2 * D:])
    s = (q @ k.transpose(-1, -2)) * (dh ** -0.5)
    s = s.masked_fill(~torch.ones(T, T, dtype=torch.bool).tril(), float("-inf"))
    att = (torch.softmax(s, dim=-1) @ v).permute(0, 2, 1, 3).reshape(B * T, D)
    x1 = p["x"] + att @ p["wo"]
    out = x1 + torch.nn.functional.silu(rms(x1, p["g2"]) @ p["w1"]) @ p["w2"]
    loss = (out * out).mean()
    loss.backward()
    return out.detach().numpy(), float(loss.detach()), {f"d{k}": p[k].grad.numpy() for k in t}


@pytest.mark.parametrize("B,T,D,H,F", [(2, 16, 64, 1, 128), (1, 40, 96, 3, 192)])
def test_cpu_plan_matches_float64_autograd(B, T, D, H, F):
    text = plan.load_text("transformer_block_train", B=B, T=T, D=D, H=H, F=F)
    text = text.replace("scale=0.125", f"scale={(D // H) ** -0.5!r}")
    t = _block_inputs(B, T, D, F, seed=T)
    cp = CpuPlan(text)
    for k, v in t.items():
        cp.bind(k, v)
    cp.run()
    out, loss, grads = _torch_block(t, B, T, D, H, F)
    assert rel_max_err(cp.get("out"), out) <= 1e-5
    assert abs(float(cp.get("loss")[0, 0]) - loss) <= 1e-5 * abs(loss)
    for name, want in grads.items():
        assert rel_max_err(cp.get(name).reshape(want.shape), want) <= 1e-5, name


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
