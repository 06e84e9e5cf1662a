"""The transformer-block training plan (config 5's graph) run by the
launch-plan executor on the GPU, against the same block differentiated by
torch autograd on the CPU in float64 (a floating-point reference of the
whole graph; every operator in it is also checked alone against the
oracle).  fp32 bar: 1e-4 relative max-norm on the forward output, the loss
and every gradient."""
import numpy as np
import pytest

import bwpp
from bwpp import plan, synth
from conftest import rel_max_err

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _inputs(B, T, D, F, seed):
    w = lambda shape, st: synth.normal(shape, seed, st, 0.0, 0.02)
    return {
        "x": synth.normal((B * T, D), seed, 0),
        "g1": synth.uniform((D,), seed, 1, 0.5, 1.5),
        "wqkv": w((D, 3 * D), 2),
        "wo": w((D, D), 3),
        "g2": synth.uniform((D,), seed, 4, 0.5, 1.5),
        "w1": w((D, F), 5),
        "w2": w((F, D), 6),
    }


def _reference(t, B, T, D, H, F):
    import torch
    p = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True) for k, v in t.items()}
    rms = lambda a, g: a / torch.sqrt((a * a).mean(dim=1, keepdim=True) + 1e-5) * g
    n1 = rms(p["x"], p["g1"])
    qkv = n1 @ p["wqkv"]
    dh = D // H

    def heads(m):
        return m.reshape(B, T, H, dh).permute(0, 2, 1, 3)

    q, k, v = heads(qkv[:, :D]), heads(qkv[:, D:2 * D]), heads(qkv[:, 2 * D:])
    s = (q @ k.transpose(-1, -2)) * 0.125
    mask = torch.ones(T, T, dtype=torch.bool).tril()
    s = s.masked_fill(~mask, float("-inf"))
    att = (torch.softmax(s, dim=-1) @ v).permute(0, 2, 1, 3).reshape(B * T, D)
    x1 = p["x"] + att @ p["wo"]
    z = rms(x1, p["g2"]) @ p["w1"]
    out = x1 + torch.nn.functional.silu(z) @ p["w2"]
    loss = (out * out).mean()
    loss.backward()
    grads = {f"d{k}": p[k].grad.numpy() for k in ("x", "g1", "wqkv", "wo", "g2", "w1", "w2")}
    return out.detach().numpy(), float(loss.detach()), grads


@pytest.mark.parametrize("B,T,D,H,F", [(2, 64, 128, 2, 256), (1, 100, 192, 3, 384)])
def test_transformer_block_train_plan(be, B, T, D, H, F):
    import torch
    t = _inputs(B, T, D, F, seed=B * 1000 + T)
    p = plan.Plan(be, plan.load_text("transformer_block_train", B=B, T=T, D=D, H=H, F=F))
    p.allocate()
    dev = {k: torch.from_numpy(v).cuda() for k, v in t.items()}
    for k, v in dev.items():
        p.bind(k, v)
    p.run()
    out = p.host("out", (B * T, D))
    loss = float(p.host("loss", (1,))[0])
    ref_out, ref_loss, ref_g = _reference(t, B, T, D, H, F)
    assert rel_max_err(out, ref_out) <= TOL
    assert abs(loss - ref_loss) <= TOL * abs(ref_loss)
    shapes = {"dx": (B * T, D), "dg1": (D,), "dwqkv": (D, 3 * D), "dwo": (D, D), "dg2": (D,),
              "dw1": (D, F), "dw2": (F, D)}
    for name, shape in shapes.items():
        got = p.host(name, shape)
        assert rel_max_err(got, ref_g[name]) <= TOL, name
    # A second run over the same arena gives the same result.
    p.run()
    assert rel_max_err(p.host("dwqkv", shapes["dwqkv"]), ref_g["dwqkv"]) <= TOL
    p.close()


def test_plan_unbound_input_is_an_error(be):
    p = plan.Plan(be, plan.load_text("transformer_block_train", B=1, T=8, D=64, H=1, F=64))
    p.allocate()
    with pytest.raises(plan.PlanError) as e:
        p.run()
    assert "not bound" in str(e.value)
    p.close()
