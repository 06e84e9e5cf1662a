"""Config 5's block (examples/tiny_model.bwpp `block`: rmsnorm -> q, k, v
projections -> causal multi-head attention -> out-projection + residual ->
rmsnorm -> SiLU MLP + residual) trained on loss = mean(out^2): synthetic
inputs from the repo's generator and a float64 torch autograd reference of
the same program, for checking the lowered plan (plans/block_train.plan)."""
import numpy as np

from bwpp import synth

PARAMS = ("x", "g1", "g2", "wq", "wk", "wv", "wo", "w1", "w2")


def block_inputs(batch, T, D, H, seed):
    """x ~ N(0,1) [batch*T, D], gamma ~ U[0.5,1.5], weights ~ N(0, 0.02);
    H is the MLP width (the DSL's name)."""
    w = lambda shape, st: synth.normal(shape, seed, st, 0.0, 0.02)
    return {"x": synth.normal((batch * T, D), seed, 0), "g1": synth.uniform((D,), seed, 1, 0.5, 1.5),
            "g2": synth.uniform((D,), seed, 2, 0.5, 1.5), "wq": w((D, D), 3), "wk": w((D, D), 4),
            "wv": w((D, D), 5), "wo": w((D, D), 6), "w1": w((D, H), 7), "w2": w((H, D), 8)}


def block_reference(t, batch, T, D, H, heads, eps=1e-5):
    """(out, loss, grads) in float64 on the CPU; grads keyed d<name>."""
    import torch
    p = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True) for k, v in t.items()}
    rms = lambda a, g: a / torch.sqrt((a * a).mean(dim=1, keepdim=True) + eps) * g
    n1 = rms(p["x"], p["g1"])
    dh = D // heads
    split = lambda m: m.reshape(batch, T, heads, dh).permute(0, 2, 1, 3)
    q, k, v = split(n1 @ p["wq"]), split(n1 @ p["wk"]), split(n1 @ p["wv"])
    s = (q @ k.transpose(-1, -2)) * (dh ** -0.5)
    s = s.masked_fill(~torch.ones(T, T, dtype=torch.bool).tril(), float("-inf"))
    ctx = (torch.softmax(s, dim=-1) @ v).permute(0, 2, 1, 3).reshape(batch * T, D)
    x1 = p["x"] + ctx @ p["wo"]
    out = x1 + torch.nn.functional.silu(rms(x1, p["g2"]) @ p["w1"]) @ p["w2"]
    loss = (out * out).mean()
    loss.backward()
    return out.detach().numpy(), float(loss.detach()), {f"d{k}": p[k].grad.numpy() for k in PARAMS}


def grad_shapes(batch, T, D, H):
    return {"dx": (batch * T, D), "dg1": (D,), "dg2": (D,), "dwq": (D, D), "dwk": (D, D), "dwv": (D, D),
            "dwo": (D, D), "dw1": (D, H), "dw2": (H, D)}
