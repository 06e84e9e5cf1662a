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


@pytest.mark.parametrize("B,T,D,H,F", [(2, 64, 128, 2, 256), (1, 100, 192, 3, 384),
                                       (8, 512, 1024, 16, 4096)])
def test_transformer_block_train_plan(be, B, T, D, H, F):
    """The last case is config 5 at full size (the step the bench times):
    there split-K runs on the K = 4096 weight-gradient GEMMs and attention
    over 128 (batch, head) slices."""
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


def test_bf16_projection_attention_plan(be, oracle):
    """A bf16 plan: qkv = x W (bf16 GEMM), causal attention on its column
    views with the lse saved; against the oracle on the exact bf16 values
    (qkv rounded to bf16 as the GEMM stores it).  Bar 2e-2."""
    import torch
    B, T, H, dh = 2, 96, 2, 128
    D = H * dh
    text = f"""bwpp.plan 1
dim BT {B * T}
dim D {D}
dim D3 {3 * D}
value x bf16 [BT,D] input
value w bf16 [D,D3] param
value qkv bf16 [BT,D3] temp
op matmul out=qkv in=x,w
view q of=qkv offset=0 ld=D3 shape=[BT,D]
view k of=qkv offset=D ld=D3 shape=[BT,D]
view v of=qkv offset=2*D ld=D3 shape=[BT,D]
value o bf16 [BT,D] output
value lse f32 [{B},{H},{T}] output
op attention out=o,lse in=q,k,v batch={B} heads={H} causal=1 scale=0.125
"""
    x = synth.normal((B * T, D), 3, 0)
    w = synth.normal((D, 3 * D), 3, 1, 0.0, 0.05)
    xb, wb = synth.to_bf16_bits(x), synth.to_bf16_bits(w)
    p = plan.Plan(be, text)
    p.allocate()
    xd = torch.from_numpy(xb.view(np.int16)).cuda()
    wd = torch.from_numpy(wb.view(np.int16)).cuda()
    p.bind("x", xd)
    p.bind("w", wd)
    p.run()
    o = synth.bf16_bits_to_f32(p.host("o", (B * T, D), np.uint16))
    lse = p.host("lse", (B, H, T))
    qkv = synth.bf16_bits_to_f32(synth.to_bf16_bits(oracle.matmul(synth.bf16_bits_to_f32(xb),
                                                                  synth.bf16_bits_to_f32(wb))))
    heads = lambda part: np.ascontiguousarray(
        qkv[:, part * D:(part + 1) * D].reshape(B, T, H, dh).transpose(0, 2, 1, 3))
    q, k, v = heads(0), heads(1), heads(2)
    want = oracle.attention_bh(q, k, v, 0.125, True).transpose(0, 2, 1, 3).reshape(B * T, D)
    assert rel_max_err(o, want) <= 2e-2
    wl = oracle.attention_lse(q, k, 0.125, True)
    assert np.max(np.abs(lse - wl)) <= 2e-2 * max(1.0, np.abs(wl).max())
    p.close()
