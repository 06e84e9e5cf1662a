"""Plans lowered by bwppc-hip from the reference's examples, run by the
launch-plan executor on the GPU.  Config 5's block (tiny_model's `block`
and its DSL autodiff) against float64 autograd of the same program and the
oracle; the rank-4 attention program in bf16 and config 3 as a DSL program
against the oracle.  fp32 bar: 1e-4 relative max-norm on the forward
output, the loss and every gradient; bf16 inputs: 2e-2."""
import numpy as np
import pytest

import bwpp
from bwpp import plan, synth
from conftest import rel_max_err
from oracle.plan_cpu import CpuPlan

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.mark.parametrize("BATCH,T,D,H,HEADS", [(2, 64, 128, 256, 2), (1, 100, 192, 384, 3),
                                               (8, 512, 1024, 4096, 16)])
def test_block_train_plan(be, oracle, BATCH, T, D, H, HEADS):
    """The plan bwppc-hip lowers from tiny_model's block and its DSL autodiff
    (plans/block_train.plan), rebound to each size; the last case is
    config 5 itself (the step the bench times), where split-K runs on the
    K = 4096 weight-gradient GEMMs and attention over 128 (batch, head)
    slices.  Against float64 autograd of the same program, and at the small
    sizes also against the same plan run op by op on the oracle."""
    import torch
    from blockref import block_inputs, block_reference, grad_shapes
    text = plan.load_text("block_train", BATCH=BATCH, T=T, D=D, H=H, HEADS=HEADS)
    t = block_inputs(BATCH, T, D, H, seed=BATCH * 1000 + T)
    p = plan.Plan(be, text)
    p.allocate()
    dev = {k: torch.from_numpy(v).cuda() for k, v in t.items()}
    for k, v in dev.items():
        p.bind(k, v)
    p.run()
    out = p.host("out", (BATCH * T, D))
    loss = float(p.host("loss", (1,))[0])
    shapes = grad_shapes(BATCH, T, D, H)
    got = {name: p.host(name, shape) for name, shape in shapes.items()}
    ref_out, ref_loss, ref_g = block_reference(t, BATCH, T, D, H, HEADS)
    assert rel_max_err(out, ref_out) <= TOL
    assert abs(loss - ref_loss) <= TOL * abs(ref_loss)
    for name in shapes:
        assert rel_max_err(got[name], ref_g[name]) <= TOL, name
    if BATCH * T <= 256:
        cp = CpuPlan(text, oracle)
        for k, v in t.items():
            cp.bind(k, v)
        cp.run()
        assert rel_max_err(out, cp.get("out")) <= TOL
        for name, shape in shapes.items():
            assert rel_max_err(got[name], cp.get(name).reshape(shape)) <= TOL, name
    # A second run over the same arena gives the same result.
    p.run()
    assert np.array_equal(p.host("dwq", shapes["dwq"]), got["dwq"])
    p.close()


def test_plan_unbound_input_is_an_error(be):
    p = plan.Plan(be, plan.load_text("block_train", BATCH=1, T=8, D=64, H=64, HEADS=1))
    p.allocate()
    with pytest.raises(plan.PlanError) as e:
        p.run()
    assert "not bound" in str(e.value)
    p.close()


def _bf16_dev(torch, a):
    return torch.from_numpy(synth.to_bf16_bits(a).view(np.int16)).cuda()


@pytest.mark.parametrize("causal", [False, True])
def test_attention_plans_bf16(be, oracle, causal):
    """attention.bwpp lowered for bf16 [B, H, T, D] operands: the training
    plan (forward with lse, backward seeded by dout) and the causal
    forward, at T = 2048, d = 128 (config 4's per-head shape), two (b, h)
    slices checked against the oracle on the exact bf16 inputs; bar 2e-2."""
    import torch
    B, H, T, D = 2, 4, 2048, 128
    vals = [synth.normal((B, H, T, D), 12, i) for i in range(4)]
    bits = [synth.to_bf16_bits(v) for v in vals]
    exact = [synth.bf16_bits_to_f32(b) for b in bits]
    name = "attention_causal_bf16" if causal else "attention_train_bf16"
    p = plan.Plan(be, plan.load_text(name, B=B, H=H, T=T, D=D))
    p.allocate()
    devs = [_bf16_dev(torch, v) for v in vals]
    for n, d in zip(("q", "k", "v", "dout"), devs):
        if not (causal and n == "dout"):
            p.bind(n, d)
    p.run()
    scale = D ** -0.5
    out = synth.bf16_bits_to_f32(p.host("out", (B, H, T, D), np.uint16))
    grads = None if causal else [synth.bf16_bits_to_f32(p.host(n, (B, H, T, D), np.uint16)) for n in ("dq", "dk", "dv")]
    for b, h in ((0, 0), (B - 1, H - 1)):
        sl = [np.ascontiguousarray(e[b:b + 1, h:h + 1]) for e in exact]
        assert rel_max_err(out[b:b + 1, h:h + 1], oracle.attention_bh(*sl[:3], scale, causal)) <= 2e-2
        if grads:
            for got, want in zip(grads, oracle.attention_grad(*sl, scale, causal)):
                assert rel_max_err(got[b:b + 1, h:h + 1], want) <= 2e-2
    p.close()


def test_c3_plan_bf16_gemm(be, oracle):
    """matmul_add_silu.bwpp lowered at config 3's size (bf16): one GEMM with
    the bias + SiLU epilogue; 64 rows against the oracle."""
    import torch
    M, K, N = 4096, 4096, 11008
    a = synth.normal((M, K), 13, 0, 0.0, 0.02)
    b = synth.normal((K, N), 13, 1, 0.0, 0.02)
    bias = synth.normal((N,), 13, 2, 0.0, 0.02)
    p = plan.Plan(be, plan.load_text("matmul_add_silu"))
    p.allocate()
    for n, v in (("a", a), ("b", b), ("bias", bias)):
        p.bind(n, _bf16_dev(torch, v))
    p.run()
    y = synth.bf16_bits_to_f32(p.host("out", (M, N), np.uint16))
    ex = lambda v: synth.bf16_bits_to_f32(synth.to_bf16_bits(v))
    rows = np.r_[0:32, M - 32:M]
    want = oracle.matmul(ex(a[rows]), ex(b), ex(bias), apply_silu=True, apply_bias=True)
    assert rel_max_err(y[rows], want) <= 2e-2
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


@pytest.mark.parametrize("C", [6, 8])
def test_copy_between_strided_views(be, C):
    """Copies into and out of column views of a wider tensor (the weight
    concatenation of grouped GEMMs): the executor's strided copy, on the
    scalar path (C = 6) and the 128-bit path (C = 8)."""
    import torch
    R = 5
    text = f"""bwpp.plan 1
dim R {R}
dim C {C}
value x f32 [R,C] input
value y f32 [R,C] input
value cat f32 [R,2*C] temp
value whole f32 [R,2*C] output
value back f32 [R,C] output
view xc of=cat offset=0 ld=2*C shape=[R,C]
view yc of=cat offset=C ld=2*C shape=[R,C]
op copy out=xc in=x bcast=full
op copy out=yc in=y bcast=full
op copy out=whole in=cat bcast=full
op copy out=back in=yc bcast=full
"""
    x, y = synth.normal((R, C), 1, 0), synth.normal((R, C), 2, 0)
    p = plan.Plan(be, text)
    p.allocate()
    xd = torch.from_numpy(x).cuda()
    yd = torch.from_numpy(y).cuda()
    p.bind("x", xd)
    p.bind("y", yd)
    p.run()
    assert np.array_equal(p.host("whole", (R, 2 * C)), np.hstack([x, y]))
    assert np.array_equal(p.host("back", (R, C)), y)
    p.close()


@pytest.mark.parametrize("C", [6, 8])
def test_multi_pair_copy(be, C):
    """`op copy out=a,b,c in=x,y,z`: three copies in one launch, into
    column blocks of a concatenation and back out of them (different row
    strides per pair), on the scalar path (C = 6) and the 128-bit path
    (C = 8); rows of unequal counts across the pairs."""
    import torch
    R = 7
    text = f"""bwpp.plan 1
dim R {R}
dim C {C}
value x f32 [R,C] input
value y f32 [R,C] input
value z f32 [R,C] input
value w f32 [3,C] input
value cat f32 [R,3*C] temp
value whole f32 [R,3*C] output
value bx f32 [R,C] output
value bz f32 [R,C] output
value w2 f32 [3,C] output
view xc of=cat offset=0 ld=3*C shape=[R,C]
view yc of=cat offset=C ld=3*C shape=[R,C]
view zc of=cat offset=2*C ld=3*C shape=[R,C]
op copy out=xc,yc,zc in=x,y,z bcast=full
op copy out=whole in=cat bcast=full
op copy out=bx,bz,w2 in=xc,zc,w bcast=full
"""
    x, y, z = (synth.normal((R, C), i, 0) for i in range(3))
    w = synth.normal((3, C), 9, 0)
    p = plan.Plan(be, text)
    p.allocate()
    for n, a in (("x", x), ("y", y), ("z", z), ("w", w)):
        p.bind(n, torch.from_numpy(a).cuda())
    p.run()
    assert np.array_equal(p.host("whole", (R, 3 * C)), np.hstack([x, y, z]))
    assert np.array_equal(p.host("bx", (R, C)), x)
    assert np.array_equal(p.host("bz", (R, C)), z)
    assert np.array_equal(p.host("w2", (3, C)), w)
    p.close()


def test_multi_pair_copy_overlap_is_an_error(be):
    """Two pairs writing overlapping views of one tensor: refused at run."""
    import torch
    text = """bwpp.plan 1
value x f32 [4,8] input
value y f32 [4,8] input
value cat f32 [4,12] output
view a of=cat offset=0 ld=12 shape=[4,8]
view b of=cat offset=4 ld=12 shape=[4,8]
op copy out=a,b in=x,y bcast=full
"""
    p = plan.Plan(be, text)
    p.allocate()
    p.bind("x", torch.zeros((4, 8), device="cuda"))
    p.bind("y", torch.zeros((4, 8), device="cuda"))
    with pytest.raises(plan.PlanError, match="overlaps"):
        p.run()
    p.close()


def test_plan_graph_replay(be):
    """bwpp_hip_plan_capture / replay: a captured training step replays
    bit-identical to the eager run, three times in a row with other eager
    work and synchronizations between the replays; rebinding an input drops
    the graph (replay refuses) until it is captured again."""
    import torch
    from blockref import block_inputs, grad_shapes
    B, T, D, H, HEADS = 2, 64, 128, 256, 2
    shapes = dict(grad_shapes(B, T, D, H), out=(B * T, D), loss=(1,))
    side = torch.cuda.Stream()
    be.set_stream(side)
    try:
        p = plan.Plan(be, plan.load_text("block_train", BATCH=B, T=T, D=D, H=H, HEADS=HEADS))
        p.allocate()
        dev = {k: torch.from_numpy(v).cuda() for k, v in block_inputs(B, T, D, H, seed=21).items()}
        torch.cuda.synchronize()
        for k, v in dev.items():
            p.bind(k, v)
        p.run()
        want = {n: p.host(n, sh) for n, sh in shapes.items()}
        p.capture()
        x = torch.randn(4096, 1024, device="cuda")
        y = torch.empty_like(x)
        torch.cuda.synchronize()
        for rep in range(3):
            p.replay()
            be.dispatch_softmax(x, y, bwpp.SoftmaxParams(4096, 1024, 1024))  # eager work on the same stream
            torch.cuda.synchronize()
            for n, sh in shapes.items():
                assert np.array_equal(p.host(n, sh).view(np.uint32), want[n].view(np.uint32)), (rep, n)
        # a different x: the graph is dropped; capture again and compare with an eager run
        x2 = torch.from_numpy(block_inputs(B, T, D, H, seed=22)["x"]).cuda()
        torch.cuda.synchronize()
        p.bind("x", x2)
        with pytest.raises(plan.PlanError):
            p.replay()
        p.run()
        want2 = p.host("dx", shapes["dx"])
        assert not np.array_equal(want2, want["dx"])
        p.capture()
        p.replay()
        assert np.array_equal(p.host("dx", shapes["dx"]).view(np.uint32), want2.view(np.uint32))
        p.close()
    finally:
        torch.cuda.synchronize()
        be.set_stream(torch.cuda.current_stream())


def test_plan_replay_after_workspace_growth():
    """A captured graph's kernels address the handle's workspace as it was
    at capture.  A later op on the handle that needs a larger workspace
    (here a split-K fp32 GEMM) reallocates it, and replay then refuses
    instead of running on freed memory -- unless the new workspace landed
    at the same address, where replay is valid; capturing again restores
    replay, bit-identical to an eager run."""
    import torch
    from blockref import block_inputs, grad_shapes
    B, T, D, H, HEADS = 2, 64, 128, 256, 2
    shapes = dict(grad_shapes(B, T, D, H), loss=(1,))
    h = bwpp.HipBackend(0)
    side = torch.cuda.Stream()
    h.set_stream(side)
    try:
        p = plan.Plan(h, plan.load_text("block_train", BATCH=B, T=T, D=D, H=H, HEADS=HEADS))
        p.allocate()
        for k, v in block_inputs(B, T, D, H, seed=23).items():
            p.bind(k, torch.from_numpy(v).cuda())
        torch.cuda.synchronize()
        p.run()
        want = {n: p.host(n, sh) for n, sh in shapes.items()}
        p.capture()
        # 1024 x 1024 x 4096, A^T B: split into K ranges, 16+ MiB of partial planes
        M, N, K = 1024, 1024, 4096
        a = torch.randn(K, M, device="cuda")
        b = torch.randn(K, N, device="cuda")
        c = torch.empty(M, N, device="cuda")
        torch.cuda.synchronize()
        h.dispatch_matmul(a, b, c, None, bwpp.MatmulParams(M, N, K, M, N, N, 0, 0, 1, 0))
        assert h.last_kernel == "bwpp_gemm_f32_splitk_reduce", h.last_kernel
        torch.cuda.synchronize()
        try:
            p.replay()
        except plan.PlanError as e:
            assert "workspace was reallocated" in str(e)
        else:
            torch.cuda.synchronize()
            for n, sh in shapes.items():
                assert np.array_equal(p.host(n, sh).view(np.uint32), want[n].view(np.uint32)), n
        p.capture()
        p.replay()
        torch.cuda.synchronize()
        for n, sh in shapes.items():
            assert np.array_equal(p.host(n, sh).view(np.uint32), want[n].view(np.uint32)), n
        p.close()
    finally:
        torch.cuda.synchronize()
        h.close()


def test_plan_capture_needs_a_stream(be):
    import torch
    be.set_stream(torch.cuda.default_stream())
    p = plan.Plan(be, "bwpp.plan 1\ndim N 4\nvalue x f32 [N] input\nvalue y f32 [N] output\nop silu out=y in=x\n")
    p.allocate()
    x = torch.ones(4, device="cuda")
    p.bind("x", x)
    with pytest.raises(plan.PlanError) as e:
        p.capture()
    assert "non-default stream" in str(e.value)
    p.close()


# ---------------------------------------------- every committed plan, on GPU
# Reduced sizes for each committed f32 plan not run above (config-size runs:
# block_train, the bf16 attention plans and matmul_add_silu).
_SMALL = {
    "matmul": dict(M=96, K=80, N=112),
    "matmul_add_bias_reshape": dict(M=96, K=80, N=112),
    "multi_fn_bias": dict(M=96, K=80, N=112),
    "norms": dict(B=64, N=300),
    "block_fwd": dict(BATCH=2, T=64, D=128, H=256, HEADS=2),
    "tiny_model_fwd": dict(BATCH=2, T=48, D=128, H=256, V=384, HEADS=2),
    "attention_train": dict(B=2, H=3, T=100, D=64),
}


def _plan_inputs(cp, seed):
    """Inputs N(0,1), weights N(0,0.1), gains U[0.5,1.5], by value kind."""
    binds = {}
    for i, (name, v) in enumerate(sorted(cp.vals.items())):
        if v["kind"] not in ("input", "param"):
            continue
        shape = tuple(v["dims"])
        if v["kind"] == "param" and len(shape) == 1 and name.startswith("g"):
            binds[name] = synth.uniform(shape, seed, i, 0.5, 1.5)
        elif v["kind"] == "param":
            binds[name] = synth.normal(shape, seed, i, 0.0, 0.1)
        else:
            binds[name] = synth.normal(shape, seed, i)
    return binds


def _run_both(be, oracle, text, seed):
    import torch
    cp = CpuPlan(text, oracle)
    binds = _plan_inputs(cp, seed)
    for k, v in binds.items():
        cp.bind(k, v)
    cp.run()
    p = plan.Plan(be, text)
    p.allocate()
    for k, v in binds.items():
        p.bind(k, torch.from_numpy(np.ascontiguousarray(v)).cuda())
    p.run()
    outs = [n for n, v in cp.vals.items() if v["kind"] == "output"]
    got = {n: p.host(n, cp.get(n).shape) for n in outs}
    return cp, p, got


@pytest.mark.parametrize("name", sorted(_SMALL))
def test_committed_plan_on_gpu_matches_cpu_plan(be, oracle, name):
    """Each committed plan the lowering emits from the reference's examples
    (examples/*.bwpp), rebound to a reduced size, run by the executor on
    the GPU against the same plan run op by op on the oracle: every output,
    1e-4 relative max-norm."""
    text = plan.load_text(name, **_SMALL[name])
    cp, p, got = _run_both(be, oracle, text, len(name))
    assert got
    for n, g in got.items():
        assert np.isfinite(g).all(), n
        assert rel_max_err(g, cp.get(n)) <= TOL, n
    p.close()


def test_reduce_max_program_on_gpu(be, oracle):
    """tests/golden/bwpp/reduce_max.bwpp lowered by bwppc-hip: y = x @ w,
    out = reduce_max(y, 1), and with --train seed its DSL autodiff (mask of
    the row maxima, times the broadcast dout, into both matmul gradients).
    The forward's maxima are bit-exact against the oracle's reduce_max of
    the GPU's own y; the whole plans against the CPU plan (1e-4)."""
    import os
    fx = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "bwpp")
    dims = dict(M=300, K=96, N=500)
    text = plan.load_text(os.path.join(fx, "reduce_max.plan"), **dims)
    cp, p, got = _run_both(be, oracle, text, 31)
    y = p.host("y", (dims["M"], dims["N"]))
    want, _ = oracle.reduce_max(y, 1)
    from conftest import assert_bits_equal
    assert_bits_equal(got["out"].reshape(-1), want)
    assert rel_max_err(got["out"], cp.get("out")) <= TOL
    p.close()
    text = plan.load_text(os.path.join(fx, "reduce_max_train.plan"), **dims)
    cp, p, got = _run_both(be, oracle, text, 31)
    assert set(got) == {"out", "dx", "dw"}
    for n, g in got.items():
        assert rel_max_err(g, cp.get(n)) <= TOL, n
    p.close()
