"""The HIP target of BW++'s compiler (bluewolf-plus-plus_amd/compiler:
lower_hip.c over the reference's own front end, graph IR and autodiff).

- The committed plans are exactly what the lowering emits from the
  reference's examples (needs the reference tree to rebuild bwppc-hip).
- Each committed plan passes the executor's checks, and the f32 ones,
  run op by op on the oracle (oracle/plan_cpu.py), match float64 torch
  evaluations of the DSL programs they come from.
- The fused attention lowering matches the op-by-op lowering of the same
  graph (matmul, transpose, softmax, their autodiff chain).
- Graph gaps are answered, not papered over: numeric literals need their
  values, batching needs the attention fused, dims must be bound."""
import os
import subprocess

import numpy as np
import pytest

from bwpp import plan, synth
from conftest import rel_max_err
from oracle.plan_cpu import CpuPlan

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
COMPILER = os.path.join(ROOT, "bluewolf-plus-plus_amd", "compiler")
PLANS = os.path.join(ROOT, "bluewolf-plus-plus_amd", "plans")
REFERENCE = os.environ.get("REFERENCE", "/root/reference")
BWPPC = os.path.join(COMPILER, "_build", "bwppc-hip")
FIXTURES = os.path.join(ROOT, "tests", "golden", "bwpp")

needs_reference = pytest.mark.skipif(not os.path.isdir(os.path.join(REFERENCE, "compiler")),
                                     reason="bwppc-hip links the reference compiler's sources")


@pytest.fixture(scope="module")
def bwppc():
    subprocess.run(["make", "-C", COMPILER, "-s"], check=True, capture_output=True)
    return BWPPC


def lower(bwppc, src, tmp_path, *args, ok=True):
    out = tmp_path / "out.plan"
    r = subprocess.run([bwppc, src, str(out), *args], capture_output=True, text=True)
    if ok:
        assert r.returncode == 0, r.stderr
        return out.read_text()
    assert r.returncode != 0
    return r.stderr


@needs_reference
def test_committed_plans_match_the_lowering():
    r = subprocess.run(["python", os.path.join(COMPILER, "emit_plans.py"), "--check"], capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stdout + r.stderr


@needs_reference
def test_inspection_flags(bwppc, tmp_path):
    """--dot / --grad-dot / --mem-plan keep the reference CLI's names
    (compiler/main.c:49-86): the forward and autodiff graphs as DOT
    (bwpp_graph_dump_dot, main.c:133-157), and the memory plan of the
    emitted launch plan (main.c:169-182), which is exactly what the library
    reports for that plan at run time: the reference dump's lines
    (mem_plan.c:176-193) with byte sizes, offsets and the arena total."""
    src = os.path.join(REFERENCE, "examples", "tiny_model.bwpp")
    mem, dot, gdot = tmp_path / "mem.txt", tmp_path / "g.dot", tmp_path / "grad.dot"
    args = ["--entry", "block", "--dim", "T=64", "--dim", "D=128", "--dim", "H=256", "--batch", "2",
            "--heads", "2", "--causal", "--attn-scale", "auto", "--train", "mean_square"]
    text = lower(bwppc, src, tmp_path, *args, "--mem-plan", str(mem), "--dot", str(dot), "--grad-dot", str(gdot))
    p = plan.Plan(None, text)
    report = mem.read_text()
    assert report == p.report()
    assert report.startswith("buffers=") and f"arena_bytes={p.arena_bytes}" in report
    lines = report.splitlines()
    nbuf = int(lines[0].split()[0].split("=")[1])
    assert sum(ln.startswith("buffer") for ln in lines[1:]) == nbuf
    p.close()
    fwd, grad = dot.read_text(), gdot.read_text()
    assert fwd.startswith("digraph") and grad.startswith("digraph")
    assert "rmsnorm" in fwd and "softmax_grad" in grad
    # the flags leave the plan itself unchanged (up to its recorded command line)
    plain = lower(bwppc, src, tmp_path, *args)
    strip = lambda t: "\n".join(ln for ln in t.splitlines() if not ln.startswith("# generated"))
    assert strip(text) == strip(plain)


def test_committed_plans_pass_the_executor_checks():
    names = sorted(f for f in os.listdir(PLANS) if f.endswith(".plan"))
    assert "block_train.plan" in names and "attention_train_bf16.plan" in names
    for n in names:
        p = plan.Plan(None, plan.load_text(n[:-5]))
        assert p.arena_bytes > 0, n
        p.close()


def _cpu(name, binds, **dims):
    cp = CpuPlan(plan.load_text(name, **dims))
    for k, v in binds.items():
        cp.bind(k, v)
    cp.run()
    return cp


def test_attention_train_plan(oracle):
    """attention.bwpp (rank-4 [B, H, T, D] operands): fused attention with
    lse, and attention_grad seeded by the plan input dout."""
    import torch
    B, H, T, D = 1, 2, 37, 16
    q, k, v, do = (synth.normal((B, H, T, D), 5, i) for i in range(4))
    cp = _cpu("attention_train", {"q": q, "k": k, "v": v, "dout": do}, B=B, H=H, T=T, D=D)
    tq, tk, tv = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (q, k, v))
    out = torch.softmax((tq @ tk.transpose(-1, -2)) * D ** -0.5, dim=-1) @ tv
    out.backward(torch.tensor(do, dtype=torch.float64))
    assert rel_max_err(cp.get("out").reshape(B, H, T, D), out.detach().numpy()) <= 1e-5
    for name, t in (("dq", tq), ("dk", tk), ("dv", tv)):
        assert rel_max_err(cp.get(name).reshape(B, H, T, D), t.grad.numpy()) <= 1e-5, name


def test_tiny_model_forward_plan():
    """Two blocks, the classifier and its softmax (examples/tiny_model.bwpp)
    over a batch of 2, 2 heads, causal, scale 1/sqrt(d)."""
    import torch
    BATCH, T, D, H, V, HEADS = 2, 12, 32, 64, 48, 2
    rng = lambda shape, st, sd=0.1: synth.normal(shape, 9, st, 0.0, sd)
    t = {"x": synth.normal((BATCH * T, D), 9, 0), "wcls": rng((D, V), 1)}
    names = ["wq{}", "wk{}", "wv{}", "wo{}", "w1{}", "w2{}", "g1{}", "g2{}"]
    shapes = [(D, D)] * 4 + [(D, H), (H, D), (D,), (D,)]
    st = 2
    for i in (1, 2):
        for n, s in zip(names, shapes):
            t[n.format(i)] = synth.uniform(s, 9, st, 0.5, 1.5) if n.startswith("g") else rng(s, st)
            st += 1
    cp = _cpu("tiny_model_fwd", t, BATCH=BATCH, T=T, D=D, H=H, V=V, HEADS=HEADS)
    p = {k: torch.tensor(v, dtype=torch.float64) for k, v in t.items()}
    rms = lambda a, g: a / torch.sqrt((a * a).mean(dim=1, keepdim=True) + 1e-5) * g
    dh = D // HEADS
    split = lambda m: m.reshape(BATCH, T, HEADS, dh).permute(0, 2, 1, 3)
    mask = ~torch.ones(T, T, dtype=torch.bool).tril()

    def block(x, i):
        n1 = rms(x, p[f"g1{i}"])
        q, k, v = (split(n1 @ p[f"w{c}{i}"]) for c in "qkv")
        s = ((q @ k.transpose(-1, -2)) * dh ** -0.5).masked_fill(mask, float("-inf"))
        x1 = x + (torch.softmax(s, -1) @ v).permute(0, 2, 1, 3).reshape(BATCH * T, D) @ p[f"wo{i}"]
        return x1 + torch.nn.functional.silu(rms(x1, p[f"g2{i}"]) @ p[f"w1{i}"]) @ p[f"w2{i}"]

    want = torch.softmax(block(block(p["x"], 1), 2) @ p["wcls"], -1).numpy()
    assert rel_max_err(cp.get("probs"), want) <= 1e-5


def test_reduce_max_program_plans(oracle):
    """reduce_max.bwpp (y = x @ w; out = reduce_max(y, 1)) lowered with and
    without --train seed: the forward against float64, the backward against
    float64 autograd (unique maxima: torch's max gradient is the graph's
    mask * dout there), and with exact ties (duplicated columns of w)
    against the graph's rule, every tied column gets dout
    (graph_ir.c:1798-1821, bwpp_cpu_ref.c:192-219)."""
    import torch
    M, K, N = 40, 24, 56
    x, w = synth.normal((M, K), 4, 0), synth.normal((K, N), 4, 1)
    dout = synth.normal((M, 1), 4, 2)
    cp = _cpu(os.path.join(FIXTURES, "reduce_max.plan"), {"x": x, "w": w}, M=M, K=K, N=N)
    y64 = x.astype(np.float64) @ w.astype(np.float64)
    assert rel_max_err(cp.get("out"), y64.max(axis=1, keepdims=True)) <= 1e-5
    cp = _cpu(os.path.join(FIXTURES, "reduce_max_train.plan"), {"x": x, "w": w, "dout": dout}, M=M, K=K, N=N)
    tx, tw = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (x, w))
    out = (tx @ tw).amax(dim=1, keepdim=True)
    out.backward(torch.tensor(dout, dtype=torch.float64))
    assert rel_max_err(cp.get("dx"), tx.grad.numpy()) <= 1e-5
    assert rel_max_err(cp.get("dw"), tw.grad.numpy()) <= 1e-5
    # exact ties: column 2j + 1 of w repeats column 2j
    wt = w.copy()
    wt[:, 1::2] = wt[:, 0::2]
    cp = _cpu(os.path.join(FIXTURES, "reduce_max_train.plan"), {"x": x, "w": wt, "dout": dout}, M=M, K=K, N=N)
    y = cp.get("out")
    yfull = oracle.matmul(x, wt)
    mask = (yfull == y).astype(np.float64)
    assert (mask.sum(axis=1) == 2).all()  # each row's maximum is tied
    dy = mask * dout.astype(np.float64)
    assert rel_max_err(cp.get("dx"), dy @ wt.astype(np.float64).T) <= 1e-5
    assert rel_max_err(cp.get("dw"), x.astype(np.float64).T @ dy) <= 1e-5


def test_gemm_example_plans(oracle):
    """matmul, bias through a reshape and across inlined functions (fused
    as the GEMM epilogue), and norms (matmul -> softmax -> rmsnorm)."""
    M, K, N = 24, 40, 56
    a, b = synth.normal((M, K), 3, 0), synth.normal((K, N), 3, 1)
    bias, g = synth.normal((N,), 3, 2), synth.uniform((N,), 3, 3, 0.5, 1.5)
    cp = _cpu("matmul", {"a": a, "b": b}, M=M, K=K, N=N)
    assert np.array_equal(cp.get("out"), oracle.matmul(a, b))
    cp = _cpu("matmul_add_bias_reshape", {"a": a, "b": b, "bias": bias}, M=M, K=K, N=N)
    assert np.array_equal(cp.get("y"), oracle.matmul(a, b, bias, apply_bias=True))
    cp = _cpu("multi_fn_bias", {"x": a, "w": b, "bias": bias}, M=M, K=K, N=N)
    assert np.array_equal(cp.get("y"), oracle.matmul(a, b, bias, apply_bias=True))
    x, w = synth.normal((M, N), 3, 4), synth.normal((N, N), 3, 5)
    cp = _cpu("norms", {"x": x, "w": w, "gamma": g}, B=M, N=N)
    want = oracle.rmsnorm(oracle.softmax(oracle.matmul(x, w)), g, None, 1e-5)
    assert np.array_equal(cp.get("out"), want)


def test_c3_plan_is_one_fused_gemm():
    text = plan.load_text("matmul_add_silu")
    ops = [l for l in text.splitlines() if l.startswith("op ")]
    assert ops == ["op matmul out=out in=a,b,bias epi=add_silu"]
    assert "value a bf16 [M,K] input" in text


@needs_reference
def test_fused_attention_matches_op_by_op_lowering(bwppc, tmp_path):
    """With one sample, one head, no mask and scale 1 (the graph's own
    semantics), the attention region lowered op by op (matmul with tb=1,
    softmax, matmul; softmax_grad and the transposed products backward)
    and the fused attention / attention_grad give the same training step."""
    from blockref import block_inputs
    src = os.path.join(REFERENCE, "examples", "tiny_model.bwpp")
    T, D, H = 24, 32, 48
    dims = ["--entry", "block", "--dim", f"T={T}", "--dim", f"D={D}", "--dim", f"H={H}", "--train", "mean_square"]
    fused = lower(bwppc, src, tmp_path, *dims)
    plain = lower(bwppc, src, tmp_path, *dims, "--no-fuse-attention")
    assert "op attention " in fused and "op attention" not in plain
    assert "op softmax_grad" in plain
    t = block_inputs(1, T, D, H, seed=4)
    runs = []
    for text in (fused, plain):
        cp = CpuPlan(text)
        for k, v in t.items():
            cp.bind(k, v)
        cp.run()
        runs.append(cp)
    for name in ("out", "loss", "dx", "dwq", "dwk", "dwv", "dwo", "dw1", "dw2", "dg1", "dg2"):
        assert rel_max_err(runs[0].get(name), runs[1].get(name)) <= 1e-5, name


@needs_reference
def test_grouped_projections_match_separate_gemms(bwppc, tmp_path):
    """q, k, v = x @ wq, x @ wk, x @ wv run as one GEMM against [wq | wk |
    wv] (column views for q, k, v), and in training dwq / dwk / dwv and
    dx's three terms as one GEMM each; the step equals the lowering with
    one GEMM per projection."""
    from blockref import block_inputs
    src = os.path.join(REFERENCE, "examples", "tiny_model.bwpp")
    B, T, D, H, HEADS = 2, 32, 48, 96, 3
    dims = ["--entry", "block", "--dim", f"T={T}", "--dim", f"D={D}", "--dim", f"H={H}", "--batch", str(B),
            "--heads", str(HEADS), "--causal", "--attn-scale", "auto", "--train", "mean_square"]
    grouped = lower(bwppc, src, tmp_path, *dims)
    separate = lower(bwppc, src, tmp_path, *dims, "--no-group-gemms")
    n_mm = lambda t: sum(l.startswith("op matmul ") for l in t.splitlines())
    assert n_mm(separate) - n_mm(grouped) == 2 + 4  # forward 3 -> 1; dW 3 -> 1, dx terms 3 -> 1
    assert "view q of=ycat offset=0 ld=3*D shape=[BATCH*T,D]" in grouped
    assert "op matmul out=dwcat in=n1,dycat ta=1" in grouped
    t = block_inputs(B, T, D, H, seed=11)
    runs = []
    for text in (grouped, separate):
        cp = CpuPlan(text)
        for k, v in t.items():
            cp.bind(k, v)
        cp.run()
        runs.append(cp)
    for name in ("out", "loss", "dx", "dwq", "dwk", "dwv", "dwo", "dw1", "dw2", "dg1", "dg2"):
        assert rel_max_err(runs[0].get(name), runs[1].get(name)) <= 1e-5, name


@needs_reference
def test_fused_tails_match_separate_ops(bwppc, tmp_path):
    """x1 = x + ctx @ wo and out = x1 + h @ w2 (residual tails), h =
    silu(n2 @ w1) with the pre-activation kept for the backward (dual
    output), silu_grad(t, dO @ w2^T) (SiLU-gradient tail), the two
    residual-gradient adds folded into rmsnorm_grad (its fourth input) and
    the mean-square loss with its seed gradient in one pass give the same
    step as the separate ops (dout and every gradient bit for bit: only the
    loss's sum order differs)."""
    from blockref import block_inputs
    src = os.path.join(REFERENCE, "examples", "tiny_model.bwpp")
    B, T, D, H, HEADS = 2, 32, 48, 96, 3
    dims = ["--entry", "block", "--dim", f"T={T}", "--dim", f"D={D}", "--dim", f"H={H}", "--batch", str(B),
            "--heads", str(HEADS), "--causal", "--attn-scale", "auto", "--train", "mean_square"]
    fused = lower(bwppc, src, tmp_path, *dims)
    plain = lower(bwppc, src, tmp_path, *dims, "--no-fuse-tails")
    for f in ("fuse=residual", "fuse=dual_silu", "fuse=silu_grad"):
        assert f in fused and f not in plain
    n_in = lambda line: len(line.split(" in=")[1].split()[0].split(","))
    acc = lambda t: [l for l in t.splitlines() if l.startswith("op rmsnorm_grad ") and n_in(l) == 4]
    assert len(acc(fused)) == 2 and not acc(plain)
    assert "op mean_square out=loss,dout in=out,inv_n,two_n" in fused and "op mean_square" not in plain
    n_ops = lambda t: sum(l.startswith("op ") for l in t.splitlines())
    # two residual adds, silu, silu_grad, two gradient adds; the loss's 5 ops -> 1
    assert n_ops(plain) - n_ops(fused) == 6 + 4
    t = block_inputs(B, T, D, H, seed=12)
    runs = []
    for text in (fused, plain):
        cp = CpuPlan(text)
        for k, v in t.items():
            cp.bind(k, v)
        cp.run()
        runs.append(cp)
    for name in ("out", "loss", "dx", "dwq", "dwk", "dwv", "dwo", "dw1", "dw2", "dg1", "dg2"):
        assert rel_max_err(runs[0].get(name), runs[1].get(name)) <= 1e-5, name


@needs_reference
def test_literal_values_must_be_supplied(bwppc, tmp_path):
    src = os.path.join(FIXTURES, "scaled.bwpp")
    err = lower(bwppc, src, tmp_path, "--dim", "M=4", "--dim", "N=8", ok=False)
    assert "without its value" in err
    text = lower(bwppc, src, tmp_path, "--dim", "M=4", "--dim", "N=8", "--const", "0.5", "--const", "3")
    assert "const=0.5" in text and "const=3" in text
    x = synth.normal((4, 8), 1, 0)
    cp = CpuPlan(text)
    cp.bind("x", x)
    cp.run()
    np.testing.assert_allclose(cp.get("y"), (x * np.float32(0.5)) + np.float32(3), rtol=0, atol=0)


@needs_reference
def test_lowering_errors(bwppc, tmp_path):
    src = os.path.join(REFERENCE, "examples", "tiny_model.bwpp")
    base = ["--entry", "block", "--dim", "T=8", "--dim", "D=16"]
    assert "not bound" in lower(bwppc, src, tmp_path, *base, ok=False)  # H missing
    err = lower(bwppc, src, tmp_path, *base, "--dim", "H=32", "--batch", "2", "--no-fuse-attention", ok=False)
    assert "mix samples" in err
    err = lower(bwppc, src, tmp_path, *base, "--dim", "H=32", "--heads", "3", ok=False)
    assert "heads" in err
