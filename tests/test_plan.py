"""Launch-plan parsing and memory planning (no GPU: the plan is created
without a device handle).  The planner follows compiler/mem_plan.c:43-146
(buffer reuse by liveness) but sizes buffers in bytes from the bound dims
and never gives an operator the buffer of one of its own inputs -- the
reference frees inputs before allocating the output (mem_plan.c:89-140)."""
import re

import pytest

from bwpp import plan

SMALL = dict(BATCH=2, T=64, D=128, H=256, HEADS=2)


def _ops_and_views(text):
    views, ops = {}, []
    for line in text.splitlines():
        t = line.split("#")[0].split()
        if not t:
            continue
        if t[0] == "view":
            views[t[1]] = dict(kv.split("=", 1) for kv in t[2:])["of"]
        elif t[0] == "op":
            kv = dict(x.split("=", 1) for x in t[2:] if "=" in x)
            ops.append((t[1], kv["out"].split(","), kv.get("in", "").split(",")))
    return ops, views


def _buffers(report):
    return {m.group(2): int(m.group(1)) for m in re.finditer(r"-> buffer(\d+)  # (\S+)", report)}


@pytest.mark.parametrize("dims", [{}, SMALL])
def test_block_plan_report_and_no_self_alias(dims):
    text = plan.load_text("block_train", **dims)
    p = plan.Plan(None, text)
    rep = p.report()
    head = rep.splitlines()[0]
    assert re.fullmatch(r"buffers=\d+ values=\d+", head)
    nbuf = int(head.split()[0].split("=")[1])
    assert all(re.fullmatch(r"buffer\d+ f32 \[[^\]]*\] row_major bytes=\d+ offset=\d+", l)
               for l in rep.splitlines()[1:1 + nbuf])
    buf = _buffers(rep)
    ops, views = _ops_and_views(text)
    base = lambda n: views.get(n, n)
    ntemps = sum(1 for l in text.splitlines() if l.split()[:1] == ["value"] and l.split()[-1] == "temp")
    assert nbuf < ntemps + 12, "temps were not reused"
    for kind, outs, ins in ops:
        ob = {buf[base(o)] for o in outs if base(o) in buf}
        ib = {buf[base(i)] for i in ins if base(i) in buf}
        assert not (ob & ib), f"{kind}: output shares a buffer with an input"
    assert p.arena_bytes == int(rep.strip().splitlines()[-1].split("=")[1])


def test_block_plan_arena_fits_reuse():
    """Full-size config 5: every temp of fwd + bwd in well under 1 GB."""
    p = plan.Plan(None, plan.load_text("block_train"))
    assert 0.3e9 < p.arena_bytes < 1.0e9


_IO = "bwpp.plan 1\nvalue a f32 [4,4] input\nvalue b f32 [4,4] input\nvalue y f32 [4,4] output\n"


@pytest.mark.parametrize("text,msg", [
    ("dim B 2\n", "bwpp.plan 1"),
    ("bwpp.plan 1\nvalue x f32 [Q,4] input\n", "unknown dim"),
    ("bwpp.plan 1\nvalue x f32 [4,4] temp\nop softmax out=y in=x\n", "unknown value"),
    ("bwpp.plan 1\nvalue x f32 [4,4] input\nview v of=x offset=8 ld=4 shape=[3,4]\n", "runs past"),
    ("bwpp.plan 1\nvalue x f32 [4,4] temp\nvalue y f32 [4,4] output\nop softmax out=y in=x\n", "never written"),
    ("bwpp.plan 1\nvalue x f32 [4,4] input\nvalue t f32 [4,4] temp\nvalue y f32 [4,4] output\n"
     "op softmax out=y in=t\nop softmax out=t in=x\n", "before it is written"),
    ("bwpp.plan 1\nvalue x bf16 [4,4] input\nvalue y f32 [4,4] output\nop softmax out=y in=x\n", "f32 values only"),
    ("bwpp.plan 1\nvalue a bf16 [4,4] input\nvalue b f32 [4,4] input\nvalue y bf16 [4,4] output\n"
     "op matmul out=y in=a,b\n", "different dtypes"),
    # Op arguments are checked when the plan is created, not when it runs.
    (_IO + "op matmul out=y in=a,b epi=gelu\n", "epi must be"),
    (_IO + "op add out=y in=a,b bcast=diag\n", "bcast must be"),
    (_IO + "op frobnicate out=y in=a\n", "unknown op"),
    ("bwpp.plan 1\nvalue a f32 [4,3] input\nvalue b f32 [4,4] input\nvalue y f32 [4,4] output\n"
     "op matmul out=y in=a,b\n", "operand shapes do not match"),
    (_IO + "op attention out=y in=a,b,b heads=3\n", "bad batch / heads"),
])
def test_plan_errors(text, msg):
    with pytest.raises(plan.PlanError) as e:
        plan.Plan(None, text)
    assert msg in str(e.value)


def test_dead_temp_buffer_is_reused():
    """A temp written but never read gives its buffer back after its op."""
    text = ("bwpp.plan 1\nvalue x f32 [8,8] input\nvalue dead f32 [8,8] temp\nvalue t f32 [8,8] temp\n"
            "value y f32 [8,8] output\nop softmax out=dead in=x\nop softmax out=t in=x\nop softmax out=y in=t\n")
    rep = plan.Plan(None, text).report()
    buf = _buffers(rep)
    assert buf["dead"] == buf["t"]
