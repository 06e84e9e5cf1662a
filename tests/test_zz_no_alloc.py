"""bwpp_hip_dispatch_attention_grad_noalloc: the attention backward with its
per-query row sums in the library's device-resident scratch array instead
of the handle's workspace (no allocation).  Checked through the C ABI
against bwpp_hip_dispatch_attention_grad, which runs the same kernels, so
dQ, dK and dV must be bit-identical; two calls in a row, the second with a
smaller input, so a stale scratch from the first would show.  Sizes beyond
the scratch maximum and the bf16 path that needs workspace copies are
refused with UNSUPPORTED before anything is launched."""
import numpy as np
import pytest

import bwpp
from bwpp import synth

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _case(B, H, M, N, d, causal, dtype, seed):
    torch = _torch()
    tdt = torch.bfloat16 if dtype == bwpp.DType.BF16 else torch.float32

    def t(shape, st):
        return torch.from_numpy(synth.normal(shape, seed, st)).cuda().to(tdt)

    q, k, v, do = t((B, H, M, d), 0), t((B, H, N, d), 1), t((B, H, N, d), 2), t((B, H, M, d), 3)
    prm = bwpp.AttentionParams(M=M, N=N, K=d, D=d, ldq=d, ldk=d, ldv=d, ldo=d, batch=B, heads=H,
                               scale=d ** -0.5, causal=int(causal), dtype=int(dtype))
    return q, k, v, do, prm


def _grads(fn, q, k, v, o, do, lse, prm):
    torch = _torch()
    g = [torch.full_like(x, 7.0) for x in (q, k, v)]
    fn(q, k, v, o, do, lse, *g, prm)
    torch.cuda.synchronize()
    return g


@pytest.mark.parametrize("dtype,d,causal", [(bwpp.DType.F32, 64, True), (bwpp.DType.BF16, 128, False),
                                            (bwpp.DType.BF16, 128, True), (bwpp.DType.F32, 40, False)])
def test_noalloc_matches_workspace_entry(be, dtype, d, causal):
    torch = _torch()
    # first call larger, second smaller: the second must not see the first's scratch
    for B, H, M, N, seed in ((2, 4, 300, 260, 1), (1, 2, 70, 90, 2)):
        q, k, v, do, prm = _case(B, H, M, N, d, causal, dtype, seed)
        o = torch.empty_like(q)
        lse = torch.empty((B, H, M), device="cuda")
        be.dispatch_attention_lse(q, k, v, o, lse, prm)
        got = _grads(be.dispatch_attention_grad_noalloc, q, k, v, o, do, lse, prm)
        want = _grads(be.dispatch_attention_grad, q, k, v, o, do, lse, prm)
        for a, b, name in zip(got, want, ("dq", "dk", "dv")):
            assert torch.isfinite(a.float()).all(), name
            assert torch.equal(a, b), (name, B, H, M, N)


def test_noalloc_accepts_scratch_maximum(be):
    """batch * heads * M = 2,097,151 query rows: their row sums (4 bytes
    each) plus the 4-byte tail fill the 8 MiB scratch exactly, the largest
    accepted size; results bit-identical to the workspace entry point."""
    torch = _torch()
    B, H, M, N, d = 1, 889, 2359, 16, 16  # 889 * 2359 = 2,097,151
    assert B * H * M == 2_097_151
    g = torch.Generator(device="cuda").manual_seed(5)
    q, do = (0.5 * torch.randn((B, H, M, d), device="cuda", generator=g) for _ in range(2))
    k, v = (0.5 * torch.randn((B, H, N, d), device="cuda", generator=g) for _ in range(2))
    o = torch.empty_like(q)
    lse = torch.empty((B, H, M), device="cuda")
    prm = bwpp.AttentionParams(M=M, N=N, K=d, D=d, ldq=d, ldk=d, ldv=d, ldo=d, batch=B, heads=H)
    be.dispatch_attention_lse(q, k, v, o, lse, prm)
    got = _grads(be.dispatch_attention_grad_noalloc, q, k, v, o, do, lse, prm)
    want = _grads(be.dispatch_attention_grad, q, k, v, o, do, lse, prm)
    for a, b, name in zip(got, want, ("dq", "dk", "dv")):
        assert torch.isfinite(a).all(), name
        assert torch.equal(a, b), name


def test_noalloc_refuses_beyond_scratch(be):
    """batch * heads * M = 2,097,152 query rows need 8 MiB + 4 bytes of row
    sums: one row over the scratch maximum.  The buffers are real and
    large enough, so nothing could read out of bounds even if a launch
    happened; the call must return UNSUPPORTED and launch nothing."""
    torch = _torch()
    B, H, M, N, d = 1, 1024, 2048, 16, 16
    q, do = (torch.zeros((B, H, M, d), device="cuda") for _ in range(2))
    k, v = (torch.zeros((B, H, N, d), device="cuda") for _ in range(2))
    o = torch.zeros_like(q)
    lse = torch.zeros((B, H, M), device="cuda")
    dq, dk, dv = torch.full_like(q, 7.0), torch.full_like(k, 7.0), torch.full_like(v, 7.0)
    prm = bwpp.AttentionParams(M=M, N=N, K=d, D=d, ldq=d, ldk=d, ldv=d, ldo=d, batch=B, heads=H)
    with pytest.raises(bwpp.BwppError) as e:
        be.dispatch_attention_grad_noalloc(q, k, v, o, do, lse, dq, dk, dv, prm)
    assert e.value.status == bwpp.Status.UNSUPPORTED
    torch.cuda.synchronize()
    assert bool((dq == 7.0).all()) and bool((dk == 7.0).all()) and bool((dv == 7.0).all())


def test_noalloc_refuses_unaligned_bf16(be):
    torch = _torch()
    B, H, M, N, d, ld = 1, 1, 40, 40, 64, 68  # 136-byte rows: not 16-byte aligned
    mk = lambda rows: torch.zeros((B, H, rows, ld), device="cuda", dtype=torch.bfloat16)
    q, k, v, o, do = mk(M), mk(N), mk(N), mk(M), mk(M)
    dq, dk, dv = mk(M), mk(N), mk(N)
    lse = torch.zeros((B, H, M), device="cuda")
    prm = bwpp.AttentionParams(M=M, N=N, K=d, D=d, ldq=ld, ldk=ld, ldv=ld, ldo=ld, batch=B, heads=H,
                               q_batch_stride=H * M * ld, q_head_stride=M * ld, k_batch_stride=H * N * ld,
                               k_head_stride=N * ld, v_batch_stride=H * N * ld, v_head_stride=N * ld,
                               o_batch_stride=H * M * ld, o_head_stride=M * ld,
                               scale=0.125, dtype=int(bwpp.DType.BF16))
    with pytest.raises(bwpp.BwppError) as e:
        be.dispatch_attention_grad_noalloc(q, k, v, o, do, lse, dq, dk, dv, prm)
    assert e.value.status == bwpp.Status.UNSUPPORTED
