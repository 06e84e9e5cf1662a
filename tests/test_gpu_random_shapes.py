"""Randomised GPU parity sweep: seeded random shapes, strides, transposes,
epilogues, masks and scales for the GEMMs, attention (forward, lse and
backward) and the row operators, each against the oracle at the bars of the
other tests (fp32 1e-4, bf16 inputs 2e-2, reduce_max values and indices bit
for bit).  The shapes mix full tiles, partial tiles and odd sizes so that
every kernel family and its edge paths are hit in combinations the
hand-picked cases do not list.  Sizes stay small so the oracle finishes in
seconds."""
import numpy as np
import pytest

import bwpp
from bwpp import synth
from conftest import rel_max_err

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4
BF16_TOL = 2e-2
CASES = 24


def _torch():
    import torch
    return torch


def dev(x):
    return _torch().from_numpy(np.ascontiguousarray(x, np.float32)).cuda()


def bf16(x):
    torch = _torch()
    bits = synth.to_bf16_bits(np.ascontiguousarray(x, np.float32))
    return torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16), synth.bf16_bits_to_f32(bits)


def host(t):
    torch = _torch()
    torch.cuda.synchronize()
    if t.dtype == torch.bfloat16:
        return synth.bf16_bits_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))
    return t.cpu().numpy()


def pick(rng, choices):
    return choices[int(rng.integers(len(choices)))]


@pytest.mark.parametrize("case", range(CASES))
def test_random_gemm(be, oracle, case):
    rng = np.random.default_rng(1000 + case)
    use_bf16 = case % 3 == 2
    big = [256, 512] if use_bf16 else [128, 256]
    M = int(pick(rng, big + [int(rng.integers(1, 300))]))
    N = int(pick(rng, big + [int(rng.integers(1, 300))]))
    K = int(pick(rng, [32, 64, 1024] + [int(rng.integers(1, 200))]))
    ta, tb = int(rng.integers(2)), int(rng.integers(2))
    epi = int(rng.integers(4))
    pad = int(pick(rng, [0, 0, 8, 5]))
    a = synth.normal((M, K), case, 0, 0.0, 0.5)
    b = synth.normal((K, N), case, 1, 0.0, 0.5)
    bias = synth.normal((N,), case, 2, 0.0, 0.5)
    sa = np.ascontiguousarray(a.T) if ta else a
    sb = np.ascontiguousarray(b.T) if tb else b
    # padded leading dimensions (row strides) on the stored operands
    lda, ldb, ldc = sa.shape[1] + pad, sb.shape[1] + pad, N + pad
    A = np.zeros((sa.shape[0], lda), np.float32)
    A[:, :sa.shape[1]] = sa
    Bm = np.zeros((sb.shape[0], ldb), np.float32)
    Bm[:, :sb.shape[1]] = sb
    torch = _torch()
    if use_bf16:
        (ad, A), (bd, Bm), (biasd, bias) = bf16(A), bf16(Bm), bf16(bias)
        c = torch.full((M, ldc), 3.0, dtype=torch.bfloat16, device="cuda")
        dt, tol = bwpp.DType.BF16, BF16_TOL
    else:
        ad, bd, biasd = dev(A), dev(Bm), dev(bias)
        c = torch.full((M, ldc), 3.0, device="cuda")
        dt, tol = bwpp.DType.F32, F32_TOL
    be.dispatch_matmul(ad, bd, c, biasd, bwpp.MatmulParams(M, N, K, lda, ldb, ldc, int(dt), epi, ta, tb))
    la = A[:, :sa.shape[1]]
    lb = Bm[:, :sb.shape[1]]
    want = oracle.matmul(np.ascontiguousarray(la.T if ta else la), np.ascontiguousarray(lb.T if tb else lb),
                         bias, apply_silu=epi in (2, 3), apply_bias=epi in (1, 3))
    got = host(c)
    assert rel_max_err(got[:, :N], want) <= tol, (M, N, K, ta, tb, epi, pad, use_bf16)
    assert np.all(got[:, N:] == 3.0)  # padding untouched


@pytest.mark.parametrize("case", range(CASES))
def test_random_attention(be, oracle, case):
    """Forward with lse and the backward, fp32 and bf16, random head dims
    (the flash, fp32-MFMA and generic kernels), masks and scales."""
    rng = np.random.default_rng(2000 + case)
    use_bf16 = case % 2 == 1
    B, H = int(rng.integers(1, 3)), int(rng.integers(1, 4))
    M, N = int(pick(rng, [1, 37, 128, 200, 300])), int(pick(rng, [1, 64, 129, 256, 300]))
    K = int(pick(rng, [64, 128, 128, 32, 96]))
    D = K if rng.integers(3) else int(pick(rng, [32, 64, 128]))
    causal = bool(rng.integers(2))
    scale = float(pick(rng, [1.0 / np.sqrt(K), 0.3, 0.05]))
    q = synth.normal((B, H, M, K), case, 0)
    k = synth.normal((B, H, N, K), case, 1)
    v = synth.normal((B, H, N, D), case, 2)
    dout = synth.normal((B, H, M, D), case, 3)
    torch = _torch()
    if use_bf16:
        (qd, q), (kd, k), (vd, v), (dod, dout) = bf16(q), bf16(k), bf16(v), bf16(dout)
        dt, tdt, tol = bwpp.DType.BF16, torch.bfloat16, BF16_TOL
    else:
        qd, kd, vd, dod = dev(q), dev(k), dev(v), dev(dout)
        dt, tdt, tol = bwpp.DType.F32, torch.float32, F32_TOL
    prm = bwpp.AttentionParams(M=M, N=N, K=K, D=D, ldq=K, ldk=K, ldv=D, ldo=D, batch=B, heads=H,
                               scale=scale, causal=int(causal), dtype=int(dt))
    o = torch.full((B, H, M, D), 3.0, dtype=tdt, device="cuda")
    lse = torch.empty((B, H, M), device="cuda")
    be.dispatch_attention_lse(qd, kd, vd, o, lse, prm)
    tag = (B, H, M, N, K, D, causal, scale, use_bf16)
    assert rel_max_err(host(o), oracle.attention_bh(q, k, v, scale, causal)) <= tol, tag
    lw = oracle.attention_lse(q, k, scale, causal)
    lg = host(lse)
    fin = np.isfinite(lw)
    assert np.array_equal(np.isfinite(lg), fin), tag
    assert np.max(np.abs(lg[fin] - lw[fin]), initial=0.0) <= 1e-4 * max(1.0, np.abs(lw[fin]).max(initial=0.0)), tag
    if K != D:
        return  # the backward takes K = D only on its matrix-core paths; the generic one is covered elsewhere
    dq, dk, dv = (torch.full_like(t, 7.0) for t in (qd, kd, vd))
    be.dispatch_attention_grad(qd, kd, vd, o, dod, lse, dq, dk, dv, prm)
    wq, wk, wv = oracle.attention_grad(q, k, v, dout, scale, causal)
    assert rel_max_err(host(dq), wq) <= tol, tag
    assert rel_max_err(host(dk), wk) <= tol, tag
    assert rel_max_err(host(dv), wv) <= tol, tag


@pytest.mark.parametrize("case", range(CASES))
def test_random_rowops(be, oracle, case):
    rng = np.random.default_rng(3000 + case)
    rows = int(pick(rng, [1, 7, 64, 333]))
    cols = int(pick(rng, [1, 3, 64, 100, 512, 1000, 4096, 5000, 16384]))
    ld = cols + int(pick(rng, [0, 0, 4, 3]))
    x = synth.normal((rows, ld), case, 0, 0.0, 2.0)
    g = synth.uniform((cols,), case, 1, 0.5, 1.5)
    bt = synth.normal((cols,), case, 2, 0.0, 0.1)
    torch = _torch()
    xd = dev(x)
    xc = np.ascontiguousarray(x[:, :cols])
    y = torch.full((rows, ld), 5.0, device="cuda")
    be.dispatch_softmax(xd, y, bwpp.SoftmaxParams(rows, cols, ld))
    got = host(y)
    assert rel_max_err(got[:, :cols], oracle.softmax(xc)) <= F32_TOL, (rows, cols, ld)
    assert np.all(got[:, cols:] == 5.0)
    be.dispatch_layernorm(xd, dev(g), dev(bt), y, bwpp.RmsnormParams(rows, cols, ld, 1e-5))
    assert rel_max_err(host(y)[:, :cols], oracle.layernorm(xc, g, bt, 1e-5)) <= F32_TOL, (rows, cols, ld)
    be.dispatch_rmsnorm(xd, dev(g), None, y, bwpp.RmsnormParams(rows, cols, ld, 1e-6))
    assert rel_max_err(host(y)[:, :cols], oracle.rmsnorm(xc, g, None, 1e-6)) <= F32_TOL, (rows, cols, ld)
    mv = torch.empty(rows, device="cuda")
    am = torch.empty(rows, dtype=torch.int32, device="cuda")
    be.dispatch_reduce_max(xd, mv, am, bwpp.ReduceParams(rows, cols, ld, 1))
    wv, wi = oracle.reduce_max(xc, 1)
    assert np.array_equal(host(mv).view(np.uint32), wv.view(np.uint32)), (rows, cols, ld)
    assert np.array_equal(host(am), wi), (rows, cols, ld)
