"""GPU parity of bwpp_hip_dispatch_matmul against the oracle (through the C ABI).

Bars: fp32 within 1e-4 relative max-norm; bf16 inputs
with fp32 accumulation within 2e-2.  bf16 inputs are rounded to bf16 first
and the oracle gets their exact fp32 values.  The full C3 shape is checked
against the oracle on a row subset (rows are independent, so those rows are
exact comparisons) and against torch's fp32 GEMM on every output."""
import numpy as np
import pytest

import bwpp
from bwpp import synth
from conftest import rel_max_err

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4
BF16_TOL = 2e-2
EPIS = [(0, False, False), (1, False, True), (2, True, False), (3, True, True)]  # (code, silu, add)


def _torch():
    import torch
    return torch


def f32_dev(x):
    return _torch().from_numpy(np.ascontiguousarray(x, np.float32)).cuda()


def bf16_dev(x):
    """Device bf16 tensor of x rounded to nearest even, and its exact fp32 value."""
    torch = _torch()
    bits = synth.to_bf16_bits(x)
    return torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16), synth.bf16_bits_to_f32(bits)


def bf16_host(t):
    torch = _torch()
    torch.cuda.synchronize()
    return synth.bf16_bits_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))


def f32_host(t):
    _torch().cuda.synchronize()
    return t.cpu().numpy()


def stored(x, trans):
    """Storage of logical matrix x: itself, or its transpose (row-major)."""
    return np.ascontiguousarray(x.T) if trans else x


def run(be, dtype, a, b, bias, M, N, K, epi, ta=0, tb=0):
    torch = _torch()
    dt = torch.bfloat16 if dtype == bwpp.DType.BF16 else torch.float32
    c = torch.full((M, N), 7.0, dtype=dt, device="cuda")
    be.dispatch_matmul(a, b, c, bias, bwpp.MatmulParams(M, N, K, 0, 0, N, int(dtype), epi, ta, tb))
    return c


def test_reference_ramp_fixture_f32(be, golden):
    """runtime/cpu/test_matmul.c fixture, all epilogues, vs the reference's outputs."""
    for tag in ("none", "add", "silu", "add_silu"):
        g = lambda k: golden[f"matmul_ramp4_{tag}/{k}"]
        epi = (2 if g("silu") else 0) | (1 if g("add") else 0)
        c = run(be, bwpp.DType.F32, f32_dev(g("a")), f32_dev(g("b")), f32_dev(g("bias")), 4, 4, 4, epi)
        assert rel_max_err(f32_host(c), g("c")) <= F32_TOL, tag
    for tag in ("none", "add_silu"):
        g = lambda k: golden[f"matmul_seed_{tag}/{k}"]
        M, K = g("a").shape
        N = g("b").shape[1]
        epi = (2 if g("silu") else 0) | (1 if g("add") else 0)
        c = run(be, bwpp.DType.F32, f32_dev(g("a")), f32_dev(g("b")), f32_dev(g("bias")), M, N, K, epi)
        assert rel_max_err(f32_host(c), g("c")) <= F32_TOL, tag


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (4, 4, 4), (17, 23, 29), (128, 128, 32), (256, 128, 96),
                                   (200, 300, 70), (384, 256, 512)])
@pytest.mark.parametrize("epi,silu,add", EPIS)
def test_f32_vs_oracle(be, oracle, M, N, K, epi, silu, add):
    a = synth.uniform((M, K), M + K, 0, -1, 1)
    b = synth.uniform((K, N), N + K, 1, -1, 1)
    bias = synth.uniform((N,), N, 2, -1, 1)
    c = run(be, bwpp.DType.F32, f32_dev(a), f32_dev(b), f32_dev(bias), M, N, K, epi)
    want = oracle.matmul(a, b, bias, apply_silu=silu, apply_bias=add)
    assert rel_max_err(f32_host(c), want) <= F32_TOL


@pytest.mark.parametrize("M,N,K", [(5, 7, 3), (64, 96, 40), (128, 256, 64), (300, 260, 100)])
@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("dtype", [bwpp.DType.F32, bwpp.DType.BF16])
def test_transposed_operands(be, oracle, M, N, K, ta, tb, dtype):
    """op(A) from a stored [K x M] and op(B) from a stored [N x K]: the GEMMs
    autodiff emits for matmul (graph_ir.c:1529-1583)."""
    a = synth.normal((M, K), 3, 0)
    b = synth.normal((K, N), 3, 1)
    if dtype == bwpp.DType.BF16:
        ad, a = bf16_dev(stored(a, ta))
        bd, b = bf16_dev(stored(b, tb))
        a = a.T.copy() if ta else a
        b = b.T.copy() if tb else b
        tol, host = BF16_TOL, bf16_host
    else:
        ad, bd = f32_dev(stored(a, ta)), f32_dev(stored(b, tb))
        tol, host = F32_TOL, f32_host
    c = run(be, dtype, ad, bd, None, M, N, K, 0, ta, tb)
    assert rel_max_err(host(c), oracle.matmul(a, b)) <= tol


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (7, 9, 13), (256, 256, 64), (512, 512, 512), (300, 520, 100),
                                   (256, 768, 1000), (64, 11008, 64)])
@pytest.mark.parametrize("epi,silu,add", EPIS)
def test_bf16_vs_oracle(be, oracle, M, N, K, epi, silu, add):
    ad, a = bf16_dev(synth.normal((M, K), 11, 0, 0.0, 0.5))
    bd, b = bf16_dev(synth.normal((K, N), 11, 1, 0.0, 0.5))
    biasd, bias = bf16_dev(synth.normal((N,), 11, 2, 0.0, 0.5))
    c = run(be, bwpp.DType.BF16, ad, bd, biasd, M, N, K, epi)
    want = oracle.matmul(a, b, bias, apply_silu=silu, apply_bias=add)
    assert rel_max_err(bf16_host(c), want) <= BF16_TOL


def test_bias_null_means_zero(be, oracle):
    ad, a = bf16_dev(synth.normal((256, 64), 5, 0))
    bd, b = bf16_dev(synth.normal((64, 256), 5, 1))
    c = run(be, bwpp.DType.BF16, ad, bd, None, 256, 256, 64, 3)  # ADD_SILU, no bias
    assert rel_max_err(bf16_host(c), oracle.matmul(a, b, None, apply_silu=True)) <= BF16_TOL


def test_zero_k_gives_epilogue_of_zero(be):
    torch = _torch()
    bias = f32_dev(np.array([1.0, -2.0, 0.5], np.float32))
    a = torch.zeros(1, dtype=torch.float32, device="cuda")
    c = run(be, bwpp.DType.F32, a, a, bias, 2, 3, 0, 3)
    x = np.array([1.0, -2.0, 0.5])
    want = np.tile(x / (1 + np.exp(-x)), (2, 1))
    assert np.allclose(f32_host(c), want, rtol=1e-5)


def test_alias_and_invalid(be):
    torch = _torch()
    a = torch.zeros((64, 64), dtype=torch.float32, device="cuda")
    b = torch.zeros((64, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(bwpp.BwppError) as e:
        be.dispatch_matmul(a, b, a, None, bwpp.MatmulParams(64, 64, 64, 64, 64, 64))
    assert e.value.status == bwpp.Status.ALIAS
    with pytest.raises(bwpp.BwppError) as e:
        be.dispatch_matmul(a, b, b[32:], None, bwpp.MatmulParams(32, 64, 64, 64, 64, 64))
    assert e.value.status == bwpp.Status.ALIAS
    c = torch.zeros((64, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(bwpp.BwppError) as e:
        be.dispatch_matmul(a, b, c, None, bwpp.MatmulParams(64, 64, 64, 64, 64, 64, 5))
    assert e.value.status == bwpp.Status.INVALID_ARG
    with pytest.raises(bwpp.BwppError) as e:
        be.dispatch_matmul(a, b, c, None, bwpp.MatmulParams(64, 64, 64, 32, 64, 64))
    assert e.value.status == bwpp.Status.INVALID_ARG


def test_c1_f32_256(be, oracle):
    """Config 1: fp32 C = A·B, M = N = K = 256, A, B ~ U[-1,1]."""
    a = synth.uniform((256, 256), 0, 0, -1, 1)
    b = synth.uniform((256, 256), 0, 1, -1, 1)
    c = run(be, bwpp.DType.F32, f32_dev(a), f32_dev(b), None, 256, 256, 256, 0)
    assert rel_max_err(f32_host(c), oracle.matmul(a, b)) <= F32_TOL


def test_c3_f32_2048(be, oracle):
    """Config 3 fp32 variant: SiLU(X·W + b) at M = N = K = 2048, U[-1,1]; all
    outputs vs torch fp32, the first 32 rows vs the oracle."""
    torch = _torch()
    n = 2048
    x = synth.uniform((n, n), 0, 0, -1, 1)
    w = synth.uniform((n, n), 0, 1, -1, 1)
    bias = synth.uniform((n,), 0, 2, -1, 1)
    xd, wd, bd = f32_dev(x), f32_dev(w), f32_dev(bias)
    c = run(be, bwpp.DType.F32, xd, wd, bd, n, n, n, 3)
    got = f32_host(c)
    torch.backends.cuda.matmul.allow_tf32 = False
    ref = torch.nn.functional.silu(xd @ wd + bd).cpu().numpy()
    assert rel_max_err(got, ref) <= F32_TOL
    want = oracle.matmul(x[:32], w, bias, apply_silu=True, apply_bias=True)
    assert rel_max_err(got[:32], want) <= F32_TOL


def test_c3_bf16_full(be, oracle):
    """Config 3: Y = SiLU(X·W + b), X [4096 x 4096], W [4096 x 11008],
    b [11008], bf16 ~ N(0, 0.02), fp32 accumulation, bf16 out."""
    torch = _torch()
    M, K, N = 4096, 4096, 11008
    xd, x = bf16_dev(synth.normal((M, K), 0, 0, 0.0, 0.02))
    wd, w = bf16_dev(synth.normal((K, N), 0, 1, 0.0, 0.02))
    bd, bias = bf16_dev(synth.normal((N,), 0, 2, 0.0, 0.02))
    c = run(be, bwpp.DType.BF16, xd, wd, bd, M, N, K, 3)
    got = bf16_host(c)
    ref = torch.nn.functional.silu(xd.float() @ wd.float() + bd.float()).cpu().numpy()
    assert rel_max_err(got, ref) <= BF16_TOL
    rows = np.r_[0:32, M - 32:M]
    want = oracle.matmul(x[rows], w, bias, apply_silu=True, apply_bias=True)
    assert rel_max_err(got[rows], want) <= BF16_TOL


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("waves", [4, 8])
def test_full_tile_kernels(oracle, monkeypatch, ta, tb, waves):
    """Both full-tile bf16 kernels (4 waves x 128x128, 8 waves x 128x64 per
    wave), every operand orientation, several K tiles of the stage ring."""
    torch = _torch()
    monkeypatch.setenv("BWPP_GEMM_WAVES", str(waves))
    be = bwpp.HipBackend(0)
    be.set_stream(torch.cuda.current_stream())
    try:
        M, N, K = 512, 256, 32 * 7
        a = synth.normal((M, K), 21, 0)
        b = synth.normal((K, N), 21, 1)
        bias = synth.normal((N,), 21, 2)
        ad, ah = bf16_dev(stored(a, ta))
        bd, bh = bf16_dev(stored(b, tb))
        biasd, biash = bf16_dev(bias)
        ah = ah.T.copy() if ta else ah
        bh = bh.T.copy() if tb else bh
        c = run(be, bwpp.DType.BF16, ad, bd, biasd, M, N, K, 3, ta, tb)
        want = oracle.matmul(ah, bh, biash, apply_silu=True, apply_bias=True)
        assert rel_max_err(bf16_host(c), want) <= BF16_TOL
    finally:
        be.close()


@pytest.mark.parametrize("tb", [0, 1])
@pytest.mark.parametrize("M,N,K", [(512, 768, 32 * 7), (256, 1000, 96), (768, 392, 32), (256, 11008, 64),
                                   (512, 384, 64)])
def test_wide_tile_kernels(oracle, monkeypatch, M, N, K, tb):
    """The 256 x 384 full-tile kernels (BWPP_GEMM_BN=384), both B
    orientations: N not a multiple of 384 (the last tile column overhangs N:
    B's last columns are re-read and only n < N stored), one and two K tiles
    (fewer than the ring's stages), and C3's column count.  Against the
    oracle; bit-identical to the 256 x 256 kernel where that one runs (each
    output takes the same MFMAs over K in the same order)."""
    torch = _torch()
    monkeypatch.setenv("BWPP_GEMM_BN", "384")
    be = bwpp.HipBackend(0)
    be.set_stream(torch.cuda.current_stream())
    ref_be = None
    try:
        a = synth.normal((M, K), 23, 0)
        b = synth.normal((K, N), 23, 1)
        bias = synth.normal((N,), 23, 2)
        ad, ah = bf16_dev(a)
        bd, bh = bf16_dev(stored(b, tb))
        biasd, biash = bf16_dev(bias)
        bh = bh.T.copy() if tb else bh
        c = run(be, bwpp.DType.BF16, ad, bd, biasd, M, N, K, 3, 0, tb)
        assert be.last_kernel == f"bwpp_gemm_bf16x384w8_t0{tb}_f", be.last_kernel
        got = bf16_host(c)
        want = oracle.matmul(ah, bh, biash, apply_silu=True, apply_bias=True)
        assert rel_max_err(got, want) <= BF16_TOL
        if N % 256 == 0:
            monkeypatch.setenv("BWPP_GEMM_BN", "256")
            ref_be = bwpp.HipBackend(0)
            ref_be.set_stream(torch.cuda.current_stream())
            c2 = run(ref_be, bwpp.DType.BF16, ad, bd, biasd, M, N, K, 3, 0, tb)
            assert ref_be.last_kernel == f"bwpp_gemm_bf16w8_t0{tb}_f", ref_be.last_kernel
            assert torch.equal(c.view(torch.int16), c2.view(torch.int16))
    finally:
        be.close()
        if ref_be is not None:
            ref_be.close()


@pytest.mark.parametrize("bn,M,N,K,ta,want", [
    ("", 512, 768, 64, 0, "bwpp_gemm_bf16w8_t00_f"),        # N a multiple of 256
    ("", 512, 1000, 64, 0, "bwpp_gemm_bf16x384w8_t00_f"),   # N a multiple of 8 only
    ("256", 512, 1000, 64, 0, "bwpp_gemm_bf16_t00_e"),      # wide tiles refused
    ("", 512, 1000, 64, 1, "bwpp_gemm_bf16_t10_e"),         # transposed A: no wide kernel
    ("", 512, 1004, 64, 0, "bwpp_gemm_bf16_t00_e"),         # N not a multiple of 8
    ("384", 512, 768, 64, 0, "bwpp_gemm_bf16x384w8_t00_f"), # asked for
])
def test_bf16_kernel_choice(oracle, monkeypatch, bn, M, N, K, ta, want):
    """Which bf16 kernel a shape takes (by name), with the result against the
    oracle."""
    torch = _torch()
    if bn:
        monkeypatch.setenv("BWPP_GEMM_BN", bn)
    else:
        monkeypatch.delenv("BWPP_GEMM_BN", raising=False)
    be = bwpp.HipBackend(0)
    be.set_stream(torch.cuda.current_stream())
    try:
        a = synth.normal((M, K), 29, 0)
        b = synth.normal((K, N), 29, 1)
        bias = synth.normal((N,), 29, 2)
        ad, ah = bf16_dev(stored(a, ta))
        bd, bh = bf16_dev(b)
        biasd, biash = bf16_dev(bias)
        ah = ah.T.copy() if ta else ah
        c = run(be, bwpp.DType.BF16, ad, bd, biasd, M, N, K, 3, ta, 0)
        assert be.last_kernel == want, be.last_kernel
        want_c = oracle.matmul(ah, bh, biash, apply_silu=True, apply_bias=True)
        assert rel_max_err(bf16_host(c), want_c) <= BF16_TOL
    finally:
        be.close()


@pytest.mark.parametrize("M,N,K,ta,tb", [(128, 128, 4096, 1, 0), (256, 384, 2048, 0, 0), (128, 256, 4000, 0, 1),
                                         (384, 128, 1056, 1, 1), (1024, 1024, 4096, 1, 0)])
@pytest.mark.parametrize("epi,silu,add", [(0, False, False), (3, True, True)])
def test_f32_split_k(be, oracle, M, N, K, ta, tb, epi, silu, add):
    """fp32 full tiles with fewer tiles than the chip holds and K >= 1024 run
    split-K (partial tiles, then an in-order reduce with the epilogue);
    K = 4000 and 1056 leave a shorter last range.  The same GEMM with
    split-K turned off must agree to the fp32 bar as well."""
    a = synth.uniform((M, K), M + K, 0, -1, 1)
    b = synth.uniform((K, N), M + K, 1, -1, 1)
    bias = synth.uniform((N,), M + K, 2, -1, 1)
    ad, bd = f32_dev(stored(a, ta)), f32_dev(stored(b, tb))
    c = run(be, bwpp.DType.F32, ad, bd, f32_dev(bias), M, N, K, epi, ta, tb)
    want = oracle.matmul(a, b, bias, apply_silu=silu, apply_bias=add)
    assert rel_max_err(f32_host(c), want) <= F32_TOL


def test_f32_split_k_off_matches(oracle, monkeypatch):
    torch = _torch()
    monkeypatch.setenv("BWPP_GEMM_SPLITK", "0")
    be = bwpp.HipBackend(0)
    be.set_stream(torch.cuda.current_stream())
    try:
        M, N, K = 256, 128, 2048
        a = synth.uniform((M, K), 3, 0, -1, 1)
        b = synth.uniform((K, N), 3, 1, -1, 1)
        c = run(be, bwpp.DType.F32, f32_dev(a), f32_dev(b), None, M, N, K, 0)
        assert rel_max_err(f32_host(c), oracle.matmul(a, b)) <= F32_TOL
    finally:
        be.close()


def test_f32_split_k_repeatable(be):
    """Split-K results do not depend on block timing: back-to-back launches
    of split-K GEMMs of different shapes, sharing the handle's workspace,
    each equal their first result bit for bit."""
    torch = _torch()
    shapes = [(1024, 1024, 4096, 1, 0), (128, 256, 4000, 0, 1), (256, 384, 2048, 0, 0)]
    devs = []
    for i, (M, N, K, ta, tb) in enumerate(shapes):
        a = synth.uniform((M, K), 50 + i, 0, -1, 1)
        b = synth.uniform((K, N), 50 + i, 1, -1, 1)
        bias = synth.uniform((N,), 50 + i, 2, -1, 1)
        devs.append((f32_dev(stored(a, ta)), f32_dev(stored(b, tb)), f32_dev(bias)))
    first = {}
    for rep in range(3):
        for i, (M, N, K, ta, tb) in enumerate(shapes):
            ad, bd, biasd = devs[i]
            c = run(be, bwpp.DType.F32, ad, bd, biasd, M, N, K, 3, ta, tb)
            torch.cuda.synchronize()
            if rep == 0:
                first[i] = c.clone()
            else:
                assert torch.equal(c, first[i]), (rep, shapes[i])


# ------------------------------------------------------------ fused tails
# (tail kind, bias epilogue): the SiLU-gradient tail (3) takes no epilogue.
_TAIL_CASES = [(1, False), (1, True), (2, False), (2, True), (3, False)]


@pytest.mark.parametrize("M,N,K", [(100, 70, 50), (256, 256, 128), (256, 128, 4096), (384, 256, 64)])
@pytest.mark.parametrize("kind,with_bias", _TAIL_CASES)
def test_fused_tails_f32(be, oracle, M, N, K, kind, with_bias):
    """bwpp_hip_dispatch_matmul_fused against the oracle's matmul followed
    by the op each tail replaces: residual add (bit-exact with the GEMM's
    own result: one fp32 rounding), SiLU gradient (the oracle's
    silu_grad), dual SiLU output.  Edge tiles (100 x 70), full tiles,
    split-K (K 4096 over 2 tiles) and an uneven tile count."""
    torch = _torch()
    a = synth.uniform((M, K), M + kind, 0, -1.0, 1.0)
    b = synth.uniform((K, N), N + kind, 1, -1.0, 1.0)
    bias = synth.uniform((N,), 3, 2, -1.0, 1.0)
    aux = synth.normal((M, N), 4, 3)
    epi = 1 if with_bias else 0
    want = oracle.matmul(a, b, bias if with_bias else None, apply_silu=False, apply_bias=with_bias)
    c = torch.full((M, N), 7.0, device="cuda")
    c2 = torch.full((M, N), 7.0, device="cuda")
    auxd = f32_dev(aux)
    be.dispatch_matmul_fused(f32_dev(a), f32_dev(b), c, f32_dev(bias) if with_bias else None,
                             auxd if kind != 2 else None, c2 if kind == 2 else None,
                             bwpp.MatmulParams(M, N, K, 0, 0, N, 0, epi, 0, 0), bwpp.FusionParams(kind, N, N))
    got = f32_host(c)
    if kind == 1:
        assert rel_max_err(got, np.add(want, aux, dtype=np.float32)) <= F32_TOL
    elif kind == 3:
        assert rel_max_err(got, oracle.silu_grad(aux, want).reshape(M, N)) <= F32_TOL
    else:
        assert rel_max_err(got, want) <= F32_TOL
        wd = want.astype(np.float64)
        assert rel_max_err(f32_host(c2), wd / (1.0 + np.exp(-wd))) <= F32_TOL


def test_fused_tails_errors(be):
    torch = _torch()
    x = torch.zeros((64, 64), device="cuda")
    y = torch.zeros((64, 64), device="cuda")
    p = bwpp.MatmulParams(64, 64, 64, 0, 0, 64, 0, 0, 0, 0)
    with pytest.raises(bwpp.BwppError):  # residual without aux
        be.dispatch_matmul_fused(x, x, y, None, None, None, p, bwpp.FusionParams(1, 0, 0))
    with pytest.raises(bwpp.BwppError):  # dual output without c2
        be.dispatch_matmul_fused(x, x, y, None, None, None, p, bwpp.FusionParams(2, 0, 0))
    with pytest.raises(bwpp.BwppError):  # c2 is C
        be.dispatch_matmul_fused(x, x, y, None, None, y, p, bwpp.FusionParams(2, 0, 0))
    with pytest.raises(bwpp.BwppError):  # SiLU-gradient tail after an epilogue
        be.dispatch_matmul_fused(x, x, y, x[0], x, None, bwpp.MatmulParams(64, 64, 64, 0, 0, 64, 0, 1, 0, 0),
                                 bwpp.FusionParams(3, 0, 0))
    with pytest.raises(bwpp.BwppError):  # bf16
        be.dispatch_matmul_fused(x, x, y, None, x, None, bwpp.MatmulParams(64, 64, 64, 0, 0, 64, 1, 0, 0, 0),
                                 bwpp.FusionParams(1, 0, 0))
    # residual in place (aux is C): C = A.B + C
    a = torch.eye(64, device="cuda")
    c = torch.full((64, 64), 2.0, device="cuda")
    be.dispatch_matmul_fused(a, a, c, None, c, None, p, bwpp.FusionParams(1, 64, 0))
    assert np.array_equal(f32_host(c), np.eye(64, dtype=np.float32) + 2.0)


@pytest.mark.parametrize("mode,family", [(0, "bwpp_gemm_f32_t"), (2, "bwpp_gemm_f32q_t"), (3, "bwpp_gemm_f32p_t")])
@pytest.mark.parametrize("split", [0, 1])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_f32_full_tile_kernels(oracle, monkeypatch, mode, family, split, ta, tb):
    """Each fp32 full-tile kernel forced through BWPP_GEMM_F32_PIPE (0 the
    register-staged one, 2 the 4-stage LDS-DMA ring, 3 the 2-stage ring),
    with split-K on (256 x 256 x 1024: four tiles, cut into K ranges) and
    off, for every transpose pair, with bias + SiLU and with the residual
    tail, against the oracle.  K = 32 (one tile: prologue and drain only)
    and K = 96 (fewer tiles than ring stages) are included."""
    torch = _torch()
    monkeypatch.setenv("BWPP_GEMM_F32_PIPE", str(mode))
    monkeypatch.setenv("BWPP_GEMM_SPLITK", str(split))
    h = bwpp.HipBackend(0)
    try:
        h.set_stream(torch.cuda.current_stream())
        for M, N, K in [(256, 256, 1024), (384, 128, 32), (128, 512, 96), (256, 128, 160)]:
            a = synth.uniform((M, K), M + ta, 0, -1.0, 1.0)
            b = synth.uniform((K, N), N + tb, 1, -1.0, 1.0)
            bias = synth.uniform((N,), K, 2, -1.0, 1.0)
            ad = f32_dev(np.ascontiguousarray(a.T) if ta else a)
            bd = f32_dev(np.ascontiguousarray(b.T) if tb else b)
            c = torch.full((M, N), 7.0, device="cuda")
            h.dispatch_matmul(ad, bd, c, f32_dev(bias), bwpp.MatmulParams(M, N, K, 0, 0, N, 0, 3, ta, tb))
            kern = h.last_kernel
            want = oracle.matmul(a, b, bias, apply_silu=True, apply_bias=True)
            assert rel_max_err(f32_host(c), want) <= F32_TOL, (M, N, K, kern)
            if split and (M, N, K) == (256, 256, 1024):
                assert kern == "bwpp_gemm_f32_splitk_reduce", kern
            elif not split:
                assert kern.startswith(family) and kern.endswith("_f"), kern
            aux = synth.normal((M, N), M, 3)
            c.fill_(7.0)
            h.dispatch_matmul_fused(ad, bd, c, None, f32_dev(aux), None, bwpp.MatmulParams(M, N, K, 0, 0, N, 0, 0, ta, tb),
                                    bwpp.FusionParams(1, N, N))
            want = oracle.matmul(a, b, None, apply_silu=False, apply_bias=False)
            assert rel_max_err(f32_host(c), np.add(want, aux, dtype=np.float32)) <= F32_TOL, (M, N, K, kern)
    finally:
        h.close()


# (M, N, K, trans_a, trans_b, kernel the cost model picks on 256 CUs): the
# C5 block step's GEMM shapes; "split" = K cut into ranges (the launch ends
# with the split-K reduce).
C5_CHOICES = [
    (4096, 3072, 1024, 0, 0, "bwpp_gemm_f32p_t00_f"),   # q/k/v: 2-stage ring, last wave half full
    (4096, 1024, 1024, 0, 0, "bwpp_gemm_f32q_t00_f"),   # out-projection: one tile per CU
    (4096, 4096, 1024, 0, 1, "bwpp_gemm_f32p_t01_f"),
    (4096, 1024, 4096, 0, 0, "split"),
    (1024, 4096, 4096, 1, 0, "split"),
    (1024, 1024, 4096, 1, 0, "split"),
]


@pytest.mark.parametrize("M,N,K,ta,tb,want", C5_CHOICES)
def test_f32_kernel_choice_c5_shapes(be, M, N, K, ta, tb, want):
    """The fp32 kernel / split-K choice on the C5 step's GEMM shapes (checked
    by kernel name on a 256-CU part), with the result against a float64
    product of the same operands."""
    torch = _torch()
    gen = torch.Generator(device="cuda").manual_seed(M + N + K + ta)
    a = torch.rand((K, M) if ta else (M, K), device="cuda", generator=gen) - 0.5
    b = torch.rand((N, K) if tb else (K, N), device="cuda", generator=gen) - 0.5
    c = torch.full((M, N), 7.0, device="cuda")
    be.dispatch_matmul(a, b, c, None, bwpp.MatmulParams(M, N, K, a.shape[1], b.shape[1], N, 0, 0, ta, tb))
    kern = be.last_kernel
    if be.cus == 256:
        assert kern == ("bwpp_gemm_f32_splitk_reduce" if want == "split" else want), kern
    if kern == "bwpp_gemm_f32_splitk_reduce":  # the split GEMM itself launched just before
        first = be.recent_kernel(1)
        assert first.startswith("bwpp_gemm_f32") and first.endswith(f"_t{ta}{tb}_s"), first
    ad = (a.t() if ta else a).double()
    bd = (b.t() if tb else b).double()
    ref = ad @ bd
    err = ((c.double() - ref).abs().max() / ref.abs().max()).item()
    assert err <= 1e-5, (kern, err)

