"""GPU parity of bwpp_hip_dispatch_attention against the oracle (C ABI).

The reference computes single-head, unscaled, unmasked fp32 attention
(runtime/cpu/bwpp_cpu_ref.c:92-144); the build adds batch x heads, a score
scale and a bottom-right aligned causal mask (oracle_attention_bh_f32).
Bars: fp32 1e-4 relative max-norm, bf16 inputs with fp32 softmax and
accumulation 2e-2.  bf16 inputs are rounded first; the oracle sees their
exact fp32 values.  d = 128 bf16 runs the MFMA flash kernel; everything
else the generic kernel."""
import numpy as np
import pytest

import bwpp
from bwpp import synth
from conftest import assert_bits_equal, rel_max_err

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4
BF16_TOL = 2e-2


def _torch():
    import torch
    return torch


def f32_dev(x):
    return _torch().from_numpy(np.ascontiguousarray(x, np.float32)).cuda()


def bf16_dev(x):
    torch = _torch()
    bits = synth.to_bf16_bits(np.ascontiguousarray(x, np.float32))
    return torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16), synth.bf16_bits_to_f32(bits)


def host(t):
    torch = _torch()
    torch.cuda.synchronize()
    if t.dtype == torch.bfloat16:
        return synth.bf16_bits_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))
    return t.cpu().numpy()


def params(B, H, M, N, K, D, scale, causal, dtype):
    return bwpp.AttentionParams(M=M, N=N, K=K, D=D, ldq=K, ldk=K, ldv=D, ldo=D, batch=B, heads=H,
                                scale=scale, causal=int(causal), dtype=int(dtype))


def run(be, q, k, v, B, H, M, N, K, D, scale, causal, dtype):
    torch = _torch()
    dt = torch.bfloat16 if dtype == bwpp.DType.BF16 else torch.float32
    o = torch.full((B, H, M, D), 3.0, dtype=dt, device="cuda")
    be.dispatch_attention(q, k, v, o, params(B, H, M, N, K, D, scale, causal, dtype))
    return o


def inputs(B, H, M, N, K, D, seed, bf16):
    q = synth.normal((B, H, M, K), seed, 0)
    k = synth.normal((B, H, N, K), seed, 1)
    v = synth.normal((B, H, N, D), seed, 2)
    if bf16:
        (qd, q), (kd, k), (vd, v) = bf16_dev(q), bf16_dev(k), bf16_dev(v)
    else:
        qd, kd, vd = f32_dev(q), f32_dev(k), f32_dev(v)
    return (qd, kd, vd), (q, k, v)


def test_reference_fixtures_f32(be, golden):
    """test_metal_parity.c:237-248 fixture and a seeded case, vs the
    reference's own outputs (scale 1, no mask, one head)."""
    for name in ("attention_ramp", "attention_seed"):
        q, k, v = (golden[f"{name}/{t}"] for t in "qkv")
        M, K = q.shape
        N, D = v.shape
        o = run(be, f32_dev(q), f32_dev(k), f32_dev(v), 1, 1, M, N, K, D, 0.0, False, bwpp.DType.F32)
        assert rel_max_err(host(o)[0, 0], golden[f"{name}/o"]) <= F32_TOL, name


@pytest.mark.parametrize("B,H,M,N,K,D", [(1, 1, 1, 1, 1, 1), (2, 3, 37, 37, 16, 24), (1, 2, 70, 130, 64, 64),
                                         (1, 1, 130, 70, 32, 8), (1, 1, 65, 200, 512, 100)])
@pytest.mark.parametrize("causal", [False, True])
def test_generic_f32(be, oracle, B, H, M, N, K, D, causal):
    (qd, kd, vd), (q, k, v) = inputs(B, H, M, N, K, D, M + N, False)
    scale = 1.0 / np.sqrt(K)
    o = run(be, qd, kd, vd, B, H, M, N, K, D, scale, causal, bwpp.DType.F32)
    assert rel_max_err(host(o), oracle.attention_bh(q, k, v, scale, causal)) <= F32_TOL


@pytest.mark.parametrize("B,H,M,N,D", [(1, 2, 100, 100, 64), (2, 1, 33, 90, 32)])
@pytest.mark.parametrize("causal", [False, True])
def test_generic_bf16(be, oracle, B, H, M, N, D, causal):
    (qd, kd, vd), (q, k, v) = inputs(B, H, M, N, D, D, 7, True)
    scale = 1.0 / np.sqrt(D)
    o = run(be, qd, kd, vd, B, H, M, N, D, D, scale, causal, bwpp.DType.BF16)
    assert rel_max_err(host(o), oracle.attention_bh(q, k, v, scale, causal)) <= BF16_TOL


@pytest.mark.parametrize("B,H,M,N", [(1, 2, 256, 256), (1, 1, 300, 300), (2, 2, 200, 513), (1, 1, 513, 200),
                                     (1, 1, 64, 1000), (1, 3, 1024, 1024), (1, 1, 1, 1),
                                     # odd query-tile count (causal blocks pair tiles 4+0, 3+1, 2 alone);
                                     # grids that are / are not multiples of the 8 XCDs
                                     (1, 5, 1280, 1280), (2, 4, 2048, 2048), (1, 1, 1100, 1300)])
@pytest.mark.parametrize("causal", [False, True])
def test_flash_bf16_d128(be, oracle, B, H, M, N, causal):
    (qd, kd, vd), (q, k, v) = inputs(B, H, M, N, 128, 128, B * 1000 + M + N, True)
    scale = 1.0 / np.sqrt(128)
    o = run(be, qd, kd, vd, B, H, M, N, 128, 128, scale, causal, bwpp.DType.BF16)
    assert rel_max_err(host(o), oracle.attention_bh(q, k, v, scale, causal)) <= BF16_TOL


@pytest.mark.parametrize("M,N", [(2048, 2048), (1000, 1300), (1300, 700), (1280, 1280)])
@pytest.mark.parametrize("causal", [False, True])
def test_flash_bf16_d128_persistent(oracle, monkeypatch, M, N, causal):
    """More items than CUs ((slice, query tile) items; causal: pairs of query
    tiles): the forward runs the persistent kernel (one block per CU working
    through its items, the next item's first K / V stage and Q rows
    requested during the current item's last key tile).  Against the
    one-block-per-item kernels (BWPP_ATTN_FLASH_PERSIST=0), O and lse are
    bit-identical -- with M and N not multiples of the 256-query / 128-key
    tiles, an item count that is not a multiple of the CU count, M > N causal
    (query tiles that see no key at all) and an odd tile count (a causal
    pair with one tile) -- and one slice matches the oracle."""
    torch = pytest.importorskip("torch")
    cs = "_causal" if causal else ""
    outs = []
    for persist in ("3", "0"):
        monkeypatch.setenv("BWPP_ATTN_FLASH_PERSIST", persist)
        b2 = bwpp.HipBackend(0)
        try:
            b2.set_stream(torch.cuda.current_stream())
            H = 2 * b2.cus + 3  # items = H * ceil(M / 256) (causal: pairs) > CUs, not a multiple of them
            (qd, kd, vd), (q, k, v) = inputs(1, H, M, N, 128, 128, M + 7 * N, True)
            prm = bwpp.AttentionParams(M=M, N=N, K=128, D=128, ldq=128, ldk=128, ldv=128, ldo=128, batch=1,
                                       heads=H, scale=128 ** -0.5, causal=int(causal), dtype=int(bwpp.DType.BF16))
            o = torch.full((1, H, M, 128), 3.0, device="cuda").to(torch.bfloat16)
            lse = torch.full((1, H, M), 3.0, device="cuda")
            b2.dispatch_attention_lse(qd, kd, vd, o, lse, prm)
            torch.cuda.synchronize()
            assert b2.last_kernel == "bwpp_attn_bf16_d128" + cs + ("_p" if persist == "3" else "")
            outs.append((o, lse, q, k, v, H))
        finally:
            b2.close()
    (o1, l1, q, k, v, H), (o0, l0, *_) = outs
    assert torch.equal(o1, o0) and torch.equal(l1, l0)
    h = H - 1
    got = host(o1[:, h:h + 1].contiguous())
    want = oracle.attention_bh(q[:, h:h + 1], k[:, h:h + 1], v[:, h:h + 1], 128 ** -0.5, causal)
    assert rel_max_err(got, want) <= BF16_TOL


def test_flash_unscaled_matches_reference_semantics(be, oracle):
    """scale 0 means 1 (the reference applies no scale)."""
    (qd, kd, vd), (q, k, v) = inputs(1, 1, 128, 192, 128, 128, 5, True)
    q2 = q * 0.1  # keep the unscaled scores in a sane range
    qd2, q2 = bf16_dev(q2)
    o = run(be, qd2, kd, vd, 1, 1, 128, 192, 128, 128, 0.0, False, bwpp.DType.BF16)
    assert rel_max_err(host(o), oracle.attention_bh(q2, k, v, 1.0, False)) <= BF16_TOL


@pytest.mark.parametrize("dtype", [bwpp.DType.BF16, bwpp.DType.F32])
def test_causal_first_row_is_first_value(be, dtype):
    """Causal, M == N: query 0 sees only key 0, so O[0] = V[0] exactly."""
    bf = dtype == bwpp.DType.BF16
    (qd, kd, vd), (q, k, v) = inputs(2, 2, 300, 300, 128, 128, 9, bf)
    o = run(be, qd, kd, vd, 2, 2, 300, 300, 128, 128, 0.0883883, True, dtype)
    assert_bits_equal(host(o)[:, :, 0, :], v[:, :, 0, :])


def test_alias_rejected(be):
    torch = _torch()
    x = torch.zeros((1, 1, 64, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(bwpp.BwppError) as e:
        be.dispatch_attention(x, x.clone(), x.clone(), x, params(1, 1, 64, 64, 128, 128, 0, 0, bwpp.DType.BF16))
    assert e.value.status == bwpp.Status.ALIAS


def _torch_attention(q, k, v, scale, causal):
    """fp32 math on the GPU (library matmuls), heads in chunks."""
    torch = _torch()
    B, H, M, _ = q.shape
    N = k.shape[2]
    out = torch.empty((B, H, M, v.shape[3]), dtype=torch.float32, device="cuda")
    mask = None
    if causal:
        mask = torch.arange(N, device="cuda")[None, :] > (torch.arange(M, device="cuda")[:, None] + (N - M))
    for b in range(B):
        for h0 in range(0, H, 8):
            qs = q[b, h0:h0 + 8].float().contiguous()
            ks = k[b, h0:h0 + 8].float().transpose(1, 2).contiguous()
            s = torch.matmul(qs, ks) * scale
            if mask is not None:
                s = s.masked_fill(mask, float("-inf"))
            out[b, h0:h0 + 8] = torch.matmul(torch.softmax(s, dim=-1), v[b, h0:h0 + 8].float().contiguous())
    return out


@pytest.mark.parametrize("causal", [False, True])
def test_c4_full(be, oracle, causal):
    """Config 4: B 8, H 32, S 2048, d 128, bf16 Q/K/V ~ N(0,1), scale
    1/sqrt(128).  Two (b, h) slices vs the oracle; every slice vs torch fp32."""
    torch = _torch()
    B, H, S, d = 8, 32, 2048, 128
    scale = 1.0 / np.sqrt(d)
    (qd, kd, vd), (q, k, v) = inputs(B, H, S, S, d, d, 0, True)
    o = run(be, qd, kd, vd, B, H, S, S, d, d, scale, causal, bwpp.DType.BF16)
    got = host(o)
    ref = _torch_attention(qd, kd, vd, scale, causal).cpu().numpy()
    assert rel_max_err(got, ref) <= BF16_TOL
    for b, h in ((0, 0), (7, 31)):
        want = oracle.attention_bh(q[b:b + 1, h:h + 1], k[b:b + 1, h:h + 1], v[b:b + 1, h:h + 1], scale, causal)
        assert rel_max_err(got[b:b + 1, h:h + 1], want) <= BF16_TOL
    del ref
    torch.cuda.empty_cache()


@pytest.mark.parametrize("growth", [0.05, -0.05])
@pytest.mark.parametrize("causal", [False, True])
def test_flash_running_max_moves(be, oracle, growth, causal):
    """Scores whose row maximum keeps rising (or falling) from tile to tile,
    so the running offset is raised many times (and the output rescaled)."""
    B, H, M, N, d = 1, 2, 256, 1024, 128
    q = synth.normal((B, H, M, d), 11, 0)
    k = synth.normal((B, H, N, d), 11, 1) * (1.0 + growth * np.arange(N, dtype=np.float32))[None, None, :, None]
    v = synth.normal((B, H, N, d), 11, 2)
    (qd, q), (kd, k), (vd, v) = bf16_dev(q), bf16_dev(k.astype(np.float32)), bf16_dev(v)
    o = run(be, qd, kd, vd, B, H, M, N, d, d, 0.5, causal, bwpp.DType.BF16)
    assert rel_max_err(host(o), oracle.attention_bh(q, k, v, 0.5, causal)) <= BF16_TOL


def test_negative_scale_d128(be, oracle):
    """A negative scale flips which score is largest; d = 128 bf16 with such
    a scale runs the generic kernel."""
    (qd, kd, vd), (q, k, v) = inputs(1, 2, 100, 300, 128, 128, 12, True)
    o = run(be, qd, kd, vd, 1, 2, 100, 300, 128, 128, -0.1, True, bwpp.DType.BF16)
    assert rel_max_err(host(o), oracle.attention_bh(q, k, v, -0.1, True)) <= BF16_TOL


# ------------------------------------------------------------- backward
@pytest.mark.parametrize("B,H,M,N,K,D", [(1, 1, 1, 1, 1, 1), (2, 3, 37, 37, 16, 24), (1, 2, 70, 130, 64, 64),
                                         (1, 1, 130, 70, 32, 8), (1, 2, 100, 100, 128, 128)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("bf16", [False, True])
def test_attention_grad(be, oracle, B, H, M, N, K, D, causal, bf16):
    """lse forward + backward vs the oracle's closed form (pinned by finite
    differences); fp32 bar 1e-4, bf16 storage 2e-2."""
    torch = _torch()
    (qd, kd, vd), (q, k, v) = inputs(B, H, M, N, K, D, M * 7 + N, bf16)
    dout = synth.normal((B, H, M, D), M + N, 3)
    dt = bwpp.DType.BF16 if bf16 else bwpp.DType.F32
    if bf16:
        dod, dout = bf16_dev(dout)
    else:
        dod = f32_dev(dout)
    scale = 1.0 / np.sqrt(K)
    tdt = torch.bfloat16 if bf16 else torch.float32
    o = torch.empty((B, H, M, D), dtype=tdt, device="cuda")
    lse = torch.empty((B, H, M), device="cuda")
    prm = params(B, H, M, N, K, D, scale, causal, dt)
    be.dispatch_attention_lse(qd, kd, vd, o, lse, prm)
    tol = BF16_TOL if bf16 else F32_TOL
    lse_want = oracle.attention_lse(q, k, scale, causal)
    fin = np.isfinite(lse_want)
    got_lse = host(lse)
    assert np.array_equal(np.isfinite(got_lse), fin)
    assert np.max(np.abs(got_lse[fin] - lse_want[fin]), initial=0.0) <= 1e-4 * max(1.0, np.abs(lse_want[fin]).max(initial=0.0))
    dq = torch.full_like(qd, 7.0)
    dk = torch.full_like(kd, 7.0)
    dv = torch.full_like(vd, 7.0)
    be.dispatch_attention_grad(qd, kd, vd, o, dod, lse, dq, dk, dv, prm)
    # The oracle differentiates the exact forward; feed it the same inputs.
    wq, wk, wv = oracle.attention_grad(q, k, v, dout, scale, causal)
    assert rel_max_err(host(dq), wq) <= tol
    assert rel_max_err(host(dk), wk) <= tol
    assert rel_max_err(host(dv), wv) <= tol


def test_attention_grad_alias_rejected(be):
    torch = _torch()
    x = torch.zeros((1, 1, 8, 16), device="cuda")
    lse = torch.zeros((1, 1, 8), device="cuda")
    p = params(1, 1, 8, 8, 16, 16, 0.0, False, bwpp.DType.F32)
    with pytest.raises(bwpp.BwppError) as e:
        be.dispatch_attention_grad(x, x.clone(), x.clone(), x.clone(), x.clone(), lse, x, x.clone(), x.clone(), p)
    assert e.value.status == bwpp.Status.ALIAS
