"""GPU parity of the fp32 matrix-core attention kernels (head dims 64 and
128: forward with lse, dQ and dK/dV passes) against the oracle.  fp32 bar:
1e-4 relative max-norm; lse 1e-4 absolute relative to max(1, |lse|).

Shapes cover partial 32-row tiles on both sides, M > N (causal rows that
see no key: O = 0, lse = -inf, dQ = 0), M < N, several slices, packed
projections read through strides (the layout of config 5's qkv buffer),
negative scales and the full config-5 shape (checked on two slices).
A head dim or layout the kernels do not take runs the generic kernel,
checked here too (d = 64 with a leading dimension that breaks 16-byte
rows)."""
import numpy as np
import pytest

import bwpp
from bwpp import synth
from conftest import rel_max_err

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _torch():
    import torch
    return torch


def dev(x):
    return _torch().from_numpy(np.ascontiguousarray(x, np.float32)).cuda()


def host(t):
    _torch().cuda.synchronize()
    return t.cpu().numpy()


def _check_lse(got, want):
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin)
    assert np.array_equal(got[~fin], want[~fin])
    err = np.max(np.abs(got[fin] - want[fin]), initial=0.0)
    assert err <= TOL * max(1.0, np.abs(want[fin]).max(initial=0.0))


def _run_all(be, q, k, v, dout, scale, causal, prm):
    torch = _torch()
    B, H, M = q.shape[:3]
    D = v.shape[3]
    qd, kd, vd, dod = dev(q), dev(k), dev(v), dev(dout)
    o = torch.full((B, H, M, D), 5.0, device="cuda")
    lse = torch.full((B, H, M), 5.0, device="cuda")
    be.dispatch_attention_lse(qd, kd, vd, o, lse, prm)
    o2 = torch.full((B, H, M, D), 5.0, device="cuda")
    be.dispatch_attention(qd, kd, vd, o2, prm)
    dq, dk, dv = (torch.full_like(t, 7.0) for t in (qd, kd, vd))
    be.dispatch_attention_grad(qd, kd, vd, o, dod, lse, dq, dk, dv, prm)
    return host(o), host(o2), host(lse), host(dq), host(dk), host(dv)


@pytest.mark.parametrize("B,H,M,N,D", [
    (1, 1, 1, 1, 64), (1, 1, 31, 33, 64), (2, 3, 64, 64, 64), (1, 2, 97, 200, 64), (1, 1, 200, 97, 64),
    (1, 1, 130, 130, 128), (2, 1, 65, 190, 128), (1, 1, 190, 65, 128)])
@pytest.mark.parametrize("causal", [False, True])
def test_mfma_f32_fwd_bwd(be, oracle, B, H, M, N, D, causal):
    seed = B * 1000 + M * 7 + N
    q = synth.normal((B, H, M, D), seed, 0)
    k = synth.normal((B, H, N, D), seed, 1)
    v = synth.normal((B, H, N, D), seed, 2)
    dout = synth.normal((B, H, M, D), seed, 3)
    scale = 1.0 / np.sqrt(D)
    prm = bwpp.AttentionParams(M=M, N=N, K=D, D=D, ldq=D, ldk=D, ldv=D, ldo=D, batch=B, heads=H,
                               scale=scale, causal=int(causal), dtype=int(bwpp.DType.F32))
    o, o2, lse, dq, dk, dv = _run_all(be, q, k, v, dout, scale, causal, prm)
    want = oracle.attention_bh(q, k, v, scale, causal)
    assert rel_max_err(o, want) <= TOL
    assert rel_max_err(o2, want) <= TOL
    _check_lse(lse, oracle.attention_lse(q, k, scale, causal))
    wq, wk, wv = oracle.attention_grad(q, k, v, dout, scale, causal)
    assert rel_max_err(dq, wq) <= TOL
    assert rel_max_err(dk, wk) <= TOL
    assert rel_max_err(dv, wv) <= TOL
    if causal and M > N:  # rows that see no key
        assert np.all(o[:, :, :M - N] == 0.0) and np.all(dq[:, :, :M - N] == 0.0)


@pytest.mark.parametrize("D", [64, 128])
def test_mfma_f32_causal_zigzag_order(be, oracle, monkeypatch, D):
    """Causal fp32 passes on a grid that is resident in one go at two blocks
    per CU (more blocks than CUs, at most twice as many: cus / 2 slices of
    four 128-row tiles), where the forward, dQ and dK/dV passes send their
    tiles out in zigzag order: the results equal the heaviest-first order
    (BWPP_ATTN_ZIGZAG=0) bit for bit, and one slice matches the oracle."""
    torch = _torch()
    cus = be.cus
    B, H, S = 2, max(1, cus // 4), 512
    seed = 77 + D
    q, k, v, dout = (synth.normal((B, H, S, D), seed, i) for i in range(4))
    scale = 1.0 / np.sqrt(D)
    prm = bwpp.AttentionParams(M=S, N=S, K=D, D=D, ldq=D, ldk=D, ldv=D, ldo=D, batch=B, heads=H,
                               scale=scale, causal=1, dtype=int(bwpp.DType.F32))
    outs = []
    for zz in ("1", "0"):
        monkeypatch.setenv("BWPP_ATTN_ZIGZAG", zz)
        b2 = bwpp.HipBackend(0)
        try:
            b2.set_stream(torch.cuda.current_stream())
            outs.append(_run_all(b2, q, k, v, dout, scale, True, prm))
        finally:
            b2.close()
    for a, b in zip(*outs):
        assert np.all(np.isfinite(a) | np.isneginf(a))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    o, _, lse, dq, dk, dv = outs[0]
    s1 = (slice(1, 2), slice(H - 1, H))
    want = oracle.attention_bh(q[s1], k[s1], v[s1], scale, True)
    assert rel_max_err(o[s1], want) <= TOL
    _check_lse(lse[s1], oracle.attention_lse(q[s1], k[s1], scale, True))
    wq, wk, wv = oracle.attention_grad(q[s1], k[s1], v[s1], dout[s1], scale, True)
    assert rel_max_err(dq[s1], wq) <= TOL
    assert rel_max_err(dk[s1], wk) <= TOL
    assert rel_max_err(dv[s1], wv) <= TOL


@pytest.mark.parametrize("B,H,M,N,D", [(1, 1, 1, 1, 64), (1, 1, 31, 33, 64), (2, 3, 64, 64, 64), (1, 2, 97, 200, 64),
                                       (1, 1, 200, 97, 64), (1, 1, 130, 130, 128), (2, 1, 65, 190, 128),
                                       (1, 1, 190, 65, 128), (1, 4, 512, 512, 64)])
@pytest.mark.parametrize("causal", [False, True])
def test_mfma_f32_grad_stored_ds_matches_recompute(monkeypatch, B, H, M, N, D, causal):
    """The stored-dS scheme of the fp32 passes (the dK/dV pass stores dS^T,
    the dQ pass multiplies it by K; the default) against the scheme that
    recomputes S and dP in the dQ pass (BWPP_ATTN_BWD_DS_MB=0): both form
    every dS the same way and feed the MFMAs the same operands in the same
    order, so dQ, dK, dV are equal (an all-zero sum may differ in the sign
    of zero only).  Ragged tiles on both sides, M > N causal (queries that
    see no key), both head dims; the last launch is checked to be the
    dQ = dS K pass."""
    torch = _torch()
    seed = 31 * B + M + 3 * N + D
    q, k, v, dout = (synth.normal(sh, seed, i) for i, sh in
                     enumerate([(B, H, M, D), (B, H, N, D), (B, H, N, D), (B, H, M, D)]))
    scale = 1.0 / np.sqrt(D)
    prm = bwpp.AttentionParams(M=M, N=N, K=D, D=D, ldq=D, ldk=D, ldv=D, ldo=D, batch=B, heads=H,
                               scale=scale, causal=int(causal), dtype=int(bwpp.DType.F32))
    cs = "_causal" if causal else ""
    outs = []
    for ds in (False, True):
        if ds:
            monkeypatch.delenv("BWPP_ATTN_BWD_DS_MB", raising=False)
        else:
            monkeypatch.setenv("BWPP_ATTN_BWD_DS_MB", "0")
        b2 = bwpp.HipBackend(0)
        try:
            b2.set_stream(torch.cuda.current_stream())
            outs.append(_run_all(b2, q, k, v, dout, scale, causal, prm))
            want = f"bwpp_attn_bwd_f32_mfma_d{D}{cs}_" + ("dq_ds" if ds else "dkdv")
            assert b2.last_kernel == want, b2.last_kernel
        finally:
            b2.close()
    for a, b in zip(outs[0][3:], outs[1][3:]):
        assert np.all(np.isfinite(a))
        assert np.array_equal(a, b)


@pytest.mark.parametrize("scale", [-0.3, 2.0])
def test_mfma_f32_scales(be, oracle, scale):
    B, H, M, N, D = 1, 2, 100, 140, 64
    q = synth.normal((B, H, M, D), 5, 0)
    k = synth.normal((B, H, N, D), 5, 1)
    v = synth.normal((B, H, N, D), 5, 2)
    dout = synth.normal((B, H, M, D), 5, 3)
    prm = bwpp.AttentionParams(M=M, N=N, K=D, D=D, ldq=D, ldk=D, ldv=D, ldo=D, batch=B, heads=H,
                               scale=scale, causal=1, dtype=int(bwpp.DType.F32))
    o, _, lse, dq, dk, dv = _run_all(be, q, k, v, dout, scale, True, prm)
    assert rel_max_err(o, oracle.attention_bh(q, k, v, scale, True)) <= TOL
    _check_lse(lse, oracle.attention_lse(q, k, scale, True))
    for got, want in zip((dq, dk, dv), oracle.attention_grad(q, k, v, dout, scale, True)):
        assert rel_max_err(got, want) <= TOL


def _packed(B, T, H, dh, seed):
    """qkv [B*T, 3*H*dh] and dout [B*T, H*dh] as config 5 lays them out."""
    D = H * dh
    qkv = synth.normal((B * T, 3 * D), seed, 0)
    dout = synth.normal((B * T, D), seed, 1)
    return qkv, dout


def _unpack(qkv, B, T, H, dh, part):
    D = H * dh
    x = qkv[:, part * D:(part + 1) * D].reshape(B, T, H, dh)
    return np.ascontiguousarray(x.transpose(0, 2, 1, 3))


@pytest.mark.parametrize("B,T,H,dh,ld_pad,check", [(2, 96, 3, 64, 0, None), (8, 512, 16, 64, 0, [(0, 0), (7, 15)]),
                                                   (1, 70, 2, 64, 1, None)])
def test_packed_views(be, oracle, B, T, H, dh, ld_pad, check):
    """Q, K, V as column blocks of one [B*T, 3*H*dh] buffer (head stride dh,
    batch stride T*ld), O / dO as [B*T, H*dh]; causal, scale 1/8.  ld_pad = 1
    makes rows 4-byte aligned only, so the generic kernel runs."""
    torch = _torch()
    D = H * dh
    qkv, dout = _packed(B, T, H, dh, B * T + H)
    ld = 3 * D + ld_pad
    buf = np.zeros((B * T, ld), np.float32)
    buf[:, :3 * D] = qkv
    dbuf = dev(buf)
    flat = dbuf.view(-1)
    qd, kd, vd = flat[0:], flat[D:], flat[2 * D:]
    ldo = D + ld_pad
    obuf = np.zeros((B * T, ldo), np.float32)
    obuf[:, :D] = dout
    dod = dev(obuf)
    o = torch.zeros((B * T, ldo), device="cuda")
    lse = torch.zeros((B, H, T), device="cuda")
    scale = 0.125
    prm = bwpp.AttentionParams(M=T, N=T, K=dh, D=dh, ldq=ld, ldk=ld, ldv=ld, ldo=ldo, batch=B, heads=H,
                               q_batch_stride=T * ld, q_head_stride=dh, k_batch_stride=T * ld, k_head_stride=dh,
                               v_batch_stride=T * ld, v_head_stride=dh, o_batch_stride=T * ldo, o_head_stride=dh,
                               scale=scale, causal=1, dtype=int(bwpp.DType.F32))
    be.dispatch_attention_lse(qd, kd, vd, o, lse, prm)
    # dQ / dK / dV take the strides of Q / K / V, each in a buffer of its own
    # (the public entry point rejects outputs whose byte ranges interleave).
    gbufs = [torch.zeros((B * T, ld), device="cuda") for _ in range(3)]
    be.dispatch_attention_grad(qd, kd, vd, o, dod, lse, *(gb.view(-1)[i * D:] for i, gb in enumerate(gbufs)), prm)
    q, k, v = (_unpack(qkv, B, T, H, dh, i) for i in range(3))
    g = np.ascontiguousarray(dout.reshape(B, T, H, dh).transpose(0, 2, 1, 3))
    oh = host(o)[:, :D].reshape(B, T, H, dh).transpose(0, 2, 1, 3)
    gq, gk, gv = (_unpack(host(gb), B, T, H, dh, i) for i, gb in enumerate(gbufs))
    for i, gb in enumerate(host(gb) for gb in gbufs):  # outside its column block: untouched
        rest = np.delete(gb, np.s_[i * D:(i + 1) * D], axis=1)
        assert np.all(rest == 0.0)
    lh = host(lse)
    for (b, h) in (check or [(b, h) for b in range(B) for h in range(H)]):
        sl = lambda t: t[b:b + 1, h:h + 1]
        assert rel_max_err(oh[b, h], oracle.attention_bh(sl(q), sl(k), sl(v), scale, True)[0, 0]) <= TOL
        _check_lse(lh[b, h], oracle.attention_lse(sl(q), sl(k), scale, True)[0, 0])
        wq, wk, wv = oracle.attention_grad(sl(q), sl(k), sl(v), sl(g), scale, True)
        assert rel_max_err(gq[b, h], wq[0, 0]) <= TOL
        assert rel_max_err(gk[b, h], wk[0, 0]) <= TOL
        assert rel_max_err(gv[b, h], wv[0, 0]) <= TOL


def _bf16_dev(x):
    torch = _torch()
    bits = synth.to_bf16_bits(np.ascontiguousarray(x, np.float32))
    return torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16), synth.bf16_bits_to_f32(bits)


def _bf16_host(t):
    torch = _torch()
    torch.cuda.synchronize()
    return synth.bf16_bits_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))


@pytest.mark.parametrize("B,H,M,N,D", [(1, 2, 97, 200, 64), (2, 1, 130, 130, 128), (1, 1, 190, 65, 128),
                                       (1, 2, 256, 256, 128), (1, 3, 160, 300, 128), (1, 1, 288, 100, 64)])
@pytest.mark.parametrize("causal", [False, True])
def test_bf16_grad_mfma(be, oracle, B, H, M, N, D, causal):
    """bf16 storage, head dim 64 / 128, 16-byte rows: the forward saves lse
    (the flash kernel at d = 128), the backward runs the bf16 matrix-core
    passes (bwpp_attn_bwd_bf16_mfma_*).  Bar 2e-2 against the oracle on the
    exact bf16 input values."""
    _bf16_grad_case(be, oracle, B, H, M, N, D, causal, D)


@pytest.mark.parametrize("B,H,M,N,D", [(1, 1, 1, 1, 128), (1, 2, 5, 3, 64), (2, 1, 3, 40, 128), (1, 1, 33, 2, 128)])
@pytest.mark.parametrize("causal", [False, True])
def test_bf16_grad_tiny(be, oracle, B, H, M, N, D, causal):
    """Shapes below one 32-row block: the tile loads re-read the last row
    for every row past the end (straight into LDS), which the passes must
    mask; M > N causal leaves queries that see no key (lse = -inf)."""
    _bf16_grad_case(be, oracle, B, H, M, N, D, causal, D)


@pytest.mark.parametrize("B,H,M,N,D", [(1, 2, 97, 200, 64), (1, 1, 130, 90, 128)])
@pytest.mark.parametrize("causal", [False, True])
def test_bf16_grad_padded_rows(be, oracle, B, H, M, N, D, causal):
    """Rows of D + 8 bf16 (16-byte aligned, padded): the bf16 matrix-core
    passes load through the row stride and leave the padding untouched."""
    _bf16_grad_case(be, oracle, B, H, M, N, D, causal, D + 8)


@pytest.mark.parametrize("B,H,M,N,D", [(1, 2, 97, 200, 64), (1, 1, 130, 90, 128)])
@pytest.mark.parametrize("causal", [False, True])
def test_bf16_grad_unaligned_rows(be, oracle, B, H, M, N, D, causal):
    """Rows of D + 4 bf16 (8-byte aligned only): the backward takes fp32
    copies through the fp32 matrix-core passes and rounds back to bf16."""
    _bf16_grad_case(be, oracle, B, H, M, N, D, causal, D + 4)


def _backend_with(monkeypatch, w8_mask, ds=True):
    """A backend with the 8-wave dK/dV pass allowed per w8_mask (bit 0
    unmasked, bit 1 causal) and the stored-dS scheme on or off."""
    monkeypatch.setenv("BWPP_ATTN_BWD_W8", str(w8_mask))
    if ds:
        monkeypatch.delenv("BWPP_ATTN_BWD_DS_MB", raising=False)
    else:
        monkeypatch.setenv("BWPP_ATTN_BWD_DS_MB", "0")
    be = bwpp.HipBackend(0)
    be.set_stream(_torch().cuda.current_stream())
    return be


W8_DKDV = "bwpp_attn_bwd_bf16_mfma_d128{}_dkdv_w8"
DQ_DS = "bwpp_attn_bwd_bf16_mfma_d128{}_dq_ds"


@pytest.mark.parametrize("M,N", [(40, 70), (70, 40)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("ds", [False, True])
def test_bf16_grad_8wave(oracle, monkeypatch, M, N, causal, ds):
    """d = 128 with one slice per CU: slices x ceil(N / 256) blocks give
    every CU one, so the runtime takes the 8-wave dK/dV pass (256 keys per
    block, V rows in LDS) -- checked against the oracle, with dS recomputed
    in the dQ pass (the launch checked to have been the 8-wave pass, the
    last one) and with dS stored (the last launch the dQ = dS K pass)."""
    be = _backend_with(monkeypatch, 3, ds)
    try:
        _bf16_grad_case(be, oracle, 1, be.cus, M, N, 128, causal, 128)
        assert be.last_kernel == (DQ_DS if ds else W8_DKDV).format("_causal" if causal else "")
    finally:
        be.close()


def _grad_variants(monkeypatch, B, H, M, N, D, causal, variants, seed=5):
    """dQ, dK, dV of one seeded bf16 problem from a backend per (w8_mask,
    ds) variant, with the last kernel each launched."""
    torch = _torch()
    gen = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(B, H, M, D, device="cuda", generator=gen).bfloat16()
    k = torch.randn(B, H, N, D, device="cuda", generator=gen).bfloat16()
    v = torch.randn(B, H, N, D, device="cuda", generator=gen).bfloat16()
    do = torch.randn(B, H, M, D, device="cuda", generator=gen).bfloat16()
    prm = bwpp.AttentionParams(M=M, N=N, K=D, D=D, ldq=D, ldk=D, ldv=D, ldo=D, batch=B, heads=H,
                               scale=D ** -0.5, causal=int(causal), dtype=int(bwpp.DType.BF16))
    outs = []
    for mask, ds in variants:
        be = _backend_with(monkeypatch, mask, ds)
        try:
            o = torch.empty_like(q)
            lse = torch.empty(B, H, M, device="cuda")
            be.dispatch_attention_lse(q, k, v, o, lse, prm)
            g = [torch.full_like(t, 7.0) for t in (q, k, v)]
            be.dispatch_attention_grad(q, k, v, o, do, lse, *g, prm)
            torch.cuda.synchronize()
            outs.append((g, be.last_kernel))
        finally:
            be.close()
    return outs


@pytest.mark.parametrize("causal", [False, True])
def test_bf16_grad_8wave_matches_4wave(monkeypatch, causal):
    """The 8-wave dK/dV pass against the 4-wave one (BWPP_ATTN_BWD_W8=0) at a
    shape with several 256-key blocks per slice, M < N and partial tiles,
    each with dS recomputed and with dS stored: all add the same 32-query
    blocks in the same order, so dQ, dK, dV are bit-identical."""
    be0 = _backend_with(monkeypatch, 3)
    cus = be0.cus
    be0.close()
    # ceil(1000 / 256) = 4 key blocks per slice: cus / 4 slices fill the chip.
    B, H, M, N, D = 1, max(1, cus // 4), 600, 1000, 128
    outs = _grad_variants(monkeypatch, B, H, M, N, D, causal, [(3, False), (0, False), (3, True), (0, True)])
    cs = "_causal" if causal else ""
    assert [kern for _, kern in outs] == [W8_DKDV.format(cs), f"bwpp_attn_bwd_bf16_mfma_d128{cs}_dkdv",
                                          DQ_DS.format(cs), DQ_DS.format(cs)]
    ref = outs[0][0]
    for g, _ in outs[1:]:
        for a, b in zip(ref, g):
            assert torch_isfinite_all(a)
            assert _torch().equal(a, b)


def torch_isfinite_all(t):
    return bool(_torch().isfinite(t.float()).all())


@pytest.mark.parametrize("B,H,M,N", [(1, 2, 97, 200), (2, 3, 130, 130), (1, 2, 190, 65), (1, 1, 1, 1),
                                     (1, 2, 33, 2), (2, 1, 3, 40), (1, 4, 512, 384), (1, 2, 300, 1000)])
@pytest.mark.parametrize("causal", [False, True])
def test_bf16_grad_stored_ds_matches_recompute(monkeypatch, B, H, M, N, causal):
    """The stored-dS scheme (dK/dV pass stores dS^T, the dQ pass multiplies
    it by K) against the two-pass scheme that recomputes S and dP in the dQ
    pass (BWPP_ATTN_BWD_DS_MB=0), head dim 128: ragged M and N (tiles past
    both ends, M > N causal with queries that see no key), 4-wave dK/dV
    blocks.  Both form every dS the same way and feed the MFMAs the same
    operands in the same order: dQ, dK, dV bit-identical (torch.equal; an
    all-zero sum may differ in the sign of zero only)."""
    outs = _grad_variants(monkeypatch, B, H, M, N, 128, causal, [(3, False), (3, True)], seed=11)
    cs = "_causal" if causal else ""
    assert outs[1][1] == DQ_DS.format(cs)
    assert outs[0][1] != DQ_DS.format(cs)
    for a, b in zip(outs[0][0], outs[1][0]):
        assert torch_isfinite_all(a)
        assert _torch().equal(a, b)


def test_bf16_grad_stored_ds_falls_back_when_device_memory_is_short(monkeypatch):
    """One slice of 400,000 queries and keys (d = 128): its stored dS would
    take ~320 GB, more than the device holds.  With the cap raised above
    that, the workspace allocation fails and the call recomputes S and dP
    instead of returning OUT_OF_MEMORY: the launches are the recompute
    scheme's and the results equal those with the scheme turned off."""
    torch = _torch()
    monkeypatch.setenv("BWPP_ATTN_BWD_DS_MB", str(1 << 30))
    B, H, S, D = 1, 1, 400_000, 128
    gen = torch.Generator(device="cuda").manual_seed(3)
    q, k, v, do = (torch.randn(B, H, S, D, device="cuda", generator=gen).bfloat16() for _ in range(4))
    prm = bwpp.AttentionParams(M=S, N=S, K=D, D=D, ldq=D, ldk=D, ldv=D, ldo=D, batch=B, heads=H,
                               scale=D ** -0.5, causal=1, dtype=int(bwpp.DType.BF16))
    outs = []
    for cap in (str(1 << 30), "0"):
        monkeypatch.setenv("BWPP_ATTN_BWD_DS_MB", cap)
        be = bwpp.HipBackend(0)
        try:
            be.set_stream(torch.cuda.current_stream())
            o = torch.empty_like(q)
            lse = torch.empty(B, H, S, device="cuda")
            be.dispatch_attention_lse(q, k, v, o, lse, prm)
            g = [torch.empty_like(t) for t in (q, k, v)]
            be.dispatch_attention_grad(q, k, v, o, do, lse, *g, prm)
            torch.cuda.synchronize()
            assert be.last_kernel == W8_DKDV.format("_causal"), be.last_kernel
            outs.append(g)
        finally:
            be.close()
    for a, b in zip(*outs):
        assert torch_isfinite_all(a)
        assert torch.equal(a, b)


@pytest.mark.parametrize("causal", [False, True])
def test_bf16_grad_c4_shape(be, oracle, causal):
    """Config 4's shape, the one the bench times: B8 H32 S2048 d128 bf16,
    scale 1/sqrt(128).  The forward saves lse through the flash kernel and
    the backward stores dS and ends with the dQ = dS K pass (both checked
    by kernel name);
    O and dQ, dK, dV of two (b, h) slices against the oracle on the exact
    bf16 inputs.  Bar 2e-2."""
    torch = _torch()
    B, H, S, D = 8, 32, 2048, 128
    cs = "_causal" if causal else ""
    bits = [synth.to_bf16_bits(synth.normal((B, H, S, D), 21, i)) for i in range(4)]
    q, k, v, do = (torch.from_numpy(b.view(np.int16)).cuda().view(torch.bfloat16) for b in bits)
    scale = D ** -0.5
    prm = bwpp.AttentionParams(M=S, N=S, K=D, D=D, ldq=D, ldk=D, ldv=D, ldo=D, batch=B, heads=H,
                               scale=scale, causal=int(causal), dtype=int(bwpp.DType.BF16))
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), device="cuda")
    be.dispatch_attention_lse(q, k, v, o, lse, prm)
    assert be.last_kernel == "bwpp_attn_bf16_d128" + (cs or "_p")
    dq, dk, dv = (torch.full_like(t, 7.0) for t in (q, k, v))
    be.dispatch_attention_grad(q, k, v, o, do, lse, dq, dk, dv, prm)
    assert be.last_kernel == DQ_DS.format(cs)
    torch.cuda.synchronize()
    for b, h in ((0, 0), (B - 1, H - 1)):
        qs, ks, vs, dos = (synth.bf16_bits_to_f32(np.ascontiguousarray(x[b:b + 1, h:h + 1])) for x in bits)
        assert rel_max_err(_bf16_host(o[b:b + 1, h:h + 1]), oracle.attention_bh(qs, ks, vs, scale, causal)) <= 2e-2
        for got, want in zip((dq, dk, dv), oracle.attention_grad(qs, ks, vs, dos, scale, causal)):
            assert rel_max_err(_bf16_host(got[b:b + 1, h:h + 1]), want) <= 2e-2, (b, h)


def _bf16_grad_case(be, oracle, B, H, M, N, D, causal, ld):
    torch = _torch()
    seed = B * 100 + M + N
    shapes = [(B, H, M, D), (B, H, N, D), (B, H, N, D), (B, H, M, D)]
    vals = [synth.bf16_bits_to_f32(synth.to_bf16_bits(synth.normal(s, seed, i))) for i, s in enumerate(shapes)]
    q, k, v, dout = vals

    def dev(x, rows):
        # [B, H, rows, ld] bf16 with the values in the first D columns.
        full = np.zeros((B, H, rows, ld), np.float32)
        full[..., :D] = x
        return _bf16_dev(full)[0]

    qd, kd, vd, dod = dev(q, M), dev(k, N), dev(v, N), dev(dout, M)
    scale = 1.0 / np.sqrt(D)
    prm = bwpp.AttentionParams(M=M, N=N, K=D, D=D, ldq=ld, ldk=ld, ldv=ld, ldo=ld, batch=B, heads=H,
                               q_batch_stride=H * M * ld, q_head_stride=M * ld, k_batch_stride=H * N * ld,
                               k_head_stride=N * ld, v_batch_stride=H * N * ld, v_head_stride=N * ld,
                               o_batch_stride=H * M * ld, o_head_stride=M * ld,
                               scale=scale, causal=int(causal), dtype=int(bwpp.DType.BF16))
    o = dev(np.zeros((B, H, M, D), np.float32), M)
    lse = torch.full((B, H, M), 5.0, device="cuda")
    be.dispatch_attention_lse(qd, kd, vd, o, lse, prm)
    _check_lse(host(lse), oracle.attention_lse(q, k, scale, causal))
    assert rel_max_err(_bf16_host(o)[..., :D], oracle.attention_bh(q, k, v, scale, causal)) <= 2e-2
    dq, dk, dv = (torch.full_like(t, 7.0) for t in (qd, kd, vd))
    be.dispatch_attention_grad(qd, kd, vd, o, dod, lse, dq, dk, dv, prm)
    for got, want in zip((dq, dk, dv), oracle.attention_grad(q, k, v, dout, scale, causal)):
        g = _bf16_host(got)
        assert rel_max_err(g[..., :D], want) <= 2e-2
        assert np.all(g[..., D:] == 7.0)  # padding columns untouched
