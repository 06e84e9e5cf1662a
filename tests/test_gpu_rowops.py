"""GPU parity of the row operators against the oracle, through the C ABI.

Bars: fp32 within 1e-4 relative max-norm
(max|gpu - cpu| / max|cpu|); reduce_max values, argmax indices, the
reference mask and both grads bit-exact.  Column counts are chosen to hit
every register-path configuration (full and partial) and the multi-pass
fallback; odd row counts leave partial blocks."""
import numpy as np
import pytest

import bwpp
from bwpp import synth
from conftest import assert_bits_equal, rel_max_err

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4

# cols -> default register config (VPT, WPR), f = full / p = partial:
# 200 (1,1)p, 256 (1,1)f, 300 (2,1)p, 512 (2,1)f, 1000 (1,4)p, 1024 (1,4)f,
# 2000 (2,4)p, 2048 (2,4)f, 4000 (4,4)p, 4096 (4,4)f, 5000 (8,4)p, 8192 (8,4)f,
# 10000 (16,4)p, 16384 (16,4)f, 20000 (16,8)p, 32768 (16,8)f, 32769 fallback;
# softmax uses 8 waves from 4096 columns (4096 (2,8)f, 5000 (4,8)p, ...).
COLS = [1, 3, 200, 256, 300, 512, 1000, 1024, 2000, 2048, 4000, 4096, 5000, 8192,
        10000, 16384, 20000, 32768, 32769]
# every (VPT, WPR) the library builds, in its kRowCfgs order
ROW_CFGS = [(1, 1), (2, 1), (4, 1), (8, 1), (16, 1), (2, 2), (4, 2), (8, 2), (1, 4),
            (2, 4), (4, 4), (8, 4), (16, 4), (2, 8), (4, 8), (8, 8), (16, 8)]


def _torch():
    import torch
    return torch


def dev(a):
    return _torch().from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch = _torch()
    torch.cuda.synchronize()
    return t.cpu().numpy()


def strided(x, ld):
    """Device buffer of shape [rows, ld] holding x in its first cols columns."""
    rows, cols = x.shape
    buf = np.full((rows, ld), 7.0, np.float32)
    buf[:, :cols] = x
    return dev(buf)


def _inputs(rows, cols, seed):
    x = synth.normal((rows, cols), seed, 0)
    g = synth.uniform((cols,), seed, 1, 0.5, 1.5)
    b = synth.normal((cols,), seed, 2, 0.0, 0.1)
    return x, g, b


@pytest.mark.parametrize("cols", COLS)
def test_softmax(be, oracle, cols):
    rows = 5
    x, _, _ = _inputs(rows, cols, cols)
    x *= 3
    y = dev(np.zeros_like(x))
    be.dispatch_softmax(dev(x), y, bwpp.SoftmaxParams(rows, cols, cols))
    assert rel_max_err(host(y), oracle.softmax(x)) <= FP32_TOL


@pytest.mark.parametrize("cols", COLS)
@pytest.mark.parametrize("op", ["rmsnorm", "layernorm"])
def test_norms(be, oracle, cols, op):
    rows = 9
    x, g, b = _inputs(rows, cols, 100 + cols)
    eps = 1e-6 if op == "rmsnorm" else 1e-5
    fn = be.dispatch_rmsnorm if op == "rmsnorm" else be.dispatch_layernorm
    ofn = oracle.rmsnorm if op == "rmsnorm" else oracle.layernorm
    for gg, bb in ((g, b), (g, None), (None, None)):
        y = dev(np.zeros_like(x))
        fn(dev(x), None if gg is None else dev(gg), None if bb is None else dev(bb), y,
           bwpp.RmsnormParams(rows, cols, cols, eps))
        assert rel_max_err(host(y), ofn(x, gg, bb, eps)) <= FP32_TOL, (gg is None, bb is None)


@pytest.mark.parametrize("ld_pad", [4, 1])  # 4: aligned rows (register path); 1: fallback
def test_strided_rows(be, oracle, ld_pad):
    rows, cols = 7, 1000
    ld = cols + ld_pad
    x, g, b = _inputs(rows, cols, 55)
    xd = strided(x, ld)
    y = strided(np.zeros_like(x), ld)
    be.dispatch_softmax(xd, y, bwpp.SoftmaxParams(rows, cols, ld))
    out = host(y)
    assert rel_max_err(out[:, :cols], oracle.softmax(x)) <= FP32_TOL
    assert np.all(out[:, cols:] == 7.0)  # padding untouched
    y = strided(np.zeros_like(x), ld)
    be.dispatch_rmsnorm(xd, dev(g), dev(b), y, bwpp.RmsnormParams(rows, cols, ld, 1e-6))
    assert rel_max_err(host(y)[:, :cols], oracle.rmsnorm(x, g, b, 1e-6)) <= FP32_TOL


def test_in_place(be, oracle):
    x, g, b = _inputs(6, 4096, 9)
    t = dev(x)
    be.dispatch_softmax(t, t, bwpp.SoftmaxParams(6, 4096, 4096))
    assert rel_max_err(host(t), oracle.softmax(x)) <= FP32_TOL
    t = dev(x)
    be.dispatch_layernorm(t, dev(g), dev(b), t, bwpp.RmsnormParams(6, 4096, 4096, 1e-5))
    assert rel_max_err(host(t), oracle.layernorm(x, g, b, 1e-5)) <= FP32_TOL


def test_softmax_special_values(be, oracle, golden):
    x = golden["softmax_special/x"]
    want = golden["softmax_special/y"]  # the reference's own outputs
    for cols_pad in (0, 4092):  # tiny row (register v1) and a 4096-wide row
        xx = np.full((x.shape[0], x.shape[1] + cols_pad), -np.inf, np.float32)
        xx[:, : x.shape[1]] = x
        y = dev(np.zeros_like(xx))
        be.dispatch_softmax(dev(xx), y, bwpp.SoftmaxParams(*xx.shape, xx.shape[1]))
        got = host(y)
        ref_full = oracle.softmax(xx)
        assert np.array_equal(np.isnan(got), np.isnan(ref_full))
        fin = ~np.isnan(ref_full)
        assert np.max(np.abs(got[fin] - ref_full[fin])) <= FP32_TOL
        if cols_pad == 0:
            assert np.array_equal(np.isnan(got), np.isnan(want))


def test_golden_row_vectors(be, golden):
    """GPU vs the reference's outputs stored in tests/golden."""
    for name in ("softmax_ramp", "softmax_seed"):
        x = golden[f"{name}/x"]
        y = dev(np.zeros_like(x))
        be.dispatch_softmax(dev(x), y, bwpp.SoftmaxParams(*x.shape, x.shape[1]))
        assert rel_max_err(host(y), golden[f"{name}/y"]) <= FP32_TOL, name
    for name in ("rmsnorm_ramp", "rmsnorm_seed_gb", "rmsnorm_seed_g", "rmsnorm_seed_none"):
        x = golden[f"{name}/x"]
        g = golden.get(f"{name}/gamma")
        b = golden.get(f"{name}/beta")
        y = dev(np.zeros_like(x))
        be.dispatch_rmsnorm(dev(x), None if g is None else dev(g), None if b is None else dev(b), y,
                            bwpp.RmsnormParams(*x.shape, x.shape[1], float(golden[f"{name}/eps"])))
        assert rel_max_err(host(y), golden[f"{name}/y"]) <= FP32_TOL, name


# (cols, {op: (float4 chunks per thread, waves per row)}) of the default
# layout choice: one wave per row up to 1024 columns (1536 for the norms
# and softmax), two up to 2048 (not softmax) and, for the norms, two waves
# of 8 chunks up to 3072; four beyond, eight for softmax and RMSNorm from
# 4096, LayerNorm above 4096 and the reduce_max gradient from 4096 to 8192.
LAYOUTS = [
    (1000, {"rmsnorm": (4, 1), "layernorm": (4, 1), "softmax": (4, 1), "max": (4, 1), "maxgrad": (4, 1)}),
    (1536, {"rmsnorm": (8, 1), "layernorm": (8, 1), "softmax": (8, 1), "max": (4, 2), "maxgrad": (4, 2)}),
    (2048, {"rmsnorm": (4, 2), "layernorm": (4, 2), "softmax": (2, 4), "max": (4, 2), "maxgrad": (4, 2)}),
    (3072, {"rmsnorm": (8, 2), "layernorm": (8, 2), "softmax": (4, 4), "max": (4, 4), "maxgrad": (4, 4)}),
    (4096, {"rmsnorm": (2, 8), "layernorm": (4, 4), "softmax": (2, 8), "max": (4, 4), "maxgrad": (2, 8)}),
    (8192, {"rmsnorm": (4, 8), "layernorm": (4, 8), "softmax": (4, 8), "max": (8, 4), "maxgrad": (4, 8)}),
    (16384, {"rmsnorm": (8, 8), "layernorm": (8, 8), "softmax": (8, 8), "max": (16, 4), "maxgrad": (16, 4)}),
]


@pytest.mark.parametrize("cols,want", LAYOUTS)
def test_default_layouts(be, oracle, cols, want):
    """The layout each operator gets by default (kernel name of the launch),
    with its result checked against the oracle."""
    torch = _torch()
    rows = 37
    x, g, b = _inputs(rows, cols, cols + 1)
    xd, y = dev(x), dev(np.zeros_like(x))
    full = lambda vw: "f" if 256 * vw[0] * vw[1] == cols else "p"
    name = lambda op, vw: f"bwpp_row_{op}_v{vw[0]}_w{vw[1]}_{full(vw)}"
    be.dispatch_rmsnorm(xd, dev(g), None, y, bwpp.RmsnormParams(rows, cols, cols, 1e-6))
    assert be.last_kernel == name("rmsnorm", want["rmsnorm"])
    assert rel_max_err(host(y), oracle.rmsnorm(x, g, None, 1e-6)) <= FP32_TOL
    be.dispatch_layernorm(xd, dev(g), dev(b), y, bwpp.RmsnormParams(rows, cols, cols, 1e-5))
    assert be.last_kernel == name("layernorm", want["layernorm"])
    assert rel_max_err(host(y), oracle.layernorm(x, g, b, 1e-5)) <= FP32_TOL
    be.dispatch_softmax(xd, y, bwpp.SoftmaxParams(rows, cols, cols))
    assert be.last_kernel == name("softmax", want["softmax"])
    assert rel_max_err(host(y), oracle.softmax(x)) <= FP32_TOL
    mv = torch.zeros(rows, dtype=torch.float32, device="cuda")
    ix = torch.zeros(rows, dtype=torch.int32, device="cuda")
    be.dispatch_reduce_max(xd, mv, ix, bwpp.ReduceParams(rows, cols, cols, 1))
    assert be.last_kernel == name("max", want["max"])
    wm, wi = oracle.reduce_max(x, 1)
    assert_bits_equal(host(mv), wm)
    assert np.array_equal(host(ix), wi)
    dy = np.random.default_rng(cols).standard_normal(rows).astype(np.float32)
    be.dispatch_reduce_max_grad_argmax(xd, None, dev(dy), y, bwpp.ReduceParams(rows, cols, cols, 1))
    assert be.last_kernel == name("maxgrad", want["maxgrad"])
    assert_bits_equal(host(y), oracle.reduce_max_grad(dy, x.shape, x=x, axis=1))


@pytest.mark.parametrize("idx", range(len(ROW_CFGS)))
@pytest.mark.parametrize("grid_cap", [0, 3])
def test_every_row_config(oracle, monkeypatch, idx, grid_cap):
    """Each register configuration, forced through BWPP_ROW_CFG, on a full and a
    partial row width; 13 rows leave partial blocks for the multi-row-per-block
    layouts, and a grid capped at 3 blocks (BWPP_ROW_GRID) makes every block
    loop over several row groups with the next group prefetched."""
    import torch
    vpt, wpr = ROW_CFGS[idx]
    cap = 256 * wpr * vpt
    monkeypatch.setenv("BWPP_ROW_CFG", str(idx))
    monkeypatch.setenv("BWPP_ROW_GRID", str(grid_cap))
    be = bwpp.HipBackend(0)
    be.set_stream(torch.cuda.current_stream())
    try:
        for cols in (cap, cap - 5):
            for rows in (13, 16, 32):
                x, g, b = _inputs(rows, cols, idx * 7 + cols + rows)
                xd = dev(x)
                y = dev(np.zeros_like(x))
                be.dispatch_softmax(xd, y, bwpp.SoftmaxParams(rows, cols, cols))
                assert rel_max_err(host(y), oracle.softmax(x)) <= FP32_TOL
                be.dispatch_layernorm(xd, dev(g), dev(b), y, bwpp.RmsnormParams(rows, cols, cols, 1e-5))
                assert rel_max_err(host(y), oracle.layernorm(x, g, b, 1e-5)) <= FP32_TOL
                mv = torch.zeros(rows, dtype=torch.float32, device="cuda")
                ix = torch.zeros(rows, dtype=torch.int32, device="cuda")
                be.dispatch_reduce_max(xd, mv, ix, bwpp.ReduceParams(rows, cols, cols, 1))
                wm, wi = oracle.reduce_max(x, 1)
                assert_bits_equal(host(mv), wm)
                assert np.array_equal(host(ix), wi)
    finally:
        be.close()


# ------------------------------------------------------------------ reduce_max
def _tie_matrix(rows, cols, seed):
    rng = np.random.default_rng(seed)
    x = rng.integers(-3, 4, (rows, cols)).astype(np.float32)
    if rows > 3:
        x[1] = -np.inf
        x[2] = np.nan
        x[3, ::2] = np.nan
    return x


@pytest.mark.parametrize("cols", [1, 5, 256, 300, 4096, 5000, 16384, 16385])
@pytest.mark.parametrize("kind", ["normal", "ties"])
def test_reduce_max_axis1(be, oracle, cols, kind):
    torch = _torch()
    rows = 9
    x = synth.normal((rows, cols), cols, 3) if kind == "normal" else _tie_matrix(rows, cols, cols)
    mv = torch.zeros(rows, dtype=torch.float32, device="cuda")
    ix = torch.zeros(rows, dtype=torch.int32, device="cuda")
    be.dispatch_reduce_max(dev(x), mv, ix, bwpp.ReduceParams(rows, cols, cols, 1))
    wm, wi = oracle.reduce_max(x, 1)
    assert_bits_equal(host(mv), wm)
    assert np.array_equal(host(ix), wi)


@pytest.mark.parametrize("rows,cols", [(1, 1), (9, 33), (300, 7), (64, 4096)])
def test_reduce_max_axis0(be, oracle, rows, cols):
    torch = _torch()
    x = _tie_matrix(rows, cols, rows + cols)
    mv = torch.zeros(cols, dtype=torch.float32, device="cuda")
    ix = torch.zeros(cols, dtype=torch.int32, device="cuda")
    be.dispatch_reduce_max(dev(x), mv, ix, bwpp.ReduceParams(rows, cols, cols, 0))
    wm, wi = oracle.reduce_max(x, 0)
    assert_bits_equal(host(mv), wm)
    assert np.array_equal(host(ix), wi)


def _signed_zero_rows(cols, seed):
    """Rows whose maximum is a zero reached with both signs: -0 first, +0
    first, the tie split across lanes, waves and the row's two halves, and a
    row of one lone -0 among negatives."""
    rng = np.random.default_rng(seed)
    rows = []
    for first, second in ((-0.0, 0.0), (0.0, -0.0)):
        for a, b in ((0, 1), (0, cols // 2), (cols // 3, cols - 1), (1, 64 % cols), (cols - 2, cols - 1)):
            if a == b or max(a, b) >= cols:
                continue
            r = -np.abs(rng.standard_normal(cols)).astype(np.float32) - 0.5
            r[a], r[b] = first, second
            rows.append(r)
    r = -np.abs(rng.standard_normal(cols)).astype(np.float32) - 0.5
    r[cols // 2] = -0.0
    rows.append(r)
    return np.ascontiguousarray(np.stack(rows), np.float32)


@pytest.mark.parametrize("cols", [2, 5, 256, 300, 1024, 2000, 4096, 5000, 16384, 32769])
def test_reduce_max_signed_zero_ties(be, oracle, cols):
    """A zero maximum keeps the sign of the first zero (the reference's strict
    fold, bwpp_cpu_ref.c:159-165): maxv bit-exact, argmax its index, along
    rows (register paths with one and several waves per row, the fallback)
    and along columns."""
    torch = _torch()
    x = _signed_zero_rows(cols, cols)
    rows = x.shape[0]
    for axis, xx in ((1, x), (0, np.ascontiguousarray(x.T))):
        r, c = xx.shape
        n = r if axis == 1 else c
        mv = torch.zeros(n, dtype=torch.float32, device="cuda")
        ix = torch.zeros(n, dtype=torch.int32, device="cuda")
        be.dispatch_reduce_max(dev(xx), mv, ix, bwpp.ReduceParams(r, c, c, axis))
        wm, wi = oracle.reduce_max(xx, axis)
        assert_bits_equal(host(mv), wm, f"axis {axis}")
        assert np.array_equal(host(ix), wi), f"axis {axis}"
    assert rows > 2


@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("rows,cols", [(2, 3), (17, 300), (8, 4096), (3, 16385)])
def test_reduce_max_mask_and_grads(be, oracle, axis, rows, cols):
    torch = _torch()
    x = _tie_matrix(rows, cols, 7 * rows + cols)
    n = cols if axis == 0 else rows
    dy = synth.normal((n,), 4, 4)
    p = bwpp.ReduceParams(rows, cols, cols, axis)
    # reference semantics: all-ties mask, dx = mask * dy
    mask = dev(np.zeros_like(x))
    be.dispatch_reduce_max_mask(dev(x), mask, p)
    want_mask = oracle.reduce_max_mask(x, axis)
    assert_bits_equal(host(mask), want_mask)
    dx = dev(np.zeros_like(x))
    be.dispatch_reduce_max_grad(mask, dev(dy), dx, p)
    assert_bits_equal(host(dx), oracle.reduce_max_grad_mask(want_mask, dy, axis))
    # one-hot to the lowest index, from x and from saved indices
    want = oracle.reduce_max_grad(dy, x.shape, x=x, axis=axis)
    dx = dev(np.full_like(x, 9.0))
    be.dispatch_reduce_max_grad_argmax(dev(x), None, dev(dy), dx, p)
    assert np.array_equal(host(dx), want)
    _, ix = oracle.reduce_max(x, axis)
    dx = dev(np.full_like(x, 9.0))
    be.dispatch_reduce_max_grad_argmax(None, torch.from_numpy(ix).cuda(), dev(dy), dx, p)
    assert np.array_equal(host(dx), want)


def test_reference_reduce_max_fixture(be, golden):
    """runtime/cpu/test_reduce_max.c fixture through the GPU."""
    x = golden["rmax_ramp_axis1/x"]
    p = bwpp.ReduceParams(2, 3, 3, 1)
    mask = dev(np.zeros_like(x))
    be.dispatch_reduce_max_mask(dev(x), mask, p)
    assert np.array_equal(host(mask), golden["rmax_ramp_axis1/mask"])
    dx = dev(np.zeros_like(x))
    be.dispatch_reduce_max_grad(mask, dev(golden["rmax_ramp_axis1/dy"]), dx, p)
    assert np.array_equal(host(dx), golden["rmax_ramp_axis1/dx"])


# ------------------------------------------------------------------ C2 size
def test_c2_full_size(be, oracle):
    """Config 2 at full size: X[8192 x 4096] ~ N(0,1), gamma ~ U[0.5,1.5],
    beta ~ N(0,0.1); all five operators."""
    torch = _torch()
    rows, cols = 8192, 4096
    x, g, b = _inputs(rows, cols, 0)
    xd, gd, bd = dev(x), dev(g), dev(b)
    y = torch.empty_like(xd)
    be.dispatch_softmax(xd, y, bwpp.SoftmaxParams(rows, cols, cols))
    assert rel_max_err(host(y), oracle.softmax(x)) <= FP32_TOL
    be.dispatch_layernorm(xd, gd, bd, y, bwpp.RmsnormParams(rows, cols, cols, 1e-5))
    assert rel_max_err(host(y), oracle.layernorm(x, g, b, 1e-5)) <= FP32_TOL
    be.dispatch_rmsnorm(xd, gd, None, y, bwpp.RmsnormParams(rows, cols, cols, 1e-6))
    assert rel_max_err(host(y), oracle.rmsnorm(x, g, None, 1e-6)) <= FP32_TOL
    mv = torch.empty(rows, dtype=torch.float32, device="cuda")
    ix = torch.empty(rows, dtype=torch.int32, device="cuda")
    be.dispatch_reduce_max(xd, mv, ix, bwpp.ReduceParams(rows, cols, cols, 1))
    wm, wi = oracle.reduce_max(x, 1)
    assert_bits_equal(host(mv), wm)
    assert np.array_equal(host(ix), wi)
    dy = synth.normal((rows,), 0, 3)
    be.dispatch_reduce_max_grad_argmax(xd, None, dev(dy), y, bwpp.ReduceParams(rows, cols, cols, 1))
    assert np.array_equal(host(y), oracle.reduce_max_grad(dy, x.shape, x=x, axis=1))


def test_invalid_arguments(be):
    x = dev(np.zeros((2, 4), np.float32))
    with pytest.raises(bwpp.BwppError) as e:
        be.dispatch_softmax(x, None, bwpp.SoftmaxParams(2, 4, 4))
    assert e.value.status == bwpp.Status.INVALID_ARG
    with pytest.raises(bwpp.BwppError) as e:
        be.dispatch_softmax(x, x, bwpp.SoftmaxParams(2, 4, 3))  # ld < cols
    assert e.value.status == bwpp.Status.INVALID_ARG
    with pytest.raises(bwpp.BwppError):
        be.dispatch_reduce_max(x, None, None, bwpp.ReduceParams(2, 4, 4, 1))
    be.dispatch_softmax(x, x, bwpp.SoftmaxParams(0, 4, 4))  # empty is a no-op


def test_arena(be):
    """Device arena mirrors runtime/core/arena.c: aligned bump, NULL on
    exhaustion, reset rewinds."""
    import ctypes
    lib = bwpp.load_library()
    arena = bwpp._lib.Arena()
    assert lib.bwpp_hip_arena_init(be._h, ctypes.byref(arena), 4096) == 0
    p1 = lib.bwpp_hip_arena_alloc(ctypes.byref(arena), 100, 256)
    p2 = lib.bwpp_hip_arena_alloc(ctypes.byref(arena), 100, 256)
    assert p1 % 256 == 0 and p2 % 256 == 0 and p2 - p1 == 256
    assert lib.bwpp_hip_arena_alloc(ctypes.byref(arena), 8192, 16) is None
    src = np.arange(25, dtype=np.float32)
    assert lib.bwpp_hip_copy_to_device(be._h, p1, src.ctypes.data, 100) == 0
    back = np.zeros(25, np.float32)
    assert lib.bwpp_hip_copy_to_host(be._h, back.ctypes.data, p1, 100) == 0
    assert np.array_equal(src, back)
    lib.bwpp_hip_arena_reset(ctypes.byref(arena))
    assert lib.bwpp_hip_arena_alloc(ctypes.byref(arena), 4096, 1) == arena.buffer
    lib.bwpp_hip_arena_destroy(ctypes.byref(arena))
    assert arena.buffer is None
