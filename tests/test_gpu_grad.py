"""GPU parity of the autodiff grad ops and elementwise glue (C ABI) against
the oracle, whose closed forms are pinned by finite differences in
tests/test_oracle_closed_forms.py.  fp32 bar: 1e-4 relative max-norm; the
broadcast/elementwise ops are single roundings and must match bit for bit.
Shapes include config 5's ([4096 x 1024] activations, [65536 x 512]
attention probabilities)."""
import numpy as np
import pytest

import bwpp
from bwpp import synth
from conftest import assert_bits_equal, rel_max_err

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _torch():
    import torch
    return torch


def dev(a):
    return _torch().from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def host(t):
    _torch().cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("n", [1, 5, 12289, 4096 * 4096])
@pytest.mark.parametrize("offset", [0, 1])
def test_silu_grad(be, oracle, n, offset):
    torch = _torch()
    x = synth.normal((n,), n, 0, 0.0, 3.0)
    dy = synth.normal((n,), n, 1)
    xb = torch.zeros(n + 1, device="cuda")
    db = torch.zeros(n + 1, device="cuda")
    ob = torch.zeros(n + 1, device="cuda")
    xb[offset:offset + n] = dev(x)
    db[offset:offset + n] = dev(dy)
    be.dispatch_silu_grad(xb[offset:], db[offset:], ob[offset:], n)
    assert rel_max_err(host(ob)[offset:offset + n], oracle.silu_grad(x, dy)) <= TOL


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 7), (9, 4096), (8 * 16 * 512, 512)])
def test_softmax_grad(be, oracle, rows, cols):
    torch = _torch()
    y = oracle.softmax(synth.normal((rows, cols), cols, 0))
    dy = synth.normal((rows, cols), cols, 1)
    dx = torch.empty((rows, cols), device="cuda")
    be.dispatch_softmax_grad(dev(y), dev(dy), dx, bwpp.SoftmaxParams(rows, cols, cols))
    assert rel_max_err(host(dx), oracle.softmax_grad(y, dy)) <= TOL


# cols = 1 is excluded: there dx = inv * g * eps / (x^2 + eps) is pure
# cancellation and its relative error only measures rounding order.
@pytest.mark.parametrize("rows,cols", [(1, 8), (5, 33), (300, 1000), (4096, 1024)])
@pytest.mark.parametrize("with_gamma", [True, False])
def test_rmsnorm_grad(be, oracle, rows, cols, with_gamma):
    torch = _torch()
    x = synth.normal((rows, cols), rows + cols, 0)
    g = synth.uniform((cols,), cols, 1, 0.5, 1.5) if with_gamma else None
    dy = synth.normal((rows, cols), rows + cols, 2)
    dx = torch.empty((rows, cols), device="cuda")
    dg = torch.full((cols,), 9.0, device="cuda")
    db = torch.full((cols,), 9.0, device="cuda")
    be.dispatch_rmsnorm_grad(dev(x), None if g is None else dev(g), dev(dy), dx, dg, db,
                             bwpp.RmsnormParams(rows, cols, cols, 1e-5))
    wdx, wdg, wdb = oracle.rmsnorm_grad(x, g, dy, 1e-5)
    assert rel_max_err(host(dx), wdx) <= TOL
    assert rel_max_err(host(dg), wdg) <= TOL
    assert rel_max_err(host(db), wdb) <= TOL
    # dx alone (no column sums requested)
    dx2 = torch.empty((rows, cols), device="cuda")
    be.dispatch_rmsnorm_grad(dev(x), None if g is None else dev(g), dev(dy), dx2, None, None,
                             bwpp.RmsnormParams(rows, cols, cols, 1e-5))
    assert rel_max_err(host(dx2), wdx) <= TOL


@pytest.mark.parametrize("rows,cols,ld", [(3, 2048, 2048), (1029, 512, 516), (2, 256, 256), (7, 1996, 2000),
                                         (2049, 20, 24)])
def test_rmsnorm_grad_wave_rows(be, oracle, rows, cols, ld):
    """The wave-per-row kernel (16-byte rows, <= 2048 columns): row counts
    that leave blocks partly empty, padded rows, partial float4 lanes."""
    torch = _torch()
    x = synth.normal((rows, cols), rows, 0)
    g = synth.uniform((cols,), cols, 1, 0.5, 1.5)
    dy = synth.normal((rows, cols), rows, 2)
    pad = lambda a: np.pad(a, ((0, 0), (0, ld - cols)))
    dx = torch.full((rows, ld), 5.0, device="cuda")
    dg = torch.zeros(cols, device="cuda")
    db = torch.zeros(cols, device="cuda")
    be.dispatch_rmsnorm_grad(dev(pad(x)), dev(g), dev(pad(dy)), dx, dg, db, bwpp.RmsnormParams(rows, cols, ld, 1e-5))
    wdx, wdg, wdb = oracle.rmsnorm_grad(x, g, dy, 1e-5)
    out = host(dx)
    assert rel_max_err(out[:, :cols], wdx) <= TOL
    assert np.all(out[:, cols:] == 5.0)
    assert rel_max_err(host(dg), wdg) <= TOL
    assert rel_max_err(host(db), wdb) <= TOL


@pytest.mark.parametrize("rows,cols,ld", [(1029, 512, 516), (4096, 1024, 1024), (7, 3000, 3000), (5, 37, 37)])
def test_rmsnorm_grad_acc(be, oracle, rows, cols, ld):
    """dx = acc + rmsnorm_grad: bit for bit the separate rmsnorm_grad
    followed by the add (one fp32 rounding of each), on the wave-per-row
    kernel (16-byte rows <= 2048 columns) and the generic one (3000 and 37
    columns); acc may be dx itself (in place); the column sums are
    unchanged; padding is untouched."""
    torch = _torch()
    x = synth.normal((rows, cols), rows, 0)
    g = synth.uniform((cols,), cols, 1, 0.5, 1.5)
    dy = synth.normal((rows, cols), rows, 2)
    acc = synth.normal((rows, cols), rows, 3)
    pad = lambda a: np.pad(a, ((0, 0), (0, ld - cols)))
    prm = bwpp.RmsnormParams(rows, cols, ld, 1e-5)
    xd, gd, dyd, accd = dev(pad(x)), dev(g), dev(pad(dy)), dev(pad(acc))
    sep = torch.full((rows, ld), 5.0, device="cuda")
    dg0, db0 = torch.zeros(cols, device="cuda"), torch.zeros(cols, device="cuda")
    be.dispatch_rmsnorm_grad(xd, gd, dyd, sep, dg0, db0, prm)
    want = np.add(acc, host(sep)[:, :cols], dtype=np.float32)
    dx = torch.full((rows, ld), 5.0, device="cuda")
    dg, db = torch.zeros(cols, device="cuda"), torch.zeros(cols, device="cuda")
    be.dispatch_rmsnorm_grad_acc(xd, gd, dyd, accd, dx, dg, db, prm)
    out = host(dx)
    assert_bits_equal(out[:, :cols], want)
    assert np.all(out[:, cols:] == 5.0)
    assert_bits_equal(host(dg), host(dg0))
    assert_bits_equal(host(db), host(db0))
    wdx = oracle.rmsnorm_grad(x, g, dy, 1e-5)[0]
    assert rel_max_err(out[:, :cols], np.add(acc, wdx, dtype=np.float32)) <= TOL
    inplace = accd.clone()
    be.dispatch_rmsnorm_grad_acc(xd, gd, dyd, inplace, inplace, None, None, prm)
    assert_bits_equal(host(inplace)[:, :cols], want)


@pytest.mark.parametrize("rows,cols,ld", [(4096, 1024, 1024), (333, 100, 104), (7, 3, 3), (1, 5, 5), (5000, 37, 37)])
def test_mean_square(be, rows, cols, ld):
    """loss = s_l * sum(x^2) against an fp64 sum, dX = s_g * x bit for bit
    (one fp32 product), on the 16-byte path and the scalar one (odd
    columns); dX in place (= x); either output alone; NULL scales = 1."""
    torch = _torch()
    x = synth.normal((rows, cols), rows + cols, 0, 0.0, 2.0)
    n = rows * cols
    sl = torch.tensor([1.0 / n], device="cuda")
    sg = torch.tensor([2.0 / n], device="cuda")
    xd = dev(np.pad(x, ((0, 0), (0, ld - cols)), constant_values=7.0))
    prm = bwpp.MeanSquareParams(rows, cols, ld)
    loss = torch.full((1,), 9.0, device="cuda")
    dx = torch.full((rows, ld), 5.0, device="cuda")
    be.dispatch_mean_square(xd, sl, sg, loss, dx, prm)
    want = np.sum(x.astype(np.float64) ** 2) * np.float64(np.float32(1.0 / n))
    assert abs(float(host(loss)[0]) - want) <= 1e-5 * want
    out = host(dx)
    assert_bits_equal(out[:, :cols], x * np.float32(2.0 / n))
    assert np.all(out[:, cols:] == 5.0)
    l2 = torch.full((1,), 9.0, device="cuda")
    be.dispatch_mean_square(xd, None, None, l2, None, prm)  # loss alone, scales 1
    assert abs(float(host(l2)[0]) - np.sum(x.astype(np.float64) ** 2)) <= 1e-5 * np.sum(x.astype(np.float64) ** 2)
    inplace = xd.clone()
    be.dispatch_mean_square(inplace, None, sg, None, inplace, prm)  # dX alone, in place
    assert_bits_equal(host(inplace)[:, :cols], x * np.float32(2.0 / n))


def test_mean_square_errors(be):
    torch = _torch()
    x = torch.ones((8, 64), device="cuda")
    with pytest.raises(bwpp.BwppError):  # no output
        be.dispatch_mean_square(x, None, None, None, None, bwpp.MeanSquareParams(8, 64, 64))
    buf = torch.zeros((9, 64), device="cuda")
    with pytest.raises(bwpp.BwppError):  # dX overlaps X one row apart
        be.dispatch_mean_square(buf[:8], None, None, None, buf[1:], bwpp.MeanSquareParams(8, 64, 64))


def test_rmsnorm_grad_acc_alias(be):
    torch = _torch()
    buf = torch.zeros((9, 64), device="cuda")
    x = torch.ones((8, 64), device="cuda")
    with pytest.raises(bwpp.BwppError):  # acc overlaps dx one row apart
        be.dispatch_rmsnorm_grad_acc(x, None, x, buf[1:], buf[:8], None, None, bwpp.RmsnormParams(8, 64, 64, 1e-5))


@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 300), (4096, 1024), (1000, 3)])
@pytest.mark.parametrize("axis", [0, 1])
def test_reduce_sum(be, oracle, rows, cols, axis):
    torch = _torch()
    x = synth.normal((rows, cols), rows * cols, 0)
    out = torch.empty(cols if axis == 0 else rows, device="cuda")
    be.dispatch_reduce_sum(dev(x), out, bwpp.ReduceParams(rows, cols, cols, axis))
    assert rel_max_err(host(out), oracle.reduce_sum(x, axis)) <= TOL


@pytest.mark.parametrize("op", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("bmode", [0, 1, 2, 3])
@pytest.mark.parametrize("rows,cols,ld,shift", [(13, 70, 70, 0), (13, 72, 72, 0), (9, 1024, 1028, 0),
                                                (5, 72, 76, 1)])
def test_elementwise(be, op, bmode, rows, cols, ld, shift):
    """Scalar path (cols 70, or a / b / out one element off 16-byte
    alignment) and 128-bit path (cols and ld multiples of 4), padded rows
    left untouched."""
    torch = _torch()
    a = synth.normal((rows, ld), 1, 0)
    bshape = {0: (rows, ld), 1: (cols,), 2: (rows,), 3: (1,)}[bmode]
    b = synth.uniform(bshape, 2, 1, 0.5, 2.0)
    base = torch.full((rows * ld + shift,), 9.0, device="cuda")
    out = base[shift:].view(rows, ld)
    ad = torch.zeros(rows * ld + shift, device="cuda")
    ad[shift:] = dev(a).reshape(-1)
    bd = torch.zeros(b.size + shift, device="cuda")
    bd[shift:] = dev(b).reshape(-1)
    be.dispatch_elementwise(ad[shift:], bd[shift:], out, bwpp.ElementwiseParams(rows, cols, ld, op, bmode))
    bb = b[:, :cols] if bmode == 0 else b[None, :] if bmode == 1 else b[:, None] if bmode == 2 else b.reshape(1, 1)
    bb = np.broadcast_to(bb, (rows, cols)).astype(np.float32)
    aa = a[:, :cols]
    want = {0: aa + bb, 1: aa - bb, 2: aa * bb, 3: aa / bb, 4: bb}[op].astype(np.float32)
    got = host(out)
    assert_bits_equal(got[:, :cols], want)
    assert np.all(got[:, cols:] == 9.0)


@pytest.mark.parametrize("n", [1, 70, 4096 * 1024 + 3])
def test_elementwise_silu(be, n):
    """Op 5 (unary SiLU, the executor's forward activation when it is not
    fused into a GEMM) of the b operand: b / (1 + exp(-b)) in fp32 against float64; the GPU
    exp is not correctly rounded, so the bar is a few ulps, not bits."""
    x = synth.normal((1, n), n, 0, 0.0, 4.0)
    out = _torch().empty((1, n), device="cuda")
    be.dispatch_elementwise(None, dev(x), out, bwpp.ElementwiseParams(1, n, n, 5, 0))
    xd = x.astype(np.float64)
    assert rel_max_err(host(out), xd / (1.0 + np.exp(-xd))) <= 1e-6


def test_grad_invalid_args(be):
    torch = _torch()
    x = torch.zeros(8, device="cuda")
    with pytest.raises(bwpp.BwppError):
        be.dispatch_silu_grad(x, None, x, 8)
    with pytest.raises(bwpp.BwppError) as e:
        be.dispatch_elementwise(x, x, x, bwpp.ElementwiseParams(2, 4, 4, 9, 0))
    assert e.value.status == bwpp.Status.INVALID_ARG
    big = torch.zeros((2, 9000), device="cuda")
    with pytest.raises(bwpp.BwppError) as e:
        be.dispatch_rmsnorm_grad(big, None, big, big.clone(), torch.zeros(9000, device="cuda"), None,
                                 bwpp.RmsnormParams(2, 9000, 9000, 1e-5))
    assert e.value.status == bwpp.Status.UNSUPPORTED
