"""Pins for the oracle functions the reference does not implement
numerically: LayerNorm, scaled/causal batched attention, reduce_max with
argmax, the one-hot grad, the autodiff grad ops, reduce_sum, transposed
GEMMs and bf16 rounding.

Each is checked against something the mathematics fixes -- fp64 brute
force, central finite differences, invariants, reduction to the reference
at special cases, or a library routine -- chosen so that a dropped term, a
wrong sign or a transposed operand fails."""
import numpy as np
import pytest

from conftest import assert_bits_equal, rel_max_err


def _rng(s):
    return np.random.default_rng(s)


# ------------------------------------------------------------------ LayerNorm
def _layernorm64(x, g, b, eps):
    x = x.astype(np.float64)
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps)
    if g is not None:
        y = y * g
    if b is not None:
        y = y + b
    return y


@pytest.mark.parametrize("cols", [1, 2, 8, 100, 4096])
def test_layernorm_vs_fp64(oracle, cols):
    r = _rng(cols)
    x = r.normal(2.0, 3.0, (5, cols)).astype(np.float32)
    g = r.uniform(0.5, 1.5, cols).astype(np.float32)
    b = r.normal(0, 0.1, cols).astype(np.float32)
    for eps in (1e-5, 0.5):  # a large eps makes its placement under the sqrt matter
        y = oracle.layernorm(x, g, b, eps)
        assert rel_max_err(y, _layernorm64(x, g, b, eps)) < 2e-6


def test_layernorm_invariants(oracle):
    x = _rng(1).normal(5.0, 2.0, (7, 64)).astype(np.float32)
    y = oracle.layernorm(x, None, None, 1e-6).astype(np.float64)
    assert np.all(np.abs(y.mean(axis=1)) < 1e-5)
    assert np.all(np.abs(y.var(axis=1) - 1.0) < 1e-4)  # population variance


def test_layernorm_zero_mean_input_equals_rmsnorm_form(oracle):
    """Rows with exactly zero mean: LayerNorm and RMSNorm coincide."""
    x = np.array([[1.0, -1.0, 2.0, -2.0], [0.5, -0.25, -0.25, 0.0]], np.float32)
    assert_bits_equal(oracle.layernorm(x, None, None, 1e-5), oracle.rmsnorm(x, None, None, 1e-5))


# ------------------------------------------------------------------ attention
def _attention64(q, k, v, scale, causal):
    B, H, M, _ = q.shape
    N = k.shape[2]
    s = np.einsum("bhmk,bhnk->bhmn", q.astype(np.float64), k.astype(np.float64)) * scale
    if causal:
        m = np.arange(M)[:, None]
        n = np.arange(N)[None, :]
        s = np.where(n <= m + (N - M), s, -np.inf)
    mx = s.max(axis=-1, keepdims=True)
    with np.errstate(invalid="ignore"):
        p = np.exp(s - mx)
    p = np.nan_to_num(p)
    den = p.sum(axis=-1, keepdims=True)
    p = np.divide(p, den, out=np.zeros_like(p), where=den > 0)
    return np.einsum("bhmn,bhnd->bhmd", p, v.astype(np.float64))


@pytest.mark.parametrize("B,H,M,N,K,D", [(1, 1, 5, 5, 4, 3), (2, 3, 16, 16, 8, 8), (1, 2, 7, 19, 16, 5),
                                         (1, 1, 19, 7, 4, 4)])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_bh_vs_fp64(oracle, B, H, M, N, K, D, causal):
    r = _rng(B * H * M * N + K + D)
    q = r.normal(size=(B, H, M, K)).astype(np.float32)
    k = r.normal(size=(B, H, N, K)).astype(np.float32)
    v = r.normal(size=(B, H, N, D)).astype(np.float32)
    scale = 1.0 / np.sqrt(K)
    o = oracle.attention_bh(q, k, v, scale, causal)
    assert rel_max_err(o, _attention64(q, k, v, scale, causal)) < 1e-5


def test_attention_causal_first_row_is_first_value(oracle):
    """Causal, M == N: query 0 sees only key 0, so O[0] = V[0] exactly."""
    r = _rng(5)
    q, k, v = (r.normal(size=(2, 2, 9, 6)).astype(np.float32) for _ in range(3))
    o = oracle.attention_bh(q, k, v, 0.37, True)
    assert_bits_equal(o[:, :, 0, :], v[:, :, 0, :])


def test_attention_causal_rows_without_keys_are_zero(oracle):
    """M > N with bottom-right alignment: the first M - N rows see no key."""
    r = _rng(6)
    q = r.normal(size=(1, 1, 6, 4)).astype(np.float32)
    k = r.normal(size=(1, 1, 2, 4)).astype(np.float32)
    v = r.normal(size=(1, 1, 2, 3)).astype(np.float32)
    o = oracle.attention_bh(q, k, v, 1.0, True)
    assert np.all(o[0, 0, :4] == 0.0)
    assert_bits_equal(o[0, 0, 4], v[0, 0, 0])


def test_attention_scale_equals_prescaled_query(oracle):
    """scale*(q.k) == (2q).k when scale = 2 (exact: powers of two)."""
    r = _rng(8)
    q, k, v = (r.normal(size=(1, 1, 8, 4)).astype(np.float32) for _ in range(3))
    assert_bits_equal(oracle.attention_bh(q, k, v, 2.0, False), oracle.attention_bh(2 * q, k, v, 1.0, False))


# ------------------------------------------------------------------ reduce_max
def _max_brute(x, axis):
    lines = x.T if axis == 0 else x
    mv, ix = [], []
    for line in lines:
        m = -np.inf
        for t in line:
            if t > m:
                m = t
        idx = -1
        for i, t in enumerate(line):
            if t == m:
                idx = i
                break
        mv.append(m)
        ix.append(idx)
    return np.array(mv, np.float32), np.array(ix, np.int32)


@pytest.mark.parametrize("axis", [0, 1])
def test_reduce_max_vs_brute(oracle, axis):
    r = _rng(20 + axis)
    x = r.integers(-2, 3, (13, 11)).astype(np.float32)
    x[3] = np.nan
    x[5] = -np.inf
    x[:, 2] = np.nan
    mv, ix = oracle.reduce_max(x, axis)
    bm, bi = _max_brute(x, axis)
    assert_bits_equal(mv, bm)
    assert np.array_equal(ix, bi)


def test_reduce_max_tie_and_special_fixtures(oracle):
    x = np.array([[3, 1, 3, 2], [-np.inf] * 4, [np.nan] * 4, [-0.0, 0.0, -0.0, 0.0],
                  [0.0, -0.0, 1.0, 1.0], [np.nan, 2.0, np.nan, 2.0]], np.float32)
    mv, ix = oracle.reduce_max(x, 1)
    assert list(ix) == [0, 0, -1, 0, 2, 1]
    assert np.signbit(mv[3]) and mv[3] == 0.0  # first maximum's bits (-0.0)
    assert mv[1] == -np.inf and mv[2] == -np.inf


def test_reduce_max_argmax_is_first_reference_mask_hit(oracle):
    """argmax = lowest column where the reference's all-ties mask is 1."""
    x = _rng(9).integers(0, 3, (40, 9)).astype(np.float32)
    _, ix = oracle.reduce_max(x, 1)
    mask = oracle.reduce_max_mask(x, 1)
    assert np.array_equal(ix, mask.argmax(axis=1))


@pytest.mark.parametrize("axis", [0, 1])
def test_onehot_grad_equals_reference_grad_for_unique_maxima(oracle, axis):
    """With unique maxima (N(0,1) data) the one-hot grad is the reference's
    mask * dy (bwpp_cpu_ref.c:146-219)."""
    r = _rng(30 + axis)
    x = r.normal(size=(12, 10)).astype(np.float32)
    dy = r.normal(size=10 if axis == 0 else 12).astype(np.float32)
    want = oracle.reduce_max_grad_mask(oracle.reduce_max_mask(x, axis), dy, axis)
    got_x = oracle.reduce_max_grad(dy, x.shape, x=x, axis=axis)
    _, ix = oracle.reduce_max(x, axis)
    got_i = oracle.reduce_max_grad(dy, x.shape, argmax=ix, axis=axis)
    assert np.array_equal(got_x, want) and np.array_equal(got_i, want)


def test_onehot_grad_routes_ties_to_lowest(oracle):
    x = np.array([[1, 5, 5, 0], [2, 2, 2, 2]], np.float32)
    dx = oracle.reduce_max_grad(np.array([3.0, -1.0], np.float32), x.shape, x=x, axis=1)
    assert np.array_equal(dx, np.array([[0, 3, 0, 0], [-1, 0, 0, 0]], np.float32))


# ------------------------------------------------------------------ grad ops
def _fd(f, x, h=1e-6):
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        xp = x.copy()
        xm = x.copy()
        xp[i] += h
        xm[i] -= h
        g[i] = (f(xp) - f(xm)) / (2 * h)
    return g


def test_silu_grad_vs_finite_differences(oracle):
    x = np.linspace(-8, 8, 41).astype(np.float32)
    dy = _rng(1).normal(size=41).astype(np.float32)
    silu = lambda t: t / (1 + np.exp(-t))
    fd = np.array([(silu(np.float64(t) + 1e-6) - silu(np.float64(t) - 1e-6)) / 2e-6 for t in x]) * dy
    assert rel_max_err(oracle.silu_grad(x, dy), fd) < 1e-5


def test_softmax_grad_vs_finite_differences(oracle):
    r = _rng(2)
    x = r.normal(size=(3, 6))
    dy = r.normal(size=(3, 6))

    def sm(t):
        e = np.exp(t - t.max(axis=1, keepdims=True))
        return e / e.sum(axis=1, keepdims=True)

    fd = _fd(lambda t: float((sm(t) * dy).sum()), x)
    got = oracle.softmax_grad(sm(x).astype(np.float32), dy.astype(np.float32))
    assert rel_max_err(got, fd) < 1e-5


@pytest.mark.parametrize("use_gamma", [True, False])
def test_rmsnorm_grad_vs_finite_differences(oracle, use_gamma):
    r = _rng(3)
    x = r.normal(size=(4, 7))
    g = r.uniform(0.5, 1.5, 7) if use_gamma else None
    bt = r.normal(0, 0.1, 7)
    dy = r.normal(size=(4, 7))
    eps = 1e-2

    def rms(t, gg, bb):
        y = t / np.sqrt((t * t).mean(axis=1, keepdims=True) + eps)
        return (y * (gg if gg is not None else 1.0)) + bb

    fdx = _fd(lambda t: float((rms(t, g, bt) * dy).sum()), x)
    g0 = g if g is not None else np.ones(7)
    fdg = _fd(lambda t: float((rms(x, t, bt) * dy).sum()), g0)
    fdb = _fd(lambda t: float((rms(x, g, t) * dy).sum()), bt)
    dx, dg, db = oracle.rmsnorm_grad(x.astype(np.float32),
                                     None if g is None else g.astype(np.float32),
                                     dy.astype(np.float32), eps)
    assert rel_max_err(dx, fdx) < 1e-5
    assert rel_max_err(dg, fdg) < 1e-5
    assert rel_max_err(db, fdb) < 1e-5


def test_reduce_sum(oracle):
    x = _rng(4).normal(size=(9, 5)).astype(np.float32)
    assert rel_max_err(oracle.reduce_sum(x, 0), x.astype(np.float64).sum(0)) < 1e-6
    assert rel_max_err(oracle.reduce_sum(x, 1), x.astype(np.float64).sum(1)) < 1e-6


# ------------------------------------------------------------------ GEMM forms
@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0), (1, 1)])
def test_transposed_matmul(oracle, ta, tb):
    """op(A) from a stored transpose is the same operation sequence as the
    plain matmul of the explicit transpose (bit-identical), and matches fp64."""
    r = _rng(10 + 2 * ta + tb)
    a = r.normal(size=(6, 9)).astype(np.float32)  # logical [M=6, K=9]
    b = r.normal(size=(9, 4)).astype(np.float32)  # logical [K=9, N=4]
    sa = np.ascontiguousarray(a.T) if ta else a
    sb = np.ascontiguousarray(b.T) if tb else b
    c = oracle.matmul(sa, sb, trans_a=bool(ta), trans_b=bool(tb))
    assert_bits_equal(c, oracle.matmul(a, b))
    assert rel_max_err(c, a.astype(np.float64) @ b.astype(np.float64)) < 1e-6


# ------------------------------------------------------------------ bf16
def test_bf16_round_matches_torch(oracle):
    import torch
    r = _rng(11)
    vals = [r.normal(size=2000).astype(np.float32),
            np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-40, -1e-40,
                      1.0, 1.00390625, 1.01171875], np.float32)]
    # exact halfway cases with even and odd kept LSB
    bits = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x00008000, 0x7F7F8000], np.uint32)
    vals.append(bits.view(np.float32))
    x = np.concatenate(vals)
    got = oracle.round_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert_bits_equal(got, want)
    assert np.isnan(oracle.round_bf16(np.array([np.nan], np.float32)))[0]


# ------------------------------------------------------- attention backward
@pytest.mark.parametrize("B,H,M,N,K,D", [(1, 2, 5, 7, 4, 3), (1, 1, 7, 5, 3, 4), (2, 1, 6, 6, 5, 2)])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_grad_vs_finite_differences(oracle, B, H, M, N, K, D, causal):
    r = _rng(B * 100 + M * 10 + N + int(causal))
    q = r.normal(size=(B, H, M, K))
    k = r.normal(size=(B, H, N, K))
    v = r.normal(size=(B, H, N, D))
    dout = r.normal(size=(B, H, M, D))
    scale = 0.7
    loss = lambda qq, kk, vv: float((_attention64(qq, kk, vv, scale, causal) * dout).sum())
    fq = _fd(lambda t: loss(t, k, v), q)
    fk = _fd(lambda t: loss(q, t, v), k)
    fv = _fd(lambda t: loss(q, k, t), v)
    dq, dk, dv = oracle.attention_grad(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32),
                                       dout.astype(np.float32), scale, causal)
    assert rel_max_err(dq, fq) < 2e-5
    assert rel_max_err(dk, fk) < 2e-5
    assert rel_max_err(dv, fv) < 2e-5


@pytest.mark.parametrize("causal", [False, True])
def test_attention_lse_vs_fp64(oracle, causal):
    r = _rng(31)
    q = r.normal(size=(2, 2, 9, 8)).astype(np.float32)
    k = r.normal(size=(2, 2, 6, 8)).astype(np.float32)
    s = np.einsum("bhmk,bhnk->bhmn", q.astype(np.float64), k.astype(np.float64)) * 0.5
    if causal:
        s = np.where(np.arange(6)[None, :] <= np.arange(9)[:, None] + (6 - 9), s, -np.inf)
    with np.errstate(divide="ignore"):
        want = np.log(np.exp(s).sum(axis=-1))
    got = oracle.attention_lse(q, k, 0.5, causal)
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin)
    assert np.max(np.abs(got[fin] - want[fin])) < 1e-5
