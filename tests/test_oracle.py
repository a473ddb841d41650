"""Pin the CPU oracle before trusting it (CPU-only).

Each oracle function is checked against something independent of its own
formula: the closed forms in the reference's tests (same seeds and shapes),
brute-force simulations of the reference kernels on small inputs, finite
differences for every backward, and identities.  Each check is chosen so a
plausible slip (dropped term, wrong tie rule, wrong eps, transposed operand)
fails it.
"""

import math

import numpy as np
import pytest

from conftest import assert_close, rng
from oracle import activations as oa
from oracle import elementwise as oe
from oracle import gemm as og
from oracle import norms as on
from oracle import reductions as orr

# ---------------------------------------------------------------- reductions


def test_reduce_matches_reference_test_closed_forms():
    # reference tests/test_reductions.py:10-15
    a = rng(0).standard_normal((4, 5)).astype(np.float32)
    assert_close(orr.reduce(a), np.array([a.sum()], np.float32), atol=1e-5)
    assert_close(orr.reduce(a, axis=0), a.sum(axis=0), atol=1e-5)
    assert_close(orr.reduce(a, axis=1, keepdims=True), a.sum(axis=1, keepdims=True), atol=1e-5)
    assert_close(orr.reduce(a, axis=-1, mode=1), a.mean(axis=-1), atol=1e-5)
    assert_close(orr.reduce(a, axis=1, mode=2), (a.astype(np.float64) ** 2).sum(axis=1), atol=1e-5)


def _simulate_minmax_row(row, op):
    """Literal scalar simulation of reduce_minmax.wgsl for one output."""
    init = -1e38 if op == 0 else 1e38

    def better(c, cur):
        return c > cur if op == 0 else c < cur

    vals, idxs = [], []
    for t in range(256):
        bv, bi = np.float32(init), 0
        r = t
        while r < len(row):
            if better(row[r], bv):
                bv, bi = row[r], r
            r += 256
        vals.append(bv)
        idxs.append(bi)
    s = 128
    while s >= 1:
        for i in range(s):
            if better(vals[i + s], vals[i]):
                vals[i], idxs[i] = vals[i + s], idxs[i + s]
        s //= 2
    return vals[0], idxs[0]


def test_minmax_matches_reference_test():
    # reference tests/test_reductions.py:18-24
    a = rng(1).standard_normal((3, 4)).astype(np.float32)
    v, i = orr.minmax(a, axis=1, op=0)
    assert_close(v, a.max(axis=1))
    assert np.array_equal(i.astype(np.int64), a.argmax(axis=1))
    v2, _ = orr.minmax(a, axis=0, op=1)
    assert_close(v2, a.min(axis=0))


@pytest.mark.parametrize("op", [0, 1])
def test_minmax_tie_rule_brute_force(op):
    r = rng(7)
    cases = [
        np.where(np.arange(600) % 7 == 3, 5.0, 0.0),   # many ties across lanes and chunks
        np.array([0.0, 5.0, 5.0] + [0.0] * 10),        # lanes 1 and 2 tie: lane 2 wins
        np.full(300, -1e38),                            # never strictly better than init
        np.full(10, -np.inf),
        np.array([np.nan, 1.0, np.nan, 1.0]),
        r.integers(-2, 3, size=1000).astype(np.float64),
    ]
    for row in cases:
        row = (row if op == 0 else -row).astype(np.float32)
        ev, ei = _simulate_minmax_row(row, op)
        v, i = orr.minmax(row, axis=None, op=op)
        assert int(i[0]) == ei, (row[:8], int(i[0]), ei)
        assert np.float32(v[0]) == np.float32(ev)
    # the reference rule is not numpy's first occurrence
    _, i = orr.minmax(np.array([0.0, 5.0, 5.0], np.float32), axis=None, op=0)
    assert int(i[0]) == 2


def test_minmax_inner_axis_brute_force():
    x = rng(8).integers(0, 3, size=(3, 300, 4)).astype(np.float32)
    v, i = orr.minmax(x, axis=1, op=0)
    for o in range(3):
        for k in range(4):
            ev, ei = _simulate_minmax_row(x[o, :, k], 0)
            assert int(i[o, k]) == ei and v[o, k] == ev


def test_maxmin_backward_routes_to_index():
    x = rng(9).standard_normal((4, 6)).astype(np.float32)
    v, i = orr.minmax(x, axis=1, op=0)
    g = rng(10).standard_normal(4).astype(np.float32)
    d = orr.maxmin_backward(g, i, x.shape, axis=1)
    expect = np.zeros_like(x)
    expect[np.arange(4), x.argmax(axis=1)] = g
    assert np.array_equal(d, expect)


# ---------------------------------------------------------------- softmax / unary


def test_softmax_matches_reference_test_closed_form():
    # reference tests/test_activations.py:34-38
    a = rng(3).standard_normal((3, 5)).astype(np.float32)
    ref = np.exp(a) / np.exp(a).sum(axis=-1, keepdims=True)
    assert_close(oa.softmax(a, -1), ref, atol=1e-5)
    # along another axis, and shift invariance
    b = rng(4).standard_normal((4, 6, 3)).astype(np.float32)
    assert_close(oa.softmax(b, 1), oa.softmax(b + 100.0, 1), atol=1e-5)
    assert_close(oa.softmax(b, 1).sum(axis=1), np.ones((4, 3), np.float32), atol=1e-6)


def test_activations_match_reference_tests():
    # reference tests/test_activations.py:9-31
    a = rng(0).standard_normal((5, 7)).astype(np.float32)
    tanh_gelu = a * 0.5 * (1 + np.tanh(np.sqrt(2 / np.pi) * (a + 0.044715 * a ** 3)))
    assert_close(oa.gelu(a), tanh_gelu, atol=1e-3)
    assert_close(oa.sigmoid(a), 1 / (1 + np.exp(-a)), atol=1e-5)
    assert_close(oa.UNARY["relu"](a), np.maximum(a, 0))
    b = (rng(1).standard_normal((4, 6)) * 0.5).astype(np.float32)
    assert_close(oa.UNARY["sin"](b), np.sin(b), atol=1e-6)
    assert_close(oa.UNARY["cos"](b), np.cos(b), atol=1e-6)
    # clamps of the reference kernels
    assert oa.gelu(np.float32(11.0)) == np.float32(11.0)
    assert oa.gelu(np.float32(-11.0)) == 0.0
    assert oa.gelubackwards(np.float32(12.0)) == 1.0
    assert oa.sigmoid(np.float32(-1000.0)) > 0.0  # clamped at -88, not 0


@pytest.mark.parametrize("name,fwd", [("gelubackwards", "gelu"), ("selubackwards", "selu"),
                                      ("relubackwards", "relu"), ("sinback", "sin"),
                                      ("cosback", "cos")])
def test_local_derivatives_by_finite_differences(name, fwd):
    # h = 1e-3 keeps float32 output rounding (~1e-4 here) below the
    # tolerance while a wrong derivative constant is off by > 1e-2.
    x = np.linspace(-3.0, 3.0, 61) + 0.013  # avoid the kink of relu at 0
    h = 1e-3
    f = oa.UNARY[fwd]
    num = (f(x + h).astype(np.float64) - f(x - h)) / (2 * h)
    assert_close(oa.UNARY[name](x), num, rtol=2e-3, atol=2e-3)


def test_sigmoid_derivative_from_output():
    x = np.linspace(-4, 4, 17)
    y = oa.sigmoid(x)
    num = (oa.sigmoid(x + 1e-3).astype(np.float64) - oa.sigmoid(x - 1e-3)) / 2e-3
    assert_close(oa.sigmoidbackwards(y), num, rtol=1e-3, atol=1e-4)


# ---------------------------------------------------------------- norms


def test_layernorm_matches_reference_test():
    # reference tests/test_normalization.py:12-21
    x = rng(0).standard_normal((2, 3, 4)).astype(np.float32)
    y, mu, inv = on.meanvarnorm(x, np.ones(4), np.zeros(4), axis=-1)
    ref = (x - x.mean(axis=-1, keepdims=True)) / np.sqrt(x.var(axis=-1, keepdims=True) + 1e-5)
    assert_close(y, ref, atol=1e-4)
    assert_close(mu, x.mean(axis=-1))


def test_rmsnorm_matches_reference_test():
    # reference tests/test_normalization.py:24-30
    x = rng(1).standard_normal((2, 4)).astype(np.float32)
    y, r = on.rmsnorm(x, np.ones(4), axis=-1)
    ref = x / np.sqrt((x ** 2).mean(axis=-1, keepdims=True) + 1e-6)
    assert_close(y, ref, atol=1e-4)


def test_norm_zero_rules_and_row_cap():
    x = np.zeros((3, 8), np.float32)
    x[1] = rng(2).standard_normal(8)
    g = rng(3).standard_normal(8).astype(np.float32)
    b = rng(4).standard_normal(8).astype(np.float32)
    y, mu, inv = on.meanvarnorm(x, g, b)
    assert inv[0] == 0.0 and inv[2] == 0.0 and inv[1] > 0
    assert_close(y[0], b)  # zero-variance row: inv_std = 0 -> y = beta
    y2, r = on.rmsnorm(x, g)
    assert r[0] == 0.0 and np.all(y2[0] == 0.0)
    yc, _, ic = on.meanvarnorm(x, g, b, row_cap=2)
    assert np.all(yc[2] == 0.0) and ic[2] == 0.0 and np.array_equal(yc[:2], y[:2])


def _fd_grad(f, x, eps=1e-5):
    g = np.zeros_like(x, dtype=np.float64)
    flat = x.reshape(-1)
    for k in range(flat.size):
        old = flat[k]
        flat[k] = old + eps
        fp = f(x)
        flat[k] = old - eps
        fm = f(x)
        flat[k] = old
        g.reshape(-1)[k] = (fp - fm) / (2 * eps)
    return g


def test_layernorm_backward_by_finite_differences():
    r = rng(5)
    x = r.standard_normal((3, 6))
    g = r.standard_normal(6)
    b = r.standard_normal(6)
    dy = r.standard_normal((3, 6))

    def ln64(xx, gg=g, bb=b):
        mu = xx.mean(axis=-1, keepdims=True)
        var = (xx * xx).mean(axis=-1, keepdims=True) - mu * mu
        return (xx - mu) / np.sqrt(var + 1e-5) * gg + bb

    _, mu, inv = on.meanvarnorm(x.astype(np.float32), g, b)
    dx = on.meanvarnormdx(dy, x, g, mu, inv)
    num = _fd_grad(lambda xx: float((ln64(xx) * dy).sum()), x.copy())
    assert_close(dx, num, rtol=1e-3, atol=1e-4)
    dg, db = on.meanvarnormdg(dy, x, mu, inv)
    num_g = _fd_grad(lambda gg: float((ln64(x, gg=gg) * dy).sum()), g.copy())
    assert_close(dg, num_g, rtol=1e-3, atol=1e-4)
    assert_close(db, dy.sum(axis=0), atol=1e-5)


def test_rmsnorm_backward_by_finite_differences():
    r = rng(6)
    x = r.standard_normal((2, 5))
    g = r.standard_normal(5)
    dy = r.standard_normal((2, 5))

    def rms64(xx, gg=g):
        return xx / np.sqrt((xx * xx).mean(axis=-1, keepdims=True) + 1e-6) * gg

    _, irms = on.rmsnorm(x.astype(np.float32), g)
    dx = on.rmsnormdx(dy, x, g, irms)
    assert_close(dx, _fd_grad(lambda xx: float((rms64(xx) * dy).sum()), x.copy()),
                 rtol=1e-3, atol=1e-4)
    dg = on.rmsnormdg(dy, x, irms)
    assert_close(dg, _fd_grad(lambda gg: float((rms64(x, gg) * dy).sum()), g.copy()),
                 rtol=1e-3, atol=1e-4)


def test_layernorm_inner_axis_equals_transposed_last_axis():
    x = rng(11).standard_normal((2, 5, 3)).astype(np.float32)
    g = rng(12).standard_normal(5)
    b = rng(13).standard_normal(5)
    y, mu, inv = on.meanvarnorm(x, g, b, axis=1)
    yt, mut, invt = on.meanvarnorm(np.ascontiguousarray(x.transpose(0, 2, 1)), g, b, axis=-1)
    assert_close(y, yt.transpose(0, 2, 1), atol=1e-6)
    assert_close(mu, mut, atol=1e-6)


def test_batchnorm_statistics_and_backward():
    r = rng(14)
    x = r.standard_normal((4, 3, 2, 2))
    g = r.standard_normal(3)
    b = r.standard_normal(3)
    y, mu, inv, rm, rv = on.batchnorm(x, g, b, np.zeros(3), np.ones(3), training=True)
    assert_close(mu, x.mean(axis=(0, 2, 3)), atol=1e-6)
    assert_close(inv, 1 / np.sqrt(x.var(axis=(0, 2, 3)) + 1e-5), rtol=1e-5)
    assert_close(rm, 0.1 * x.mean(axis=(0, 2, 3)), atol=1e-6)
    assert_close(rv, 0.9 + 0.1 * x.var(axis=(0, 2, 3), ddof=1), atol=1e-6)
    ye, *_ = on.batchnorm(x, g, b, rm, rv, training=False)
    assert_close(ye, (x - rm.reshape(1, 3, 1, 1)) / np.sqrt(rv.reshape(1, 3, 1, 1) + 1e-5)
                 * g.reshape(1, 3, 1, 1) + b.reshape(1, 3, 1, 1), atol=1e-5)
    dy = r.standard_normal(x.shape)

    def bn64(xx):
        m = xx.mean(axis=(0, 2, 3), keepdims=True)
        v = xx.var(axis=(0, 2, 3), keepdims=True)
        return ((xx - m) / np.sqrt(v + 1e-5) * g.reshape(1, 3, 1, 1) + b.reshape(1, 3, 1, 1))

    dg, db = on.batchnormdg(dy, x, mu, inv)
    dx = on.batchnormdx(dy, x, g, dg, db, mu, inv)
    assert_close(dx, _fd_grad(lambda xx: float((bn64(xx) * dy).sum()), x.copy()),
                 rtol=1e-3, atol=1e-4)
    assert_close(db, dy.sum(axis=(0, 2, 3)), atol=1e-5)


# ---------------------------------------------------------------- GEMM


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_closed_form_and_fma_chain(ta, tb):
    r = rng(20)
    M, N, K = 7, 5, 9
    A = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    bias = r.standard_normal(N).astype(np.float32)
    c = og.matmul_add(A, B, bias, ta, tb)
    a = A.T if ta else A
    b = B.T if tb else B
    brute = np.array([[sum(float(a[i, k]) * float(b[k, j]) for k in range(K)) + bias[j]
                       for j in range(N)] for i in range(M)])
    assert_close(c, brute, atol=1e-5)
    cf = og.matmul_add_fma(A, B, bias, ta, tb)
    assert_close(cf, brute, rtol=1e-5, atol=1e-5)
    # the C oracle is the fma chain in ascending k, then one bias add
    for i in range(M):
        for j in range(N):
            acc = np.float32(0.0)
            for k in range(K):
                exact = np.float64(a[i, k]) * np.float64(b[k, j]) + np.float64(acc)
                acc = np.float32(exact)
            assert abs(float(cf[i, j]) - float(np.float32(acc + bias[j]))) <= 2 * np.spacing(
                np.float32(abs(cf[i, j]) + 1e-30)
            )


def test_gemm_batch_and_bias_modes():
    r = rng(21)
    A = r.standard_normal((3, 4, 6)).astype(np.float32)
    W = r.standard_normal((6, 5)).astype(np.float32)
    for bias in (None, r.standard_normal(5), r.standard_normal((4, 5)),
                 r.standard_normal((3, 4, 5))):
        c = og.matmul_add(A, W, bias)
        ref = np.einsum("bik,kj->bij", A.astype(np.float64), W.astype(np.float64))
        if bias is not None:
            ref = ref + bias
        assert_close(c, ref, atol=1e-5)
        assert_close(og.matmul_add_fma(A, W, None if bias is None else bias.astype(np.float32)),
                     ref, atol=1e-4)
    with pytest.raises(ValueError):
        og.matmul_add(A, r.standard_normal((2, 6, 5)))
    with pytest.raises(ValueError):
        og.matmul_add(A, W, r.standard_normal((5, 4)))


def test_gemm_fma_row_sample_is_rows_of_full():
    r = rng(22)
    A = r.standard_normal((64, 48)).astype(np.float32)
    B = r.standard_normal((48, 40)).astype(np.float32)
    full = og.matmul_add_fma(A, B)
    part = og.matmul_add_fma(A, B, rows=(8, 24))
    assert np.array_equal(part[8:24], full[8:24])
    assert np.all(part[:8] == 0) and np.all(part[24:] == 0)


# ---------------------------------------------------------------- elementwise


def test_pow_rules_match_reference_test():
    # reference tests/test_pointwise.py:33-68
    arr = np.array([[-2.0, -0.5, 0.5, 2.0], [0.25, 1.5, 3.0, 4.0]], np.float32)
    assert_close(oe.scalarpointwise(arr, 3, 3), arr ** 3, atol=1e-5)
    assert_close(oe.scalarpointwise(arr, -1, 3), arr ** -1, atol=1e-5)
    assert_close(oe.scalarpointwise(arr, 2, 4, reverse=1), 2.0 / arr, atol=1e-6)
    assert_close(oe.scalarpointwise(arr, 2.5, 3, reverse=1), 2.5 ** arr, atol=1e-5)
    neg = np.array([[-2.0, -3.0, 2.0, 3.0]], np.float32)
    assert_close(oe.scalarpointwise(neg, 3, 3), np.array([[-8.0, -27.0, 8.0, 27.0]]))
    frac = oe.scalarpointwise(neg, 0.5, 3)
    assert np.isnan(frac[0, :2]).all()
    assert_close(frac[0, 2:], np.sqrt(np.array([2.0, 3.0])))
    assert_close(oe.scalarpointwise(neg, 2, 3), neg ** 2)


def test_binary_broadcast_matches_reference_test():
    # reference tests/test_pointwise.py:81-87 and :16-21
    a = rng(2).standard_normal((3, 1)).astype(np.float32)
    b = rng(3).standard_normal((1, 4)).astype(np.float32)
    assert_close(oe.pointwise(a, b, 2), a * b)
    x = rng(0).standard_normal((5, 7)).astype(np.float32)
    y = rng(1).standard_normal((5, 7)).astype(np.float32)
    for op, f in enumerate([np.add, np.subtract, np.multiply, np.divide]):
        assert_close(oe.pointwise(x, y, op), f(x, y))


def test_clamp_equal_fill():
    x = np.array([-2.0, -0.5, 0.0, 0.5, 2.0], np.float32)
    assert np.array_equal(oe.clamp(x, -1, 1), np.clip(x, -1, 1))
    assert np.array_equal(oe.clampbackwards(x, -1, 1), np.array([0, 1, 1, 1, 0], np.float32))
    assert np.array_equal(oe.masked_fill(x, -9.0), np.array([-2, -0.5, -9, 0.5, 2], np.float32))
    assert np.array_equal(oe.equal(x, 0.5), (x == 0.5).astype(np.float32))
    assert math.isclose(float(oe.mul_backward(x, x, 2 * x)[0][0]), 8.0)


# ---------------------------------------------------------------------- FFT
from oracle import fft as of  # noqa: E402


def _dft_brute(x, n):
    """Definition of the DFT with explicit loops, after the reference's
    zero-pad / truncate of each row (fft_bitrev_real.wgsl:39-51)."""
    x = np.asarray(x, np.float64)
    rows = x.reshape(-1, x.shape[-1])
    out = np.zeros((rows.shape[0], n // 2 + 1), np.complex128)
    for r in range(rows.shape[0]):
        xr = [rows[r, j] if j < rows.shape[1] else 0.0 for j in range(n)]
        for k in range(n // 2 + 1):
            out[r, k] = sum(xr[j] * complex(math.cos(2 * math.pi * j * k / n),
                                            -math.sin(2 * math.pi * j * k / n))
                            for j in range(n))
    return out.reshape(x.shape[:-1] + (n // 2 + 1,))


def _idft_brute(X, n):
    """The reference's inverse taken literally: Hermitian expansion with the
    mirror rule of fft_bitrev_complex.wgsl:41-53, full complex inverse DFT,
    real part times 1/n (ifft_write_real.wgsl:25-28)."""
    X = np.asarray(X, np.complex128)
    rows = X.reshape(-1, X.shape[-1])
    in_len = rows.shape[1]
    out = np.zeros((rows.shape[0], n))
    for r in range(rows.shape[0]):
        full = []
        for i in range(n):
            if i <= n // 2:
                full.append(rows[r, i] if i < in_len else 0j)
            else:
                m = n - i
                full.append(np.conj(rows[r, m]) if m < in_len else 0j)
        for j in range(n):
            acc = sum(full[k] * complex(math.cos(2 * math.pi * j * k / n),
                                        math.sin(2 * math.pi * j * k / n)) for k in range(n))
            out[r, j] = acc.real / n
    return out.reshape(X.shape[:-1] + (n,))


@pytest.mark.parametrize("n,in_len", [(1, 1), (1, 3), (2, 2), (4, 3), (8, 8), (8, 11), (16, 5)])
def test_rfft_oracle_matches_brute_force_dft(n, in_len):
    x = rng(n * 31 + in_len).standard_normal((3, in_len))
    np.testing.assert_allclose(of.rfft(x, n), _dft_brute(x, n), atol=1e-9)


@pytest.mark.parametrize("n,in_len", [(2, 2), (4, 3), (8, 5), (8, 2), (8, 9), (16, 9)])
def test_irfft_oracle_matches_literal_hermitian_inverse(n, in_len):
    g = rng(n * 7 + in_len)
    X = g.standard_normal((2, in_len)) + 1j * g.standard_normal((2, in_len))
    # non-zero imaginary DC / Nyquist parts are part of the check
    np.testing.assert_allclose(of.irfft(X, n), _idft_brute(X, n), atol=1e-9)


def test_fft_identities():
    g = rng(5)
    x = g.standard_normal((4, 64))
    X = of.rfft(x)
    # round trip, Parseval (one-sided form), delta -> flat, linearity
    np.testing.assert_allclose(of.irfft(X, 64), x, atol=1e-12)
    energy = (np.abs(X[:, 0]) ** 2 + np.abs(X[:, -1]) ** 2
              + 2 * (np.abs(X[:, 1:-1]) ** 2).sum(axis=1)) / 64
    np.testing.assert_allclose(energy, (x ** 2).sum(axis=1), rtol=1e-12)
    delta = np.zeros((1, 32))
    delta[0, 0] = 1
    np.testing.assert_allclose(of.rfft(delta), np.ones((1, 17)), atol=1e-12)
    y = g.standard_normal((4, 64))
    np.testing.assert_allclose(of.rfft(2 * x - y), 2 * X - of.rfft(y), atol=1e-10)


@pytest.mark.parametrize("n", [2, 8, 256, 2048])
def test_reference_float32_arithmetic_error_is_small(n):
    # The reference's own f32 radix-2 result sits within ~1e-6 of the closed
    # form (relative to the row's largest bin), which sizes the tolerance the
    # HIP kernels are held to.
    x = rng(n).standard_normal((3, n)).astype(np.float32)
    want = of.rfft(x)
    got = of.rfft_radix2_f32(x)
    scale = np.abs(want).max(axis=-1, keepdims=True)
    assert (np.abs(got - want) / scale).max() < 2e-6
    back = of.irfft_radix2_f32(want.astype(np.complex64), n)
    np.testing.assert_allclose(back, x, atol=2e-6 * np.abs(x).max())


# ------------------------------------------- softmax backward, selu, complex


@pytest.mark.parametrize("shape,dim", [((5, 9), -1), ((3, 7, 4), 1), ((2, 3, 6), 0)])
def test_softmax_backward_against_torch_autograd_and_differences(shape, dim):
    # the chain of reference autograd/reductions.py:25-35: y * (g - sum(g y))
    # pinned by torch's float64 autograd of softmax (independent code) and by
    # central differences of oa.softmax; a dropped y factor, a flipped sign or
    # a sum over the wrong axis fails both
    import torch

    r = rng(sum(shape) + dim)
    x = r.standard_normal(shape)
    g = r.standard_normal(shape)
    y = oa.softmax(x, dim)
    got = oa.softmax_backward(y, g, dim)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    torch.softmax(xt, dim).backward(torch.tensor(g, dtype=torch.float64))
    assert_close(got, xt.grad.numpy(), rtol=1e-5, atol=1e-6)
    # directional derivative: <dL/dx, v> = d/dt <g, softmax(x + t v)> at t = 0
    v = r.standard_normal(shape)
    h = 1e-3
    num = ((g * oa.softmax(x + h * v, dim)).sum() - (g * oa.softmax(x - h * v, dim)).sum()) / (2 * h)
    assert abs(float((got.astype(np.float64) * v).sum()) - num) < 1e-3 * (1 + abs(num))


def test_selu_against_torch():
    # selu.wgsl's constants and branch (x > 0 -> SCALE x, else SCALE ALPHA (e^x - 1))
    import torch

    x = np.concatenate([np.linspace(-6, 6, 241), [0.0, -0.0, 1e-8, -1e-8, 30.0, -30.0]])
    ref = torch.nn.functional.selu(torch.tensor(x, dtype=torch.float64)).numpy()
    assert_close(oa.selu(x), ref, rtol=1e-6, atol=1e-7)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    torch.nn.functional.selu(xt).sum().backward()
    d = xt.grad.numpy()
    # torch takes the left branch's derivative at exactly 0 as well
    nz = x != 0
    assert_close(oa.selubackwards(x)[nz], d[nz], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("conj_a", [False, True])
@pytest.mark.parametrize("conj_b", [False, True])
def test_complex_mul_against_real_expansion(conj_a, conj_b):
    # complex_mul.wgsl: conjugation negates the operand's imaginary part before
    # (ac - bd, ad + bc); checked against that expansion written on real
    # pairs and against Python's own complex product on scalars
    r = rng(int(conj_a) * 2 + int(conj_b))
    a = (r.standard_normal((4, 9)) + 1j * r.standard_normal((4, 9))).astype(np.complex64)
    b = (r.standard_normal((4, 9)) + 1j * r.standard_normal((4, 9))).astype(np.complex64)
    ar, ai = a.real.astype(np.float64), a.imag.astype(np.float64) * (-1 if conj_a else 1)
    br, bi = b.real.astype(np.float64), b.imag.astype(np.float64) * (-1 if conj_b else 1)
    got = of.complex_mul(a, b, conj_a, conj_b)
    assert_close(got.real, ar * br - ai * bi, rtol=1e-6, atol=1e-6)
    assert_close(got.imag, ar * bi + ai * br, rtol=1e-6, atol=1e-6)
    for i, j in [(0, 0), (3, 8), (2, 5)]:
        za, zb = complex(a[i, j]), complex(b[i, j])
        za = za.conjugate() if conj_a else za
        zb = zb.conjugate() if conj_b else zb
        assert abs(complex(got[i, j]) - za * zb) < 1e-5 * (1 + abs(za * zb))
    # broadcast over leading dims
    bb = b[0]
    assert np.array_equal(of.complex_mul(a, bb, conj_a, conj_b),
                          np.stack([of.complex_mul(a[k], bb, conj_a, conj_b) for k in range(4)]))
    # a * conj(a) = |a|^2, real
    s = of.complex_mul(a, a, False, True)
    assert_close(s.real, np.abs(a.astype(np.complex128)) ** 2, rtol=1e-6, atol=1e-6)
    assert np.all(np.abs(s.imag) <= 1e-6 * (1 + s.real))


@pytest.mark.parametrize("in_len,out_len", [(5, 9), (9, 5), (7, 7), (1, 4), (6, 1)])
def test_complex_pad_against_reference_index_rule(in_len, out_len):
    # complex_pad.wgsl: Y[b, j] = X[b, j] for j < in_len else 0, over a
    # contiguous (batch, in_len) source; restated here as a literal loop
    r = rng(in_len * 10 + out_len)
    x = (r.standard_normal((3, 2, in_len)) + 1j * r.standard_normal((3, 2, in_len))).astype(
        np.complex64)
    flat = x.reshape(-1)
    batch = 6
    want = np.empty(batch * out_len, np.complex64)
    for idx in range(batch * out_len):
        bi, j = divmod(idx, out_len)
        want[idx] = flat[bi * in_len + j] if j < in_len else 0
    got = of.complex_pad(x, out_len)
    assert got.shape == (3, 2, out_len)
    assert np.array_equal(got.reshape(-1), want)


@pytest.mark.parametrize("shape,axis,keepdims", [((6, 7), None, False), ((6, 7), 1, True),
                                                 ((3, 4, 5), (0, 2), False), ((9,), 0, False)])
def test_var_std_against_numpy(shape, axis, keepdims):
    # population variance (ddof = 0) of reference functional/reductions.py:315-336;
    # numpy's var / std are independent code, and a ddof = 1 slip or a mean over
    # the wrong axis fails
    x = rng(len(shape)).standard_normal(shape) * 3 + 1
    want = np.var(x.astype(np.float32).astype(np.float64), axis=axis, keepdims=keepdims)
    assert_close(orr.var(x, axis, keepdims), np.asarray(want).reshape(np.shape(want) or (1,)),
                 rtol=1e-6, atol=1e-7)
    wstd = np.std(x.astype(np.float32).astype(np.float64), axis=axis, keepdims=keepdims)
    assert_close(orr.std(x, axis, keepdims), np.asarray(wstd).reshape(np.shape(wstd) or (1,)),
                 rtol=1e-6, atol=1e-7)
    assert np.all(orr.var(np.full(shape, 2.5), axis, keepdims) == 0)
