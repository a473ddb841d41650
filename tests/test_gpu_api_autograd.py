"""GPU: autograd through the reference API.

* finite-difference gradchecks of Linear, GELU, exp, sqrt, cos, pow and the
  reflected scalar operators, and slice/narrow backward (the behaviours of
  reference tests/test_autograd_gradcheck.py);
* matmul / matmuladd backward (reference autograd/utils.py:40-140) for every
  transpose combination, batched and broadcast operands, against float64
  products;
* rfft / irfft / complex_mul backward (reference autograd/utils.py:549-718)
  against the analytic gradients written with explicit float64 DFT matrices
  (the real-valued loss L = sum Re(conj(g) out) differentiated by hand);
* Tensor.unfold views and their backward (reference tests/test_unfold.py),
  against numpy's sliding_window_view and a scatter-add of an index map.
"""

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu


def wxx():
    import wxx_amd

    return wxx_amd


def f32(a, grad=False):
    t = wxx().functional.from_numpy(np.asarray(a, np.float32))
    t.requires_grad = grad
    return t


def c64(a, grad=False):
    from wxx_amd.functional.fft import from_numpy_complex

    t = from_numpy_complex(np.asarray(a, np.complex64))
    t.requires_grad = grad
    return t


# ---- finite-difference gradchecks ------------------------------------------


def _fd_check(param, loss_fn, idxs, eps):
    F = wxx().functional
    base = param.numpy().copy()
    param.grad = None
    loss_fn().backward()
    analytic = param.grad.numpy().copy()
    for idx in idxs:
        vals = []
        for sgn in (1, -1):
            a = base.copy()
            a[idx] += sgn * eps
            F.assign(param, f32(a))
            vals.append(loss_fn().item())
        F.assign(param, f32(base))
        numeric = (vals[0] - vals[1]) / (2 * eps)
        rel = abs(analytic[idx] - numeric) / max(1e-4, abs(analytic[idx]) + abs(numeric))
        assert rel < 5e-2, (idx, analytic[idx], numeric)


def test_linear_gradcheck(device):
    lin = wxx().nn.Linear(3, 2)
    x = f32(rng(0).standard_normal((4, 3)))
    w = f32(rng(1).standard_normal((4, 2)))
    loss = lambda: (lin(x) * w).sum()  # noqa: E731
    _fd_check(lin.weight, loss, [(0, 0), (1, 1), (2, 0)], 1e-2)
    _fd_check(lin.bias, loss, [(1,)], 1e-2)


UNARY = {
    "gelu": (lambda t: t.gelu(), None),
    "exp": (lambda t: t.exp(), None),
    "sqrt": (lambda t: t.sqrt(), "positive"),
    "cos": (lambda t: t.cos(), "fixed"),
    "pow3": (lambda t: t.pow(3), "fixed"),
    "pow_m1": (lambda t: t ** -1, "fixed"),
    "rpow2": (lambda t: 2 ** t, "fixed"),
    "rpow2.5": (lambda t: 2.5 ** t, "fixed"),
    "rdiv2": (lambda t: 2 / t, "fixed"),
}


@pytest.mark.parametrize("name", list(UNARY))
def test_unary_gradcheck(device, name):
    fn, kind = UNARY[name]
    if kind == "fixed":
        a = np.array([[-2.0, -0.5, 0.5, 2.0], [0.25, 1.5, 3.0, 4.0]], np.float32)
        idxs = [(0, 0), (0, 2), (1, 0)]
    elif kind == "positive":
        a = np.abs(rng(6).standard_normal((3, 4))) + 0.5
        idxs = [(0, 0), (1, 1), (2, 3)]
    else:
        a = rng(2).standard_normal((3, 4))
        idxs = [(0, 0), (1, 1), (2, 3)]
    x = f32(a, grad=True)
    w = f32(rng(3).standard_normal(np.shape(a)))
    _fd_check(x, lambda: (fn(x) * w).sum(), idxs, 1e-3)


def test_slice_and_narrow_backward_scatter(device):
    x = f32(rng(8).standard_normal((2, 5, 4)), grad=True)
    w = rng(9).standard_normal((2, 2, 4)).astype(np.float32)
    (x.slice(1, 1, 2) * f32(w)).sum().backward()  # slice: the differentiable narrow
    want = np.zeros((2, 5, 4), np.float32)
    want[:, 1:3] = w
    np.testing.assert_array_equal(x.grad.numpy(), want)

    y = f32(rng(10).standard_normal((3, 6)), grad=True)
    g = rng(11).standard_normal((3, 3)).astype(np.float32)
    (y[:, :3] * f32(g)).sum().backward()
    want = np.zeros((3, 6), np.float32)
    want[:, :3] = g
    np.testing.assert_array_equal(y.grad.numpy(), want)

    z = f32(rng(12).standard_normal((4, 5)), grad=True)
    h = rng(13).standard_normal(5).astype(np.float32)
    (z[2] * f32(h)).sum().backward()
    want = np.zeros((4, 5), np.float32)
    want[2] = h
    np.testing.assert_array_equal(z.grad.numpy(), want)


# ---- matmul backward ----------------------------------------------------------


def _op(a, t):
    return np.swapaxes(a, -1, -2) if t else a


def _reduce_to(g, shape):
    while g.ndim > len(shape):
        g = g.sum(axis=0)
    return g


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("layout", ["2d", "A_batched", "both_batched", "B_batched"])
def test_matmul_backward(device, ta, tb, layout):
    from wxx_amd import autograd

    M, K, N, b = 5, 7, 6, 3
    r = rng(20)
    sa = (K, M) if ta else (M, K)
    sb = (N, K) if tb else (K, N)
    if layout in ("A_batched", "both_batched"):
        sa = (b,) + sa
    if layout in ("B_batched", "both_batched"):
        sb = (b,) + sb
    A = r.standard_normal(sa)
    B = r.standard_normal(sb)
    a, bb = f32(A, True), f32(B, True)
    out = autograd.matmul(a, bb).forward(a, bb, ta, tb)
    G = r.standard_normal(out.shape)
    (out * f32(G)).sum().backward()
    A32, B32 = A.astype(np.float32).astype(np.float64), B.astype(np.float32).astype(np.float64)
    G = G.astype(np.float32).astype(np.float64)
    # C = op(A) op(B): d op(A) = G op(B)^T, d op(B) = op(A)^T G
    dopa = G @ np.swapaxes(_op(B32, tb), -1, -2)
    dopb = np.swapaxes(_op(A32, ta), -1, -2) @ G
    np.testing.assert_allclose(a.grad.numpy(), _reduce_to(_op(dopa, ta), sa), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(bb.grad.numpy(), _reduce_to(_op(dopb, tb), sb), rtol=1e-4,
                               atol=1e-5)


@pytest.mark.parametrize("bias_shape", ["vec", "mat"])
def test_linear_3d_backward(device, bias_shape):
    # Linear over (batch, rows, in): dW is one GEMM over K = batch x rows
    from wxx_amd import autograd

    B, S, D, O = 3, 33, 20, 12
    r = rng(21)
    X, W = r.standard_normal((B, S, D)), r.standard_normal((D, O))
    bias = r.standard_normal(O if bias_shape == "vec" else (S, O))
    x, w, bi = f32(X, True), f32(W, True), f32(bias, True)
    out = autograd.matmuladd(x, w, bi).forward(x, w, bi)
    G = r.standard_normal(out.shape)
    (out * f32(G)).sum().backward()
    X, W, G = (v.astype(np.float32).astype(np.float64) for v in (X, W, G))
    np.testing.assert_allclose(x.grad.numpy(), G @ W.T, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(w.grad.numpy(), np.einsum("bsd,bso->do", X, G), rtol=1e-4,
                               atol=1e-4)
    want_b = G.sum(axis=(0, 1)) if bias_shape == "vec" else G.sum(axis=0)
    np.testing.assert_allclose(bi.grad.numpy(), want_b, rtol=1e-4, atol=1e-5)


# ---- FFT autograd ------------------------------------------------------------


def _dft_forward(n_out_bins, N):
    k = np.arange(n_out_bins)[:, None]
    n = np.arange(N)[None, :]
    return np.exp(-2j * np.pi * k * n / N)  # X_k = sum_n x_n e^{-i 2 pi k n / N}


@pytest.mark.parametrize("L,n", [(16, None), (12, 16), (20, 16), (2, None)])
def test_rfft_backward_is_the_true_gradient(device, L, n):
    # L = sum_k Re(conj(g_k) X_k), X = rfft(x zero-padded / truncated to N):
    # dL/dx_j = Re(sum_k g_k e^{+i 2 pi k j / N}) for j < min(L, N), else 0
    r = rng(30 + L)
    N = n or L
    nb = N // 2 + 1
    x = f32(r.standard_normal((3, L)), True)
    g = (r.standard_normal((3, nb)) + 1j * r.standard_normal((3, nb))).astype(np.complex64)
    out = x.rfft(n)
    assert out.shape == [3, nb]
    # sum Re(conj(g) X) = sum (Re g Re X + Im g Im X): seed the sweep with g
    out.grad = c64(g)
    out.backward()
    Fm = _dft_forward(nb, N)
    want = np.real(g.astype(np.complex128) @ np.conj(Fm))
    full = np.zeros((3, L))
    m = min(L, N)
    full[:, :m] = want[:, :m]
    np.testing.assert_allclose(x.grad.numpy(), full, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("bins,n", [(9, None), (9, 16), (5, 16), (12, 16)])
def test_irfft_backward_is_the_true_gradient(device, bins, n):
    # y_j = (1/N) [Re X_0 + Re X_{N/2} (-1)^j + sum_{0<k<N/2} 2 Re(X_k e^{i 2 pi k j/N})]
    # over the bins present; L = sum g_j y_j.
    r = rng(40 + bins)
    N = n or 2 * (bins - 1)
    X = (r.standard_normal((2, bins)) + 1j * r.standard_normal((2, bins))).astype(np.complex64)
    x = c64(X, True)
    y = x.irfft(n)
    assert y.shape == [2, N]
    G = r.standard_normal((2, N)).astype(np.float32)
    y.grad = f32(G)
    y.backward()
    want = np.zeros((2, bins), np.complex128)
    j = np.arange(N)
    for k in range(min(bins, N // 2 + 1)):
        wk = 1.0 if k in (0, N // 2) else 2.0
        c, s = np.cos(2 * np.pi * k * j / N), np.sin(2 * np.pi * k * j / N)
        want[:, k] = wk / N * (G @ c) - 1j * wk / N * (G @ s)
        if k in (0, N // 2):
            want[:, k] = want[:, k].real  # Re() drops the imaginary part of DC / Nyquist
    np.testing.assert_allclose(x.grad.numpy(), want, rtol=1e-4, atol=1e-5)


def test_complex_mul_backward_with_broadcast(device):
    r = rng(50)
    A = (r.standard_normal((4, 3, 9)) + 1j * r.standard_normal((4, 3, 9))).astype(np.complex64)
    B = (r.standard_normal((3, 9)) + 1j * r.standard_normal((3, 9))).astype(np.complex64)
    G = (r.standard_normal((4, 3, 9)) + 1j * r.standard_normal((4, 3, 9))).astype(np.complex64)
    a, b = c64(A, True), c64(B, True)
    out = a.complex_mul(b)
    np.testing.assert_allclose(out.numpy(), A * B, rtol=1e-5, atol=1e-5)
    out.grad = c64(G)
    out.backward()
    # d/dA Re(conj(G) A B) = G conj(B); the broadcast operand sums over the batch
    np.testing.assert_allclose(a.grad.numpy(), G * np.conj(B), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(b.grad.numpy(), (G * np.conj(A)).sum(axis=0), rtol=1e-5,
                               atol=1e-4)


def test_fft_convolution_end_to_end_gradient(device):
    # y = irfft(rfft(x, 2L) * rfft(h, 2L))[:L]: a causal linear convolution
    # (the Hyena long-convolution shape); gradients against direct float64 sums
    r = rng(60)
    L = 32
    X, H = r.standard_normal((2, L)), r.standard_normal((1, L))
    x, h = f32(X, True), f32(H, True)
    y = x.rfft(2 * L).complex_mul(h.rfft(2 * L)).irfft(2 * L)[:, :L]
    Y = np.array([[sum(X[b, t - s] * H[0, s] for s in range(t + 1)) for t in range(L)]
                  for b in range(2)])
    np.testing.assert_allclose(y.numpy(), Y, rtol=1e-4, atol=1e-4)
    G = r.standard_normal((2, L))
    (y * f32(G)).sum().backward()
    G = G.astype(np.float32).astype(np.float64)
    dX = np.array([[sum(G[b, t] * H[0, t - u] for t in range(u, L)) for u in range(L)]
                   for b in range(2)])
    dH = np.array([[sum(G[b, t] * X[b, t - s] for b in range(2) for t in range(s, L))
                    for s in range(L)]])
    np.testing.assert_allclose(x.grad.numpy(), dX, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(h.grad.numpy(), dH, rtol=1e-4, atol=1e-4)


# (x shape, filter shape, n): the small-row transforms, the persistent ones
# at 2^11..2^14 complex points (n = 4096 .. 32768, the Hyena rows at 16384),
# a ragged odd length, a filter longer than the signal, n below 2 L (crop of
# a circular product) and one row
FFT_CONV = [
    ((2, 3, 32), (3, 32), 64),
    ((2, 4, 101), (4, 101), 256),
    ((3, 2, 20), (2, 37), 64),
    ((2, 3, 48), (3, 48), 64),
    ((1, 1, 9), (1, 9), 16),
    ((2, 2, 2048), (2, 2048), 4096),
    ((2, 3, 3000), (3, 3000), 8192),
    ((2, 4, 8192), (4, 8192), 16384),
    ((1, 2, 16384), (2, 16384), 32768),
]


@pytest.mark.parametrize("xs,hs,n", FFT_CONV)
def test_fft_conv_equals_composed_ops_bit_for_bit(device, xs, hs, n):
    # the fused long convolution against rfft / complex_mul / irfft composed
    # through their own Functions: output and both gradients identical bits
    W = wxx()
    r = rng(61)
    X, H, G = (r.standard_normal(xs), r.standard_normal(hs),
               r.standard_normal(xs[:-1] + (min(xs[-1], n),)))
    length = min(xs[-1], n)
    x0, h0 = f32(X, True), f32(H, True)
    y0 = x0.rfft(n).complex_mul(h0.rfft(n)).irfft(n, length)
    (y0 * f32(G)).sum().backward()
    x1, h1 = f32(X, True), f32(H, True)
    y1 = W.autograd.fft_conv(x1, h1).forward(x1, h1, n, length)
    (y1 * f32(G)).sum().backward()
    assert np.array_equal(y1.numpy(), y0.numpy())
    assert np.array_equal(x1.grad.numpy(), x0.grad.numpy())
    assert np.array_equal(h1.grad.numpy(), h0.grad.numpy())


def test_fft_conv_filter_only_gradient(device):
    # only the filter trains (a signal without requires_grad): no signal
    # gradient is formed and the filter's still matches the composed ops
    W = wxx()
    r = rng(62)
    X, H, G = r.standard_normal((3, 2, 40)), r.standard_normal((2, 40)), r.standard_normal((3, 2, 40))
    h0 = f32(H, True)
    (f32(X).rfft(128).complex_mul(h0.rfft(128)).irfft(128, 40) * f32(G)).sum().backward()
    x1, h1 = f32(X), f32(H, True)
    (W.autograd.fft_conv(x1, h1).forward(x1, h1, 128, 40) * f32(G)).sum().backward()
    assert x1.grad is None
    assert np.array_equal(h1.grad.numpy(), h0.grad.numpy())


@pytest.mark.parametrize("batch", [1, 3, 4, 5, 8, 9])
def test_complex_mul_batch_sum_equals_product_then_sum(device, batch):
    # one pass against complex_mul followed by the sum over the batch: the
    # same bits, for batches below, at and past multiples of four
    W = wxx()
    F = W.functional
    r = rng(63)
    A = r.standard_normal((batch, 3, 77)) + 1j * r.standard_normal((batch, 3, 77))
    Cc = r.standard_normal((batch, 3, 77)) + 1j * r.standard_normal((batch, 3, 77))
    a, c = c64(A), c64(Cc)
    for conj in (False, True):
        got = F.complex_mul_batch_sum(a, c, conj_c=conj, keep=2).numpy()
        prod = F.complex_mul(a, c, conj_b=conj)
        from wxx_amd.autograd.utils import _sum_to_shape_complex

        want = _sum_to_shape_complex(prod, (3, 77)).numpy()
        assert np.array_equal(got, want)
        ref = (A.astype(np.complex64).astype(np.complex128)
               * (np.conj(Cc) if conj else Cc).astype(np.complex64)).sum(axis=0)
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("n", [16, 1024, 16384])
def test_spectrum_products_fused_into_transforms(device, n):
    # rfft_mul and irfft_mul against rfft / complex_mul / irfft with a filter
    # broadcast over a leading dim, conjugated or not, and a weight row
    W = wxx()
    F = W.functional
    r = rng(64)
    bins = n // 2 + 1
    x = f32(r.standard_normal((2, 3, n)))
    Hn = r.standard_normal((3, bins)) + 1j * r.standard_normal((3, bins))
    h = c64(Hn)
    edge, mid = 0.75, -1.3  # any real weights; the adjoints use powers of two
    w = F.complex_weights([edge] + [mid] * (bins - 2) + [edge])
    spec, _ = F.rfft(x, n)
    assert np.array_equal(F.rfft_mul(x, n, (edge, mid)).numpy(), F.complex_mul(spec, w).numpy())
    for conj in (False, True):
        want = F.irfft(F.complex_mul(F.complex_mul(spec, h, conj_b=conj), w), n,
                       length=n - 3, scale=2.0).numpy()
        got = F.irfft_mul(spec, n, h=h, conj_h=conj, bin_weights=(edge, mid), length=n - 3,
                          scale=2.0).numpy()
        assert np.array_equal(got, want)
        want = F.irfft(F.complex_mul(spec, h, conj_b=conj), n).numpy()
        assert np.array_equal(F.irfft_mul(spec, n, h=h, conj_h=conj).numpy(), want)
    assert np.array_equal(F.irfft_mul(spec, n).numpy(), F.irfft(spec, n).numpy())


def test_spectrum_products_reject_bad_operands(device):
    F = wxx().functional
    x = f32(np.zeros((2, 64)))
    spec, _ = F.rfft(x, 64)
    with pytest.raises(ValueError):
        F.rfft_mul(x, 65536, (1.0, 0.5))
    with pytest.raises(ValueError):
        F.irfft_mul(spec, 128, bin_weights=(1.0, 0.5))  # 33 bins, 65 needed
    with pytest.raises(ValueError):
        F.irfft_mul(spec, 64, h=c64(np.zeros((3, 33))))  # not a trailing shape
    with pytest.raises(ValueError):
        F.complex_mul_batch_sum(spec, spec, keep=2)  # no batch dim left


# ---- unfold ---------------------------------------------------------------------


def _np_unfold(a, dim, size, step):
    w = np.lib.stride_tricks.sliding_window_view(a, size, axis=dim)
    idx = [slice(None)] * a.ndim
    idx[dim] = slice(None, None, step)
    return w[tuple(idx)]


def _np_unfold_grad(shape, dim, size, step, g):
    ids = np.arange(int(np.prod(shape))).reshape(shape)
    win = _np_unfold(ids, dim, size, step)
    out = np.zeros(int(np.prod(shape)))
    np.add.at(out, win.reshape(-1), g.reshape(-1).astype(np.float64))
    return out.reshape(shape)


@pytest.mark.parametrize("dim", [0, 1, 2, 3, -1, -2])
@pytest.mark.parametrize("size,step", [(1, 1), (2, 2), (3, 1), (3, 2), (4, 3)])
def test_unfold_values(device, dim, size, step):
    a = rng(0).standard_normal((2, 3, 7, 5)).astype(np.float32)
    d = dim % 4
    if size > a.shape[d]:
        pytest.skip("window longer than the axis")
    out = f32(a).unfold(dim, size, step)
    want = _np_unfold(a, d, size, step)
    assert out.shape == list(want.shape)
    np.testing.assert_array_equal(out.numpy(), want)


def test_unfold_is_a_view_and_handles_strided_inputs(device):
    a = rng(1).standard_normal((3, 8)).astype(np.float32)
    x = f32(a)
    out = x.unfold(1, 3, 2)
    assert out.buffer is x.buffer and out._base is x and out.offset == x.offset
    assert list(out.stride) == [x.stride[0], 2 * x.stride[1], x.stride[1]]
    np.testing.assert_array_equal(out.numpy(), _np_unfold(a, 1, 3, 2))
    b = rng(2).standard_normal((4, 6)).astype(np.float32)
    y = f32(b)
    t = y.permute(1, 0)
    assert not t.is_contiguous()
    np.testing.assert_array_equal(t.unfold(0, 3, 2).numpy(), _np_unfold(b.T, 0, 3, 2))
    np.testing.assert_array_equal(y[:3, 1:6].unfold(1, 3, 1).numpy(),
                                  _np_unfold(b[:3, 1:6], 1, 3, 1))


@pytest.mark.parametrize("dim,size,step", [(0, 2, 1), (1, 3, 2), (2, 4, 1), (2, 3, 2)])
def test_unfold_backward(device, dim, size, step):
    a = rng(3).standard_normal((2, 3, 6)).astype(np.float32)
    x = f32(a, True)
    out = x.unfold(dim, size, step)
    w = rng(4 + dim + size).standard_normal(tuple(out.shape)).astype(np.float32)
    (out * f32(w)).sum().backward()
    np.testing.assert_allclose(x.grad.numpy(), _np_unfold_grad(a.shape, dim, size, step, w),
                               rtol=1e-6, atol=1e-6)


def test_unfold_backward_through_permute_and_u32(device):
    a = rng(5).standard_normal((3, 8)).astype(np.float32)
    base = f32(a, True)
    out = base.permute(1, 0).unfold(1, 3, 2)
    w = rng(6).standard_normal(tuple(out.shape)).astype(np.float32)
    (out * f32(w)).sum().backward()
    np.testing.assert_allclose(base.grad.numpy(), _np_unfold_grad((8, 3), 1, 3, 2, w).T,
                               rtol=1e-6, atol=1e-6)
    ids = wxx().functional.from_numpy(np.arange(24).reshape(2, 3, 4), np.uint32)
    u = ids.unfold(2, 2, 1)
    assert u.type == "u32"
    np.testing.assert_array_equal(u.numpy(), _np_unfold(np.arange(24).reshape(2, 3, 4), 2, 2, 1))


def test_unfold_argument_errors(device):
    x = f32(np.zeros((2, 5)))
    for size in (0, -1, 6):
        with pytest.raises(ValueError):
            x.unfold(1, size)
    for step in (0, -1):
        with pytest.raises(ValueError):
            x.unfold(1, 2, step)
    for bad in (1.5, "2", True):
        with pytest.raises(TypeError):
            x.unfold(1, bad)
    for dim in (2, -3):
        with pytest.raises((IndexError, ValueError)):
            x.unfold(dim, 2)
    with pytest.raises(ValueError):
        f32(np.zeros((2,) * 6)).unfold(0, 2)


# ---- slice gradients reaching one tensor ----------------------------------------


def test_chunk_gradients_tile_the_input(device):
    a = rng(70).standard_normal((3, 8, 12)).astype(np.float32)
    x = f32(a, True)
    ws = [rng(71 + i).standard_normal((3, 8, 3)).astype(np.float32) for i in range(4)]
    parts = x.chunk(4, dim=-1)
    loss = None
    for p, w in zip(parts, ws):
        t = (p * f32(w)).sum()
        loss = t if loss is None else loss + t
    loss.backward()
    np.testing.assert_array_equal(x.grad.numpy(), np.concatenate(ws, axis=-1))


def test_partial_and_overlapping_slice_gradients(device):
    a = rng(72).standard_normal((4, 10)).astype(np.float32)
    # only chunks 0 and 2 of 5 used: zeros elsewhere
    x = f32(a, True)
    c = x.chunk(5, dim=1)
    w0, w2 = (rng(73 + i).standard_normal((4, 2)).astype(np.float32) for i in range(2))
    ((c[0] * f32(w0)).sum() + (c[2] * f32(w2)).sum()).backward()
    want = np.zeros((4, 10), np.float32)
    want[:, 0:2], want[:, 4:6] = w0, w2
    np.testing.assert_array_equal(x.grad.numpy(), want)
    # overlapping slices, a dense use of the same tensor, and a slice along another dim
    y = f32(a, True)
    u = rng(75).standard_normal((4, 3)).astype(np.float32)
    v = rng(76).standard_normal((4, 4)).astype(np.float32)
    d = rng(77).standard_normal((4, 10)).astype(np.float32)
    r = rng(78).standard_normal((2, 10)).astype(np.float32)
    loss = ((y[:, 0:3] * f32(u)).sum() + (y.slice(1, 2, 4) * f32(v)).sum()
            + (y * f32(d)).sum() + (y.slice(0, 1, 2) * f32(r)).sum())
    loss.backward()
    want = d.astype(np.float64).copy()
    want[:, 0:3] += u
    want[:, 2:6] += v
    want[1:3, :] += r
    np.testing.assert_allclose(y.grad.numpy(), want, rtol=1e-6, atol=1e-6)
