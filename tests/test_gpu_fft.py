"""GPU parity: rfft / irfft and the complex ops vs the oracle.

Tolerance.  The reference computes the transform in float32 (radix-2, f32
twiddles), so per-bin errors scale with the row's largest bin, not with the
bin itself: a near-zero bin of a 16384-point transform carries an absolute
error of ~1e-5 in any float32 FFT.  The bar is therefore the north-star
rtol 1e-4 / atol 1e-5 applied against the row's scale:
``|got - want| <= 1e-5 + 1e-4 * max|want_row|`` per element, where ``want``
is the float64 closed form.  The same test also checks that the error is no
worse than 4x the reference's own float32 arithmetic (oracle.fft.*_radix2_f32)
where that restatement is cheap enough to run.
"""

import numpy as np
import pytest

from conftest import rng
from oracle import fft as of

pytestmark = pytest.mark.gpu


def F():
    from wxx_amd import functional

    return functional


def up(a):
    return F().from_numpy(np.asarray(a, np.float32))


def upc(a):
    return F().from_numpy_complex(np.asarray(a))


def assert_fft_close(got, want, msg=""):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, f"{msg} shape {got.shape} != {want.shape}"
    scale = np.abs(want).reshape(-1, want.shape[-1]).max(axis=-1) if want.size else np.zeros(0)
    scale = scale.reshape(want.shape[:-1] + (1,))
    err = np.abs(got.astype(np.complex128) - want)
    bound = 1e-5 + 1e-4 * scale
    if not (err <= bound).all():
        worst = (err / bound).max()
        raise AssertionError(f"{msg} error {worst:.3g}x the bound (max abs err {err.max():.3g})")
    return err


# (rows shape, in_len, n): n = 1 .. 32768, padding (in_len < n), truncation
# (in_len > n), odd in_len (scalar loads), ragged row counts.
RFFT_CASES = [
    ((3,), 1, 1), ((2,), 5, 1), ((4,), 2, 2), ((5,), 3, 4), ((7,), 8, 8), ((3,), 16, 16),
    ((2, 3), 32, 32), ((9,), 64, 64), ((5,), 100, 128), ((3,), 300, 256), ((6,), 512, 512),
    ((4,), 1024, 1024), ((3,), 1500, 2048), ((2,), 4096, 4096), ((3,), 8191, 8192),
    ((2, 2), 8192, 16384), ((3,), 16384, 16384), ((2,), 20000, 32768), ((2,), 33000, 32768),
]


@pytest.mark.parametrize("rows,in_len,n", RFFT_CASES)
def test_rfft_matches_closed_form(device, rows, in_len, n):
    x = rng(n + in_len).standard_normal(rows + (in_len,)).astype(np.float32)
    X, n_out = F().rfft(up(x), n)
    assert n_out == n and X.type == "c64"
    got = X.numpy()
    want = of.rfft(x, n)
    err = assert_fft_close(got, want, f"rfft n={n}")
    if n >= 2:
        # no worse than 4x the reference's own float32 radix-2 arithmetic
        ref_err = np.abs(of.rfft_radix2_f32(x, n) - want)
        scale = np.abs(want).max()
        assert err.max() <= 4 * ref_err.max() + 1e-6 * scale


IRFFT_CASES = [
    ((3,), 2, 2), ((4,), 3, 4), ((2,), 2, 8), ((5,), 5, 8), ((3,), 9, 8), ((2, 3), 17, 32),
    ((7,), 65, 128), ((3,), 100, 256), ((4,), 513, 1024), ((3,), 1025, 2048),
    ((2,), 2049, 4096), ((3,), 4097, 8192), ((2, 2), 8193, 16384), ((2,), 6000, 16384),
    ((2,), 16385, 32768),
]


@pytest.mark.parametrize("rows,in_len,n", IRFFT_CASES)
def test_irfft_matches_closed_form(device, rows, in_len, n):
    g = rng(3 * n + in_len)
    X = (g.standard_normal(rows + (in_len,)) + 1j * g.standard_normal(rows + (in_len,)))
    X = X.astype(np.complex64)
    got = F().irfft(upc(X), n).numpy()
    want = of.irfft(X, n)
    assert got.shape == rows + (n,)
    err = assert_fft_close(got, want, f"irfft n={n}")
    ref_err = np.abs(of.irfft_radix2_f32(X, n) - want)
    assert err.max() <= 4 * ref_err.max() + 1e-6 * np.abs(want).max()


def test_irfft_default_length_and_empty(device):
    X = (rng(1).standard_normal((3, 9)) + 1j * rng(2).standard_normal((3, 9))).astype(np.complex64)
    got = F().irfft(upc(X)).numpy()
    assert got.shape == (3, 16)
    assert_fft_close(got, of.irfft(X, 16))
    empty = F().rfft(up(np.zeros((0, 8))), 8)[0]
    assert tuple(empty.shape) == (0, 5)
    assert F().irfft(upc(np.zeros((0, 5), np.complex64)), 8).numpy().shape == (0, 8)


def test_rfft_rejects_bad_lengths(device):
    with pytest.raises(ValueError):
        F().rfft(up(np.zeros((2, 6))), 6)
    with pytest.raises(ValueError):
        F().irfft(upc(np.zeros((2, 5), np.complex64)), 1)


def test_rfft_strided_input(device):
    x = rng(4).standard_normal((64, 6)).astype(np.float32)
    t = F().permute(up(x), 1, 0)
    assert not t.is_contiguous()
    assert_fft_close(F().rfft(t, 64)[0].numpy(), of.rfft(x.T, 64))


def test_fft_full_size_properties(device):
    # Standalone config: [2048 x 16384] f32.  Whole-size checks that do not
    # need the float64 oracle on every row: round trip, Parseval, linearity,
    # plus the closed form on a sample of rows.
    x = rng(5).standard_normal((2048, 16384)).astype(np.float32)
    tx = up(x)
    X, _ = F().rfft(tx, 16384)
    back = F().irfft(X, 16384).numpy()
    assert np.abs(back - x).max() < 2e-5 * np.abs(x).max() * 10
    Xh = X.numpy()
    energy = (np.abs(Xh[:, 0]) ** 2 + np.abs(Xh[:, -1]) ** 2
              + 2 * (np.abs(Xh[:, 1:-1]) ** 2).sum(axis=1)) / 16384
    np.testing.assert_allclose(energy, (x.astype(np.float64) ** 2).sum(axis=1), rtol=1e-5)
    sample = [0, 1, 777, 2047]
    assert_fft_close(Xh[sample], of.rfft(x[sample], 16384))
    two = F().rfft(F().scalarpointwise(tx, 2.0, 2), 16384)[0].numpy()
    assert_fft_close(two, 2 * Xh.astype(np.complex128))


@pytest.mark.parametrize("rows,n", [(300, 4096), (3000, 4096), (1100, 8192), (1300, 16384),
                                    (600, 32768)])
def test_fft_many_rows_every_row(device, rows, n):
    # More rows than one pass of the resident workgroups holds, so every
    # workgroup walks several rows; every row is checked.
    x = rng(rows + n).standard_normal((rows, n)).astype(np.float32)
    X, _ = F().rfft(up(x), n)
    assert_fft_close(X.numpy(), of.rfft(x, n), f"rfft rows={rows} n={n}")
    Xc = (rng(n).standard_normal((rows, n // 2 + 1))
          + 1j * rng(n + 1).standard_normal((rows, n // 2 + 1))).astype(np.complex64)
    assert_fft_close(F().irfft(upc(Xc), n).numpy(), of.irfft(Xc, n), f"irfft rows={rows} n={n}")


@pytest.mark.parametrize("length", [8192, 8191])
def test_irfft_crop_many_rows(device, length):
    # 1300 rows leave every persistent n = 16384 workgroup 2 or 3 rows; each
    # cropped row must equal the full transform's first `length` samples
    n, rows = 16384, 1300
    r = rng(length)
    X = (r.standard_normal((rows, n // 2 + 1))
         + 1j * r.standard_normal((rows, n // 2 + 1))).astype(np.complex64)
    full = F().irfft(upc(X), n).numpy()
    got = F().irfft(upc(X), n, length=length, scale=2.0).numpy()
    np.testing.assert_allclose(got, 2.0 * full[:, :length], rtol=0,
                               atol=2e-6 * np.abs(full).max())


def test_hyena_shapes(device):
    # Hyena fft_conv1d: x (8, 256, 8192) -> rfft(16384) -> (8, 256, 8193);
    # here a 2-batch slice of it, checked on sampled rows.
    x = rng(6).standard_normal((2, 256, 8192)).astype(np.float32)
    X, n = F().rfft(up(x), 16384)
    assert tuple(X.shape) == (2, 256, 8193) and n == 16384
    Xh = X.numpy()
    assert_fft_close(Xh[:, ::97], of.rfft(x[:, ::97], 16384))
    y = F().irfft(X, 16384).numpy()
    assert np.abs(y[..., :8192] - x).max() < 1e-4 and np.abs(y[..., 8192:]).max() < 1e-4


@pytest.mark.parametrize("sa,sb", [((4, 9), (4, 9)), ((2, 3, 17), (3, 17)), ((5, 1), (1, 6)),
                                   ((8, 256, 33), (256, 33))])
@pytest.mark.parametrize("ca,cb", [(False, False), (True, False), (False, True)])
def test_complex_mul_broadcast(device, sa, sb, ca, cb):
    g = rng(7)
    a = (g.standard_normal(sa) + 1j * g.standard_normal(sa)).astype(np.complex64)
    b = (g.standard_normal(sb) + 1j * g.standard_normal(sb)).astype(np.complex64)
    got = F().complex_mul(upc(a), upc(b), conj_a=ca, conj_b=cb).numpy()
    want = of.complex_mul(a, b, ca, cb)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)


def test_complex_support_ops(device):
    g = rng(8)
    a = (g.standard_normal((3, 10)) + 1j * g.standard_normal((3, 10))).astype(np.complex64)
    b = (g.standard_normal((10,)) + 1j * g.standard_normal((10,))).astype(np.complex64)
    ta = upc(a)
    assert np.array_equal(F().complex_conj(ta).numpy(), np.conj(a))
    assert np.array_equal(F().complex_pad(ta, 14).numpy(), of.complex_pad(a, 14))
    assert np.array_equal(F().complex_pad(ta, 4).numpy(), of.complex_pad(a, 4))
    np.testing.assert_allclose(F().complex_add(ta, upc(b)).numpy(), a + b, rtol=1e-6)
    F().complex_add_inplace(ta, upc(b))
    np.testing.assert_allclose(ta.numpy(), a + b, rtol=1e-6)
    w = F().complex_weights([1.0, 0.5, 2.0]).numpy()
    assert np.array_equal(w, np.array([1.0, 0.5, 2.0], np.complex64))
    # strided complex view -> contiguous (bit exact)
    t = upc(a)[:, ::3]
    assert not t.is_contiguous()
    assert np.array_equal(F().complex_contiguous(t).numpy(), a[:, ::3])
    assert np.array_equal(F().complex_conj(t).numpy(), np.conj(a[:, ::3]))


@pytest.mark.parametrize("n,length", [(16, 16), (16, 8), (16, 5), (64, 33), (4096, 2048),
                                      (16384, 8192), (16384, 8191), (16384, 1)])
@pytest.mark.parametrize("scale", [1.0, 16384.0])
def test_irfft_crop_equals_full_transform_sliced(device, n, length, scale):
    # the cropping inverse transform computes the full transform's first
    # `length` samples (times `scale`) with the same arithmetic; kernels
    # compiled for different crop modes may fuse a different product of an
    # a*b + c into an FMA, so agreement is to ~1 ulp of the row's scale
    r = rng(n + length)
    rows, nb = 5, n // 2 + 1
    X = (r.standard_normal((rows, nb)) + 1j * r.standard_normal((rows, nb))).astype(np.complex64)
    full = F().irfft(upc(X), n).numpy()
    want = full[:, :length]
    if scale != 1.0:
        want = want * np.float32(scale)
    got = F().irfft(upc(X), n, length=length, scale=scale).numpy()
    assert got.shape == (rows, length)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-6 * np.abs(full).max() * scale)
    with pytest.raises(ValueError):
        F().irfft(upc(X), n, length=n + 1)


@pytest.mark.parametrize("L,n", [(8, 16), (7, 16), (2048, 4096), (8192, 16384)])
def test_fft_conv_crop_autograd_matches_sliced_path(device, L, n):
    # the Hyena long convolution with the fused crop: output and both input
    # gradients equal (to ~1 ulp, see above) to irfft(...)[..., :L] through
    # the slice backward
    r = rng(L)
    X = r.standard_normal((2, 3, L)).astype(np.float32)
    H = r.standard_normal((3, L)).astype(np.float32)
    G = r.standard_normal((2, 3, L)).astype(np.float32)
    res = []
    for fused in (True, False):
        x, h = up(X), up(H)
        x.requires_grad = h.requires_grad = True
        spec = x.rfft(n).complex_mul(h.rfft(n))
        y = spec.irfft(n, L) if fused else spec.irfft(n)[..., :L]
        (y * up(G)).sum().backward()
        res.append((y.numpy(), x.grad.numpy(), h.grad.numpy()))
    for a, b in zip(*res):
        np.testing.assert_allclose(a, b, rtol=0, atol=1e-6 * np.abs(b).max())


# Lengths beyond one workgroup's LDS (n > 32768): the four-step path.
@pytest.mark.parametrize("rows,in_len,n", [((2,), 65536, 65536), ((3,), 40000, 65536),
                                           ((1,), 70001, 65536), ((2,), 131072, 131072),
                                           ((1,), 262144, 262144)])
def test_rfft_irfft_beyond_lds(device, rows, in_len, n):
    x = rng(n + in_len).standard_normal(rows + (in_len,)).astype(np.float32)
    X, _ = F().rfft(up(x), n)
    want = of.rfft(x, n)
    err = assert_fft_close(X.numpy(), want, f"rfft n={n}")
    ref_err = np.abs(of.rfft_radix2_f32(x, n) - want)
    assert err.max() <= 4 * ref_err.max() + 1e-6 * np.abs(want).max()
    # inverse of a random one-sided spectrum (DC / Nyquist imaginary parts and
    # a truncated / padded in_len included)
    g = rng(n)
    for k_in in (n // 2 + 1, n // 2 - 7, n // 2 + 9):
        Xs = (g.standard_normal(rows + (k_in,)) + 1j * g.standard_normal(rows + (k_in,)))
        Xs = Xs.astype(np.complex64)
        got = F().irfft(upc(Xs), n).numpy()
        want = of.irfft(Xs, n)
        err = assert_fft_close(got, want, f"irfft n={n} in_len={k_in}")
        ref_err = np.abs(of.irfft_radix2_f32(Xs, n) - want)
        assert err.max() <= 4 * ref_err.max() + 1e-6 * np.abs(want).max()
    # the round trip, and the Hyena crop with a post scale
    back = F().irfft(X, n).numpy()
    xin = of._fit(x, n)
    assert np.abs(back - xin).max() < 1e-5 * np.abs(xin).max() * 10
    L = n // 2 - 3
    crop = F().irfft(X, n, L, 2.0).numpy()
    assert crop.shape == rows + (L,)
    assert np.array_equal(crop, (back[..., :L] * np.float32(2.0)).astype(np.float32))


def test_fft_conv_beyond_lds_matches_direct_sum(device):
    # Hyena's long convolution at L = 20000 (n = next_pow2(2 L) = 65536):
    # irfft(rfft(z, n) rfft(h, n), n)[:L] against the direct causal sum
    from wxx_amd import nn

    L, D = 20000, 2
    r = rng(77)
    z = r.standard_normal((1, D, L)).astype(np.float32)
    h = (r.standard_normal((D, L)) * np.exp(-np.arange(L) / 500.0)).astype(np.float32)
    op = nn.HyenaOperator(D, order=1)
    got = op.fft_conv1d(up(z), up(h)).numpy()
    want = np.stack([np.convolve(z[0, d].astype(np.float64), h[d].astype(np.float64))[:L]
                     for d in range(D)])[None]
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= 2e-6 * scale * np.sqrt(L)
