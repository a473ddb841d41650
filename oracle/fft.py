"""Real FFT / inverse and complex ops restated from the reference (test
infrastructure only).

* ``rfft(x, n)`` (reference src/wxx/functional/fft.py:484-563,
  shaders/helpers/fft_bitrev_real.wgsl:39-51, fft_wg_real.wgsl:51-60): each
  row is zero-padded or truncated to the power of two ``n`` and the one-sided
  DFT ``X[k] = sum_j x[j] exp(-2 pi i j k / n)``, k = 0..n/2, is returned.
  Computed in float64 with numpy's FFT (the closed form).
* ``irfft(X, n)`` (fft.py:566-645, fft_bitrev_complex.wgsl:41-53,
  fft_wg_inverse.wgsl:48-61, ifft_write_real.wgsl:25-28): bins below
  ``min(in_len, n/2+1)`` are used, missing bins are zero, the spectrum is
  extended by Hermitian symmetry and the real part of the inverse times 1/n
  is returned.  The imaginary parts of the DC and Nyquist bins cancel out of
  the real part, which is what numpy's c2r transform assumes too.
* ``rfft_radix2_f32`` / ``irfft_radix2_f32``: float32 restatement of the
  reference's own arithmetic (bit-reversed load, radix-2 DIT butterflies with
  a per-butterfly ``cos/sin(-2 pi k / m)`` twiddle in f32,
  fft_stage.wgsl:37-66, fft_wg_real.wgsl:63-88), used to size the rounding
  error the reference itself makes.
* ``complex_mul`` (complex_mul.wgsl:41-62), ``complex_pad``
  (complex_pad.wgsl), ``complex_conj``: numpy.
"""

import numpy as np


def _fit(x, n):
    x = np.asarray(x, np.float64)
    m = x.shape[-1]
    if m >= n:
        return x[..., :n]
    pad = np.zeros(x.shape[:-1] + (n - m,), np.float64)
    return np.concatenate([x, pad], axis=-1)


def rfft(x, n=None):
    x = np.asarray(x)
    n = x.shape[-1] if n is None else int(n)
    return np.fft.rfft(_fit(x, n), n=n, axis=-1)


def _one_sided(X, n):
    X = np.asarray(X, np.complex128)
    half = n // 2 + 1
    k = X.shape[-1]
    if k >= half:
        X = X[..., :half].copy()
    else:
        X = np.concatenate([X, np.zeros(X.shape[:-1] + (half - k,), np.complex128)], axis=-1)
    X[..., 0] = X[..., 0].real
    X[..., -1] = X[..., -1].real
    return X


def irfft(X, n=None):
    X = np.asarray(X)
    n = 2 * (X.shape[-1] - 1) if n is None else int(n)
    return np.fft.irfft(_one_sided(X, n), n=n, axis=-1)


def _bitrev_perm(n):
    bits = n.bit_length() - 1
    idx = np.arange(n)
    rev = np.zeros(n, np.int64)
    for b in range(bits):
        rev |= ((idx >> b) & 1) << (bits - 1 - b)
    return rev


def _radix2_f32(z, inverse):
    """In-place radix-2 DIT over the last axis of a bit-reversed complex64 array."""
    n = z.shape[-1]
    re = z.real.astype(np.float32)
    im = z.imag.astype(np.float32)
    m = 2
    sign = np.float32(2.0 if inverse else -2.0)
    pi = np.float32(np.pi)
    while m <= n:
        half = m // 2
        k = np.arange(half, dtype=np.float32)
        angle = sign * pi * k / np.float32(m)
        wr = np.cos(angle).astype(np.float32)
        wi = np.sin(angle).astype(np.float32)
        re = re.reshape(re.shape[:-1] + (n // m, m))
        im = im.reshape(im.shape[:-1] + (n // m, m))
        ur, ui = re[..., :half].copy(), im[..., :half].copy()
        vr, vi = re[..., half:], im[..., half:]
        tr = vr * wr - vi * wi
        ti = vr * wi + vi * wr
        re = np.concatenate([ur + tr, ur - tr], axis=-1).reshape(re.shape[:-2] + (n,))
        im = np.concatenate([ui + ti, ui - ti], axis=-1).reshape(im.shape[:-2] + (n,))
        m *= 2
    return re, im


def rfft_radix2_f32(x, n=None):
    """The reference's float32 arithmetic for rfft (see module docstring)."""
    x = np.asarray(x, np.float32)
    n = x.shape[-1] if n is None else int(n)
    xr = _fit(x, n).astype(np.float32)
    z = xr[..., _bitrev_perm(n)].astype(np.complex64)
    re, im = _radix2_f32(z, inverse=False)
    half = n // 2 + 1
    return (re[..., :half] + 1j * im[..., :half]).astype(np.complex64)


def irfft_radix2_f32(X, n=None):
    """The reference's float32 arithmetic for irfft."""
    X = np.asarray(X, np.complex64)
    n = 2 * (X.shape[-1] - 1) if n is None else int(n)
    in_len = X.shape[-1]
    full = np.zeros(X.shape[:-1] + (n,), np.complex64)
    for i in range(n):
        if i <= n // 2:
            if i < in_len:
                full[..., i] = X[..., i]
        else:
            mirror = n - i
            if mirror < in_len:
                full[..., i] = np.conj(X[..., mirror])
    z = full[..., _bitrev_perm(n)]
    re, _ = _radix2_f32(z, inverse=True)
    return (re * np.float32(1.0 / n)).astype(np.float32)


def complex_mul(a, b, conj_a=False, conj_b=False):
    a = np.asarray(a, np.complex64)
    b = np.asarray(b, np.complex64)
    if conj_a:
        a = np.conj(a)
    if conj_b:
        b = np.conj(b)
    return (a * b).astype(np.complex64)


def complex_pad(x, out_len):
    x = np.asarray(x, np.complex64)
    k = x.shape[-1]
    if out_len <= k:
        return x[..., :out_len].copy()
    return np.concatenate([x, np.zeros(x.shape[:-1] + (out_len - k,), np.complex64)], axis=-1)
