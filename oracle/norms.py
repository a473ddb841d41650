"""LayerNorm, RMSNorm and BatchNorm restated from the reference (test
infrastructure only).  Statistics are accumulated in float64 (or, with
``dtype=np.float32``, in single precision: the rounding floor an fp32
evaluation of the same formulas carries) and follow the reference's
formulas, including its special cases:

* LayerNorm (meanvarnorm.wgsl:29-111): single pass mu = S/n,
  var = max(0, Q/n - mu^2), inv_std = var > 0 ? 1/sqrt(var + eps) : 0,
  eps 1e-5 (src/wxx/functional/normalization.py:94).
* LayerNorm dx (meanvarnormdx.wgsl:44-89) and dgamma/dbeta
  (meanvarnormdg.wgsl:36-58) from the saved (mean, inv_std).
* RMSNorm (rmsnorm.wgsl:33-79): r = ms > 0 ? 1/sqrt(ms + 1e-6) : 0;
  dx (rmsnormdx.wgsl:29-69), dgamma (rmsnormdg.wgsl:29-54).
* BatchNorm (batchnorm.wgsl:39-111): var = max(0, E[x^2] - mu^2),
  inv = 1/sqrt(var + 1e-5) without a zero rule, running stats
  (1-m) r + m s with the unbiased variance M/(M-1); dx/dgamma/dbeta from
  batchnormdx.wgsl:43-48 and batchnormdg.wgsl:43-73.
* ``row_cap``: rows >= cap are zeros (the reference's 65 535 row limit).
"""

import numpy as np

from .reductions import reduce_dims


def _view(x, axis):
    outer, red, inner, out_shape = reduce_dims(x.shape, axis)
    return x.reshape(outer, red, inner), out_shape


def meanvarnorm(x, gamma, beta, axis=-1, eps=1e-5, row_cap=0, dtype=np.float64):
    x = np.asarray(x, dtype=np.float32)
    v, out_shape = _view(x.astype(dtype), axis)
    n = v.shape[1]
    mu = v.sum(axis=1) / n
    var = np.maximum(0.0, (v * v).sum(axis=1) / n - mu * mu)
    safe = np.where(var > 0, var + eps, 1.0)
    inv = np.where(var > 0, 1.0 / np.sqrt(safe), 0.0)
    g = np.asarray(gamma, dtype).reshape(1, n, 1)
    b = np.asarray(beta, dtype).reshape(1, n, 1)
    y = (v - mu[:, None, :]) * inv[:, None, :] * g + b
    if row_cap:
        y[row_cap:] = 0.0
        mu[row_cap:] = 0.0
        inv[row_cap:] = 0.0
    return (
        y.astype(np.float32).reshape(x.shape),
        mu.astype(np.float32).reshape(out_shape),
        inv.astype(np.float32).reshape(out_shape),
    )


def meanvarnormdx(dy, x, gamma, mean, inv_std, axis=-1, row_cap=0, dtype=np.float64):
    x = np.asarray(x, np.float32)
    v, _ = _view(x.astype(dtype), axis)
    d, _ = _view(np.asarray(dy, dtype), axis)
    n = v.shape[1]
    mu = np.asarray(mean, dtype).reshape(v.shape[0], 1, v.shape[2])
    inv = np.asarray(inv_std, dtype).reshape(v.shape[0], 1, v.shape[2])
    db = d * np.asarray(gamma, dtype).reshape(1, n, 1)
    xh = (v - mu) * inv
    c1 = db.sum(axis=1, keepdims=True) / n
    c2 = (db * xh).sum(axis=1, keepdims=True) / n
    dx = inv * (db - c1 - xh * c2)
    if row_cap:
        dx[row_cap:] = 0.0
    return dx.astype(np.float32).reshape(x.shape)


def meanvarnormdg(dy, x, mean, inv_std, axis=-1, dtype=np.float64):
    x = np.asarray(x, np.float32)
    v, _ = _view(x.astype(dtype), axis)
    d, _ = _view(np.asarray(dy, dtype), axis)
    mu = np.asarray(mean, dtype).reshape(v.shape[0], 1, v.shape[2])
    inv = np.asarray(inv_std, dtype).reshape(v.shape[0], 1, v.shape[2])
    xh = (v - mu) * inv
    dg = (d * xh).sum(axis=(0, 2))
    db = d.sum(axis=(0, 2))
    return dg.astype(np.float32), db.astype(np.float32)


def rmsnorm(x, gamma, axis=-1, eps=1e-6, row_cap=0, dtype=np.float64):
    x = np.asarray(x, dtype=np.float32)
    v, out_shape = _view(x.astype(dtype), axis)
    n = v.shape[1]
    ms = (v * v).sum(axis=1) / n
    r = np.where(ms > 0, 1.0 / np.sqrt(np.where(ms > 0, ms + eps, 1.0)), 0.0)
    y = v * r[:, None, :] * np.asarray(gamma, dtype).reshape(1, n, 1)
    if row_cap:
        y[row_cap:] = 0.0
        r[row_cap:] = 0.0
    return y.astype(np.float32).reshape(x.shape), r.astype(np.float32).reshape(out_shape)


def rmsnormdx(dy, x, gamma, inv_rms, axis=-1, dtype=np.float64):
    x = np.asarray(x, np.float32)
    v, _ = _view(x.astype(dtype), axis)
    d, _ = _view(np.asarray(dy, dtype), axis)
    n = v.shape[1]
    r = np.asarray(inv_rms, dtype).reshape(v.shape[0], 1, v.shape[2])
    db = d * np.asarray(gamma, dtype).reshape(1, n, 1)
    c = (r * r / n) * (db * v).sum(axis=1, keepdims=True)
    return (r * (db - v * c)).astype(np.float32).reshape(x.shape)


def rmsnormdg(dy, x, inv_rms, axis=-1, dtype=np.float64):
    x = np.asarray(x, np.float32)
    v, _ = _view(x.astype(dtype), axis)
    d, _ = _view(np.asarray(dy, dtype), axis)
    r = np.asarray(inv_rms, dtype).reshape(v.shape[0], 1, v.shape[2])
    return (d * v * r).sum(axis=(0, 2)).astype(np.float32)


def batchnorm(x, gamma, beta, running_mean, running_var, training, eps=1e-5, momentum=0.1,
              dtype=np.float64):
    """Returns (y, saved_mean, inv_std, new_running_mean, new_running_var)."""
    x64 = np.asarray(x, dtype)
    B, C, H, W = x64.shape
    M = B * H * W
    rm = np.asarray(running_mean, dtype).copy()
    rv = np.asarray(running_var, dtype).copy()
    if training:
        mu = x64.sum(axis=(0, 2, 3)) / M
        var = np.maximum(0.0, (x64 * x64).sum(axis=(0, 2, 3)) / M - mu * mu)
        inv = 1.0 / np.sqrt(var + eps)
        rm = (1 - momentum) * rm + momentum * mu
        unb = var * (M / (M - 1.0)) if M > 1 else var
        rv = (1 - momentum) * rv + momentum * unb
    else:
        mu = rm.copy()
        inv = 1.0 / np.sqrt(rv + eps)
    g = np.asarray(gamma, dtype).reshape(1, C, 1, 1)
    b = np.asarray(beta, dtype).reshape(1, C, 1, 1)
    y = (x64 - mu.reshape(1, C, 1, 1)) * inv.reshape(1, C, 1, 1) * g + b
    f = np.float32
    return y.astype(f), mu.astype(f), inv.astype(f), rm.astype(f), rv.astype(f)


def batchnormdg(dy, x, mean, inv_std, dtype=np.float64):
    x64 = np.asarray(x, dtype)
    C = x64.shape[1]
    xh = (x64 - np.asarray(mean, dtype).reshape(1, C, 1, 1)) * np.asarray(
        inv_std, dtype
    ).reshape(1, C, 1, 1)
    d = np.asarray(dy, dtype)
    return (d * xh).sum(axis=(0, 2, 3)).astype(np.float32), d.sum(axis=(0, 2, 3)).astype(np.float32)


def batchnormdx(dy, x, gamma, dgamma, dbeta, mean, inv_std, dtype=np.float64):
    x64 = np.asarray(x, dtype)
    B, C, H, W = x64.shape
    M = float(B * H * W)

    def r(a):
        return np.asarray(a, dtype).reshape(1, C, 1, 1)

    xh = (x64 - r(mean)) * r(inv_std)
    dx = (r(gamma) * r(inv_std) / M) * (M * np.asarray(dy, dtype) - r(dbeta) - xh * r(dgamma))
    return dx.astype(np.float32)
