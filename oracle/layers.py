"""Cross-entropy, AdamW, gradient-norm clipping, embedding, dropout and the
Hyena decay window, restated from the reference (test infrastructure only).

* cceloss (shaders/loss/cceloss.wgsl:21-85, host functional/loss.py:20-101):
  m = max(-1e38, max_j z_j), s = sum_j exp(z_j - m),
  loss = (log s + m) - z[t], dz_j = exp(z_j - m) / s - [j == t].
* adamw (shaders/optimizers/adamw.wgsl:35-56; bc1/bc2 from
  nn/optimizer.py:60-63): m = b1 m + (1-b1) g; v = b2 v + (1-b2) g g;
  p = p - lr (m/bc1 / (sqrt(v/bc2) + eps) + wd p), all in float32 in that
  order.
* clip_grad_norm (nn/utils.py:62-103): norm = sqrt(sum_g sum(g^2));
  coef = max_norm / (norm + 1e-6); grads *= coef only when coef < 1.
* embed / embeddx (shaders/layers/embed.wgsl:22-36, embeddx.wgsl:22-47):
  out[t] = W[id[t]]; grad[v] = sum over tokens with id == v (ids >= V are
  skipped in the backward).
* dropout (shaders/layers/dropout.wgsl:14-36, host functional/layers.py:73-115):
  h(x) = ((x>>16)^x)*0x45d9f3b twice, then (x>>16)^x, in uint32; element i is
  kept when f32(h(i ^ seed) >> 8) * 2^-24 >= p; kept values are x * 1/(1-p).
* decay_window (shaders/helpers/decay_window.wgsl:22-33): W[d, t] =
  exp(-|r[stage, d]| t); backward (decay_window_backward.wgsl:24-46):
  out[stage, d] = sum_t g[d, t] W[d, t] (-sign(r) t), other rows zero.
"""

import numpy as np


def cceloss(z, targets):
    z = np.asarray(z, np.float64)
    t = np.asarray(targets, np.int64).reshape(-1)
    B, K = z.shape
    if t.max(initial=0) >= K:
        raise ValueError("target out of range")
    m = np.maximum(-1e38, z.max(axis=1))
    e = np.exp(z - m[:, None])
    s = e.sum(axis=1)
    loss = (np.log(s) + m) - z[np.arange(B), t]
    dz = e / s[:, None]
    dz[np.arange(B), t] -= 1.0
    return loss.reshape(B, 1).astype(np.float32), dz.astype(np.float32)


def adamw(p, g, m, v, lr, beta1, beta2, eps, weight_decay, bc1, bc2):
    """Returns the updated (p, m, v) as new float32 arrays."""
    f = np.float32
    p = np.asarray(p, f)
    g = np.asarray(g, f)
    m = f(beta1) * np.asarray(m, f) + (f(1.0) - f(beta1)) * g
    v = f(beta2) * np.asarray(v, f) + (f(1.0) - f(beta2)) * g * g
    m_hat = m / f(bc1)
    v_hat = v / f(bc2)
    step = m_hat / (np.sqrt(v_hat) + f(eps))
    p = p - f(lr) * (step + f(weight_decay) * p)
    return p.astype(f), m.astype(f), v.astype(f)


def bias_corrections(step, beta1, beta2):
    """bc1, bc2 as the reference's AdamW.step computes them (nn/optimizer.py:60-63)."""
    return 1.0 - beta1 ** step, 1.0 - beta2 ** step


def clip_grad_norm(grads, max_norm):
    """Returns (total_norm, clipped grads) in float64."""
    total = sum(float(np.sum(np.asarray(g, np.float64) ** 2)) for g in grads)
    norm = total ** 0.5
    coef = max_norm / (norm + 1e-6)
    if coef < 1.0:
        return norm, [np.asarray(g, np.float64) * coef for g in grads]
    return norm, [np.asarray(g, np.float64) for g in grads]


def embed(ids, W):
    return np.asarray(W)[np.asarray(ids, np.int64)]


def embeddx(g, ids, vocab_size):
    g = np.asarray(g, np.float64)
    ids = np.asarray(ids, np.int64).reshape(-1)
    D = g.shape[-1]
    g = g.reshape(-1, D)[: ids.size]
    out = np.zeros((vocab_size, D), np.float64)
    ok = ids < vocab_size
    np.add.at(out, ids[ok], g[ok])
    return out


def dropout_hash(x):
    """The reference's 32-bit integer hash, vectorised over uint32 arrays."""
    x = np.asarray(x, np.uint32).astype(np.uint64)
    mask = np.uint64(0xFFFFFFFF)
    x = (((x >> np.uint64(16)) ^ x) * np.uint64(0x45D9F3B)) & mask
    x = (((x >> np.uint64(16)) ^ x) * np.uint64(0x45D9F3B)) & mask
    x = (x >> np.uint64(16)) ^ x
    return x.astype(np.uint32)


def dropout_keep(n, seed, p):
    idx = np.arange(n, dtype=np.uint64).astype(np.uint32)
    h = dropout_hash(idx ^ np.uint32(seed & 0xFFFFFFFF))
    r = (h >> np.uint32(8)).astype(np.float32) * np.float32(1.0 / 16777216.0)
    return r >= np.float32(p)


def dropout(x, seed, p):
    x = np.asarray(x, np.float32)
    keep = dropout_keep(x.size, seed, p).reshape(x.shape)
    scale = np.float32(1.0 / (1.0 - p))
    return np.where(keep, x * scale, np.float32(0.0)).astype(np.float32)


def decay_window(decay, stage, length):
    r = np.asarray(decay, np.float64)[stage]
    t = np.arange(length, dtype=np.float64)
    return np.exp(-np.abs(r)[:, None] * t[None, :])


def decay_window_backward(g, decay, stage, length):
    decay = np.asarray(decay, np.float64)
    rows, channels = decay.shape
    r = decay[stage]
    t = np.arange(length, dtype=np.float64)
    w = np.exp(-np.abs(r)[:, None] * t[None, :])
    out = np.zeros((rows, channels), np.float64)
    out[stage] = (np.asarray(g, np.float64).reshape(channels, length) * w
                  * (-np.sign(r)[:, None] * t[None, :])).sum(axis=1)
    return out
