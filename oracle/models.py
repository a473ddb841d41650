"""GPT-2 train step restated in float64 numpy (test infrastructure only).

Follows reference src/wxx/nn/gpt.py:23-120 and nn/module.py:447-495 with the
op semantics of the kernels it calls:
* embeddings: tok[x] + pos[arange(S)] (embed.wgsl);
* LayerNorm (meanvarnorm.wgsl:29-111): var = max(0, E[x^2] - mu^2),
  inv = 1/sqrt(var + 1e-5) when var > 0 else 0;
* attention: (q k^T) * (1/sqrt(d_head)) + mask, mask 0 on/below the diagonal
  and -1e9 above (gpt.py:75-96), softmax (softmax.wgsl), attn @ v;
* MLP: gelu(a W1 + b1) W2 + b2 with the tanh GELU clamped at +-10
  (gelu.wgsl:20-27, gelubackwards.wgsl:21-32);
* tied head logits = h tok^T; loss = mean over rows of
  log(sum exp(z - m)) + m - z[t] (cceloss.wgsl, nn/loss.py:26-44);
* dropout p = 0 keeps every element with scale 1 (dropout.wgsl).
The backward is written out by hand from those definitions.

``adamw_sequence`` replays the reference optimizer loop (nn/optimizer.py:59-84)
over the parameter list as ``named_parameters`` yields it, aliases included:
LayerNorm's ``weight``/``bias`` are the same tensors as ``weightg``/``weightb``
(module.py:198-208), so those tensors are updated twice per step, each time
with moment buffers of their own.
"""

import numpy as np

SQRT_2_OVER_PI = 0.7978845608
GELU_C = 0.044715


def _ln(x, g, b, eps=1e-5):
    mu = x.mean(axis=-1, keepdims=True)
    var = np.maximum(0.0, (x * x).mean(axis=-1, keepdims=True) - mu * mu)
    inv = np.where(var > 0, 1.0 / np.sqrt(np.where(var > 0, var + eps, 1.0)), 0.0)
    xh = (x - mu) * inv
    return xh * g + b, (xh, inv)


def _ln_back(dy, g, cache):
    xh, inv = cache
    n = xh.shape[-1]
    gdy = dy * g
    c1 = gdy.sum(axis=-1, keepdims=True) / n
    c2 = (gdy * xh).sum(axis=-1, keepdims=True) / n
    dx = inv * (gdy - c1 - xh * c2)
    red = tuple(range(dy.ndim - 1))
    return dx, (dy * xh).sum(axis=red), dy.sum(axis=red)


def _gelu(x):
    u = SQRT_2_OVER_PI * (x + GELU_C * x ** 3)
    y = 0.5 * x * (1.0 + np.tanh(u))
    return np.where(x > 10.0, x, np.where(x < -10.0, 0.0, y))


def _gelu_grad(x):
    u = SQRT_2_OVER_PI * (x + GELU_C * x ** 3)
    t = np.tanh(u)
    d = 0.5 * (1.0 + t) + 0.5 * x * (1.0 - t * t) * SQRT_2_OVER_PI * (1.0 + 3 * GELU_C * x * x)
    return np.where(x > 10.0, 1.0, np.where(x < -10.0, 0.0, d))


def _softmax(x):
    m = np.maximum(x.max(axis=-1, keepdims=True), -1e38)
    e = np.exp(x - m)
    return e / e.sum(axis=-1, keepdims=True)


def _outer_sum(a, b):
    """sum over (batch, seq) of a[..., i] b[..., o]: one BLAS product
    (config-5 sizes are far too slow through einsum's loops)."""
    return a.reshape(-1, a.shape[-1]).T @ b.reshape(-1, b.shape[-1])


def gpt2_loss_and_grads(params, x, y, n_heads, n_layers):
    """Loss and gradients (keyed by the tensors' first names: ``weightg`` /
    ``weightb`` for LayerNorm) of one GPT-2 forward + backward."""
    P = {k: np.asarray(v, np.float64) for k, v in params.items()}
    x = np.asarray(x, np.int64)
    y = np.asarray(y, np.int64).reshape(-1)
    B, S = x.shape
    tok, pos = P["tok_emb.weight"], P["pos_emb.weight"]
    V, D = tok.shape
    H, hd = n_heads, D // n_heads
    mask = np.where(np.arange(S)[None, :] <= np.arange(S)[:, None], 0.0, -1e9)
    scale = 1.0 / np.sqrt(hd)

    def heads(t):
        return t.reshape(B, S, H, hd).transpose(0, 2, 1, 3)

    def merge(t):
        return t.transpose(0, 2, 1, 3).reshape(B, S, D)

    h = tok[x] + pos[np.arange(S)][None]
    caches = []
    for i in range(n_layers):
        p = f"blocks.{i}."
        a, c1 = _ln(h, P[p + "ln1.weightg"], P[p + "ln1.weightb"])
        q, k, v = (heads(a @ P[p + f"attn.{n}.weight"]) for n in ("q", "k", "v"))
        att = _softmax(q @ k.transpose(0, 1, 3, 2) * scale + mask)
        o = merge(att @ v)
        h1 = h + o @ P[p + "attn.out.weight"]
        a2, c2 = _ln(h1, P[p + "ln2.weightg"], P[p + "ln2.weightb"])
        z1 = a2 @ P[p + "mlp.0.weight"] + P[p + "mlp.0.bias"]
        g1 = _gelu(z1)
        h2 = h1 + g1 @ P[p + "mlp.2.weight"] + P[p + "mlp.2.bias"]
        caches.append((a, c1, q, k, v, att, o, h1, a2, c2, z1, g1))
        h = h2
    hf, cf = _ln(h, P["ln_f.weightg"], P["ln_f.weightb"])
    logits = hf @ tok.T
    z = logits.reshape(-1, V)
    m = np.maximum(z.max(axis=1), -1e38)
    e = np.exp(z - m[:, None])
    s = e.sum(axis=1)
    rows = np.arange(z.shape[0])
    loss = float(np.mean(np.log(s) + m - z[rows, y]))

    G = {k: np.zeros_like(v) for k, v in P.items()}
    dz = e / s[:, None]
    dz[rows, y] -= 1.0
    dz /= z.shape[0]
    dlog = dz.reshape(B, S, V)
    G["tok_emb.weight"] += _outer_sum(dlog, hf)
    dhf = dlog @ tok
    dh, dg, db = _ln_back(dhf, P["ln_f.weightg"], cf)
    G["ln_f.weightg"] += dg
    G["ln_f.weightb"] += db
    for i in reversed(range(n_layers)):
        p = f"blocks.{i}."
        a, c1, q, k, v, att, o, h1, a2, c2, z1, g1 = caches[i]
        # MLP
        G[p + "mlp.2.bias"] += dh.sum(axis=(0, 1))
        G[p + "mlp.2.weight"] += _outer_sum(g1, dh)
        dz1 = (dh @ P[p + "mlp.2.weight"].T) * _gelu_grad(z1)
        G[p + "mlp.0.bias"] += dz1.sum(axis=(0, 1))
        G[p + "mlp.0.weight"] += _outer_sum(a2, dz1)
        da2 = dz1 @ P[p + "mlp.0.weight"].T
        dx2, dg2, db2 = _ln_back(da2, P[p + "ln2.weightg"], c2)
        G[p + "ln2.weightg"] += dg2
        G[p + "ln2.weightb"] += db2
        dh1 = dh + dx2
        # attention
        G[p + "attn.out.weight"] += _outer_sum(o, dh1)
        do = heads(dh1 @ P[p + "attn.out.weight"].T)
        datt = do @ v.transpose(0, 1, 3, 2)
        dv = att.transpose(0, 1, 3, 2) @ do
        dsc = att * (datt - (datt * att).sum(axis=-1, keepdims=True)) * scale
        dq = dsc @ k
        dk = dsc.transpose(0, 1, 3, 2) @ q
        da = np.zeros_like(a)
        for n, dt in (("q", dq), ("k", dk), ("v", dv)):
            dt = merge(dt)
            G[p + f"attn.{n}.weight"] += _outer_sum(a, dt)
            da += dt @ P[p + f"attn.{n}.weight"].T
        dx1, dg1, db1 = _ln_back(da, P[p + "ln1.weightg"], c1)
        G[p + "ln1.weightg"] += dg1
        G[p + "ln1.weightb"] += db1
        dh = dh1 + dx1
    np.add.at(G["tok_emb.weight"], x.reshape(-1), dh.reshape(-1, D))
    G["pos_emb.weight"][:S] += dh.sum(axis=0)
    return loss, G


def adamw_apply(p, g, m, v, lr, beta1, beta2, eps, wd, bc1, bc2):
    """adamw.wgsl:39-54 in float64."""
    m = beta1 * m + (1.0 - beta1) * g
    v = beta2 * v + (1.0 - beta2) * g * g
    p = p - lr * ((m / bc1) / (np.sqrt(v / bc2) + eps) + wd * p)
    return p, m, v


def adamw_sequence(params, grads, order, states, step, lr, beta1=0.9, beta2=0.999, eps=1e-7,
                   weight_decay=1e-4):
    """One optimizer step over ``order`` (storage keys in ``named_parameters``
    order, an aliased tensor appearing once per name).  ``states[i]`` is the
    (m, v) pair of entry i and is updated in place; returns the new params."""
    bc1 = 1.0 - beta1 ** step
    bc2 = 1.0 - beta2 ** step
    out = {k: np.asarray(v, np.float64).copy() for k, v in params.items()}
    for i, key in enumerate(order):
        m, v = states[i]
        out[key], m, v = adamw_apply(out[key], grads[key], m, v, lr, beta1, beta2, eps,
                                     weight_decay, bc1, bc2)
        states[i] = (m, v)
    return out
