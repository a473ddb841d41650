"""Hyena language model restated in float64 on the CPU (TEST INFRASTRUCTURE ONLY).

The forward pass follows the reference module tree op by op
(src/wxx/nn/hyena.py:96-246, nn/module.py:172-236, 525-597) with the
semantics of the kernels it calls:

* embedding gather ``W[ids]`` (embed.wgsl);
* RMSNorm ``y = x r gamma`` with ``r = 1/sqrt(mean(x^2) + 1e-6)`` when
  ``mean(x^2) > 0`` else 0 (rmsnorm.wgsl:57-60).  With ``row_cap`` the rows
  at or beyond it (counted over all leading dims) yield 0, as the
  reference's 65 535-row dispatch cap leaves them (rmsnorm.wgsl:23-24,
  normalization.py:64);
* Linear layers with W stored (in, out) (module.py:154-169), the tied head
  ``h W_embed^T`` (module.py:555-562);
* the depthwise causal short convolution ``y[b,d,n] = bias[d] +
  sum_k w[d,k] x[b,d,n-k]`` (causal_conv1d.wgsl);
* the implicit filter: positional encoding built in float32 exactly as
  module.py:576-584 does (``t = linspace(0, 1, L)``, angles ``2 pi t k``),
  ``Linear -> sin(omega x) -> Linear``, transposed to (d, L), times the
  decay window ``exp(-|decay[i, d]| t)`` with integer ``t``
  (decay_window.wgsl);
* the long convolution ``irfft(rfft(z, n) rfft(h, n), n)[..., :L]`` with
  ``n = next_pow2(2 L)`` (hyena.py:208-216), the order-n gating chain
  ``z_i = x_i (h_i * z_{i-1})`` (hyena.py:224-242);
* SwiGLU ``w3(silu(w1 x) * w2 x)`` with ``silu(x) = sigmoid(x) x`` and the
  sigmoid's input clamped to [-88, 88] (module.py:541-552, Tensor.py:724-727,
  sigmoid.wgsl:20);
* the loss of CCELoss: mean over rows of ``logsumexp(z) - z[target]``.

Gradients are taken by torch's float64 autograd of that forward.  The
oracle is pinned in tests/test_oracle_models.py against the numpy per-op
oracles (which have their own pins), finite differences of the loss, and
the parameter count the reference's own test holds.
"""

import numpy as np
import torch

F64 = torch.float64


def next_pow2(n):
    n = int(n)
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


def positional_encoding(length, features):
    """(L, 2K + 1) float32 table of module.py:576-584, returned as float64."""
    t = np.linspace(0.0, 1.0, int(length), dtype=np.float32)
    k = np.arange(features, dtype=np.float32)
    ang = (2.0 * np.pi) * np.outer(t, k)
    pe = np.concatenate([t[:, None], np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)
    return torch.tensor(pe.astype(np.float64))


def rmsnorm(x, gamma, eps=1e-6, row_cap=0):
    ms = (x * x).mean(dim=-1, keepdim=True)
    safe = torch.where(ms > 0, ms, torch.ones_like(ms))
    r = torch.where(ms > 0, 1.0 / torch.sqrt(safe + eps), torch.zeros_like(ms))
    y = x * r * gamma
    if row_cap:
        rows = y.reshape(-1, y.shape[-1])
        keep = (torch.arange(rows.shape[0]) < row_cap).to(F64)[:, None]
        y = (rows * keep).reshape(y.shape)
    return y


def causal_short_conv(x, w, b):
    """x (B, D, L); y[..., n] = b + sum_k w[:, k] x[..., n - k]."""
    ks = w.shape[1]
    L = x.shape[-1]
    y = b[None, :, None].expand(x.shape[0], -1, L).clone()
    for k in range(ks):
        if k == 0:
            y = y + w[None, :, 0:1] * x
        elif k < L:
            shifted = torch.nn.functional.pad(x[..., : L - k], (k, 0))
            y = y + w[None, :, k:k + 1] * shifted
    return y


def fft_conv(z, h):
    """Linear causal convolution of z (B, D, L) with h (D, L) through an
    n = next_pow2(2 L) real FFT, cropped to L (hyena.py:208-216)."""
    L = z.shape[-1]
    n = next_pow2(2 * L)
    if n < L:
        n = next_pow2(L)
    spec = torch.fft.rfft(z, n=n) * torch.fft.rfft(h, n=n)
    return torch.fft.irfft(spec, n=n)[..., :L]


def sigmoid(x):
    return 1.0 / (1.0 + torch.exp(-torch.clamp(x, -88.0, 88.0)))


def hyena_forward(P, ids, n_layers, order, pe_features=8, omega=10.0, row_cap=0,
                  tie_weights=True):
    """Logits (B, L, V) of the model with parameters ``P`` (name -> float64
    tensor, the names of ``Hyena.named_parameters``)."""
    ids = torch.as_tensor(np.asarray(ids, np.int64))
    B, L = ids.shape
    W = P["embed.weight"]
    D = W.shape[1]
    h = W[ids]
    pe = positional_encoding(L, pe_features)
    t = torch.arange(L, dtype=F64)
    for li in range(n_layers):
        p = f"layers.{li}."
        m = p + "mixer."
        a = rmsnorm(h, P[p + "norm1.weight"], row_cap=row_cap)
        v = (a @ P[m + "proj_v.weight"]).transpose(1, 2)
        gates = [g.transpose(1, 2) for g in torch.chunk(a @ P[m + "proj_x.weight"], order, dim=-1)]
        cw, cb = P[m + "short_conv.weight"], P[m + "short_conv.bias"]
        z = causal_short_conv(v, cw, cb)
        gates = [causal_short_conv(g, cw, cb) for g in gates]
        for i in range(order):
            f = f"{m}filter_mlp.{i}.mlp."
            hid = torch.sin(omega * (pe @ P[f + "0.weight"] + P[f + "0.bias"]))
            filt = (hid @ P[f + "2.weight"] + P[f + "2.bias"]).transpose(0, 1)  # (D, L)
            window = torch.exp(-torch.abs(P[m + "decay"][i])[:, None] * t[None, :])
            z = gates[i] * fft_conv(z, filt * window)
        h = h + z.transpose(1, 2) @ P[m + "out_proj.weight"]
        a2 = rmsnorm(h, P[p + "norm2.weight"], row_cap=row_cap)
        u = a2 @ P[p + "feed_forward.w1.weight"]
        h = h + ((sigmoid(u) * u) * (a2 @ P[p + "feed_forward.w2.weight"])) @ \
            P[p + "feed_forward.w3.weight"]
    hn = rmsnorm(h, P["norm.weight"], row_cap=row_cap)
    if tie_weights:
        return hn @ W.transpose(0, 1)
    return hn @ P["head.weight"] + P["head.bias"]


def cce_mean(logits, targets):
    z = logits.reshape(-1, logits.shape[-1])
    tg = torch.as_tensor(np.asarray(targets, np.int64).reshape(-1))
    return (torch.logsumexp(z, dim=1) - z[torch.arange(z.shape[0]), tg]).mean()


def hyena_loss_and_grads(params, ids, targets, n_layers, order, **kw):
    """(loss, {name: float64 gradient}) of CCELoss(Hyena(ids), targets)."""
    torch.set_num_threads(max(1, min(16, torch.get_num_threads())))
    P = {k: torch.tensor(np.asarray(v, np.float64), requires_grad=True) for k, v in params.items()}
    loss = cce_mean(hyena_forward(P, ids, n_layers, order, **kw), targets)
    loss.backward()
    return float(loss.detach()), {k: v.grad.numpy() if v.grad is not None else np.zeros(v.shape)
                         for k, v in P.items()}


def hyena_param_count(vocab, d_model, n_layers, order, mlp_ratio=4, short_conv_kernel=3,
                      filter_hidden=64, pe_features=8):
    """Parameters of Hyena(vocab, d_model, n_layers, order=order) with a tied
    head, counted from the module tree above."""
    hidden = int(2 * (mlp_ratio * d_model) / 3)
    pe = 2 * pe_features + 1
    filt = (pe * filter_hidden + filter_hidden) + (filter_hidden * d_model + d_model)
    mixer = (d_model * d_model + d_model * order * d_model + d_model * d_model
             + d_model * short_conv_kernel + d_model + order * filt + order * d_model)
    block = 2 * d_model + mixer + 3 * d_model * hidden
    return vocab * d_model + n_layers * block + d_model
