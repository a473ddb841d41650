"""Multi-head attention restated from the reference (test infrastructure only).

Forward (reference src/wxx/nn/module.py:460-495, MultiHeadAttention): the
(B, S, D) projections q, k, v are split into H heads of d = D / H
((B, S, H, d) -> (B * H, S, d)), then
    scores = (q k^T) * (1 / sqrt(d));  scores += mask  (GPT-2's causal mask:
             -1e9 above the diagonal, nn/gpt.py causal_mask);
    probs  = softmax(scores, -1);  probs = dropout(probs)  (flat index of the
             (B * H, S, S) probabilities, oracle.layers.dropout_keep);
    out    = probs v, merged back to (B, S, D).
Backward: with Z the keep mask scaled by 1 / (1 - p) and P the softmax,
    dV = (P o Z)^T dO,  dP = (dO V^T) o Z,  dS = P o (dP - rowsum(P o dP)),
    dQ = scale dS K,  dK = scale dS^T Q
(the chain rule through the reference's ops: matmul, scalar multiply, mask
add, softmax (functional/reductions.py softmax backward), dropout).

Pinned by tests/test_oracle_models.py against torch's float64
scaled_dot_product_attention (forward, causal and not) and torch autograd
of the same composition with the dropout mask as a constant (gradients).
"""

import math

import numpy as np

from .layers import dropout_keep

MASKED = -1e9


def _split(t, H):
    B, S, D = t.shape
    return t.reshape(B, S, H, D // H).transpose(0, 2, 1, 3).reshape(B * H, S, D // H)


def _merge(t, B, H):
    BH, S, d = t.shape
    return t.reshape(B, H, S, d).transpose(0, 2, 1, 3).reshape(B, S, H * d)


def _keep(B, H, S, p, seed, dtype):
    """The dropout multiplier Z (keep / (1 - p), else 0) over (B * H, S, S),
    or None without dropout."""
    if not p:
        return None
    keep = dropout_keep(B * H * S * S, seed, p).reshape(B * H, S, S)
    return np.where(keep, dtype(1.0 / (1.0 - p)), dtype(0.0)).astype(dtype)


def _probs(q, k, H, causal, dtype):
    d = q.shape[2] // H
    qs, ks = _split(q, H), _split(k, H)
    scores = (qs @ ks.transpose(0, 2, 1)) * dtype(1.0 / math.sqrt(d))
    S = q.shape[1]
    if causal:
        scores = scores + np.triu(np.full((S, S), MASKED, dtype), k=1)
    e = np.exp(scores - scores.max(axis=-1, keepdims=True))
    return (e / e.sum(axis=-1, keepdims=True)).astype(dtype)


def attention(q, k, v, n_heads, causal, p=0.0, seed=0, dtype=np.float64):
    """(B, S, D) output of the reference's attention path in ``dtype``."""
    q, k, v = (np.asarray(t, dtype) for t in (q, k, v))
    B, S, _ = q.shape
    P = _probs(q, k, n_heads, causal, dtype)
    Z = _keep(B, n_heads, S, p, seed, dtype)
    Pd = P if Z is None else P * Z
    return _merge(Pd @ _split(v, n_heads), B, n_heads)


def attention_grads(q, k, v, dout, n_heads, causal, p=0.0, seed=0, dtype=np.float64):
    """(dq, dk, dv), each (B, S, D), for the upstream gradient ``dout``."""
    q, k, v, dout = (np.asarray(t, dtype) for t in (q, k, v, dout))
    B, S, D = q.shape
    H = n_heads
    scale = dtype(1.0 / math.sqrt(D // H))
    P = _probs(q, k, H, causal, dtype)
    Z = _keep(B, H, S, p, seed, dtype)
    qs, ks, vs, dos = (_split(t, H) for t in (q, k, v, dout))
    Pd = P if Z is None else P * Z
    dv = Pd.transpose(0, 2, 1) @ dos
    dP = dos @ vs.transpose(0, 2, 1)
    if Z is not None:
        dP = dP * Z
    dS = P * (dP - (P * dP).sum(axis=-1, keepdims=True))
    dq = (dS @ ks) * scale
    dk = (dS.transpose(0, 2, 1) @ qs) * scale
    return tuple(_merge(t, B, H) for t in (dq, dk, dv))
