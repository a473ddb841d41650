"""Fused multi-head attention (the reference composes it from projections,
head permutes, two matmuls, a softmax and dropout: nn/module.py:460-495).

``q``, ``k`` and ``v`` are the (B, S, D) outputs of the three projections;
head h of row (b, s) is columns [h d, (h + 1) d) with d = D / n_heads.  The
result is the merged (B, S, D) context that the reference feeds to the output
projection, so no head permute is materialised.  Only the per-row
log-sum-exp (B * H * S floats) is kept for the backward instead of the
(B * H, S, S) probabilities.
"""

import ctypes as C
import math
import random

from .. import graphs
from ._common import call, empty, ptr
from .layers import DeviceSeed, _draw_seed

HEAD_DIMS = (32, 64, 128)
"""Head sizes the fused kernels are built for."""


def supported(x, n_heads):
    """Whether the fused kernels take (B, S, D) f32 projections with ``n_heads`` heads."""
    if x.type != "f32" or len(x.shape) != 3 or n_heads <= 0 or x.shape[2] % n_heads:
        return False
    return x.shape[2] // n_heads in HEAD_DIMS


def _seed_args(seed):
    if isinstance(seed, DeviceSeed):
        return 0, C.c_void_p(seed.ptr)
    return int(seed) & 0xFFFFFFFF, None


def draw_seed():
    """The dropout seed of one attention call, drawn as the reference's
    Dropout module draws it (one host RNG draw per training call), or a
    per-replay device word inside a step graph recording."""
    if graphs.capturing():
        return DeviceSeed(graphs.per_replay(1, _draw_seed))
    return random.randint(0, 2**32 - 1)


def _check(q, k, v, n_heads):
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not supported(t, n_heads):
            raise ValueError(f"fused attention {name}: need (B, S, D) f32 with D / n_heads in "
                             f"{HEAD_DIMS}, got {t.type} {tuple(t.shape)} for {n_heads} heads")
    if not (tuple(q.shape) == tuple(k.shape) == tuple(v.shape)):
        raise ValueError(f"fused attention needs q, k, v of one shape, got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")


def fused_attention(q, k, v, n_heads, causal, p=0.0, seed=0):
    """``(out, lse)``: per head softmax(q k^T / sqrt(d) [+ causal mask]), dropout
    with probability ``p`` under ``seed`` (as the reference's elementwise
    dropout of the (B * H, S, S) probabilities), times v; ``out`` is (B, S, D)."""
    _check(q, k, v, n_heads)
    q, k, v = (t if t.is_contiguous() else t.contiguous() for t in (q, k, v))
    B, S, D = q.shape
    hd = D // n_heads
    out = empty(q.shape)
    lse = empty((B * n_heads * S,))
    s, sp = _seed_args(seed)
    call("wxx_attention_fwd", ptr(q), ptr(k), ptr(v), ptr(out), ptr(lse), B, S, n_heads, hd,
         int(bool(causal)), float(1.0 / math.sqrt(hd)), float(p),
         float(1 / (1 - p)) if p else 1.0, s, sp)
    return out, lse


def fused_attention_backward(q, k, v, out, grad, lse, n_heads, causal, p=0.0, seed=0):
    """``(dq, dk, dv)`` of :func:`fused_attention` for the upstream gradient ``grad``."""
    _check(q, k, v, n_heads)
    q, k, v, out, grad = (t if t.is_contiguous() else t.contiguous()
                          for t in (q, k, v, out, grad))
    B, S, D = q.shape
    hd = D // n_heads
    dq, dk, dv = empty(q.shape), empty(q.shape), empty(q.shape)
    s, sp = _seed_args(seed)
    call("wxx_attention_bwd", ptr(q), ptr(k), ptr(v), ptr(out), ptr(grad), ptr(lse), ptr(dq),
         ptr(dk), ptr(dv), B, S, n_heads, hd, int(bool(causal)), float(1.0 / math.sqrt(hd)),
         float(p), float(1 / (1 - p)) if p else 1.0, s, sp)
    return dq, dk, dv


__all__ = ["HEAD_DIMS", "supported", "draw_seed", "fused_attention", "fused_attention_backward"]
