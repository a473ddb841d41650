"""Reductions restated from the reference (test infrastructure only).

* ``reduce``: sum / mean / sum-of-squares over a contiguous range of axes
  viewed as (outer, reduce, inner) — reference src/wxx/backend/dispatch.py:173-214
  (axis mapping) and src/wxx/shaders/helpers/reduce.wgsl:31-66 (mean divides
  by f32(reduce), mode 2 squares before summing).  Accumulated in float64.
* ``var`` / ``std``: population (ddof=0) variance as the reference composes
  it — mean, subtract, square, mean (src/wxx/functional/reductions.py:315-336);
  std = sqrt(var).  Accumulated in float64.
* ``minmax``: value and u32 index with the reference's exact tie rule —
  src/wxx/shaders/helpers/reduce_minmax.wgsl:41-71: 256 lanes scan
  r = t, t+256, ... keeping the first strictly better value (init -1e38 /
  +1e38 with index 0), then a halving tree s = 128..1 in which slot i takes
  slot i+s only if strictly better.
"""

import numpy as np

WG = 256


def reduce_dims(shape, axis):
    """(outer, reduce, inner, out_shape) of reference dispatch.py:173-214."""
    ndim = len(shape)
    if axis is None:
        return 1, int(np.prod(shape)), 1, (1,)
    axes = (axis,) if isinstance(axis, int) else tuple(axis)
    axes = tuple(sorted(a + ndim if a < 0 else a for a in axes))
    first, last = axes[0], axes[-1]
    outer = int(np.prod(shape[:first])) if first > 0 else 1
    red = int(np.prod(shape[first:last + 1]))
    inner = int(np.prod(shape[last + 1:])) if last < ndim - 1 else 1
    out_shape = tuple(s for d, s in enumerate(shape) if d not in axes) or (1,)
    return outer, red, inner, out_shape


def reduce(x, axis=None, keepdims=False, mode=0):
    """mode 0 sum, 1 mean, 2 sum of squares; float32 result."""
    x = np.asarray(x, dtype=np.float32)
    outer, red, inner, out_shape = reduce_dims(x.shape, axis)
    v = x.reshape(outer, red, inner).astype(np.float64)
    if mode == 2:
        v = v * v
    s = v.sum(axis=1)
    if mode == 1:
        s = s / red
    if keepdims:
        if axis is None:
            out_shape = (1,) * x.ndim
        else:
            axes = (axis,) if isinstance(axis, int) else tuple(axis)
            axes = {a + x.ndim if a < 0 else a for a in axes}
            out_shape = tuple(1 if d in axes else n for d, n in enumerate(x.shape))
    return s.astype(np.float32).reshape(out_shape)


def var(x, axis=None, keepdims=False):
    """mean((x - mean(x, keepdims))^2) over ``axis``; float32 result."""
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    ax = None if axis is None else (axis if isinstance(axis, int) else tuple(axis))
    m = x.mean(axis=ax, keepdims=True)
    d = x - m
    v = (d * d).mean(axis=ax, keepdims=keepdims)
    return np.asarray(v, np.float32).reshape(np.shape(v) or (1,))


def std(x, axis=None, keepdims=False):
    return np.sqrt(var(x, axis, keepdims).astype(np.float64)).astype(np.float32)


def minmax(x, axis=None, op=0):
    """(values f32, indices u32) of reference reduce_minmax.wgsl; op 0 max, 1 min."""
    x = np.asarray(x, dtype=np.float32)
    outer, red, inner, out_shape = reduce_dims(x.shape, axis)
    v = x.reshape(outer, red, inner).transpose(0, 2, 1).reshape(outer * inner, red)
    init = np.float32(-1e38) if op == 0 else np.float32(1e38)
    pad_val = -np.inf if op == 0 else np.inf
    chunks = (red + WG - 1) // WG
    padded = np.full((v.shape[0], chunks * WG), pad_val, dtype=np.float64)
    padded[:, :red] = v
    # NaN is never "strictly better": it cannot displace anything.
    padded[np.isnan(padded)] = pad_val
    lanes = padded.reshape(v.shape[0], chunks, WG)  # [out, chunk, lane]
    # Per lane: first occurrence of the best value along its strided scan.
    if op == 0:
        k = np.argmax(lanes, axis=1)
    else:
        k = np.argmin(lanes, axis=1)
    best = np.take_along_axis(lanes, k[:, None, :], axis=1)[:, 0, :]
    better_than_init = best > init if op == 0 else best < init
    val = np.where(better_than_init, best, np.float64(init))
    idx = np.where(better_than_init, k * WG + np.arange(WG)[None, :], 0).astype(np.int64)
    s = WG // 2
    while s >= 1:
        a_v, b_v = val[:, :s], val[:, s:2 * s]
        a_i, b_i = idx[:, :s], idx[:, s:2 * s]
        take = b_v > a_v if op == 0 else b_v < a_v
        val = np.where(take, b_v, a_v)
        idx = np.where(take, b_i, a_i)
        s //= 2
    return (
        val[:, 0].astype(np.float32).reshape(out_shape),
        idx[:, 0].astype(np.uint32).reshape(out_shape),
    )


def maxmin_backward(grad, indices, input_shape, axis=None):
    """Scatter ``grad`` to the selected index (reference maxmin_backward.wgsl:25-38)."""
    outer, red, inner, _ = reduce_dims(tuple(input_shape), axis)
    g = np.asarray(grad, dtype=np.float32).reshape(outer, 1, inner)
    ind = np.asarray(indices).astype(np.int64).reshape(outer, 1, inner)
    r = np.arange(red).reshape(1, red, 1)
    out = np.where(r == ind, g, np.float32(0.0))
    return out.astype(np.float32).reshape(input_shape)
