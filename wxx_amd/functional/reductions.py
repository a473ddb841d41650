"""Reductions: sum / mean / sumsq, max / min with u32 indices, var / std and
the max/min backward scatter (reference src/wxx/functional/reductions.py:27-342)."""

from .. import validation
from ..backend.dispatch import _get_reduce_dims, keepdims_shape
from ._common import call, empty, ptr


def _reduce(tensor1, axis, keepdims, mode):
    if tensor1.type != "f32":
        raise TypeError(f"reduction expects an f32 tensor, got {tensor1.type!r}")
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    outer, red, inner, out_shape = _get_reduce_dims(tensor1.shape, axis)
    if keepdims:
        out_shape = keepdims_shape(tensor1.shape, axis)
    out = empty(out_shape)
    call("wxx_reduce", ptr(tensor1), ptr(out), outer, red, inner, mode)
    return out


def sum(tensor1, axis=None, keepdims=False, *, keepdim=None):
    if keepdim is not None:
        keepdims = keepdim
    return _reduce(tensor1, axis, keepdims, 0)


def mean(tensor1, axis=None, keepdims=False, *, keepdim=None):
    if keepdim is not None:
        keepdims = keepdim
    return _reduce(tensor1, axis, keepdims, 1)


def sumsq(tensor1, axis=None, keepdims=False, *, keepdim=None):
    """Fused sum of squares (used by the gradient-norm clip)."""
    if keepdim is not None:
        keepdims = keepdim
    return _reduce(tensor1, axis, keepdims, 2)


def _minmax(tensor1, axis, keepdims, op):
    if tensor1.type != "f32":
        raise TypeError(f"max/min expects an f32 tensor, got {tensor1.type!r}")
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    outer, red, inner, out_shape = _get_reduce_dims(tensor1.shape, axis)
    if keepdims:
        out_shape = keepdims_shape(tensor1.shape, axis)
    vals = empty(out_shape)
    idx = empty(out_shape, dtype="u32")
    call("wxx_reduce_minmax", ptr(tensor1), ptr(vals), ptr(idx), outer, red, inner, op)
    return vals, idx


def max(tensor1, axis=None, keepdims=False, *, keepdim=None):
    if keepdim is not None:
        keepdims = keepdim
    return _minmax(tensor1, axis, keepdims, 0)


def min(tensor1, axis=None, keepdims=False, *, keepdim=None):
    if keepdim is not None:
        keepdims = keepdim
    return _minmax(tensor1, axis, keepdims, 1)


def maxmin_backward(grad_output, indices, input_shape, axis=None):
    """Route ``grad_output`` to the arg-max/min position of each reduced slice."""
    if not grad_output.is_contiguous():
        grad_output = grad_output.contiguous()
    if not indices.is_contiguous():
        indices = indices.contiguous()
    outer, red, inner, _ = _get_reduce_dims(input_shape, axis)
    for t, name in ((grad_output, "grad_output"), (indices, "indices")):
        if validation.numel(t.shape) != outer * inner:
            raise ValueError(
                f"{name} has {validation.numel(t.shape)} elements, expected {outer * inner}"
            )
    if indices.type != "u32":
        raise TypeError(f"indices must be u32, got {indices.type!r}")
    out = empty(tuple(input_shape))
    call("wxx_maxmin_backward", ptr(grad_output), ptr(indices), ptr(out), outer, red, inner)
    return out


def var(tensor1, axis=None, keepdims=False, *, keepdim=None):
    """Population variance (ddof=0): mean((x - mean(x))^2)."""
    from .pointwise import pointwise

    if keepdim is not None:
        keepdims = keepdim
    if tensor1.type != "f32":
        raise TypeError(f"var expects an f32 tensor, got {tensor1.type!r}")
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    m = mean(tensor1, axis, keepdims=True)
    diff = pointwise(tensor1, m, 1)
    return mean(pointwise(diff, diff, 2), axis, keepdims)


def std(tensor1, axis=None, keepdims=False, *, keepdim=None):
    from .pointwise import sqrt

    if keepdim is not None:
        keepdims = keepdim
    return sqrt(var(tensor1, axis=axis, keepdims=keepdims))


__all__ = ["sum", "mean", "sumsq", "max", "min", "maxmin_backward", "var", "std"]
