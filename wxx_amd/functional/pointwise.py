"""Elementwise binary / scalar / unary ops (reference src/wxx/functional/pointwise.py).

``pointwise`` reads strided views directly (offset + strides) like the
reference; ``_pointwise`` accumulates in place into a contiguous ``A``
(autograd gradient accumulation) and reads ``B`` with broadcasting.
"""

from .. import validation
from ..backend.dispatch import (
    broadcast_shapes,
    compute_broadcast_strides,
    supports_strided,
    view_broadcast_strides,
)
from ..Tensor import Tensor
from ._common import call, empty, i64_array, ptr
from .activations import unary


def pointwise(tensor1, tensor2, op):
    """``A op B`` with broadcasting; op 0 add, 1 sub, 2 mul, 3 div."""
    if not isinstance(tensor2, Tensor):
        return scalarpointwise(tensor1, tensor2, op)
    if not supports_strided(tensor1):
        tensor1 = tensor1.contiguous()
    if not supports_strided(tensor2):
        tensor2 = tensor2.contiguous()
    if tensor1.type != "f32" or tensor2.type != "f32":
        raise TypeError(
            f"pointwise expects f32 tensors, got {tensor1.type!r} and {tensor2.type!r}"
        )
    out_shape, _, _ = broadcast_shapes(tensor1.shape, tensor2.shape)
    rank = validation.check_rank(out_shape, name="pointwise output")
    out = empty(out_shape, requires_grad=tensor1.requires_grad or tensor2.requires_grad)
    if validation.numel(out_shape):
        call(
            "wxx_pointwise",
            ptr(out),
            ptr(tensor1),
            ptr(tensor2),
            rank,
            i64_array(out_shape),
            i64_array(out.stride),
            i64_array(view_broadcast_strides(tensor1, out_shape)),
            i64_array(view_broadcast_strides(tensor2, out_shape)),
            int(op),
        )
    return out


def scalarpointwise(tensor1, value, op, reverse=0):
    """``X op value`` (``value op X`` when ``reverse``); op 0 add, 1 sub, 2 mul, 3 pow, 4 div."""
    if tensor1.type != "f32":
        raise TypeError(f"scalarpointwise expects f32 input, got {tensor1.type!r}")
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    out = empty(tensor1.shape, requires_grad=tensor1.requires_grad)
    call("wxx_scalarpointwise", ptr(tensor1), ptr(out), validation.numel(tensor1.shape), int(op),
         float(value), int(bool(reverse)))
    return out


def clamp(tensor1, min, max):
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    out = empty(tensor1.shape, requires_grad=tensor1.requires_grad)
    call("wxx_clamp", ptr(tensor1), ptr(out), validation.numel(tensor1.shape), float(min),
         float(max), 0)
    return out


def clampbackwards(tensor1, min, max):
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    out = empty(tensor1.shape, requires_grad=tensor1.requires_grad)
    call("wxx_clamp", ptr(tensor1), ptr(out), validation.numel(tensor1.shape), float(min),
         float(max), 1)
    return out


def _pointwise(tensor1, tensor2, op):
    """In place ``A op= B`` (B broadcast to A's shape)."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if not tensor2.is_contiguous():
        tensor2 = tensor2.contiguous()
    if tensor1.type != "f32" or tensor2.type != "f32":
        raise TypeError(
            f"_pointwise expects f32 tensors, got {tensor1.type!r} and {tensor2.type!r}"
        )
    out_shape, pad_a, pad_b = broadcast_shapes(tensor1.shape, tensor2.shape)
    rank = validation.check_rank(out_shape, name="_pointwise output")
    if tuple(out_shape) != tuple(tensor1.shape):
        raise ValueError(
            f"_pointwise target {tuple(tensor1.shape)} cannot hold the broadcast result "
            f"{tuple(out_shape)}"
        )
    # A and B may share storage (x + x accumulates a gradient into itself).
    # Reading and writing the very same element in one thread is race-free;
    # any other overlap is not, so B is copied first in that case.
    if tensor1.buffer is tensor2.buffer and not (
        tensor1.offset == tensor2.offset
        and tuple(tensor1.shape) == tuple(tensor2.shape)
        and tuple(tensor1.stride) == tuple(tensor2.stride)
    ):
        tensor2 = scalarpointwise(tensor2, 0.0, 0)
    if validation.numel(out_shape):
        sa = compute_broadcast_strides(pad_a, out_shape)
        call(
            "wxx_pointwise",
            ptr(tensor1),
            ptr(tensor1),
            ptr(tensor2),
            rank,
            i64_array(out_shape),
            i64_array(sa),
            i64_array(sa),
            i64_array(compute_broadcast_strides(pad_b, out_shape)),
            int(op),
        )


def negate(tensor1):
    return unary(tensor1, "negate")


def abs(tensor1):
    return unary(tensor1, "abs")


def sign(tensor1):
    return unary(tensor1, "sign")


def square(tensor1):
    return unary(tensor1, "square")


def exp(tensor1):
    return unary(tensor1, "exp")


def sqrt(tensor1):
    return unary(tensor1, "sqrt")


def rsqrt(tensor1):
    return unary(tensor1, "rsqrt")


def log(tensor1):
    return unary(tensor1, "log")


def mul_backward(grad, tensor_a, tensor_b):
    """``(grad * b, grad * a)`` in one pass (all three same-shape and contiguous)."""
    validation.check_same_shape(grad.shape, tensor_a.shape, tensor_b.shape,
                                name="mul_backward operands")
    if not (grad.is_contiguous() and tensor_a.is_contiguous() and tensor_b.is_contiguous()):
        raise ValueError("mul_backward expects contiguous operands")
    n = validation.numel(grad.shape)
    da = empty(grad.shape)
    db = empty(grad.shape)
    call("wxx_mul_backward", ptr(grad), ptr(tensor_a), ptr(tensor_b), ptr(da), ptr(db), n)
    return da, db


def decay_window(decay, stage, length):
    """Causal window ``exp(-|decay[stage, d]| * t)`` as a ``(channels, length)`` tensor."""
    if decay.type != "f32":
        raise TypeError(f"decay_window expects f32 decay, got {decay.type!r}")
    if not decay.is_contiguous():
        decay = decay.contiguous()
    if len(decay.shape) != 2:
        raise ValueError(f"decay_window expects a 2-D decay, got {decay.shape}")
    rows, channels = decay.shape
    if not isinstance(length, int) or length < 1:
        raise ValueError(f"decay_window length must be a positive int, got {length!r}")
    if not 0 <= stage < rows:
        raise IndexError(f"decay_window stage {stage} out of range for {rows} rows")
    out = empty((channels, length), requires_grad=decay.requires_grad)
    call("wxx_decay_window", ptr(decay), ptr(out), rows, channels, length, stage)
    return out


def decay_window_backward(grad, decay, stage, length):
    """Gradient of :func:`decay_window` for the whole ``(rows, channels)`` parameter."""
    if not grad.is_contiguous():
        grad = grad.contiguous()
    if decay.type != "f32":
        raise TypeError(f"decay_window expects f32 decay, got {decay.type!r}")
    if not decay.is_contiguous():
        decay = decay.contiguous()
    if len(decay.shape) != 2:
        raise ValueError(f"decay_window expects a 2-D decay, got {decay.shape}")
    rows, channels = decay.shape
    if not isinstance(length, int) or length < 1:
        raise ValueError(f"decay_window length must be a positive int, got {length!r}")
    if not 0 <= stage < rows:
        raise IndexError(f"decay_window stage {stage} out of range for {rows} rows")
    out = empty((rows, channels))
    call("wxx_decay_window_backward", ptr(grad), ptr(decay), ptr(out), rows, channels, length,
         stage)
    return out
