"""Activation functions, their local derivatives and softmax
(reference src/wxx/functional/activations.py:22-173).

The ``*backwards`` / ``*back`` functions return the local derivative, as in
the reference; autograd multiplies by the incoming gradient.
"""

from .. import validation
from ..backend.dispatch import _get_reduce_dims
from ._common import call, empty, ptr

# Must match enum Unary in csrc/elementwise.hip.
UNARY = {
    "relu": 0,
    "relubackwards": 1,
    "gelu": 2,
    "gelubackwards": 3,
    "sigmoid": 4,
    "sigmoidbackwards": 5,
    "selu": 6,
    "selubackwards": 7,
    "sin": 8,
    "sinback": 9,
    "cos": 10,
    "cosback": 11,
    "abs": 12,
    "exp": 13,
    "log": 14,
    "negate": 15,
    "rsqrt": 16,
    "sign": 17,
    "sqrt": 18,
    "square": 19,
}


def unary(tensor1, name):
    """Run unary kernel ``name`` on a contiguous copy of ``tensor1``."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    validation.check_rank(tensor1.shape, name="unary op input")
    out = empty(tensor1.shape, requires_grad=tensor1.requires_grad)
    call("wxx_unary", ptr(tensor1), ptr(out), validation.numel(tensor1.shape), UNARY[name])
    return out


# Derivative op used by unary_backward for each differentiable activation.
_DERIVATIVE = {
    "relu": "relubackwards",
    "gelu": "gelubackwards",
    "sigmoid": "sigmoidbackwards",
    "selu": "selubackwards",
    "sin": "sinback",
    "cos": "cosback",
}


def unary_backward(src, grad, name):
    """``f'(src) * grad`` for activation ``name`` in one kernel (for sigmoid
    ``src`` is the forward output, as the reference's sigmoidbackwards takes)."""
    if name not in _DERIVATIVE:
        raise ValueError(f"no fused backward for {name!r}")
    if not src.is_contiguous():
        src = src.contiguous()
    if not grad.is_contiguous():
        grad = grad.contiguous()
    if tuple(src.shape) != tuple(grad.shape):
        raise ValueError(
            f"unary_backward shapes differ: {tuple(src.shape)} vs {tuple(grad.shape)}"
        )
    out = empty(src.shape)
    call("wxx_unary_backward", ptr(src), ptr(grad), ptr(out), validation.numel(src.shape),
         UNARY[_DERIVATIVE[name]])
    return out


def swiglu_gate(a, b):
    """``silu(a) * b`` in one kernel, equal bit for bit to ``sigmoid(a) * a * b``."""
    a, b = _same_dense(a, b, "swiglu_gate")
    out = empty(a.shape)
    call("wxx_swiglu_gate", ptr(a), ptr(b), ptr(out), validation.numel(a.shape))
    return out


def swiglu_gate_backward(grad, a, b):
    """``(da, db)`` of :func:`swiglu_gate` for the output gradient ``grad``, equal bit
    for bit to the composed ops' backwards."""
    a, b = _same_dense(a, b, "swiglu_gate_backward")
    grad, _ = _same_dense(grad, a, "swiglu_gate_backward")
    da = empty(a.shape)
    db = empty(a.shape)
    call("wxx_swiglu_gate_backward", ptr(grad), ptr(a), ptr(b), ptr(da), ptr(db),
         validation.numel(a.shape))
    return da, db


def _same_dense(x, y, what):
    if not x.is_contiguous():
        x = x.contiguous()
    if not y.is_contiguous():
        y = y.contiguous()
    if tuple(x.shape) != tuple(y.shape):
        raise ValueError(f"{what} shapes differ: {tuple(x.shape)} vs {tuple(y.shape)}")
    return x, y


def relu(tensor1):
    return unary(tensor1, "relu")


def relubackwards(tensor1):
    return unary(tensor1, "relubackwards")


def gelu(tensor1):
    return unary(tensor1, "gelu")


def gelubackwards(tensor1):
    return unary(tensor1, "gelubackwards")


def sigmoid(tensor1):
    return unary(tensor1, "sigmoid")


def sigmoidbackwards(tensor1):
    """Local derivative from the sigmoid *output* ``y``: ``y (1 - y)``."""
    return unary(tensor1, "sigmoidbackwards")


def selu(tensor1):
    return unary(tensor1, "selu")


def selubackwards(tensor1):
    return unary(tensor1, "selubackwards")


def sin(tensor1):
    return unary(tensor1, "sin")


def sinback(tensor1):
    return unary(tensor1, "sinback")


def cos(tensor1):
    return unary(tensor1, "cos")


def cosback(tensor1):
    return unary(tensor1, "cosback")


def softmax(tensor1, dim):
    """Softmax along ``dim``."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    rank = validation.check_rank(tensor1.shape, name="softmax input")
    dim = validation.normalize_dim(dim, rank, name="dim")
    if tensor1.type != "f32":
        raise TypeError(f"softmax expects f32 input, got {tensor1.type!r}")
    outer, c, inner, _ = _get_reduce_dims(tensor1.shape, dim)
    out = empty(tensor1.shape, requires_grad=tensor1.requires_grad)
    if validation.numel(tensor1.shape):
        call("wxx_softmax", ptr(tensor1), ptr(out), outer, c, inner)
    return out


def softmax_backward(y, grad, dim):
    """``y * (grad - sum(grad * y, dim))`` from the softmax output ``y`` in one
    kernel (the chain of reference src/wxx/autograd/reductions.py:25-35)."""
    if not y.is_contiguous():
        y = y.contiguous()
    if not grad.is_contiguous():
        grad = grad.contiguous()
    if tuple(y.shape) != tuple(grad.shape):
        raise ValueError(
            f"softmax_backward shapes differ: {tuple(y.shape)} vs {tuple(grad.shape)}"
        )
    rank = validation.check_rank(y.shape, name="softmax_backward input")
    dim = validation.normalize_dim(dim, rank, name="dim")
    outer, c, inner, _ = _get_reduce_dims(y.shape, dim)
    out = empty(y.shape)
    if validation.numel(y.shape):
        call("wxx_softmax_backward", ptr(y), ptr(grad), ptr(out), outer, c, inner)
    return out


def _fused_softmax_ok(x, mask):
    if len(x.shape) < 1 or x.type != "f32" or x.shape[-1] > 16384:
        return False
    if mask is None:
        return True
    return (len(mask.shape) == 2 and mask.type == "f32" and mask.shape[1] == x.shape[-1]
            and mask.stride[1] == 1 and len(x.shape) >= 2 and x.shape[-2] == mask.shape[0])


def softmax_scale_mask(tensor1, scale, mask=None):
    """``softmax(tensor1 * scale + mask, dim=-1)`` in one pass; ``mask`` is
    None or a (rows, C) tensor broadcast over the leading dimensions (the
    attention score path of the reference's MultiHeadAttention,
    nn/module.py:478-483, whose three launches it replaces; same roundings)."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if not _fused_softmax_ok(tensor1, mask):
        from .pointwise import pointwise, scalarpointwise

        z = scalarpointwise(tensor1, scale, 2)
        if mask is not None:
            z = pointwise(z, mask, 0)
        return softmax(z, -1)
    C = tensor1.shape[-1]
    rows = validation.numel(tensor1.shape) // C
    out = empty(tensor1.shape, requires_grad=tensor1.requires_grad)
    if rows:
        call("wxx_softmax_scale_mask", ptr(tensor1), ptr(mask) if mask is not None else None,
             ptr(out), rows, C, mask.shape[0] if mask is not None else 1,
             mask.stride[0] if mask is not None else 0, float(scale))
    return out


def softmax_causal(tensor1, scale, skip=False):
    """``softmax(tensor1 * scale + causal_mask, dim=-1)`` for the (..., S, S)
    scores of attention under GPT-2's causal mask (0 on and below the
    diagonal, -1e9 above): each row reads its columns j <= i only and the
    result is exactly 0 above the diagonal, the numbers of
    :func:`softmax_scale_mask` with that mask.  ``skip`` leaves the zeros
    above the diagonal unwritten (for consumers reading only the lower
    triangle)."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    S, C = tensor1.shape[-2], tensor1.shape[-1]
    if C > 16384 or S != C:
        raise ValueError(f"causal softmax needs square score blocks of <= 16384, got {S}x{C}")
    rows = validation.numel(tensor1.shape) // C
    out = empty(tensor1.shape, requires_grad=tensor1.requires_grad)
    if rows:
        call("wxx_softmax_causal", ptr(tensor1), ptr(out), rows, C, S, float(scale),
             1 if skip else 0)
    return out


def softmax_backward_causal(y, grad, scale, skip=False):
    """Gradient of :func:`softmax_causal` (``grad`` read on and below the
    diagonal only; 0 above it, left unwritten when ``skip``)."""
    if not y.is_contiguous():
        y = y.contiguous()
    if not grad.is_contiguous():
        grad = grad.contiguous()
    S, C = y.shape[-2], y.shape[-1]
    rows = validation.numel(y.shape) // C
    out = empty(y.shape)
    if rows:
        call("wxx_softmax_backward_causal", ptr(y), ptr(grad), ptr(out), rows, C, S,
             float(scale), 1 if skip else 0)
    return out


def softmax_backward_scale(y, grad, scale):
    """Gradient of :func:`softmax_scale_mask`: ``scale * y * (grad - sum(grad * y))``."""
    if not y.is_contiguous():
        y = y.contiguous()
    if not grad.is_contiguous():
        grad = grad.contiguous()
    C = y.shape[-1]
    if C > 16384:
        from .pointwise import scalarpointwise

        return scalarpointwise(softmax_backward(y, grad, -1), scale, 2)
    rows = validation.numel(y.shape) // C
    out = empty(y.shape)
    if rows:
        call("wxx_softmax_backward_scale", ptr(y), ptr(grad), ptr(out), rows, C, float(scale))
    return out
