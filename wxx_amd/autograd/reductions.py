"""Differentiable reductions and softmax (gradients as in reference
src/wxx/autograd/reductions.py:11-297).

The softmax gradient ``y * (g - sum(g * y))`` is formed by one fused row
kernel (``functional.softmax_backward``) instead of the reference's chain of
multiply, sum, unsqueeze, subtract and multiply launches; ``sum``/``mean``
backward broadcast the (scaled) output gradient with one strided kernel
instead of multiplying a host-built ones tensor.
"""

import builtins
import math

from .. import functional, validation
from ..backend.dispatch import _expand_grad_output
from .function import Function


class softmax(Function):
    def forward(self, tensor1, dim):
        dim = validation.normalize_dim(dim, len(tensor1.shape), name="dim")
        self.dim = dim
        out = functional.softmax(tensor1, dim)
        out.requires_grad = tensor1.requires_grad
        if out.requires_grad:
            self.hold_output(out)
        return self.attach(out)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        return functional.softmax_backward(self.held_output(), g, self.dim)


class scaled_masked_softmax(Function):
    """``softmax(x * scale + mask)`` along the last axis as one Function (the
    multiply, add and softmax Functions of the reference's attention score
    path, nn/module.py:478-483); the mask receives no gradient."""

    def forward(self, tensor1, scale, mask=None, causal=0):
        # causal: 0 general mask; 1 / 2 GPT-2's causal mask, the probabilities
        # above the diagonal written as 0 / left unwritten (2 when every
        # consumer reads only the lower triangle)
        if causal:
            out = functional.softmax_causal(tensor1, scale, skip=causal == 2)
        else:
            out = functional.softmax_scale_mask(tensor1, scale, mask)
        out.requires_grad = tensor1.requires_grad
        self.scale, self.causal = scale, causal
        if out.requires_grad:
            self.hold_output(out)
        return self.attach(out)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        y = self.held_output()
        if self.causal:
            return functional.softmax_backward_causal(y, g, self.scale, skip=self.causal == 2)
        return functional.softmax_backward_scale(y, g, self.scale)


class _reduction(Function):
    KIND = "sum"

    def forward(self, tensor1, axis=None, keepdims=False, *, keepdim=None):
        if keepdim is not None:
            keepdims = keepdim
        self.axis, self.keepdims = axis, keepdims
        self.shape = tuple(tensor1.shape)
        out = getattr(functional, self.KIND)(tensor1, axis, keepdims)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out)

    def _broadcast(self, g, scale):
        g = _expand_grad_output(g, shape=self.shape, axis=self.axis, keepdims=self.keepdims)
        return functional.broadcast_to(g, self.shape, scale)


class sum(_reduction):
    KIND = "sum"

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        return self._broadcast(g, 1.0)


class mean(_reduction):
    KIND = "mean"

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        n = math.prod(self.shape) // builtins.max(1, math.prod(g.shape))
        return self._broadcast(g, 1.0 / n)


class var(Function):
    """Population variance; gradient ``2 (x - mean) g / N``."""

    def forward(self, tensor1, axis=None, keepdims=False, *, keepdim=None):
        if keepdim is not None:
            keepdims = keepdim
        self.axis, self.keepdims = axis, keepdims
        self.numel_in = math.prod(tensor1.shape)
        out = functional.var(tensor1, axis, keepdims)
        out.requires_grad = tensor1.requires_grad
        if out.requires_grad:
            return self.attach(out, tensor1=tensor1,
                               mean=functional.mean(tensor1, axis, keepdims=True))
        return out

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        x = self.tensor1
        g = _expand_grad_output(g, shape=x.shape, axis=self.axis, keepdims=self.keepdims)
        n = self.numel_in // math.prod(g.shape)
        diff = functional.pointwise(x, self.mean, 1)
        self.tensor1 = self.mean = None
        return functional.scalarpointwise(functional.pointwise(diff, g, 2), 2.0 / n, 2)


class std(Function):
    """Population standard deviation; gradient ``(x - mean) g / (N std)``."""

    def forward(self, tensor1, axis=None, keepdims=False, *, keepdim=None):
        if keepdim is not None:
            keepdims = keepdim
        self.axis, self.keepdims = axis, keepdims
        self.numel_in = math.prod(tensor1.shape)
        out = functional.std(tensor1, axis, keepdims)
        out.requires_grad = tensor1.requires_grad
        if out.requires_grad:
            return self.attach(out, tensor1=tensor1,
                               mean=functional.mean(tensor1, axis, keepdims=True),
                               std=functional.std(tensor1, axis, keepdims=True))
        return out

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        x = self.tensor1
        g = _expand_grad_output(g, shape=x.shape, axis=self.axis, keepdims=self.keepdims)
        n = self.numel_in // math.prod(g.shape)
        diff = functional.pointwise(x, self.mean, 1)
        denom = functional.scalarpointwise(self.std, float(n), 2)
        self.tensor1 = self.mean = self.std = None
        return functional.pointwise(diff, functional.pointwise(g, denom, 3), 2)


class _minmax(Function):
    OP = "max"

    def forward(self, tensor1, axis=None, keepdims=False, *, keepdim=None):
        if keepdim is not None:
            keepdims = keepdim
        self.axis = axis
        out, idx = getattr(functional, self.OP)(tensor1, axis, keepdims)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out, input_shape=tuple(tensor1.shape), indices=idx)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        idx, self.indices = self.indices, None
        return functional.maxmin_backward(g, idx, self.input_shape, self.axis)


class max(_minmax):
    OP = "max"


class min(_minmax):
    OP = "min"


class argmax(Function):
    def forward(self, tensor1, axis=None, keepdims=False, *, keepdim=None):
        if keepdim is not None:
            keepdims = keepdim
        return functional.max(tensor1, axis, keepdims)[1]

    def backward(self, g):
        return None


class argmin(Function):
    def forward(self, tensor1, axis=None, keepdims=False, *, keepdim=None):
        if keepdim is not None:
            keepdims = keepdim
        return functional.min(tensor1, axis, keepdims)[1]

    def backward(self, g):
        return None
