"""Differentiable elementwise ops (gradients as in reference
src/wxx/autograd/pointwise.py:11-598).

Where the reference multiplies the incoming gradient by a separately
computed local derivative (two launches), the unary activations here call
``functional.unary_backward`` which forms ``f'(x) * g`` in one pass; the
values are the same products.
"""

import math

from .. import functional
from ..backend.dispatch import _sum_to_shape
from .function import Function


def _binary_out(self, out, a, b, save=False):
    out.requires_grad = a.requires_grad or b.requires_grad
    if save:
        return self.attach(out, tensor1=a, tensor2=b)
    return self.attach(out)


class add(Function):
    def forward(self, tensor1, tensor2):
        return _binary_out(self, functional.pointwise(tensor1, tensor2, 0), tensor1, tensor2)

    def backward(self, g):
        return (
            _sum_to_shape(g, self.inputs[0].shape) if self.needs_input_grad[0] else None,
            _sum_to_shape(g, self.inputs[1].shape) if self.needs_input_grad[1] else None,
        )


class sub(Function):
    def forward(self, tensor1, tensor2):
        return _binary_out(self, functional.pointwise(tensor1, tensor2, 1), tensor1, tensor2)

    def backward(self, g):
        return (
            _sum_to_shape(g, self.inputs[0].shape) if self.needs_input_grad[0] else None,
            _sum_to_shape(functional.negate(g), self.inputs[1].shape)
            if self.needs_input_grad[1] else None,
        )


class mul(Function):
    def forward(self, tensor1, tensor2):
        return _binary_out(self, functional.pointwise(tensor1, tensor2, 2), tensor1, tensor2, True)

    def backward(self, g):
        a, b = self.tensor1, self.tensor2
        self.tensor1 = self.tensor2 = None
        if (self.needs_input_grad[0] and self.needs_input_grad[1]
                and tuple(g.shape) == tuple(a.shape) == tuple(b.shape)
                and g.is_contiguous() and a.is_contiguous() and b.is_contiguous()):
            return functional.mul_backward(g, a, b)
        ga = (_sum_to_shape(functional.pointwise(g, b, 2), self.inputs[0].shape)
              if self.needs_input_grad[0] else None)
        gb = (_sum_to_shape(functional.pointwise(g, a, 2), self.inputs[1].shape)
              if self.needs_input_grad[1] else None)
        return ga, gb


class div(Function):
    def forward(self, tensor1, tensor2):
        return _binary_out(self, functional.pointwise(tensor1, tensor2, 3), tensor1, tensor2, True)

    def backward(self, g):
        a, b = self.tensor1, self.tensor2
        self.tensor1 = self.tensor2 = None
        ga = (_sum_to_shape(functional.pointwise(g, b, 3), self.inputs[0].shape)
              if self.needs_input_grad[0] else None)
        gb = None
        if self.needs_input_grad[1]:
            num = functional.negate(functional.pointwise(g, a, 2))
            gb = _sum_to_shape(functional.pointwise(num, functional.square(b), 3),
                               self.inputs[1].shape)
        return ga, gb


class _scalar(Function):
    OP = 0
    REVERSE = 0

    def forward(self, tensor1, value):
        out = functional.scalarpointwise(tensor1, value, self.OP, self.REVERSE)
        out.requires_grad = tensor1.requires_grad
        self.value = value
        return self.attach(out)


class addscaler(_scalar):
    OP = 0

    def backward(self, g):
        return g if self.needs_input_grad[0] else None


class subscaler(_scalar):
    OP = 1

    def backward(self, g):
        return g if self.needs_input_grad[0] else None


class mulscaler(_scalar):
    OP = 2

    def backward(self, g):
        return functional.scalarpointwise(g, self.value, 2) if self.needs_input_grad[0] else None


class powscaler(Function):
    """``x ** c``: gradient ``g * c * x ** (c - 1)``."""

    def forward(self, tensor1, value):
        out = functional.scalarpointwise(tensor1, value, 3)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out, value=value, tensor1=tensor1)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        x, self.tensor1 = self.tensor1, None
        local = functional.scalarpointwise(functional.scalarpointwise(x, self.value - 1, 3),
                                           self.value, 2)
        return functional.pointwise(g, local, 2)


class rpowscaler(Function):
    """``c ** x`` (c > 0): gradient ``g * c ** x * ln c``."""

    def forward(self, tensor1, value):
        out = functional.scalarpointwise(tensor1, value, 3, reverse=1)
        out.requires_grad = tensor1.requires_grad
        self.value = value
        if out.requires_grad:
            self.hold_output(out)
        return self.attach(out)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        out = self.held_output()
        return functional.pointwise(g, functional.scalarpointwise(out, math.log(self.value), 2), 2)


class rdivscaler(Function):
    """``c / x``: gradient ``-c g / x^2``."""

    def forward(self, tensor1, value):
        out = functional.scalarpointwise(tensor1, value, 4, reverse=1)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out, value=value, tensor1=tensor1)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        x, self.tensor1 = self.tensor1, None
        sq = functional.pointwise(x, x, 2)
        return functional.scalarpointwise(functional.pointwise(g, sq, 3), -self.value, 2)


class _unary(Function):
    """f(x) with gradient f'(x) * g from one fused kernel."""

    NAME = ""
    SAVE_OUTPUT = False  # derivative expressed through the output (sigmoid)

    def forward(self, tensor1):
        out = functional.unary(tensor1, self.NAME)
        out.requires_grad = tensor1.requires_grad
        if out.requires_grad and self.SAVE_OUTPUT:
            self.hold_output(out)
            return self.attach(out)
        return self.attach(out, tensor1=tensor1)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        src = self.held_output() if self.SAVE_OUTPUT else self.tensor1
        self.tensor1 = None
        return functional.unary_backward(src, g, self.NAME)


class relu(_unary):
    NAME = "relu"


class gelu(_unary):
    NAME = "gelu"


class sigmoid(_unary):
    NAME = "sigmoid"
    SAVE_OUTPUT = True


class selu(_unary):
    NAME = "selu"


class sin(_unary):
    NAME = "sin"


class cos(_unary):
    NAME = "cos"


class negate(Function):
    def forward(self, tensor1):
        out = functional.negate(tensor1)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out)

    def backward(self, g):
        return functional.negate(g) if self.needs_input_grad[0] else None


class abs(Function):
    def forward(self, tensor1):
        out = functional.abs(tensor1)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out, tensor1=tensor1)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        x, self.tensor1 = self.tensor1, None
        return functional.pointwise(g, functional.sign(x), 2)


class sign(Function):
    def forward(self, tensor1):
        out = functional.sign(tensor1)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out)

    def backward(self, g):
        return None


class square(Function):
    def forward(self, tensor1):
        out = functional.square(tensor1)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out, tensor1=tensor1)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        x, self.tensor1 = self.tensor1, None
        return functional.pointwise(g, functional.scalarpointwise(x, 2, 2), 2)


class exp(Function):
    def forward(self, tensor1):
        out = functional.exp(tensor1)
        out.requires_grad = tensor1.requires_grad
        if out.requires_grad:
            self.hold_output(out)
        return self.attach(out)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        return functional.pointwise(g, self.held_output(), 2)


class sqrt(Function):
    def forward(self, tensor1):
        out = functional.sqrt(tensor1)
        out.requires_grad = tensor1.requires_grad
        if out.requires_grad:
            self.hold_output(out)
        return self.attach(out)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        out = self.held_output()
        return functional.pointwise(g, functional.scalarpointwise(out, 2, 2), 3)


class rsqrt(Function):
    def forward(self, tensor1):
        out = functional.rsqrt(tensor1)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out, tensor1=tensor1)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        x, self.tensor1 = self.tensor1, None
        return functional.pointwise(functional.scalarpointwise(x, -1.5, 3),
                                    functional.scalarpointwise(g, -0.5, 2), 2)


class log(Function):
    def forward(self, tensor1):
        out = functional.log(tensor1)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out, tensor1=tensor1)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        x, self.tensor1 = self.tensor1, None
        return functional.pointwise(g, x, 3)


class clamp(Function):
    def forward(self, tensor1, min, max):
        out = functional.clamp(tensor1, min, max)
        out.requires_grad = tensor1.requires_grad
        self.min, self.max = min, max
        return self.attach(out, tensor1=tensor1)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        x, self.tensor1 = self.tensor1, None
        return functional.pointwise(g, functional.clampbackwards(x, self.min, self.max), 2)


class decay_window(Function):
    def forward(self, decay, stage, length):
        out = functional.decay_window(decay, stage, length)
        out.requires_grad = decay.requires_grad
        return self.attach(out, decay=decay, stage=stage, length=length)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        d, self.decay = self.decay, None
        return functional.decay_window_backward(g, d, self.stage, self.length)
