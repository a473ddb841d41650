"""Differentiable convolution and pooling (reference src/wxx/autograd/convolution.py:1-322)."""

from .. import functional
from ..backend import context
from .function import Function


class Conv2D(Function):
    def forward(self, tensor1, W, bias=None, stride=(1, 1), padding=(0, 0), dilation=(1, 1)):
        self.Xshape, self.wshape = tensor1.shape, W.shape
        self.stride, self.padding, self.dilation = stride, padding, dilation
        out = functional.conv2d(tensor1, W, stride, padding, dilation, bias)
        out.requires_grad = any(self.needs_input_grad)
        return self.attach(out, tensor1=tensor1, W=W, bias=bias)

    def backward(self, grad_output):
        x, w, bias = self.tensor1, self.W, self.bias
        self.tensor1 = self.W = self.bias = None
        args = (self.stride, self.padding, self.dilation, self.Xshape, self.wshape)
        # a gradient nobody asked for is not computed (the network input's dX)
        dw = functional.conv2ddw(grad_output, x, *args) if self.needs_input_grad[1] else None
        dx = functional.conv2ddx(grad_output, w, *args) if self.needs_input_grad[0] else None
        if bias is None:
            return dx, dw
        if not self.needs_input_grad[2]:
            return dx, dw, None
        if len(grad_output.shape) == 4:
            db = grad_output.sum(axis=(2, 3)).sum(axis=0)
        else:
            db = grad_output.sum(axis=0)
        return dx, dw, db


class Conv2DTranspose(Function):
    def forward(self, tensor1, W, bias=None, stride=(1, 1), padding=(0, 0),
                output_padding=(0, 0), dilation=(1, 1)):
        self.Xshape, self.wshape = tensor1.shape, W.shape
        self.stride, self.padding, self.dilation = stride, padding, dilation
        out = functional.conv2dtranspose(tensor1, W, stride, padding, dilation, output_padding,
                                         bias)
        self.out_shape = out.shape
        out.requires_grad = any(self.needs_input_grad)
        return self.attach(out, tensor1=tensor1, W=W, bias=bias)

    def backward(self, grad_output):
        x, w, bias = self.tensor1, self.W, self.bias
        self.tensor1 = self.W = self.bias = None
        dx = (functional.conv2dtranspose_dx(grad_output, w, self.stride, self.padding,
                                            self.dilation, self.Xshape, self.wshape,
                                            self.out_shape)
              if self.needs_input_grad[0] else None)
        dw = (functional.conv2dtranspose_dw(grad_output, x, self.stride, self.padding,
                                            self.dilation, self.out_shape, self.wshape)
              if self.needs_input_grad[1] else None)
        if bias is None:
            return dx, dw
        return dx, dw, grad_output.sum(axis=(2, 3)).sum(axis=0)


class _maxpool(Function):
    _fwd = None
    _bwd = None

    def forward(self, tensor1, kernel, stride, padding, return_indices=False):
        need = tensor1.requires_grad or return_indices
        if need:
            out, indices = type(self)._fwd(tensor1, kernel, stride, padding, True)
        else:
            out, indices = type(self)._fwd(tensor1, kernel, stride, padding), None
        out.requires_grad = tensor1.requires_grad
        if out.requires_grad and context.MODE == 0:
            self.tensor1, self.indices = tensor1, indices
            self.kernel, self.stride, self.padding = kernel, stride, padding
            out.creator = self
        return (out, indices) if return_indices else out

    def backward(self, grad_output):
        if not self.needs_input_grad[0]:
            return None
        g = type(self)._bwd(grad_output, self.tensor1, self.indices, self.kernel, self.stride,
                            self.padding)
        self.tensor1 = self.indices = None
        return g


class maxpooling2d(_maxpool):
    _fwd = staticmethod(functional.maxpool2d)
    _bwd = staticmethod(functional.maxpool2ddx)


class maxpooling1d(_maxpool):
    _fwd = staticmethod(functional.maxpool1d)
    _bwd = staticmethod(functional.maxpool1ddx)


class _avgpool(Function):
    _fwd = None
    _bwd = None

    def forward(self, tensor1, kernel, stride, padding, return_indices=False):
        result = type(self)._fwd(tensor1, kernel, stride, padding, return_indices)
        out = result[0] if return_indices else result
        out.requires_grad = tensor1.requires_grad
        if out.requires_grad and context.MODE == 0:
            self.tensor1 = tensor1
            self.kernel, self.stride, self.padding = kernel, stride, padding
            out.creator = self
        return result

    def backward(self, grad_output):
        if not self.needs_input_grad[0]:
            return None
        g = type(self)._bwd(grad_output, self.tensor1, self.kernel, self.stride, self.padding)
        self.tensor1 = None
        return g


class avgpooling2d(_avgpool):
    _fwd = staticmethod(functional.avgpool2d)
    _bwd = staticmethod(functional.avgpool2ddx)


class avgpooling1d(_avgpool):
    _fwd = staticmethod(functional.avgpool1d)
    _bwd = staticmethod(functional.avgpool1ddx)


class adaptive_avgpooling2d(Function):
    def forward(self, tensor1, output_size):
        out = functional.adaptive_avgpool2d(tensor1, output_size)
        out.requires_grad = tensor1.requires_grad
        if out.requires_grad and context.MODE == 0:
            self.input_shape = tuple(tensor1.shape)
            self.output_size = output_size
            out.creator = self
        return out

    def backward(self, grad_output):
        if not self.needs_input_grad[0]:
            return None
        g = functional.adaptive_avgpool2ddx(grad_output, self.input_shape, self.output_size)
        self.input_shape = None
        return g


class causal_conv1d(Function):
    """Depthwise causal 1-D convolution (one forward and one backward launch pair)."""

    def forward(self, tensor1, weight, bias):
        out = functional.causal_conv1d(tensor1, weight, bias)
        out.requires_grad = any(self.needs_input_grad)
        return self.attach(out, tensor1=tensor1, weight=weight, bias=bias)

    def backward(self, grad_output):
        need_w = self.needs_input_grad[1] or self.needs_input_grad[2]
        dx, dw, db = functional.causal_conv1d_backward(grad_output, self.tensor1, self.weight,
                                                       self.bias, need_weight_grad=need_w)
        self.tensor1 = self.weight = self.bias = None
        return (dx if self.needs_input_grad[0] else None,
                dw if self.needs_input_grad[1] else None,
                db if self.needs_input_grad[2] else None)
