"""Differentiable RMSNorm, LayerNorm and BatchNorm (reference
src/wxx/autograd/normalization.py:6-108)."""

from .. import functional
from .function import Function


class rmsnorm(Function):
    def forward(self, tensor1, gamma, axis=None):
        out, irms = functional.rmsnorm(tensor1, gamma, axis)
        out.requires_grad = tensor1.requires_grad or gamma.requires_grad
        self.axis = axis
        return self.attach(out, tensor1=tensor1, irms=irms, gamma=gamma)

    def backward(self, g):
        x, gamma, irms = self.tensor1, self.gamma, self.irms
        self.tensor1 = self.gamma = self.irms = None
        gx = functional.rmsnormdx(g, x, gamma, irms, self.axis) if self.needs_input_grad[0] else None
        gg = functional.rmsnormdg(g, x, gamma, irms, self.axis) if self.needs_input_grad[1] else None
        return gx, gg


class meanvarnorm(Function):
    def forward(self, tensor1, gamma, beta, axis=None):
        out, mean, istd = functional.meanvarnorm(tensor1, gamma, beta, axis)
        out.requires_grad = tensor1.requires_grad or gamma.requires_grad or beta.requires_grad
        self.axis = axis
        return self.attach(out, tensor1=tensor1, gamma=gamma, mean=mean, istd=istd)

    def backward(self, g):
        x, gamma, mean, istd = self.tensor1, self.gamma, self.mean, self.istd
        self.tensor1 = self.gamma = self.mean = self.istd = None
        gx = (functional.meanvarnormdx(g, x, gamma, mean, istd, self.axis)
              if self.needs_input_grad[0] else None)
        gg = gb = None
        if self.needs_input_grad[1] or self.needs_input_grad[2]:
            gg, gb = functional.meanvarnormdg(g, x, mean, istd, self.axis)
        return gx, gg, gb


class batchnorm(Function):
    def forward(self, tensor1, gamma, beta, running_mean, running_var, training=False):
        out, mean, istd = functional.batchnorm(tensor1, gamma, beta, running_mean, running_var,
                                               training)
        out.requires_grad = tensor1.requires_grad or gamma.requires_grad or beta.requires_grad
        return self.attach(out, tensor1=tensor1, gamma=gamma, mean=mean, istd=istd)

    def backward(self, g):
        x, gamma, mean, istd = self.tensor1, self.gamma, self.mean, self.istd
        self.tensor1 = self.gamma = self.mean = self.istd = None
        gx, gg, gb = functional.batchnorm_backward(g, x, gamma, mean, istd)
        grads = [gx, gg, gb]
        return grads + [None] * (len(self.inputs) - 3)


class batchnorm_act(Function):
    """Training-mode batchnorm, + residual and ReLU as one op (built as
    ``batchnorm_act(x, gamma, beta[, residual])``); its backward is the
    composed ops' (batchnorm's, the add's, the ReLU's) in one kernel."""

    def forward(self, tensor1, gamma, beta, residual, running_mean, running_var, updates=1,
                relu=True):
        out, mean, istd = functional.batchnorm_act(tensor1, gamma, beta, residual, running_mean,
                                                   running_var, updates, relu)
        out.requires_grad = any(t.requires_grad for t in (tensor1, gamma, beta, residual)
                                if t is not None)
        return self.attach(out, tensor1=tensor1, gamma=gamma, beta=beta, residual=residual,
                           mean=mean, istd=istd, relu=relu)

    def backward(self, g):
        x, gamma, beta, r = self.tensor1, self.gamma, self.beta, self.residual
        mean, istd = self.mean, self.istd
        self.tensor1 = self.gamma = self.beta = self.residual = self.mean = self.istd = None
        gx, gg, gb, gr = functional.batchnorm_act_backward(g, x, gamma, beta, r, mean, istd,
                                                           self.relu)
        return [gx, gg, gb, gr][:len(self.inputs)]
