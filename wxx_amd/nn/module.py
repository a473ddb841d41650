"""Layers of the nn API (reference src/wxx/nn/module.py:18-597).

Same class names, constructor arguments, parameter names and forward
semantics as the reference, so models and state_dicts move between the two
unchanged.  Two reference behaviours are kept on purpose because training
results depend on them:

* a ``Parameter`` assigned to a second attribute is registered under both
  names (``LayerNorm`` exposes ``weightg``/``weightb`` and the aliases
  ``weight``/``bias``), so ``parameters()`` yields it twice and an optimizer
  steps it twice (module.py:23-35, 198-208);
* ``Embedding`` and the GPT-2 / Hyena initialisers draw from unseeded numpy
  generators, as the reference does; parity tests inject weights through
  ``load_state_dict``.
"""

import math

import numpy as np

from .. import autograd, functional
from ..backend import context
from ..backend.device import get_cmd_buffer
from ..Tensor import Parameter, Tensor

cmd_encoder = get_cmd_buffer()


class Module:
    def __init__(self):
        object.__setattr__(self, "_parameters", {})
        object.__setattr__(self, "_modules", {})

    def __setattr__(self, name, value):
        if isinstance(value, Parameter):
            self._parameters[name] = value
        elif isinstance(value, Module):
            self._modules[name] = value
        object.__setattr__(self, name, value)

    def __call__(self, *x):
        return self.forward(*x)

    def parameters(self, recurse=True):
        """``("", parameter)`` pairs: own parameters first, then submodules'."""
        for p in self._parameters.values():
            if p is not None:
                yield ("", p)
        if recurse:
            for m in self._modules.values():
                if m is not None:
                    yield from m.parameters(recurse=True)

    def named_parameters(self, prefix="", recurse=True):
        for name, p in self._parameters.items():
            if p is not None:
                yield (prefix + name, p)
        if recurse:
            for name, m in self._modules.items():
                if m is not None:
                    yield from m.named_parameters(prefix + name + ".", recurse=True)

    def state_dict(self, prefix="", destination=None):
        """Parameter name -> host numpy copy."""
        dest = {} if destination is None else destination
        for name, p in self._parameters.items():
            if p is not None:
                dest[prefix + name] = np.asarray(p.numpy() if hasattr(p, "numpy") else p).copy()
        for name, m in self._modules.items():
            if m is not None:
                m.state_dict(prefix + name + ".", dest)
        return dest

    def load_state_dict(self, state_dict, strict=True):
        own = set(self.state_dict().keys())
        for name, p in self.named_parameters():
            if name in state_dict:
                val = state_dict[name]
                if hasattr(val, "numpy") and not isinstance(val, np.ndarray):
                    val = val.numpy()
                val = np.asarray(val)
                if p.type == "c64":
                    functional.assign(p, functional.from_numpy_complex(val))
                elif p.type == "u32":
                    functional.assign(p, functional.from_numpy(val, dtype=np.uint32))
                else:
                    functional.assign(p, functional.from_numpy(val))
            elif strict:
                raise KeyError(f"Missing key in state_dict: {name}")
        if strict:
            missing = own - set(state_dict.keys())
            unexpected = set(state_dict.keys()) - own
            if missing:
                raise RuntimeError(f"Missing keys: {sorted(missing)}")
            if unexpected:
                raise RuntimeError(f"Unexpected keys: {sorted(unexpected)}")

    def zero_grad(self, wait=False):
        for _, p in self.named_parameters():
            if p.grad is not None:
                p.grad = None
        cmd_encoder.flush(wait=wait)

    def forward(self, *args, **kwargs):
        raise NotImplementedError

    def __repr__(self):
        lines = [type(self).__name__ + "("]
        lines += [f"  ({n}): {m!r}" for n, m in self._modules.items()]
        lines.append(")")
        return "\n".join(lines)


class ModuleList(Module):
    def __init__(self, modules=None):
        super().__init__()
        for i, m in enumerate(modules or []):
            setattr(self, str(i), m)

    def __getitem__(self, idx):
        if isinstance(idx, slice):
            return [self._modules[str(i)] for i in range(*idx.indices(len(self)))]
        return self._modules[str(idx)]

    def __iter__(self):
        return iter(self._modules.values())

    def __len__(self):
        return len(self._modules)

    def append(self, module):
        setattr(self, str(len(self._modules)), module)

    def forward(self, x, *args, **kwargs):
        for m in self._modules.values():
            x = m(x, *args, **kwargs)
        return x


class Sequential(Module):
    def __init__(self, *modules):
        super().__init__()
        for i, m in enumerate(modules):
            setattr(self, str(i), m)

    def forward(self, x, *args, **kwargs):
        for m in self._modules.values():
            x = m(x, *args, **kwargs)
        return x


class Linear(Module):
    """``y = x @ W + b`` with ``W`` of shape (in, out), Kaiming-normal init."""

    def __init__(self, in_features, out_features, bias=True):
        super().__init__()
        self.weight = Parameter(Tensor((in_features, out_features)))
        functional._kaiming_normal_init(self.weight, in_features)
        self.bias = Parameter(Tensor((out_features,), value=0.0)) if bias else None

    def forward(self, x):
        if self.bias is None:
            return autograd.matmul(x, self.weight).forward(x, self.weight)
        return autograd.matmuladd(x, self.weight, self.bias).forward(x, self.weight, self.bias)


class Embedding(Module):
    def __init__(self, num_embeddings, embedding_dim, init_std=0.02):
        super().__init__()
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        self.weight = Parameter(Tensor((num_embeddings, embedding_dim)))
        functional.assign(self.weight,
                          functional.normal(0, init_std, (num_embeddings, embedding_dim)))

    def forward(self, x):
        n = x.shape[0] * x.shape[1] if len(x.shape) > 1 else x.shape[0]
        return autograd.Embedding(x, self.weight).forward(x, self.weight, n, self.embedding_dim,
                                                          self.num_embeddings)


class Dropout(Module):
    def __init__(self, p=0.5):
        super().__init__()
        self.p = p

    def forward(self, x):
        if context.MODE != 0:
            return x
        return autograd.Dropout(x).forward(x, self.p)


class LayerNorm(Module):
    def __init__(self, normalized_shape, eps=1e-5):
        super().__init__()
        if isinstance(normalized_shape, int):
            normalized_shape = (normalized_shape,)
        self.normalized_shape = tuple(normalized_shape)
        self.eps = eps
        self.weightg = Parameter(Tensor(self.normalized_shape, value=1.0))
        self.weightb = Parameter(Tensor(self.normalized_shape, value=0.0))
        # aliases, registered as parameters too (reference module.py:206-207)
        self.weight = self.weightg
        self.bias = self.weightb

    def forward(self, x):
        nd = len(self.normalized_shape)
        axis = tuple(range(len(x.shape) - nd, len(x.shape)))
        return autograd.meanvarnorm(x, self.weightg, self.weightb).forward(
            x, self.weightg, self.weightb, axis=axis if len(axis) > 1 else axis[0])


class RMSNorm(Module):
    def __init__(self, d_model, eps=1e-6):
        super().__init__()
        self.d_model = d_model
        self.eps = eps
        self.weight = Parameter(Tensor((d_model,), value=1.0))

    def forward(self, x):
        return autograd.rmsnorm(x, self.weight).forward(x, self.weight, -1)


class BatchNorm(Module):
    """Training-mode batch statistics; ``running_std`` holds the running
    variance (its name is the reference's, module.py:238)."""

    def __init__(self, num_features, eps=1e-5, momentum=0.1):
        super().__init__()
        self.num_features = num_features
        self.eps = eps
        self.momentum = momentum
        self.weight = Parameter(Tensor((num_features,), value=1.0))
        self.bias = Parameter(Tensor((num_features,), value=0.0))
        self.running_mean = Tensor((num_features,), value=0.0)
        self.running_std = Tensor((num_features,), value=1.0)

    def forward(self, x):
        return autograd.batchnorm(x, self.weight, self.bias).forward(
            x, self.weight, self.bias, self.running_mean, self.running_std, context.MODE == 0)


def _pair(v):
    return (v, v) if isinstance(v, int) else v


class Conv2D(Module):
    def __init__(self, in_channels, out_channels, kernel=3, stride=1, padding=0, dilation=1,
                 bias=True):
        super().__init__()
        kernel, stride, padding, dilation = map(_pair, (kernel, stride, padding, dilation))
        self.kernel, self.stride, self.padding, self.dilation = kernel, stride, padding, dilation
        self.W = Parameter(Tensor((out_channels, in_channels, kernel[0], kernel[1])))
        functional._kaiming_normal_init(self.W, math.prod(kernel) * in_channels)
        self.bias = Parameter(Tensor((out_channels,), value=0.0)) if bias else None

    def forward(self, x):
        if self.bias is None:
            return autograd.Conv2D(x, self.W).forward(x, self.W, None, self.stride, self.padding,
                                                      self.dilation)
        return autograd.Conv2D(x, self.W, self.bias).forward(x, self.W, self.bias, self.stride,
                                                             self.padding, self.dilation)


class Conv2DTranspose(Module):
    """``ConvTranspose2d``: ``W`` is (in, out, KH, KW); spatial size
    ``(H - 1) * stride - 2 * padding + dilation * (K - 1) + output_padding + 1``."""

    def __init__(self, in_channels, out_channels, kernel=3, stride=1, padding=0,
                 output_padding=0, dilation=1, bias=True):
        super().__init__()
        kernel, stride, padding, output_padding, dilation = map(
            _pair, (kernel, stride, padding, output_padding, dilation))
        for axis, name in enumerate(("height", "width")):
            limit = max(stride[axis], dilation[axis])
            if not 0 <= output_padding[axis] < limit:
                raise ValueError(f"output_padding[{axis}] must be in [0, {limit}) for {name}, "
                                 f"got {output_padding[axis]}")
        self.kernel, self.stride, self.padding = kernel, stride, padding
        self.output_padding, self.dilation = output_padding, dilation
        self.W = Parameter(Tensor((in_channels, out_channels, kernel[0], kernel[1])))
        functional._kaiming_normal_init(self.W, math.prod(kernel) * in_channels)
        self.bias = Parameter(Tensor((out_channels,), value=0.0)) if bias else None

    def forward(self, x):
        args = (self.stride, self.padding, self.output_padding, self.dilation)
        if self.bias is None:
            return autograd.Conv2DTranspose(x, self.W).forward(x, self.W, None, *args)
        return autograd.Conv2DTranspose(x, self.W, self.bias).forward(x, self.W, self.bias, *args)


class MaxPool1d(Module):
    def __init__(self, kernel, stride=None, padding=0, return_indices=False):
        super().__init__()
        self.kernel = kernel
        self.stride = kernel if stride is None else stride
        self.padding = padding
        self.return_indices = return_indices

    def forward(self, x):
        return autograd.maxpooling1d(x).forward(x, self.kernel, self.stride, self.padding,
                                                self.return_indices)


class MaxPool2d(Module):
    def __init__(self, kernel, stride=None, padding=0, return_indices=False):
        super().__init__()
        self.kernel = _pair(kernel)
        self.stride = self.kernel if stride is None else _pair(stride)
        self.padding = _pair(padding)
        self.return_indices = return_indices

    def forward(self, x):
        return autograd.maxpooling2d(x).forward(x, self.kernel, self.stride, self.padding,
                                                self.return_indices)


class AvgPool1d(Module):
    def __init__(self, kernel, stride=None, padding=0, return_indices=False):
        super().__init__()
        self.kernel = kernel
        self.stride = kernel if stride is None else stride
        self.padding = padding
        self.return_indices = return_indices

    def forward(self, x):
        return autograd.avgpooling1d(x).forward(x, self.kernel, self.stride, self.padding,
                                                self.return_indices)


class AvgPool2d(Module):
    def __init__(self, kernel, stride=None, padding=0, return_indices=False):
        super().__init__()
        self.kernel = _pair(kernel)
        self.stride = self.kernel if stride is None else _pair(stride)
        self.padding = _pair(padding)
        self.return_indices = return_indices

    def forward(self, x):
        return autograd.avgpooling2d(x).forward(x, self.kernel, self.stride, self.padding,
                                                self.return_indices)


class AdaptiveAvgPool2d(Module):
    def __init__(self, output_size):
        super().__init__()
        self.output_size = tuple(int(v) for v in _pair(output_size))

    def forward(self, x):
        return autograd.adaptive_avgpooling2d(x).forward(x, self.output_size)


class MultiHeadAttention(Module):
    """Softmax attention over (B, S, D): per-head Q K^T / sqrt(d_head) (+ mask),
    softmax, dropout, times V, output projection; no projection biases."""

    def __init__(self, d_model, n_heads, dropout=0.0):
        super().__init__()
        assert d_model % n_heads == 0
        self.d_model = d_model
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads
        self.q = Linear(d_model, d_model, bias=False)
        self.k = Linear(d_model, d_model, bias=False)
        self.v = Linear(d_model, d_model, bias=False)
        self.out = Linear(d_model, d_model, bias=False)
        self.drop = Dropout(dropout)

    def _heads(self, t, b, seq):
        return (t.reshape((b, seq, self.n_heads, self.head_dim)).permute(0, 2, 1, 3)
                .reshape((b * self.n_heads, seq, self.head_dim)))

    def forward(self, x, mask=None):
        b, seq, _ = x.shape
        q = self._heads(self.q(x), b, seq)
        k = self._heads(self.k(x), b, seq)
        v = self._heads(self.v(x), b, seq)
        # Under GPT-2's causal mask (-1e9 above the diagonal) the scores above
        # the diagonal get probability exactly 0 and their gradients are
        # exactly 0, so the products skip those triangles with unchanged results.
        causal = (mask is not None and getattr(mask, "_causal", False)
                  and tuple(mask.shape) == (seq, seq) and seq <= 16384)
        # Without attention dropout every consumer of the scores, the
        # probabilities and their gradients reads only the lower triangle, so
        # the upper one is not even written.
        skip = causal and self.drop.p == 0
        suffix = "_skip" if skip else ""
        score = autograd.matmul(q, k).forward(q, k, transpose_b=True,
                                              causal="scores" + suffix if causal else None)
        scale = 1.0 / math.sqrt(self.head_dim)
        if causal:
            attn = autograd.scaled_masked_softmax(score).forward(score, scale, mask,
                                                                 causal=2 if skip else 1)
        elif mask is None or (len(mask.shape) == 2 and not mask.requires_grad):
            # scale, mask add and softmax as one pass over the scores (same
            # roundings as the three separate ops)
            attn = autograd.scaled_masked_softmax(score).forward(score, scale, mask)
        else:
            score = score * scale
            attn = (score + mask).softmax(dim=-1)
        attn = self.drop(attn)
        out = autograd.matmul(attn, v).forward(attn, v,
                                               causal="probs" + suffix if causal else None)
        out = (out.reshape((b, self.n_heads, seq, self.head_dim)).permute(0, 2, 1, 3)
               .reshape((b, seq, self.d_model)))
        return self.out(out)


class Attention(Module):
    def __init__(self, d_model, n_heads=1):
        super().__init__()
        self.mha = MultiHeadAttention(d_model, n_heads)

    def forward(self, x, mask=None):
        return self.mha(x, mask)


class GELU(Module):
    def forward(self, x):
        return x.gelu()


class Sine(Module):
    """``sin(omega * x)``."""

    def __init__(self, omega=10.0):
        super().__init__()
        self.omega = float(omega)

    def forward(self, x):
        return (x * self.omega).sin()

    def extra_repr(self):
        return f"omega={self.omega}"


class SwiGLU(Module):
    """``w3(silu(w1 x) * w2 x)``; hidden width int(2 * mlp_ratio * d / 3) by default."""

    def __init__(self, d_model, hidden_dim=None, mlp_ratio=4):
        super().__init__()
        if hidden_dim is None:
            hidden_dim = int(2 * (mlp_ratio * d_model) / 3)
        self.hidden_dim = hidden_dim
        self.w1 = Linear(d_model, hidden_dim, bias=False)
        self.w2 = Linear(d_model, hidden_dim, bias=False)
        self.w3 = Linear(hidden_dim, d_model, bias=False)

    def forward(self, x):
        return self.w3(self.w1(x).silu() * self.w2(x))


class TiedLinear(Module):
    """``x @ E^T`` with the embedding table ``E`` (not registered a second time)."""

    def __init__(self, embedding):
        super().__init__()
        object.__setattr__(self, "_embedding", embedding)

    def forward(self, x):
        w = self._embedding.weight
        return autograd.matmul(x, w).forward(x, w, False, True)


class PositionalEncoding(Module):
    """``[t, cos(2 pi k t), sin(2 pi k t)]`` for t = linspace(0, 1, L), k < features."""

    def __init__(self, features=8):
        super().__init__()
        features = int(features)
        if features < 1:
            raise ValueError(f"positional features must be >= 1, got {features}")
        self.features = features
        self.out_features = 2 * features + 1
        self._cache = {}

    def _build(self, length):
        t = np.linspace(0.0, 1.0, int(length), dtype=np.float32)
        ang = (2.0 * np.pi) * np.outer(t, np.arange(self.features, dtype=np.float32))
        return np.concatenate([t[:, None], np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)

    def forward(self, length):
        key = (int(length), self.features)
        pe = self._cache.get(key)
        if pe is None:
            pe = Tensor((key[0], self.out_features), data=self._build(length).tobytes())
            self._cache[key] = pe
        return pe

    def extra_repr(self):
        return f"features={self.features}, out_features={self.out_features}"
