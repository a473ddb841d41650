"""Hyena long-convolution language model (reference src/wxx/nn/hyena.py:1-329).

One mixer layer, of order n, is a chain of gated long convolutions:

    v, (g_1 .. g_n) = short_conv(x W_v), short_conv(chunk_n(x W_x))
    z_0 = v;   z_i = g_i * (h_i (*) z_{i-1});   y = z_n W_o

``(*)`` is a causal convolution over the sequence, done in the frequency
domain at length next_pow2(2 L) so that it does not wrap, and cropped back to
L samples by the inverse transform itself.  The filters h_i are implicit: a
small network (Linear -> sin(omega x) -> Linear) of a positional encoding of
the L positions, times an exponential window exp(-|decay_i| t).  One
depthwise short convolution is shared by v and every gate.

The parameter tree is the state_dict contract (``embed``, ``layers.<j>.
{norm1, mixer.{proj_v, proj_x, out_proj, short_conv, filter_mlp.<i>.mlp.
{0,2}, decay}, norm2, feed_forward.{w1,w2,w3}}``, ``norm``, ``head``); the
decay rates start uniform in [0, 1) from numpy's global generator, as in
the reference.
"""

import numpy as np

from .. import autograd, functional
from ..Tensor import Parameter, Tensor
from .module import (
    Embedding,
    Linear,
    Module,
    ModuleList,
    PositionalEncoding,
    RMSNorm,
    Sequential,
    Sine,
    SwiGLU,
    TiedLinear,
)


def _pow2_at_least(n):
    """The smallest power of two >= n (1 for n <= 1)."""
    n = int(n)
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


class CausalShortConv1d(Module):
    """Depthwise causal convolution of (B, D, L): y[..., t] = b + sum_k w[:, k] x[..., t - k]
    (torch's Conv1d with the kernel reversed); weights N(0, 0.02), bias 0."""

    def __init__(self, d_model, kernel_size=3):
        super().__init__()
        self.d_model = d_model
        self.kernel_size = kernel_size
        self.weight = Parameter(functional.normal(0, 0.02, (d_model, kernel_size)))
        self.bias = Parameter(Tensor((d_model,), value=0.0))

    def forward(self, x):
        op = autograd.causal_conv1d(x, self.weight, self.bias)
        return op.forward(x, self.weight, self.bias)


class ImplicitFilter(Module):
    """The (d_model, L) filter of one stage: the filter network applied to
    the (L, 2K + 1) positional encoding, transposed."""

    def __init__(self, d_model, hidden_dim=64, pe_features=8, omega=10.0):
        super().__init__()
        self.d_model = d_model
        self.hidden_dim = hidden_dim
        self.pe_features = pe_features
        self.positional_encoding = PositionalEncoding(pe_features)
        width = self.positional_encoding.out_features
        self.mlp = Sequential(Linear(width, hidden_dim), Sine(omega), Linear(hidden_dim, d_model))

    def forward(self, L):
        return self.mlp(self.positional_encoding(L)).transpose(0, 1)


class HyenaOperator(Module):
    def __init__(self, d_model, order=2, fft_size=None, short_conv_kernel=3, filter_hidden=64,
                 pe_features=8, filter_omega=10.0):
        super().__init__()
        for what, value in (("order", order), ("short_conv_kernel", short_conv_kernel)):
            if value < 1:
                raise ValueError(f"{what} must be >= 1, got {value}")
        self.d_model = d_model
        self.order = int(order)
        self.fft_size = fft_size
        self.proj_v = Linear(d_model, d_model, bias=False)
        self.proj_x = Linear(d_model, self.order * d_model, bias=False)
        self.out_proj = Linear(d_model, d_model, bias=False)
        self.short_conv = CausalShortConv1d(d_model, kernel_size=short_conv_kernel)
        self.filter_mlp = ModuleList([ImplicitFilter(d_model, filter_hidden, pe_features,
                                                     filter_omega)
                                      for _ in range(self.order)])
        rates = np.random.rand(self.order, d_model).astype(np.float32)
        self.decay = Parameter(functional.from_numpy(rates))

    def _fft_size(self, length):
        """The transform length: ``fft_size`` if given (raised to the next
        power of two >= length when it is shorter), else next_pow2(2 L)."""
        n = _pow2_at_least(2 * length) if self.fft_size is None else int(self.fft_size)
        return n if n >= length else _pow2_at_least(length)

    def fft_conv1d(self, x, h):
        """Causal convolution of (B, D, L) signals with (D, L) filters, cropped
        to L: irfft(rfft(x) * rfft(h)), as one fused op (``autograd.fft_conv``,
        equal bit for bit to the composed ops) where the transform length
        allows."""
        length = x.shape[-1]
        n = self._fft_size(length)
        if (functional.fused_spectrum_supported(n) and len(h.shape) == 2
                and len(x.shape) >= 2 and h.shape[0] == x.shape[-2]):
            return autograd.fft_conv(x, h).forward(x, h, n, min(length, n))
        spectrum = x.rfft(n).complex_mul(h.rfft(n))
        return spectrum.irfft(n, min(length, n))

    def _filter(self, stage, length):
        window = autograd.decay_window(self.decay).forward(self.decay, stage, length)
        return self.filter_mlp[stage](length) * window

    def forward(self, x):
        length = x.shape[1]
        to_channels = [t.transpose(1, 2) for t in
                       [self.proj_v(x)] + list(self.proj_x(x).chunk(self.order, dim=-1))]
        z, *gates = [self.short_conv(t) for t in to_channels]
        for stage, gate in enumerate(gates):
            z = gate * self.fft_conv1d(z, self._filter(stage, length))
        return self.out_proj(z.transpose(1, 2))


class HyenaBlock(Module):
    """Pre-norm residual pair: + Hyena(RMSNorm x), + SwiGLU(RMSNorm x)."""

    def __init__(self, d_model, mlp_ratio=4, hidden_dim=None, order=2, short_conv_kernel=3,
                 filter_hidden=64, pe_features=8, filter_omega=10.0):
        super().__init__()
        self.norm1 = RMSNorm(d_model)
        self.mixer = HyenaOperator(d_model, order=order, short_conv_kernel=short_conv_kernel,
                                   filter_hidden=filter_hidden, pe_features=pe_features,
                                   filter_omega=filter_omega)
        self.norm2 = RMSNorm(d_model)
        self.feed_forward = SwiGLU(d_model, hidden_dim=hidden_dim, mlp_ratio=mlp_ratio)

    def forward(self, x):
        mixed = x + self.mixer(self.norm1(x))
        return mixed + self.feed_forward(self.norm2(mixed))


class Hyena(Module):
    """Token embedding, ``n_layers`` Hyena blocks, RMSNorm and a head tied to
    the embedding (or a biased Linear with ``tie_weights=False``)."""

    def __init__(self, vocab_size, d_model=256, n_layers=8, mlp_ratio=4, hidden_dim=None,
                 tie_weights=True, embed_init_std=0.02, order=2, short_conv_kernel=3,
                 filter_hidden=64, pe_features=8, filter_omega=10.0):
        super().__init__()
        self.vocab_size = vocab_size
        self.d_model = d_model
        self.order = order
        self.embed = Embedding(vocab_size, d_model, init_std=embed_init_std)
        block_args = dict(mlp_ratio=mlp_ratio, hidden_dim=hidden_dim, order=order,
                          short_conv_kernel=short_conv_kernel, filter_hidden=filter_hidden,
                          pe_features=pe_features, filter_omega=filter_omega)
        self.layers = ModuleList([HyenaBlock(d_model, **block_args) for _ in range(n_layers)])
        self.norm = RMSNorm(d_model)
        self.head = TiedLinear(self.embed) if tie_weights else Linear(d_model, vocab_size)

    def forward(self, x):
        h = self.embed(x)
        for block in self.layers:
            h = block(h)
        return self.head(self.norm(h))


__all__ = ["Sine", "PositionalEncoding", "CausalShortConv1d", "ImplicitFilter", "HyenaOperator",
           "SwiGLU", "HyenaBlock", "TiedLinear", "Hyena"]
