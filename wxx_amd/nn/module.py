"""Layers of the nn API (reference src/wxx/nn/module.py:18-597).

The class names, constructor arguments, attribute and parameter names and
the forward semantics are the reference's, so models and state_dicts move
between the two unchanged.  Two reference behaviours are kept on purpose
because training results depend on them:

* a ``Parameter`` assigned to a second attribute is registered under both
  names (``LayerNorm`` has ``weightg``/``weightb`` and the aliases
  ``weight``/``bias``), so ``parameters()`` yields it twice and an optimizer
  steps it twice (module.py:23-35, 198-208);
* weights are drawn from unseeded numpy generators, as the reference does;
  parity tests inject weights through ``load_state_dict``.

A module keeps its own parameters and children in two ordered registries
(``_parameters``, ``_modules``) filled by attribute assignment; every
traversal (``parameters``, ``named_parameters``, ``state_dict``) is the
same depth-first walk over them, own parameters before children.
"""

import math

import numpy as np

from .. import autograd, functional
from ..backend import context
from ..backend.device import get_cmd_buffer
from ..Tensor import Parameter, Tensor

cmd_encoder = get_cmd_buffer()

# how a host array is uploaded into a parameter of each dtype
_UPLOAD = {
    "f32": lambda a: functional.from_numpy(a),
    "u32": lambda a: functional.from_numpy(a, dtype=np.uint32),
    "c64": lambda a: functional.from_numpy_complex(a),
}


def _host(value):
    """A numpy array of a device tensor or an array-like."""
    if hasattr(value, "numpy") and not isinstance(value, np.ndarray):
        value = value.numpy()
    return np.asarray(value)


class Module:
    def __init__(self):
        object.__setattr__(self, "_parameters", {})
        object.__setattr__(self, "_modules", {})

    def __setattr__(self, name, value):
        registry = (self._parameters if isinstance(value, Parameter)
                    else self._modules if isinstance(value, Module) else None)
        if registry is not None:
            registry[name] = value
        object.__setattr__(self, name, value)

    def __call__(self, *x):
        return self.forward(*x)

    def forward(self, *args, **kwargs):
        raise NotImplementedError(f"{type(self).__name__} does not define forward")

    def _walk(self, prefix, recurse):
        """(qualified name, parameter) depth first, own parameters first."""
        for name, p in self._parameters.items():
            if p is not None:
                yield prefix + name, p
        if recurse:
            for name, child in self._modules.items():
                if child is not None:
                    yield from child._walk(f"{prefix}{name}.", True)

    def parameters(self, recurse=True):
        """``("", parameter)`` pairs (the optimizers' input format)."""
        return (("", p) for _, p in self._walk("", recurse))

    def named_parameters(self, prefix="", recurse=True):
        return self._walk(prefix, recurse)

    def state_dict(self, prefix="", destination=None):
        """Parameter name -> host numpy copy (aliases under each name)."""
        out = {} if destination is None else destination
        for name, p in self._walk(prefix, True):
            out[name] = np.array(_host(p), copy=True)
        return out

    def load_state_dict(self, state_dict, strict=True):
        """Copy the arrays of ``state_dict`` into the parameters of the same
        names.  ``strict``: a parameter without an entry is a ``KeyError``,
        and entries or parameters left unmatched a ``RuntimeError``."""
        names = [name for name, _ in self._walk("", True)]
        for name, p in self._walk("", True):
            if name not in state_dict:
                if strict:
                    raise KeyError(f"Missing key in state_dict: {name}")
                continue
            functional.assign(p, _UPLOAD[p.type](_host(state_dict[name])))
        if strict:
            given, own = set(state_dict), set(names)
            if own - given:
                raise RuntimeError(f"Missing keys: {sorted(own - given)}")
            if given - own:
                raise RuntimeError(f"Unexpected keys: {sorted(given - own)}")

    def zero_grad(self, wait=False):
        for _, p in self._walk("", True):
            p.grad = None
        cmd_encoder.flush(wait=wait)

    def __repr__(self):
        inner = [f"  ({name}): {child!r}" for name, child in self._modules.items()]
        return "\n".join([f"{type(self).__name__}("] + inner + [")"])


class Sequential(Module):
    """Children named "0", "1", ... applied in order."""

    def __init__(self, *modules):
        super().__init__()
        for i, m in enumerate(modules):
            setattr(self, str(i), m)

    def forward(self, x, *args, **kwargs):
        for child in self._modules.values():
            x = child(x, *args, **kwargs)
        return x


class ModuleList(Sequential):
    """An indexable, appendable list of children (forward applies them in order)."""

    def __init__(self, modules=None):
        super().__init__(*(modules or ()))

    def __getitem__(self, idx):
        if isinstance(idx, slice):
            return [self._modules[str(i)] for i in range(*idx.indices(len(self)))]
        return self._modules[str(idx)]

    def __iter__(self):
        return iter(self._modules.values())

    def __len__(self):
        return len(self._modules)

    def append(self, module):
        setattr(self, str(len(self)), module)


def _kaiming(shape, fan_in):
    t = Tensor(shape)
    functional._kaiming_normal_init(t, fan_in)
    return t


def _filled(shape, value):
    return Tensor(shape, value=value)


class Linear(Module):
    """y = x W (+ b) with W stored (in, out); W Kaiming-normal, b zero."""

    def __init__(self, in_features, out_features, bias=True):
        super().__init__()
        self.weight = Parameter(_kaiming((in_features, out_features), in_features))
        self.bias = Parameter(_filled((out_features,), 0.0)) if bias else None

    def forward(self, x):
        if self.bias is not None:
            return autograd.matmuladd(x, self.weight, self.bias).forward(x, self.weight,
                                                                          self.bias)
        return autograd.matmul(x, self.weight).forward(x, self.weight)


class Embedding(Module):
    """Rows of a (num_embeddings, embedding_dim) table, N(0, init_std) at start."""

    def __init__(self, num_embeddings, embedding_dim, init_std=0.02):
        super().__init__()
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        shape = (num_embeddings, embedding_dim)
        self.weight = Parameter(functional.normal(0, init_std, shape))

    def forward(self, x):
        tokens = math.prod(x.shape[:2])
        op = autograd.Embedding(x, self.weight)
        return op.forward(x, self.weight, tokens, self.embedding_dim, self.num_embeddings)


class Dropout(Module):
    """Inverted dropout while recording; the identity in inference mode."""

    def __init__(self, p=0.5):
        super().__init__()
        self.p = p

    def forward(self, x):
        if context.MODE == 0:
            return autograd.Dropout(x).forward(x, self.p)
        return x


class LayerNorm(Module):
    """Over the trailing ``normalized_shape`` dims, gamma ``weightg`` and beta
    ``weightb``, also registered as ``weight`` / ``bias``."""

    def __init__(self, normalized_shape, eps=1e-5):
        super().__init__()
        shape = (normalized_shape,) if isinstance(normalized_shape, int) else normalized_shape
        self.normalized_shape = tuple(shape)
        self.eps = eps
        self.weightg = Parameter(_filled(self.normalized_shape, 1.0))
        self.weightb = Parameter(_filled(self.normalized_shape, 0.0))
        self.weight, self.bias = self.weightg, self.weightb

    def forward(self, x):
        rank, k = len(x.shape), len(self.normalized_shape)
        axes = tuple(range(rank - k, rank))
        op = autograd.meanvarnorm(x, self.weightg, self.weightb)
        return op.forward(x, self.weightg, self.weightb, axis=axes[0] if k == 1 else axes)


class RMSNorm(Module):
    def __init__(self, d_model, eps=1e-6):
        super().__init__()
        self.d_model = d_model
        self.eps = eps
        self.weight = Parameter(_filled((d_model,), 1.0))

    def forward(self, x):
        return autograd.rmsnorm(x, self.weight).forward(x, self.weight, -1)


class BatchNorm(Module):
    """Batch statistics while recording, running ones in inference mode;
    ``running_std`` holds the running variance (the reference's name,
    module.py:238)."""

    def __init__(self, num_features, eps=1e-5, momentum=0.1):
        super().__init__()
        self.num_features = num_features
        self.eps = eps
        self.momentum = momentum
        self.weight = Parameter(_filled((num_features,), 1.0))
        self.bias = Parameter(_filled((num_features,), 0.0))
        self.running_mean = _filled((num_features,), 0.0)
        self.running_std = _filled((num_features,), 1.0)

    def forward(self, x):
        op = autograd.batchnorm(x, self.weight, self.bias)
        return op.forward(x, self.weight, self.bias, self.running_mean, self.running_std,
                          context.MODE == 0)

    def act(self, x, residual=None, relu=True, updates=1):
        """``relu(self(x) + residual)`` (add and ReLU optional) after ``updates``
        evaluations of ``self(x)``: while recording, one fused kernel where it
        takes the shape (the running statistics take the ``updates`` EMA steps
        the repeated calls would), otherwise the calls themselves."""
        recording = context.MODE == 0
        if recording and functional.batchnorm_act_supported(x):
            inputs = (x, self.weight, self.bias) + (() if residual is None else (residual,))
            return autograd.batchnorm_act(*inputs).forward(
                x, self.weight, self.bias, residual, self.running_mean, self.running_std,
                updates, relu)
        for _ in range(updates - 1 if recording else 0):
            self(x)
        out = self(x)
        if residual is not None:
            out = out + residual
        return out.relu() if relu else out


def _pair(v):
    return (v, v) if isinstance(v, int) else v


class Conv2D(Module):
    """NCHW convolution; W (out, in, KH, KW), Kaiming-normal over in KH KW."""

    def __init__(self, in_channels, out_channels, kernel=3, stride=1, padding=0, dilation=1,
                 bias=True):
        super().__init__()
        self.kernel, self.stride, self.padding, self.dilation = (
            _pair(v) for v in (kernel, stride, padding, dilation))
        kh, kw = self.kernel
        self.W = Parameter(_kaiming((out_channels, in_channels, kh, kw), kh * kw * in_channels))
        self.bias = Parameter(_filled((out_channels,), 0.0)) if bias else None

    def forward(self, x):
        inputs = (x, self.W) if self.bias is None else (x, self.W, self.bias)
        return autograd.Conv2D(*inputs).forward(x, self.W, self.bias, self.stride, self.padding,
                                                self.dilation)


class Conv2DTranspose(Module):
    """``ConvTranspose2d``: W (in, out, KH, KW); the spatial size grows to
    (H - 1) stride - 2 padding + dilation (K - 1) + output_padding + 1, with
    0 <= output_padding < max(stride, dilation) per axis."""

    def __init__(self, in_channels, out_channels, kernel=3, stride=1, padding=0,
                 output_padding=0, dilation=1, bias=True):
        super().__init__()
        self.kernel, self.stride, self.padding, self.output_padding, self.dilation = (
            _pair(v) for v in (kernel, stride, padding, output_padding, dilation))
        for axis, label in enumerate(("height", "width")):
            bound = max(self.stride[axis], self.dilation[axis])
            if not 0 <= self.output_padding[axis] < bound:
                raise ValueError(f"output_padding[{axis}] must be in [0, {bound}) for {label}, "
                                 f"got {self.output_padding[axis]}")
        kh, kw = self.kernel
        self.W = Parameter(_kaiming((in_channels, out_channels, kh, kw), kh * kw * in_channels))
        self.bias = Parameter(_filled((out_channels,), 0.0)) if bias else None

    def forward(self, x):
        inputs = (x, self.W) if self.bias is None else (x, self.W, self.bias)
        return autograd.Conv2DTranspose(*inputs).forward(
            x, self.W, self.bias, self.stride, self.padding, self.output_padding, self.dilation)


def _pooling(name, function, two_d, doc):
    """A pooling module class: ``kernel`` / ``stride`` (default: the kernel) /
    ``padding`` are ints, or pairs for the 2-D pools, and ``return_indices``
    asks the max pools for their flat u32 input indices too."""

    def __init__(self, kernel, stride=None, padding=0, return_indices=False):
        Module.__init__(self)
        norm = _pair if two_d else (lambda v: v)
        self.kernel = norm(kernel)
        self.stride = self.kernel if stride is None else norm(stride)
        self.padding = norm(padding)
        self.return_indices = return_indices

    def forward(self, x):
        op = getattr(autograd, function)(x)
        return op.forward(x, self.kernel, self.stride, self.padding, self.return_indices)

    return type(name, (Module,), {"__init__": __init__, "forward": forward, "__doc__": doc})


MaxPool1d = _pooling("MaxPool1d", "maxpooling1d", False, "Max pooling over the last axis.")
MaxPool2d = _pooling("MaxPool2d", "maxpooling2d", True, "Max pooling over H and W.")
AvgPool1d = _pooling("AvgPool1d", "avgpooling1d", False, "Average pooling over the last axis.")
AvgPool2d = _pooling("AvgPool2d", "avgpooling2d", True, "Average pooling over H and W.")


class AdaptiveAvgPool2d(Module):
    def __init__(self, output_size):
        super().__init__()
        self.output_size = tuple(int(v) for v in _pair(output_size))

    def forward(self, x):
        return autograd.adaptive_avgpooling2d(x).forward(x, self.output_size)


class MultiHeadAttention(Module):
    """Attention over (B, S, D) with ``n_heads`` heads of D / n_heads: per head
    softmax(Q K^T / sqrt(d_head) + mask) V, dropout on the probabilities,
    bias-free projections ``q``, ``k``, ``v``, ``out``."""

    # longest sequence whose causal path (triangle-skipping products and
    # row kernels) is used
    CAUSAL_MAX_SEQ = 16384

    def __init__(self, d_model, n_heads, dropout=0.0):
        super().__init__()
        if d_model % n_heads:  # an assertion in the reference: same exception type
            raise AssertionError(f"d_model {d_model} is not a multiple of n_heads {n_heads}")
        self.d_model = d_model
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads
        for name in ("q", "k", "v", "out"):
            setattr(self, name, Linear(d_model, d_model, bias=False))
        self.drop = Dropout(dropout)

    def _split(self, t, b, seq):
        """(B, S, D) -> (B heads, S, d_head)."""
        t = t.reshape((b, seq, self.n_heads, self.head_dim)).permute(0, 2, 1, 3)
        return t.reshape((b * self.n_heads, seq, self.head_dim))

    def _merge(self, t, b, seq):
        """(B heads, S, d_head) -> (B, S, D)."""
        t = t.reshape((b, self.n_heads, seq, self.head_dim)).permute(0, 2, 1, 3)
        return t.reshape((b, seq, self.d_model))

    def _probabilities(self, q, k, mask, seq):
        scale = 1.0 / math.sqrt(self.head_dim)
        # GPT-2's marked causal mask (-1e9 above the diagonal): the scores there
        # get probability exactly 0 and gradient exactly 0, so the products and
        # the softmax skip that triangle with unchanged results; without
        # attention dropout nothing downstream reads it, so it is not written.
        causal = (mask is not None and getattr(mask, "_causal", False)
                  and tuple(mask.shape) == (seq, seq) and seq <= self.CAUSAL_MAX_SEQ)
        if causal:
            unwritten = self.drop.p == 0
            tag = "_skip" if unwritten else ""
            scores = autograd.matmul(q, k).forward(q, k, transpose_b=True, causal="scores" + tag)
            probs = autograd.scaled_masked_softmax(scores).forward(
                scores, scale, mask, causal=2 if unwritten else 1)
            return probs, "probs" + tag
        scores = autograd.matmul(q, k).forward(q, k, transpose_b=True)
        if mask is None or (len(mask.shape) == 2 and not mask.requires_grad):
            # scale, mask add and softmax in one pass (the three ops' roundings)
            return autograd.scaled_masked_softmax(scores).forward(scores, scale, mask), None
        return ((scores * scale) + mask).softmax(dim=-1), None

    def _fused_mode(self, x, mask, seq):
        """None, or whether the fused kernels run causal: GPT-2's marked causal
        mask or no mask, over head sizes the kernels are built for."""
        if not functional.attention_ops.supported(x, self.n_heads):
            return None
        if mask is None:
            return False
        if getattr(mask, "_causal", False) and tuple(mask.shape) == (seq, seq):
            return True
        return None

    def forward(self, x, mask=None):
        b, seq, _ = x.shape
        causal = self._fused_mode(x, mask, seq)
        if causal is not None:
            # the whole score / softmax / dropout / value path in two kernels
            # (forward, backward) on the projections' own layout
            q, k, v = self.q(x), self.k(x), self.v(x)
            p = self.drop.p if context.MODE == 0 else None
            ctx = autograd.FusedAttention(q, k, v).forward(q, k, v, self.n_heads, causal, p)
            return self.out(ctx)
        q, k, v = (self._split(proj(x), b, seq) for proj in (self.q, self.k, self.v))
        probs, causal = self._probabilities(q, k, mask, seq)
        probs = self.drop(probs)
        ctx = autograd.matmul(probs, v).forward(probs, v, causal=causal)
        return self.out(self._merge(ctx, b, seq))


class Attention(Module):
    """MultiHeadAttention under the name ``mha``, one head by default."""

    def __init__(self, d_model, n_heads=1):
        super().__init__()
        self.mha = MultiHeadAttention(d_model, n_heads)

    def forward(self, x, mask=None):
        return self.mha(x, mask)


class GELU(Module):
    def forward(self, x):
        return x.gelu()


class Sine(Module):
    """sin(omega x), the Hyena filter network's activation."""

    def __init__(self, omega=10.0):
        super().__init__()
        self.omega = float(omega)

    def forward(self, x):
        return (x * self.omega).sin()

    def extra_repr(self):
        return f"omega={self.omega}"


class SwiGLU(Module):
    """w3(silu(w1 x) * w2 x), bias-free; hidden width int(2 mlp_ratio d / 3)
    unless given."""

    def __init__(self, d_model, hidden_dim=None, mlp_ratio=4):
        super().__init__()
        self.hidden_dim = int(2 * (mlp_ratio * d_model) / 3) if hidden_dim is None else hidden_dim
        self.w1 = Linear(d_model, self.hidden_dim, bias=False)
        self.w2 = Linear(d_model, self.hidden_dim, bias=False)
        self.w3 = Linear(self.hidden_dim, d_model, bias=False)

    def forward(self, x):
        d, hid = self.w1.weight.shape
        rows = math.prod(x.shape[:-1])
        if (context.MODE == 0 and hid % 128 and d % 128 == 0 and rows % 128 == 0
                and self.w1.bias is None and self.w2.bias is None and self.w3.bias is None):
            # the hidden width padded to a multiple of 128 inside one op, so
            # every product takes the direct-to-LDS tiles (Hyena's 682)
            hp = (hid + 127) // 128 * 128
            w1, w2, w3 = self.w1.weight, self.w2.weight, self.w3.weight
            return autograd.swiglu_padded(x, w1, w2, w3).forward(x, w1, w2, w3, hp)
        gate = self.w1(x).silu()
        return self.w3(gate * self.w2(x))


class TiedLinear(Module):
    """x E^T against an Embedding's table E, which stays registered only
    under the embedding."""

    def __init__(self, embedding):
        super().__init__()
        object.__setattr__(self, "_embedding", embedding)

    def forward(self, x):
        table = self._embedding.weight
        return autograd.matmul(x, table).forward(x, table, False, True)


class PositionalEncoding(Module):
    """(L, 2 features + 1) table [t, cos(2 pi k t), sin(2 pi k t)] for t on
    linspace(0, 1, L) and k < features, computed in float32 and cached on the
    device per length."""

    def __init__(self, features=8):
        super().__init__()
        features = int(features)
        if features < 1:
            raise ValueError(f"positional features must be >= 1, got {features}")
        self.features = features
        self.out_features = 2 * features + 1
        self._cache = {}

    def _table(self, length):
        # the reference's float32 arithmetic, operation for operation
        # (module.py:576-584): t k first, then times 2 pi
        t = np.linspace(0.0, 1.0, int(length), dtype=np.float32)
        phase = (2.0 * np.pi) * np.outer(t, np.arange(self.features, dtype=np.float32))
        return np.hstack([t[:, None], np.cos(phase), np.sin(phase)]).astype(np.float32)

    def forward(self, length):
        key = (int(length), self.features)
        if key not in self._cache:
            self._cache[key] = Tensor((key[0], self.out_features),
                                      data=self._table(length).tobytes())
        return self._cache[key]

    def extra_repr(self):
        return f"features={self.features}, out_features={self.out_features}"
