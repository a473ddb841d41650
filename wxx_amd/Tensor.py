"""Dense tensors backed by HIP device memory.

Same contract as the reference's WebGPU tensor (reference
src/wxx/Tensor.py:28-872): ``shape`` is a list, ``stride`` a tuple in
elements, ``offset`` an element offset into ``buffer``, ``type`` one of
``"f32"``, ``"u32"``, ``"c64"`` (interleaved real/imag float32 pairs, strides
counted in complex elements).  Views share the parent's buffer and keep it
alive through ``_base``.  Arithmetic and unary methods dispatch to
``wxx_amd.autograd`` which records the graph and calls ``wxx_amd.functional``.

Storage differs from the reference only in mechanism: ``buffer`` is a
:class:`~wxx_amd.backend.device.DeviceBuffer` (``.size`` in bytes, like a
wgpu buffer), value fills run as a device kernel instead of uploading a
host array, and ``numpy()`` copies back only the span the view covers.
"""

import ctypes as C
import numbers

import numpy as np

from . import _views, validation
from .backend import lib as _lib
from .backend.device import get_buffer_pool, get_cmd_buffer

buffer_pool = get_buffer_pool()
cmd_buf = get_cmd_buffer()

_DTYPES = ("f32", "u32", "c64")
_NP = {"f32": np.float32, "u32": np.uint32, "c64": np.complex64}


def _f32_bits(value):
    return int(np.array([value], dtype=np.float32).view(np.uint32)[0])


class Tensor:
    """N-dimensional tensor backed by a device buffer."""

    def __init__(
        self,
        shape,
        buffer=None,
        data=None,
        value=1.0,
        offset=0,
        stride=None,
        requires_grad=False,
        dtype=None,
    ):
        shape = validation.normalize_shape(shape)
        if not isinstance(offset, int) or isinstance(offset, bool) or offset < 0:
            raise ValueError(f"offset must be a non-negative int, got {offset!r}")
        if dtype is not None and dtype not in _DTYPES:
            raise ValueError(f"unsupported dtype {dtype!r}; expected one of {_DTYPES}")

        self.shape = list(shape)
        self.offset = offset
        self._base = None
        self.type = dtype if dtype is not None else "f32"
        if stride is None:
            self.stride = validation.contiguous_strides(self.shape)
        else:
            stride = tuple(stride)
            if len(stride) != len(self.shape):
                raise ValueError(
                    f"stride {stride} must have one entry per shape dimension "
                    f"{tuple(self.shape)}"
                )
            self.stride = stride
        self.nbytes = validation.numel(self.shape) * self.itemsize()
        self.data = None

        if buffer is not None:
            self.buffer = buffer
        elif data is not None:
            self.buffer = buffer_pool.create_buffer_with_data(data=bytes(data), label="Tensor")
        else:
            n = validation.numel(self.shape)
            self.buffer = buffer_pool.create_buffer(self.nbytes, label="Tensor")
            if self.type == "c64":
                bits, words = 0, 2 * n
            elif self.type == "u32":
                bits, words = int(value) & 0xFFFFFFFF, n
            else:
                bits, words = _f32_bits(value), n
            if words:
                _lib.call("wxx_fill_u32", C.c_void_p(self.buffer.ptr), words, bits)
        self.requires_grad = requires_grad
        self.creator = None
        self.grad = None

    @classmethod
    def _wrap(cls, shape, buffer, dtype="f32", requires_grad=False):
        """A contiguous tensor over ``buffer`` for an op's output, skipping the
        argument validation of ``__init__`` (``shape`` is a list of ints the
        op has already checked); the same attributes as ``__init__``."""
        t = cls.__new__(cls)
        t.shape = shape
        t.offset = 0
        t._base = None
        t.type = dtype
        t.stride = validation.contiguous_strides(shape)
        t.nbytes = validation.numel(shape) * (8 if dtype == "c64" else 4)
        t.data = None
        t.buffer = buffer
        t.requires_grad = requires_grad
        t.creator = None
        t.grad = None
        return t

    # ------------------------------------------------------------------
    # Layout
    # ------------------------------------------------------------------
    def itemsize(self):
        """Bytes per logical element (complex64 holds two float32s)."""
        return 8 if self.type == "c64" else 4

    def calc_contiguous_strides(self):
        return validation.contiguous_strides(self.shape)

    def is_contiguous(self):
        """Row-major and starting at element 0 of the buffer (like the reference)."""
        if self.offset != 0:
            return False
        return validation.is_contiguous_layout(self.shape, self.stride)

    def data_ptr(self):
        """Device address of element ``offset`` (for the C ABI)."""
        return self.buffer.ptr + self.offset * self.itemsize()

    # ------------------------------------------------------------------
    # Indexing
    # ------------------------------------------------------------------
    def __getitem__(self, index):
        """A view for ints / slices / ``...`` (through autograd while
        recording), a gathered copy for list / array / tensor entries."""
        from .functional.utils import from_numpy

        entries, advanced = _views.expand(index, len(self.shape), from_numpy)
        if advanced:
            return self._advanced_getitem(entries)
        from .backend import context

        if self.requires_grad and context.MODE == 0:
            from . import autograd

            return autograd.getitem(self).forward(self, entries)
        return self._basic_getitem(entries)

    def _view(self, offset, shape, stride):
        out = Tensor(shape=shape, buffer=self.buffer, stride=stride, offset=offset,
                     requires_grad=self.requires_grad, dtype=self.type)
        out._base = self
        return out

    def _basic_getitem(self, index):
        """Zero-copy view selected by ints and slices (one entry per axis)."""
        return self._view(*_views.basic(self.shape, self.stride, self.offset, index))

    def _advanced_getitem(self, index):
        """Gather by integer / mask entries through a host copy (as the
        reference does); a new tensor of this one's dtype."""
        from .functional.utils import from_numpy

        picked = _views.gather(self.numpy(), index)
        if self.type == "c64":
            from .functional.fft import from_numpy_complex

            out = from_numpy_complex(picked)
        else:
            out = from_numpy(picked, dtype=np.uint32) if self.type == "u32" else from_numpy(picked)
        out.requires_grad = self.requires_grad
        return out

    def __setitem__(self, index, value):
        from . import functional

        functional.assign(self[index], value)

    # ------------------------------------------------------------------
    # Views
    # ------------------------------------------------------------------
    def narrow(self, dim, start, length):
        dim = validation.normalize_dim(dim, len(self.shape))
        offset, shape = _views.narrow(self.shape, self.stride, self.offset, dim, start, length)
        return self._view(offset, shape, self.stride)

    def slice(self, dim, start, length):
        from . import autograd

        return autograd.narrow(self).forward(self, dim, start, length)

    def unfold(self, dimension, size, step=1):
        from . import autograd

        return autograd.unfold(self).forward(self, dimension, size, step)

    def diagonal(self, offset=0, dim1=0, dim2=1):
        from . import autograd

        return autograd.diagonal(self).forward(self, offset, dim1, dim2)

    def chunk(self, chunks, dim=0):
        dim = validation.normalize_dim(dim, len(self.shape), name="dim")
        if not isinstance(chunks, int) or isinstance(chunks, bool) or chunks < 1:
            raise ValueError(f"chunks must be a positive int, got {chunks!r}")
        size = self.shape[dim]
        if size % chunks:
            raise ValueError(
                f"cannot split dimension {dim} of size {size} into {chunks} equal chunks"
            )
        step = size // chunks
        from . import autograd

        return tuple(autograd.narrow(self).forward(self, dim, i * step, step) for i in range(chunks))

    def reshape(self, *shape):
        shape = tuple(shape[0]) if len(shape) == 1 and isinstance(shape[0], (tuple, list)) else shape
        from . import autograd

        return autograd.reshape(self).forward(self, tuple(shape))

    def view(self, *shape):
        return self.reshape(*shape)

    def permute(self, *axis):
        from . import autograd

        return autograd.permute(self).forward(self, axis)

    def transpose(self, dim0, dim1):
        rank = len(self.shape)
        dim0 = validation.normalize_dim(dim0, rank, name="dim0")
        dim1 = validation.normalize_dim(dim1, rank, name="dim1")
        axis = list(range(rank))
        axis[dim0], axis[dim1] = axis[dim1], axis[dim0]
        from . import autograd

        return autograd.permute(self).forward(self, axis)

    def t(self):
        if len(self.shape) < 2:
            raise IndexError("t() expects a tensor with at least 2 dimensions")
        return self.transpose(-1, -2)

    def contiguous(self):
        from . import functional

        return functional.contiguous(self)

    def unsqueeze(self, dim):
        from . import autograd

        return autograd.unsqueeze(self).forward(self, dim)

    def squeeze(self, dim=None):
        from . import autograd

        return autograd.squeeze(self).forward(self, dim)

    def flatten(self, start_dim=0, end_dim=-1):
        from . import autograd

        return autograd.flatten(self).forward(self, start_dim, end_dim)

    # ------------------------------------------------------------------
    # Autograd
    # ------------------------------------------------------------------
    def detach(self):
        if self.buffer is None:
            raise RuntimeError("cannot detach a tensor whose buffer was released")
        out = Tensor(
            shape=self.shape,
            buffer=self.buffer,
            stride=self.stride,
            offset=self.offset,
            dtype=self.type,
        )
        out._base = self
        return out

    def detach_(self):
        self.requires_grad = False
        self.creator = None
        self.grad = None
        return self

    def backward(self):
        """Reverse-mode sweep over the recorded graph (reference Tensor.py:430-517)."""
        from .autograd.engine import run_backward

        run_backward(self)

    # ------------------------------------------------------------------
    # Host access
    # ------------------------------------------------------------------
    def numpy(self):
        """Copy this view to a NumPy array (synchronises the device stream)."""
        dtype = _NP.get(self.type)
        if dtype is None:
            raise TypeError(f"unsupported tensor type {self.type!r}")
        n = validation.numel(self.shape)
        if n == 0:
            return np.zeros(tuple(self.shape), dtype=dtype)
        if any(s < 0 for s in self.stride):
            raise ValueError("negative strides are not supported by numpy()")
        span = 1 + sum((d - 1) * s for d, s in zip(self.shape, self.stride))
        host = np.empty(span, dtype=dtype)
        _lib.call(
            "wxx_d2h",
            host.ctypes.data_as(C.c_void_p),
            C.c_void_p(self.data_ptr()),
            span * self.itemsize(),
        )
        if self.is_contiguous() or validation.is_contiguous_layout(self.shape, self.stride):
            return host[:n].reshape(tuple(self.shape)).copy()
        view = np.lib.stride_tricks.as_strided(
            host,
            shape=tuple(self.shape),
            strides=tuple(s * host.itemsize for s in self.stride),
        )
        return view.copy()

    def read_buffer(self):
        """Read the whole backing buffer into ``self.data`` (bytes)."""
        size = self.buffer.size
        host = np.empty(size, dtype=np.uint8)
        _lib.call("wxx_d2h", host.ctypes.data_as(C.c_void_p), C.c_void_p(self.buffer.ptr), size)
        self.data = host.tobytes()

    def __repr__(self):
        array_str = np.array2string(self.numpy(), prefix="tensor(", precision=4, suppress_small=True)
        return f"tensor({array_str}, shape={self.shape}), require grad={self.requires_grad}"

    def item(self):
        if validation.numel(self.shape) != 1:
            raise RuntimeError("cannot convert a tensor with more than one element to a scalar")
        return self.numpy().item()

    def destroy(self):
        """Release the buffer now (views defer to their base)."""
        if getattr(self, "buffer", None) is not None and self._base is None:
            buf = self.buffer
            self.buffer = None
            cmd_buf.defer_destroy(buf)

    # ------------------------------------------------------------------
    # Arithmetic
    # ------------------------------------------------------------------
    def __add__(self, other):
        from . import autograd

        if not isinstance(other, Tensor):
            return autograd.addscaler(self).forward(self, float(other))
        return autograd.add(self, other).forward(self, other)

    def __radd__(self, other):
        return self.__add__(other)

    def __sub__(self, other):
        from . import autograd

        if not isinstance(other, Tensor):
            return autograd.subscaler(self).forward(self, float(other))
        return autograd.sub(self, other).forward(self, other)

    def __neg__(self):
        from . import autograd

        return autograd.negate(self).forward(self)

    def __mul__(self, other):
        from . import autograd

        if not isinstance(other, Tensor):
            return autograd.mulscaler(self).forward(self, float(other))
        return autograd.mul(self, other).forward(self, other)

    def __rmul__(self, other):
        return self.__mul__(other)

    def __truediv__(self, other):
        from . import autograd

        if not isinstance(other, Tensor):
            return autograd.mulscaler(self).forward(self, 1.0 / float(other))
        return autograd.div(self, other).forward(self, other)

    def __rtruediv__(self, other):
        from . import autograd

        if not isinstance(other, numbers.Real):
            return NotImplemented
        return autograd.rdivscaler(self).forward(self, float(other))

    def __matmul__(self, other):
        from . import autograd

        return autograd.matmul(self, other).forward(self, other)

    def matmul(self, other):
        return self.__matmul__(other)

    def __pow__(self, other):
        from . import autograd

        if isinstance(other, numbers.Real) and other == 2:
            return autograd.square(self).forward(self)
        if isinstance(other, numbers.Real):
            return autograd.powscaler(self).forward(self, float(other))
        raise TypeError(f"tensor exponents are not supported, got {type(other).__name__}")

    def __rpow__(self, other):
        from . import autograd

        if not isinstance(other, numbers.Real):
            return NotImplemented
        base = float(other)
        if base <= 0.0:
            raise ValueError(f"a tensor exponent requires a positive base, got {base}")
        return autograd.rpowscaler(self).forward(self, base)

    def pow(self, exponent):
        return self.__pow__(exponent)

    def __eq__(self, other):
        from . import functional

        return functional.equal(self, other)

    __hash__ = object.__hash__

    def matmul_add(self, other, bias):
        from . import autograd

        return autograd.matmuladd(self, other, bias).forward(self, other, bias)

    # ------------------------------------------------------------------
    # Unary / reduction methods
    # ------------------------------------------------------------------
    def _unary(self, name):
        from . import autograd

        return getattr(autograd, name)(self).forward(self)

    def relu(self):
        return self._unary("relu")

    def gelu(self):
        return self._unary("gelu")

    def sin(self):
        return self._unary("sin")

    def cos(self):
        return self._unary("cos")

    def sigmoid(self):
        return self._unary("sigmoid")

    def silu(self):
        return self._unary("sigmoid") * self

    def selu(self):
        return self._unary("selu")

    def softmax(self, dim=-1):
        from . import autograd

        return autograd.softmax(self).forward(self, dim)

    def square(self):
        return self._unary("square")

    def exp(self):
        return self._unary("exp")

    def sqrt(self):
        return self._unary("sqrt")

    def rsqrt(self):
        return self._unary("rsqrt")

    def log(self):
        return self._unary("log")

    def abs(self):
        return self._unary("abs")

    def sign(self):
        return self._unary("sign")

    def clamp(self, min=np.finfo(np.float32).min, max=np.finfo(np.float32).max):
        from . import autograd

        return autograd.clamp(self).forward(self, min, max)

    def _reduce(self, name, axis, keepdims, keepdim):
        from . import autograd

        if keepdim is not None:
            keepdims = keepdim
        return getattr(autograd, name)(self).forward(self, axis, keepdims)

    def sum(self, axis=None, keepdims=False, *, keepdim=None):
        return self._reduce("sum", axis, keepdims, keepdim)

    def mean(self, axis=None, keepdims=False, *, keepdim=None):
        return self._reduce("mean", axis, keepdims, keepdim)

    def var(self, axis=None, keepdims=False, *, keepdim=None):
        return self._reduce("var", axis, keepdims, keepdim)

    def std(self, axis=None, keepdims=False, *, keepdim=None):
        return self._reduce("std", axis, keepdims, keepdim)

    def max(self, dim=None, keepdims=False, *, keepdim=None):
        return self._reduce("max", dim, keepdims, keepdim)

    def min(self, dim=None, keepdims=False, *, keepdim=None):
        return self._reduce("min", dim, keepdims, keepdim)

    def argmax(self, dim=None, keepdims=False, *, keepdim=None):
        return self._reduce("argmax", dim, keepdims, keepdim)

    def argmin(self, dim=None, keepdims=False, *, keepdim=None):
        return self._reduce("argmin", dim, keepdims, keepdim)

    # ------------------------------------------------------------------
    # FFT / complex
    # ------------------------------------------------------------------
    def rfft(self, n=None):
        from . import autograd

        return autograd.rfft(self).forward(self, n)

    def irfft(self, n=None, length=None):
        from . import autograd

        return autograd.irfft(self).forward(self, n, length)

    def complex_mul(self, other):
        from . import autograd

        return autograd.complex_mul(self, other).forward(self, other)

    def conj(self):
        from . import autograd

        return autograd.complex_conj(self).forward(self)


class Parameter(Tensor):
    """A tensor registered as a learnable parameter (shares the tensor's buffer)."""

    def __init__(self, tensor, requires_grad=True):
        super().__init__(
            shape=tensor.shape,
            buffer=tensor.buffer,
            offset=tensor.offset,
            stride=tensor.stride,
            requires_grad=requires_grad,
            dtype=tensor.type,
        )
        self._base = tensor
        self.Tensor = tensor
