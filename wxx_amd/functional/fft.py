"""Real FFT and complex-valued ops (reference src/wxx/functional/fft.py:1-658).

Complex tensors have ``type == "c64"``: interleaved (real, imag) float32
pairs whose logical shape omits the pair, strides counted in complex
elements.  ``rfft``/``irfft`` run as one kernel launch each (the whole
transform of a row stays in LDS) instead of the reference's
``log2(n) + 2`` launches for n > 1024.
"""

import ctypes as C

import numpy as np

from .. import validation
from ..backend.dispatch import broadcast_shapes
from ._common import buffer_pool, call, empty, i64_array, ptr
from ..Tensor import Tensor

MAX_RANK = validation.MAX_RANK


def _check_pow2(n):
    if n < 1 or (n & (n - 1)) != 0:
        raise ValueError(f"FFT length must be a positive power of two, got {n}")


def _require_c64(t, name):
    if t.type != "c64":
        raise TypeError(f"{name} expects complex64 tensors")


def from_numpy_complex(array):
    """Upload a numpy array as a c64 tensor (real arrays get a zero imaginary part)."""
    array = np.asarray(array)
    array = np.ascontiguousarray(array.astype(np.complex64))
    buf = buffer_pool.create_buffer_with_data(array.view(np.float32), label="from_numpy_complex")
    return Tensor(list(array.shape), buf, dtype="c64")


def complex_weights(weights):
    """Real weights as a 1-D complex tensor (imaginary part 0)."""
    return from_numpy_complex(np.asarray(weights, dtype=np.float32).astype(np.complex64))


def _broadcast_strides(tensor, out_shape):
    rank = len(out_shape)
    pad = rank - len(tensor.shape)
    if pad < 0:
        raise ValueError(f"cannot broadcast shape {tuple(tensor.shape)} to {tuple(out_shape)}")
    strides = []
    for i in range(rank):
        if i < pad:
            strides.append(0)
            continue
        dim = tensor.shape[i - pad]
        if dim == out_shape[i]:
            strides.append(tensor.stride[i - pad])
        elif dim == 1:
            strides.append(0)
        else:
            raise ValueError(
                f"cannot broadcast shape {tuple(tensor.shape)} to {tuple(out_shape)}"
            )
    return strides


def _complex_binary(out, a, b, out_shape, op, conj_a=False, conj_b=False):
    rank = len(out_shape)
    if rank > MAX_RANK:
        raise ValueError(f"Maximum rank supported by complex kernels is {MAX_RANK}")
    s_out = _broadcast_strides(out, out_shape)
    call(
        "wxx_complex_binary",
        ptr(out),
        ptr(a),
        ptr(b),
        rank,
        i64_array(out_shape),
        i64_array(s_out),
        i64_array(_broadcast_strides(a, out_shape)),
        i64_array(_broadcast_strides(b, out_shape)),
        op,
        1 if conj_a else 0,
        1 if conj_b else 0,
    )


def complex_mul(tensor_a, tensor_b, conj_a=False, conj_b=False):
    """Broadcasting complex product; ``conj_a``/``conj_b`` conjugate an operand
    inside the kernel (reference fft.py:168-213)."""
    _require_c64(tensor_a, "complex_mul")
    _require_c64(tensor_b, "complex_mul")
    out_shape = list(broadcast_shapes(tensor_a.shape, tensor_b.shape)[0])
    out = empty(out_shape, dtype="c64",
                requires_grad=tensor_a.requires_grad or tensor_b.requires_grad)
    _complex_binary(out, tensor_a, tensor_b, out_shape, 0, conj_a, conj_b)
    return out


def complex_add(tensor_a, tensor_b):
    """Out-of-place ``a + b`` for complex tensors (``b`` broadcast to ``a``)."""
    _require_c64(tensor_a, "complex_add")
    _require_c64(tensor_b, "complex_add")
    out_shape = list(tensor_a.shape)
    out = empty(out_shape, dtype="c64")
    _complex_binary(out, tensor_a, tensor_b, out_shape, 1)
    return out


def complex_add_inplace(tensor_a, tensor_b):
    """``tensor_a += tensor_b`` (reference fft.py:216-245)."""
    _require_c64(tensor_a, "complex_add_inplace")
    _require_c64(tensor_b, "complex_add_inplace")
    _complex_binary(tensor_a, tensor_a, tensor_b, list(tensor_a.shape), 1)
    return tensor_a


def complex_conj(tensor1):
    """Conjugate into a new contiguous tensor (reference fft.py:248-292)."""
    _require_c64(tensor1, "complex_conj")
    rank = len(tensor1.shape)
    if rank > MAX_RANK:
        raise ValueError(f"Maximum rank supported by complex kernels is {MAX_RANK}")
    out = empty(tensor1.shape, dtype="c64", requires_grad=tensor1.requires_grad)
    call("wxx_complex_conj", ptr(out), ptr(tensor1), rank, i64_array(tensor1.shape),
         i64_array(out.stride), i64_array(tensor1.stride))
    return out


def complex_contiguous(tensor1):
    """Dense copy of a strided complex view (reference fft.py:295-342)."""
    if tensor1.is_contiguous():
        return tensor1
    _require_c64(tensor1, "complex_contiguous")
    rank = len(tensor1.shape)
    if rank > MAX_RANK:
        raise ValueError(f"Maximum rank supported by complex kernels is {MAX_RANK}")
    out = empty(tensor1.shape, dtype="c64", requires_grad=tensor1.requires_grad)
    call("wxx_copy_strided", ptr(out), ptr(tensor1), 8, rank, i64_array(tensor1.shape),
         i64_array(out.stride), i64_array(tensor1.stride))
    return out


def complex_pad(tensor1, out_len):
    """Zero-pad or truncate the last dimension (reference fft.py:345-383)."""
    _require_c64(tensor1, "complex_pad")
    if not tensor1.is_contiguous():
        tensor1 = complex_contiguous(tensor1)
    out_len = int(out_len)
    if out_len < 0:
        raise ValueError(f"complex_pad length must be >= 0, got {out_len}")
    in_len = tensor1.shape[-1]
    batch = validation.numel(tensor1.shape[:-1])
    out_shape = list(tensor1.shape)
    out_shape[-1] = out_len
    out = empty(out_shape, dtype="c64", requires_grad=tensor1.requires_grad)
    call("wxx_complex_pad", ptr(tensor1), ptr(out), batch, in_len, out_len)
    return out


def rfft(tensor1, n=None):
    """Real FFT along the last dimension (reference fft.py:484-563).

    Returns ``(spectrum, n)``: a c64 tensor of shape ``(..., n // 2 + 1)``;
    each row is zero-padded or truncated to the power of two ``n``
    (default: the input length).
    """
    if tensor1.type == "c64":
        raise TypeError("rfft expects a real-valued tensor")
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    validation.check_rank(tensor1.shape, min_rank=1, name="rfft input")
    shape = list(tensor1.shape)
    in_len = shape[-1]
    n = in_len if n is None else int(n)
    _check_pow2(n)
    rows = validation.numel(shape[:-1])
    out_shape = shape[:-1] + [n // 2 + 1]
    out = empty(out_shape, dtype="c64", requires_grad=tensor1.requires_grad)
    call("wxx_rfft", ptr(tensor1), ptr(out), rows, in_len, n)
    return out, n


def irfft(tensor1, n=None, length=None, scale=1.0):
    """Inverse real FFT along the last dimension (reference fft.py:566-645).

    ``tensor1`` is a one-sided spectrum; bins at or beyond ``n // 2 + 1`` are
    ignored, missing bins count as zero.  Default ``n = 2 * (in_len - 1)``.
    ``length`` (default ``n``) keeps only the first ``length`` samples of each
    row, ``irfft(tensor1, n)[..., :length]`` computed by the same arithmetic
    without the full-length intermediate; ``scale`` multiplies the result
    after the 1/n normalisation, as a separate multiply would.
    """
    if tensor1.type != "c64":
        raise TypeError("irfft expects a complex64 tensor")
    if not tensor1.is_contiguous():
        tensor1 = complex_contiguous(tensor1)
    validation.check_rank(tensor1.shape, min_rank=1, name="irfft input")
    shape = list(tensor1.shape)
    in_len = shape[-1]
    n = 2 * (in_len - 1) if n is None else int(n)
    _check_pow2(n)
    if n < 2:
        raise ValueError("irfft length must be at least 2")
    length = n if length is None else int(length)
    if not 1 <= length <= n:
        raise ValueError(f"irfft length must be in [1, {n}], got {length}")
    rows = validation.numel(shape[:-1])
    out = empty(shape[:-1] + [length], requires_grad=tensor1.requires_grad)
    if length == n and scale == 1.0:
        call("wxx_irfft", ptr(tensor1), ptr(out), rows, in_len, n)
    else:
        call("wxx_irfft_crop", ptr(tensor1), ptr(out), rows, in_len, n, length,
             C.c_float(scale))
    return out


# the fused spectrum products run inside the LDS-resident transforms
FUSED_MAX_N = 32768


def fused_spectrum_supported(n):
    """Whether ``rfft_mul`` / ``irfft_mul`` take transform length ``n``."""
    n = int(n)
    return 2 <= n <= FUSED_MAX_N and (n & (n - 1)) == 0


def _contig_c64(t, name):
    _require_c64(t, name)
    return t if t.is_contiguous() else complex_contiguous(t)


def _bin_weights(bin_weights):
    edge, mid = bin_weights
    return C.c_float(float(edge)), C.c_float(float(mid))


def rfft_mul(tensor1, n, bin_weights):
    """``complex_mul(rfft(tensor1, n)[0], w)`` in one kernel, for the real bin
    weights ``bin_weights = (edge, mid)``: w_k = edge at k = 0 and n/2, mid
    between (the weights of the rfft / irfft adjoints), multiplied as the
    transform stores each bin and rounded as complex_mul rounds with the
    vector (w_k, 0) (the irfft backward's spectrum product, reference
    autograd/utils.py:549-718)."""
    if tensor1.type == "c64":
        raise TypeError("rfft_mul expects a real-valued tensor")
    n = int(n)
    if not fused_spectrum_supported(n):
        raise ValueError(f"rfft_mul needs a power-of-two n in [2, {FUSED_MAX_N}], got {n}")
    edge, mid = _bin_weights(bin_weights)
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    validation.check_rank(tensor1.shape, min_rank=1, name="rfft_mul input")
    shape = list(tensor1.shape)
    rows = validation.numel(shape[:-1])
    out = empty(shape[:-1] + [n // 2 + 1], dtype="c64")
    call("wxx_rfft_mul", ptr(tensor1), ptr(out), rows, shape[-1], n, edge, mid)
    return out


def irfft_mul(tensor1, n, h=None, conj_h=False, bin_weights=None, length=None, scale=1.0):
    """``irfft(tensor1 * h * w, n, length, scale)`` with the products formed
    as the bins load, rounded as complex_mul rounds.  ``h`` (c64, the trailing
    dims of ``tensor1``'s shape) broadcasts over ``tensor1``'s leading dims
    and is conjugated when ``conj_h``; ``bin_weights = (edge, mid)`` are real
    bin weights as in ``rfft_mul`` (the spectrum then needs its n/2 + 1
    bins); either may be None.  The Hyena long convolution's forward product
    and its backward's filter product (reference nn/hyena.py:208-216)."""
    tensor1 = _contig_c64(tensor1, "irfft_mul")
    validation.check_rank(tensor1.shape, min_rank=1, name="irfft_mul input")
    n = int(n)
    if not fused_spectrum_supported(n):
        raise ValueError(f"irfft_mul needs a power-of-two n in [2, {FUSED_MAX_N}], got {n}")
    shape = list(tensor1.shape)
    in_len = shape[-1]
    rows = validation.numel(shape[:-1])
    hrows = 1
    if h is not None:
        h = _contig_c64(h, "irfft_mul")
        hs = list(h.shape)
        if len(hs) == 0 or len(hs) > len(shape) or shape[len(shape) - len(hs):] != hs:
            raise ValueError(f"irfft_mul operand shape {tuple(hs)} is not a trailing part "
                             f"of {tuple(shape)}")
        hrows = validation.numel(hs[:-1])
    weighted = bin_weights is not None
    if weighted and in_len != n // 2 + 1:
        raise ValueError(f"irfft_mul bin weights need the {n // 2 + 1} bins of the spectrum, "
                         f"got {in_len}")
    edge, mid = _bin_weights(bin_weights if weighted else (1.0, 1.0))
    length = n if length is None else int(length)
    if not 1 <= length <= n:
        raise ValueError(f"irfft length must be in [1, {n}], got {length}")
    out = empty(shape[:-1] + [length])
    call("wxx_irfft_mul", ptr(tensor1), ptr(h) if h is not None else None, ptr(out), rows,
         in_len, max(hrows, 1), 1 if conj_h else 0, 1 if weighted else 0, edge, mid, n, length,
         C.c_float(scale))
    return out


def complex_mul_batch_sum(tensor_a, tensor_c, conj_c=False, keep=1):
    """``sum(tensor_a * tensor_c, leading dims)`` in one pass, keeping the
    last ``keep`` dims (``tensor_c`` conjugated when ``conj_c``): the
    broadcast operand's gradient of complex_mul (reference
    autograd/utils.py:549-718), equal bit for bit to complex_mul followed by
    the reduction over the leading dims."""
    tensor_a = _contig_c64(tensor_a, "complex_mul_batch_sum")
    tensor_c = _contig_c64(tensor_c, "complex_mul_batch_sum")
    if tuple(tensor_a.shape) != tuple(tensor_c.shape):
        raise ValueError(f"complex_mul_batch_sum shapes differ: {tuple(tensor_a.shape)} "
                         f"and {tuple(tensor_c.shape)}")
    shape = list(tensor_a.shape)
    if not 1 <= keep < len(shape):
        raise ValueError(f"complex_mul_batch_sum keeps {keep} of {len(shape)} dims")
    out_shape = shape[len(shape) - keep:]
    n = validation.numel(out_shape)
    batch = validation.numel(shape[:len(shape) - keep])
    if batch == 0:
        raise ValueError("complex_mul_batch_sum needs a non-empty batch")
    out = empty(out_shape, dtype="c64")
    call("wxx_complex_mul_batch_sum", ptr(out), ptr(tensor_a), ptr(tensor_c), batch, n,
         1 if conj_c else 0)
    return out


__all__ = [
    "rfft_mul",
    "irfft_mul",
    "complex_mul_batch_sum",
    "fused_spectrum_supported",
    "rfft",
    "irfft",
    "complex_mul",
    "complex_add",
    "complex_add_inplace",
    "complex_conj",
    "complex_contiguous",
    "complex_pad",
    "complex_weights",
    "from_numpy_complex",
]
