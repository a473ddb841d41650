"""Tensor utilities: assignment, views, contiguous copies, the batched GEMM
entry, comparisons, constructors and init helpers.

Signatures and validation follow reference src/wxx/functional/utils.py
(assign :29-101, permute :104-129, diagonal :132-185, unfold :188-236,
unfolddx :239-287, reshape :290-313, contiguous :316-369, matmul_add
:378-499, equal/equal_number :502-556, masked_fill :558-597, constructors
:600-696, init helpers :703-741, scatter_zeros :760-827); every kernel is a
call into libwxx_hip.so.
"""

import math

import numpy as np

from .. import validation
from ..backend.device import get_buffer_pool
from ..Tensor import Tensor
from ._common import call, empty, f32_bits, i64_array, ptr

buffer_pool = get_buffer_pool()


def assign(tensor1, val):
    """Copy ``val`` into the (possibly strided) view ``tensor1``, or fill it with a scalar."""
    rank = validation.check_rank(tensor1.shape, name="assign target")
    shape = i64_array(tensor1.shape)
    dst_strides = i64_array(tensor1.stride)
    if isinstance(val, (float, int)) and not isinstance(val, bool):
        if tensor1.type == "u32":
            bits = int(val) & 0xFFFFFFFF
        else:
            bits = f32_bits(float(val))
        if tensor1.type == "c64":
            # A complex scalar fill writes (val, 0) pairs: go through a c64 source.
            from .fft import from_numpy_complex

            src = from_numpy_complex(np.full(tensor1.shape, complex(val), dtype=np.complex64))
            return assign(tensor1, src)
        call("wxx_fill_strided", ptr(tensor1), rank, shape, dst_strides, bits)
        return tensor1
    if not isinstance(val, Tensor):
        raise TypeError(f"assign expects a Tensor or a scalar, got {type(val).__name__}")
    if tuple(val.shape) != tuple(tensor1.shape):
        raise ValueError(
            f"assign shape mismatch: target {tuple(tensor1.shape)} vs source {tuple(val.shape)}"
        )
    if val.type != tensor1.type:
        raise TypeError(f"assign dtype mismatch: target {tensor1.type!r} vs source {val.type!r}")
    call(
        "wxx_copy_strided",
        ptr(tensor1),
        ptr(val),
        tensor1.itemsize(),
        rank,
        shape,
        dst_strides,
        i64_array(val.stride),
    )
    return tensor1


def permute(tensor1, *axes):
    """View with dimensions reordered by ``axes``."""
    if len(axes) == 1 and isinstance(axes[0], (tuple, list)):
        axes = tuple(axes[0])
    rank = len(tensor1.shape)
    if len(axes) != rank:
        raise ValueError(
            f"permute expects {rank} axes for shape {tuple(tensor1.shape)}, got {len(axes)}"
        )
    axes = validation.normalize_dims(axes, rank, name="axes", allow_duplicates=False)
    out = Tensor(
        shape=tuple(tensor1.shape[i] for i in axes),
        buffer=tensor1.buffer,
        stride=tuple(tensor1.stride[i] for i in axes),
        offset=tensor1.offset,
        requires_grad=tensor1.requires_grad,
        dtype=tensor1.type,
    )
    out._base = tensor1
    return out


def diagonal(tensor1, offset=0, dim1=0, dim2=1):
    """View of the diagonal of the (dim1, dim2) plane, as ``torch.diagonal``."""
    rank = len(tensor1.shape)
    if rank < 2:
        raise ValueError(f"diagonal expects at least 2 dimensions, got shape {tuple(tensor1.shape)}")
    if not isinstance(offset, int) or isinstance(offset, bool):
        raise TypeError(f"offset must be an int, got {type(offset).__name__}")
    dim1 = validation.normalize_dim(dim1, rank, name="dim1")
    dim2 = validation.normalize_dim(dim2, rank, name="dim2")
    if dim1 == dim2:
        raise ValueError(f"dim1 and dim2 must differ, got {dim1} and {dim2}")
    rows, cols = tensor1.shape[dim1], tensor1.shape[dim2]
    if offset >= 0:
        r0, c0 = 0, offset
        length = min(rows, cols - offset)
    else:
        r0, c0 = -offset, 0
        length = min(rows + offset, cols)
    if length <= 0:
        r0 = c0 = length = 0
    shape = [s for a, s in enumerate(tensor1.shape) if a not in (dim1, dim2)] + [length]
    stride = [s for a, s in enumerate(tensor1.stride) if a not in (dim1, dim2)]
    stride.append(tensor1.stride[dim1] + tensor1.stride[dim2])
    out = Tensor(
        shape=tuple(shape),
        buffer=tensor1.buffer,
        stride=tuple(stride),
        offset=tensor1.offset + r0 * tensor1.stride[dim1] + c0 * tensor1.stride[dim2],
        requires_grad=tensor1.requires_grad,
        dtype=tensor1.type,
    )
    out._base = tensor1
    return out


def unfold(tensor1, dimension, size, step=1):
    """Sliding-window view (``torch.Tensor.unfold``)."""
    rank = len(tensor1.shape)
    dim = validation.normalize_dim(dimension, rank, name="dimension")
    if isinstance(size, bool) or not isinstance(size, int):
        raise TypeError(f"size must be an int, got {type(size).__name__}")
    if isinstance(step, bool) or not isinstance(step, int):
        raise TypeError(f"step must be an int, got {type(step).__name__}")
    if size < 1:
        raise ValueError(f"size must be positive, got {size}")
    if step < 1:
        raise ValueError(f"step must be positive, got {step}")
    if rank + 1 > validation.MAX_RANK:
        raise ValueError(
            f"unfold would produce rank {rank + 1}, but the maximum supported rank is "
            f"{validation.MAX_RANK}"
        )
    length = tensor1.shape[dim]
    if size > length:
        raise ValueError(f"size {size} is larger than dimension {dim} of size {length}")
    windows = (length - size) // step + 1
    shape = list(tensor1.shape)
    shape[dim] = windows
    shape.append(size)
    stride = list(tensor1.stride)
    stride[dim] *= step
    stride.append(tensor1.stride[dim])
    out = Tensor(
        shape=tuple(shape),
        buffer=tensor1.buffer,
        stride=tuple(stride),
        offset=tensor1.offset,
        requires_grad=tensor1.requires_grad,
        dtype=tensor1.type,
    )
    out._base = tensor1
    return out


def unfolddx(grad, input_shape, dimension, size, step=1):
    """Backward of :func:`unfold`: gather-sum of overlapping windows."""
    dim = validation.normalize_dim(dimension, len(input_shape), name="dimension")
    if grad.type != "f32":
        raise TypeError(f"unfold expects f32 grad, got {grad.type!r}")
    if not grad.is_contiguous():
        grad = grad.contiguous()
    prefix = math.prod(input_shape[:dim]) if dim else 1
    suffix = math.prod(input_shape[dim + 1:]) if dim + 1 < len(input_shape) else 1
    length = input_shape[dim]
    windows = (length - size) // step + 1
    expect = prefix * windows * suffix * size
    if validation.numel(grad.shape) != expect:
        raise ValueError(
            f"unfold grad has {validation.numel(grad.shape)} elements, expected {expect}"
        )
    out = empty(tuple(input_shape))
    call("wxx_unfolddx", ptr(grad), ptr(out), prefix, length, suffix, windows, size, step)
    return out


def reshape(tensor1, new_shape):
    """Same elements laid out as ``new_shape`` (copies a non-contiguous input)."""
    total = validation.numel(tensor1.shape)
    new_shape = validation.infer_shape(new_shape, total, name="new shape")
    base = tensor1 if tensor1.is_contiguous() else tensor1.contiguous()
    out = Tensor(
        shape=new_shape,
        buffer=base.buffer,
        offset=base.offset,
        requires_grad=tensor1.requires_grad,
        dtype=tensor1.type,
    )
    out._base = base
    return out


def contiguous(tensor1):
    """``tensor1`` itself when contiguous, else a dense copy."""
    if tensor1.is_contiguous():
        return tensor1
    rank = validation.check_rank(tensor1.shape, name="contiguous input")
    out = empty(tensor1.shape, dtype=tensor1.type, requires_grad=tensor1.requires_grad)
    call(
        "wxx_copy_strided",
        ptr(out),
        ptr(tensor1),
        tensor1.itemsize(),
        rank,
        i64_array(tensor1.shape),
        i64_array(out.stride),
        i64_array(tensor1.stride),
    )
    return out


def matmul_add(tensor1, tensor2, tensor3, transpose_A=False, transpose_B=False, tri=0,
               tile=0):
    """Batched ``op(A) @ op(B) (+ bias)`` over the last two dimensions.

    ``tri`` (no bias) marks causal-attention structure whose zero triangle
    the kernel skips, with the same result: 1 the square output is only
    needed on and below the diagonal (zeros above), 2 ``op(A)`` is square
    lower triangular, 3 ``op(A)`` is square upper triangular.  ``tile`` is
    the kernel's tile code (0: its own choice; see ``wxx_matmul_add``).
    """
    validation.check_rank(tensor1.shape, min_rank=2, name="matmul left operand")
    validation.check_rank(tensor2.shape, min_rank=2, name="matmul right operand")
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if not tensor2.is_contiguous():
        tensor2 = tensor2.contiguous()
    if transpose_A:
        M, K = tensor1.shape[-1], tensor1.shape[-2]
    else:
        M, K = tensor1.shape[-2], tensor1.shape[-1]
    if transpose_B:
        K_B, N = tensor2.shape[-1], tensor2.shape[-2]
    else:
        K_B, N = tensor2.shape[-2], tensor2.shape[-1]
    if K != K_B:
        raise ValueError(f"Inner dimension mismatch: {K} vs {K_B}")
    batch_a = list(tensor1.shape[:-2])
    batch_b = list(tensor2.shape[:-2])
    if batch_a and batch_b and batch_a != batch_b:
        raise ValueError(
            f"Batch dimensions must match or be unbatched: {batch_a} vs {batch_b}"
        )
    out_batch = batch_a or batch_b
    batch = int(math.prod(out_batch)) if out_batch else 1
    s_a = M * K if batch_a else 0
    s_b = K * N if batch_b else 0

    bias_mode, s_bias = 0, 0
    bias_ptr = None
    if tensor3 is not None and tensor3.shape is not None:
        if not tensor3.is_contiguous():
            tensor3 = tensor3.contiguous()
        bshape = tuple(tensor3.shape)
        if bshape == (N,):
            bias_mode = 1
        elif bshape == (M, N):
            bias_mode = 2
        elif bshape == tuple(out_batch) + (M, N):
            bias_mode = 3
            s_bias = M * N
        else:
            raise ValueError(
                f"Bias shape {bshape} is not broadcastable to {tuple(out_batch) + (M, N)}"
            )
        bias_ptr = ptr(tensor3)
    out = empty(
        out_batch + [M, N],
        requires_grad=(
            tensor1.requires_grad
            or tensor2.requires_grad
            or (tensor3 is not None and tensor3.requires_grad)
        ),
    )
    if tri:
        if bias_ptr is not None:
            raise ValueError("a triangular product takes no bias")
        call("wxx_matmul_tri", ptr(tensor1), ptr(tensor2), ptr(out), M, N, K, batch, s_a, s_b,
             1 if transpose_A else 0, 1 if transpose_B else 0, int(tri))
        return out
    call(
        "wxx_matmul_add",
        ptr(tensor1),
        ptr(tensor2),
        bias_ptr,
        ptr(out),
        M,
        N,
        K,
        batch,
        s_a,
        s_b,
        s_bias,
        bias_mode,
        1 if transpose_A else 0,
        1 if transpose_B else 0,
        int(tile),
    )
    return out


def _equal_impl(tensor1, tensor2, mode, number=0):
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if tensor2 is not None and not tensor2.is_contiguous():
        tensor2 = tensor2.contiguous()
    n = validation.numel(tensor1.shape)
    out = empty(tensor1.shape, requires_grad=tensor1.requires_grad)
    call(
        "wxx_equal",
        ptr(tensor1),
        ptr(tensor2) if tensor2 is not None else None,
        ptr(out),
        n,
        mode,
        int(number) & 0xFFFFFFFF,
    )
    return out


def equal(tensor1, tensor2):
    """Elementwise equality as f32 1.0 / 0.0."""
    if isinstance(tensor2, (int, float)):
        return equal_number(tensor1, tensor2)
    if tensor1.type not in ("f32", "u32") or tensor1.type != tensor2.type:
        raise TypeError(
            f"equal expects matching f32 or u32 tensors, got {tensor1.type!r} and {tensor2.type!r}"
        )
    if tuple(tensor1.shape) != tuple(tensor2.shape):
        raise ValueError(
            f"equal expects equal shapes, got {tuple(tensor1.shape)} and {tuple(tensor2.shape)}"
        )
    return _equal_impl(tensor1, tensor2, 0 if tensor1.type == "f32" else 1)


def equal_number(tensor1, number):
    """Compare every element with a scalar."""
    if tensor1.type == "f32":
        return _equal_impl(tensor1, None, 2, f32_bits(float(number)))
    if tensor1.type == "u32":
        return _equal_impl(tensor1, None, 3, int(number))
    raise TypeError(f"equal_number expects an f32 or u32 tensor, got {tensor1.type!r}")


def masked_fill(tensor1, number):
    """``x`` where ``x != 0`` else ``number``."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    out = empty(tensor1.shape, requires_grad=tensor1.requires_grad)
    call("wxx_clamp", ptr(tensor1), ptr(out), validation.numel(tensor1.shape), float(number), 0.0, 2)
    return out


def linspace(start, end, steps):
    values = np.linspace(start, end, int(steps), dtype=np.float32)
    return Tensor((int(steps),), data=values.tobytes())


def ones_like(tensor1):
    return Tensor(tensor1.shape, value=1)


def arange(start, shape):
    """Values ``(i % shape[-1]) + start`` over ``shape`` (reference utils.py:612-625)."""
    if isinstance(shape, int):
        shape = (shape,)
    shape = tuple(shape)
    n = math.prod(shape)
    values = (np.arange(n) % shape[-1] + start).astype(np.float32)
    return Tensor(shape, data=values.tobytes())


def normal(mu, sigma, shape):
    rng = np.random.default_rng()
    shape = (shape,) if isinstance(shape, int) else tuple(shape)
    values = rng.normal(mu, sigma, size=math.prod(shape)).astype(np.float32)
    return Tensor(shape, data=values.tobytes())


def uniform(a, b, shape):
    rng = np.random.default_rng()
    shape = (shape,) if isinstance(shape, int) else tuple(shape)
    values = rng.uniform(a, b, size=math.prod(shape)).astype(np.float32)
    return Tensor(shape, data=values.tobytes())


def empty_like_shape(shape, dtype="f32"):
    """A new uninitialised tensor of ``shape`` and ``dtype``."""
    return empty(list(shape), dtype=dtype)


def broadcast_to(tensor1, shape, scale=1.0):
    """Dense ``tensor1 * scale`` broadcast to ``shape`` in one strided kernel
    (the backward of sum / mean)."""
    shape = list(validation.normalize_shape(shape, name="shape"))
    rank = validation.check_rank(shape, name="broadcast_to shape")
    from ..backend.dispatch import view_broadcast_strides

    strides = view_broadcast_strides(tensor1, shape)
    out = empty(shape)
    if validation.numel(shape):
        call("wxx_broadcast_scale", ptr(out), ptr(tensor1), rank, i64_array(shape),
             i64_array(strides), float(scale))
    return out


def from_numpy(array, dtype=np.float32):
    """Upload a NumPy array (float32, or uint32 when ``dtype`` is ``np.uint32``)."""
    if dtype == np.uint32:
        array = np.ascontiguousarray(array, dtype=np.uint32)
        buf = buffer_pool.create_buffer_with_data(array, label="from_numpy")
        return Tensor(list(array.shape), buf, dtype="u32")
    array = np.ascontiguousarray(array, dtype=np.float32)
    buf = buffer_pool.create_buffer_with_data(array, label="from_numpy")
    return Tensor(list(array.shape), buf)


def from_tensor(array, type=np.float32):
    """Upload a torch tensor or NumPy array."""
    if hasattr(array, "detach"):
        array = array.detach().cpu().contiguous().numpy()
    return from_numpy(np.asarray(array), dtype=type)


def concat(tensors, dim):
    from .. import autograd

    return autograd.concat(*tensors).forward(tensors, dim)


def _zero_init(tensor):
    tensor[:] = 0


def _xavier_normal_init(tensor, fan_in, fan_out):
    assign(tensor, normal(0, math.sqrt(2 / (fan_in + fan_out)), tensor.shape))


def _xavier_uniform_init(tensor, fan_in, fan_out):
    a = math.sqrt(6 / (fan_in + fan_out))
    assign(tensor, uniform(-a, a, tensor.shape))


def _kaiming_normal_init(tensor, fan_in):
    assign(tensor, normal(0, math.sqrt(2 / fan_in), tensor.shape))


def _kaiming_uniform_init(tensor, fan_in):
    a = math.sqrt(6 / fan_in)
    assign(tensor, uniform(-a, a, tensor.shape))


def scatter_zeros(grad, out_shape, dim, start):
    """Zeros of ``out_shape`` with ``grad`` placed at ``start`` along ``dim``."""
    out_shape = list(validation.normalize_shape(out_shape, name="out_shape"))
    rank = validation.check_rank(out_shape, name="scatter_zeros output")
    dim = validation.normalize_dim(dim, rank, name="dim")
    length = grad.shape[dim]
    if not 0 <= start <= out_shape[dim] - length:
        raise IndexError(
            f"scatter_zeros bounds out of range: start={start}, length={length}, "
            f"dim {dim} has size {out_shape[dim]}"
        )
    for axis, (actual, expected) in enumerate(zip(grad.shape, out_shape)):
        if axis != dim and actual != expected:
            raise ValueError(
                f"scatter_zeros gradient shape {tuple(grad.shape)} does not fit output shape "
                f"{tuple(out_shape)}"
            )
    if any(s < 0 for s in grad.stride):
        grad = grad.contiguous()
    out = empty(out_shape)
    call(
        "wxx_scatter_zeros",
        ptr(out),
        ptr(grad),
        rank,
        i64_array(out_shape),
        i64_array(grad.stride),
        dim,
        start,
        length,
    )
    return out
