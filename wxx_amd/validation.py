"""Host-side shape, dimension and layout checks shared by the ops.

These inspect metadata only (shape, stride, offset) and never touch device
memory, mirroring the contract of the reference's validators
(reference src/wxx/validation.py:1-208): the same checks raise the same
exception types (``TypeError`` for wrong kinds, ``ValueError`` for bad
values, ``IndexError`` for out-of-range dimensions) before any kernel is
enqueued.
"""

import math

MAX_RANK = 6
"""Highest rank the strided kernels address (shape/stride arrays of six)."""


def numel(shape):
    """Element count of ``shape`` (1 for a 0-d shape)."""
    return int(math.prod(shape)) if len(shape) else 1


def _is_int(v):
    return isinstance(v, int) and not isinstance(v, bool)


def normalize_shape(shape, *, name="shape", allow_infer=False):
    """Return ``shape`` as a tuple of non-negative ints (one ``-1`` if allowed)."""
    if _is_int(shape):
        shape = (shape,)
    try:
        dims = tuple(shape)
    except TypeError:
        raise TypeError(
            f"{name} must be an int or an iterable of ints, got {type(shape).__name__}"
        ) from None
    n_infer = 0
    for pos, d in enumerate(dims):
        if not _is_int(d):
            raise TypeError(f"{name}[{pos}] must be an int, got {type(d).__name__}")
        if d == -1 and allow_infer:
            n_infer += 1
            if n_infer > 1:
                raise ValueError(f"{name} may contain at most one -1, got {dims}")
        elif d < 0:
            raise ValueError(f"{name}[{pos}] must be non-negative, got {d}")
    return dims


def infer_shape(shape, total, *, name="shape"):
    """Resolve a ``-1`` entry and check that ``shape`` holds ``total`` elements."""
    dims = normalize_shape(shape, name=name, allow_infer=True)
    if -1 in dims:
        at = dims.index(-1)
        known = 1
        for pos, d in enumerate(dims):
            if pos != at:
                known *= d
        if known == 0 or total % known:
            raise ValueError(f"cannot infer {name} {dims} for {total} elements")
        dims = dims[:at] + (total // known,) + dims[at + 1:]
    if numel(dims) != total:
        raise ValueError(f"{name} {dims} describes {numel(dims)} elements, expected {total}")
    return dims


def normalize_dim(dim, rank, *, name="dim"):
    """Map a possibly negative dimension index into ``[0, rank)``."""
    if not _is_int(dim):
        raise TypeError(f"{name} must be an int, got {type(dim).__name__}")
    if rank == 0:
        raise IndexError(f"{name}={dim} is invalid for a 0-d tensor")
    d = dim + rank if dim < 0 else dim
    if not 0 <= d < rank:
        raise IndexError(f"{name}={dim} is out of range for a tensor of rank {rank}")
    return d


def normalize_dims(dims, rank, *, name="dims", allow_duplicates=True):
    """Normalise an int or an iterable of dimension indices into a tuple."""
    if _is_int(dims):
        dims = (dims,)
    try:
        items = tuple(dims)
    except TypeError:
        raise TypeError(
            f"{name} must be an int or an iterable of ints, got {type(dims).__name__}"
        ) from None
    out = tuple(normalize_dim(d, rank, name=f"{name}[{i}]") for i, d in enumerate(items))
    if not allow_duplicates and len(set(out)) != len(out):
        raise ValueError(f"{name} contains duplicate dimensions: {out}")
    return out


def check_rank(shape, *, min_rank=0, max_rank=MAX_RANK, name="tensor"):
    """Raise ``ValueError`` unless ``min_rank <= len(shape) <= max_rank``."""
    rank = len(shape)
    if rank < min_rank or (max_rank is not None and rank > max_rank):
        if max_rank is None:
            want = f"at least {min_rank}"
        elif min_rank == max_rank:
            want = str(min_rank)
        else:
            want = f"{min_rank}..{max_rank}"
        raise ValueError(f"{name} must have rank {want}, got {rank}")
    return rank


def check_same_shape(*shapes, name="tensors"):
    """Require identical shapes; return the common shape."""
    if not shapes:
        raise ValueError(f"{name} must contain at least one shape")
    first = tuple(shapes[0])
    for i, s in enumerate(shapes[1:], 1):
        if tuple(s) != first:
            raise ValueError(
                f"{name} must have the same shape, got {first} and {tuple(s)} (at index {i})"
            )
    return first


def check_broadcastable(shape, out_shape, *, name="tensor"):
    """Raise unless ``shape`` broadcasts to ``out_shape``."""
    if len(shape) > len(out_shape):
        raise ValueError(f"{name} of shape {tuple(shape)} cannot broadcast to {tuple(out_shape)}")
    pad = len(out_shape) - len(shape)
    for i, d in enumerate(shape):
        if d != out_shape[i + pad] and d != 1:
            raise ValueError(
                f"{name} of shape {tuple(shape)} cannot broadcast to {tuple(out_shape)}"
            )
    return tuple(out_shape)


def contiguous_strides(shape):
    """Row-major strides (in elements) for ``shape``."""
    strides = [1] * len(shape)
    for i in range(len(shape) - 2, -1, -1):
        strides[i] = strides[i + 1] * shape[i + 1]
    return tuple(strides)


def is_contiguous_layout(shape, stride):
    """True when ``stride`` is row-major for ``shape`` (size-1 dims may have any stride)."""
    expect = 1
    for size, step in zip(reversed(shape), reversed(stride)):
        if size > 1 and step != expect:
            return False
        expect *= size
    return True


def check_contiguous(tensor, *, name="tensor"):
    if not tensor.is_contiguous():
        raise ValueError(
            f"{name} must be contiguous, got shape={tuple(tensor.shape)} "
            f"stride={tuple(tensor.stride)} offset={tensor.offset}"
        )
    return tensor


def check_no_negative_stride(tensor, *, name="tensor"):
    if any(s < 0 for s in tensor.stride):
        raise ValueError(
            f"{name} has a negative stride {tuple(tensor.stride)}; call .contiguous() first"
        )
    return tensor


__all__ = [
    "MAX_RANK",
    "numel",
    "normalize_shape",
    "infer_shape",
    "normalize_dim",
    "normalize_dims",
    "check_rank",
    "check_same_shape",
    "check_broadcastable",
    "contiguous_strides",
    "is_contiguous_layout",
    "check_contiguous",
    "check_no_negative_stride",
]
