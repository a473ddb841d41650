"""Host-side argument checks on tensor metadata (reference src/wxx/validation.py).

Everything here looks at shapes, strides and offsets only: no device memory
is read and nothing is enqueued, so a bad argument is reported before any
kernel runs.  The error contract is the reference's: ``TypeError`` when a
value has the wrong kind, ``ValueError`` when it has a bad value, and
``IndexError`` when a dimension index is out of range.  The module imports
nothing from the package, so ``Tensor`` and the backend can both use it.
"""

import math

MAX_RANK = 6
"""Highest rank the strided kernels take (their shape / stride arrays hold six)."""


def numel(shape):
    """Number of elements of ``shape``; a 0-d shape holds one."""
    return math.prod(shape)


def _as_int(value):
    """``value`` if it is an int (bools are not), else None."""
    return value if isinstance(value, int) and not isinstance(value, bool) else None


def _as_tuple(seq, name):
    """``seq`` as a tuple; a lone int becomes a 1-tuple."""
    if _as_int(seq) is not None:
        return (seq,)
    try:
        return tuple(seq)
    except TypeError:
        raise TypeError(f"{name} must be an int or an iterable of ints, "
                        f"got {type(seq).__name__}") from None


def normalize_shape(shape, *, name="shape", allow_infer=False):
    """``shape`` as a tuple of non-negative ints; with ``allow_infer`` one
    entry may be -1 (resolved by :func:`infer_shape`)."""
    dims = _as_tuple(shape, name)
    wildcards = 0
    for pos, size in enumerate(dims):
        if _as_int(size) is None:
            raise TypeError(f"{name}[{pos}] must be an int, got {type(size).__name__}")
        if size >= 0:
            continue
        if size == -1 and allow_infer and wildcards == 0:
            wildcards = 1
            continue
        if size == -1 and allow_infer:
            raise ValueError(f"{name} may contain at most one -1, got {dims}")
        raise ValueError(f"{name}[{pos}] must be non-negative, got {size}")
    return dims


def infer_shape(shape, total, *, name="shape"):
    """Fill in a -1 entry of ``shape`` from ``total`` and require the
    result to hold exactly ``total`` elements."""
    dims = normalize_shape(shape, name=name, allow_infer=True)
    if -1 in dims:
        at = dims.index(-1)
        rest = numel(dims[:at] + dims[at + 1:])
        if rest == 0 or total % rest:
            raise ValueError(f"cannot infer {name} {dims} for {total} elements")
        dims = dims[:at] + (total // rest,) + dims[at + 1:]
    count = numel(dims)
    if count != total:
        raise ValueError(f"{name} {dims} describes {count} elements, expected {total}")
    return dims


def normalize_dim(dim, rank, *, name="dim"):
    """A dimension index (negative counts from the end) as one in [0, rank)."""
    if _as_int(dim) is None:
        raise TypeError(f"{name} must be an int, got {type(dim).__name__}")
    if rank == 0:
        raise IndexError(f"{name}={dim} is invalid for a 0-d tensor")
    pos = dim % rank if -rank <= dim < rank else None
    if pos is None:
        raise IndexError(f"{name}={dim} is out of range for a tensor of rank {rank}")
    return pos


def normalize_dims(dims, rank, *, name="dims", allow_duplicates=True):
    """Each entry of an int or iterable of dimension indices, normalised."""
    picked = tuple(normalize_dim(d, rank, name=f"{name}[{i}]")
                   for i, d in enumerate(_as_tuple(dims, name)))
    if not allow_duplicates and len(set(picked)) < len(picked):
        raise ValueError(f"{name} contains duplicate dimensions: {picked}")
    return picked


def check_rank(shape, *, min_rank=0, max_rank=MAX_RANK, name="tensor"):
    """The rank of ``shape``, which must lie in [min_rank, max_rank]
    (``max_rank`` None: no upper bound)."""
    rank = len(shape)
    high = math.inf if max_rank is None else max_rank
    if min_rank <= rank <= high:
        return rank
    if max_rank is None:
        allowed = f"at least {min_rank}"
    elif min_rank == max_rank:
        allowed = f"{min_rank}"
    else:
        allowed = f"{min_rank}..{max_rank}"
    raise ValueError(f"{name} must have rank {allowed}, got {rank}")


def check_same_shape(*shapes, name="tensors"):
    """The shape every argument shares; ``ValueError`` on the first mismatch."""
    if len(shapes) == 0:
        raise ValueError(f"{name} must contain at least one shape")
    ref = tuple(shapes[0])
    mismatch = next((i for i, s in enumerate(shapes) if tuple(s) != ref), None)
    if mismatch is not None:
        raise ValueError(f"{name} must have the same shape, got {ref} and "
                         f"{tuple(shapes[mismatch])} (at index {mismatch})")
    return ref


def check_broadcastable(shape, out_shape, *, name="tensor"):
    """``out_shape`` if ``shape`` broadcasts to it (numpy rules), else ``ValueError``."""
    lead = len(out_shape) - len(shape)
    fits = lead >= 0 and all(d in (1, out_shape[lead + i]) for i, d in enumerate(shape))
    if not fits:
        raise ValueError(f"{name} of shape {tuple(shape)} cannot broadcast to {tuple(out_shape)}")
    return tuple(out_shape)


def contiguous_strides(shape):
    """Row-major element strides of ``shape``."""
    rank = len(shape)
    if rank == 1:
        return (1,)
    if rank == 2:
        return (shape[1], 1)
    out = [1] * rank
    step = 1
    for d in range(rank - 1, 0, -1):
        step *= shape[d]
        out[d - 1] = step
    return tuple(out)


def is_contiguous_layout(shape, stride):
    """Whether ``stride`` lays ``shape`` out row-major and dense (the stride
    of a dimension of size 0 or 1 does not matter)."""
    want = 1
    for d in range(len(shape) - 1, -1, -1):
        size = shape[d]
        if size > 1 and stride[d] != want:
            return False
        want *= size
    return True


def check_contiguous(tensor, *, name="tensor"):
    if tensor.is_contiguous():
        return tensor
    raise ValueError(f"{name} must be contiguous, got shape={tuple(tensor.shape)} "
                     f"stride={tuple(tensor.stride)} offset={tensor.offset}")


def check_no_negative_stride(tensor, *, name="tensor"):
    if min(tensor.stride, default=0) >= 0:
        return tensor
    raise ValueError(f"{name} has a negative stride {tuple(tensor.stride)}; "
                     "call .contiguous() first")


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
