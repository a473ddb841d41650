"""Host-side helpers shared by the ops: broadcasting, reduction views and the
broadcast adjoint (reference src/wxx/backend/dispatch.py:17-246).

Only metadata is computed here; launch geometry lives in the kernels
themselves (each entry point sizes its own grid), so there is no
``_dispatch_1d`` / ``_dispatch_tiled_rows`` counterpart.
"""

from .. import validation

WORKGROUP_SIZE = 256


def broadcast_shapes(shape_a, shape_b):
    """NumPy broadcasting of two shapes -> (out_shape, padded_a, padded_b)."""
    shape_a = validation.normalize_shape(shape_a, name="shape_a")
    shape_b = validation.normalize_shape(shape_b, name="shape_b")
    rank = max(len(shape_a), len(shape_b))
    validation.check_rank(shape_a, max_rank=validation.MAX_RANK, name="shape_a")
    validation.check_rank(shape_b, max_rank=validation.MAX_RANK, name="shape_b")
    pa = (1,) * (rank - len(shape_a)) + shape_a
    pb = (1,) * (rank - len(shape_b)) + shape_b
    out = []
    for a, b in zip(pa, pb):
        if a == b or b == 1:
            out.append(a)
        elif a == 1:
            out.append(b)
        else:
            raise ValueError(f"cannot broadcast shapes {tuple(shape_a)} and {tuple(shape_b)}")
    return tuple(out), pa, pb


def compute_broadcast_strides(padded_shape, out_shape):
    """Row-major strides of a dense ``padded_shape`` read over ``out_shape`` (0 = broadcast)."""
    if len(padded_shape) != len(out_shape):
        raise ValueError(
            f"padded shape {tuple(padded_shape)} and output shape {tuple(out_shape)} "
            "must have the same rank"
        )
    strides = [0] * len(out_shape)
    acc = 1
    for i in range(len(out_shape) - 1, -1, -1):
        strides[i] = 0 if padded_shape[i] == 1 else acc
        acc *= padded_shape[i]
    return tuple(strides)


def view_broadcast_strides(tensor, out_shape):
    """Strides mapping ``out_shape`` onto a (possibly strided) view of ``tensor``."""
    validation.check_broadcastable(tensor.shape, out_shape, name="pointwise operand")
    rank = len(out_shape)
    pad = rank - len(tensor.shape)
    strides = [0] * rank
    for i in range(rank):
        src = i - pad
        strides[i] = 0 if src < 0 or tensor.shape[src] == 1 else tensor.stride[src]
    return tuple(strides)


def supports_strided(tensor):
    """True when the strided kernels can address ``tensor`` directly."""
    return len(tensor.shape) <= validation.MAX_RANK and all(s >= 0 for s in tensor.stride)


def _get_reduce_dims(shape, axis=None):
    """Map a reduction axis (or contiguous range of axes) onto (outer, reduce, inner)."""
    shape = validation.normalize_shape(shape, name="reduction input")
    ndim = len(shape)
    if not ndim:
        raise ValueError("cannot reduce a 0-d tensor")
    if axis is None:
        return 1, validation.numel(shape), 1, (1,)
    axes = tuple(sorted(validation.normalize_dims(axis, ndim, name="axis", allow_duplicates=False)))
    if not axes:
        raise ValueError("axis must contain at least one dimension")
    if any(axes[i] != axes[i - 1] + 1 for i in range(1, len(axes))):
        raise ValueError(
            f"non-contiguous multi-axis reduction {axes} on shape {shape} "
            "requires permuting the tensor first"
        )
    first, last = axes[0], axes[-1]
    outer = validation.numel(shape[:first]) if first > 0 else 1
    reduce = validation.numel(shape[first:last + 1])
    inner = validation.numel(shape[last + 1:]) if last < ndim - 1 else 1
    out_shape = tuple(s for d, s in enumerate(shape) if d not in axes) or (1,)
    return outer, reduce, inner, out_shape


def keepdims_shape(shape, axis):
    """Output shape of a reduction with ``keepdims=True``."""
    if axis is None:
        return (1,) * len(shape)
    reduced = set(validation.normalize_dims(axis, len(shape)))
    return tuple(1 if d in reduced else s for d, s in enumerate(shape))


def _sum_to_shape(gradient, target_shape):
    """Sum ``gradient`` down to ``target_shape`` (adjoint of broadcasting)."""
    from .. import functional

    target_shape = validation.normalize_shape(target_shape, name="target_shape")
    if len(gradient.shape) < len(target_shape):
        raise ValueError(
            f"cannot reduce gradient {tuple(gradient.shape)} to {target_shape}: "
            "target has higher rank"
        )
    validation.check_broadcastable(target_shape, gradient.shape, name="target_shape")
    lead = len(gradient.shape) - len(target_shape)
    if lead > 0:
        # Leading broadcast dims are contiguous: one reduction over all of them.
        gradient = functional.sum(gradient, axis=tuple(range(lead)))
    for axis, size in enumerate(target_shape):
        if size == 1 and gradient.shape[axis] != 1:
            gradient = functional.sum(gradient, axis=axis, keepdims=True)
    if tuple(gradient.shape) != target_shape:
        gradient = functional.reshape(gradient, target_shape)
    return gradient


def _expand_grad_output(tensor1, shape, axis, keepdims=False):
    """Re-insert reduced dimensions (size 1) so a gradient broadcasts back to ``shape``."""
    ndim = len(shape)
    if keepdims:
        return tensor1
    if axis is None:
        return tensor1.reshape((1,) * ndim)
    reduced = set(validation.normalize_dims(axis, ndim, name="axis", allow_duplicates=False))
    expanded = []
    j = 0
    gshape = tensor1.shape
    for i in range(ndim):
        if i in reduced:
            expanded.append(1)
        elif j < len(gshape):
            expanded.append(gshape[j])
            j += 1
        else:
            expanded.append(1)
    return tensor1.reshape(tuple(expanded))
