"""Index expressions to strided views (the indexing contract of reference
src/wxx/Tensor.py:120-260).

A tensor is (buffer, offset, shape, stride) in elements, so a basic index
(ints and slices) is pure arithmetic on that triple: each axis either keeps
a range of positions (a slice: the view starts ``start * stride`` further on
and steps ``step * stride``) or pins one position (an int: the axis
disappears).  This module does that arithmetic without touching the device.

Contract details kept from the reference:
* a non-tuple index is a 1-tuple; the first ``...`` stands for as many full
  slices as the other entries leave axes (more entries than axes is an
  ``IndexError``); missing trailing entries are full slices;
* a list or ndarray entry makes the whole index "advanced": the entries are
  uploaded as tensors (as the reference does, through ``from_numpy``) and the
  selection is gathered on the host;
* ints are bounds-checked (negative ones count from the end) with an
  ``IndexError``; any other entry type is an ``IndexError``.
"""

import numpy as np


def _is_int(v):
    return isinstance(v, int) and not isinstance(v, bool)


def expand(index, rank, upload):
    """``(entries, advanced)`` of an index expression for a tensor of
    ``rank``; ``upload`` turns a list / ndarray entry into a device tensor."""
    entries = index if isinstance(index, tuple) else (index,)
    for pos, e in enumerate(entries):
        if e is Ellipsis:
            fill = rank - (len(entries) - 1)
            if fill < 0:
                raise IndexError("too many indices for tensor")
            entries = entries[:pos] + (slice(None),) * fill + entries[pos + 1:]
            break
    entries = tuple(upload(np.asarray(e)) if isinstance(e, (list, np.ndarray)) else e
                    for e in entries)
    advanced = any(hasattr(e, "buffer") for e in entries)
    if not advanced:
        if len(entries) > rank:
            raise IndexError("too many indices for tensor")
        entries = entries + (slice(None),) * (rank - len(entries))
    return entries, advanced


def basic(shape, stride, offset, entries):
    """(offset, shape, stride) of the view that ints and slices select."""
    out_shape, out_stride = [], []
    for axis, (size, step, e) in enumerate(zip(shape, stride, entries)):
        if isinstance(e, slice):
            positions = range(*e.indices(size))
            offset += positions.start * step
            out_shape.append(len(positions))
            out_stride.append(positions.step * step)
        elif _is_int(e):
            at = e + size if e < 0 else e
            if at < 0 or at >= size:
                raise IndexError(f"index {e} out of bounds for axis {axis} with size {size}")
            offset += at * step
        else:
            raise IndexError(f"unsupported index type {type(e).__name__}")
    return offset, out_shape, out_stride


def gather(host, entries):
    """The advanced selection on the host copy ``host`` of the tensor.  A
    leading Python / numpy bool selects through a flat mask; otherwise every
    entry (device tensors read back as int64 positions) indexes numpy-style."""
    head = entries[0]
    if isinstance(head, (bool, np.bool_)):
        return host.reshape(-1)[np.flatnonzero(np.asarray(head))]
    key = tuple(e.numpy().astype(np.int64) if hasattr(e, "numpy") else e for e in entries)
    return host[key]


def narrow(shape, stride, offset, dim, start, length):
    """(offset, shape) of positions [start, start + length) along ``dim``."""
    for name, v in (("start", start), ("length", length)):
        if not _is_int(v):
            raise TypeError(f"{name} must be an int, got {type(v).__name__}")
    if start < 0 or length < 0 or start + length > shape[dim]:
        raise IndexError(f"narrow bounds out of range: start={start}, length={length}, "
                         f"dim {dim} has size {shape[dim]}")
    new_shape = list(shape)
    new_shape[dim] = length
    return offset + start * stride[dim], new_shape
