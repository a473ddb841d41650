"""Small helpers shared by the functional modules (output allocation, raw
device pointers, f32 bit patterns)."""

import ctypes as C

import numpy as np

from .. import validation
from ..backend import lib as _lib
from ..backend.device import get_buffer_pool
from ..Tensor import Tensor

buffer_pool = get_buffer_pool()
call = _lib.call


def empty(shape, dtype="f32", requires_grad=False, label=None):
    """A new uninitialised tensor of ``shape`` (device memory from the cache)."""
    shape = [int(s) for s in shape]
    if dtype not in ("f32", "u32", "c64") or any(s < 0 for s in shape):
        return Tensor(shape, None, requires_grad=requires_grad, dtype=dtype)  # raises
    item = 8 if dtype == "c64" else 4
    buf = buffer_pool.create_buffer(validation.numel(shape) * item, label=label or "op output")
    return Tensor._wrap(shape, buf, dtype, requires_grad)


def ptr(t):
    """Device address of ``t``'s first element as a ctypes pointer."""
    return C.c_void_p(t.data_ptr())


def f32_bits(value):
    return int(np.array([value], dtype=np.float32).view(np.uint32)[0])


def i64_array(values):
    arr = (C.c_int64 * max(1, len(values)))()
    for i, v in enumerate(values):
        arr[i] = int(v)
    return arr


def contiguous_f32(t, name="tensor"):
    if t.type != "f32":
        raise TypeError(f"{name} expects an f32 tensor, got {t.type!r}")
    return t if t.is_contiguous() else t.contiguous()


__all__ = ["empty", "ptr", "f32_bits", "i64_array", "contiguous_f32", "call", "Tensor"]
