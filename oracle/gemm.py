"""Batched matmul with bias modes, restated from the reference (test
infrastructure only).

``matmul_add`` follows the shape/batch/bias rules of reference
src/wxx/functional/utils.py:378-499 (batch dims must match or one side is
unbatched; bias (N,), (M, N) or batch + (M, N)) and evaluates in float64.
``matmul_add_fma`` calls the exact-order fp32 C restatement
(oracle/csrc/gemm_ref.c) of matmul.wgsl's per-element fma chain; it needs
``oracle/lib/liboracle.so`` (``python oracle/build.py``).
"""

import ctypes as C
import os

import numpy as np

_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "liboracle.so")
_lib = None


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            from . import build

            build.build(verbose=False)
        lib = C.CDLL(_LIB)
        lib.oracle_gemm_fma.restype = None
        lib.oracle_gemm_fma.argtypes = [C.c_void_p] * 4 + [C.c_int64] * 6 + [C.c_int] * 3 + [
            C.c_int64
        ] * 2
        _lib = lib
    return _lib


def _dims(a_shape, b_shape, transpose_A, transpose_B):
    M, K = (a_shape[-1], a_shape[-2]) if transpose_A else (a_shape[-2], a_shape[-1])
    KB, N = (b_shape[-1], b_shape[-2]) if transpose_B else (b_shape[-2], b_shape[-1])
    if K != KB:
        raise ValueError(f"Inner dimension mismatch: {K} vs {KB}")
    ba, bb = tuple(a_shape[:-2]), tuple(b_shape[:-2])
    if ba and bb and ba != bb:
        raise ValueError(f"Batch dimensions must match or be unbatched: {ba} vs {bb}")
    return M, N, K, ba or bb, bool(ba), bool(bb)


def bias_mode(bias_shape, out_batch, M, N):
    if bias_shape is None:
        return 0
    bias_shape = tuple(bias_shape)
    if bias_shape == (N,):
        return 1
    if bias_shape == (M, N):
        return 2
    if bias_shape == tuple(out_batch) + (M, N):
        return 3
    raise ValueError(f"Bias shape {bias_shape} is not broadcastable")


def matmul_add(A, B, bias=None, transpose_A=False, transpose_B=False, rounded=True):
    """C = op(A) op(B) + bias in float64; ``rounded`` returns it rounded to
    float32, else the float64 values themselves."""
    A = np.asarray(A, np.float32)
    B = np.asarray(B, np.float32)
    M, N, K, out_batch, _, _ = _dims(A.shape, B.shape, transpose_A, transpose_B)
    mode = bias_mode(None if bias is None else np.shape(bias), out_batch, M, N)
    a = A.astype(np.float64)
    b = B.astype(np.float64)
    if transpose_A:
        a = np.swapaxes(a, -1, -2)
    if transpose_B:
        b = np.swapaxes(b, -1, -2)
    c = np.matmul(a, b)
    if mode:
        c = c + np.asarray(bias, np.float64)
    c = c.reshape(tuple(out_batch) + (M, N))
    return c.astype(np.float32) if rounded else c


def matmul_add_fma(A, B, bias=None, transpose_A=False, transpose_B=False, rows=None):
    """Exact-order fp32 reference result; ``rows=(r0, r1)`` computes a row sample."""
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    M, N, K, out_batch, has_a, has_b = _dims(A.shape, B.shape, transpose_A, transpose_B)
    mode = bias_mode(None if bias is None else np.shape(bias), out_batch, M, N)
    batch = int(np.prod(out_batch)) if out_batch else 1
    out = np.zeros(tuple(out_batch) + (M, N), np.float32)
    bias_arr = np.ascontiguousarray(bias, np.float32) if mode else np.zeros(1, np.float32)
    r0, r1 = rows if rows is not None else (0, M)
    _load().oracle_gemm_fma(
        A.ctypes.data, B.ctypes.data, bias_arr.ctypes.data, out.ctypes.data,
        M, N, K, batch, M * K if has_a else 0, K * N if has_b else 0,
        mode, int(bool(transpose_A)), int(bool(transpose_B)), r0, r1,
    )
    return out
