"""Cross-entropy loss (reference src/wxx/functional/loss.py:20-101)."""

import ctypes as C

import numpy as np

from .. import graphs, validation
from ..backend import lib as _lib
from ._common import call, empty, ptr

_bad_flag = {"buf": None}


def _flag():
    """The 4-byte device word for the out-of-range-target flag: a persistent
    one, or inside a step graph recording one per call (checked after every
    replay)."""
    from ..backend.device import get_buffer_pool

    if graphs.capturing():
        return get_buffer_pool().create_buffer(4, label="cceloss flag (graph)")
    if _bad_flag["buf"] is None:
        _bad_flag["buf"] = get_buffer_pool().create_buffer(4, label="cceloss flag")
    return _bad_flag["buf"]


def _raise_if_flagged(flag, targets, K):
    bad = np.zeros(1, np.int32)
    _lib.call("wxx_d2h", bad.ctypes.data_as(C.c_void_p), C.c_void_p(flag.ptr), 4)
    if bad[0]:
        tmax = int(targets.numpy().max())
        raise ValueError(f"cceloss targets must be in [0, {K}), got max target {tmax}")


def _check_targets(flag, targets, K):
    """Raise now (eager), or after every replay of the step graph being
    recorded, when a target was out of range."""
    if graphs.capturing():
        graphs.keep_alive(flag, targets)
        graphs.after_replay(lambda: _raise_if_flagged(flag, targets, K))
    else:
        _raise_if_flagged(flag, targets, K)


def cceloss(tensor1, tensor2):
    """Softmax cross-entropy of ``(B, K)`` logits against ``(B,)`` u32 targets.

    Returns ``(loss (B, 1), dlogits (B, K))``.  A target ``>= K`` raises
    ``ValueError`` like the reference; the check runs on the device and costs
    one 4-byte readback instead of reading back every target.
    """
    validation.check_rank(tensor1.shape, min_rank=2, max_rank=2, name="logits")
    validation.check_rank(tensor2.shape, min_rank=1, max_rank=1, name="targets")
    if tensor1.type != "f32":
        raise TypeError(f"cceloss expects f32 logits, got {tensor1.type!r}")
    if tensor2.type != "u32":
        raise TypeError(f"cceloss expects u32 targets, got {tensor2.type!r}")
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if not tensor2.is_contiguous():
        tensor2 = tensor2.contiguous()
    B, K = tensor1.shape
    if tensor2.shape[0] != B:
        raise ValueError(
            f"cceloss expects one target per row, got {tensor2.shape[0]} targets for {B} rows"
        )
    if B < 1 or K < 1:
        raise ValueError(f"cceloss expects non-empty logits, got {(B, K)}")
    flag = _flag()
    call("wxx_fill_u32", C.c_void_p(flag.ptr), 1, 0)
    loss = empty((B, 1), requires_grad=tensor1.requires_grad)
    grad = empty(tensor1.shape)
    call("wxx_cceloss", ptr(tensor1), ptr(tensor2), ptr(loss), ptr(grad), B, K,
         C.c_void_p(flag.ptr))
    _check_targets(flag, tensor2, K)
    return loss, grad


def cceloss_stats(tensor1, tensor2):
    """Forward half of :func:`cceloss` for the autograd path: ``(loss (B, 1),
    stats (B, 2))`` with each row's max and exp-sum; the logits gradient is
    produced later by :func:`cceloss_grad` (same values as cceloss's dlogits
    times the upstream gradient).  None when the rows are too long for it."""
    if (len(tensor1.shape) != 2 or len(tensor2.shape) != 1 or tensor1.type != "f32"
            or tensor2.type != "u32" or min(tensor1.shape) < 1 or tensor1.shape[1] > 65536):
        return None  # cceloss itself validates (and raises) or handles the long rows
    B, K = tensor1.shape
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if not tensor2.is_contiguous():
        tensor2 = tensor2.contiguous()
    if tensor2.shape[0] != B:
        raise ValueError(
            f"cceloss expects one target per row, got {tensor2.shape[0]} targets for {B} rows"
        )
    flag = _flag()
    call("wxx_fill_u32", C.c_void_p(flag.ptr), 1, 0)
    loss = empty((B, 1), requires_grad=tensor1.requires_grad)
    stats = empty((B, 2))
    call("wxx_cceloss_stats", ptr(tensor1), ptr(tensor2), ptr(loss), ptr(stats), B, K,
         C.c_void_p(flag.ptr))
    _check_targets(flag, tensor2, K)
    return loss, stats, tensor1, tensor2


def cceloss_grad(logits, targets, stats, grad):
    """``(softmax(logits) - onehot(targets)) * grad[row]`` from :func:`cceloss_stats`."""
    B, K = logits.shape
    if len(grad.shape) == 0 or grad.shape[0] != B or validation.numel(grad.shape) != B:
        raise ValueError(f"cceloss gradient of shape {grad.shape} for {B} rows")
    out = empty(logits.shape)
    call("wxx_cceloss_backward", ptr(logits), ptr(targets), ptr(stats), ptr(grad),
         grad.stride[0], ptr(out), B, K)
    return out
