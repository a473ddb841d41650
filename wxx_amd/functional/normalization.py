"""Normalisation: RMSNorm, LayerNorm ("meanvarnorm") and BatchNorm, forward
and backward (reference src/wxx/functional/normalization.py:24-513).

Eps values follow the reference: LayerNorm 1e-5 (normalization.py:94),
RMSNorm 1e-6 (:36), BatchNorm 1e-5 with momentum 0.1 (:157).
"""

from .. import validation
from ..backend import compat
from ..backend.dispatch import _get_reduce_dims
from ._common import call, contiguous_f32, empty, ptr

LN_EPS = 1e-5
RMS_EPS = 1e-6
BN_EPS = 1e-5
BN_MOMENTUM = 0.1


def _check_param(t, n, name):
    """The kernels index per-feature parameters by the reduce coordinate:
    a parameter with fewer than ``n`` elements would be read out of bounds,
    so a size mismatch is rejected before launch."""
    if t.type != "f32":
        raise TypeError(f"{name} must be an f32 tensor, got {t.type!r}")
    if validation.numel(t.shape) != n:
        raise ValueError(
            f"{name} has {validation.numel(t.shape)} elements but the normalised extent is {n}"
        )


def _check_stats(t, n, name):
    if validation.numel(t.shape) != n:
        raise ValueError(f"{name} has {validation.numel(t.shape)} elements, expected {n}")


def rmsnorm(tensor1, gamma, axis=None):
    """``y = x * r * gamma`` with ``r = rsqrt(mean(x^2) + 1e-6)`` (0 for an all-zero slice)."""
    tensor1 = contiguous_f32(tensor1)
    gamma = contiguous_f32(gamma, "gamma")
    outer, red, inner, out_shape = _get_reduce_dims(tensor1.shape, axis)
    _check_param(gamma, red, "gamma")
    y = empty(tensor1.shape)
    irms = empty(out_shape)
    call("wxx_rmsnorm", ptr(tensor1), ptr(gamma), ptr(y), ptr(irms), outer, red, inner,
         RMS_EPS, compat.row_cap())
    return y, irms


def meanvarnorm(tensor1, gamma, beta, axis=None):
    """LayerNorm over ``axis``; returns ``(y, mean, inv_std)``."""
    tensor1 = contiguous_f32(tensor1)
    gamma = contiguous_f32(gamma, "gamma")
    beta = contiguous_f32(beta, "beta")
    outer, red, inner, out_shape = _get_reduce_dims(tensor1.shape, axis)
    _check_param(gamma, red, "gamma")
    _check_param(beta, red, "beta")
    y = empty(tensor1.shape)
    mean = empty(out_shape)
    istd = empty(out_shape)
    call("wxx_meanvarnorm", ptr(tensor1), ptr(gamma), ptr(beta), ptr(y), ptr(mean), ptr(istd),
         outer, red, inner, LN_EPS, compat.row_cap())
    return y, mean, istd


def meanvarnormdx(grad, tensor1, gamma, mean, var, axis=None):
    """LayerNorm input gradient (``var`` is the saved inv_std, as in the reference)."""
    tensor1 = contiguous_f32(tensor1)
    gamma = contiguous_f32(gamma, "gamma")
    grad = contiguous_f32(grad, "grad")
    outer, red, inner, _ = _get_reduce_dims(tensor1.shape, axis)
    _check_param(gamma, red, "gamma")
    validation.check_same_shape(grad.shape, tensor1.shape, name="grad and input")
    _check_stats(mean, outer * inner, "mean")
    _check_stats(var, outer * inner, "inv_std")
    dx = empty(tensor1.shape)
    call("wxx_meanvarnormdx", ptr(grad), ptr(tensor1), ptr(gamma), ptr(mean), ptr(var), ptr(dx),
         outer, red, inner, compat.row_cap())
    return dx


def meanvarnormdg(grad, tensor1, mean, var, axis=None):
    """LayerNorm ``(dgamma, dbeta)``."""
    tensor1 = contiguous_f32(tensor1)
    grad = contiguous_f32(grad, "grad")
    outer, red, inner, _ = _get_reduce_dims(tensor1.shape, axis)
    validation.check_same_shape(grad.shape, tensor1.shape, name="grad and input")
    _check_stats(mean, outer * inner, "mean")
    _check_stats(var, outer * inner, "inv_std")
    dg = empty((red,))
    db = empty((red,))
    call("wxx_meanvarnormdg", ptr(grad), ptr(tensor1), ptr(mean), ptr(var), ptr(dg), ptr(db),
         outer, red, inner)
    return dg, db


def rmsnormdx(grad, tensor1, gamma, irms, axis=None):
    tensor1 = contiguous_f32(tensor1)
    gamma = contiguous_f32(gamma, "gamma")
    grad = contiguous_f32(grad, "grad")
    outer, red, inner, _ = _get_reduce_dims(tensor1.shape, axis)
    _check_param(gamma, red, "gamma")
    validation.check_same_shape(grad.shape, tensor1.shape, name="grad and input")
    _check_stats(irms, outer * inner, "inv_rms")
    dx = empty(tensor1.shape)
    call("wxx_rmsnormdx", ptr(grad), ptr(tensor1), ptr(gamma), ptr(irms), ptr(dx),
         outer, red, inner)
    return dx


def rmsnormdg(grad, tensor1, gamma, irms, axis=None):
    tensor1 = contiguous_f32(tensor1)
    grad = contiguous_f32(grad, "grad")
    outer, red, inner, _ = _get_reduce_dims(tensor1.shape, axis)
    _check_param(gamma, red, "gamma")
    validation.check_same_shape(grad.shape, tensor1.shape, name="grad and input")
    _check_stats(irms, outer * inner, "inv_rms")
    dg = empty(gamma.shape)
    call("wxx_rmsnormdg", ptr(grad), ptr(tensor1), ptr(irms), ptr(dg), outer, red, inner)
    return dg


def batchnorm(tensor1, gamma, beta, running_mean, running_std, training=False):
    """Per-channel BatchNorm over (B, H, W) of an NCHW tensor; returns ``(y, mean, inv_std)``.

    ``running_std`` holds the running *variance* (reference naming).
    """
    tensor1 = contiguous_f32(tensor1)
    gamma = contiguous_f32(gamma, "gamma")
    validation.check_rank(tensor1.shape, min_rank=4, max_rank=4, name="batchnorm input")
    B, Cc, H, W = tensor1.shape
    for t, name in ((gamma, "gamma"), (beta, "beta"), (running_mean, "running_mean"),
                    (running_std, "running_std")):
        _check_param(t, Cc, name)
    y = empty(tensor1.shape)
    mean = empty((Cc,))
    istd = empty((Cc,))
    call("wxx_batchnorm", ptr(tensor1), ptr(gamma), ptr(beta), ptr(running_mean),
         ptr(running_std), ptr(y), ptr(mean), ptr(istd), B, Cc, H * W, BN_EPS, BN_MOMENTUM,
         1 if training else 0)
    return y, mean, istd


def batchnormdx(grad, tensor1, gamma, dgamma, dbeta, saved_mean, saved_std):
    tensor1 = contiguous_f32(tensor1)
    gamma = contiguous_f32(gamma, "gamma")
    grad = contiguous_f32(grad, "grad")
    validation.check_rank(tensor1.shape, min_rank=4, max_rank=4, name="batchnorm input")
    B, Cc, H, W = tensor1.shape
    validation.check_same_shape(grad.shape, tensor1.shape, name="grad and input")
    for t, name in ((gamma, "gamma"), (dgamma, "dgamma"), (dbeta, "dbeta"),
                    (saved_mean, "saved_mean"), (saved_std, "saved_std")):
        _check_param(t, Cc, name)
    dx = empty(tensor1.shape)
    call("wxx_batchnormdx", ptr(grad), ptr(tensor1), ptr(gamma), ptr(dgamma), ptr(dbeta),
         ptr(saved_mean), ptr(saved_std), ptr(dx), B, Cc, H * W)
    return dx


def batchnorm_backward(grad, tensor1, gamma, saved_mean, saved_std):
    """``(dx, dgamma, dbeta)``: :func:`batchnormdg` then :func:`batchnormdx` in one call."""
    tensor1 = contiguous_f32(tensor1)
    gamma = contiguous_f32(gamma, "gamma")
    grad = contiguous_f32(grad, "grad")
    validation.check_rank(tensor1.shape, min_rank=4, max_rank=4, name="batchnorm input")
    B, Cc, H, W = tensor1.shape
    validation.check_same_shape(grad.shape, tensor1.shape, name="grad and input")
    for t, name in ((gamma, "gamma"), (saved_mean, "saved_mean"), (saved_std, "saved_std")):
        _check_param(t, Cc, name)
    dx = empty(tensor1.shape)
    dg = empty((Cc,))
    db = empty((Cc,))
    call("wxx_batchnorm_backward", ptr(grad), ptr(tensor1), ptr(gamma), ptr(saved_mean),
         ptr(saved_std), ptr(dg), ptr(db), ptr(dx), B, Cc, H * W)
    return dx, dg, db


def batchnorm_act_supported(tensor1):
    """Whether :func:`batchnorm_act` takes this NCHW input (non-empty channels,
    32-bit element indices)."""
    if len(tensor1.shape) != 4:
        return False
    B, Cc, H, W = tensor1.shape
    return 0 < B * H * W and B * Cc * H * W < 2**31


def batchnorm_act(tensor1, gamma, beta, residual, running_mean, running_std, updates=1,
                  relu=True):
    """Training-mode :func:`batchnorm`, then ``+ residual`` (``None``: no add) and ReLU
    (``relu``), in one kernel; returns ``(y, mean, inv_std)``.

    The running statistics take ``updates`` (1 or 2) EMA updates, the second one
    being the reference ResNet block's repeated ``bn1`` evaluation
    (src/wxx/nn/resnet.py:33).  Inputs outside :func:`batchnorm_act_supported`
    raise (callers compose batchnorm, add and relu there).
    """
    tensor1 = contiguous_f32(tensor1)
    gamma = contiguous_f32(gamma, "gamma")
    validation.check_rank(tensor1.shape, min_rank=4, max_rank=4, name="batchnorm input")
    B, Cc, H, W = tensor1.shape
    for t, name in ((gamma, "gamma"), (beta, "beta"), (running_mean, "running_mean"),
                    (running_std, "running_std")):
        _check_param(t, Cc, name)
    if residual is not None:
        residual = contiguous_f32(residual, "residual")
        validation.check_same_shape(residual.shape, tensor1.shape, name="residual and input")
    y = empty(tensor1.shape)
    mean = empty((Cc,))
    istd = empty((Cc,))
    call("wxx_batchnorm_act", ptr(tensor1), ptr(gamma), ptr(beta),
         ptr(residual) if residual is not None else None, ptr(running_mean), ptr(running_std),
         ptr(y), ptr(mean), ptr(istd), B, Cc, H * W, BN_EPS, BN_MOMENTUM, int(updates),
         1 if relu else 0)
    return y, mean, istd


def batchnorm_act_backward(grad, tensor1, gamma, beta, residual, saved_mean, saved_std,
                           relu=True):
    """``(dx, dgamma, dbeta, dresidual)`` of :func:`batchnorm_act` (``dresidual`` is
    ``None`` without a residual); relu' is taken from the recomputed pre-activation."""
    tensor1 = contiguous_f32(tensor1)
    gamma = contiguous_f32(gamma, "gamma")
    grad = contiguous_f32(grad, "grad")
    validation.check_rank(tensor1.shape, min_rank=4, max_rank=4, name="batchnorm input")
    B, Cc, H, W = tensor1.shape
    validation.check_same_shape(grad.shape, tensor1.shape, name="grad and input")
    for t, name in ((gamma, "gamma"), (beta, "beta"), (saved_mean, "saved_mean"),
                    (saved_std, "saved_std")):
        _check_param(t, Cc, name)
    dr = None
    if residual is not None:
        residual = contiguous_f32(residual, "residual")
        validation.check_same_shape(residual.shape, tensor1.shape, name="residual and input")
        dr = empty(tensor1.shape)
    dx = empty(tensor1.shape)
    dg = empty((Cc,))
    db = empty((Cc,))
    call("wxx_batchnorm_act_backward", ptr(grad), ptr(tensor1), ptr(gamma), ptr(beta),
         ptr(residual) if residual is not None else None, ptr(saved_mean), ptr(saved_std),
         ptr(dg), ptr(db), ptr(dx), ptr(dr) if dr is not None else None, B, Cc, H * W,
         1 if relu else 0)
    return dx, dg, db, dr


def batchnormdg(grad, tensor1, saved_mean, saved_std):
    tensor1 = contiguous_f32(tensor1)
    grad = contiguous_f32(grad, "grad")
    validation.check_rank(tensor1.shape, min_rank=4, max_rank=4, name="batchnorm input")
    B, Cc, H, W = tensor1.shape
    validation.check_same_shape(grad.shape, tensor1.shape, name="grad and input")
    _check_param(saved_mean, Cc, "saved_mean")
    _check_param(saved_std, Cc, "saved_std")
    dg = empty((Cc,))
    db = empty((Cc,))
    call("wxx_batchnormdg", ptr(grad), ptr(tensor1), ptr(saved_mean), ptr(saved_std), ptr(dg),
         ptr(db), B, Cc, H * W)
    return dg, db
