"""AdamW, dropout and embedding ops (reference src/wxx/functional/layers.py:21-254)."""

import ctypes as C
import math
import random

from .. import graphs, validation
from ._common import Tensor, call, empty, ptr


def adamw(tensor1, grad, exp_avg, exp_avg_sq, step, lr, beta1, beta2, eps, weight_decay, bc1,
          bc2):
    """In-place AdamW update of ``tensor1`` and its two moment buffers."""
    if not tensor1.is_contiguous():
        raise ValueError("adamw updates its parameter in place: it must be contiguous")
    n = validation.numel(tensor1.shape)
    for t, name in ((grad, "grad"), (exp_avg, "exp_avg"), (exp_avg_sq, "exp_avg_sq")):
        if validation.numel(t.shape) != n or not t.is_contiguous():
            raise ValueError(f"adamw {name} must be contiguous with {n} elements")
    call("wxx_adamw", ptr(tensor1), ptr(grad), ptr(exp_avg), ptr(exp_avg_sq), n, float(lr),
         float(beta1), float(beta2), float(eps), float(weight_decay), float(bc1), float(bc2))


def adamw_multi(params, grads, exp_avgs, exp_avg_sqs, lr, beta1, beta2, eps, weight_decay, bc1,
                bc2):
    """AdamW over a whole parameter list in one launch (same per-element math)."""
    count = len(params)
    if not count:
        return
    arrs = [(C.c_void_p * count)() for _ in range(4)]
    sizes = (C.c_int64 * count)()
    for i, group in enumerate(zip(params, grads, exp_avgs, exp_avg_sqs)):
        n = validation.numel(group[0].shape)
        for a, t in zip(arrs, group):
            if validation.numel(t.shape) != n or not t.is_contiguous():
                raise ValueError("adamw_multi expects contiguous tensors of matching size")
            a[i] = t.data_ptr()
        sizes[i] = n
    call("wxx_adamw_multi", *arrs, sizes, count, float(lr), float(beta1), float(beta2),
         float(eps), float(weight_decay), float(bc1), float(bc2))


def _multi_tables(groups, what):
    """ctypes pointer arrays (one per tensor role) and element counts for a
    multi-tensor launch; every group holds contiguous tensors of one size."""
    count = len(groups)
    arrs = [(C.c_void_p * count)() for _ in range(len(groups[0]))]
    sizes = (C.c_int64 * count)()
    for i, group in enumerate(groups):
        n = validation.numel(group[0].shape)
        for a, t in zip(arrs, group):
            if validation.numel(t.shape) != n or not t.is_contiguous() or t.type != "f32":
                raise ValueError(f"{what} expects contiguous f32 tensors of matching size")
            a[i] = t.data_ptr()
        sizes[i] = n
    return arrs, sizes


def adamw_multi_dev(params, grads, exp_avgs, exp_avg_sqs, hyper):
    """:func:`adamw_multi` with the hyper-parameters (lr, beta1, beta2, eps,
    weight_decay, bc1, bc2 as 7 f32 words) read from device address ``hyper``
    when the kernel runs."""
    if not params:
        return
    arrs, sizes = _multi_tables(list(zip(params, grads, exp_avgs, exp_avg_sqs)), "adamw_multi")
    call("wxx_adamw_multi_dev", *arrs, sizes, len(params), C.c_void_p(hyper))


def _unique_storages(tensors):
    seen, uniq = set(), []
    for t in tensors:
        key = (t.data_ptr(), validation.numel(t.shape))
        if key not in seen:
            seen.add(key)
            uniq.append(t)
    return uniq


def clip_scale_multi(tensors, sumsq, max_norm):
    """Rescale ``tensors`` in place by max_norm / (sqrt(s) + 1e-6) when that
    is below 1, with s the device scalar ``sumsq`` (decided on the device);
    returns a (1,) tensor holding sqrt(s)."""
    norm = empty((1,))
    uniq = _unique_storages(tensors)
    if uniq:
        (arr,), sizes = _multi_tables([(t,) for t in uniq], "clip_scale_multi")
    else:
        arr, sizes = (C.c_void_p * 1)(), (C.c_int64 * 1)()
    call("wxx_clip_scale_multi", arr, sizes, len(uniq), ptr(sumsq), float(max_norm), ptr(norm))
    return norm


def sumsq_multi(tensors):
    """Device scalar (shape (1,)) holding the sum of squares of every tensor."""
    count = len(tensors)
    out = empty((1,))
    ptrs = (C.c_void_p * max(1, count))()
    sizes = (C.c_int64 * max(1, count))()
    for i, t in enumerate(tensors):
        if not t.is_contiguous() or t.type != "f32":
            raise ValueError("sumsq_multi expects contiguous f32 tensors")
        ptrs[i] = t.data_ptr()
        sizes[i] = validation.numel(t.shape)
    call("wxx_sumsq_multi", ptrs, sizes, count, ptr(out))
    return out


def scale_multi(tensors, coef):
    """Multiply every tensor in place by ``coef`` (each storage once)."""
    seen = set()
    uniq = []
    for t in tensors:
        key = (t.data_ptr(), validation.numel(t.shape))
        if key not in seen:
            seen.add(key)
            uniq.append(t)
    count = len(uniq)
    if not count:
        return
    ptrs = (C.c_void_p * count)()
    sizes = (C.c_int64 * count)()
    for i, t in enumerate(uniq):
        if not t.is_contiguous() or t.type != "f32":
            raise ValueError("scale_multi expects contiguous f32 tensors")
        ptrs[i] = t.data_ptr()
        sizes[i] = validation.numel(t.shape)
    call("wxx_scale_multi", ptrs, sizes, count, float(coef))


def _same_values(t):
    """A new tensor object over ``t``'s (contiguous) storage."""
    out = Tensor(list(t.shape), buffer=t.buffer, offset=t.offset, dtype=t.type)
    out._base = t
    return out


def _copy_of(t):
    """A fresh buffer holding ``t``'s (contiguous) values."""
    out = empty(t.shape)
    call("wxx_d2d", ptr(out), ptr(t), 4 * math.prod(t.shape))
    return out


class DeviceSeed:
    """A dropout seed that lives in a step graph's per-replay words (device
    address ``ptr``): each replay writes a fresh draw of the host RNG there."""

    __slots__ = ("ptr",)

    def __init__(self, ptr):
        self.ptr = ptr


def _draw_seed(words):
    words[0] = random.randint(0, 2**32 - 1)


def dropout(tensor1, p, share_at_zero=False):
    """Inverted dropout; returns ``(y, seed)`` with a fresh 32-bit seed per call.

    At ``p == 0`` every element is kept with scale exactly 1, so the result
    holds the input's values and the seed is still drawn (the host RNG
    advances exactly as in the reference).  The result is a fresh buffer, as
    in the reference, unless ``share_at_zero`` asks for a tensor over the
    input's storage instead (the autograd layer's choice: it saves a copy of
    attention's probabilities; an in-place write into such a result also
    changes the input).
    """
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    n = math.prod(tensor1.shape)
    scale = 1 / (1 - p)
    if graphs.capturing():
        # each replay draws this call's seed from the host RNG, in call order
        r = DeviceSeed(graphs.per_replay(1, _draw_seed))
    else:
        r = random.randint(0, 2**32 - 1)
    if p == 0:
        return (_same_values(tensor1) if share_at_zero else _copy_of(tensor1)), r
    out = empty(tensor1.shape)
    if isinstance(r, DeviceSeed):
        call("wxx_dropout_dev", ptr(tensor1), ptr(out), n, C.c_void_p(r.ptr), float(p),
             float(scale))
    else:
        call("wxx_dropout", ptr(tensor1), ptr(out), n, r, float(p), float(scale))
    return out, r


def dropoutdx(tensor1, p, seed, share_at_zero=False):
    """Gradient of :func:`dropout` with the forward call's ``seed`` (the
    gradient's own values at ``p == 0``, in a fresh buffer unless
    ``share_at_zero``)."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if p == 0:
        return _same_values(tensor1) if share_at_zero else _copy_of(tensor1)
    n = math.prod(tensor1.shape)
    out = empty(tensor1.shape)
    if isinstance(seed, DeviceSeed):
        call("wxx_dropout_dev", ptr(tensor1), ptr(out), n, C.c_void_p(seed.ptr), float(p),
             float(1 / (1 - p)))
    else:
        call("wxx_dropout", ptr(tensor1), ptr(out), n, int(seed) & 0xFFFFFFFF, float(p),
             float(1 / (1 - p)))
    return out


def embed(tensor1, tensor2, n_token, embed_dim):
    """Gather rows of ``tensor2`` (V, D) by the u32 ids in ``tensor1`` (B, L)."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if not tensor2.is_contiguous():
        tensor2 = tensor2.contiguous()
    if tensor1.type != "u32":
        raise TypeError(f"embed expects u32 ids, got {tensor1.type!r}")
    if validation.numel(tensor1.shape) < n_token:
        raise ValueError(f"embed: {n_token} tokens requested, ids hold {validation.numel(tensor1.shape)}")
    V = tensor2.shape[0]
    if validation.numel(tensor2.shape) != V * embed_dim:
        raise ValueError(f"embed weight {tuple(tensor2.shape)} does not have width {embed_dim}")
    out = empty((tensor1.shape[0], tensor1.shape[1], embed_dim))
    call("wxx_embed", ptr(tensor1), ptr(tensor2), ptr(out), n_token, embed_dim, V)
    return out


def embeddx(tensor1, tensor2, n_token, embed_dim, vocab_size):
    """Weight gradient of :func:`embed` (``tensor1`` = grad, ``tensor2`` = ids)."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if not tensor2.is_contiguous():
        tensor2 = tensor2.contiguous()
    if validation.numel(tensor1.shape) < n_token * embed_dim:
        raise ValueError("embeddx grad is smaller than n_token * embed_dim")
    if validation.numel(tensor2.shape) < n_token:
        raise ValueError("embeddx ids are fewer than n_token")
    grad = empty((vocab_size, embed_dim))
    call("wxx_embeddx", ptr(tensor1), ptr(tensor2), ptr(grad), n_token, embed_dim, vocab_size)
    return grad
