"""Gradient clipping (reference src/wxx/nn/utils.py:1-103)."""

import numpy as np

from .. import functional, graphs


def _iter_params(parameters):
    if hasattr(parameters, "parameters") and not hasattr(parameters, "grad"):
        parameters = parameters.parameters()
    out = []
    for p in parameters:
        if isinstance(p, tuple):
            p = p[1]
        if p is not None:
            out.append(p)
    return out


def clip_grad_norm_(parameters, max_norm, norm_type=2.0):
    """Scale every gradient by max_norm / (total_norm + 1e-6) when that is
    below 1; returns the total norm (a float).

    L2 over f32 gradients (the training case) runs on the device: one
    multi-tensor sum-of-squares launch, one scalar readback, one multi-tensor
    rescale.  A gradient listed twice (aliased parameters) counts twice in the
    norm and is rescaled once, as in the reference.  Other norms read the
    gradients back to the host, as the reference's fallback does.

    Inside a step graph recording nothing may be read back: the coefficient
    is decided on the device (same float64 arithmetic) and the norm is
    returned as a (1,) device tensor that each replay rewrites.
    """
    pairs = [(p, p.grad) for p in _iter_params(parameters) if p.grad is not None]
    if not pairs:
        return 0.0
    grads = [g for _, g in pairs]
    l2_f32 = norm_type == 2.0 and all(g.type == "f32" and g.offset == 0 for g in grads)
    if graphs.capturing():
        if not l2_f32:
            raise RuntimeError("inside a step graph clip_grad_norm_ supports the L2 norm "
                               "of f32 gradients only")
        dense = [g if g.is_contiguous() else g.contiguous() for g in grads]
        norm = functional.clip_scale_multi(dense, functional.sumsq_multi(dense), max_norm)
        for (p, g), d in zip(pairs, dense):
            if d is not g:
                p.grad = d
        return norm
    if l2_f32:
        dense = [g if g.is_contiguous() else g.contiguous() for g in grads]
        total = float(functional.sumsq_multi(dense).numpy()[0]) ** 0.5
        coef = max_norm / (total + 1e-6)
        if coef < 1.0:
            functional.scale_multi(dense, coef)
            for (p, g), d in zip(pairs, dense):
                if d is not g:
                    p.grad = d
        return float(total)
    arrays = [g.numpy() for g in grads]
    if norm_type == float("inf"):
        total = max(float(np.max(np.abs(a))) for a in arrays)
    else:
        total = sum(float(np.sum(np.abs(a) ** norm_type)) for a in arrays) ** (1.0 / norm_type)
    coef = max_norm / (total + 1e-6)
    if coef < 1.0:
        for g, a in zip(grads, arrays):
            scaled = np.asarray(a) * coef
            if g.type == "c64":
                functional.assign(g, functional.from_numpy_complex(scaled))
            else:
                functional.assign(g, functional.from_numpy(np.asarray(scaled, np.float32)))
    return float(total)
