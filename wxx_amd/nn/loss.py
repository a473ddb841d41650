"""Loss functions (reference src/wxx/nn/loss.py:1-47).

A loss object is a callable that maps (prediction, target[, mask]) to a
scalar autograd Tensor; ``backward`` on that Tensor drives the gradients.
The public names are those of the reference: the base class ``loss``,
``MAELoss`` and ``CCELoss``.
"""

import math

from .. import autograd


class loss:
    """Base of the losses: subclasses define ``__call__``."""

    def __call__(self, *args, **kwargs):
        return None


class MAELoss(loss):
    """Mean absolute error over every element."""

    def __call__(self, prediction, truth):
        return (truth - prediction).abs().mean()


class CCELoss(loss):
    """Softmax cross-entropy of (rows, classes) logits against (rows,) u32
    class ids, averaged over rows; with ``mask`` (one weight per row) the
    weighted mean sum(l_r m_r) / sum(m_r)."""

    def __call__(self, prediction, truth, mask=None):
        rows = prediction.shape[0]
        per_row = autograd.CrossEntropyLoss(prediction).forward(prediction, truth)  # (rows, 1)
        if mask is None:
            return per_row.mean()
        n_mask = math.prod(mask.shape)
        if n_mask != rows:
            raise ValueError(f"CCELoss mask holds {n_mask} values; the prediction has {rows} rows "
                             "and needs one mask value per row")
        weights = mask.reshape((rows, 1))
        return (per_row * weights).sum() / weights.sum()


__all__ = ["loss", "MAELoss", "CCELoss"]
