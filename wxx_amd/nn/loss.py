"""Losses (reference src/wxx/nn/loss.py:1-47)."""

import math

from .. import autograd


class loss:
    def __init__(self):
        pass

    def __call__(self):
        pass


class MAELoss(loss):
    def __call__(self, prediction, truth):
        return (truth - prediction).abs().mean()


class CCELoss(loss):
    """Mean softmax cross-entropy of (B, K) logits against (B,) u32 targets;
    with ``mask`` (one value per row) the masked mean."""

    def __call__(self, prediction, truth, mask=None):
        token_loss = autograd.CrossEntropyLoss(prediction).forward(prediction, truth)
        if mask is None:
            return token_loss.mean()
        if math.prod(mask.shape) != prediction.shape[0]:
            raise ValueError(
                f"mask must contain one value per prediction row; got "
                f"{math.prod(mask.shape)} values for {prediction.shape[0]} rows")
        mask = mask.reshape((prediction.shape[0], 1))
        return (token_loss * mask).sum() / mask.sum()
