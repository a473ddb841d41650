"""Modules, models, losses, optimizers and schedulers (surface of reference
src/wxx/nn/__init__.py:1-87)."""

from .gpt import GPT2, GPT2Block
from .hyena import CausalShortConv1d, Hyena, HyenaBlock, HyenaOperator, ImplicitFilter
from .loss import CCELoss, MAELoss, loss
from .module import (
    GELU,
    AdaptiveAvgPool2d,
    Attention,
    AvgPool1d,
    AvgPool2d,
    BatchNorm,
    Conv2D,
    Conv2DTranspose,
    Dropout,
    Embedding,
    LayerNorm,
    Linear,
    MaxPool1d,
    MaxPool2d,
    Module,
    ModuleList,
    MultiHeadAttention,
    PositionalEncoding,
    RMSNorm,
    Sequential,
    Sine,
    SwiGLU,
    TiedLinear,
)
from .optimizer import SGD, AdamW, Optimizer
from .resnet import ResBlock, ResNet18
from .scheduler import (
    CosineAnnealingLR,
    ExponentialLR,
    LambdaLR,
    LRScheduler,
    StepLR,
    WarmupCosineLR,
)
from .utils import clip_grad_norm_

__all__ = [
    "loss", "MAELoss", "CCELoss", "AdaptiveAvgPool2d", "Attention", "AvgPool1d", "AvgPool2d",
    "BatchNorm", "CausalShortConv1d", "Conv2D", "Conv2DTranspose", "Dropout", "Embedding",
    "GELU", "LayerNorm", "Linear", "MaxPool1d", "MaxPool2d", "Module", "ModuleList",
    "MultiHeadAttention", "RMSNorm", "Sequential", "AdamW", "Optimizer", "SGD", "LRScheduler",
    "LambdaLR", "StepLR", "ExponentialLR", "CosineAnnealingLR", "WarmupCosineLR", "Sine",
    "ImplicitFilter", "PositionalEncoding", "HyenaOperator", "SwiGLU", "HyenaBlock", "Hyena",
    "TiedLinear", "clip_grad_norm_", "GPT2", "GPT2Block", "ResBlock", "ResNet18",
]
