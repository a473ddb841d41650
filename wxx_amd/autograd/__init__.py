"""Differentiable ops recorded into a reverse-mode graph (the surface of
reference src/wxx/autograd/__init__.py:1-128)."""

from .function import Function
from .convolution import (
    Conv2D,
    Conv2DTranspose,
    adaptive_avgpooling2d,
    avgpooling1d,
    avgpooling2d,
    causal_conv1d,
    maxpooling1d,
    maxpooling2d,
)
from .layers import CrossEntropyLoss, Dropout, Embedding, FusedAttention, swiglu_padded
from .normalization import batchnorm, batchnorm_act, meanvarnorm, rmsnorm
from .pointwise import (
    abs,
    add,
    addscaler,
    clamp,
    cos,
    decay_window,
    div,
    exp,
    gelu,
    log,
    mul,
    mulscaler,
    negate,
    powscaler,
    rdivscaler,
    relu,
    rpowscaler,
    rsqrt,
    selu,
    sigmoid,
    sign,
    sin,
    sqrt,
    square,
    sub,
    subscaler,
)
from .reductions import (
    argmax,
    argmin,
    max,
    mean,
    min,
    scaled_masked_softmax,
    softmax,
    std,
    sum,
    var,
)
from .utils import (
    complex_conj,
    complex_mul,
    concat,
    diagonal,
    flatten,
    getitem,
    irfft,
    matmul,
    matmuladd,
    narrow,
    permute,
    reshape,
    rfft,
    squeeze,
    unfold,
    unsqueeze,
)
