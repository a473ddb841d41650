"""Softmax and unary activations restated from the reference (test infrastructure only).

softmax: reference src/wxx/shaders/activations/softmax.wgsl:47-74 —
  m = max(-1e38, max x), y = exp(x - m) * (1 / sum exp(x - m)); float64 here.
gelu / gelu': tanh form with clamps, gelu.wgsl:20-27, gelubackwards.wgsl:21-32
  (constants 0.7978845608, 0.044715, 0.134145).
sigmoid: input clamped to [-88, 88], sigmoid.wgsl:20; sigmoid' takes y.
selu: selu.wgsl / selubackwards.wgsl (ALPHA, SCALE constants).
relu' = [x > 0]; sin' = cos; cos' = -sin; sign(0) = 0.
"""

import numpy as np

SQRT_2_OVER_PI = 0.7978845608
GELU_C = 0.044715
GELU_DC = 0.134145
SELU_ALPHA = 1.6732632423543772848170429916717
SELU_SCALE = 1.0507009873554804934193349852946


def softmax(x, dim=-1, dtype=np.float64, rounded=True):
    """``dtype=np.float32``: the same steps in single precision (the rounding
    floor of an fp32 evaluation); ``rounded=False`` keeps the float64 values."""
    x = np.asarray(x, dtype=np.float32).astype(dtype)
    m = np.maximum(np.max(x, axis=dim, keepdims=True), dtype(-1e38))
    e = np.exp(x - m)
    y = e * (dtype(1.0) / e.sum(axis=dim, keepdims=True))
    return y.astype(np.float32) if rounded else y


def softmax_backward(y, g, dim=-1, dtype=np.float64, rounded=True):
    """Softmax gradient from the output: y * (g - sum(g * y, dim)) (reference
    src/wxx/autograd/reductions.py:25-35)."""
    y = np.asarray(y, dtype=dtype)
    g = np.asarray(g, dtype=dtype)
    dot = (g * y).sum(axis=dim, keepdims=True)
    out = y * (g - dot)
    return out.astype(np.float32) if rounded else out


def gelu(x):
    x = np.asarray(x, dtype=np.float64)
    u = SQRT_2_OVER_PI * (x + GELU_C * x ** 3)
    y = 0.5 * x * (1.0 + np.tanh(u))
    y = np.where(x > 10.0, x, np.where(x < -10.0, 0.0, y))
    return y.astype(np.float32)


def gelubackwards(x):
    x = np.asarray(x, dtype=np.float64)
    u = SQRT_2_OVER_PI * (x + GELU_C * x ** 3)
    t = np.tanh(u)
    du = SQRT_2_OVER_PI * (1.0 + GELU_DC * x * x)
    d = 0.5 * (1.0 + t) + 0.5 * x * (1.0 - t * t) * du
    d = np.where(x > 10.0, 1.0, np.where(x < -10.0, 0.0, d))
    return d.astype(np.float32)


def sigmoid(x):
    x = np.clip(np.asarray(x, dtype=np.float64), -88.0, 88.0)
    return (1.0 / (1.0 + np.exp(-x))).astype(np.float32)


def sigmoidbackwards(y):
    y = np.asarray(y, dtype=np.float64)
    return (y * (1.0 - y)).astype(np.float32)


def selu(x):
    x = np.asarray(x, dtype=np.float64)
    return np.where(x > 0, SELU_SCALE * x, SELU_SCALE * SELU_ALPHA * (np.exp(x) - 1.0)).astype(
        np.float32
    )


def selubackwards(x):
    x = np.asarray(x, dtype=np.float64)
    return np.where(x > 0, SELU_SCALE, SELU_SCALE * SELU_ALPHA * np.exp(x)).astype(np.float32)


def _f(fn):
    def wrapped(x):
        return fn(np.asarray(x, dtype=np.float64)).astype(np.float32)

    return wrapped


UNARY = {
    "relu": _f(lambda x: np.maximum(0.0, x)),
    "relubackwards": _f(lambda x: (x > 0).astype(np.float64)),
    "gelu": gelu,
    "gelubackwards": gelubackwards,
    "sigmoid": sigmoid,
    "sigmoidbackwards": sigmoidbackwards,
    "selu": selu,
    "selubackwards": selubackwards,
    "sin": _f(np.sin),
    "sinback": _f(np.cos),
    "cos": _f(np.cos),
    "cosback": _f(lambda x: -np.sin(x)),
    "abs": _f(np.abs),
    "exp": _f(np.exp),
    "log": _f(np.log),
    "negate": _f(lambda x: -x),
    "rsqrt": _f(lambda x: 1.0 / np.sqrt(x)),
    "sign": _f(np.sign),
    "sqrt": _f(np.sqrt),
    "square": _f(lambda x: x * x),
}
