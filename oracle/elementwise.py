"""Elementwise ops restated from the reference (test infrastructure only).

* ``pointwise`` (pointwise.wgsl:45-58): broadcast a op b, op 0 add, 1 sub,
  2 mul, 3 div, anything else add.
* ``scalarpointwise`` (scalarpointwise.wgsl:35-69): op 0 add, 1 sub (reverse
  c - x), 2 mul, 3 pow, 4 div (reverse c / x).  pow with reverse is c ** x
  (host rejects c <= 0); a negative base with an integer exponent keeps the
  sign of odd exponents, a fractional exponent gives NaN.
* ``clamp`` / ``clampbackwards`` (clamp.wgsl, clampbackwards.wgsl),
  ``equal`` (equal.wgsl: 1.0 / 0.0), ``masked_fill`` (maskedfill.wgsl:
  x != 0 ? x : fill), ``mul_backward`` (mul_backward.wgsl).
"""

import numpy as np


def pointwise(a, b, op):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        if op == 1:
            r = a - b
        elif op == 2:
            r = a * b
        elif op == 3:
            r = a / b
        else:
            r = a + b
    return r.astype(np.float32)


def scalarpointwise(x, c, op, reverse=0):
    x = np.asarray(x, np.float32)
    c32 = np.float32(c)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        if op == 0:
            return x + c32
        if op == 1:
            return (c32 - x) if reverse else (x - c32)
        if op == 2:
            return x * c32
        if op == 4:
            return (c32 / x) if reverse else (x / c32)
        if op == 3:
            x64 = x.astype(np.float64)
            c64 = float(c32)
            if reverse:
                return np.power(c64, x64).astype(np.float32)
            mag = np.power(np.abs(x64), c64)
            if c64 == np.trunc(c64):
                odd = (abs(c64) * 0.5) % 1.0 > 0.25
                neg = -mag if odd else mag
            else:
                neg = np.full_like(mag, np.nan)
            return np.where(x64 < 0, neg, np.power(np.where(x64 < 0, 1.0, x64), c64)).astype(
                np.float32
            )
    return x.copy()


def clamp(x, lo, hi):
    return np.minimum(np.maximum(np.asarray(x, np.float32), np.float32(lo)), np.float32(hi))


def clampbackwards(x, lo, hi):
    x = np.asarray(x, np.float32)
    return ((x >= np.float32(lo)) & (x <= np.float32(hi))).astype(np.float32)


def equal(a, b):
    return (np.asarray(a) == np.asarray(b)).astype(np.float32)


def masked_fill(x, fill):
    x = np.asarray(x, np.float32)
    return np.where(x != 0, x, np.float32(fill)).astype(np.float32)


def mul_backward(g, a, b):
    g = np.asarray(g, np.float32)
    return (g * np.asarray(b, np.float32)).astype(np.float32), (
        g * np.asarray(a, np.float32)
    ).astype(np.float32)
