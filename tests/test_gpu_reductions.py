"""GPU parity: reductions and softmax against the oracle (via the C ABI)."""

import numpy as np
import pytest

from conftest import assert_close, assert_error_floor, rng
from oracle import activations as oa
from oracle import reductions as orr

pytestmark = pytest.mark.gpu


def F():
    from wxx_amd import functional

    return functional


def up(a):
    return F().from_numpy(np.asarray(a, np.float32))


@pytest.mark.parametrize("shape,axis,keepdims", [
    ((4, 5), None, False), ((4, 5), 0, False), ((4, 5), 1, True), ((4, 5), -1, False),
    ((2, 3, 4, 5), (1, 2), False), ((7,), 0, False), ((3, 100000), 1, False),
    ((1, 10_000_000), None, False), ((8, 589824), 0, False), ((1000, 3, 7), 1, True),
    ((5, 1, 9), 1, False), ((2, 4097, 3), 1, False),
])
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_reduce_modes(device, shape, axis, keepdims, mode):
    x = rng(sum(shape) + mode).standard_normal(shape).astype(np.float32)
    fn = [F().sum, F().mean, F().sumsq][mode]
    got = fn(up(x), axis=axis, keepdims=keepdims).numpy()
    exp = orr.reduce(x, axis=axis, keepdims=keepdims, mode=mode)
    # fp32 summation in a different order than the float64 oracle: allow
    # 1e-6 of each output's L1 mass (a wrong index or a dropped block is off
    # by O(sqrt(n)) times more).
    mass = orr.reduce(np.abs(x), axis=axis, keepdims=keepdims, mode=2 if mode == 2 else mode)
    atol = 1e-5 + 1e-6 * np.abs(mass).astype(np.float64)
    err = np.abs(got.astype(np.float64) - exp)
    assert got.shape == exp.shape
    assert np.all(err <= atol + 1e-4 * np.abs(exp)), float(np.max(err - atol))


def test_reduce_reference_test_case(device):
    # reference tests/test_reductions.py:10-15
    a = rng(0).standard_normal((4, 5)).astype(np.float32)
    t = up(a)
    assert_close(F().sum(t).numpy(), a.sum(keepdims=False).reshape(1), atol=1e-4)
    assert_close(F().sum(t, axis=0).numpy(), a.sum(axis=0), atol=1e-4)
    assert_close(F().sum(t, axis=1, keepdims=True).numpy(), a.sum(axis=1, keepdims=True), atol=1e-4)
    assert_close(F().mean(t, axis=-1).numpy(), a.mean(axis=-1), atol=1e-4)


@pytest.mark.parametrize("op", [0, 1])
@pytest.mark.parametrize("shape,axis", [((3, 4), 1), ((3, 4), 0), ((5, 700), 1), ((2, 600, 3), 1),
                                        ((1, 100000), None), ((64, 1024), -1)])
def test_minmax_bit_exact(device, op, shape, axis):
    r = rng(40 + op)
    x = r.integers(-3, 4, size=shape).astype(np.float32)  # many ties: exercises the tie rule
    fn = F().max if op == 0 else F().min
    v, i = fn(up(x), axis=axis)
    ev, ei = orr.minmax(x, axis=axis, op=op)
    assert np.array_equal(v.numpy(), ev)
    assert i.type == "u32"
    assert np.array_equal(i.numpy(), ei)


def test_minmax_special_values(device):
    x = np.array([[0.0, 5.0, 5.0, 1.0], [-np.inf, -np.inf, -np.inf, -np.inf],
                  [np.nan, 2.0, np.nan, 2.0], [-1e38, -1e38, -2e38, -1e38]], np.float32)
    v, i = F().max(up(x), axis=1)
    ev, ei = orr.minmax(x, axis=1, op=0)
    assert np.array_equal(i.numpy(), ei) and np.array_equal(v.numpy(), ev)
    assert list(ei) == [2, 0, 1, 0]


def test_maxmin_backward(device):
    x = rng(5).standard_normal((6, 33)).astype(np.float32)
    g = rng(6).standard_normal(6).astype(np.float32)
    _, i = F().max(up(x), axis=1)
    d = F().maxmin_backward(up(g), i, x.shape, axis=1).numpy()
    assert np.array_equal(d, orr.maxmin_backward(g, i.numpy(), x.shape, axis=1))


@pytest.mark.parametrize("shape,dim", [((3, 5), -1), ((8192, 4096), -1), ((96, 1024, 1024), -1),
                                       ((512, 128), -1), ((7, 3000), 1), ((4, 20000), -1),
                                       ((2, 50304), -1), ((4, 6, 3), 1), ((5, 7), 0),
                                       ((33, 1), -1), ((10, 10), -1)])
def test_softmax(device, shape, dim):
    # every element (config 2's [8192 x 4096] included) against float64, at
    # rtol 1e-5 plus 4x the error of the same steps in float32; the
    # 96 x 1024 x 1024 attention case is checked on 64 of its rows, and its
    # row sums everywhere
    x = (rng(7).standard_normal(shape) * 3).astype(np.float32)
    got = F().softmax(up(x), dim).numpy()
    if np.prod(shape) > 50_000_000:
        assert_close(got.sum(axis=dim), np.ones(got.sum(axis=dim).shape, np.float32), atol=2e-6)
        idx = rng(8).integers(0, shape[0], 64)
        got, x = got[idx], x[idx]
    assert_error_floor(got, oa.softmax(x, dim, rounded=False), oa.softmax(x, dim, np.float32),
                       rtol=1e-5)


def test_softmax_reference_test_case(device):
    a = rng(3).standard_normal((3, 5)).astype(np.float32)
    ref = np.exp(a) / np.exp(a).sum(axis=-1, keepdims=True)
    assert_close(F().softmax(up(a), dim=-1).numpy(), ref, atol=1e-5)


def test_softmax_masked_rows(device):
    x = rng(9).standard_normal((4, 64)).astype(np.float32)
    x[:, 10:] += -1e9  # additive causal-mask style
    got = F().softmax(up(x), -1).numpy()
    assert_close(got, oa.softmax(x, -1))
    assert np.all(got[:, 10:] == 0)


@pytest.mark.parametrize("shape,dim", [((5, 7), -1), ((64, 1024), -1), ((8, 12, 33, 129), -1),
                                       ((4, 50257), -1), ((6, 5, 9), 1), ((3, 70000), -1)])
def test_softmax_backward(device, shape, dim):
    r = rng(21)
    y = oa.softmax(r.standard_normal(shape).astype(np.float32) * 2, dim)
    g = r.standard_normal(shape).astype(np.float32)
    got = F().softmax_backward(up(y), up(g), dim).numpy()
    assert_error_floor(got, oa.softmax_backward(y, g, dim, rounded=False),
                       oa.softmax_backward(y, g, dim, np.float32), rtol=1e-5)


@pytest.mark.parametrize("src,shape,scale", [((1, 1), (4, 5), 1.0), ((4, 1), (4, 5), 0.25),
                                             ((1, 5), (4, 5), 2.0), ((3, 1, 6), (3, 4, 6), 1.0),
                                             ((1,), (1000,), 0.001)])
def test_broadcast_to(device, src, shape, scale):
    g = rng(22).standard_normal(src).astype(np.float32)
    got = F().broadcast_to(up(g), shape, scale).numpy()
    assert np.array_equal(got, (np.broadcast_to(g, shape) * np.float32(scale)).astype(np.float32))


@pytest.mark.parametrize("rows,C,mask_rows,ld", [(96 * 16, 128, 128, 256), (7, 1024, 0, 0),
                                                 (33, 37, 11, 37), (6, 5000, 3, 5000),
                                                 (96 * 1024, 1024, 1024, 1024)])
def test_softmax_scale_mask_fused(device, rows, C, mask_rows, ld):
    # attention score path: softmax(x * scale + mask) and its gradient scale * dsoftmax
    r = rng(rows + C)
    x = (r.standard_normal((rows, C)) * 3).astype(np.float32)
    scale = np.float32(0.125)
    mask = None
    if mask_rows:
        big = np.where(r.random((mask_rows, ld)) < 0.3, -1e9, 0.0).astype(np.float32)
        mask = big[:, :C]
    shape = (rows // mask_rows, mask_rows, C) if mask_rows else (rows, C)  # (B*H, S, S) layout
    tx = F().from_numpy(x.reshape(shape))
    tm = None
    if mask is not None:
        tm = F().from_numpy(big).narrow(1, 0, C) if ld != C else F().from_numpy(mask)
    y = F().softmax_scale_mask(tx, float(scale), tm).numpy().reshape(rows, C)
    z = (x * scale).astype(np.float32)
    if mask is not None:
        z = (z + np.tile(mask, (rows // mask_rows + 1, 1))[:rows]).astype(np.float32)
    want = oa.softmax(z, -1)
    assert_close(y, want, rtol=1e-4, atol=1e-6)
    g = r.standard_normal((rows, C)).astype(np.float32)
    dx = F().softmax_backward_scale(F().from_numpy(y), F().from_numpy(g), float(scale)).numpy()
    assert_close(dx, oa.softmax_backward(y, g, -1) * scale, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("BH,S", [(3, 7), (2, 64), (2, 130), (1, 1024)])
def test_softmax_causal_equals_masked_softmax(device, BH, S):
    # the causal path reads only j <= i and must give the masked fused
    # softmax's numbers bit for bit: those entries equal, zeros above
    from wxx_amd.functional._common import empty

    r = rng(BH * S)
    x = (r.standard_normal((BH, S, S)) * 3).astype(np.float32)
    i = np.arange(S)
    mask = np.where(i[None, :] <= i[:, None], 0.0, -1e9).astype(np.float32)
    lower = np.broadcast_to(i[None, :] <= i[:, None], (BH, S, S))
    scale = 0.125
    want = F().softmax_scale_mask(F().from_numpy(x), scale, F().from_numpy(mask)).numpy()
    y = F().softmax_causal(F().from_numpy(x), scale).numpy()
    assert np.array_equal(y, want)
    assert np.all(y[~lower] == 0)
    # skip mode: the upper triangle keeps whatever the buffer held
    from wxx_amd.backend import lib
    import ctypes as C

    out = F().from_numpy(np.full((BH, S, S), 7.0, np.float32))
    tx = F().from_numpy(x)
    lib.call("wxx_softmax_causal", C.c_void_p(tx.data_ptr()), C.c_void_p(out.data_ptr()), BH * S,
             S, S, C.c_float(scale), 1)
    got = out.numpy()
    assert np.array_equal(got[lower], want[lower]) and np.all(got[~lower] == 7.0)
    # backward: the masked gradient's numbers on and below the diagonal, 0 above
    g = r.standard_normal((BH, S, S)).astype(np.float32)
    wdx = F().softmax_backward_scale(F().from_numpy(want), F().from_numpy(g), scale).numpy()
    dx = F().softmax_backward_causal(F().from_numpy(want), F().from_numpy(g), scale).numpy()
    assert np.array_equal(dx[lower], wdx[lower]) and np.all(dx[~lower] == 0)
    dxs = F().softmax_backward_causal(F().from_numpy(want), F().from_numpy(g), scale,
                                      skip=True).numpy()
    assert np.array_equal(dxs[lower], wdx[lower])


@pytest.mark.parametrize("shape,axis,keepdims", [
    ((6, 7), None, False), ((6, 7), 1, True), ((3, 4, 5), (1, 2), False), ((9,), 0, False),
    ((64, 4096), -1, False), ((8, 1024, 768), 2, True), ((5, 1, 3), 1, False),
])
def test_var_std(device, shape, axis, keepdims):
    # the reference's composite (functional/reductions.py:315-336): mean,
    # subtract, square, mean; std = sqrt(var); population variance
    x = (rng(sum(shape)).standard_normal(shape) * 2 + 0.5).astype(np.float32)
    v = F().var(up(x), axis=axis, keepdims=keepdims).numpy()
    s = F().std(up(x), axis=axis, keepdims=keepdims).numpy()
    assert_close(v, orr.var(x, axis, keepdims), rtol=1e-4, atol=1e-5)
    assert_close(s, orr.std(x, axis, keepdims), rtol=1e-4, atol=1e-5)
    # the Tensor methods take the same path, and var backward is 2 (x - mean) / n
    from wxx_amd.Tensor import Tensor

    t = Tensor(list(x.shape), data=x, requires_grad=True)
    tv = t.var(axis=axis, keepdims=keepdims)
    assert_close(tv.numpy(), v, rtol=0, atol=0)
    tv.sum().backward()
    ax = None if axis is None else axis
    n = x.size if axis is None else int(np.prod([x.shape[a] for a in np.atleast_1d(axis)]))
    xd = x.astype(np.float64)
    want = 2 * (xd - xd.mean(axis=ax, keepdims=True)) / n
    assert_close(t.grad.numpy(), want, rtol=1e-4, atol=1e-5)


def test_var_rejects_non_contiguous_axes(device):
    # as the reference's reduction mapping (backend/dispatch.py:173-214)
    with pytest.raises(ValueError):
        F().var(up(np.ones((3, 4, 5))), axis=(0, 2))
