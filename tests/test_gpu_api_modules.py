"""GPU: pooling and convolution through the nn modules and the functional
argument checks (the behaviours of reference tests/test_pooling.py and
tests/test_convolution.py at module level; the kernels themselves are
pinned against the oracle in test_gpu_conv.py)."""

import numpy as np
import pytest

from conftest import assert_close, rng
from oracle import conv as oc

pytestmark = pytest.mark.gpu


def wxx():
    import wxx_amd

    return wxx_amd


def f32(a, grad=False):
    t = wxx().functional.from_numpy(np.asarray(a, np.float32))
    t.requires_grad = grad
    return t


def _pool1d(X, k, s, p, avg):
    out, idx = oc.pool2d(X[:, :, None, :], (1, k), (1, s), (0, p), avg=avg)
    return out[:, :, 0], idx[:, :, 0]


def _pool1d_dx(g, idx, shape, k, s, p, avg):
    B, C, L = shape
    return oc.pool2d_backward(g[:, :, None], None if avg else idx[:, :, None], (B, C, 1, L),
                              (1, k), (1, s), (0, p), avg=avg)[:, :, 0]


@pytest.mark.parametrize("avg", [False, True])
def test_pool1d_modules_indices_and_backward(device, avg):
    nn = wxx().nn
    X = rng(34).standard_normal((2, 2, 10)).astype(np.float32)
    mod = (nn.AvgPool1d if avg else nn.MaxPool1d)(3, stride=2, padding=1, return_indices=True)
    x = f32(X, True)
    out, idx = mod(x)
    eo, ei = _pool1d(X, 3, 2, 1, avg)
    assert idx.type == "u32"
    assert_close(out.numpy(), eo, rtol=1e-6, atol=1e-6)
    # avg pooling reports the window arg-max too (reference semantics)
    np.testing.assert_array_equal(idx.numpy(), _pool1d(X, 3, 2, 1, False)[1])
    out.sum().backward()
    want = _pool1d_dx(np.ones(eo.shape), ei, X.shape, 3, 2, 1, avg)
    assert_close(x.grad.numpy(), want, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("avg", [False, True])
def test_pool2d_modules_indices_and_backward(device, avg):
    nn = wxx().nn
    X = rng(35).standard_normal((2, 2, 6, 6)).astype(np.float32)
    mod = (nn.AvgPool2d if avg else nn.MaxPool2d)(2, stride=2, return_indices=True)
    x = f32(X, True)
    out, idx = mod(x)
    eo, ei = oc.pool2d(X, (2, 2), (2, 2), (0, 0), avg=avg)
    assert_close(out.numpy(), eo, rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(idx.numpy(), oc.pool2d(X, (2, 2), (2, 2), (0, 0), avg=False)[1])
    out.sum().backward()
    want = oc.pool2d_backward(np.ones(eo.shape), None if avg else ei, X.shape, (2, 2), (2, 2),
                              (0, 0), avg=avg)
    assert_close(x.grad.numpy(), want, rtol=1e-6, atol=1e-6)


def test_pool_modules_without_indices_return_a_tensor(device):
    nn = wxx().nn
    x = f32(rng(36).standard_normal((2, 3, 8, 8)))
    for mod in (nn.MaxPool2d(2), nn.AvgPool2d(3, stride=1, padding=1)):
        assert isinstance(mod(x), wxx().Tensor)
    out = nn.AvgPool1d(3, stride=2, padding=1)(f32(np.zeros((2, 2, 9))))
    assert isinstance(out, wxx().Tensor) and out.shape == [2, 2, 5]


def test_adaptive_avgpool_module_backward(device):
    X = rng(3).standard_normal((2, 3, 8, 9)).astype(np.float32)
    x = f32(X, True)
    y = wxx().nn.AdaptiveAvgPool2d((2, 3))(x)
    assert_close(y.numpy(), oc.adaptive_avgpool2d(X, (2, 3)), rtol=1e-6, atol=1e-6)
    G = rng(4).standard_normal(y.shape).astype(np.float32)
    (y * f32(G)).sum().backward()
    assert_close(x.grad.numpy(), oc.adaptive_avgpool2ddx(G, X.shape), rtol=1e-6, atol=1e-6)


def test_pool_argument_errors(device):
    F = wxx().functional
    x1, x2 = f32(np.zeros((2, 2, 8))), f32(np.zeros((2, 2, 4, 4)))
    for fn, x in ((F.avgpool1d, x2), (F.maxpool1d, x2), (F.avgpool2d, x1), (F.maxpool2d, x1)):
        with pytest.raises(ValueError):
            fn(x, 2, 2, 0)
    for fn in (F.avgpool1d, F.maxpool1d):
        for bad in (0, -1):
            with pytest.raises(ValueError):
                fn(x1, bad, 1, 0)
    for fn, shape in ((F.avgpool2d, (2, 2, 4, 4)), (F.maxpool2d, (2, 2, 4, 4)),
                      (F.avgpool1d, (2, 2, 8)), (F.maxpool1d, (2, 2, 8))):
        with pytest.raises(TypeError):
            fn(F.from_numpy(np.zeros(shape), np.uint32), 2, 2, 0)


def test_conv2d_module_forward_and_bias_grad(device):
    nn, F = wxx().nn, wxx().functional
    c = nn.Conv2D(2, 3, kernel=(3, 3), stride=(1, 1), padding=(1, 1))
    W = rng(30).standard_normal(tuple(c.W.shape)).astype(np.float32)
    b = rng(31).standard_normal(tuple(c.bias.shape)).astype(np.float32)
    F.assign(c.W, f32(W))
    F.assign(c.bias, f32(b))
    X = rng(32).standard_normal((2, 2, 5, 5)).astype(np.float32)
    x = f32(X, True)
    out = c(x)
    assert out.shape == [2, 3, 5, 5]
    assert_close(out.numpy(), oc.conv2d(X, W, (1, 1), (1, 1), (1, 1), b), rtol=1e-4, atol=1e-5)
    G = rng(33).standard_normal(tuple(out.shape)).astype(np.float32)
    (out * f32(G)).sum().backward()
    assert_close(c.bias.grad.numpy(), G.sum(axis=(0, 2, 3)), rtol=1e-5, atol=1e-5)
    assert_close(c.W.grad.numpy(), oc.conv2ddw(G, X, (1, 1), (1, 1), (1, 1), W.shape), rtol=1e-4,
                 atol=1e-4)
    assert_close(x.grad.numpy(), oc.conv2ddx(G, W, (1, 1), (1, 1), (1, 1), X.shape), rtol=1e-4,
                 atol=1e-4)


def _tconv_module(shape, wshape, stride, padding, dilation, out_pad, seed, bias=True):
    nn, F = wxx().nn, wxx().functional
    r = rng(seed)
    m = nn.Conv2DTranspose(wshape[0], wshape[1], kernel=wshape[2:], stride=stride,
                           padding=padding, dilation=dilation, output_padding=out_pad, bias=bias)
    X = r.standard_normal(shape).astype(np.float32)
    W = r.standard_normal(wshape).astype(np.float32)
    F.assign(m.W, f32(W))
    b = None
    if bias:
        b = r.standard_normal(wshape[1]).astype(np.float32)
        F.assign(m.bias, f32(b))
    return m, X, W, b


def test_conv2dtranspose_output_padding_cells(device):
    # cells reachable only through output_padding hold the bias (or exactly 0)
    m, X, W, b = _tconv_module((2, 2, 5, 5), (2, 3, 3, 3), (2, 2), (0, 0), (1, 1), (1, 1), 60)
    out = m(f32(X)).numpy()
    assert out.shape[2:] == (12, 12)
    plain, _, _, _ = _tconv_module((2, 2, 5, 5), (2, 3, 3, 3), (2, 2), (0, 0), (1, 1), (0, 0), 60)
    assert_close(plain(f32(X)).numpy(), out[:, :, :11, :11], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(out[:, :, 11, :], np.broadcast_to(b[None, :, None], (2, 3, 12)),
                               atol=1e-6)
    np.testing.assert_allclose(out[:, :, :, 11], np.broadcast_to(b[None, :, None], (2, 3, 12)),
                               atol=1e-6)
    nb, Xn, _, _ = _tconv_module((2, 2, 5, 5), (2, 3, 3, 3), (2, 2), (0, 0), (1, 1), (1, 1), 60,
                                 bias=False)
    o = nb(f32(Xn)).numpy()
    assert np.all(o[:, :, 11, :] == 0.0) and np.all(o[:, :, :, 11] == 0.0)


def test_conv2dtranspose_module_backward_long_spatial(device):
    # B * Ho * Wo well above 2048 (the reference splits its dW reduction there)
    m, X, W, b = _tconv_module((3, 2, 16, 16), (2, 2, 3, 3), (2, 2), (1, 1), (1, 1), (0, 0), 70)
    x = f32(X, True)
    out = m(x)
    assert out.shape == [3, 2, 31, 31]
    G = rng(71).standard_normal(tuple(out.shape)).astype(np.float32)
    (out * f32(G)).sum().backward()
    assert_close(m.W.grad.numpy(), oc.conv2dtranspose_dw(G, X, (2, 2), (1, 1), (1, 1), W.shape),
                 rtol=1e-4, atol=1e-3)
    assert_close(x.grad.numpy(), oc.conv2dtranspose_dx(G, W, (2, 2), (1, 1), (1, 1), X.shape),
                 rtol=1e-4, atol=1e-4)
    assert_close(m.bias.grad.numpy(), G.sum(axis=(0, 2, 3)), rtol=1e-5, atol=1e-4)


def test_conv2dtranspose_1x1_is_a_channel_mix(device):
    m, X, W, b = _tconv_module((2, 3, 4, 5), (3, 2, 1, 1), (1, 1), (0, 0), (1, 1), (0, 0), 80)
    out = m(f32(X))
    assert out.shape == [2, 2, 4, 5]
    want = np.einsum("bchw,cd->bdhw", X.astype(np.float64), W[:, :, 0, 0]) + b[None, :, None, None]
    assert_close(out.numpy(), want, rtol=1e-5, atol=1e-5)


def test_conv2dtranspose_argument_errors(device):
    nn, F = wxx().nn, wxx().functional
    for kw in ({"stride": 2, "output_padding": 2}, {"stride": 1, "dilation": 1, "output_padding": 1},
               {"stride": (2, 3), "output_padding": (1, 3)}):
        with pytest.raises(ValueError):
            nn.Conv2DTranspose(2, 3, kernel=3, **kw)
    with pytest.raises(ValueError):
        F.conv2dtranspose(f32(np.zeros((1, 3, 4, 4))), f32(np.zeros((2, 2, 3, 3))), (1, 1),
                          (0, 0), (1, 1), (0, 0))
