"""GPU parity: conv2d / conv2ddx / conv2ddw (implicit-GEMM MFMA kernels with
split-K), max / average / adaptive pooling (indices bit-exact) and the
depthwise causal conv1d, against the oracle (float64 restatements)."""

import numpy as np
import pytest

from conftest import assert_close, assert_error_floor, rng
from oracle import conv as oc

pytestmark = pytest.mark.gpu


def F():
    from wxx_amd import functional

    return functional


def up(a):
    return F().from_numpy(np.asarray(a, np.float32))


def tol(K):
    # fp32 sums of K products of N(0,1) values: magnitudes ~ sqrt(K)
    return dict(rtol=1e-4, atol=1e-5 * max(1.0, np.sqrt(K)))


# (B, Cin, H, W, Cout, KH, KW, stride, padding, dilation): small ragged cases
# plus every distinct conv of ResNet18 at batch 128 on 32x32 inputs.
SMALL = [
    (1, 1, 1, 1, 1, 1, 1, (1, 1), (0, 0), (1, 1)),
    (2, 3, 9, 9, 4, 3, 3, (1, 1), (1, 1), (1, 1)),
    (2, 3, 11, 10, 5, 7, 7, (2, 2), (3, 3), (1, 1)),
    (1, 4, 8, 8, 6, 1, 1, (2, 2), (0, 0), (1, 1)),
    (2, 2, 12, 9, 3, 3, 2, (2, 1), (2, 0), (2, 3)),
    (3, 5, 4, 4, 2, 3, 3, (1, 1), (0, 0), (1, 1)),
    (2, 17, 13, 11, 70, 3, 3, (1, 1), (1, 1), (1, 1)),
    (4, 130, 5, 6, 129, 3, 3, (2, 2), (1, 1), (1, 1)),
]
RESNET18 = [
    (128, 3, 32, 32, 64, 7, 7, (2, 2), (3, 3), (1, 1)),
    (128, 64, 8, 8, 64, 3, 3, (1, 1), (1, 1), (1, 1)),
    (128, 64, 8, 8, 128, 3, 3, (2, 2), (1, 1), (1, 1)),
    (128, 64, 8, 8, 128, 1, 1, (2, 2), (0, 0), (1, 1)),
    (128, 128, 4, 4, 128, 3, 3, (1, 1), (1, 1), (1, 1)),
    (128, 128, 4, 4, 256, 3, 3, (2, 2), (1, 1), (1, 1)),
    (128, 256, 2, 2, 256, 3, 3, (1, 1), (1, 1), (1, 1)),
    (128, 256, 2, 2, 512, 3, 3, (2, 2), (1, 1), (1, 1)),
    (128, 512, 1, 1, 512, 3, 3, (1, 1), (1, 1), (1, 1)),
]


def _run_conv(case, seed, bias):
    B, Cin, H, W, Cout, KH, KW, s, p, d = case
    r = rng(seed)
    X = r.standard_normal((B, Cin, H, W)).astype(np.float32)
    Wt = r.standard_normal((Cout, Cin, KH, KW)).astype(np.float32)
    b = r.standard_normal(Cout).astype(np.float32) if bias else None
    y = F().conv2d(up(X), up(Wt), s, p, d, up(b) if bias else None)
    ey = oc.conv2d(X, Wt, s, p, d, b)
    assert y.shape == list(ey.shape)
    assert_error_floor(y.numpy(), ey, oc.conv2d(X, Wt, s, p, d, b, np.float32), msg="conv2d")
    g = r.standard_normal(ey.shape).astype(np.float32)
    dx = F().conv2ddx(up(g), up(Wt), s, p, d, X.shape, Wt.shape)
    assert_error_floor(dx.numpy(), oc.conv2ddx(g, Wt, s, p, d, X.shape),
                       oc.conv2ddx(g, Wt, s, p, d, X.shape, np.float32), msg="conv2ddx")
    dw = F().conv2ddw(up(g), up(X), s, p, d, X.shape, Wt.shape)
    assert_error_floor(dw.numpy(), oc.conv2ddw(g, X, s, p, d, Wt.shape),
                       oc.conv2ddw(g, X, s, p, d, Wt.shape, np.float32), msg="conv2ddw")


@pytest.mark.parametrize("case", SMALL)
@pytest.mark.parametrize("bias", [False, True])
def test_conv2d_small(device, case, bias):
    _run_conv(case, 1 + SMALL.index(case), bias)


@pytest.mark.parametrize("case", RESNET18)
def test_conv2d_resnet18_shapes(device, case):
    _run_conv(case, 100 + RESNET18.index(case), True)


# Kernels that reach past the input on every output: only their live taps
# run (the others read nothing but padding); dW is zero at the dead taps.
DEAD_TAPS = [
    (3, 6, 1, 1, 5, 3, 3, (1, 1), (1, 1), (1, 1)),    # 1 x 1 map: the centre tap only
    (2, 4, 2, 2, 3, 3, 3, (2, 2), (1, 1), (1, 1)),    # 2 x 2 -> 1 x 1: taps 1..2
    (2, 3, 1, 3, 4, 5, 3, (1, 1), (2, 1), (1, 1)),    # rows pruned, columns kept
    (1, 2, 2, 1, 3, 3, 5, (1, 2), (1, 2), (1, 1)),    # W = 1: column taps 2 only
    (2, 3, 1, 1, 2, 3, 3, (1, 1), (2, 2), (2, 2)),    # dilation 2, padding 2: tap 1
    (2, 5, 1, 2, 3, 4, 2, (1, 1), (2, 0), (1, 1)),    # even kernel, taps 2..2
]


@pytest.mark.parametrize("case", DEAD_TAPS)
def test_conv2d_dead_taps(device, case):
    _run_conv(case, 200 + DEAD_TAPS.index(case), True)
    B, Cin, H, W, Cout, KH, KW, s, p, d = case
    r = rng(300 + DEAD_TAPS.index(case))
    X = r.standard_normal((B, Cin, H, W)).astype(np.float32)
    Ho = (H + 2 * p[0] - d[0] * (KH - 1) - 1) // s[0] + 1
    Wo = (W + 2 * p[1] - d[1] * (KW - 1) - 1) // s[1] + 1
    g = r.standard_normal((B, Cout, Ho, Wo)).astype(np.float32)
    dw = F().conv2ddw(up(g), up(X), s, p, d, X.shape, (Cout, Cin, KH, KW)).numpy()
    ew = oc.conv2ddw(g, X, s, p, d, (Cout, Cin, KH, KW))
    dead = np.all(ew == 0, axis=(0, 1))  # taps no output reaches the input through
    assert dead.any()
    assert np.all(dw[:, :, dead] == 0)


def test_conv2d_strided_input_view(device):
    X = rng(3).standard_normal((2, 5, 6, 3)).astype(np.float32)  # NHWC on the host
    Wt = rng(4).standard_normal((4, 3, 3, 3)).astype(np.float32)
    xt = F().permute(up(X), 0, 3, 1, 2)  # (2, 3, 5, 6) non-contiguous view
    y = F().conv2d(xt, up(Wt), (1, 1), (1, 1), (1, 1))
    assert_close(y.numpy(), oc.conv2d(np.transpose(X, (0, 3, 1, 2)), Wt, (1, 1), (1, 1), (1, 1)),
                 **tol(27))


# ------------------------------------------------------------------ pooling


POOLS = [((128, 64, 16, 16), (3, 3), (2, 2), (1, 1)),  # ResNet18 stem
         ((2, 3, 7, 9), (2, 3), (2, 1), (1, 1)),
         ((1, 1, 1, 2), (2, 1), (1, 1), (2, 0)),       # empty windows
         ((3, 2, 6, 6), (2, 2), (2, 2), (0, 0))]


@pytest.mark.parametrize("shape,k,s,p", POOLS)
def test_maxpool2d_bit_exact(device, shape, k, s, p):
    X = rng(5).standard_normal(shape).astype(np.float32)
    X[0, 0, 0, :2] = 1.5  # a tie inside a window: first in scan order wins
    out, idx = F().maxpool2d(up(X), k, s, p, return_indices=True)
    eo, ei = oc.pool2d(X, k, s, p, avg=False)
    assert np.array_equal(out.numpy(), eo.astype(np.float32))
    assert np.array_equal(idx.numpy(), ei)
    only = F().maxpool2d(up(X), k, s, p)
    assert np.array_equal(only.numpy(), eo.astype(np.float32))
    g = rng(6).standard_normal(eo.shape).astype(np.float32)
    dx = F().maxpool2ddx(up(g), up(X), idx, k, s, p)
    assert_close(dx.numpy(), oc.pool2d_backward(g, ei, shape, k, s, p, avg=False),
                 rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("shape,k,s,p", POOLS)
def test_avgpool2d(device, shape, k, s, p):
    X = rng(7).standard_normal(shape).astype(np.float32)
    out, idx = F().avgpool2d(up(X), k, s, p, return_indices=True)
    eo, ei = oc.pool2d(X, k, s, p, avg=True)
    assert_close(out.numpy(), eo, rtol=1e-6, atol=1e-6)
    assert np.array_equal(idx.numpy(), ei)
    g = rng(8).standard_normal(eo.shape).astype(np.float32)
    dx = F().avgpool2ddx(up(g), up(X), k, s, p)
    assert_close(dx.numpy(), oc.pool2d_backward(g, None, shape, k, s, p, avg=True),
                 rtol=1e-5, atol=1e-6)


def test_pool1d(device):
    X = rng(9).standard_normal((3, 4, 29)).astype(np.float32)
    out, idx = F().maxpool1d(up(X), 3, (2,), 1, return_indices=True)
    eo, ei = oc.pool2d(X[:, :, None, :], (1, 3), (1, 2), (0, 1), avg=False)
    assert np.array_equal(out.numpy(), eo[:, :, 0].astype(np.float32))
    assert np.array_equal(idx.numpy(), ei[:, :, 0])
    g = rng(10).standard_normal(out.shape).astype(np.float32)
    dx = F().maxpool1ddx(up(g), up(X), idx, 3, 2, 1)
    assert_close(dx.numpy(), oc.pool2d_backward(g[:, :, None], ei, (3, 4, 1, 29), (1, 3), (1, 2),
                                                (0, 1), avg=False)[:, :, 0], rtol=1e-6, atol=1e-6)
    a = F().avgpool1d(up(X), 4, 3, 2)
    ea, _ = oc.pool2d(X[:, :, None, :], (1, 4), (1, 3), (0, 2), avg=True)
    assert_close(a.numpy(), ea[:, :, 0], rtol=1e-6, atol=1e-6)
    ga = rng(11).standard_normal(a.shape).astype(np.float32)
    da = F().avgpool1ddx(up(ga), up(X), 4, 3, 2)
    assert_close(da.numpy(), oc.pool2d_backward(ga[:, :, None], None, (3, 4, 1, 29), (1, 4),
                                                (1, 3), (0, 2), avg=True)[:, :, 0],
                 rtol=1e-5, atol=1e-6)
    with pytest.raises(ValueError):
        F().maxpool1d(up(X), (3, 3), 1, 0)
    with pytest.raises(ValueError):
        F().maxpool2d(up(X[:, :, None, :2]), (1, 5), (1, 1), (0, 0))


@pytest.mark.parametrize("shape,out", [((128, 512, 1, 1), (1, 1)), ((2, 3, 8, 6), (2, 3)),
                                       ((2, 3, 5, 5), (3, 3)), ((1, 2, 4, 4), 1)])
def test_adaptive_avgpool2d(device, shape, out):
    X = rng(12).standard_normal(shape).astype(np.float32)
    y = F().adaptive_avgpool2d(up(X), out)
    hw = (out, out) if isinstance(out, int) else out
    assert_close(y.numpy(), oc.adaptive_avgpool2d(X, hw), rtol=1e-6, atol=1e-6)
    g = rng(13).standard_normal(y.shape).astype(np.float32)
    dx = F().adaptive_avgpool2ddx(up(g), list(shape), out)
    assert_close(dx.numpy(), oc.adaptive_avgpool2ddx(g, shape), rtol=1e-6, atol=1e-6)


# -------------------------------------------------------- causal conv1d


@pytest.mark.parametrize("B,D,L,K,view", [(2, 5, 17, 3, False), (8, 256, 8192, 3, True),
                                           (1, 3, 2, 4, False),
                                           (3, 70, 130, 5, True),    # partial channel / position tiles
                                           (2, 65, 200, 8, False),   # largest tiled kernel size
                                           (2, 9, 40, 9, True),      # untiled kernels (K > 8)
                                           (2, 7, 36, 6, False),     # 16-byte dx, third load
                                           (3, 4, 12, 7, True),      # taps past the row end
                                           (5, 130, 64, 1, True)])
def test_causal_conv1d(device, B, D, L, K, view):
    r = rng(D)
    w = r.standard_normal((D, K)).astype(np.float32)
    b = r.standard_normal(D).astype(np.float32)
    if view:
        xh = r.standard_normal((B, L, D)).astype(np.float32)  # (B, L, D) -> (B, D, L) view
        xt = F().permute(up(xh), 0, 2, 1)
        x = np.transpose(xh, (0, 2, 1))
    else:
        x = r.standard_normal((B, D, L)).astype(np.float32)
        xt = up(x)
    y = F().causal_conv1d(xt, up(w), up(b))
    assert_close(y.numpy(), oc.causal_conv1d(x, w, b), rtol=1e-5, atol=1e-5)
    g = r.standard_normal((B, D, L)).astype(np.float32)
    dx, dw, db = F().causal_conv1d_backward(up(g), xt, up(w), up(b))
    ex, ew, eb = oc.causal_conv1d_backward(g, x, w)
    assert_close(dx.numpy(), ex, rtol=1e-5, atol=1e-5)
    assert_close(dw.numpy(), ew, **tol(B * L))
    assert_close(db.numpy(), eb, **tol(B * L))
    dx2, dw2, db2 = F().causal_conv1d_backward(up(g), xt, up(w), up(b), need_weight_grad=False)
    assert dw2 is None and db2 is None
    assert np.array_equal(dx2.numpy(), dx.numpy())


# --------------------------------------------------- transposed convolution

TCONV = [
    (2, 3, 5, 4, 4, 3, 3, (2, 2), (1, 1), (1, 1), (1, 0)),
    (1, 2, 3, 3, 5, 2, 2, (2, 2), (0, 0), (1, 1), (0, 0)),
    (2, 4, 4, 5, 3, 3, 2, (1, 2), (1, 0), (2, 1), (1, 1)),
    (8, 64, 8, 8, 32, 4, 4, (2, 2), (1, 1), (1, 1), (0, 0)),
]


@pytest.mark.parametrize("case", TCONV)
def test_conv2dtranspose(device, case):
    B, Cin, H, W, Cout, KH, KW, s, p, d, op = case
    r = rng(Cin * 31 + Cout)
    X = r.standard_normal((B, Cin, H, W)).astype(np.float32)
    Wt = r.standard_normal((Cin, Cout, KH, KW)).astype(np.float32)
    b = r.standard_normal(Cout).astype(np.float32)
    y = F().conv2dtranspose(up(X), up(Wt), s, p, d, op, up(b))
    Ho = (H - 1) * s[0] - 2 * p[0] + d[0] * (KH - 1) + op[0] + 1
    Wo = (W - 1) * s[1] - 2 * p[1] + d[1] * (KW - 1) + op[1] + 1
    assert y.shape == [B, Cout, Ho, Wo]
    assert_close(y.numpy(), oc.conv2dtranspose(X, Wt, s, p, d, (Ho, Wo), b), **tol(Cin * KH * KW))
    g = r.standard_normal((B, Cout, Ho, Wo)).astype(np.float32)
    dx = F().conv2dtranspose_dx(up(g), up(Wt), s, p, d, X.shape, Wt.shape, y.shape)
    assert_close(dx.numpy(), oc.conv2dtranspose_dx(g, Wt, s, p, d, X.shape),
                 **tol(Cout * KH * KW))
    dw = F().conv2dtranspose_dw(up(g), up(X), s, p, d, y.shape, Wt.shape)
    assert_close(dw.numpy(), oc.conv2dtranspose_dw(g, X, s, p, d, Wt.shape), **tol(B * H * W))
    with pytest.raises(ValueError):
        F().conv2dtranspose(up(X), up(Wt), s, p, d, (max(s[0], d[0]), 0))


# ---------------------------------------------------------------- autograd


def test_conv_pool_autograd_graph(device):
    """conv -> maxpool -> conv (no bias) -> adaptive avgpool -> sum, backward."""
    from wxx_amd import autograd

    r = rng(77)
    X = r.standard_normal((4, 3, 12, 12)).astype(np.float32)
    W1 = r.standard_normal((8, 3, 3, 3)).astype(np.float32)
    b1 = r.standard_normal(8).astype(np.float32)
    W2 = r.standard_normal((5, 8, 3, 3)).astype(np.float32)
    tx, tw1, tb1, tw2 = up(X), up(W1), up(b1), up(W2)
    for t in (tx, tw1, tb1, tw2):
        t.requires_grad = True
    y1 = autograd.Conv2D(tx, tw1, tb1).forward(tx, tw1, tb1, (1, 1), (1, 1), (1, 1))
    y2 = autograd.maxpooling2d(y1).forward(y1, (3, 3), (2, 2), (1, 1))
    y3 = autograd.Conv2D(y2, tw2).forward(y2, tw2, None, (2, 2), (1, 1), (1, 1))
    y4 = autograd.adaptive_avgpooling2d(y3).forward(y3, (1, 1))
    loss = y4.sum()
    loss.backward()
    # oracle chain, float64, with the same maxpool routing
    e1 = oc.conv2d(X, W1, (1, 1), (1, 1), (1, 1), b1)
    e2, i2 = oc.pool2d(e1.astype(np.float32), (3, 3), (2, 2), (1, 1), avg=False)
    e3 = oc.conv2d(e2, W2, (2, 2), (1, 1), (1, 1))
    g4 = np.ones((4, 5, 1, 1))
    g3 = oc.adaptive_avgpool2ddx(g4, e3.shape)
    gw2 = oc.conv2ddw(g3, e2, (2, 2), (1, 1), (1, 1), W2.shape)
    g2 = oc.conv2ddx(g3, W2, (2, 2), (1, 1), (1, 1), e2.shape)
    g1 = oc.pool2d_backward(g2, i2, e1.shape, (3, 3), (2, 2), (1, 1), avg=False)
    gw1 = oc.conv2ddw(g1, X, (1, 1), (1, 1), (1, 1), W1.shape)
    gx = oc.conv2ddx(g1, W1, (1, 1), (1, 1), (1, 1), X.shape)
    assert_close(loss.numpy(), np.array(e3.mean(axis=(2, 3)).sum(), np.float32).reshape(1),
                 rtol=1e-4, atol=1e-3)
    assert_close(tw2.grad.numpy(), gw2, **tol(4 * 36))
    assert_close(tw1.grad.numpy(), gw1, **tol(4 * 144))
    assert_close(tb1.grad.numpy(), g1.sum(axis=(0, 2, 3)), **tol(4 * 144))
    assert_close(tx.grad.numpy(), gx, **tol(8 * 9))
