"""Pin the oracle's convolution / pooling restatements (CPU-only).

Independent checks: torch's CPU conv2d / pooling / conv1d and their autograd
adjoints (float64), a seven-loop brute-force convolution, and hand-worked
window cases for the reference's pooling rules (empty windows, flat indices).
"""

import numpy as np
import pytest

from conftest import assert_close, rng
from oracle import conv as oc

torch = pytest.importorskip("torch")
TF = torch.nn.functional

CONV_CASES = [
    # (B, Cin, H, W, Cout, KH, KW, stride, padding, dilation)
    (2, 3, 9, 9, 4, 3, 3, (1, 1), (1, 1), (1, 1)),
    (2, 3, 11, 10, 5, 7, 7, (2, 2), (3, 3), (1, 1)),
    (1, 4, 8, 8, 6, 1, 1, (2, 2), (0, 0), (1, 1)),
    (2, 2, 12, 9, 3, 3, 2, (2, 1), (2, 0), (2, 3)),
    (3, 5, 4, 4, 2, 3, 3, (1, 1), (0, 0), (1, 1)),
]


def _t(a, grad=False):
    return torch.tensor(np.asarray(a, np.float64), requires_grad=grad)


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv2d_and_gradients_match_torch(case):
    B, Cin, H, W, Cout, KH, KW, s, p, d = case
    X = rng(1).standard_normal((B, Cin, H, W))
    Wt = rng(2).standard_normal((Cout, Cin, KH, KW))
    b = rng(3).standard_normal(Cout)
    y = oc.conv2d(X, Wt, s, p, d, b)
    tx, tw, tb = _t(X, True), _t(Wt, True), _t(b, True)
    ty = TF.conv2d(tx, tw, tb, stride=s, padding=p, dilation=d)
    assert_close(y, ty.detach().numpy(), rtol=1e-12, atol=1e-12)
    g = rng(4).standard_normal(y.shape)
    ty.backward(_t(g))
    assert_close(oc.conv2ddx(g, Wt, s, p, d, X.shape), tx.grad.numpy(), rtol=1e-12, atol=1e-12)
    assert_close(oc.conv2ddw(g, X, s, p, d, Wt.shape), tw.grad.numpy(), rtol=1e-12, atol=1e-12)


def test_conv2d_brute_force_loops():
    B, Cin, H, W, Cout, KH, KW = 1, 2, 5, 6, 3, 3, 2
    s, p, d = (2, 1), (1, 1), (1, 2)
    X = rng(5).standard_normal((B, Cin, H, W))
    Wt = rng(6).standard_normal((Cout, Cin, KH, KW))
    y = oc.conv2d(X, Wt, s, p, d)
    Ho, Wo = oc.conv_out(H, W, KH, KW, s, p, d)
    ref = np.zeros((B, Cout, Ho, Wo))
    for b in range(B):
        for co in range(Cout):
            for oh in range(Ho):
                for ow in range(Wo):
                    acc = 0.0
                    for ci in range(Cin):
                        for kh in range(KH):
                            for kw in range(KW):
                                ih = oh * s[0] - p[0] + kh * d[0]
                                iw = ow * s[1] - p[1] + kw * d[1]
                                if 0 <= ih < H and 0 <= iw < W:
                                    acc += X[b, ci, ih, iw] * Wt[co, ci, kh, kw]
                    ref[b, co, oh, ow] = acc
    assert_close(y, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("shape,k,s,p", [((2, 3, 16, 16), (3, 3), (2, 2), (1, 1)),
                                          ((1, 2, 7, 9), (2, 3), (2, 1), (1, 1)),
                                          ((2, 2, 6, 6), (2, 2), (2, 2), (0, 0))])
def test_pools_match_torch(shape, k, s, p):
    X = rng(7).standard_normal(shape).astype(np.float32)
    B, C, H, W = shape
    out, idx = oc.pool2d(X, k, s, p, avg=False)
    tx = _t(X, True)
    ty, ti = TF.max_pool2d(tx, k, s, p, return_indices=True)
    assert_close(out, ty.detach().numpy(), rtol=0, atol=0)
    plane = (np.arange(B)[:, None] * C + np.arange(C)[None, :]) * H * W
    assert np.array_equal(idx.astype(np.int64), ti.numpy() + plane[:, :, None, None])
    g = rng(8).standard_normal(out.shape)
    ty.backward(_t(g))
    assert_close(oc.pool2d_backward(g, idx, shape, k, s, p, avg=False), tx.grad.numpy(),
                 rtol=1e-12, atol=1e-12)
    aout, _ = oc.pool2d(X, k, s, p, avg=True)
    tx2 = _t(X, True)
    ta = TF.avg_pool2d(tx2, k, s, p, count_include_pad=False)
    assert_close(aout, ta.detach().numpy(), rtol=1e-12, atol=1e-12)
    ta.backward(_t(g))
    assert_close(oc.pool2d_backward(g, None, shape, k, s, p, avg=True), tx2.grad.numpy(),
                 rtol=1e-12, atol=1e-12)


def test_pool_empty_window_and_flat_index():
    # H = 1, kernel 2, padding 2: output row 0 covers input rows -2..-1 only
    X = np.array([[[[5.0, -1.0]]]], np.float32)
    out, idx = oc.pool2d(X, (2, 1), (1, 1), (2, 0), avg=False)
    assert out.shape == (1, 1, 4, 2)
    assert out[0, 0, 0, 0] == np.float32(-1e38) and idx[0, 0, 0, 0] == 0xFFFFFFFF
    assert out[0, 0, 2, 0] == 5.0 and idx[0, 0, 2, 0] == 0
    assert idx[0, 0, 2, 1] == 1
    aout, _ = oc.pool2d(X, (2, 1), (1, 1), (2, 0), avg=True)
    assert aout[0, 0, 0, 0] == 0.0
    # second image / channel: indices are flat over (B, C, H, W)
    X2 = rng(9).standard_normal((2, 3, 2, 2)).astype(np.float32)
    _, idx2 = oc.pool2d(X2, (2, 2), (2, 2), (0, 0), avg=False)
    for b in range(2):
        for c in range(3):
            assert idx2[b, c, 0, 0] == (b * 3 + c) * 4 + int(np.argmax(X2[b, c]))


@pytest.mark.parametrize("hw,out", [((4, 4), (1, 1)), ((8, 6), (2, 3)), ((5, 7), (5, 7)),
                                    ((5, 5), (3, 3))])
def test_adaptive_avgpool_matches_torch(hw, out):
    X = rng(10).standard_normal((2, 3) + hw)
    tx = _t(X, True)
    ty = TF.adaptive_avg_pool2d(tx, out)
    assert_close(oc.adaptive_avgpool2d(X, out), ty.detach().numpy(), rtol=1e-12, atol=1e-12)
    g = rng(11).standard_normal(ty.shape)
    ty.backward(_t(g))
    assert_close(oc.adaptive_avgpool2ddx(g, X.shape), tx.grad.numpy(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("B,D,L,K", [(2, 5, 17, 3), (1, 3, 2, 4)])
def test_causal_conv1d_matches_torch(B, D, L, K):
    x = rng(13).standard_normal((B, D, L))
    w = rng(14).standard_normal((D, K))
    b = rng(15).standard_normal(D)
    tx, tw, tb = _t(x, True), _t(w, True), _t(b, True)
    # y[n] = sum_k w[k] x[n-k]  ==  cross-correlation with the flipped kernel, left pad K-1
    ty = TF.conv1d(TF.pad(tx, (K - 1, 0)), torch.flip(tw, [1]).unsqueeze(1), tb, groups=D)
    assert_close(oc.causal_conv1d(x, w, b), ty.detach().numpy(), rtol=1e-12, atol=1e-12)
    g = rng(16).standard_normal((B, D, L))
    ty.backward(_t(g))
    dx, dw, db = oc.causal_conv1d_backward(g, x, w)
    assert_close(dx, tx.grad.numpy(), rtol=1e-12, atol=1e-12)
    assert_close(dw, tw.grad.numpy(), rtol=1e-12, atol=1e-12)
    assert_close(db, tb.grad.numpy(), rtol=1e-12, atol=1e-12)


TCONV_CASES = [
    # (B, Cin, H, W, Cout, KH, KW, stride, padding, dilation, output_padding)
    (2, 3, 5, 4, 4, 3, 3, (2, 2), (1, 1), (1, 1), (1, 0)),
    (1, 2, 3, 3, 5, 2, 2, (2, 2), (0, 0), (1, 1), (0, 0)),
    (2, 4, 4, 5, 3, 3, 2, (1, 2), (1, 0), (2, 1), (1, 1)),
]


@pytest.mark.parametrize("case", TCONV_CASES)
def test_conv2dtranspose_and_gradients_match_torch(case):
    B, Cin, H, W, Cout, KH, KW, s, p, d, op = case
    X = rng(20).standard_normal((B, Cin, H, W))
    Wt = rng(21).standard_normal((Cin, Cout, KH, KW))
    b = rng(22).standard_normal(Cout)
    tx, tw, tb = _t(X, True), _t(Wt, True), _t(b, True)
    ty = TF.conv_transpose2d(tx, tw, tb, stride=s, padding=p, output_padding=op, dilation=d)
    Ho = (H - 1) * s[0] - 2 * p[0] + d[0] * (KH - 1) + op[0] + 1
    Wo = (W - 1) * s[1] - 2 * p[1] + d[1] * (KW - 1) + op[1] + 1
    assert tuple(ty.shape[2:]) == (Ho, Wo)
    y = oc.conv2dtranspose(X, Wt, s, p, d, (Ho, Wo), b)
    assert_close(y, ty.detach().numpy(), rtol=1e-12, atol=1e-12)
    g = rng(23).standard_normal(y.shape)
    ty.backward(_t(g))
    assert_close(oc.conv2dtranspose_dx(g, Wt, s, p, d, X.shape), tx.grad.numpy(),
                 rtol=1e-12, atol=1e-12)
    assert_close(oc.conv2dtranspose_dw(g, X, s, p, d, Wt.shape), tw.grad.numpy(),
                 rtol=1e-12, atol=1e-12)
