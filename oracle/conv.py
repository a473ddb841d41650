"""2-D convolution, pooling and depthwise causal conv1d restated from the
reference (test infrastructure only), in float64.

* conv2d (shaders/layers/conv2d.wgsl:33-111): im2col row
  (b, oh, ow) x column (ci, kh, kw) with ih = oh sh - ph + kh dh (zero outside),
  times W reshaped (Cout, Cin KH KW), plus bias; output NCHW with
  Ho = (H + 2 ph - dh (KH - 1) - 1) // sh + 1 (functional/convolution.py:679-680).
* conv2ddx (conv2ddx.wgsl:33-118): dX[b,ci,ih,iw] = sum over (co, kh, kw) with
  th = ih + ph - kh dh >= 0, th % sh == 0, oh = th / sh < Ho (same along w) of
  dY[b,co,oh,ow] W[co,ci,kh,kw].
* conv2ddw (conv2ddw.wgsl + conv2ddw_reduce.wgsl): dW = dY (Cout, B Ho Wo) x im2col.
* pools (maxpool2d.wgsl, avgpool2d.wgsl, maxpool2ddx.wgsl, avgpool2ddx.wgsl,
  adaptive_avgpool2d*.wgsl): written as the reference's loops over a window
  (max from -1e38 with index 0xFFFFFFFF and strict '>', flat input index;
  average over in-range cells), and the backward gathers with the
  reference's truncating bounds.
* causal_conv1d (helpers/causal_conv1d*.wgsl): y[b,d,n] = bias[d] +
  sum_k w[d,k] x[b,d,n-k], and its three gradients.
"""

import numpy as np


def conv_out(H, W, KH, KW, stride, padding, dilation):
    sh, sw = stride
    ph, pw = padding
    dh, dw = dilation
    return (H + 2 * ph - dh * (KH - 1) - 1) // sh + 1, (W + 2 * pw - dw * (KW - 1) - 1) // sw + 1


def im2col(X, KH, KW, stride, padding, dilation, dtype=np.float64):
    """(B*Ho*Wo, Cin*KH*KW) patch matrix, zero outside the input."""
    X = np.asarray(X, dtype)
    B, Cin, H, W = X.shape
    sh, sw = stride
    ph, pw = padding
    dh, dw = dilation
    Ho, Wo = conv_out(H, W, KH, KW, stride, padding, dilation)
    Xp = np.zeros((B, Cin, H + 2 * ph + dh * KH + sh, W + 2 * pw + dw * KW + sw), dtype)
    Xp[:, :, ph:ph + H, pw:pw + W] = X
    cols = np.empty((B, Ho, Wo, Cin, KH, KW), dtype)
    for kh in range(KH):
        for kw in range(KW):
            h0, w0 = kh * dh, kw * dw
            patch = Xp[:, :, h0:h0 + sh * Ho:sh, w0:w0 + sw * Wo:sw]  # (B, Cin, Ho, Wo)
            cols[:, :, :, :, kh, kw] = patch.transpose(0, 2, 3, 1)
    return cols.reshape(B * Ho * Wo, Cin * KH * KW), (Ho, Wo)


def conv2d(X, Wt, stride, padding, dilation, bias=None, dtype=np.float64):
    """``dtype=np.float32`` evaluates the same sums in single precision (an
    fp32 BLAS product): the rounding a float32 evaluation carries, against
    which a device result's error is judged."""
    B = X.shape[0]
    Cout, Cin, KH, KW = Wt.shape
    cols, (Ho, Wo) = im2col(X, KH, KW, stride, padding, dilation, dtype)
    y = cols @ np.asarray(Wt, dtype).reshape(Cout, -1).T  # (B Ho Wo, Cout)
    if bias is not None:
        y = y + np.asarray(bias, dtype)[None, :]
    return y.reshape(B, Ho, Wo, Cout).transpose(0, 3, 1, 2)


def conv2ddx(dY, Wt, stride, padding, dilation, Xshape, dtype=np.float64):
    """Literal restatement of the conv2ddx gather (vectorised over b, ci)."""
    dY = np.asarray(dY, dtype)
    Wt = np.asarray(Wt, dtype)
    B, Cin, H, W = Xshape
    Cout, _, KH, KW = Wt.shape
    sh, sw = stride
    ph, pw = padding
    dh, dw = dilation
    Ho, Wo = dY.shape[2], dY.shape[3]
    dX = np.zeros((B, Cin, H, W), dtype)
    for kh in range(KH):
        for kw in range(KW):
            for ih in range(H):
                th = ih + ph - kh * dh
                if th < 0 or th % sh or th // sh >= Ho:
                    continue
                oh = th // sh
                for iw in range(W):
                    tw = iw + pw - kw * dw
                    if tw < 0 or tw % sw or tw // sw >= Wo:
                        continue
                    ow = tw // sw
                    dX[:, :, ih, iw] += dY[:, :, oh, ow] @ Wt[:, :, kh, kw]
    return dX


def conv2ddw(dY, X, stride, padding, dilation, wshape, dtype=np.float64):
    Cout, Cin, KH, KW = wshape
    cols, _ = im2col(X, KH, KW, stride, padding, dilation, dtype)
    g = np.asarray(dY, dtype).transpose(0, 2, 3, 1).reshape(-1, Cout)
    return (g.T @ cols).reshape(wshape)


def pool2d(X, kernel, stride, padding, avg):
    """(out, flat indices) of the reference's max / average pooling loop."""
    X = np.asarray(X, np.float32)
    B, C, H, W = X.shape
    KH, KW = kernel
    sh, sw = stride
    ph, pw = padding
    Ho = (H + 2 * ph - KH) // sh + 1
    Wo = (W + 2 * pw - KW) // sw + 1
    flat = X.reshape(-1)
    base = (np.arange(B)[:, None] * C + np.arange(C)[None, :]) * H * W  # (B, C)
    best = np.full((B, C, Ho, Wo), -1e38, np.float32)
    bidx = np.full((B, C, Ho, Wo), 0xFFFFFFFF, np.uint64)
    ssum = np.zeros((B, C, Ho, Wo), np.float64)
    cnt = np.zeros((Ho, Wo), np.float64)
    for ho in range(Ho):
        for wo in range(Wo):
            for kh in range(KH):
                ih = ho * sh - ph + kh
                if ih < 0 or ih >= H:
                    continue
                for kw in range(KW):
                    iw = wo * sw - pw + kw
                    if iw < 0 or iw >= W:
                        continue
                    idx = base + ih * W + iw
                    v = flat[idx]
                    ssum[:, :, ho, wo] += v
                    cnt[ho, wo] += 1
                    upd = v > best[:, :, ho, wo]
                    best[:, :, ho, wo] = np.where(upd, v, best[:, :, ho, wo])
                    bidx[:, :, ho, wo] = np.where(upd, idx, bidx[:, :, ho, wo])
    if avg:
        out = np.where(cnt > 0, ssum / np.maximum(cnt, 1), 0.0)
    else:
        out = best.astype(np.float64)
    return out, bidx.astype(np.uint32)


def _out_range(i, p, k, s, n_out):
    ip = i + p
    lo = max(0, int((ip - k + s) / s))  # truncating division, as WGSL i32 '/'
    hi = min(n_out - 1, ip // s)
    return lo, hi


def pool2d_backward(dY, idx, Xshape, kernel, stride, padding, avg):
    dY = np.asarray(dY, np.float64)
    B, C, H, W = Xshape
    KH, KW = kernel
    sh, sw = stride
    ph, pw = padding
    Ho, Wo = dY.shape[2], dY.shape[3]
    dX = np.zeros((B, C, H, W))
    base = (np.arange(B)[:, None] * C + np.arange(C)[None, :]) * H * W
    for ih in range(H):
        hlo, hhi = _out_range(ih, ph, KH, sh, Ho)
        for iw in range(W):
            wlo, whi = _out_range(iw, pw, KW, sw, Wo)
            acc = np.zeros((B, C))
            for ho in range(hlo, hhi + 1):
                for wo in range(wlo, whi + 1):
                    if avg:
                        hs, ws = ho * sh - ph, wo * sw - pw
                        n = (min(H, hs + KH) - max(0, hs)) * (min(W, ws + KW) - max(0, ws))
                        if n > 0:
                            acc += dY[:, :, ho, wo] / n
                    else:
                        hit = idx[:, :, ho, wo].astype(np.int64) == base + ih * W + iw
                        acc += np.where(hit, dY[:, :, ho, wo], 0.0)
            dX[:, :, ih, iw] = acc
    return dX


def adaptive_avgpool2d(X, out_hw):
    X = np.asarray(X, np.float64)
    B, C, H, W = X.shape
    Ho, Wo = out_hw
    y = np.zeros((B, C, Ho, Wo))
    for oh in range(Ho):
        hs, he = (oh * H) // Ho, ((oh + 1) * H + Ho - 1) // Ho
        for ow in range(Wo):
            ws, we = (ow * W) // Wo, ((ow + 1) * W + Wo - 1) // Wo
            y[:, :, oh, ow] = X[:, :, hs:he, ws:we].sum(axis=(2, 3)) / ((he - hs) * (we - ws))
    return y


def adaptive_avgpool2ddx(dY, Xshape):
    dY = np.asarray(dY, np.float64)
    B, C, H, W = Xshape
    Ho, Wo = dY.shape[2], dY.shape[3]
    dX = np.zeros((B, C, H, W))
    for ih in range(H):
        ohs, ohe = (ih * Ho) // H, ((ih + 1) * Ho - 1) // H
        for iw in range(W):
            ows, owe = (iw * Wo) // W, ((iw + 1) * Wo - 1) // W
            for oh in range(ohs, ohe + 1):
                hs, he = (oh * H) // Ho, ((oh + 1) * H + Ho - 1) // Ho
                for ow in range(ows, owe + 1):
                    ws, we = (ow * W) // Wo, ((ow + 1) * W + Wo - 1) // Wo
                    dX[:, :, ih, iw] += dY[:, :, oh, ow] / ((he - hs) * (we - ws))
    return dX


def causal_conv1d(x, w, bias):
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    B, D, L = x.shape
    y = np.broadcast_to(np.asarray(bias, np.float64)[None, :, None], (B, D, L)).copy()
    for k in range(min(w.shape[1], L)):
        y[:, :, k:] += w[None, :, k, None] * x[:, :, :L - k]
    return y


def causal_conv1d_backward(dy, x, w):
    dy = np.asarray(dy, np.float64)
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    B, D, L = x.shape
    dx = np.zeros_like(x)
    dw = np.zeros_like(w)
    for k in range(min(w.shape[1], L)):
        dx[:, :, :L - k] += w[None, :, k, None] * dy[:, :, k:]
        dw[:, k] = (dy[:, :, k:] * x[:, :, :L - k]).sum(axis=(0, 2))
    return dx, dw, dy.sum(axis=(0, 2))


def conv2dtranspose(X, Wt, stride, padding, dilation, out_hw, bias=None):
    """Transposed conv (shaders/layers/conv2dtranspose.wgsl): the scatter of every
    input cell (b, ci, h, w) times W[ci, co, kh, kw] to output
    (h sh - ph + kh dh, w sw - pw + kw dw), written as a direct loop."""
    X = np.asarray(X, np.float64)
    Wt = np.asarray(Wt, np.float64)
    B, Cin, H, W = X.shape
    _, Cout, KH, KW = Wt.shape
    sh, sw = stride
    ph, pw = padding
    dh, dw = dilation
    Ho, Wo = out_hw
    y = np.zeros((B, Cout, Ho, Wo))
    for kh in range(KH):
        for kw in range(KW):
            for h in range(H):
                oh = h * sh - ph + kh * dh
                if oh < 0 or oh >= Ho:
                    continue
                for w in range(W):
                    ow = w * sw - pw + kw * dw
                    if ow < 0 or ow >= Wo:
                        continue
                    y[:, :, oh, ow] += X[:, :, h, w] @ Wt[:, :, kh, kw]
    if bias is not None:
        y += np.asarray(bias, np.float64)[None, :, None, None]
    return y


def conv2dtranspose_dx(dY, Wt, stride, padding, dilation, Xshape, dtype=np.float64):
    """dX[b,ci,h,w] = sum_{co,kh,kw} dY[b,co,h sh - ph + kh dh, ...] W[ci,co,kh,kw]."""
    dY = np.asarray(dY, dtype)
    Wt = np.asarray(Wt, dtype)
    B, Cin, H, W = Xshape
    _, Cout, KH, KW = Wt.shape
    sh, sw = stride
    ph, pw = padding
    dh, dw = dilation
    Ho, Wo = dY.shape[2], dY.shape[3]
    dX = np.zeros((B, Cin, H, W), dtype)
    for kh in range(KH):
        for kw in range(KW):
            for h in range(H):
                oh = h * sh - ph + kh * dh
                if oh < 0 or oh >= Ho:
                    continue
                for w in range(W):
                    ow = w * sw - pw + kw * dw
                    if ow < 0 or ow >= Wo:
                        continue
                    dX[:, :, h, w] += dY[:, :, oh, ow] @ Wt[:, :, kh, kw].T
    return dX


def conv2dtranspose_dw(dY, X, stride, padding, dilation, wshape):
    """dW[ci,co,kh,kw] = sum_{b,h,w} X[b,ci,h,w] dY[b,co,h sh - ph + kh dh, ...]."""
    dY = np.asarray(dY, np.float64)
    X = np.asarray(X, np.float64)
    Cin, Cout, KH, KW = wshape
    B, _, H, W = X.shape
    sh, sw = stride
    ph, pw = padding
    dh, dw = dilation
    Ho, Wo = dY.shape[2], dY.shape[3]
    dW = np.zeros(wshape)
    for kh in range(KH):
        for kw in range(KW):
            for h in range(H):
                oh = h * sh - ph + kh * dh
                if oh < 0 or oh >= Ho:
                    continue
                for w in range(W):
                    ow = w * sw - pw + kw * dw
                    if ow < 0 or ow >= Wo:
                        continue
                    dW[:, :, kh, kw] += X[:, :, h, w].T @ dY[:, :, oh, ow]
    return dW
