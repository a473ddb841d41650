"""2-D convolution, pooling and the depthwise causal conv1d (reference
src/wxx/functional/convolution.py).  Same signatures, argument meaning and
host-side errors as the reference; each op is one call into libwxx_hip.so."""

import ctypes as C

from .. import validation
from ._common import call, empty, ptr


def _as_pool1d_int(value, name):
    """An int or a 1-tuple, as the reference accepts (convolution.py:24-38)."""
    if isinstance(value, bool):
        raise TypeError(f"{name} must be an int, got {type(value).__name__}")
    if isinstance(value, int):
        return value
    if isinstance(value, (tuple, list)):
        if len(value) != 1:
            raise ValueError(f"{name} must be an int or a 1-tuple, got {value!r}")
        if isinstance(value[0], bool) or not isinstance(value[0], int):
            raise TypeError(f"{name}[0] must be an int, got {type(value[0]).__name__}")
        return value[0]
    raise TypeError(f"{name} must be an int or a 1-tuple, got {value!r}")


def _check_pool_input(tensor1, rank, name):
    if len(tensor1.shape) != rank:
        expected = "(B, C, L)" if rank == 3 else "(B, C, H, W)"
        raise ValueError(f"{name} expects {expected}, got {tensor1.shape}")
    if tensor1.type != "f32":
        raise TypeError(f"{name} expects f32 input, got {tensor1.type!r}")


def _check_pool_out(shape):
    if any(size < 1 for size in shape):
        raise ValueError(f"pooling produces an empty output {tuple(shape)}")


def _pool_out(H, W, KH, KW, sh, sw, ph, pw):
    Ho = (H + 2 * ph - KH) // sh + 1
    Wo = (W + 2 * pw - KW) // sw + 1
    _check_pool_out((Ho, Wo))
    return Ho, Wo


def _pool2d(tensor1, kernel, stride, padding, return_indices, avg, name):
    _check_pool_input(tensor1, 4, name)
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    B, Cc, H, W = tensor1.shape
    KH, KW = kernel
    sh, sw = stride
    ph, pw = padding
    Ho, Wo = _pool_out(H, W, KH, KW, sh, sw, ph, pw)
    out = empty((B, Cc, Ho, Wo))
    idx = empty((B, Cc, Ho, Wo), dtype="u32") if return_indices else None
    call("wxx_pool2d", ptr(tensor1), ptr(out), ptr(idx) if idx is not None else None, B, Cc, H,
         W, KH, KW, sh, sw, ph, pw, int(avg))
    return (out, idx) if return_indices else out


def _pool1d(tensor1, kernel, stride, padding, return_indices, avg, name):
    _check_pool_input(tensor1, 3, name)
    kernel = _as_pool1d_int(kernel, "kernel")
    stride = _as_pool1d_int(stride, "stride")
    padding = _as_pool1d_int(padding, "padding")
    if kernel < 1 or stride < 1 or padding < 0:
        raise ValueError(
            f"{name} expects kernel >= 1, stride >= 1, padding >= 0, got "
            f"kernel={kernel}, stride={stride}, padding={padding}"
        )
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    B, Cc, L = tensor1.shape
    Lo = (L + 2 * padding - kernel) // stride + 1
    _check_pool_out((Lo,))
    out = empty((B, Cc, Lo))
    idx = empty((B, Cc, Lo), dtype="u32") if return_indices else None
    call("wxx_pool2d", ptr(tensor1), ptr(out), ptr(idx) if idx is not None else None, B, Cc, 1,
         L, 1, kernel, 1, stride, 0, padding, int(avg))
    return (out, idx) if return_indices else out


def maxpool2d(tensor1, kernel, stride, padding, return_indices=False):
    """Max pooling over ``(B, C, H, W)``; with ``return_indices`` also the u32
    flat input index of every window's maximum (reference convolution.py:60-125)."""
    return _pool2d(tensor1, kernel, stride, padding, return_indices, False, "maxpool2d")


def avgpool2d(tensor1, kernel, stride, padding, return_indices=False):
    """Average pooling over ``(B, C, H, W)``, padded cells excluded from the
    divisor (reference convolution.py:128-192)."""
    return _pool2d(tensor1, kernel, stride, padding, return_indices, True, "avgpool2d")


def avgpool1d(tensor1, kernel, stride, padding, return_indices=False):
    """Average pooling over ``(B, C, L)`` (reference convolution.py:195-257)."""
    return _pool1d(tensor1, kernel, stride, padding, return_indices, True, "avgpool1d")


def maxpool1d(tensor1, kernel, stride, padding, return_indices=False):
    """Max pooling over ``(B, C, L)`` (reference convolution.py:260-321)."""
    return _pool1d(tensor1, kernel, stride, padding, return_indices, False, "maxpool1d")


def maxpool1ddx(grad, tensor1, indices, kernel, stride, padding):
    """Backward of :func:`maxpool1d` through ``indices`` (reference convolution.py:324-372)."""
    if not grad.is_contiguous():
        grad = grad.contiguous()
    B, Cc, L = tensor1.shape
    kernel = _as_pool1d_int(kernel, "kernel")
    stride = _as_pool1d_int(stride, "stride")
    padding = _as_pool1d_int(padding, "padding")
    Lo = (L + 2 * padding - kernel) // stride + 1
    _check_pool_out((Lo,))
    out = empty((B, Cc, L))
    call("wxx_pool2d_backward", ptr(grad), ptr(indices), ptr(out), B, Cc, 1, L, 1, kernel, 1,
         stride, 0, padding, 0)
    return out


def avgpool1ddx(grad, tensor1, kernel, stride, padding):
    """Backward of :func:`avgpool1d` (reference convolution.py:375-422)."""
    if not grad.is_contiguous():
        grad = grad.contiguous()
    B, Cc, L = tensor1.shape
    kernel = _as_pool1d_int(kernel, "kernel")
    stride = _as_pool1d_int(stride, "stride")
    padding = _as_pool1d_int(padding, "padding")
    Lo = (L + 2 * padding - kernel) // stride + 1
    _check_pool_out((Lo,))
    out = empty((B, Cc, L))
    call("wxx_pool2d_backward", ptr(grad), None, ptr(out), B, Cc, 1, L, 1, kernel, 1, stride, 0,
         padding, 1)
    return out


def avgpool2ddx(grad, tensor1, kernel, stride, padding):
    """Backward of :func:`avgpool2d` (reference convolution.py:425-476)."""
    if not grad.is_contiguous():
        grad = grad.contiguous()
    B, Cc, H, W = tensor1.shape
    KH, KW = kernel
    sh, sw = stride
    ph, pw = padding
    _pool_out(H, W, KH, KW, sh, sw, ph, pw)
    out = empty((B, Cc, H, W))
    call("wxx_pool2d_backward", ptr(grad), None, ptr(out), B, Cc, H, W, KH, KW, sh, sw, ph, pw, 1)
    return out


def maxpool2ddx(grad, tensor1, indicies, kernel, stride, padding):
    """Backward of :func:`maxpool2d` through the saved indices (reference
    convolution.py:601-653)."""
    if not grad.is_contiguous():
        grad = grad.contiguous()
    B, Cc, H, W = tensor1.shape
    KH, KW = kernel
    sh, sw = stride
    ph, pw = padding
    _pool_out(H, W, KH, KW, sh, sw, ph, pw)
    out = empty((B, Cc, H, W))
    call("wxx_pool2d_backward", ptr(grad), ptr(indicies), ptr(out), B, Cc, H, W, KH, KW, sh, sw,
         ph, pw, 0)
    return out


def _normalize_output_size(output_size):
    if isinstance(output_size, int):
        output_size = (output_size, output_size)
    if len(output_size) != 2:
        raise ValueError(f"output_size must be an int or 2-tuple, got {output_size!r}")
    h_out, w_out = (int(output_size[0]), int(output_size[1]))
    if h_out < 1 or w_out < 1:
        raise ValueError(f"output_size entries must be positive, got {output_size!r}")
    return h_out, w_out


def adaptive_avgpool2d(tensor1, output_size):
    """Adaptive average pooling to ``output_size`` (reference convolution.py:490-543)."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if tensor1.type != "f32":
        raise TypeError(f"adaptive_avgpool2d expects f32 input, got {tensor1.type!r}")
    if validation.check_rank(tensor1.shape, name="adaptive_avgpool2d input") != 4:
        raise ValueError(f"adaptive_avgpool2d expects (B, C, H, W), got {tensor1.shape}")
    h_out, w_out = _normalize_output_size(output_size)
    B, Cc, H, W = tensor1.shape
    out = empty((B, Cc, h_out, w_out), requires_grad=tensor1.requires_grad)
    call("wxx_adaptive_avgpool2d", ptr(tensor1), ptr(out), B, Cc, H, W, h_out, w_out)
    return out


def adaptive_avgpool2ddx(grad, input_shape, output_size):
    """Backward of :func:`adaptive_avgpool2d` (reference convolution.py:546-598)."""
    if not grad.is_contiguous():
        grad = grad.contiguous()
    if grad.type != "f32":
        raise TypeError(f"adaptive_avgpool2ddx expects f32 grad, got {grad.type!r}")
    if validation.check_rank(input_shape, name="adaptive_avgpool2ddx input") != 4:
        raise ValueError(f"adaptive_avgpool2ddx expects a 4-D input shape, got {input_shape}")
    h_out, w_out = _normalize_output_size(output_size)
    B, Cc, H, W = input_shape
    expected = (B, Cc, h_out, w_out)
    if tuple(grad.shape) != expected:
        raise ValueError(
            f"adaptive_avgpool2ddx grad shape {tuple(grad.shape)} does not match "
            f"expected {expected}"
        )
    out = empty(input_shape)
    call("wxx_adaptive_avgpool2ddx", ptr(grad), ptr(out), B, Cc, H, W, h_out, w_out)
    return out


def _conv_dims(Xshape, wshape, stride, padding, dilation):
    B, Cin, H, W = Xshape
    Cout, _, KH, KW = wshape
    sh, sw = stride
    ph, pw = padding
    dh, dw = dilation
    return B, Cin, H, W, Cout, KH, KW, sh, sw, ph, pw, dh, dw


def _conv_out(H, W, KH, KW, sh, sw, ph, pw, dh, dw):
    return ((H + 2 * ph - dh * (KH - 1) - 1) // sh + 1,
            (W + 2 * pw - dw * (KW - 1) - 1) // sw + 1)


def conv2d(tensor1, W, stride, padding, dilation, bias=None):
    """NCHW convolution of ``tensor1`` (B, Cin, H, W) with ``W`` (Cout, Cin, KH, KW)
    plus an optional (Cout,) bias (reference convolution.py:658-729)."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if not W.is_contiguous():
        W = W.contiguous()
    if bias is not None and not bias.is_contiguous():
        bias = bias.contiguous()
    d = _conv_dims(tensor1.shape, W.shape, stride, padding, dilation)
    B, Cin, H, Wd, Cout, KH, KW, sh, sw, ph, pw, dh, dw = d
    Ho, Wo = _conv_out(H, Wd, KH, KW, sh, sw, ph, pw, dh, dw)
    out = empty((B, Cout, Ho, Wo), requires_grad=tensor1.requires_grad)
    call("wxx_conv2d", ptr(tensor1), ptr(W), ptr(bias) if bias is not None else None, ptr(out),
         *d)
    return out


def conv2ddx(tensor1, W, stride, padding, dilation, Xshape, wshape):
    """Input gradient of :func:`conv2d`; ``tensor1`` is dY (reference convolution.py:732-793)."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if not W.is_contiguous():
        W = W.contiguous()
    d = _conv_dims(Xshape, wshape, stride, padding, dilation)
    out = empty(tuple(Xshape), requires_grad=tensor1.requires_grad)
    call("wxx_conv2ddx", ptr(tensor1), ptr(W), ptr(out), *d)
    return out


def conv2ddw(tensor1, X, stride, padding, dilation, Xshape, wshape):
    """Weight gradient of :func:`conv2d`; ``tensor1`` is dY (reference convolution.py:796-908)."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if not X.is_contiguous():
        X = X.contiguous()
    d = _conv_dims(Xshape, wshape, stride, padding, dilation)
    out = empty(tuple(wshape), requires_grad=tensor1.requires_grad)
    call("wxx_conv2ddw", ptr(tensor1), ptr(X), ptr(out), *d)
    return out


def _tconv_dims(Xshape, wshape, stride, padding, dilation, out_shape):
    B, Cin, H, W = Xshape
    _, Cout, KH, KW = wshape
    sh, sw = stride
    ph, pw = padding
    dh, dw = dilation
    return (B, Cin, H, W, Cout, KH, KW, sh, sw, ph, pw, dh, dw, out_shape[2], out_shape[3])


def conv2dtranspose(tensor1, W, stride, padding, dilation, output_padding, bias=None):
    """Transposed 2-D convolution; ``W`` is (C_in, C_out, KH, KW) and the output
    size is (H_in - 1) * stride - 2 * padding + dilation * (K - 1) + output_padding + 1
    (reference convolution.py:911-1000)."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if not W.is_contiguous():
        W = W.contiguous()
    if bias is not None and not bias.is_contiguous():
        bias = bias.contiguous()
    B, C_in, H_in, W_in = tensor1.shape
    weight_in_c, C_out, KH, KW = W.shape
    if weight_in_c != C_in:
        raise ValueError(f"conv2dtranspose weight expects {C_in} input channels, got {weight_in_c}")
    sh, sw = stride
    ph, pw = padding
    dh, dw = dilation
    oph, opw = output_padding
    if not (0 <= oph < max(sh, dh)) or not (0 <= opw < max(sw, dw)):
        raise ValueError(
            f"output_padding {(oph, opw)} must be >= 0 and smaller than "
            f"max(stride, dilation) {(max(sh, dh), max(sw, dw))}"
        )
    H_out = (H_in - 1) * sh - 2 * ph + dh * (KH - 1) + oph + 1
    W_out = (W_in - 1) * sw - 2 * pw + dw * (KW - 1) + opw + 1
    if H_out < 1 or W_out < 1:
        raise ValueError(f"conv2dtranspose produces an empty output ({H_out}, {W_out})")
    out = empty((B, C_out, H_out, W_out), requires_grad=tensor1.requires_grad)
    d = _tconv_dims(tensor1.shape, W.shape, stride, padding, dilation, out.shape)
    call("wxx_conv2dtranspose", ptr(tensor1), ptr(W), ptr(bias) if bias is not None else None,
         ptr(out), *d)
    return out


def conv2dtranspose_dx(tensor1, W, stride, padding, dilation, Xshape, wshape, out_shape):
    """Input gradient of :func:`conv2dtranspose`; ``tensor1`` is dY
    (reference convolution.py:1003-1064)."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if not W.is_contiguous():
        W = W.contiguous()
    d = _tconv_dims(Xshape, wshape, stride, padding, dilation, out_shape)
    out = empty(tuple(Xshape), requires_grad=tensor1.requires_grad)
    call("wxx_conv2dtranspose_dx", ptr(tensor1), ptr(W), ptr(out), *d)
    return out


def conv2dtranspose_dw(tensor1, X, stride, padding, dilation, out_shape, wshape):
    """Weight gradient of :func:`conv2dtranspose`; ``tensor1`` is dY
    (reference convolution.py:1067-1185)."""
    if not tensor1.is_contiguous():
        tensor1 = tensor1.contiguous()
    if not X.is_contiguous():
        X = X.contiguous()
    d = _tconv_dims(X.shape, wshape, stride, padding, dilation, out_shape)
    out = empty((X.shape[1], wshape[1], wshape[2], wshape[3]), requires_grad=tensor1.requires_grad)
    call("wxx_conv2dtranspose_dw", ptr(tensor1), ptr(X), ptr(out), *d)
    return out


def causal_conv1d(tensor1, weight, bias):
    """Depthwise causal conv over ``(B, D, L)``: out[b,d,n] = bias[d] +
    sum_k weight[d,k] x[b,d,n-k]; ``tensor1`` may be a strided view
    (reference convolution.py:1188-1257)."""
    if len(tensor1.shape) != 3:
        raise ValueError(f"causal_conv1d expects a 3-D input, got {tensor1.shape}")
    if len(weight.shape) != 2:
        raise ValueError(f"causal_conv1d weight must be (D, K), got {weight.shape}")
    if any(s < 0 for s in tensor1.stride):
        tensor1 = tensor1.contiguous()
    if not weight.is_contiguous():
        weight = weight.contiguous()
    if not bias.is_contiguous():
        bias = bias.contiguous()
    B, D, L = tensor1.shape
    KS = weight.shape[1]
    out = empty((B, D, L), requires_grad=(tensor1.requires_grad or weight.requires_grad))
    base = C.c_void_p(tensor1.buffer.ptr)
    call("wxx_causal_conv1d", base, tensor1.offset, *tensor1.stride, ptr(weight), ptr(bias),
         ptr(out), B, D, L, KS)
    return out


def causal_conv1d_backward(grad_output, tensor1, weight, bias, need_weight_grad=True):
    """``(dX, dWeight, dBias)`` of :func:`causal_conv1d`; the weight and bias
    gradients are ``None`` when not needed (reference convolution.py:1260-1351)."""
    if not grad_output.is_contiguous():
        grad_output = grad_output.contiguous()
    if any(s < 0 for s in tensor1.stride):
        tensor1 = tensor1.contiguous()
    if not weight.is_contiguous():
        weight = weight.contiguous()
    B, D, L = tensor1.shape
    KS = weight.shape[1]
    dX = empty((B, D, L))
    dW = empty((D, KS)) if need_weight_grad else None
    dB = empty((D,)) if need_weight_grad else None
    base = C.c_void_p(tensor1.buffer.ptr)
    call("wxx_causal_conv1d_backward", ptr(grad_output), base, tensor1.offset, *tensor1.stride,
         ptr(weight), ptr(dX), ptr(dW) if dW is not None else None,
         ptr(dB) if dB is not None else None, B, D, L, KS)
    return dX, dW, dB
