"""ctypes binding of ``libwxx_hip.so`` (the C ABI declared in include/wxx_hip.h).

The library is loaded from ``wxx_amd/lib`` (built in-tree by
``wxx_amd.build``).  There is no fallback: if the library is missing or the
HIP runtime has no device, the first op raises ``RuntimeError``.

Every entry point returns 0 or a negative code; :func:`call` turns a
non-zero code into ``RuntimeError`` carrying ``wxx_last_error()``.
"""

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libwxx_hip.so")

P = C.c_void_p
I64 = C.c_int64
I32 = C.c_int
U32 = C.c_uint32
F32 = C.c_float
SZ = C.c_size_t

# name -> (restype, argtypes).  Kept in the order of include/wxx_hip.h.
SIGNATURES = {
    # runtime
    "wxx_last_error": (C.c_char_p, []),
    "wxx_device_count": (I32, [C.POINTER(I32)]),
    "wxx_init": (I32, [I32]),
    "wxx_device_info": (I32, [C.POINTER(I32), C.c_char_p, I32, C.POINTER(SZ)]),
    "wxx_alloc": (P, [SZ]),
    "wxx_free": (I32, [P]),
    "wxx_empty_cache": (I32, []),
    "wxx_mem_stats": (I32, [C.POINTER(SZ), C.POINTER(SZ), C.POINTER(SZ), C.POINTER(SZ)]),
    "wxx_h2d": (I32, [P, P, SZ]),
    "wxx_d2h": (I32, [P, P, SZ]),
    "wxx_d2d": (I32, [P, P, SZ]),
    "wxx_fill_u32": (I32, [P, I64, U32]),
    "wxx_sync": (I32, []),
    "wxx_stream": (P, []),
    "wxx_timer_record": (I32, [I32]),
    "wxx_timer_elapsed": (I32, [I32, I32, C.POINTER(F32)]),
    # step graphs
    "wxx_graph_begin": (I32, []),
    "wxx_graph_end": (I32, [C.POINTER(P), C.POINTER(I64)]),
    "wxx_graph_abort": (I32, []),
    "wxx_graph_launch": (I32, [P]),
    "wxx_graph_destroy": (I32, [P]),
    "wxx_graph_capturing": (I32, [C.POINTER(I32)]),
    # GEMM
    "wxx_matmul_add": (
        I32,
        [P, P, P, P, I64, I64, I64, I64, I64, I64, I64, I32, I32, I32, I32],
    ),
    "wxx_matmul_add_noalloc": (
        I32,
        [P, P, P, P, I64, I64, I64, I64, I64, I64, I64, I32, I32, I32, I32],
    ),
    "wxx_matmul_tri": (I32, [P, P, P, I64, I64, I64, I64, I64, I64, I32, I32, I32]),
    # convolution / pooling
    "wxx_conv2d": (I32, [P, P, P, P] + [I64] * 13),
    "wxx_conv2ddx": (I32, [P, P, P] + [I64] * 13),
    "wxx_conv2ddw": (I32, [P, P, P] + [I64] * 13),
    "wxx_conv2dtranspose": (I32, [P, P, P, P] + [I64] * 15),
    "wxx_conv2dtranspose_dx": (I32, [P, P, P] + [I64] * 15),
    "wxx_conv2dtranspose_dw": (I32, [P, P, P] + [I64] * 15),
    "wxx_pool2d": (I32, [P, P, P] + [I64] * 10 + [I32]),
    "wxx_pool2d_backward": (I32, [P, P, P] + [I64] * 10 + [I32]),
    "wxx_adaptive_avgpool2d": (I32, [P, P] + [I64] * 6),
    "wxx_adaptive_avgpool2ddx": (I32, [P, P] + [I64] * 6),
    "wxx_causal_conv1d": (I32, [P, I64, I64, I64, I64, P, P, P, I64, I64, I64, I64]),
    "wxx_causal_conv1d_backward": (I32, [P, P, I64, I64, I64, I64, P, P, P, P, I64, I64, I64,
                                         I64]),
    # reductions
    "wxx_reduce": (I32, [P, P, I64, I64, I64, I32]),
    "wxx_reduce_minmax": (I32, [P, P, P, I64, I64, I64, I32]),
    "wxx_maxmin_backward": (I32, [P, P, P, I64, I64, I64]),
    "wxx_softmax": (I32, [P, P, I64, I64, I64]),
    "wxx_softmax_backward": (I32, [P, P, P, I64, I64, I64]),
    "wxx_softmax_scale_mask": (I32, [P, P, P, I64, I64, I64, I64, F32]),
    "wxx_softmax_backward_scale": (I32, [P, P, P, I64, I64, F32]),
    "wxx_softmax_causal": (I32, [P, P, I64, I64, I64, F32, I32]),
    "wxx_softmax_backward_causal": (I32, [P, P, P, I64, I64, I64, F32, I32]),
    # normalisation
    "wxx_meanvarnorm": (I32, [P, P, P, P, P, P, I64, I64, I64, F32, I64]),
    "wxx_meanvarnormdx": (I32, [P, P, P, P, P, P, I64, I64, I64, I64]),
    "wxx_meanvarnormdg": (I32, [P, P, P, P, P, P, I64, I64, I64]),
    "wxx_rmsnorm": (I32, [P, P, P, P, I64, I64, I64, F32, I64]),
    "wxx_rmsnormdx": (I32, [P, P, P, P, P, I64, I64, I64]),
    "wxx_rmsnormdg": (I32, [P, P, P, P, I64, I64, I64]),
    "wxx_batchnorm": (I32, [P, P, P, P, P, P, P, P, I64, I64, I64, F32, F32, I32]),
    "wxx_batchnormdg": (I32, [P, P, P, P, P, P, I64, I64, I64]),
    "wxx_batchnormdx": (I32, [P, P, P, P, P, P, P, P, I64, I64, I64]),
    "wxx_batchnorm_backward": (I32, [P, P, P, P, P, P, P, P, I64, I64, I64]),
    "wxx_batchnorm_act": (I32, [P, P, P, P, P, P, P, P, P, I64, I64, I64, F32, F32, I32, I32]),
    "wxx_batchnorm_act_backward": (I32, [P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I32]),
    # elementwise / layout
    "wxx_pointwise": (I32, [P, P, P, I32, P, P, P, P, I32]),
    "wxx_scalarpointwise": (I32, [P, P, I64, I32, F32, I32]),
    "wxx_unary": (I32, [P, P, I64, I32]),
    "wxx_unary_backward": (I32, [P, P, P, I64, I32]),
    "wxx_swiglu_gate": (I32, [P, P, P, I64]),
    "wxx_swiglu_gate_backward": (I32, [P, P, P, P, P, I64]),
    "wxx_broadcast_scale": (I32, [P, P, I32, P, P, F32]),
    "wxx_clamp": (I32, [P, P, I64, F32, F32, I32]),
    "wxx_equal": (I32, [P, P, P, I64, I32, U32]),
    "wxx_mul_backward": (I32, [P, P, P, P, P, I64]),
    "wxx_copy_strided": (I32, [P, P, I32, I32, P, P, P]),
    "wxx_fill_strided": (I32, [P, I32, P, P, U32]),
    "wxx_scatter_zeros": (I32, [P, P, I32, P, P, I32, I64, I64]),
    "wxx_unfolddx": (I32, [P, P, I64, I64, I64, I64, I64, I64]),
    # FFT / complex
    "wxx_rfft": (I32, [P, P, I64, I64, I64]),
    "wxx_irfft": (I32, [P, P, I64, I64, I64]),
    "wxx_irfft_crop": (I32, [P, P, I64, I64, I64, I64, F32]),
    "wxx_complex_binary": (I32, [P, P, P, I32, P, P, P, P, I32, I32, I32]),
    "wxx_complex_conj": (I32, [P, P, I32, P, P, P]),
    "wxx_complex_pad": (I32, [P, P, I64, I64, I64]),
    "wxx_rfft_mul": (I32, [P, P, I64, I64, I64, F32, F32]),
    "wxx_irfft_mul": (I32, [P, P, P, I64, I64, I64, I32, I32, F32, F32, I64, I64, F32]),
    "wxx_complex_mul_batch_sum": (I32, [P, P, P, I64, I64, I32]),
    # loss
    "wxx_cceloss": (I32, [P, P, P, P, I64, I64, P]),
    "wxx_cceloss_stats": (I32, [P, P, P, P, I64, I64, P]),
    "wxx_cceloss_backward": (I32, [P, P, P, P, I64, P, I64, I64]),
    # optimizer / grad norm
    "wxx_adamw": (I32, [P, P, P, P, I64, F32, F32, F32, F32, F32, F32, F32]),
    "wxx_adamw_multi": (I32, [P, P, P, P, P, I32, F32, F32, F32, F32, F32, F32, F32]),
    "wxx_sumsq_multi": (I32, [P, P, I32, P]),
    "wxx_scale_multi": (I32, [P, P, I32, F32]),
    "wxx_adamw_multi_dev": (I32, [P, P, P, P, P, I32, P]),
    "wxx_clip_scale_multi": (I32, [P, P, I32, P, C.c_double, P]),
    # embedding / dropout / decay window
    "wxx_embed": (I32, [P, P, P, I64, I64, I64]),
    "wxx_embeddx": (I32, [P, P, P, I64, I64, I64]),
    "wxx_dropout": (I32, [P, P, I64, U32, F32, F32]),
    "wxx_dropout_dev": (I32, [P, P, I64, P, F32, F32]),
    # fused attention
    "wxx_attention_fwd": (I32, [P, P, P, P, P, I64, I64, I64, I64, I32, F32, F32, F32, U32, P]),
    "wxx_attention_bwd": (I32, [P] * 9 + [I64, I64, I64, I64, I32, F32, F32, F32, U32, P]),
    "wxx_decay_window": (I32, [P, P, I64, I64, I64, I64]),
    "wxx_decay_window_backward": (I32, [P, P, P, I64, I64, I64, I64]),
}

_lib = None


def load():
    """Load the shared library once and attach the signatures."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m wxx_amd.build` "
            "(there is no CPU fallback)"
        )
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error():
    msg = load().wxx_last_error()
    return msg.decode() if msg else ""


class HIPError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""

    def __init__(self, name, code, message):
        super().__init__(f"{name} failed ({code}): {message}")
        self.code = code


def call(name, *args):
    """Call ``name`` and raise :class:`HIPError` on a non-zero return code."""
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise HIPError(name, rc, last_error())
    return rc


__all__ = ["LIB_PATH", "SIGNATURES", "load", "call", "last_error", "HIPError"]
