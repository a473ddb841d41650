"""Test configuration.

Markers: ``gpu`` tests need a HIP device and call the C ABI of
``libwxx_hip.so``; everything else runs on the CPU (oracle pinning, host
logic, library exports).  GPU tests never skip for a missing device: on a
GPU box a missing device or library is a failure.
"""

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


# Test-only hook: run the GPU tests against the AddressSanitizer CPU build of
# the kernels (tests/cpu_emu) by pointing the loader at that library.  Never
# set on a GPU box; the product loader has no fallback of its own.
_EMU = os.environ.get("WXX_TEST_EMU_LIB")
if _EMU:
    from wxx_amd.backend import lib as _wlib

    _wlib.LIB_PATH = _EMU


# Cases too large for the CPU emulation (multi-GFLOP GEMMs, 100M-element rows);
# they run unchanged on the GPU.
_EMU_HEAVY = ("test_matmul_config2_sizes", "test_matmul_tri_modes[1024", "test_train_steps_do_not_grow_live_buffers", "test_matmul_every_tile_code", "test_softmax[shape2", "test_softmax[shape1-",
              "test_layernorm_fwd_bwd[shape1-", "test_rmsnorm_fwd_bwd[shape1-",
              "test_fft_full_size_properties", "test_hyena_shapes",
              "test_embed_bit_exact_and_embeddx[50304", "test_dropout_bit_exact[6291459",
              "test_cceloss[64-50304", "test_conv2d_resnet18_shapes", "test_causal_conv1d[8-256",
              "test_maxpool2d_bit_exact[shape0", "test_avgpool2d[shape0",
              "test_adaptive_avgpool2d[shape0", "test_fft_many_rows_every_row[3000",
              "test_fft_many_rows_every_row[1100", "test_fft_many_rows_every_row[600",
              "test_gpt2_config1_train_step_matches_oracle", "test_resnet18_forward_backward",
              "test_hyena_parameter_counts_and_tying", "test_softmax_scale_mask_fused[98304",
              "test_matmul_split_k[True-False-768")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and libwxx_hip.so")


def pytest_collection_modifyitems(config, items):
    if not _EMU:
        return
    skip = pytest.mark.skip(reason="too large for the CPU emulation; runs on the GPU")
    for item in items:
        if any(item.nodeid.split("::")[-1].startswith(h) for h in _EMU_HEAVY):
            item.add_marker(skip)


@pytest.fixture(scope="session")
def device():
    """Open the HIP device once (fails loudly when unavailable)."""
    from wxx_amd.backend import device as dev

    dev.ensure_device()
    return dev


def rng(seed=0):
    return np.random.default_rng(seed)


def assert_close(actual, expected, rtol=1e-4, atol=1e-5, msg=""):
    actual = np.asarray(actual)
    expected = np.asarray(expected)
    assert actual.shape == expected.shape, f"{msg} shape {actual.shape} != {expected.shape}"
    if not np.allclose(actual, expected, rtol=rtol, atol=atol, equal_nan=True):
        err = np.abs(actual.astype(np.float64) - expected.astype(np.float64))
        bad = ~np.isclose(actual, expected, rtol=rtol, atol=atol, equal_nan=True)
        raise AssertionError(
            f"{msg} max abs err {np.nanmax(err):.3g}; {int(bad.sum())} of {bad.size} "
            f"elements outside rtol={rtol} atol={atol}"
        )


def assert_error_floor(got, want64, ref32, c=4.0, rtol=1e-4, msg="", atol=0.0):
    """A float result against float64 with the float32 rounding floor as the
    yardstick: ref32 is the same sums evaluated in single precision (another
    order), and the device may miss the float64 value by at most c times
    the largest miss of ref32 (plus rtol of the element itself, plus atol).
    Unlike a tolerance scaled by sqrt(K), a wrong or dropped term (an error
    far above what single precision produces) fails.  ``atol`` is for
    results that are exact zeros in the composition the floor is taken
    from but sums of cancelling terms in another order."""
    got, w, f = (np.asarray(a, np.float64) for a in (got, want64, ref32))
    assert got.shape == w.shape, f"{msg} shape {got.shape} != {w.shape}"
    floor = float(np.abs(f - w).max()) if f.size else 0.0
    err = np.abs(got - w)
    bad = err > c * floor + rtol * np.abs(w) + atol + 1e-30
    if bad.any():
        raise AssertionError(f"{msg} {int(bad.sum())} of {bad.size} elements beyond {c} x the "
                             f"fp32 floor {floor:.3g}; max err {err.max():.3g}")
