"""CPU check of the convolution kernels' load addressing (no GPU).

Compiles tests/conv_addr_check.cpp (g++, against wxx_amd/csrc/conv_addr.h,
the same header the gfx950 kernels include) and walks every slot of every
chunk of every tile of each mode, operand layout and K split for the
ResNet18 config-3 convolutions, the small ragged cases of the GPU conv tests
and random shapes: every source must lie inside its tensor and be the element
the convolution's definition names (zero exactly where it says zero)."""

import os
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "conv_addr_check.cpp")

# (B, Cin, H, W, Cout, KH, KW, sh, sw, ph, pw, dh, dw)
RESNET18 = [
    (128, 3, 32, 32, 64, 7, 7, 2, 2, 3, 3, 1, 1),
    (128, 64, 8, 8, 64, 3, 3, 1, 1, 1, 1, 1, 1),
    (128, 64, 8, 8, 128, 3, 3, 2, 2, 1, 1, 1, 1),
    (128, 64, 8, 8, 128, 1, 1, 2, 2, 0, 0, 1, 1),
    (128, 128, 4, 4, 128, 3, 3, 1, 1, 1, 1, 1, 1),
    (128, 128, 4, 4, 256, 3, 3, 2, 2, 1, 1, 1, 1),
    (128, 128, 4, 4, 256, 1, 1, 2, 2, 0, 0, 1, 1),
    (128, 256, 2, 2, 256, 3, 3, 1, 1, 1, 1, 1, 1),
    (128, 256, 2, 2, 512, 3, 3, 2, 2, 1, 1, 1, 1),
    (128, 256, 2, 2, 512, 1, 1, 2, 2, 0, 0, 1, 1),
    (128, 512, 1, 1, 512, 3, 3, 1, 1, 1, 1, 1, 1),
]
SMALL = [
    (1, 1, 1, 1, 1, 1, 1, 1, 1, 0, 0, 1, 1),
    (2, 3, 9, 9, 4, 3, 3, 1, 1, 1, 1, 1, 1),
    (2, 3, 11, 10, 5, 7, 7, 2, 2, 3, 3, 1, 1),
    (1, 4, 8, 8, 6, 1, 1, 2, 2, 0, 0, 1, 1),
    (2, 2, 12, 9, 3, 3, 2, 2, 1, 2, 0, 2, 3),
    (3, 5, 4, 4, 2, 3, 3, 1, 1, 0, 0, 1, 1),
    (2, 17, 13, 11, 70, 3, 3, 1, 1, 1, 1, 1, 1),
    (4, 130, 5, 6, 129, 3, 3, 2, 2, 1, 1, 1, 1),
    (3, 9, 8, 4, 33, 2, 2, 1, 1, 0, 1, 1, 1),
    (5, 8, 4, 8, 40, 3, 1, 1, 2, 1, 0, 1, 1),
    (2, 70, 6, 6, 66, 3, 3, 1, 1, 1, 1, 1, 1),
]


def _random_shapes(n, seed):
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        kh, kw = int(r.integers(1, 5)), int(r.integers(1, 5))
        sh, sw = int(r.integers(1, 4)), int(r.integers(1, 4))
        dh, dw = int(r.integers(1, 3)), int(r.integers(1, 3))
        ph, pw = int(r.integers(0, 3)), int(r.integers(0, 3))
        H, W = int(r.integers(1, 12)), int(r.integers(1, 12))
        if H + 2 * ph - dh * (kh - 1) - 1 < 0 or W + 2 * pw - dw * (kw - 1) - 1 < 0:
            continue
        out.append((int(r.integers(1, 5)), int(r.integers(1, 40)), H, W, int(r.integers(1, 90)),
                    kh, kw, sh, sw, ph, pw, dh, dw))
    return out


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("conv_addr") / "conv_addr_check")
    p = subprocess.run(["g++", "-O2", "-std=c++17", "-o", exe, SRC], capture_output=True, text=True)
    assert p.returncode == 0, p.stderr
    return exe


@pytest.mark.parametrize("name,shapes", [("resnet18", RESNET18), ("small", SMALL),
                                         ("random", _random_shapes(60, 7))])
def test_conv_dma_addresses(checker, name, shapes):
    text = "\n".join(" ".join(map(str, s)) for s in shapes) + "\n"
    p = subprocess.run([checker], input=text, capture_output=True, text=True, timeout=600)
    assert p.returncode == 0, p.stderr[-2000:]
    assert p.stdout.startswith(f"ok {len(shapes)} shapes"), p.stdout
