"""Build the oracle's C restatements into ``oracle/lib/liboracle.so`` (gcc, OpenMP).

TEST INFRASTRUCTURE ONLY.  The reference itself is Python + WGSL run through
wgpu-py, so there is no reference C/C++ source to compile into ``oracle/_ref``;
this library holds our own restatements (oracle/csrc/*.c).
"""

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "liboracle.so")

# -ffp-contract=off: only the explicit fmaf calls fuse, exactly as written.
CFLAGS = ["-O3", "-fPIC", "-shared", "-fopenmp", "-mavx2", "-mfma", "-ffp-contract=off",
          "-std=c99"]


def build(verbose=True):
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sorted(os.path.join(SRC, f) for f in os.listdir(SRC) if f.endswith(".c"))
    tmp = LIB + ".tmp"
    cmd = ["gcc", *CFLAGS, "-o", tmp, *srcs, "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
