"""Build ``wxx_amd/lib/libwxx_hip.so`` from ``wxx_amd/csrc/*.hip`` for gfx950.

Each source is compiled by ``hipcc`` in parallel into ``wxx_amd/_build`` and
linked into one shared library kept in-tree (it travels with the source tree
to the GPU host; nothing is installed into site-packages).

Run ``python -m wxx_amd.build`` (or ``python wxx_amd/build.py``).
"""

import concurrent.futures as _cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libwxx_hip.so")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-fp32 VALU ops are disabled for every device pass: hipcc would
# otherwise form v_pk_*_f32 from ordinary float code.
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


# Per-source additions.  The attention kernels keep every MFMA accumulator in
# ordinary VGPRs (the VGPR form of v_mfma): their softmax reads and rescales
# the accumulators between products, which the AGPR form turns into
# accvgpr read / write copies around every tile.
EXTRA_FLAGS = {
    "attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def sources():
    return sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip")
    )


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *CFLAGS, *EXTRA_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            f"hipcc failed for {os.path.basename(src)}:\n{proc.stdout}\n{proc.stderr}"
        )
    return obj


def build(jobs=None, verbose=True):
    """Compile every kernel source and link the shared library. Returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    with _cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB + ".tmp"
    # --no-undefined: a symbol the objects reference but none defines (e.g. a
    # kernel launch stub the host pass did not emit) fails the build here
    # rather than the library's load on a GPU host
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", tmp,
           *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    try:
        build()
    except RuntimeError as exc:
        print(exc, file=sys.stderr)
        sys.exit(1)
