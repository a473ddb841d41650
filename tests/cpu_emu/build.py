"""Build the CPU emulation of libwxx_hip.so with AddressSanitizer.

TEST INFRASTRUCTURE ONLY.  Compiles the unchanged kernel sources
(wxx_amd/csrc/*.hip) as host C++ against the HIP-on-CPU shim in
tests/cpu_emu/include, so every global-memory access of every kernel is
checked by ASan.  Output: tests/cpu_emu/lib/libwxx_emu.so.
"""

import concurrent.futures as cf
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
CSRC = os.path.join(ROOT, "wxx_amd", "csrc")
OUT = os.path.join(HERE, "lib")
OBJ = os.path.join(HERE, "_build")
CXX = "/opt/rocm/llvm/bin/clang++"
FLAGS = ["-std=c++17", "-fPIC", "-g", "-O1", "-fno-omit-frame-pointer", "-fsanitize=address",
         "-pthread", "-I", os.path.join(HERE, "include"), "-Wno-unused-result"]


def _cc(src):
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [CXX, *FLAGS, "-x", "c++", "-c", src, "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode:
        raise RuntimeError(f"{os.path.basename(src)}:\n{p.stderr[-4000:]}")
    return obj


def build():
    os.makedirs(OUT, exist_ok=True)
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    srcs.append(os.path.join(HERE, "emu_runtime.cpp"))
    with cf.ThreadPoolExecutor(8) as ex:
        objs = list(ex.map(_cc, srcs))
    lib = os.path.join(OUT, "libwxx_emu.so")
    # Link to a temporary name and rename: a process still running the old
    # library keeps its mapping intact.
    tmp = lib + ".tmp"
    p = subprocess.run([CXX, "-shared", "-fsanitize=address", "-pthread", "-o", tmp, *objs],
                       capture_output=True, text=True)
    if p.returncode:
        raise RuntimeError(p.stderr)
    os.replace(tmp, lib)
    return lib


def asan_runtime():
    p = subprocess.run([CXX, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                       text=True)
    return p.stdout.strip()


if __name__ == "__main__":
    print(build())
    print(asan_runtime())
