"""The C ABI: the library loads and exports every entry point that
include/wxx_hip.h declares, with the argument count the ctypes table uses.
No compute call is made (CPU-only)."""

import ctypes
import os
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "wxx_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:const\s+)?\w+\s*\*?\s*(wxx_\w+)\s*\(([^)]*)\)\s*;", text):
        args = m.group(2).strip()
        n = 0 if args in ("", "void") else len([a for a in args.split(",") if a.strip()])
        out[m.group(1)] = n
    return out


@pytest.fixture(scope="module")
def lib_path():
    from wxx_amd.backend import lib

    if not os.path.exists(lib.LIB_PATH):
        from wxx_amd import build

        build.build(verbose=False)
    return lib.LIB_PATH


def test_header_parses():
    fns = header_functions()
    assert "wxx_matmul_add" in fns and fns["wxx_matmul_add"] == 15
    assert len(fns) >= 30


def test_library_exports_every_header_symbol(lib_path):
    lib = ctypes.CDLL(lib_path)
    missing = [name for name in header_functions() if not hasattr(lib, name)]
    assert not missing, f"declared in wxx_hip.h but not exported: {missing}"


def test_ctypes_table_matches_header(lib_path):
    from wxx_amd.backend.lib import SIGNATURES

    fns = header_functions()
    assert set(fns) == set(SIGNATURES), (
        f"header-only: {sorted(set(fns) - set(SIGNATURES))}, "
        f"table-only: {sorted(set(SIGNATURES) - set(fns))}"
    )
    for name, nargs in fns.items():
        assert len(SIGNATURES[name][1]) == nargs, f"{name}: header {nargs} args"


def test_no_unexpected_exports(lib_path):
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path], capture_output=True, text=True)
    exported = {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}
    ours = {s for s in exported if s.startswith("wxx_")}
    assert ours == set(header_functions()), sorted(ours ^ set(header_functions()))


def test_library_is_gfx950(lib_path):
    data = open(lib_path, "rb").read()
    assert b"gfx950" in data
