"""The C-ABI library loads and exports every symbol include/*.h declares
(CPU only: no compute call is made)."""
import ctypes
import glob
import os
import re

import pytest

from fastllm_py import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:bool|int|void|float)\s+\**\s*(\w+)\s*\(", text, flags=re.M):
            names.append(m.group(1))
    return names


def test_header_declares_symbols():
    names = declared_symbols()
    assert "FastllmCudaMarlinHalfInt4Gemm" in names
    assert len(names) == len(set(names))


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_native.LIB_PATH):
        pytest.fail(f"{_native.LIB_PATH} not built (run python fastllm-py_amd/build_native.py)")
    lib = ctypes.CDLL(_native.LIB_PATH)
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_table_matches_header():
    assert set(_native.SIGNATURES) == set(declared_symbols())
