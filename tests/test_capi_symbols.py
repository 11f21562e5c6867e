"""The C-ABI library loads and exports every entry point include/*.h declares
(no compute call: this runs without a GPU)."""

from __future__ import annotations

import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols() -> set[str]:
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        txt = open(h).read()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        names |= set(re.findall(r"\b(mgq_\w+)\s*\(", txt))
    return names


def test_header_declares_entry_points():
    assert len(declared_symbols()) >= 14


def test_library_exports_every_declared_symbol():
    from mlx_gptq import _native

    if not _native.LIB_PATH.exists():
        pytest.fail(f"{_native.LIB_PATH} not built (python mlx-gptq-mxfp_amd/build.py)")
    lib = ctypes.CDLL(str(_native.LIB_PATH))
    missing = [n for n in sorted(declared_symbols()) if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_table_matches_header():
    from mlx_gptq import _native

    assert set(_native.SIGNATURES) == declared_symbols()
    lib = _native.load()
    assert lib.mgq_version() >= 100
