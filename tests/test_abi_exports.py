"""CPU-side checks of the C-ABI boundary: the built library loads and exports
every entry point that include/nrs_hip.h declares (no GPU calls)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nrs_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared("nrs_hip.h")
    assert "nrs_gemm" in names and "nrs_conv2d_backward" in names and len(names) >= 25


def test_library_exports_every_declared_symbol():
    from neuralrs_amd import _abi

    if not os.path.exists(_abi.LIB_PATH):
        pytest.skip("libnrs_hip.so not built")
    lib = ctypes.CDLL(_abi.LIB_PATH)
    missing = [n for n in declared("nrs_hip.h") if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_header():
    from neuralrs_amd import _abi

    assert set(declared("nrs_hip.h")) == set(_abi.SIGNATURES)


def test_rust_binding_covers_header():
    """The Rust extern block a maintainer copies from INTEGRATION.md lists
    exactly the header's entry points."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = text[text.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    assert set(re.findall(r"pub fn (nrs_\w+)\(", block)) == set(declared("nrs_hip.h"))
