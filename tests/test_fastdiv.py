"""CPU check of the magic-number divider the kernels use for their index
math (neuralrs_amd/csrc/fastdiv.hpp) against the CPU's integer division."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "fastdiv_check")


def test_fastdiv_matches_integer_division():
    if not os.path.exists(BIN):
        pytest.skip("fastdiv_check not built (run __graft_entry__.build())")
    out = subprocess.run([BIN], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0 and "fastdiv ok" in out.stdout, out.stdout + out.stderr
