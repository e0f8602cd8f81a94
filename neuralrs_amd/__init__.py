"""MI355X (gfx950) backend for NeuralRs's f32 matrix-multiply family.

The product is the C ABI in ``include/nrs_hip.h`` implemented by
``libnrs_hip.so`` (hand-written HIP kernels in ``csrc/``) and the C++ host
layer ``libnrs_host.so`` that mirrors the reference's resident operator API
(``csrc/host/``). ``_abi`` is the Python ctypes binding of the C ABI used by
the tests and the benchmark.
"""
from . import _abi  # noqa: F401

__all__ = ["_abi"]
