"""ctypes binding of the C ABI declared in include/nrs_hip.h.

Loads the in-tree ``libnrs_hip.so`` (built by ``make -C neuralrs_amd/csrc``).
There is no fallback: if the library is missing or a call fails, an exception
is raised, as the reference panics (e.g. src/cuda/graph/matmul.rs:290).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnrs_hip.so")

NN, NT, TN = 0, 1, 2
EPI_NONE, EPI_BIAS_COL, EPI_BIAS_ROW, EPI_RELU = 0, 1, 2, 4

_P = ctypes.c_void_p
_I = ctypes.c_int64
_F = ctypes.c_float

GEMM_GROUP_MAX = 4


class GemmDesc(ctypes.Structure):
    """nrs_gemm_desc (include/nrs_hip.h): one nrs_gemm call of a group."""
    _fields_ = [("layout", ctypes.c_int), ("C", _P), ("A", _P), ("B", _P),
                ("rows", _I), ("cols", _I), ("inner", _I), ("beta", _F),
                ("bias", _P), ("epilogue", ctypes.c_int)]


# name -> argtypes (all return int status unless listed in _RET)
SIGNATURES = {
    "nrs_init": [ctypes.c_int],
    "nrs_shutdown": [],
    "nrs_set_stream": [_P],
    "nrs_get_stream": [],
    "nrs_last_error": [],
    "nrs_malloc": [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t],
    "nrs_free": [_P],
    "nrs_empty_cache": [],
    "nrs_memory_stats": [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)],
    "nrs_memcpy_htod": [_P, _P, ctypes.c_size_t],
    "nrs_memcpy_dtoh": [_P, _P, ctypes.c_size_t],
    "nrs_memcpy_dtod": [_P, _P, ctypes.c_size_t],
    "nrs_memset_zero": [_P, ctypes.c_size_t],
    "nrs_sync": [],
    "nrs_gemm": [ctypes.c_int, _P, _P, _P, _I, _I, _I, _F, _P, ctypes.c_int],
    "nrs_gemm_group": [ctypes.POINTER(GemmDesc), ctypes.c_int],
    "nrs_matmul_shared_lhs_backward": [_P, _P, _P, _P, _P, ctypes.c_int, _I, _I, _I, _F, _P],
    "nrs_linear_backward": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _F, _F],
    "nrs_linear_backward_relu": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _F, _F],
    "nrs_linear_cross_entropy": [_P, _P, _P, _P, _P, _P, _I, _I, _I],
    "nrs_mlp2_forward_seed": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I],
    "nrs_mlp2_backward": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _F],
    "nrs_gemm_nt_splitk": [_P, _P, _P, _I, _I, _I, _F],
    "nrs_gemm_nt_splitk_noalloc": [_P, _P, _P, _I, _I, _I, _F],
    "nrs_bmm": [ctypes.c_int, _P, _P, _P, _I, _I, _I, _I, _F],
    "nrs_bmm_backward": [ctypes.c_int, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F],
    "nrs_attention_supported": [_I, _I, _I, _I, _I],
    "nrs_attention_forward": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F],
    "nrs_attention_backward": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F],
    "nrs_im2col": [_P, _P] + [_I] * 8,
    "nrs_col2out": [_P, _P, _P, _I, _I, _I, _I],
    "nrs_out2mm": [_P, _P, _I, _I, _I, _I],
    "nrs_col2im": [_P, _P] + [_I] * 8 + [_F],
    "nrs_conv2d_bias_grad": [_P, _P, _I, _I, _I, _I, _F],
    "nrs_conv2d_forward": [_P, _P, _P, _P] + [_I] * 9,
    "nrs_conv2d_backward": [_P, _P, _P, _P, _P, _P] + [_I] * 9,
    "nrs_conv2d_backward_beta": [_P, _P, _P, _P, _P, _P] + [_I] * 9 + [_F],
    "nrs_conv2d_backward_ex": [_P, _P, _P, _P, _P, _P] + [_I] * 9 + [_F, _F],
    "nrs_conv2d_maxpool_forward": [_P, _P, _P, _P, _P, _P] + [_I] * 11,
    "nrs_maxpool_conv2d_backward": [_P, _P, _P, _P, _P, _P, _P] + [_I] * 11,
    "nrs_conv2d_relu_maxpool_forward": [_P, _P, _P, _P, _P, _P] + [_I] * 11,
    "nrs_maxpool_relu_conv2d_backward": [_P, _P, _P, _P, _P, _P, _P, _P] + [_I] * 11 + [_F],
    "nrs_conv2d_maxpool_relu_conv2d_backward": [_P] * 11 + [_I] * 16 + [_F],
    "nrs_accumulate": [_P, _P, _I],
    "nrs_vadd": [_P, _P, _P, _I],
    "nrs_bias_add": [_P, _P, _P, _I, _I],
    "nrs_sum_axis0": [_P, _P, _I, _I, _F],
    "nrs_maxpool_forward": [_P, _P, _P] + [_I] * 6,
    "nrs_maxpool_backward": [_P, _P, _P] + [_I] * 6,
    "nrs_transpose": [_P, _P, _I, _I, _I],
    "nrs_scale": [_P, _P, _F, _I, _F],
    "nrs_softmax_forward": [_P, _P, _I, _I],
    "nrs_cross_entropy_forward": [_P, _P, _P, _I, _I],
    "nrs_cross_entropy_backward": [_P, _P, _P, _I, _I],
    "nrs_softmax_backward": [_P, _P, _P, _I, _I, _F],
    "nrs_slice_cols": [_P, _P, _I, _I, _I, _I],
    "nrs_slice_cols_backward": [_P, _P, _I, _I, _I, _I, _F],
    "nrs_concat_cols": [_P, _P, _I, _I, _I, _I],
    "nrs_concat_cols_backward": [_P, _P, _I, _I, _I, _I, _F],
    "nrs_split_heads": [_P, _P, _I, _I, _I, _F],
    "nrs_layernorm_forward": [_P, _P, _P, _P, _P, _P, _I, _I, _F],
    "nrs_add_layernorm_forward": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _F],
    "nrs_layernorm_backward": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _F],
    "nrs_add_layernorm_backward": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _F, _F, _F],
    "nrs_merge_heads": [_P, _P, _I, _I, _I, _F],
    "nrs_softmax_forward_scaled": [_P, _P, _I, _I, _F],
    "nrs_softmax_backward_scaled": [_P, _P, _P, _I, _I, _F, _F],
    "nrs_relu_forward": [_P, _P, _I],
    "nrs_relu_backward": [_P, _P, _P, _I, _F],
}
_RET = {"nrs_get_stream": ctypes.c_void_p, "nrs_last_error": ctypes.c_char_p}


class NrsError(RuntimeError):
    pass


_lib = None


def load():
    """Load libnrs_hip.so (no initialisation, no GPU needed)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NrsError(
                f"HIP extension missing: {LIB_PATH}. Build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'`.")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RET.get(name, ctypes.c_int)
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().nrs_last_error().decode(errors="replace")
        raise NrsError(f"{what}: status {rc}: {msg}")


def call(name: str, *args) -> None:
    """Call an entry point. DeviceBuffer / torch-tensor arguments are passed as
    their device pointers and stay referenced until the launch is enqueued
    (nrs_free caches the block; it is reused only by work enqueued later on
    the library stream, so queued launches finish with it first)."""
    conv = [_ptr(a) if isinstance(a, DeviceBuffer) or hasattr(a, "data_ptr") else a for a in args]
    check(getattr(load(), name)(*conv), name)


def init(device: int = 0) -> None:
    call("nrs_init", device)


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    if hasattr(x, "data_ptr"):  # torch tensor
        return x.data_ptr()
    return int(x)


class DeviceBuffer:
    """A device allocation owned through nrs_malloc/nrs_free (f32 or i32)."""

    def __init__(self, n: int, dtype=np.float32):
        self.n = int(n)
        self.dtype = np.dtype(dtype)
        self.nbytes = self.n * self.dtype.itemsize
        p = ctypes.c_void_p()
        call("nrs_malloc", ctypes.byref(p), self.nbytes)
        self.ptr = p.value

    @classmethod
    def from_host(cls, arr, dtype=np.float32):
        a = np.ascontiguousarray(arr, dtype=dtype)
        buf = cls(a.size, dtype)
        if a.size:
            call("nrs_memcpy_htod", buf.ptr, a.ctypes.data, a.nbytes)
        return buf

    @classmethod
    def zeros(cls, n: int, dtype=np.float32):
        buf = cls(n, dtype)
        if buf.nbytes:
            call("nrs_memset_zero", buf.ptr, buf.nbytes)
        return buf

    def to_host(self, shape=None):
        out = np.empty(self.n, self.dtype)
        if self.n:
            call("nrs_memcpy_dtoh", out.ctypes.data, self.ptr, self.nbytes)
        return out.reshape(shape) if shape is not None else out

    def free(self):
        if self.ptr:
            load().nrs_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ----------------------------------------------------------- thin wrappers
def gemm(layout, C, A, B, rows, cols, inner, beta=0.0, bias=None, epilogue=EPI_NONE):
    call("nrs_gemm", layout, _ptr(C), _ptr(A), _ptr(B), rows, cols, inner, beta, _ptr(bias),
         epilogue)


def gemm_group(calls):
    """Several gemm calls in one nrs_gemm_group launch; each call is a tuple
    (layout, C, A, B, rows, cols, inner[, beta[, bias[, epilogue]]])."""
    descs = (GemmDesc * max(1, len(calls)))()
    for d, c in zip(descs, calls):
        layout, C, A, B, rows, cols, inner = c[:7]
        beta = c[7] if len(c) > 7 else 0.0
        bias = c[8] if len(c) > 8 else None
        epi = c[9] if len(c) > 9 else EPI_NONE
        d.layout, d.C, d.A, d.B = layout, _ptr(C), _ptr(A), _ptr(B)
        d.rows, d.cols, d.inner, d.beta, d.bias, d.epilogue = rows, cols, inner, beta, _ptr(bias), epi
    call("nrs_gemm_group", descs, len(calls))


def matmul_shared_lhs_backward(dx, dws, gs, x, ws, rows, inner, cols, beta_x=0.0,
                               beta_w=None):
    """dx and dW_i of y_i = x . W_i (i < len(ws) <= 3) in one call: dx adds
    g_i . W_i^T in index order after beta_x * dx, dW_i = x^T . g_i +
    beta_w[i] * dW_i."""
    n = len(ws)
    ptrs = lambda bufs: (ctypes.c_void_p * 3)(*[_ptr(b) for b in bufs])
    betas = (ctypes.c_float * 3)(*(list(beta_w) if beta_w is not None else [0.0] * n))
    call("nrs_matmul_shared_lhs_backward", _ptr(dx), ptrs(dws), ptrs(gs), _ptr(x), ptrs(ws), n,
         rows, inner, cols, beta_x, betas)


def gemm_nt_splitk(C, A, B, rows, cols, inner, beta=0.0):
    call("nrs_gemm_nt_splitk", _ptr(C), _ptr(A), _ptr(B), rows, cols, inner, beta)


def bmm(layout, C, A, B, batch, rows, cols, inner, beta=0.0):
    call("nrs_bmm", layout, _ptr(C), _ptr(A), _ptr(B), batch, rows, cols, inner, beta)


def bmm_backward(layout, dA, dB, G, A, B, batch, m, k, n, beta=0.0):
    """Both gradients of C = A . op(B) per item (A m x k, G m x n; op(B) = B
    [k x n] for NN, B^T with B [n x k] for NT); dA or dB may be None."""
    call("nrs_bmm_backward", layout, _ptr(dA), _ptr(dB), _ptr(G), _ptr(A), _ptr(B),
         batch, m, k, n, beta)


def sync():
    call("nrs_sync")
