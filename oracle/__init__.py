"""CPU oracle for the NeuralRs f32 matrix-multiply family (test infrastructure).

This package is the CHECKER, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it. It wraps ``liboracle.so`` (built from ``nrs_oracle.c`` by ``make -C
oracle``), a plain-C restatement of the reference's CPU algorithms; each C
function cites the reference file:line it follows.

Parity status per function (see tests/test_oracle.py for the checks):
  dot_simd, matmul_simd, matmul_naive, graph_matmul_{forward,backward},
  graph_bmm_{forward,backward}, graph_add_bias_{forward,backward}, im2col,
  conv2d_im2col, conv2d_forward, conv2d_backward, gpu_im2col, gpu_col2out,
  gpu_out2mm, gpu_col2im, gpu_bias_grad, sum_axis0, maxpool_{forward,backward},
  slice_cols{,_backward}, concat_cols{,_backward}, layernorm_{forward,backward},
  gemm_f64 -- all pinned by the reference's known-answer tests, f64 ground
  truth, invariants and central-difference gradchecks.
  conv2d_backward's weight/bias gradient: the reference folds with a run-time
  chosen Rayon partition, so its exact bits cannot be reproduced by anyone;
  the restatement is pinned to tolerance (gradcheck + f64), not to bits.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
I64 = ctypes.c_int64


def build() -> None:
    """Compile liboracle.so in place (gcc; no GPU needed)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(_LIB_PATH)
        sig = {
            "orc_dot_simd": (ctypes.c_float, [f32p, f32p, I64]),
            "orc_matmul_simd": (None, [f32p, f32p, f32p, I64, I64, I64, ctypes.c_int]),
            "orc_matmul_simd_rows": (None, [f32p, f32p, f32p, I64, I64, I64, I64, I64, ctypes.c_int]),
            "orc_matmul_naive": (None, [f32p, f32p, f32p, I64, I64, I64]),
            "orc_graph_matmul_forward": (None, [f32p, f32p, f32p, I64, I64, I64]),
            "orc_graph_matmul_backward": (None, [f32p, f32p, f32p, f32p, f32p, I64, I64, I64]),
            "orc_graph_bmm_forward": (None, [f32p, f32p, f32p, I64, I64, I64, I64]),
            "orc_graph_bmm_backward": (None, [f32p, f32p, f32p, f32p, f32p, I64, I64, I64, I64]),
            "orc_graph_add_bias_forward": (None, [f32p, f32p, f32p, I64, I64]),
            "orc_graph_add_bias_backward": (None, [f32p, f32p, f32p, I64, I64]),
            "orc_im2col": (None, [f32p, f32p] + [I64] * 8),
            "orc_conv2d_im2col": (None, [f32p, f32p, f32p, f32p] + [I64] * 9 + [ctypes.c_int]),
            "orc_conv2d_forward": (None, [f32p, f32p, f32p, f32p] + [I64] * 9),
            "orc_conv2d_backward": (None, [f32p, f32p, f32p, f32p, f32p, f32p] + [I64] * 9),
            "orc_gpu_im2col": (None, [f32p, f32p] + [I64] * 8),
            "orc_gpu_col2out": (None, [f32p, f32p, f32p, I64, I64, I64]),
            "orc_gpu_out2mm": (None, [f32p, f32p, I64, I64, I64]),
            "orc_gpu_col2im": (None, [f32p, f32p] + [I64] * 8),
            "orc_gpu_bias_grad": (None, [f32p, f32p, I64, I64, I64]),
            "orc_sum_axis0": (None, [f32p, f32p, I64, I64]),
            "orc_maxpool_forward": (None, [f32p, f32p, i32p] + [I64] * 6),
            "orc_maxpool_backward": (None, [f32p, i32p, f32p, I64]),
            "orc_gemm_f64": (None, [ctypes.c_int, f32p, f32p, f64p, f64p, I64, I64, I64]),
            "orc_gemm_f64_rowset": (None, [ctypes.c_int, f32p, f32p, f64p, f64p, I64, I64, I64,
                                           i64p, I64]),
            "orc_max_threads": (ctypes.c_int, []),
            "orc_set_threads": (None, [ctypes.c_int]),
            "orc_transpose": (None, [f32p, f32p, I64, I64, I64]),
            "orc_transpose_backward": (None, [f32p, f32p, I64, I64, I64]),
            "orc_scale": (None, [f32p, f32p, ctypes.c_float, I64]),
            "orc_scale_backward": (None, [f32p, f32p, ctypes.c_float, I64]),
            "orc_softmax_forward": (None, [f32p, f32p, I64, I64]),
            "orc_softmax_backward": (None, [f32p, f32p, f32p, I64, I64]),
            "orc_relu_forward": (None, [f32p, f32p, I64]),
            "orc_cross_entropy_loss": (ctypes.c_float, [f32p, f32p, I64, I64]),
            "orc_cross_entropy_grad": (None, [f32p, f32p, f32p, I64, I64]),
            "orc_relu_backward": (None, [f32p, f32p, f32p, I64]),
            "orc_slice_cols": (None, [f32p, f32p, I64, I64, I64, I64]),
            "orc_layernorm_forward": (None, [f32p] * 6 + [I64, I64, ctypes.c_float]),
            "orc_layernorm_backward": (None, [f32p] * 7 + [I64, I64]),
            "orc_slice_cols_backward": (None, [f32p, f32p, I64, I64, I64, I64]),
            "orc_concat_part": (None, [f32p, f32p, I64, I64, I64, I64]),
            "orc_concat_part_backward": (None, [f32p, f32p, I64, I64, I64, I64]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


# --- src/ops/simd.rs -------------------------------------------------------
def dot_simd(a, b) -> np.float32:
    a, b = _f32(a), _f32(b)
    assert a.shape == b.shape
    return np.float32(lib().orc_dot_simd(a, b, a.size))


def matmul_simd(a, b, nthreads: int = 0):
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    k2, n = b.shape
    if k != k2:
        raise ValueError("Shapes are not matching")
    c = np.empty((m, n), np.float32)
    lib().orc_matmul_simd(a, b, c, m, k, n, nthreads)
    return c


def matmul_simd_rows(a, b, row0: int, rows: int, nthreads: int = 0):
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((rows, n), np.float32)
    lib().orc_matmul_simd_rows(a, b, c, m, k, n, row0, rows, nthreads)
    return c


def matmul_naive(a, b):
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float32)
    lib().orc_matmul_naive(a, b, c, m, k, n)
    return c


# --- src/autograd/graph/{matmul,bmm,add}.rs ---------------------------------
def graph_matmul_forward(a, b):
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float32)
    lib().orc_graph_matmul_forward(a, b, c, m, k, n)
    return c


def graph_matmul_backward(a, b, g, da=None, db=None):
    """Returns (da, db) after ``+=`` of the matmul gradients (matmul.rs:37-63)."""
    a, b, g = _f32(a), _f32(b), _f32(g)
    m, k = a.shape
    n = b.shape[1]
    da = np.zeros((m, k), np.float32) if da is None else _f32(da).copy()
    db = np.zeros((k, n), np.float32) if db is None else _f32(db).copy()
    lib().orc_graph_matmul_backward(a, b, g, da, db, m, k, n)
    return da, db


def graph_bmm_forward(a, b):
    a, b = _f32(a), _f32(b)
    bt, m, k = a.shape
    n = b.shape[2]
    c = np.empty((bt, m, n), np.float32)
    lib().orc_graph_bmm_forward(a, b, c, bt, m, k, n)
    return c


def graph_bmm_backward(a, b, g, da=None, db=None):
    a, b, g = _f32(a), _f32(b), _f32(g)
    bt, m, k = a.shape
    n = b.shape[2]
    da = np.zeros(a.shape, np.float32) if da is None else _f32(da).copy()
    db = np.zeros(b.shape, np.float32) if db is None else _f32(db).copy()
    lib().orc_graph_bmm_backward(a, b, g, da, db, bt, m, k, n)
    return da, db


def graph_add_bias_forward(a, bias):
    a, bias = _f32(a), _f32(bias)
    rows, cols = a.shape
    out = np.empty_like(a)
    lib().orc_graph_add_bias_forward(a, bias, out, rows, cols)
    return out


def graph_add_bias_backward(g, da=None, dbias=None):
    g = _f32(g)
    rows, cols = g.shape
    da = np.zeros_like(g) if da is None else _f32(da).copy()
    dbias = np.zeros(cols, np.float32) if dbias is None else _f32(dbias).copy()
    lib().orc_graph_add_bias_backward(g, da, dbias, rows, cols)
    return da, dbias


# --- src/ops/im2col.rs, src/nn/conv.rs --------------------------------------
def conv_out_hw(in_h, in_w, kh, kw, stride, pad):
    return (in_h + 2 * pad - kh) // stride + 1, (in_w + 2 * pad - kw) // stride + 1


def im2col(data, n, c, in_h, in_w, kh, kw, stride, pad):
    data = _f32(data)
    oh, ow = conv_out_hw(in_h, in_w, kh, kw, stride, pad)
    col = np.empty(n * c * kh * kw * oh * ow, np.float32)
    lib().orc_im2col(data, col, n, c, in_h, in_w, kh, kw, stride, pad)
    return col, c * kh * kw, oh * ow


def conv2d_im2col(data, weight, bias, n, c_in, c_out, in_h, in_w, kh, kw, stride, pad,
                  nthreads: int = 0):
    data, weight, bias = _f32(data), _f32(weight), _f32(bias)
    oh, ow = conv_out_hw(in_h, in_w, kh, kw, stride, pad)
    out = np.empty(n * c_out * oh * ow, np.float32)
    lib().orc_conv2d_im2col(data, weight, bias, out, n, c_in, c_out, in_h, in_w, kh, kw,
                            stride, pad, nthreads)
    return out, oh, ow


def conv2d_forward(inp, weight, bias, n, c_in, c_out, in_h, in_w, kh, kw, stride, pad):
    inp, weight, bias = _f32(inp), _f32(weight), _f32(bias)
    oh, ow = conv_out_hw(in_h, in_w, kh, kw, stride, pad)
    out = np.empty(n * c_out * oh * ow, np.float32)
    lib().orc_conv2d_forward(inp, weight, bias, out, n, c_in, c_out, in_h, in_w, kh, kw,
                             stride, pad)
    return out, oh, ow


def conv2d_backward(inp, weight, grad, n, c_in, c_out, in_h, in_w, kh, kw, stride, pad):
    """Returns (dinput, dweight, dbias) of nn::conv::Conv2d (conv.rs:110-200)."""
    inp, weight, grad = _f32(inp), _f32(weight), _f32(grad)
    di = np.zeros(n * c_in * in_h * in_w, np.float32)
    dw = np.zeros(c_out * c_in * kh * kw, np.float32)
    db = np.zeros(c_out, np.float32)
    lib().orc_conv2d_backward(inp, weight, grad, di, dw, db, n, c_in, c_out, in_h, in_w, kh, kw,
                              stride, pad)
    return di, dw, db


# --- GPU primitive index semantics (src/cuda/nn/conv.rs, reduce.rs, maxpool.rs)
def gpu_im2col(inp, N, c_in, in_h, in_w, kh, kw, stride, pad):
    inp = _f32(inp)
    oh, ow = conv_out_hw(in_h, in_w, kh, kw, stride, pad)
    cols = np.empty((c_in * kh * kw, N * oh * ow), np.float32)
    lib().orc_gpu_im2col(inp, cols, N, c_in, in_h, in_w, kh, kw, stride, pad)
    return cols


def gpu_col2out(mm, bias, N, c_out, P):
    mm, bias = _f32(mm), _f32(bias)
    out = np.empty(N * c_out * P, np.float32)
    lib().orc_gpu_col2out(mm, bias, out, N, c_out, P)
    return out


def gpu_out2mm(grad, N, c_out, P):
    grad = _f32(grad)
    mm = np.empty((c_out, N * P), np.float32)
    lib().orc_gpu_out2mm(grad, mm, N, c_out, P)
    return mm


def gpu_col2im(dcols, N, c_in, in_h, in_w, kh, kw, stride, pad):
    dcols = _f32(dcols)
    di = np.empty(N * c_in * in_h * in_w, np.float32)
    lib().orc_gpu_col2im(dcols, di, N, c_in, in_h, in_w, kh, kw, stride, pad)
    return di


def gpu_bias_grad(grad, N, c_out, P):
    grad = _f32(grad)
    db = np.empty(c_out, np.float32)
    lib().orc_gpu_bias_grad(grad, db, N, c_out, P)
    return db


def sum_axis0(x):
    x = _f32(x)
    rows, cols = x.shape
    out = np.empty(cols, np.float32)
    lib().orc_sum_axis0(x, out, rows, cols)
    return out


def maxpool_forward(inp, N, C, in_h, in_w, k, stride):
    inp = _f32(inp)
    oh, ow = (in_h - k) // stride + 1, (in_w - k) // stride + 1
    out = np.empty(N * C * oh * ow, np.float32)
    am = np.empty(N * C * oh * ow, np.int32)
    lib().orc_maxpool_forward(inp, out, am, N, C, in_h, in_w, k, stride)
    return out, am


def maxpool_backward(grad, argmax, in_len, dinput=None):
    grad = _f32(grad)
    argmax = np.ascontiguousarray(argmax, np.int32)
    di = np.zeros(in_len, np.float32) if dinput is None else _f32(dinput).copy()
    lib().orc_maxpool_backward(grad, argmax, di, grad.size)
    return di


# --- f64 ground truth -------------------------------------------------------
LAYOUTS = {"nn": 0, "nt": 1, "tn": 2}


def gemm_f64(layout, a, b, rows, cols, inner, rowidx=None):
    """f64 product and sum|a||b| for layout nn/nt/tn (optionally selected rows)."""
    a, b = _f32(a), _f32(b)
    lay = LAYOUTS[layout] if isinstance(layout, str) else int(layout)
    if rowidx is None:
        c = np.empty((rows, cols), np.float64)
        ab = np.empty((rows, cols), np.float64)
        lib().orc_gemm_f64(lay, a, b, c, ab, rows, cols, inner)
    else:
        rowidx = np.ascontiguousarray(rowidx, np.int64)
        c = np.empty((rowidx.size, cols), np.float64)
        ab = np.empty((rowidx.size, cols), np.float64)
        lib().orc_gemm_f64_rowset(lay, a, b, c, ab, rows, cols, inner, rowidx, rowidx.size)
    return c, ab


def transpose(x, batch, rows, cols):
    x = _f32(x)
    out = np.empty(batch * rows * cols, np.float32)
    lib().orc_transpose(x.ravel(), out, batch, rows, cols)
    return out


def transpose_backward(g, ga, batch, rows, cols):
    lib().orc_transpose_backward(_f32(g).ravel(), ga, batch, rows, cols)


def scale(x, s):
    x = _f32(x).ravel()
    out = np.empty_like(x)
    lib().orc_scale(x, out, float(s), x.size)
    return out


def scale_backward(g, ga, s):
    lib().orc_scale_backward(_f32(g).ravel(), ga, float(s), ga.size)


def softmax_forward(x, width):
    x = _f32(x).ravel()
    out = np.empty_like(x)
    lib().orc_softmax_forward(x, out, x.size // width, width)
    return out


def softmax_backward(y, g, ga, width):
    y = _f32(y).ravel()
    lib().orc_softmax_backward(y, _f32(g).ravel(), ga, y.size // width, width)


def slice_cols(a, rows, total_cols, col_start, col_end):
    out = np.empty(rows * (col_end - col_start), np.float32)
    lib().orc_slice_cols(_f32(a).ravel(), out, rows, total_cols, col_start, col_end)
    return out


def slice_cols_backward(grad, ga, rows, total_cols, col_start, col_end):
    lib().orc_slice_cols_backward(_f32(grad).ravel(), ga, rows, total_cols, col_start, col_end)


def concat_cols(parts, rows):
    """parts side by side along the last dim (one orc_concat_part each)."""
    widths = [np.asarray(p).size // rows for p in parts]
    total = sum(widths)
    out = np.empty(rows * total, np.float32)
    off = 0
    for p, w in zip(parts, widths):
        lib().orc_concat_part(_f32(p).ravel(), out, rows, total, off, w)
        off += w
    return out


def concat_cols_backward(grad, gparts, rows):
    """gparts[i] += its column block of grad, in place."""
    widths = [g.size // rows for g in gparts]
    total, off = sum(widths), 0
    for gp, w in zip(gparts, widths):
        lib().orc_concat_part_backward(_f32(grad).ravel(), gp, rows, total, off, w)
        off += w


def layernorm_forward(x, gamma, beta, rows, features, eps):
    """(out, x_norm, inv_std) of nn::normalization::LayerNorm's forward."""
    out = np.empty(rows * features, np.float32)
    xn = np.empty(rows * features, np.float32)
    istd = np.empty(rows, np.float32)
    lib().orc_layernorm_forward(_f32(x).ravel(), _f32(gamma).ravel(), _f32(beta).ravel(), out, xn,
                                istd, rows, features, float(eps))
    return out, xn, istd


def layernorm_backward(grad, gamma, x_norm, inv_std, din, dgamma, dbeta, rows, features):
    """Accumulates the backward into din, dgamma, dbeta (float32 arrays)."""
    lib().orc_layernorm_backward(_f32(grad).ravel(), _f32(gamma).ravel(), _f32(x_norm).ravel(),
                                 _f32(inv_std).ravel(), din, dgamma, dbeta, rows, features)


def cross_entropy_loss(logits, target, classes):
    """CrossEntropyLoss::forward (src/nn/loss.rs:49-75): batch-mean loss."""
    logits, target = _f32(logits).ravel(), _f32(target).ravel()
    return float(lib().orc_cross_entropy_loss(logits, target, logits.size // classes, classes))


def cross_entropy_grad(logits, target, classes):
    """CrossEntropyLoss::backward's seed (src/nn/loss.rs:77-106): (softmax - t) / batch."""
    logits, target = _f32(logits).ravel(), _f32(target).ravel()
    out = np.empty_like(logits)
    lib().orc_cross_entropy_grad(logits, target, out, logits.size // classes, classes)
    return out


def relu_forward(x):
    x = _f32(x).ravel()
    out = np.empty_like(x)
    lib().orc_relu_forward(x, out, x.size)
    return out


def relu_backward(x, g, ga):
    x = _f32(x).ravel()
    lib().orc_relu_backward(x, _f32(g).ravel(), ga, x.size)


def max_threads() -> int:
    return int(lib().orc_max_threads())


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))
