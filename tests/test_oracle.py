"""Pins the CPU oracle (oracle/nrs_oracle.c) before anything is checked against it.

Each oracle function is checked by at least one of:
  * the reference's own known answers (tests/golden/reference_kats.json);
  * exact integer arithmetic against numpy's int64 routines (small-integer f32
    inputs make every partial sum exact, so an index, sign or transpose
    mistake changes the integer result);
  * f64 ground truth with the deterministic rounding bound gamma_K;
  * adjoint identities (<conv(x), g> == <x, dconv(g)>) and central-difference
    gradchecks, as the reference's gradcheck tests do.
No test retypes the oracle's own loop.
"""
import numpy as np
import pytest

from kat import formula, int_matrix, kats

K = kats()
U = np.finfo(np.float32).eps / 2  # unit roundoff 2^-24


def gamma(n):
    return n * U / (1 - n * U)


# ---------------------------------------------------------------- dot_simd
def test_dot_simd_known_answers(orc):
    for case in K["dot_simd"]:
        r = orc.dot_simd(np.array(case["a"], np.float32), np.array(case["b"], np.float32))
        assert abs(r - case["expect"]) < case["tol"], case["src"]


def test_dot_simd_vs_naive(orc):
    c = K["dot_simd_vs_naive"]
    a = formula(c["a"], c["n"])
    b = formula(c["b"], c["n"])
    naive = np.float32(0)
    for x, y in zip(a, b):
        naive = np.float32(naive + np.float32(x * y))
    assert abs(orc.dot_simd(a, b) - naive) < c["tol"]


@pytest.mark.parametrize("n", [0, 1, 7, 8, 9, 15, 16, 17, 1000])
def test_dot_simd_unit_vectors_and_integers(orc, n):
    rng = np.random.default_rng(n)
    a = int_matrix(rng, (n,))
    b = int_matrix(rng, (n,))
    assert orc.dot_simd(a, b) == np.float32(int(np.dot(a.astype(np.int64), b.astype(np.int64))))
    for j in range(n):  # picks every lane and every tail position exactly once
        e = np.zeros(n, np.float32)
        e[j] = 1.0
        assert orc.dot_simd(a, e) == a[j]


# ---------------------------------------------------------------- matmul
@pytest.mark.parametrize("fn", ["matmul_simd", "matmul_naive", "graph_matmul_forward"])
def test_matmul_known_answers(orc, fn):
    for case in K["matmul"]:
        a = np.array(case["a"], np.float32).reshape(case["a_shape"])
        b = np.array(case["b"], np.float32).reshape(case["b_shape"])
        c = getattr(orc, fn)(a, b).ravel()
        if case.get("exact"):
            assert c.tolist() == case["expect"], case["src"]
        else:
            assert np.all(np.abs(c - np.array(case["expect"])) < case["tol"]), case["src"]


def test_matmul_simd_vs_naive(orc):
    c = K["matmul_simd_vs_naive"]
    a = formula(c["a"], c["m"] * c["k"]).reshape(c["m"], c["k"])
    b = formula(c["b"], c["k"] * c["n"]).reshape(c["k"], c["n"])
    assert np.all(np.abs(orc.matmul_simd(a, b) - orc.matmul_naive(a, b)) < c["tol"])


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 2), (17, 33, 9), (64, 129, 31)])
def test_matmul_exact_integers(orc, m, k, n):
    rng = np.random.default_rng(m * 1000 + k)
    a = int_matrix(rng, (m, k))
    b = int_matrix(rng, (k, n))
    ref = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    for fn in ("matmul_simd", "matmul_naive", "graph_matmul_forward"):
        assert np.array_equal(getattr(orc, fn)(a, b), ref), fn


def test_matmul_simd_f64_bound(orc):
    """cfg1 (512^3, U(-1,1), seed 0): the f32 result sits inside gamma_K of f64."""
    rng = np.random.default_rng(0)
    a = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    b = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    c = orc.matmul_simd(a, b)
    c64 = a.astype(np.float64) @ b.astype(np.float64)
    ab = np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))
    assert np.all(np.abs(c - c64) <= gamma(512) * ab)
    rows = np.arange(0, 512, 37)
    c64o, abo = orc.gemm_f64("nn", a, b, 512, 512, 512, rowidx=rows)
    assert np.allclose(c64o, c64[rows], rtol=1e-12, atol=1e-12)
    assert np.allclose(abo, ab[rows], rtol=1e-12, atol=1e-12)


def test_matmul_simd_rows_is_row_slice(orc):
    rng = np.random.default_rng(5)
    a = rng.uniform(-1, 1, (40, 24)).astype(np.float32)
    b = rng.uniform(-1, 1, (24, 13)).astype(np.float32)
    full = orc.matmul_simd(a, b)
    assert np.array_equal(orc.matmul_simd_rows(a, b, 7, 11), full[7:18])


@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
def test_gemm_f64_layouts(orc, layout):
    rng = np.random.default_rng(11)
    rows, cols, inner = 9, 7, 5
    a = int_matrix(rng, (rows, inner) if layout != "tn" else (inner, rows))
    b = int_matrix(rng, (inner, cols) if layout != "nt" else (cols, inner))
    A = a if layout != "tn" else a.T
    B = b if layout != "nt" else b.T
    c, ab = orc.gemm_f64(layout, a, b, rows, cols, inner)
    assert np.array_equal(c, A.astype(np.float64) @ B.astype(np.float64))
    assert np.array_equal(ab, np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64)))


def test_graph_matmul_backward_exact_and_gradcheck(orc):
    rng = np.random.default_rng(3)
    m, k, n = 6, 5, 4
    a, b, g = int_matrix(rng, (m, k)), int_matrix(rng, (k, n)), int_matrix(rng, (m, n))
    da0, db0 = int_matrix(rng, (m, k)), int_matrix(rng, (k, n))
    da, db = orc.graph_matmul_backward(a, b, g, da0, db0)
    ai, bi, gi = (x.astype(np.int64) for x in (a, b, g))
    assert np.array_equal(da, da0 + (gi @ bi.T).astype(np.float32))
    assert np.array_equal(db, db0 + (ai.T @ gi).astype(np.float32))


def _literal_graph_matmul(a, b, g, da0, db0):
    """The reference's loops of src/autograd/graph/matmul.rs:17-63 verbatim in
    numpy float32 scalars (every product and sum rounded to f32, no fused
    multiply-add): forward data[i,j] += a[i,t]*b[t,j] over t; dA[i,t] +=
    sum_j g[i,j]*b[t,j]; dB[t,j] += sum_i a[i,t]*g[i,j]."""
    f = np.float32
    m, k = a.shape
    n = b.shape[1]
    c = np.zeros((m, n), np.float32)
    for i in range(m):
        for j in range(n):
            s = f(0)
            for t in range(k):
                s = f(s + f(a[i, t] * b[t, j]))
            c[i, j] = s
    da, db = da0.copy(), db0.copy()
    for i in range(m):
        for t in range(k):
            s = f(0)
            for j in range(n):
                s = f(s + f(g[i, j] * b[t, j]))
            da[i, t] = f(da[i, t] + s)
    for t in range(k):
        for j in range(n):
            s = f(0)
            for i in range(m):
                s = f(s + f(a[i, t] * g[i, j]))
            db[t, j] = f(db[t, j] + s)
    return c, da, db


@pytest.mark.parametrize("m,k,n", [(7, 13, 5), (12, 9, 17), (1, 1, 1)])
def test_graph_matmul_loop_order_is_bit_exact(orc, m, k, n):
    """The oracle runs the reference's loops with reordered nests; on random
    (non-integer) data its bits equal the literal loops', so each output's
    sequence of roundings is the reference's."""
    rng = np.random.default_rng(m * 31 + k * 7 + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    g = rng.standard_normal((m, n)).astype(np.float32)
    da0 = rng.standard_normal((m, k)).astype(np.float32)
    db0 = rng.standard_normal((k, n)).astype(np.float32)
    c_ref, da_ref, db_ref = _literal_graph_matmul(a, b, g, da0, db0)
    assert np.array_equal(orc.graph_matmul_forward(a, b), c_ref)
    da, db = orc.graph_matmul_backward(a, b, g, da0, db0)
    assert np.array_equal(da, da_ref)
    assert np.array_equal(db, db_ref)


# ---------------------------------------------------------------- bmm
def test_bmm_known_answer_and_gradcheck(orc):
    c = K["bmm_forward"]
    a = np.array(c["a"], np.float32).reshape(c["a_shape"])
    b = np.array(c["b"], np.float32).reshape(c["b_shape"])
    assert np.all(np.abs(orc.graph_bmm_forward(a, b).ravel() - c["expect"]) < c["tol"])

    c = K["bmm_gradcheck"]
    a = np.array(c["a"], np.float32).reshape(c["a_shape"])
    b = np.array(c["b"], np.float32).reshape(c["b_shape"])
    out = orc.graph_bmm_forward(a, b)
    da, db = orc.graph_bmm_backward(a, b, np.ones_like(out))
    h = np.float32(c["h"])
    for x, dx in ((a, da), (b, db)):
        for i in range(x.size):
            xp, xm = x.copy(), x.copy()
            xp.flat[i] += h
            xm.flat[i] -= h
            if x is a:
                lp, lm = orc.graph_bmm_forward(xp, b).sum(dtype=np.float32), orc.graph_bmm_forward(xm, b).sum(dtype=np.float32)
            else:
                lp, lm = orc.graph_bmm_forward(a, xp).sum(dtype=np.float32), orc.graph_bmm_forward(a, xm).sum(dtype=np.float32)
            assert abs((lp - lm) / (2 * h) - dx.flat[i]) < c["tol"]


def test_bmm_exact_integers(orc):
    rng = np.random.default_rng(4)
    bt, m, k, n = 3, 5, 7, 4
    a, b, g = int_matrix(rng, (bt, m, k)), int_matrix(rng, (bt, k, n)), int_matrix(rng, (bt, m, n))
    ai, bi, gi = (x.astype(np.int64) for x in (a, b, g))
    assert np.array_equal(orc.graph_bmm_forward(a, b), np.matmul(ai, bi).astype(np.float32))
    da, db = orc.graph_bmm_backward(a, b, g)
    assert np.array_equal(da, np.matmul(gi, bi.transpose(0, 2, 1)).astype(np.float32))
    assert np.array_equal(db, np.matmul(ai.transpose(0, 2, 1), gi).astype(np.float32))


# ---------------------------------------------------------------- add / Linear
def test_linear_batch_known_answer(orc):
    c = K["linear_batch"]
    x = np.array(c["x"], np.float32).reshape(c["x_shape"])
    w = np.array(c["w"], np.float32).reshape(c["w_shape"])
    y = orc.graph_add_bias_forward(orc.graph_matmul_forward(x, w), np.array(c["bias"], np.float32))
    assert y.ravel().tolist() == c["expect"]
    _, db = orc.graph_add_bias_backward(np.array(c["seed"], np.float32).reshape(y.shape))
    assert db.tolist() == c["expect_bias_grad"]


def test_sum_axis0_exact(orc):
    rng = np.random.default_rng(8)
    x = int_matrix(rng, (37, 11))
    assert np.array_equal(orc.sum_axis0(x), x.astype(np.int64).sum(0).astype(np.float32))


# ---------------------------------------------------------------- im2col / conv
def _np_conv(x, w, b, stride, pad):
    """Independent int64 convolution via numpy sliding windows."""
    n, c, h, wd = x.shape
    co, _, kh, kw = w.shape
    xp = np.pad(x.astype(np.int64), ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    win = np.lib.stride_tricks.sliding_window_view(xp, (kh, kw), axis=(2, 3))[:, :, ::stride, ::stride]
    out = np.einsum("ncyxij,ocij->noyx", win, w.astype(np.int64))
    return out + b.astype(np.int64)[None, :, None, None]


def test_im2col_known_answer(orc):
    c = K["im2col"]
    d = c["dims"]
    col, ch, cw = orc.im2col(np.array(c["data"], np.float32), d["n"], d["c"], d["in_h"], d["in_w"],
                             d["kh"], d["kw"], d["stride"], d["pad"])
    assert (ch, cw) == (c["expect_col_h"], c["expect_col_w"])
    assert col.tolist() == c["expect"]
    g = orc.gpu_im2col(np.array(c["data"], np.float32), d["n"], d["c"], d["in_h"], d["in_w"],
                       d["kh"], d["kw"], d["stride"], d["pad"])
    assert g.ravel().tolist() == c["expect"]  # N=1: both layouts coincide


def test_conv_forward_known_answers(orc):
    for c in K["conv_forward"]:
        n, ci, h, w = c["in_shape"]
        co, _, kh, kw = c["w_shape"]
        args = (np.array(c["input"], np.float32), np.array(c["weight"], np.float32),
                np.array(c["bias"], np.float32), n, ci, co, h, w, kh, kw, c["stride"], c["pad"])
        out, oh, ow = orc.conv2d_forward(*args)
        assert [n, co, oh, ow] == c["expect_shape"], c["src"]
        assert out.tolist() == c["expect"], c["src"]
        out2, _, _ = orc.conv2d_im2col(*args)
        assert out2.tolist() == c["expect"], c["src"]


def test_im2col_conv_matches_direct(orc):
    c = K["im2col_conv"]
    d = c["dims"]
    w_len = d["c_out"] * d["c_in"] * d["kh"] * d["kw"]
    weight = formula(c["weight"], w_len)
    bias = (np.arange(d["c_out"], dtype=np.float32) * np.float32(c["bias_scale"])).astype(np.float32)
    data = formula(c["data"], d["n"] * d["c_in"] * d["in_h"] * d["in_w"])
    args = (data, weight, bias, d["n"], d["c_in"], d["c_out"], d["in_h"], d["in_w"], d["kh"], d["kw"],
            d["stride"], d["pad"])
    a, _, _ = orc.conv2d_im2col(*args)
    b, _, _ = orc.conv2d_forward(*args)
    assert np.all(np.abs(a - b) < c["tol"])


CONV_SHAPES = [  # (n, c_in, c_out, h, w, kh, kw, stride, pad)
    (2, 3, 4, 8, 8, 3, 3, 1, 1),
    (2, 3, 5, 7, 7, 3, 3, 1, 1),
    (1, 2, 3, 9, 6, 3, 2, 2, 1),
    (3, 1, 2, 5, 5, 2, 2, 1, 0),
    (2, 2, 2, 7, 9, 3, 3, 3, 2),
]


@pytest.mark.parametrize("shape", CONV_SHAPES)
def test_conv_exact_integers(orc, shape):
    n, ci, co, h, w, kh, kw, s, p = shape
    rng = np.random.default_rng(sum(shape))
    x = int_matrix(rng, (n, ci, h, w), -4, 4)
    wt = int_matrix(rng, (co, ci, kh, kw), -4, 4)
    b = int_matrix(rng, (co,), -4, 4)
    ref = _np_conv(x, wt, b, s, p).astype(np.float32)
    out, oh, ow = orc.conv2d_forward(x, wt, b, n, ci, co, h, w, kh, kw, s, p)
    assert np.array_equal(out, ref.ravel())
    out2, _, _ = orc.conv2d_im2col(x, wt, b, n, ci, co, h, w, kh, kw, s, p)
    assert np.array_equal(out2, ref.ravel())

    # im2col (CPU layout [n][col_h][P]) and the GPU layout [col_h][n*P] agree.
    col, ch, P = orc.im2col(x, n, ci, h, w, kh, kw, s, p)
    gcol = orc.gpu_im2col(x, n, ci, h, w, kh, kw, s, p)
    assert np.array_equal(col.reshape(n, ch, P).transpose(1, 0, 2).reshape(ch, n * P), gcol)

    # Backward: adjoint identities in exact integer arithmetic.
    g = int_matrix(rng, (n, co, oh, ow), -4, 4)
    di, dw, db = orc.conv2d_backward(x, wt, g, n, ci, co, h, w, kh, kw, s, p)
    zero_b = np.zeros(co, np.float32)
    gi = g.astype(np.int64).ravel()
    # <conv(x'), g> == <x', dinput>  for a random x'
    x2 = int_matrix(rng, x.shape, -4, 4)
    lhs = int(_np_conv(x2, wt, zero_b, s, p).ravel() @ gi)
    assert lhs == int(x2.astype(np.int64).ravel() @ di.astype(np.int64))
    # <conv_w'(x), g> == <w', dweight> for a random w'
    w2 = int_matrix(rng, wt.shape, -4, 4)
    lhs = int(_np_conv(x, w2, zero_b, s, p).ravel() @ gi)
    assert lhs == int(w2.astype(np.int64).ravel() @ dw.astype(np.int64))
    assert np.array_equal(db, g.astype(np.int64).sum(axis=(0, 2, 3)).astype(np.float32))

    # GPU-layout primitives: col2im is the adjoint of im2col, col2out/out2mm
    # are the NCHW <-> [c_out, N*P] reorders (+ bias), bias_grad sums.
    y = int_matrix(rng, gcol.shape, -4, 4)
    dx = orc.gpu_col2im(y, n, ci, h, w, kh, kw, s, p)
    assert int(gcol.astype(np.int64).ravel() @ y.astype(np.int64).ravel()) == \
        int(x.astype(np.int64).ravel() @ dx.astype(np.int64))
    mm = orc.gpu_out2mm(g, n, co, oh * ow)
    assert np.array_equal(mm, g.reshape(n, co, oh * ow).transpose(1, 0, 2).reshape(co, n * oh * ow))
    assert np.array_equal(orc.gpu_col2out(mm, b, n, co, oh * ow), (g + b[None, :, None, None]).ravel())
    assert np.array_equal(orc.gpu_bias_grad(g, n, co, oh * ow), db)


def test_conv_gradchecks(orc):
    """tests/gradcheck_conv_test.rs: loss = sum (i+1) * out_i, h = 1e-3."""
    c = K["conv_gradcheck"]
    x = np.array(c["input"], np.float32)
    w = np.array(c["weight"], np.float32)
    b = np.array(c["bias"], np.float32)
    n, ci, h_, w_ = c["in_shape"]
    co, _, kh, kw = c["w_shape"]
    h = np.float32(c["h"])

    for pad, tol_in in ((0, c["tol_input"]), (c["padded_pad"], c["tol_padded_input"])):
        def loss(xx, ww, bb):
            out, _, _ = orc.conv2d_forward(xx, ww, bb, n, ci, co, h_, w_, kh, kw, 1, pad)
            return np.float32(np.sum(np.arange(1, out.size + 1, dtype=np.float32) * out, dtype=np.float32))

        out, _, _ = orc.conv2d_forward(x, w, b, n, ci, co, h_, w_, kh, kw, 1, pad)
        g = np.arange(1, out.size + 1, dtype=np.float32)
        di, dw, db = orc.conv2d_backward(x, w, g, n, ci, co, h_, w_, kh, kw, 1, pad)
        checks = [(x, di, tol_in, 0)]
        if pad == 0:  # the reference checks weight/bias grads unpadded only
            checks += [(w, dw, c["tol_weight"], 1), (b, db, c["tol_bias"], 2)]
        for vec, grad, tol, which in checks:
            for i in range(vec.size):
                vp, vm = vec.copy(), vec.copy()
                vp[i] += h
                vm[i] -= h
                argsp = [x, w, b]
                argsm = [x, w, b]
                argsp[which], argsm[which] = vp, vm
                num = (loss(*argsp) - loss(*argsm)) / (2 * h)
                assert abs(num - grad[i]) < tol, (pad, which, i, num, grad[i])


def test_maxpool_exact(orc):
    rng = np.random.default_rng(12)
    n, c, h, w, k, s = 2, 3, 6, 8, 2, 2
    x = rng.permutation(n * c * h * w).astype(np.float32)  # distinct values: argmax unique
    out, am = orc.maxpool_forward(x, n, c, h, w, k, s)
    win = np.lib.stride_tricks.sliding_window_view(x.reshape(n, c, h, w), (k, k), axis=(2, 3))[:, :, ::s, ::s]
    assert np.array_equal(out, win.max(axis=(-1, -2)).ravel())
    assert np.array_equal(x[am], out)
    g = int_matrix(rng, out.shape)
    di = orc.maxpool_backward(g, am, x.size)
    assert di.sum() == g.sum() and np.array_equal(di[am], g)


# ------------------------------------------------- attention / MLP glue twins
def test_transpose_matches_numpy_and_adjoint(orc):
    rng = np.random.default_rng(5)
    b, r, c = 3, 5, 7
    x = int_matrix(rng, (b, r, c))
    assert np.array_equal(orc.transpose(x, b, r, c), x.transpose(0, 2, 1).ravel())
    # backward is the adjoint: <T x, g> == <x, T^T g>, exactly for integers
    g = int_matrix(rng, (b, c, r))
    ga = np.zeros(b * r * c, np.float32)
    orc.transpose_backward(g, ga, b, r, c)
    assert np.array_equal(ga, g.transpose(0, 2, 1).ravel())
    lhs = np.dot(orc.transpose(x, b, r, c).astype(np.int64), g.ravel().astype(np.int64))
    assert lhs == np.dot(x.ravel().astype(np.int64), ga.astype(np.int64))


def test_scale_exact_and_backward(orc):
    rng = np.random.default_rng(6)
    x = int_matrix(rng, (257,))
    assert np.array_equal(orc.scale(x, 0.5), x * np.float32(0.5))
    ga = np.ones(257, np.float32)
    orc.scale_backward(x, ga, 0.25)
    assert np.array_equal(ga, 1 + x * np.float32(0.25))


def test_softmax_forward_vs_scipy(orc):
    from scipy.special import softmax as sp_softmax

    rng = np.random.default_rng(7)
    for rows, width in [(1, 1), (4, 5), (32, 128), (3, 1000)]:
        x = (rng.standard_normal((rows, width)) * 3).astype(np.float32)
        y = orc.softmax_forward(x, width).reshape(rows, width)
        ref = sp_softmax(x.astype(np.float64), axis=1)
        assert np.max(np.abs(y - ref)) < 1e-6 * max(1, width) ** 0.5
        # shift invariance (the max subtraction) and huge inputs stay finite
        y2 = orc.softmax_forward(x + np.float32(80.0), width).reshape(rows, width)
        assert np.all(np.isfinite(y2)) and np.max(np.abs(y2 - y)) < 1e-5


def test_softmax_backward_gradcheck(orc):
    """ga = J^T g against central differences of the oracle's own forward."""
    rng = np.random.default_rng(8)
    rows, width = 3, 6
    x = rng.standard_normal((rows, width)).astype(np.float32)
    g = rng.standard_normal((rows, width)).astype(np.float32)
    y = orc.softmax_forward(x, width)
    ga = np.zeros(rows * width, np.float32)
    orc.softmax_backward(y, g, ga, width)
    h = 1e-3
    num = np.zeros(rows * width)
    xf = x.ravel().astype(np.float64)
    for i in range(rows * width):
        xp, xm = xf.copy(), xf.copy()
        xp[i] += h
        xm[i] -= h
        fp = np.dot(orc.softmax_forward(xp.astype(np.float32), width), g.ravel())
        fm = np.dot(orc.softmax_forward(xm.astype(np.float32), width), g.ravel())
        num[i] = (fp - fm) / (2 * h)
    assert np.max(np.abs(ga - num)) < 1e-2


def test_cross_entropy_closed_form_and_gradcheck(orc):
    """CrossEntropyLoss (src/nn/loss.rs:49-106) pinned without the reference:
    with one-hot targets the loss is the batch mean of -log softmax at the
    target class (float64 log-sum-exp); the gradient equals central
    differences of the oracle's own loss, each row of it sums to zero, and
    it equals (softmax - t) / batch through the separately pinned softmax.
    A dropped max shift, a wrong sign or a missing / batch fails one of them."""
    rng = np.random.default_rng(23)
    for batch, classes in [(1, 1), (5, 10), (16, 10), (3, 7)]:
        x = (rng.standard_normal((batch, classes)) * 3).astype(np.float32)
        cls = rng.integers(0, classes, batch)
        t = np.zeros((batch, classes), np.float32)
        t[np.arange(batch), cls] = 1.0
        x64 = x.astype(np.float64)
        m = x64.max(axis=1, keepdims=True)
        lse = np.log(np.exp(x64 - m).sum(axis=1)) + m[:, 0]
        want = np.mean(lse - x64[np.arange(batch), cls])
        loss = orc.cross_entropy_loss(x, t, classes)
        assert abs(loss - want) <= 1e-5 * max(1.0, abs(want))
        # huge logits stay finite (the max shift)
        assert np.isfinite(orc.cross_entropy_loss(x + np.float32(90.0), t, classes))
        g = orc.cross_entropy_grad(x, t, classes).reshape(batch, classes)
        assert np.max(np.abs(g.sum(axis=1))) <= 1e-6
        sm = orc.softmax_forward(x, classes).reshape(batch, classes)
        assert np.max(np.abs(g - (sm - t) / batch)) <= 1e-6
        h = 1e-2
        num = np.zeros((batch, classes))
        for i in range(batch):
            for c in range(classes):
                xp, xm = x.copy(), x.copy()
                xp[i, c] += h
                xm[i, c] -= h
                num[i, c] = (orc.cross_entropy_loss(xp, t, classes) -
                             orc.cross_entropy_loss(xm, t, classes)) / (2 * h)
        assert np.max(np.abs(g - num)) < 2e-3


def test_relu_exact_and_mask(orc):
    rng = np.random.default_rng(9)
    x = int_matrix(rng, (300,))
    assert np.array_equal(orc.relu_forward(x), np.maximum(x, 0))
    g = int_matrix(rng, (300,))
    ga = np.zeros(300, np.float32)
    orc.relu_backward(x, g, ga)
    assert np.array_equal(ga, np.where(x > 0, g, 0).astype(np.float32))


def test_slice_concat_known_answers(orc):
    """tests/slice_concat_test.rs:5-31 and slice_concat_3d_test.rs:6-61."""
    k = kats()["slice_concat"]
    a = np.asarray(k["a"], np.float32)
    rows, total = k["shape"]
    left = orc.slice_cols(a, rows, total, *k["left"]["cols"])
    right = orc.slice_cols(a, rows, total, *k["right"]["cols"])
    assert np.array_equal(left, k["left"]["data"]) and np.array_equal(right, k["right"]["data"])
    joined = orc.concat_cols([left, right], rows)
    assert np.array_equal(joined, a)
    # backward of the round trip with a ones seed: every input column gets 1
    seed = np.full(rows * total, k["joined_grad_seed"], np.float32)
    gl, gr = np.zeros_like(left), np.zeros_like(right)
    orc.concat_cols_backward(seed, [gl, gr], rows)
    ga = np.zeros_like(a)
    orc.slice_cols_backward(gl, ga, rows, total, *k["left"]["cols"])
    orc.slice_cols_backward(gr, ga, rows, total, *k["right"]["cols"])
    assert np.array_equal(ga, np.full_like(a, k["a_grad"]))

    k3 = kats()["slice_concat_3d"]
    x = np.arange(16, dtype=np.float32)           # [2, 2, 4]: rows = 4 of the last dim
    s = orc.slice_cols(x, 4, 4, *k3["slice"]["cols"])
    assert np.array_equal(s, k3["slice"]["expected"])
    c = orc.concat_cols([np.asarray(k3["concat"]["a"], np.float32),
                         np.asarray(k3["concat"]["b"], np.float32)], 4)
    assert np.array_equal(c, k3["concat"]["expected"])
    xin = (np.arange(16) * np.float32(k3["roundtrip"]["input_scale"])).astype(np.float32)
    l3, r3 = orc.slice_cols(xin, 4, 4, 0, 2), orc.slice_cols(xin, 4, 4, 2, 4)
    assert np.array_equal(orc.concat_cols([l3, r3], 4), xin)
    g = (np.arange(16) + 1).astype(np.float32)
    gl3, gr3 = np.zeros(8, np.float32), np.zeros(8, np.float32)
    orc.concat_cols_backward(g, [gl3, gr3], 4)
    gin = np.zeros(16, np.float32)
    orc.slice_cols_backward(gl3, gin, 4, 4, 0, 2)
    orc.slice_cols_backward(gr3, gin, 4, 4, 2, 4)
    assert np.array_equal(gin, g)


def test_slice_concat_match_numpy_indexing(orc):
    """The restatement against numpy's column indexing on ragged shapes."""
    rng = np.random.default_rng(7)
    for rows, total, cs, ce in ((1, 1, 0, 1), (5, 9, 2, 7), (3, 8, 0, 8), (7, 33, 31, 33)):
        x = rng.standard_normal(rows * total).astype(np.float32)
        want = x.reshape(rows, total)[:, cs:ce].ravel()
        assert np.array_equal(orc.slice_cols(x, rows, total, cs, ce), want)
        g = rng.standard_normal(rows * (ce - cs)).astype(np.float32)
        ga = rng.standard_normal(rows * total).astype(np.float32)
        ref = ga.reshape(rows, total).copy()
        ref[:, cs:ce] += g.reshape(rows, ce - cs)
        orc.slice_cols_backward(g, ga, rows, total, cs, ce)
        assert np.array_equal(ga, ref.ravel())


def test_layernorm_known_answers_and_gradcheck(orc):
    """nn_layernorm_test.rs / layernorm_3d_test.rs (zero-mean rows with gamma 1,
    beta 0), gradcheck_layernorm_test.rs (central differences of sum(out^2),
    h = 1e-3, tol 1e-2), and an f64 restatement of the formula."""
    k = kats()["layernorm"]
    eps = k["eps"]
    for case in k["row_means"]:
        x = np.asarray(case["input"], np.float32)
        F = case["features"]
        rows = x.size // F
        out, _, _ = orc.layernorm_forward(x, np.ones(F, np.float32), np.zeros(F, np.float32),
                                          rows, F, eps)
        assert np.all(np.abs(out.reshape(rows, F).mean(axis=1)) < case["tol"])
    gc = k["gradcheck"]
    gamma, beta = np.asarray(gc["gamma"], np.float32), np.asarray(gc["beta"], np.float32)
    x = np.asarray(gc["input"], np.float32)
    F = x.size

    def loss(v):
        return float(np.sum(orc.layernorm_forward(v, gamma, beta, 1, F, eps)[0] ** 2))
    num = np.array([(loss(x + np.eye(F, dtype=np.float32)[i] * np.float32(gc["h"])) -
                     loss(x - np.eye(F, dtype=np.float32)[i] * np.float32(gc["h"]))) / (2 * gc["h"])
                    for i in range(F)])
    out, xn, istd = orc.layernorm_forward(x, gamma, beta, 1, F, eps)
    din, dg, db = np.zeros(F, np.float32), np.zeros(F, np.float32), np.zeros(F, np.float32)
    orc.layernorm_backward(2 * out, gamma, xn, istd, din, dg, db, 1, F)
    assert np.max(np.abs(num - din)) < gc["tol"]
    # f64 formula on random rows
    rng = np.random.default_rng(11)
    rows, F = 37, 70
    x = rng.standard_normal(rows * F).astype(np.float32)
    g, b = rng.standard_normal(F).astype(np.float32), rng.standard_normal(F).astype(np.float32)
    out, xn, istd = orc.layernorm_forward(x, g, b, rows, F, eps)
    x64 = x.reshape(rows, F).astype(np.float64)
    mu, var = x64.mean(axis=1, keepdims=True), x64.var(axis=1, keepdims=True)
    xn64 = (x64 - mu) / np.sqrt(var + eps)
    assert np.max(np.abs(out.reshape(rows, F) - (xn64 * g + b))) < 1e-5
    # backward against the f64 closed form (and dgamma/dbeta column sums)
    gr = rng.standard_normal(rows * F).astype(np.float32)
    din, dg, db = np.zeros(rows * F, np.float32), np.zeros(F, np.float32), np.zeros(F, np.float32)
    orc.layernorm_backward(gr, g, xn, istd, din, dg, db, rows, F)
    g64 = gr.reshape(rows, F).astype(np.float64)
    dxh = g64 * g
    want = (dxh - dxh.mean(axis=1, keepdims=True) -
            xn64 * (dxh * xn64).mean(axis=1, keepdims=True)) / np.sqrt(var + eps)
    assert np.max(np.abs(din.reshape(rows, F) - want)) < 1e-4
    assert np.max(np.abs(dg - (g64 * xn64).sum(axis=0))) < 1e-3
    assert np.max(np.abs(db - g64.sum(axis=0))) < 1e-4
