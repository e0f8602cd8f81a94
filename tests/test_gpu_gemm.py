"""Parity of the HIP GEMM core (nrs_gemm / nrs_gemm_nt_splitk / nrs_bmm)
against the CPU oracle, through the C ABI.

Bars:
  * small-integer inputs: bit-exact (every summation order is exact);
  * random f32 inputs: max_ij |C - C64| / (|A||B|)_ij <= 1e-5 * sqrt(K)
    (the north-star tolerance for f32 accumulation), against f64 ground truth;
  * the reference's twin-test tolerances against the restated CPU autograd ops.
"""
import numpy as np
import pytest

from kat import close, formula, gemm_tol, int_matrix, kats, rel_err

pytestmark = pytest.mark.gpu

NN, NT, TN = 0, 1, 2
LNAME = {NN: "nn", NT: "nt", TN: "tn"}


def operands(layout, rows, cols, inner, make):
    a = make((rows, inner) if layout != TN else (inner, rows))
    b = make((inner, cols) if layout != NT else (cols, inner))
    return a, b


def logical(layout, a, b):
    A = a if layout != TN else a.T
    B = b if layout != NT else b.T
    return A.astype(np.float64), B.astype(np.float64)


def run_gemm(hip, layout, a, b, rows, cols, inner, beta=0.0, c0=None, bias=None, epi=0):
    dA = hip.DeviceBuffer.from_host(a)
    dB = hip.DeviceBuffer.from_host(b)
    dC = hip.DeviceBuffer.from_host(c0) if c0 is not None else hip.DeviceBuffer(rows * cols)
    dbias = hip.DeviceBuffer.from_host(bias) if bias is not None else None
    hip.gemm(layout, dC, dA, dB, rows, cols, inner, beta, dbias, epi)
    return dC.to_host((rows, cols))


SHAPES = [  # (rows, cols, inner)
    (1, 1, 1), (2, 2, 2), (5, 7, 11), (17, 9, 5), (40, 32, 56), (64, 64, 16), (33, 65, 129),
    (128, 256, 64), (256, 128, 784), (100, 10, 9), (256, 10, 128), (300, 300, 300),
    (512, 512, 512), (32, 1024, 512), (1, 513, 257), (1000, 3, 2),
    (130, 17, 33), (257, 32, 96),  # at most 32 columns: 128x32 tiles, ragged rows
    (2048, 2048, 40), (4096, 1024, 72), (2000, 2048, 36),  # large outputs (the last ragged M)
    (2000, 2100, 1100),  # 128x128 tiles (one per CU), ragged edges
    (30, 8200, 1024),    # at most 32 rows: 32x256 tiles over K slices, ragged M and N
    # cfg4 Linear GEMMs (TransformerBlock, B32 S128 d256 dff1024): Q/K/V/O
    # projections and the two FFN layers forward (NN) and their input
    # gradients (NT); the weight gradients over K = 4096 rows (TN, split-K)
    (4096, 256, 256), (4096, 1024, 256), (4096, 256, 1024),
    (256, 256, 4096), (256, 1024, 4096), (1024, 256, 4096),
    # k-split wave sets (64x64 tiles, 8 waves) with ragged edges
    (1000, 260, 200), (4000, 300, 96),
]


@pytest.mark.parametrize("layout", [NN, NT, TN])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_gemm_exact_integers(hip, layout, shape):
    rows, cols, inner = shape
    rng = np.random.default_rng(rows * 7919 + cols * 31 + inner)
    a, b = operands(layout, rows, cols, inner, lambda s: int_matrix(rng, s, -4, 4))
    A, B = logical(layout, a, b)
    c = run_gemm(hip, layout, a, b, rows, cols, inner)
    assert np.array_equal(c, (A @ B).astype(np.float32)), f"{LNAME[layout]} {shape}"


@pytest.mark.parametrize("layout", [NN, NT, TN])
@pytest.mark.parametrize("shape", [(40, 32, 56), (300, 300, 300), (512, 512, 512),
                                   (256, 128, 784), (1024, 1024, 1024), (32, 2048, 2048),
                                   # cfg4 Linear GEMMs and weight gradients
                                   (4096, 256, 256), (4096, 1024, 256), (4096, 256, 1024),
                                   (256, 256, 4096), (256, 1024, 4096), (1024, 256, 4096)],
                         ids=lambda s: "x".join(map(str, s)))
def test_gemm_f64_tolerance(hip, orc, layout, shape):
    rows, cols, inner = shape
    rng = np.random.default_rng(sum(shape) + layout)
    a, b = operands(layout, rows, cols, inner,
                    lambda s: rng.uniform(-1, 1, s).astype(np.float32))
    c = run_gemm(hip, layout, a, b, rows, cols, inner)
    c64, ab = orc.gemm_f64(LNAME[layout], a, b, rows, cols, inner)
    err = rel_err(c, c64, ab)
    assert err <= gemm_tol(inner), (err, gemm_tol(inner))


@pytest.mark.parametrize("layout", [NN, NT, TN])
@pytest.mark.parametrize("shape", [(4096, 4096, 32), (4096, 4096, 288), (4096, 8192, 96),
                                   (4096, 4096, 100)], ids=lambda s: "x".join(map(str, s)))
def test_gemm_large_whole_tiles_exact(hip, layout, shape):
    """Plain products over whole 256x256 tiles that fill the GPU (the
    256x256 tile, with a K tail at K = 100), all three layouts: exact on
    small integers, every element."""
    rows, cols, inner = shape
    rng = np.random.default_rng(rows + cols + inner + layout)
    a, b = operands(layout, rows, cols, inner, lambda s: int_matrix(rng, s, -4, 4))
    A, B = logical(layout, a, b)
    print(f"gemm whole tiles {LNAME[layout]} {shape}", flush=True)
    c = run_gemm(hip, layout, a, b, rows, cols, inner)
    ref = A.astype(np.float64) @ B.astype(np.float64)
    assert np.array_equal(c, ref.astype(np.float32)), f"{LNAME[layout]} {shape}"


def test_gemm_cfg1_512_vs_cpu_simd(hip, orc):
    """cfg1: 512^3, U(-1,1) seed 0; the GPU and the reference's AVX2 path both
    sit within the f32 tolerance of f64, and within 2x that of each other."""
    rng = np.random.default_rng(0)
    a = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    b = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    c = run_gemm(hip, NN, a, b, 512, 512, 512)
    cpu = orc.matmul_simd(a, b)
    c64, ab = orc.gemm_f64("nn", a, b, 512, 512, 512)
    assert rel_err(c, c64, ab) <= gemm_tol(512)
    assert rel_err(cpu, c64, ab) <= gemm_tol(512)
    assert rel_err(c, cpu.astype(np.float64), ab) <= 2 * gemm_tol(512)


@pytest.mark.parametrize("n", [2048, 4096, 8192])
def test_gemm_large_square_sampled_rows(hip, orc, n):
    """cfg5 squares: f64 check on a sample of rows (every 256-row tile row
    touched, and the last 40 rows)."""
    rng = np.random.default_rng(n)
    a = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    c = run_gemm(hip, NN, a, b, n, n, n)
    step = 61 if n <= 4096 else 127
    rows = np.unique(np.concatenate([np.arange(0, n, step), np.arange(n - 40, n)]))
    c64, ab = orc.gemm_f64("nn", a, b, n, n, n, rowidx=rows)
    assert rel_err(c[rows], c64, ab) <= gemm_tol(n)


def test_gemm_skinny_cfg5(hip, orc):
    """cfg5 skinny M=32, N=K=8192 (split-K path), f64 check on all rows."""
    rng = np.random.default_rng(32)
    m, n, k = 32, 8192, 8192
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    c = run_gemm(hip, NN, a, b, m, n, k)
    c64, ab = orc.gemm_f64("nn", a, b, m, n, k)
    assert rel_err(c, c64, ab) <= gemm_tol(k)


@pytest.mark.parametrize("shape", [(70, 50, 33), (2000, 2100, 1100), (300, 20, 40), (30, 600, 1024),
                                   (4096, 4096, 64), (1000, 260, 200)],
                         ids=["64x64", "128x128", "128x32", "32x256-splitk", "256x256", "64x64-ksplit"])
def test_gemm_beta_bias_relu_epilogues(hip, shape):
    """The general epilogue (beta, column bias, row bias + ReLU) on each tile."""
    rng = np.random.default_rng(9)
    rows, cols, inner = shape
    a, b = operands(NN, rows, cols, inner, lambda s: int_matrix(rng, s, -3, 3))
    A, B = logical(NN, a, b)
    prod = (A @ B).astype(np.float32)
    c0 = int_matrix(rng, (rows, cols))
    bc = int_matrix(rng, (cols,))
    br = int_matrix(rng, (rows,))
    # beta = 1 fuses accumulate_into: C = C_old + A.B
    assert np.array_equal(run_gemm(hip, NN, a, b, rows, cols, inner, 1.0, c0), c0 + prod)
    # Linear: A.B + bias[col]
    assert np.array_equal(run_gemm(hip, NN, a, b, rows, cols, inner, 0.0, None, bc, 1),
                          prod + bc[None, :])
    # conv-style row bias, then ReLU
    assert np.array_equal(run_gemm(hip, NN, a, b, rows, cols, inner, 0.0, None, br, 2 | 4),
                          np.maximum(prod + br[:, None], 0))


def test_gemm_empty_and_zero_inner(hip):
    # K = 0: C = beta*C (here 0), no operand reads.
    dC = hip.DeviceBuffer.from_host(np.full((3, 4), 7.0, np.float32))
    hip.gemm(NN, dC, None, None, 3, 4, 0, 0.0)
    assert np.array_equal(dC.to_host((3, 4)), np.zeros((3, 4), np.float32))
    hip.gemm(NN, dC, None, None, 0, 4, 5, 0.0)  # empty output: no-op


def test_gemm_errors_raise(hip):
    dC = hip.DeviceBuffer(4)
    with pytest.raises(hip.NrsError):
        hip.gemm(7, dC, dC, dC, 2, 2, 1)
    with pytest.raises(hip.NrsError):
        hip.gemm(NN, dC, dC, dC, -1, 2, 1)
    with pytest.raises(hip.NrsError):
        hip.gemm(NN, dC, dC, dC, 2, 2, 1, 0.0, None, 1)  # bias flag, null bias


# ------------------------------------------------------------- grouped GEMMs
def group_case(hip, rng, specs, make):
    """Device operands, outputs and expected results for nrs_gemm_group:
    specs are (layout, rows, cols, inner, beta, epilogue) tuples."""
    calls, want, outs = [], [], []
    for layout, rows, cols, inner, beta, epi in specs:
        a, b = operands(layout, rows, cols, inner, make)
        A, B = logical(layout, a, b)
        c0 = make((rows, cols))
        bias = make((cols,)) if epi & 1 else (make((rows,)) if epi & 2 else None)
        v = A @ B
        if epi & 1:
            v = v + bias[None, :]
        if epi & 2:
            v = v + bias[:, None]
        if epi & 4:
            v = np.maximum(v, 0)
        want.append((v + beta * c0).astype(np.float32))
        dC = hip.DeviceBuffer.from_host(c0)
        outs.append((dC, rows, cols))
        calls.append((layout, dC, hip.DeviceBuffer.from_host(a), hip.DeviceBuffer.from_host(b),
                      rows, cols, inner, beta,
                      hip.DeviceBuffer.from_host(bias) if bias is not None else None, epi))
    return calls, want, outs


GROUPS = {
    # a Linear's backward: dX (NT) and dW (TN, K split) of the cfg4 projection
    "proj_bwd": [(NT, 4096, 256, 256, 1.0, 0), (TN, 256, 256, 4096, 0.0, 0)],
    # the FFN backward pair, dW over K = 4096 into 64 tiles
    "ffn_bwd": [(NT, 4096, 1024, 256, 0.0, 0), (TN, 1024, 256, 4096, 1.0, 0)],
    # three projections of one input (Q, K, V) and a fourth with bias + ReLU
    "four_nn": [(NN, 512, 256, 256, 0.0, 0), (NN, 512, 256, 256, 0.0, 0),
                (NN, 512, 256, 256, 0.0, 0), (NN, 300, 68, 36, 0.0, 1 | 4)],
    # ragged edges, a row-bias epilogue, a short split
    "ragged": [(NN, 130, 68, 40, 1.0, 2), (TN, 60, 36, 3000, 0.0, 0), (NT, 100, 12, 8, 0.0, 0)],
}


@pytest.mark.parametrize("name", list(GROUPS))
def test_gemm_group_exact_integers(hip, name):
    """Every call of a group gives nrs_gemm's exact result (small integers:
    any tiling and summation order is exact)."""
    rng = np.random.default_rng(len(name))
    calls, want, outs = group_case(hip, rng, GROUPS[name], lambda s: int_matrix(rng, s, -3, 3))
    hip.gemm_group(calls)
    for (dC, rows, cols), w, spec in zip(outs, want, GROUPS[name]):
        assert np.array_equal(dC.to_host((rows, cols)), w), spec


def test_gemm_group_f64_tolerance(hip, orc):
    """The cfg4 projection backward pair on U(-1, 1) data against f64."""
    rng = np.random.default_rng(4)
    specs = [(NT, 4096, 256, 256), (TN, 256, 256, 4096)]
    calls, refs = [], []
    for layout, rows, cols, inner in specs:
        a, b = operands(layout, rows, cols, inner, lambda s: rng.uniform(-1, 1, s).astype(np.float32))
        dC = hip.DeviceBuffer(rows * cols)
        calls.append((layout, dC, hip.DeviceBuffer.from_host(a), hip.DeviceBuffer.from_host(b),
                      rows, cols, inner))
        refs.append((dC, rows, cols, inner) + orc.gemm_f64(LNAME[layout], a, b, rows, cols, inner))
    hip.gemm_group(calls)
    for dC, rows, cols, inner, c64, ab in refs:
        assert rel_err(dC.to_host((rows, cols)), c64, ab) <= gemm_tol(inner)


def test_gemm_group_overlap_runs_in_order(hip):
    """Two calls into one output (the second accumulating) cannot share a
    grid: they run one after the other, as two nrs_gemm calls would."""
    rng = np.random.default_rng(5)
    a1, b1 = int_matrix(rng, (64, 32)), int_matrix(rng, (32, 48))
    a2, b2 = int_matrix(rng, (64, 16)), int_matrix(rng, (16, 48))
    dC = hip.DeviceBuffer(64 * 48)
    d = [hip.DeviceBuffer.from_host(x) for x in (a1, b1, a2, b2)]
    hip.gemm_group([(NN, dC, d[0], d[1], 64, 48, 32, 0.0), (NN, dC, d[2], d[3], 64, 48, 16, 1.0)])
    assert np.array_equal(dC.to_host((64, 48)), a1 @ b1 + a2 @ b2)


def test_gemm_group_output_over_bias_runs_in_order(hip):
    """A call whose output is another call's bias: the second call reads the
    first one's result, as two nrs_gemm calls in that order would."""
    rng = np.random.default_rng(6)
    a1, b1 = int_matrix(rng, (1, 24)), int_matrix(rng, (24, 32))
    a2, b2 = int_matrix(rng, (40, 16)), int_matrix(rng, (16, 32))
    d = [hip.DeviceBuffer.from_host(x) for x in (a1, b1, a2, b2)]
    bias, out = hip.DeviceBuffer(32), hip.DeviceBuffer(40 * 32)
    hip.gemm_group([(NN, bias, d[0], d[1], 1, 32, 24, 0.0),
                    (NN, out, d[2], d[3], 40, 32, 16, 0.0, bias, 1)])
    assert np.array_equal(out.to_host((40, 32)), a2 @ b2 + (a1 @ b1)[0][None, :])


# ------------------------------------------------- Linear backward (fused)
@pytest.mark.parametrize("batch,in_f,out_f", [(4096, 256, 1024), (4096, 1024, 256), (4096, 256, 256),
                                              (256, 784, 128), (256, 128, 10), (37, 30, 9),
                                              (5, 4, 8), (300, 64, 7), (1, 1, 1)],
                         ids=lambda v: str(v))
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_linear_backward_exact_integers(hip, batch, in_f, out_f, beta):
    """dW, db (the extra row of the weight-gradient product) and dx of one
    nrs_linear_backward against the reference's three products (exact on
    small integers): split and unsplit weight gradients, 128-bit and scalar
    operands, grouped and one-after-another launches."""
    rng = np.random.default_rng(batch * 31 + in_f * 7 + out_f)
    g, x = int_matrix(rng, (batch, out_f), -3, 3), int_matrix(rng, (batch, in_f), -3, 3)
    w = int_matrix(rng, (in_f, out_f), -3, 3)
    dx0, dw0, db0 = (int_matrix(rng, s, -3, 3) for s in ((batch, in_f), (in_f, out_f), (out_f,)))
    D = hip.DeviceBuffer.from_host
    ddx, ddw, ddb = D(dx0), D(dw0), D(db0)
    hip.call("nrs_linear_backward", ddx, ddw, ddb, D(g), D(x), D(w), batch, in_f, out_f,
             beta, beta, beta)
    assert np.array_equal(ddw.to_host((in_f, out_f)), x.T @ g + beta * dw0)
    assert np.array_equal(ddb.to_host(), g.sum(axis=0) + beta * db0)
    assert np.array_equal(ddx.to_host((batch, in_f)), g @ w.T + beta * dx0)


def test_linear_backward_optional_outputs_and_empty(hip):
    """dx and db may be NULL; no input features (db still the column sums);
    no rows (dW = beta dW, db = beta db)."""
    rng = np.random.default_rng(11)
    D = hip.DeviceBuffer.from_host
    g, x, w = int_matrix(rng, (64, 32)), int_matrix(rng, (64, 48)), int_matrix(rng, (48, 32))
    ddw = hip.DeviceBuffer(48 * 32)
    hip.call("nrs_linear_backward", None, ddw, None, D(g), D(x), D(w), 64, 48, 32, 0.0, 0.0, 0.0)
    assert np.array_equal(ddw.to_host((48, 32)), x.T @ g)
    ddb = hip.DeviceBuffer(32)
    hip.call("nrs_linear_backward", None, ddw, ddb, D(g), D(x), D(w), 64, 48, 32, 0.0, 1.0, 0.0)
    assert np.array_equal(ddb.to_host(), g.sum(axis=0))
    assert np.array_equal(ddw.to_host((48, 32)), 2 * (x.T @ g))
    # no input features: only the bias gradient has elements
    dummy = hip.DeviceBuffer(4)
    ddb2 = D(np.ones(32, np.float32))
    hip.call("nrs_linear_backward", dummy, dummy, ddb2, D(g), dummy, dummy, 64, 0, 32, 0.0, 0.0, 1.0)
    assert np.array_equal(ddb2.to_host(), g.sum(axis=0) + 1)
    # no rows: the empty sums plus beta * old
    dw0, db0 = int_matrix(rng, (48, 32)), int_matrix(rng, (32,))
    ddw0, ddb0 = D(dw0), D(db0)
    hip.call("nrs_linear_backward", None, ddw0, ddb0, dummy, dummy, dummy, 0, 48, 32, 0.0, 1.0, 0.5)
    assert np.array_equal(ddw0.to_host((48, 32)), dw0)
    assert np.array_equal(ddb0.to_host(), 0.5 * db0)
    with pytest.raises(hip.NrsError):  # the weight gradient is required
        hip.call("nrs_linear_backward", None, None, ddb0, D(g), D(x), D(w), 64, 48, 32, 0.0, 0.0, 0.0)


# (rows, inner, cols, count): cfg4's Q, K and V projections (one grouped
# launch and the sums), input-gradient products split over K (few tiles, long
# K), products small enough for the short-GEMM kernel (the closures run in
# turn), two products, and one
SHARED_LHS_SHAPES = [(4096, 256, 256, 3), (128, 64, 4096, 3), (64, 32, 48, 3),
                     (1024, 128, 512, 2), (4096, 256, 256, 1)]


@pytest.mark.parametrize("rows,inner,cols,count", SHARED_LHS_SHAPES)
@pytest.mark.parametrize("beta_x", [0.0, 1.0])
def test_matmul_shared_lhs_backward_matches_closures(hip, rows, inner, cols, count, beta_x):
    """nrs_matmul_shared_lhs_backward gives the bits of the matmul closures
    run in turn (src/cuda/graph/matmul.rs:418-431), each an nrs_gemm_group of
    dx (+)= g_i . W_i^T and dW_i = x^T . g_i + beta_w[i] * dW_i, and the f64
    result within the GEMM bar (U(-1, 1) data)."""
    rng = np.random.default_rng(rows + inner + cols + count)
    U = lambda s: rng.uniform(-1, 1, s).astype(np.float32)
    x = U((rows, inner))
    ws = [U((inner, cols)) for _ in range(count)]
    gs = [U((rows, cols)) for _ in range(count)]
    dx0, dw0 = U((rows, inner)), [U((inner, cols)) for _ in range(count)]
    beta_w = [1.0, 0.0, 1.0][:count]
    D = hip.DeviceBuffer.from_host
    xd, wd, gd = D(x), [D(w) for w in ws], [D(g) for g in gs]
    dx_a, dw_a = D(dx0), [D(w) for w in dw0]
    dx_b, dw_b = D(dx0), [D(w) for w in dw0]
    hip.matmul_shared_lhs_backward(dx_a, dw_a, gd, xd, wd, rows, inner, cols, beta_x, beta_w)
    for i in range(count):
        hip.gemm_group([(NT, dx_b, gd[i], wd[i], rows, inner, cols, beta_x if i == 0 else 1.0),
                        (TN, dw_b[i], xd, gd[i], inner, cols, rows, beta_w[i])])
    bits = lambda buf, shape: buf.to_host(shape).view(np.uint32)
    assert np.array_equal(bits(dx_a, (rows, inner)), bits(dx_b, (rows, inner)))
    for a, b in zip(dw_a, dw_b):
        assert np.array_equal(bits(a, (inner, cols)), bits(b, (inner, cols)))
    f = lambda a: a.astype(np.float64)
    want_x = beta_x * f(dx0) + sum(f(g) @ f(w).T for g, w in zip(gs, ws))
    ab_x = abs(beta_x) * np.abs(f(dx0)) + sum(np.abs(f(g)) @ np.abs(f(w)).T for g, w in zip(gs, ws))
    assert rel_err(dx_a.to_host((rows, inner)), want_x, ab_x) <= gemm_tol(count * cols + 1)
    for i in range(count):
        want = f(x).T @ f(gs[i]) + beta_w[i] * f(dw0[i])
        ab = np.abs(f(x)).T @ np.abs(f(gs[i])) + abs(beta_w[i]) * np.abs(f(dw0[i]))
        assert rel_err(dw_a[i].to_host((inner, cols)), want, ab) <= gemm_tol(rows + 1)


def test_matmul_shared_lhs_backward_shared_weight_runs_closures(hip):
    """One weight used by two products (W_0 = W_1, so dW_0 = dW_1): the
    weight-gradient outputs overlap, so the closures run in turn, the second
    adding to the first one's dW."""
    rng = np.random.default_rng(9)
    rows, inner, cols = 1024, 128, 128
    x, dx0 = int_matrix(rng, (rows, inner), -3, 3), int_matrix(rng, (rows, inner), -3, 3)
    w = int_matrix(rng, (inner, cols), -3, 3)
    g0, g1 = int_matrix(rng, (rows, cols), -3, 3), int_matrix(rng, (rows, cols), -3, 3)
    D = hip.DeviceBuffer.from_host
    dx, dw, wd = D(dx0), hip.DeviceBuffer.zeros(inner * cols), D(w)
    hip.matmul_shared_lhs_backward(dx, [dw, dw], [D(g0), D(g1)], D(x), [wd, wd], rows, inner,
                                   cols, 1.0, [0.0, 1.0])
    assert np.array_equal(dw.to_host((inner, cols)), x.T @ g0 + x.T @ g1)
    assert np.array_equal(dx.to_host((rows, inner)), dx0 + g0 @ w.T + g1 @ w.T)


def test_gemm_group_errors(hip):
    dC = hip.DeviceBuffer(4)
    with pytest.raises(hip.NrsError):  # more calls than a group holds
        hip.gemm_group([(NN, dC, dC, dC, 2, 2, 1)] * (hip.GEMM_GROUP_MAX + 1))
    with pytest.raises(hip.NrsError):  # an invalid call launches nothing
        hip.gemm_group([(NN, dC, dC, dC, 2, 2, 1), (7, dC, dC, dC, 2, 2, 1)])
    hip.gemm_group([])  # nothing to do


def test_matmul_shared_lhs_backward_errors(hip):
    import ctypes
    d = hip.DeviceBuffer(64)
    arr = (ctypes.c_void_p * 3)(d.ptr, d.ptr, d.ptr)
    betas = (ctypes.c_float * 3)()
    with pytest.raises(hip.NrsError):  # more than three products
        hip.call("nrs_matmul_shared_lhs_backward", d, arr, arr, d, arr, 4, 8, 8, 8, 0.0, betas)
    with pytest.raises(hip.NrsError):  # a null weight gradient: nothing launches
        hip.matmul_shared_lhs_backward(d, [None, d], [d, d], d, [d, d], 8, 8, 8)
    hip.matmul_shared_lhs_backward(d, [d], [d], d, [d], 0, 8, 8)  # no rows: nothing to do


# ------------------------------------------------------------------ split-K
@pytest.mark.parametrize("shape", [(32, 9, 100352), (64, 288, 25088), (5, 7, 3000), (3, 2, 1)],
                         ids=lambda s: "x".join(map(str, s)))
def test_splitk_nt(hip, orc, shape):
    rows, cols, inner = shape
    rng = np.random.default_rng(rows + cols + inner)
    a = rng.standard_normal((rows, inner)).astype(np.float32)
    b = rng.uniform(-1, 1, (cols, inner)).astype(np.float32)
    c0 = rng.standard_normal((rows, cols)).astype(np.float32)
    dA, dB = hip.DeviceBuffer.from_host(a), hip.DeviceBuffer.from_host(b)
    dC = hip.DeviceBuffer.from_host(c0)
    hip.gemm_nt_splitk(dC, dA, dB, rows, cols, inner, 1.0)
    c = dC.to_host((rows, cols))
    c64, ab = orc.gemm_f64("nt", a, b, rows, cols, inner)
    assert rel_err(c - c0, c64, ab + np.abs(c0)) <= gemm_tol(inner)
    # deterministic: the same call gives the same bits
    dC2 = hip.DeviceBuffer.from_host(c0)
    hip.gemm_nt_splitk(dC2, dA, dB, rows, cols, inner, 1.0)
    assert np.array_equal(dC2.to_host((rows, cols)), c)


@pytest.mark.parametrize("shape", [(64, 576, 8192), (64, 320, 20000), (30, 100, 30000),
                                   (128, 256, 12000), (64, 576, 1000)],
                         ids=lambda s: "x".join(map(str, s)))
def test_splitk_exact_slices_per_xcd(hip, shape):
    """Split grids whose tile count is not a multiple of 8 (9, 5, 1 tiles) are
    renumbered so each XCD owns whole K slices; one that is (8 tiles) keeps
    the per-slice tile order. Small integers make every sum exact, so a slice
    or tile computed twice or skipped would show as a bit difference."""
    rows, cols, inner = shape
    rng = np.random.default_rng(rows * cols + inner)
    a = int_matrix(rng, (rows, inner), -2, 2)
    b = int_matrix(rng, (cols, inner), -2, 2)
    c0 = int_matrix(rng, (rows, cols))
    dA, dB = hip.DeviceBuffer.from_host(a), hip.DeviceBuffer.from_host(b)
    dC = hip.DeviceBuffer.from_host(c0)
    hip.gemm_nt_splitk(dC, dA, dB, rows, cols, inner, 1.0)
    want = (c0.astype(np.float64) + a.astype(np.float64) @ b.astype(np.float64).T)
    assert np.array_equal(dC.to_host((rows, cols)), want.astype(np.float32))


def test_splitk_cfg5_wgrad_shape(hip, orc):
    """cfg5 split-K wgrad M=64, N=576, K=100352 (NT), f64 on sampled rows."""
    rng = np.random.default_rng(576)
    rows, cols, inner = 64, 576, 100352
    a = rng.uniform(-1, 1, (rows, inner)).astype(np.float32)
    b = rng.uniform(-1, 1, (cols, inner)).astype(np.float32)
    dA, dB = hip.DeviceBuffer.from_host(a), hip.DeviceBuffer.from_host(b)
    dC = hip.DeviceBuffer(rows * cols)
    hip.gemm_nt_splitk(dC, dA, dB, rows, cols, inner, 0.0)
    c = dC.to_host((rows, cols))
    sel = np.arange(0, rows, 9)
    c64, ab = orc.gemm_f64("nt", a, b, rows, cols, inner, rowidx=sel)
    assert rel_err(c[sel], c64, ab) <= gemm_tol(inner)


# ---------------------------------------------------------------------- bmm
def test_bmm_twin(hip, orc):
    """tests/cuda_manip_test.rs:76-104 (batch 2, 3x4 . 4x5), tol 1e-4."""
    t = kats()["gpu_twin"]["bmm"]
    bt, m, k, n = t["batch"], t["m"], t["k"], t["n"]
    a = formula(t["a"], bt * m * k).reshape(bt, m, k)
    b = formula(t["b"], bt * k * n).reshape(bt, k, n)
    seed = formula(t["seed"], bt * m * n).reshape(bt, m, n)
    cf = orc.graph_bmm_forward(a, b)
    cga, cgb = orc.graph_bmm_backward(a, b, seed)
    dA, dB, dG = (hip.DeviceBuffer.from_host(x) for x in (a, b, seed))
    dO = hip.DeviceBuffer(bt * m * n)
    hip.bmm(NN, dO, dA, dB, bt, m, n, k)
    gA, gB = hip.DeviceBuffer.zeros(a.size), hip.DeviceBuffer.zeros(b.size)
    hip.bmm(NT, gA, dG, dB, bt, m, k, n, 1.0)   # grad_a: G . B^T, accumulated
    hip.bmm(TN, gB, dA, dG, bt, k, n, m, 1.0)   # grad_b: A^T . G, accumulated
    close(dO.to_host(), cf, t["tol"], "bmm fwd")
    close(gA.to_host(), cga, t["tol"], "bmm grad_a")
    close(gB.to_host(), cgb, t["tol"], "bmm grad_b")


@pytest.mark.parametrize("shape", [(3, 5, 7, 4), (256, 128, 128, 32), (256, 128, 32, 128),
                                   (8, 33, 17, 65),
                                   # LDS-staged items: K split over waves with empty parts,
                                   # 9 blocks (a wave takes two), 16 blocks with K = 128
                                   (4, 36, 20, 12), (2, 96, 96, 40), (4, 128, 128, 128)],
                         ids=lambda s: "x".join(map(str, s)))
def test_bmm_exact_integers(hip, shape):
    """cfg4 per-head shapes folded into one batch (256 = 32 x 8 heads)."""
    bt, m, n, k = shape
    rng = np.random.default_rng(sum(shape))
    a = int_matrix(rng, (bt, m, k), -3, 3)
    b = int_matrix(rng, (bt, k, n), -3, 3)
    g = int_matrix(rng, (bt, m, n), -3, 3)
    ai, bi, gi = (x.astype(np.int64) for x in (a, b, g))
    dA, dB, dG = (hip.DeviceBuffer.from_host(x) for x in (a, b, g))
    dO = hip.DeviceBuffer(bt * m * n)
    hip.bmm(NN, dO, dA, dB, bt, m, n, k)
    assert np.array_equal(dO.to_host((bt, m, n)), np.matmul(ai, bi).astype(np.float32))
    gA = hip.DeviceBuffer(bt * m * k)
    hip.bmm(NT, gA, dG, dB, bt, m, k, n)
    assert np.array_equal(gA.to_host((bt, m, k)),
                          np.matmul(gi, bi.transpose(0, 2, 1)).astype(np.float32))
    gB = hip.DeviceBuffer(bt * k * n)
    hip.bmm(TN, gB, dA, dG, bt, k, n, m)
    assert np.array_equal(gB.to_host((bt, k, n)),
                          np.matmul(ai.transpose(0, 2, 1), gi).astype(np.float32))


@pytest.mark.parametrize("shape", [(256, 128, 128, 32), (256, 128, 32, 128), (3, 36, 20, 12),
                                   (2, 5, 7, 9), (4, 128, 128, 128), (2, 64, 96, 40)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("beta", [0.0, 0.5])
@pytest.mark.parametrize("layout", [NN, NT], ids=lambda l: LNAME[l])
def test_bmm_backward_both_gradients(hip, layout, shape, beta):
    """nrs_bmm_backward (bmm.rs:93-131): for C = A . op(B) per item, dA =
    G . op(B)^T + beta*dA and dB = (A^T . G or G^T . A) + beta*dB, both in
    one launch for small items (the unaligned 5x7x9 items take the
    two-product path); exact in f32 for these small integers, also one
    gradient at a time."""
    bt, m, k, n = shape
    rng = np.random.default_rng(sum(shape) + int(4 * beta) + 11 * layout)
    a = int_matrix(rng, (bt, m, k), -3, 3)
    b = int_matrix(rng, (bt, k, n) if layout == NN else (bt, n, k), -3, 3)
    g = int_matrix(rng, (bt, m, n), -3, 3)
    da0 = int_matrix(rng, (bt, m, k), -8, 8)
    db0 = int_matrix(rng, b.shape, -8, 8)
    ai, bi, gi = (x.astype(np.int64) for x in (a, b, g))
    if layout == NN:
        want_a = np.matmul(gi, bi.transpose(0, 2, 1))
        want_b = np.matmul(ai.transpose(0, 2, 1), gi)
    else:
        want_a = np.matmul(gi, bi)
        want_b = np.matmul(gi.transpose(0, 2, 1), ai)
    want_a = (want_a + beta * da0).astype(np.float32)
    want_b = (want_b + beta * db0).astype(np.float32)
    dA, dB, dG = (hip.DeviceBuffer.from_host(x) for x in (a, b, g))
    gA, gB = hip.DeviceBuffer.from_host(da0), hip.DeviceBuffer.from_host(db0)
    hip.bmm_backward(layout, gA, gB, dG, dA, dB, bt, m, k, n, beta)
    assert np.array_equal(gA.to_host(da0.shape), want_a)
    assert np.array_equal(gB.to_host(db0.shape), want_b)
    gA1, gB1 = hip.DeviceBuffer.from_host(da0), hip.DeviceBuffer.from_host(db0)
    hip.bmm_backward(layout, gA1, None, dG, dA, dB, bt, m, k, n, beta)
    hip.bmm_backward(layout, None, gB1, dG, dA, dB, bt, m, k, n, beta)
    assert np.array_equal(gA1.to_host(da0.shape), want_a)
    assert np.array_equal(gB1.to_host(db0.shape), want_b)

@pytest.mark.parametrize("shape", [(5, 40, 36, 24), (3, 20, 13, 8), (2, 128, 128, 100),
                                   (7, 1, 4, 4), (3, 128, 64, 128), (6, 32, 32, 32),
                                   (2, 68, 100, 36)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("layout", [NN, NT, TN], ids=lambda l: LNAME[l])
def test_bmm_small_items_accumulate(hip, layout, shape):
    """Items of at most 128x128x128 (the register-direct path when the item
    rows are whole float4s, the tiled path otherwise), accumulated into a
    non-zero C with beta 0.5: exact in f32 for these small integers."""
    bt, m, n, k = shape
    rng = np.random.default_rng(sum(shape) + 7 * layout)
    a = int_matrix(rng, (bt, m, k) if layout != TN else (bt, k, m), -3, 3)
    b = int_matrix(rng, (bt, k, n) if layout != NT else (bt, n, k), -3, 3)
    c0 = int_matrix(rng, (bt, m, n), -8, 8)
    A = a.astype(np.int64) if layout != TN else a.astype(np.int64).transpose(0, 2, 1)
    B = b.astype(np.int64) if layout != NT else b.astype(np.int64).transpose(0, 2, 1)
    want = (np.matmul(A, B) + 0.5 * c0).astype(np.float32)
    dA, dB, dC = (hip.DeviceBuffer.from_host(x) for x in (a, b, c0))
    hip.bmm(layout, dC, dA, dB, bt, m, n, k, 0.5)
    assert np.array_equal(dC.to_host((bt, m, n)), want)


# ------------------------------------------- short GEMMs and fused Linear heads
SHORT_SHAPES = [  # outputs of few 64x64 tiles: one launch, K split over waves
    (16, 16, 4), (15, 17, 3), (1, 1, 2000), (33, 47, 1500), (100, 7, 2048), (2, 300, 1029),
    (256, 128, 784), (256, 10, 128), (128, 10, 256), (256, 128, 10), (784, 128, 256),
    (256, 784, 128), (129, 65, 513),
]


@pytest.mark.parametrize("layout", [NN, NT, TN])
@pytest.mark.parametrize("shape", SHORT_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("offset", [0, 1], ids=["aligned", "offset"])
def test_short_gemm_exact_integers(hip, layout, shape, offset):
    """Short GEMMs (K split over the waves of one workgroup, one or several
    rounds): bit-exact on small integers, with 16-byte aligned operands
    (128-bit loads where k is contiguous) and with every operand one float
    past alignment (32-bit loads); beta = 1 accumulates."""
    rows, cols, inner = shape
    rng = np.random.default_rng(rows * 131 + cols * 17 + inner + layout)
    a, b = operands(layout, rows, cols, inner, lambda s: int_matrix(rng, s, -3, 3))
    A, B = logical(layout, a, b)
    c0 = int_matrix(rng, (rows, cols), -3, 3)

    def placed(x):
        buf = hip.DeviceBuffer.from_host(np.concatenate([np.zeros(offset, np.float32), x.ravel()]))
        return buf, buf.ptr + 4 * offset

    (bA, pA), (bB, pB), (bC, pC) = placed(a), placed(b), placed(c0)
    hip.gemm(layout, pC, pA, pB, rows, cols, inner, 1.0)
    got = bC.to_host()[offset:].reshape(rows, cols)
    assert np.array_equal(got, (A @ B).astype(np.float32) + c0), f"{LNAME[layout]} {shape}"


@pytest.mark.parametrize("shape", [(100, 30, 50), (16, 16, 1), (70, 33, 1300)],
                         ids=lambda s: "x".join(map(str, s)))
def test_short_gemm_epilogues(hip, shape):
    """Column bias, row bias + ReLU and beta on the short-GEMM path."""
    rng = np.random.default_rng(19)
    rows, cols, inner = shape
    a, b = operands(NN, rows, cols, inner, lambda s: int_matrix(rng, s, -3, 3))
    A, B = logical(NN, a, b)
    prod = (A @ B).astype(np.float32)
    c0, bc, br = int_matrix(rng, (rows, cols)), int_matrix(rng, (cols,)), int_matrix(rng, (rows,))
    assert np.array_equal(run_gemm(hip, NN, a, b, rows, cols, inner, 1.0, c0), c0 + prod)
    assert np.array_equal(run_gemm(hip, NN, a, b, rows, cols, inner, 0.0, None, bc, 1 | 4),
                          np.maximum(prod + bc[None, :], 0))
    assert np.array_equal(run_gemm(hip, NN, a, b, rows, cols, inner, 0.0, None, br, 2),
                          prod + br[:, None])


@pytest.mark.parametrize("batch,in_f,out_f", [(256, 128, 10), (256, 784, 128), (37, 30, 9),
                                              (3, 5, 2), (4096, 256, 256), (300, 1000, 64),
                                              (4096, 1024, 256), (64, 64, 4096)],
                         ids=lambda v: str(v))
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_linear_backward_relu_exact_integers(hip, orc, batch, in_f, out_f, beta):
    """nrs_linear_backward_relu: dW, db as nrs_linear_backward, and
    dx = (g . W^T) * (mask > 0) + beta dx, the Linear's input gradient passed
    through the preceding ReLU's backward (the oracle's relu_backward,
    src/autograd/graph/relu.rs), exact on small integers; the masked product
    rides the short-GEMM epilogue or the tiled kernels' epilogue (grouped
    launches; 64 x 64 over K = 4096: a split input gradient whose reduce
    applies the mask)."""
    rng = np.random.default_rng(batch + 7 * in_f + out_f)
    g, x = int_matrix(rng, (batch, out_f), -3, 3), int_matrix(rng, (batch, in_f), -3, 3)
    w = int_matrix(rng, (in_f, out_f), -3, 3)
    mask = int_matrix(rng, (batch, in_f), -2, 2)  # ReLU input: negative, zero and positive
    dx0, dw0, db0 = (int_matrix(rng, s, -3, 3) for s in ((batch, in_f), (in_f, out_f), (out_f,)))
    D = hip.DeviceBuffer.from_host
    ddx, ddw, ddb = D(dx0), D(dw0), D(db0)
    hip.call("nrs_linear_backward_relu", ddx, ddw, ddb, D(g), D(x), D(w), D(mask), batch, in_f,
             out_f, beta, beta, beta)
    dh = (g @ w.T).astype(np.float32)
    want_dx = np.zeros_like(dh)
    orc.relu_backward(mask.ravel(), dh.ravel(), want_dx.reshape(-1))
    assert np.array_equal(ddx.to_host((batch, in_f)), want_dx + beta * dx0)
    assert np.array_equal(ddw.to_host((in_f, out_f)), x.T @ g + beta * dw0)
    assert np.array_equal(ddb.to_host(), g.sum(axis=0) + beta * db0)


def test_linear_backward_relu_matches_composition(hip):
    """Same bits as nrs_linear_backward followed by nrs_relu_backward (random
    f32 data, the cfg2 hidden layer)."""
    rng = np.random.default_rng(5)
    batch, in_f, out_f = 256, 128, 10
    g = (rng.standard_normal((batch, out_f)) * 0.1).astype(np.float32)
    h = np.maximum(rng.standard_normal((batch, in_f)), 0).astype(np.float32)
    w = rng.standard_normal((in_f, out_f)).astype(np.float32)
    D = hip.DeviceBuffer.from_host
    dg, dh, dw_ = D(g), D(h), D(w)
    fx, fw, fb = hip.DeviceBuffer(batch * in_f), hip.DeviceBuffer(in_f * out_f), hip.DeviceBuffer(out_f)
    hip.call("nrs_linear_backward_relu", fx, fw, fb, dg, dh, dw_, dh, batch, in_f, out_f, 0.0, 0.0, 0.0)
    cx, cw, cb = hip.DeviceBuffer(batch * in_f), hip.DeviceBuffer(in_f * out_f), hip.DeviceBuffer(out_f)
    hip.call("nrs_linear_backward", cx, cw, cb, dg, dh, dw_, batch, in_f, out_f, 0.0, 0.0, 0.0)
    hip.call("nrs_relu_backward", cx, cx, dh, batch * in_f, 0.0)
    for f, c in ((fx, cx), (fw, cw), (fb, cb)):
        assert np.array_equal(f.to_host(), c.to_host())


@pytest.mark.parametrize("batch,in_f,classes", [(256, 128, 10), (37, 20, 16), (5, 9, 3),
                                                (1000, 64, 10), (64, 32, 40), (3, 1, 1)],
                         ids=lambda v: str(v))
def test_linear_cross_entropy(hip, orc, batch, in_f, classes):
    """nrs_linear_cross_entropy: logits = x . W + b (exact on small integers)
    and the seed (softmax - t) / batch with the same bits as
    nrs_cross_entropy_backward on those logits, within the CE test's bound of
    the oracle's CrossEntropyLoss gradient; one launch up to 16 classes, the
    GEMM and the seed kernel beyond (40 classes)."""
    rng = np.random.default_rng(batch * 3 + classes)
    x, w = int_matrix(rng, (batch, in_f), -2, 2), int_matrix(rng, (in_f, classes), -2, 2)
    x, w = x * np.float32(0.25), w * np.float32(0.25)  # exact products, moderate logits
    bias = int_matrix(rng, (classes,), -2, 2)
    t = np.zeros((batch, classes), np.float32)
    t[np.arange(batch), rng.integers(0, classes, batch)] = 1.0
    D = hip.DeviceBuffer.from_host
    dx, dw, db, dt = D(x), D(w), D(bias), D(t)
    logits, grad = hip.DeviceBuffer(batch * classes), hip.DeviceBuffer(batch * classes)
    hip.call("nrs_linear_cross_entropy", logits, grad, dx, dw, db, dt, batch, in_f, classes)
    lg = logits.to_host((batch, classes))
    assert np.array_equal(lg, (x @ w).astype(np.float32) + bias[None, :])
    seed = hip.DeviceBuffer(batch * classes)
    hip.call("nrs_cross_entropy_backward", seed, logits, dt, batch, classes)
    assert np.array_equal(grad.to_host(), seed.to_host())
    gw = orc.cross_entropy_grad(lg, t, classes)
    assert np.abs(grad.to_host() - gw).max() <= 2e-7 + 1e-6 / batch


def test_linear_cross_entropy_errors(hip):
    buf = hip.DeviceBuffer(64)
    with pytest.raises(hip.NrsError):  # the seed would overwrite the logits
        hip.call("nrs_linear_cross_entropy", buf, buf, buf, buf, None, buf, 4, 2, 3)
    # Each output against each input, one hazard per call, on the fused
    # (3 classes) and the two-launch (40 classes) paths.
    for classes in (3, 40):
        names = ("logits", "grad", "x", "w", "bias", "target")
        sizes = (4 * classes, 4 * classes, 4 * 2, 2 * classes, classes, 4 * classes)
        for out_i in (0, 1):
            for in_i in (2, 3, 4, 5):
                bufs = [hip.DeviceBuffer(n) for n in sizes]
                bufs[in_i] = bufs[out_i]
                with pytest.raises(hip.NrsError, match="must not overlap"):
                    hip.call("nrs_linear_cross_entropy", *bufs, 4, 2, classes)
                print("refused", names[out_i], "over", names[in_i], classes)
    with pytest.raises(hip.NrsError):
        hip.call("nrs_linear_backward_relu", buf, buf, None, buf, buf, buf, None, 4, 2, 3,
                 0.0, 0.0, 0.0)


MLP2_SHAPES = [(256, 784, 128, 10),   # cfg2
                (7, 50, 100, 3),       # ragged row block, hidden not a multiple of 64
                (33, 17, 256, 16),     # four hidden column groups, the most classes
                (5, 1, 64, 1),         # one input feature, one class
                (64, 300, 192, 10),    # three column groups, in_f not a multiple of 8
                # past the one-launch kernel's limits: three launches
                (8, 4100, 64, 3),      # in_f > 4096
                (9, 30, 260, 5),       # hidden > 256
                (7, 20, 32, 20)]       # classes > 16


@pytest.mark.parametrize("shape", MLP2_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_mlp2_forward_seed(hip, orc, shape):
    """nrs_mlp2_forward_seed: h = relu(x . w1 + b1) and z = h . w2 + b2
    exact on quarter-integer data (against numpy); gz with the bits of
    nrs_cross_entropy_backward on those logits and within the CE test's bound
    of the oracle's CrossEntropyLoss gradient; dh = gz . w2^T where h > 0
    against float64 within the short-GEMM bound (K = classes)."""
    batch, in_f, hidden, classes = shape
    rng = np.random.default_rng(batch + in_f + hidden + classes)
    q = np.float32(0.25)
    x = int_matrix(rng, (batch, in_f), -2, 2) * q
    w1 = int_matrix(rng, (in_f, hidden), -2, 2) * q
    b1 = int_matrix(rng, (hidden,), -2, 2)
    w2 = int_matrix(rng, (hidden, classes), -2, 2) * q
    b2 = int_matrix(rng, (classes,), -2, 2)
    t = np.zeros((batch, classes), np.float32)
    t[np.arange(batch), rng.integers(0, classes, batch)] = 1.0
    D = hip.DeviceBuffer.from_host
    h, dh = hip.DeviceBuffer(batch * hidden), hip.DeviceBuffer(batch * hidden)
    z, gz = hip.DeviceBuffer(batch * classes), hip.DeviceBuffer(batch * classes)
    print(f"mlp2 forward {shape}", flush=True)
    hip.call("nrs_mlp2_forward_seed", h, z, gz, dh, D(x), D(w1), D(b1), D(w2), D(b2), D(t),
             batch, in_f, hidden, classes)
    h_ref = np.maximum((x.astype(np.float64) @ w1 + b1), 0).astype(np.float32)
    hh = h.to_host((batch, hidden))
    assert np.array_equal(hh, h_ref)
    zz = z.to_host((batch, classes))
    assert np.array_equal(zz, (h_ref.astype(np.float64) @ w2 + b2).astype(np.float32))
    seed = hip.DeviceBuffer(batch * classes)
    hip.call("nrs_cross_entropy_backward", seed, z, D(t), batch, classes)
    g = gz.to_host((batch, classes))
    assert np.array_equal(g.ravel(), seed.to_host())
    assert np.abs(g - orc.cross_entropy_grad(zz, t, classes).reshape(batch, classes)).max() <= \
        2e-7 + 1e-6 / batch
    g64 = g.astype(np.float64)
    dh_ref = np.where(hh > 0, g64 @ w2.T.astype(np.float64), 0.0)
    bound = gemm_tol(classes) * (np.abs(g64) @ np.abs(w2.T.astype(np.float64)) + 1e-30)
    assert np.all(np.abs(dh.to_host((batch, hidden)) - dh_ref) <= bound)
    assert np.all(dh.to_host((batch, hidden))[hh <= 0] == 0.0)


@pytest.mark.parametrize("shape", MLP2_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("betas", [(0.0, 0.0), (1.0, 0.5)], ids=["write", "accumulate"])
@pytest.mark.parametrize("with_dx", [True, False], ids=["dx", "no_dx"])
def test_mlp2_backward_exact(hip, shape, betas, with_dx):
    """nrs_mlp2_backward: dx = dh . w1^T, dw1 = x^T . dh, db1 = sum(dh),
    dw2 = h^T . gz, db2 = sum(gz), exact on small integers against numpy and
    bit for bit against nrs_linear_backward on each layer; beta_p 0 over NaN
    shows the old parameter gradients are not read."""
    batch, in_f, hidden, classes = shape
    beta_x, beta_p = betas
    rng = np.random.default_rng(3 * batch + in_f + hidden + classes)
    x = int_matrix(rng, (batch, in_f), -2, 2)
    w1 = int_matrix(rng, (in_f, hidden), -2, 2)
    h = np.maximum(int_matrix(rng, (batch, hidden), -2, 2), 0)
    dh = int_matrix(rng, (batch, hidden), -2, 2)
    gz = int_matrix(rng, (batch, classes), -2, 2)
    old = [int_matrix(rng, (n,), -3, 3) if beta_p else np.full(n, np.nan, np.float32)
           for n in (in_f * hidden, hidden, hidden * classes, classes)]
    dx0 = int_matrix(rng, (batch * in_f,), -3, 3)
    D = hip.DeviceBuffer.from_host
    outs = [D(dx0)] + [D(o) for o in old]
    print(f"mlp2 backward {shape} betas={betas} dx={with_dx}", flush=True)
    hip.call("nrs_mlp2_backward", outs[0] if with_dx else None, *outs[1:], D(dh), D(gz), D(x),
             D(w1), D(h), batch, in_f, hidden, classes, beta_x, beta_p)
    f64 = np.float64
    keep = lambda o: beta_p * o if beta_p else 0
    want = [(dh.astype(f64) @ w1.T.astype(f64)).ravel() + beta_x * dx0,
            (x.T.astype(f64) @ dh).ravel() + keep(old[0]), dh.sum(0, dtype=f64) + keep(old[1]),
            (h.T.astype(f64) @ gz).ravel() + keep(old[2]), gz.sum(0, dtype=f64) + keep(old[3])]
    for i, (o, wv) in enumerate(zip(outs, want)):
        if i == 0 and not with_dx:
            assert np.array_equal(o.to_host(), dx0)
        else:
            assert np.array_equal(o.to_host(), wv.astype(np.float32)), i
    # nrs_linear_backward on each layer gives the same bits
    ref = [D(dx0)] + [D(o) for o in old]
    hip.call("nrs_linear_backward", ref[0] if with_dx else None, ref[1], ref[2], D(dh), D(x),
             D(w1), batch, in_f, hidden, beta_x, beta_p, beta_p)
    hip.call("nrs_linear_backward", None, ref[3], ref[4], D(gz), D(h), None, batch, hidden,
             classes, 0.0, beta_p, beta_p)
    for o, r in zip(outs, ref):
        assert np.array_equal(o.to_host(), r.to_host())


@pytest.mark.parametrize("shape", [(0, 12, 8, 3), (6, 0, 8, 3), (6, 12, 8, 3)],
                         ids=["no_rows", "no_inputs", "small"])
def test_mlp2_backward_degenerate(hip, shape):
    """nrs_mlp2_backward without rows (every sum empty: the parameter
    gradients become beta_p * old) or without input features (db1 still the
    column sums of dh, with no dW1 rows to carry them), against numpy."""
    batch, in_f, hidden, classes = shape
    rng = np.random.default_rng(batch + in_f)
    x = int_matrix(rng, (batch, in_f), -2, 2)
    w1 = int_matrix(rng, (in_f, hidden), -2, 2)
    h = np.maximum(int_matrix(rng, (batch, hidden), -2, 2), 0)
    dh = int_matrix(rng, (batch, hidden), -2, 2)
    gz = int_matrix(rng, (batch, classes), -2, 2)
    old = [int_matrix(rng, (n,), -3, 3) for n in (in_f * hidden, hidden, hidden * classes, classes)]
    D = hip.DeviceBuffer.from_host
    outs = [D(o) for o in old]
    print(f"mlp2 backward degenerate {shape}", flush=True)
    hip.call("nrs_mlp2_backward", None, *outs, D(dh), D(gz), D(x), D(w1), D(h), batch, in_f,
             hidden, classes, 0.0, 0.5)
    f64 = np.float64
    want = [(x.T.astype(f64) @ dh).ravel(), dh.sum(0, dtype=f64), (h.T.astype(f64) @ gz).ravel(),
            gz.sum(0, dtype=f64)]
    for o, wv, o0 in zip(outs, want, old):
        assert np.array_equal(o.to_host(), (wv + 0.5 * o0).astype(np.float32))


def test_mlp2_composed_step_vs_four_calls(hip):
    """The cfg2 step on normal data, two launches (nrs_mlp2_forward_seed,
    nrs_mlp2_backward) against the four-call form (nrs_gemm with bias and
    ReLU, nrs_linear_cross_entropy, nrs_linear_backward_relu,
    nrs_linear_backward): h, dx, dw1, db1 within the short-GEMM bound of K
    (the first products reduce in different orders), the rest likewise."""
    B, I, Hd, O = 256, 784, 128, 10
    rng = np.random.default_rng(11)
    x = rng.standard_normal((B, I)).astype(np.float32)
    w1 = (rng.standard_normal((I, Hd)) * np.sqrt(2.0 / I)).astype(np.float32)
    w2 = (rng.standard_normal((Hd, O)) * np.sqrt(2.0 / Hd)).astype(np.float32)
    b1 = (rng.standard_normal(Hd) * 0.1).astype(np.float32)
    b2 = (rng.standard_normal(O) * 0.1).astype(np.float32)
    t = np.zeros((B, O), np.float32)
    t[np.arange(B), rng.integers(0, O, B)] = 1.0
    D = hip.DeviceBuffer.from_host
    dx_, dw1_, db1_, dw2_, db2_, dt = D(x), D(w1), D(b1), D(w2), D(b2), D(t)
    # four calls
    a, z, gz, gh = (hip.DeviceBuffer(n) for n in (B * Hd, B * O, B * O, B * Hd))
    r_gx, r_gw1, r_gb1, r_gw2, r_gb2 = (hip.DeviceBuffer.zeros(n) for n in (B * I, I * Hd, Hd, Hd * O, O))
    hip.gemm(hip.NN, a, dx_, dw1_, B, Hd, I, 0.0, db1_, hip.EPI_BIAS_COL | hip.EPI_RELU)
    hip.call("nrs_linear_cross_entropy", z, gz, a, dw2_, db2_, dt, B, Hd, O)
    hip.call("nrs_linear_backward_relu", gh, r_gw2, r_gb2, gz, a, dw2_, a, B, Hd, O, 0.0, 0.0, 0.0)
    hip.call("nrs_linear_backward", r_gx, r_gw1, r_gb1, gh, dx_, dw1_, B, I, Hd, 0.0, 0.0, 0.0)
    # two launches
    h2, z2, gz2, dh2 = (hip.DeviceBuffer(n) for n in (B * Hd, B * O, B * O, B * Hd))
    gx, gw1, gb1, gw2, gb2 = (hip.DeviceBuffer(n) for n in (B * I, I * Hd, Hd, Hd * O, O))
    print("mlp2 composed step cfg2", flush=True)
    hip.call("nrs_mlp2_forward_seed", h2, z2, gz2, dh2, dx_, dw1_, db1_, dw2_, db2_, dt, B, I, Hd, O)
    hip.call("nrs_mlp2_backward", gx, gw1, gb1, gw2, gb2, dh2, gz2, dx_, dw1_, h2, B, I, Hd, O,
             0.0, 0.0)
    f64 = np.float64
    h_ref = np.maximum(x.astype(f64) @ w1 + b1, 0)
    habs = np.abs(x.astype(f64)) @ np.abs(w1) + np.abs(b1)
    for got in (h2.to_host((B, Hd)), a.to_host((B, Hd))):
        assert np.all(np.abs(got - h_ref) <= gemm_tol(I) * habs + 1e-30)
    # downstream of h the two forms see slightly different h; compare each
    # with the other within a bound scaled by the data
    pairs = [(z2, z, 1e-5), (gz2, gz, 1e-6), (dh2, gh, 1e-6), (gx, r_gx, 1e-5),
             (gw1, r_gw1, 1e-5), (gb1, r_gb1, 1e-5), (gw2, r_gw2, 1e-5), (gb2, r_gb2, 1e-5)]
    for mine, theirs, tol in pairs:
        m, r = mine.to_host(), theirs.to_host()
        assert np.abs(m - r).max() <= tol * (np.abs(r).max() + 1e-30), (tol, np.abs(m - r).max())


def test_mlp2_forward_after_nan_in_lds(hip):
    """A wave's last batch of w1 rows may run past its range (those rows read
    as zeros); their x operands must read the zero pad after the staged x
    rows, not stale LDS. Calls on NaN inputs with a slightly larger in_f leave
    NaN in LDS where a cfg2 call's overrun lands; the cfg2 call after them
    must still be exact (quarter-integer data)."""
    D = hip.DeviceBuffer.from_host
    rng = np.random.default_rng(5)
    for in_nan in (800, 820, 840):
        B, Hd, O = 256, 128, 10
        nan = D(np.full(B * in_nan, np.nan, np.float32))
        w = D(np.full(in_nan * Hd, np.nan, np.float32))
        outs = [hip.DeviceBuffer(n) for n in (B * Hd, B * O, B * O, B * Hd)]
        hip.call("nrs_mlp2_forward_seed", *outs, nan, w, None, D(np.zeros(Hd * O, np.float32)),
                 None, D(np.zeros(B * O, np.float32)), B, in_nan, Hd, O)
    batch, in_f, hidden, classes = 256, 784, 128, 10
    q = np.float32(0.25)
    x = int_matrix(rng, (batch, in_f), -2, 2) * q
    w1 = int_matrix(rng, (in_f, hidden), -2, 2) * q
    b1 = int_matrix(rng, (hidden,), -2, 2)
    w2 = int_matrix(rng, (hidden, classes), -2, 2) * q
    t = np.zeros((batch, classes), np.float32)
    t[np.arange(batch), 0] = 1.0
    h = hip.DeviceBuffer(batch * hidden)
    z, gz, dh = (hip.DeviceBuffer(n) for n in (batch * classes, batch * classes, batch * hidden))
    print("mlp2 forward after NaN-filled LDS", flush=True)
    hip.call("nrs_mlp2_forward_seed", h, z, gz, dh, D(x), D(w1), D(b1), D(w2), None, D(t), batch,
             in_f, hidden, classes)
    h_ref = np.maximum((x.astype(np.float64) @ w1 + b1), 0).astype(np.float32)
    assert np.array_equal(h.to_host((batch, hidden)), h_ref)
    assert np.isfinite(dh.to_host()).all() and np.isfinite(gz.to_host()).all()


def test_mlp2_step_vs_f64(hip, orc):
    """The two-launch cfg2 step at full size on normal data against a float64
    restatement of the step (Linear, ReLU, Linear, ce_backward's seed, both
    backward closures), each output within the f32 GEMM bound of its own
    reduction length times the float64 magnitude sum; the seed also within
    the CE test's bound of the oracle's gradient of the float64 logits."""
    B, I, Hd, O = 256, 784, 128, 10
    rng = np.random.default_rng(21)
    x = rng.standard_normal((B, I)).astype(np.float32)
    w1 = (rng.standard_normal((I, Hd)) * np.sqrt(2.0 / I)).astype(np.float32)
    w2 = (rng.standard_normal((Hd, O)) * np.sqrt(2.0 / Hd)).astype(np.float32)
    b1 = (rng.standard_normal(Hd) * 0.1).astype(np.float32)
    b2 = (rng.standard_normal(O) * 0.1).astype(np.float32)
    t = np.zeros((B, O), np.float32)
    t[np.arange(B), rng.integers(0, O, B)] = 1.0
    D = hip.DeviceBuffer.from_host
    h, z, gz, dh = (hip.DeviceBuffer(n) for n in (B * Hd, B * O, B * O, B * Hd))
    gx, gw1, gb1, gw2, gb2 = (hip.DeviceBuffer(n) for n in (B * I, I * Hd, Hd, Hd * O, O))
    print("mlp2 step vs f64 cfg2", flush=True)
    hip.call("nrs_mlp2_forward_seed", h, z, gz, dh, D(x), D(w1), D(b1), D(w2), D(b2), D(t),
             B, I, Hd, O)
    hip.call("nrs_mlp2_backward", gx, gw1, gb1, gw2, gb2, dh, gz, D(x), D(w1), h, B, I, Hd, O,
             0.0, 0.0)
    f = np.float64
    X, W1, W2 = x.astype(f), w1.astype(f), w2.astype(f)
    pre = X @ W1 + b1
    H64 = np.maximum(pre, 0)
    Z64 = H64 @ W2 + b2
    e = np.exp(Z64 - Z64.max(1, keepdims=True))
    G64 = (e / e.sum(1, keepdims=True) - t) / B
    DH64 = np.where(pre > 0, G64 @ W2.T, 0.0)

    def within(got, want, bound):
        assert np.all(np.abs(got - want) <= bound), np.max(np.abs(got - want) / (bound + 1e-300))

    hh = h.to_host((B, Hd))
    within(hh, H64, gemm_tol(I) * (np.abs(X) @ np.abs(W1) + np.abs(b1)))
    within(z.to_host((B, O)), Z64, gemm_tol(I) * (np.abs(H64) @ np.abs(W2) + np.abs(b2)) * 4)
    gzz = gz.to_host((B, O))
    within(gzz, G64, 2e-6 / B + 1e-6 * np.abs(G64))
    assert np.abs(gzz - orc.cross_entropy_grad(Z64.astype(np.float32), t, O).reshape(B, O)).max() \
        <= 2e-7 + 1e-6 / B
    # dh, and what the backward builds from the kernel's own gz and dh
    # (pre-activations within rounding of zero may switch the mask: those
    # elements are left out of dh's check)
    clear = np.abs(pre) > 1e-4 * (np.abs(X) @ np.abs(W1) + np.abs(b1))
    g64 = gzz.astype(f)
    dhh = dh.to_host((B, Hd))
    within(dhh[clear], np.where(hh > 0, g64 @ W2.T, 0.0)[clear],
           (gemm_tol(O) * (np.abs(g64) @ np.abs(W2.T)))[clear] + 1e-30)
    d64 = dhh.astype(f)
    within(gx.to_host((B, I)), d64 @ W1.T, gemm_tol(Hd) * (np.abs(d64) @ np.abs(W1.T)) + 1e-30)
    within(gw1.to_host((I, Hd)), X.T @ d64, gemm_tol(B) * (np.abs(X.T) @ np.abs(d64)) + 1e-30)
    within(gb1.to_host(), d64.sum(0), gemm_tol(B) * np.abs(d64).sum(0) + 1e-30)
    within(gw2.to_host((Hd, O)), hh.astype(f).T @ g64,
           gemm_tol(B) * (np.abs(hh.astype(f).T) @ np.abs(g64)) + 1e-30)
    within(gb2.to_host(), g64.sum(0), gemm_tol(B) * np.abs(g64).sum(0) + 1e-30)
    assert np.count_nonzero(~clear) < 0.01 * clear.size  # ~0.1% at this cut


def test_mlp2_errors(hip):
    buf = hip.DeviceBuffer(4096)
    bad = [(8, 0, 16, 3), (-1, 4, 16, 3), (8, 4, 0, 3), (8, 4, 16, 0)]
    for b, i, hd, o in bad:
        with pytest.raises(hip.NrsError):
            hip.call("nrs_mlp2_forward_seed", buf, buf, buf, buf, buf, buf, None, buf, None, buf,
                     b, i, hd, o)
    # each output over each input (and two outputs over each other)
    B, I, Hd, O = 8, 4, 16, 3
    sizes = (B * Hd, B * O, B * O, B * Hd, B * I, I * Hd, Hd, Hd * O, O, B * O)
    for out_i in range(4):
        for other in range(10):
            if other == out_i:
                continue
            bufs = [hip.DeviceBuffer(n) for n in sizes]
            bufs[other] = bufs[out_i]  # refused before any launch
            with pytest.raises(hip.NrsError, match="overlap"):
                hip.call("nrs_mlp2_forward_seed", *bufs, B, I, Hd, O)
    # no rows: nothing launched
    hip.call("nrs_mlp2_forward_seed", None, None, None, None, None, None, None, None, None, None,
             0, I, Hd, O)


@pytest.mark.parametrize("layout", [NN, TN])
@pytest.mark.parametrize("shape", [(32, 8192, 2048), (17, 1024, 300), (1, 4096, 1000),
                                   (30, 8200, 1024), (32, 1152, 8200)],
                         ids=lambda s: "x".join(map(str, s)))
def test_skinny_gemm_exact_integers(hip, layout, shape):
    """At most 32 rows over B [K][N] streamed into registers (one K slice per
    strip or split-K partials and the reduce): exact on small integers, with
    beta = 1 and with a column bias + ReLU epilogue; ragged N (8200 = 64
    strips + 8 columns), K not a multiple of the 8-k group (300, 1000, 8200)."""
    rows, cols, inner = shape
    if layout == NN and inner % 4:
        pytest.skip("NN takes 128-bit A rows: K % 4 == 0")
    rng = np.random.default_rng(rows * 3 + cols + inner + layout)
    a, b = operands(layout, rows, cols, inner, lambda s: int_matrix(rng, s, -2, 2))
    A, B = logical(layout, a, b)
    prod = (A @ B).astype(np.float32)
    c0 = int_matrix(rng, (rows, cols), -3, 3)
    assert np.array_equal(run_gemm(hip, layout, a, b, rows, cols, inner, 1.0, c0), c0 + prod)
    bc = int_matrix(rng, (cols,), -3, 3)
    assert np.array_equal(run_gemm(hip, layout, a, b, rows, cols, inner, 0.0, None, bc, 1 | 4),
                          np.maximum(prod + bc[None, :], 0))
