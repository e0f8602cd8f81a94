"""Parity of the attention/MLP glue kernels (nrs_transpose, nrs_scale,
nrs_softmax_*, nrs_relu_*) against the CPU oracle, through the C ABI, at the
reference twin sizes, edge shapes and the BASELINE cfg4 attention shape."""
import numpy as np
import pytest

from kat import int_matrix

pytestmark = pytest.mark.gpu


def dev(hip, x):
    return hip.DeviceBuffer.from_host(np.ascontiguousarray(x, np.float32))


@pytest.mark.parametrize("shape", [(1, 1, 1), (2, 3, 4), (3, 33, 65), (256, 128, 32), (1, 1000, 7)],
                         ids=lambda s: "x".join(map(str, s)))
def test_transpose_exact(hip, orc, shape):
    b, r, c = shape
    x = np.random.default_rng(r * c).standard_normal(b * r * c).astype(np.float32)
    out = hip.DeviceBuffer(x.size)
    hip.call("nrs_transpose", out.ptr, dev(hip, x), b, r, c)
    assert np.array_equal(out.to_host(), orc.transpose(x, b, r, c))


def test_scale_and_accumulate_exact(hip):
    rng = np.random.default_rng(1)
    x, acc = int_matrix(rng, (1001,)), int_matrix(rng, (1001,))
    out = dev(hip, acc)
    hip.call("nrs_scale", out.ptr, dev(hip, x), 0.25, x.size, 1.0)
    assert np.array_equal(out.to_host(), acc + x * np.float32(0.25))


@pytest.mark.parametrize("rows,width", [(4, 5), (1, 1), (7, 63), (5, 65), (9, 200), (3, 512),
                                        (2, 513), (3, 1000), (32768, 128)])
def test_softmax_fwd_bwd(hip, orc, rows, width):
    rng = np.random.default_rng(rows + width)
    x = (rng.standard_normal(rows * width) * 2).astype(np.float32)
    g = rng.standard_normal(rows * width).astype(np.float32)
    acc0 = rng.standard_normal(rows * width).astype(np.float32)
    y = hip.DeviceBuffer(x.size)
    hip.call("nrs_softmax_forward", y.ptr, dev(hip, x), rows, width)
    yc = orc.softmax_forward(x, width)
    gy = y.to_host()
    assert np.max(np.abs(gy - yc)) < 1e-6
    gin = dev(hip, acc0)
    hip.call("nrs_softmax_backward", gin.ptr, dev(hip, yc), dev(hip, g), rows, width, 1.0)
    ref = acc0.copy()
    orc.softmax_backward(yc, g, ref, width)
    assert np.max(np.abs(gin.to_host() - ref)) < 1e-5 * max(1.0, np.sqrt(width))


@pytest.mark.parametrize("rows,width", [(4, 5), (7, 63), (5, 65), (9, 200), (3, 512), (2, 513),
                                        (3, 1000), (32768, 128)])
def test_softmax_scaled_is_scale_then_softmax(hip, orc, rows, width):
    """The fused scaled softmax (forward and backward) gives the same bits as
    nrs_scale around nrs_softmax_*, as attention composes them, and matches
    the oracle's softmax of the scaled scores."""
    rng = np.random.default_rng(rows * width)
    sc = np.float32(1.0 / np.sqrt(32.0))
    x = (rng.standard_normal(rows * width) * 4).astype(np.float32)
    g = rng.standard_normal(rows * width).astype(np.float32)
    n = x.size
    # forward: scale then softmax, against the fused call
    t, y1, y2 = hip.DeviceBuffer(n), hip.DeviceBuffer(n), hip.DeviceBuffer(n)
    dx = dev(hip, x)
    hip.call("nrs_scale", t.ptr, dx.ptr, float(sc), n, 0.0)
    hip.call("nrs_softmax_forward", y1.ptr, t.ptr, rows, width)
    hip.call("nrs_softmax_forward_scaled", y2.ptr, dx.ptr, rows, width, float(sc))
    assert np.array_equal(y1.to_host(), y2.to_host())
    yc = orc.softmax_forward(x * sc, width)
    assert np.max(np.abs(y2.to_host() - yc)) < 1e-6
    # backward: softmax_backward then scale_grad, against the fused call
    dy, dg = dev(hip, yc), dev(hip, g)
    b1, b2 = hip.DeviceBuffer(n), hip.DeviceBuffer(n)
    hip.call("nrs_softmax_backward", t.ptr, dy.ptr, dg.ptr, rows, width, 0.0)
    hip.call("nrs_scale", b1.ptr, t.ptr, float(sc), n, 0.0)
    hip.call("nrs_softmax_backward_scaled", b2.ptr, dy.ptr, dg.ptr, rows, width, float(sc), 0.0)
    want = b1.to_host()
    assert np.array_equal(want, b2.to_host())
    ref = np.zeros(n, np.float32)
    orc.softmax_backward(yc, g, ref, width)
    assert np.max(np.abs(want - ref * sc)) < 1e-5 * max(1.0, np.sqrt(width))
    # accumulating form: gin += the same gradient
    acc0 = rng.standard_normal(n).astype(np.float32)
    b3 = dev(hip, acc0)
    hip.call("nrs_softmax_backward_scaled", b3.ptr, dy.ptr, dg.ptr, rows, width, float(sc), 1.0)
    assert np.max(np.abs(b3.to_host() - (acc0 + want))) < 1e-6 * max(1.0, np.abs(acc0).max())


def test_relu_fwd_bwd_exact(hip, orc):
    rng = np.random.default_rng(3)
    x, g, acc = (int_matrix(rng, (4099,)) for _ in range(3))
    y = hip.DeviceBuffer(x.size)
    hip.call("nrs_relu_forward", y.ptr, dev(hip, x), x.size)
    assert np.array_equal(y.to_host(), orc.relu_forward(x))
    gin = dev(hip, acc)
    hip.call("nrs_relu_backward", gin.ptr, dev(hip, g), dev(hip, x), x.size, 1.0)
    ref = acc.copy()
    orc.relu_backward(x, g, ref)
    assert np.array_equal(gin.to_host(), ref)


@pytest.mark.parametrize("batch,classes", [(256, 10), (16, 10), (7, 1), (33, 100), (1, 3)])
def test_cross_entropy_vs_oracle(hip, orc, batch, classes):
    """nrs_cross_entropy_forward / _backward (src/cuda/loss/cross_entropy.rs:
    18-58) against the oracle's CrossEntropyLoss (src/nn/loss.rs:49-106) on
    one-hot rows: the batch-mean loss (the row losses summed on the host) and
    the written seed (softmax - t) / batch, over an old gradient."""
    rng = np.random.default_rng(batch * 1000 + classes)
    x = (rng.standard_normal((batch, classes)) * 4).astype(np.float32)
    t = np.zeros((batch, classes), np.float32)
    t[np.arange(batch), rng.integers(0, classes, batch)] = 1.0
    dx, dt = hip.DeviceBuffer.from_host(x), hip.DeviceBuffer.from_host(t)
    rows = hip.DeviceBuffer(batch)
    hip.call("nrs_cross_entropy_forward", rows, dx, dt, batch, classes)
    loss = float(np.float32(rows.to_host().astype(np.float32).sum(dtype=np.float32)) / np.float32(batch))
    want = orc.cross_entropy_loss(x, t, classes)
    assert abs(loss - want) <= 1e-5 * max(1.0, abs(want)), (loss, want)
    g = hip.DeviceBuffer.from_host(rng.standard_normal(batch * classes).astype(np.float32))
    hip.call("nrs_cross_entropy_backward", g, dx, dt, batch, classes)
    gw = orc.cross_entropy_grad(x, t, classes)
    err = np.abs(g.to_host() - gw).max()
    assert err <= 2e-7 + 1e-6 / batch, err


def test_glue_argument_errors(hip):
    b = hip.DeviceBuffer(4)
    with pytest.raises(hip.NrsError):
        hip.call("nrs_transpose", b.ptr, b.ptr, 1, 2, 2)  # aliased
    with pytest.raises(hip.NrsError):
        hip.call("nrs_softmax_forward", b.ptr, b.ptr, 1, 0)


def test_slice_cols_twin(hip, orc):
    """tests/cuda_manip_test.rs:49-61: slice forward, and its backward
    accumulated into a zero input gradient, against the CPU op."""
    from kat import close, formula, kats
    t = kats()["gpu_twin"]["slice_cols"]
    rows, total, cs, ce = t["rows"], t["total"], t["cs"], t["ce"]
    x = formula(t["input"], rows * total)
    seed = formula(t["seed"], rows * (ce - cs))
    out = hip.DeviceBuffer(rows * (ce - cs))
    hip.call("nrs_slice_cols", out.ptr, dev(hip, x).ptr, rows, total, cs, ce - cs)
    close(out.to_host(), orc.slice_cols(x, rows, total, cs, ce), t["tol"], "slice_cols fwd")
    ga = hip.DeviceBuffer.zeros(rows * total)
    hip.call("nrs_slice_cols_backward", ga.ptr, dev(hip, seed).ptr, rows, total, cs, ce - cs, 1.0)
    ref = np.zeros(rows * total, np.float32)
    orc.slice_cols_backward(seed, ref, rows, total, cs, ce)
    close(ga.to_host(), ref, t["tol"], "slice_cols grad")


def test_concat_cols_twin(hip, orc):
    """tests/cuda_manip_test.rs:105-141: three parts side by side, and the
    gradient split back to each part."""
    from kat import close, formula, kats
    t = kats()["gpu_twin"]["concat_cols"]
    rows, w = t["rows"], t["w"]
    total = sum(w)
    parts = [formula(p, rows * pw) for p, pw in zip(t["parts"], w)]
    seed = formula(t["seed"], rows * total)
    out = hip.DeviceBuffer(rows * total)
    off = 0
    for p, pw in zip(parts, w):
        hip.call("nrs_concat_cols", out.ptr, dev(hip, p).ptr, rows, total, off, pw)
        off += pw
    close(out.to_host(), orc.concat_cols(parts, rows), t["tol"], "concat fwd")
    refs = [np.zeros(rows * pw, np.float32) for pw in w]
    orc.concat_cols_backward(seed, refs, rows)
    dseed, off = dev(hip, seed), 0
    for i, pw in enumerate(w):
        gp = hip.DeviceBuffer.zeros(rows * pw)
        hip.call("nrs_concat_cols_backward", gp.ptr, dseed.ptr, rows, total, off, pw, 1.0)
        close(gp.to_host(), refs[i], t["tol"], f"concat grad{i}")
        off += pw


@pytest.mark.parametrize("rows,total,cs,w", [(3, 10, 2, 5), (64, 256, 32, 32), (7, 1024, 4, 1000),
                                             (1, 1, 0, 1), (4096, 256, 224, 32)],
                         ids=lambda v: str(v))
def test_slice_concat_exact(hip, orc, rows, total, cs, w):
    """Copies are exact, and so are beta = 1 sums of small integers: 128-bit
    (width, offsets multiples of 4) and scalar forms."""
    rng = np.random.default_rng(rows * total + cs)
    x = int_matrix(rng, (rows * total,))
    out = hip.DeviceBuffer(rows * w)
    hip.call("nrs_slice_cols", out.ptr, dev(hip, x).ptr, rows, total, cs, w)
    assert np.array_equal(out.to_host(), orc.slice_cols(x, rows, total, cs, cs + w))
    g, acc = int_matrix(rng, (rows * w,)), int_matrix(rng, (rows * total,))
    ga = dev(hip, acc)
    hip.call("nrs_slice_cols_backward", ga.ptr, dev(hip, g).ptr, rows, total, cs, w, 1.0)
    ref = acc.copy()
    orc.slice_cols_backward(g, ref, rows, total, cs, cs + w)
    assert np.array_equal(ga.to_host(), ref)
    # concat of the slice into a wide buffer leaves the other columns alone
    wide = dev(hip, acc)
    hip.call("nrs_concat_cols", wide.ptr, dev(hip, g).ptr, rows, total, cs, w)
    ref = acc.reshape(rows, total).copy()
    ref[:, cs:cs + w] = g.reshape(rows, w)
    assert np.array_equal(wide.to_host(), ref.ravel())
    gp0 = int_matrix(rng, (rows * w,))
    gp = dev(hip, gp0)
    hip.call("nrs_concat_cols_backward", gp.ptr, dev(hip, x).ptr, rows, total, cs, w, 1.0)
    assert np.array_equal(gp.to_host(), gp0 + x.reshape(rows, total)[:, cs:cs + w].ravel())


@pytest.mark.parametrize("rows,heads,width", [(4096, 8, 32), (6, 3, 5), (128, 4, 64)])
def test_split_merge_heads(hip, orc, rows, heads, width):
    """split_heads equals the per-head slice_cols loop of MultiHeadAttention,
    merge_heads its concat_cols; each is the other's backward (beta = 1)."""
    rng = np.random.default_rng(rows + heads * width)
    x = int_matrix(rng, (rows * heads * width,))
    sp = hip.DeviceBuffer(x.size)
    hip.call("nrs_split_heads", sp.ptr, dev(hip, x).ptr, rows, heads, width, 0.0)
    want = np.concatenate([orc.slice_cols(x, rows, heads * width, h * width, (h + 1) * width)
                           for h in range(heads)])
    got = sp.to_host()
    assert np.array_equal(got, want)
    mg = hip.DeviceBuffer(x.size)
    hip.call("nrs_merge_heads", mg.ptr, sp.ptr, rows, heads, width, 0.0)
    assert np.array_equal(mg.to_host(), orc.concat_cols(np.split(want, heads), rows))
    assert np.array_equal(mg.to_host(), x)
    # accumulating forms
    acc = int_matrix(rng, (x.size,))
    a2 = dev(hip, acc)
    hip.call("nrs_merge_heads", a2.ptr, sp.ptr, rows, heads, width, 1.0)
    assert np.array_equal(a2.to_host(), acc + x)
    a3 = dev(hip, acc)
    hip.call("nrs_split_heads", a3.ptr, dev(hip, x).ptr, rows, heads, width, 1.0)
    assert np.array_equal(a3.to_host(), acc + want)


def test_slice_concat_errors(hip):
    b = hip.DeviceBuffer(16)
    with pytest.raises(hip.NrsError):
        hip.call("nrs_slice_cols", b.ptr, b.ptr, 2, 4, 0, 2)  # aliased
    c = hip.DeviceBuffer(16)
    with pytest.raises(hip.NrsError):
        hip.call("nrs_slice_cols", c.ptr, b.ptr, 2, 4, 3, 2)  # columns past the end
    with pytest.raises(hip.NrsError):
        hip.call("nrs_concat_cols_backward", c.ptr, b.ptr, 2, 4, -1, 2, 1.0)
    with pytest.raises(hip.NrsError):
        hip.call("nrs_split_heads", c.ptr, c.ptr, 2, 2, 4, 0.0)


def test_layernorm_twin(hip, orc):
    """tests/cuda_layers_test.rs:18-62: forward, input grad and gamma/beta
    grads against the CPU LayerNorm, tol 1e-4."""
    from kat import close, formula, kats
    t = kats()["gpu_twin"]["layernorm"]
    rows, F, eps = t["rows"], t["features"], t["eps"]
    x, g, b = formula(t["input"], rows * F), formula(t["gamma"], F), formula(t["beta"], F)
    seed = formula(t["seed"], rows * F)
    out, xn, istd = hip.DeviceBuffer(rows * F), hip.DeviceBuffer(rows * F), hip.DeviceBuffer(rows)
    dg_, db_ = dev(hip, g), dev(hip, b)
    hip.call("nrs_layernorm_forward", out.ptr, xn.ptr, istd.ptr, dev(hip, x).ptr, dg_.ptr,
             db_.ptr, rows, F, eps)
    cout, cxn, cistd = orc.layernorm_forward(x, g, b, rows, F, eps)
    close(out.to_host(), cout, t["tol"], "layernorm fwd")
    din, dgam, dbet = (hip.DeviceBuffer.zeros(n) for n in (rows * F, F, F))
    hip.call("nrs_layernorm_backward", din.ptr, dgam.ptr, dbet.ptr, dev(hip, seed).ptr, dg_.ptr,
             xn.ptr, istd.ptr, rows, F, 1.0)
    rin, rg, rb = np.zeros(rows * F, np.float32), np.zeros(F, np.float32), np.zeros(F, np.float32)
    orc.layernorm_backward(seed, g, cxn, cistd, rin, rg, rb, rows, F)
    close(din.to_host(), rin, t["tol"], "layernorm dinput")
    close(dgam.to_host(), rg, t["tol"], "layernorm dgamma")
    close(dbet.to_host(), rb, t["tol"], "layernorm dbeta")


@pytest.mark.parametrize("rows,F", [(4096, 256), (5, 64), (3, 65), (70, 512), (9, 600), (1, 1)])
def test_layernorm_vs_oracle(hip, orc, rows, F):
    """Register (F <= 512) and re-reading forms, the accumulating backward
    and skipped outputs, at cfg4's TransformerBlock width and edge widths."""
    rng = np.random.default_rng(rows * F)
    eps = 1e-5
    x = (rng.standard_normal(rows * F) * 3 + 1).astype(np.float32)
    g, b = rng.standard_normal(F).astype(np.float32), rng.standard_normal(F).astype(np.float32)
    gr = rng.standard_normal(rows * F).astype(np.float32)
    out, xn, istd = hip.DeviceBuffer(rows * F), hip.DeviceBuffer(rows * F), hip.DeviceBuffer(rows)
    dg_ = dev(hip, g)
    hip.call("nrs_layernorm_forward", out.ptr, xn.ptr, istd.ptr, dev(hip, x).ptr, dg_.ptr,
             dev(hip, b).ptr, rows, F, eps)
    cout, cxn, cistd = orc.layernorm_forward(x, g, b, rows, F, eps)
    scale = 1.0 + np.abs(g).max() + np.abs(b).max()
    assert np.max(np.abs(out.to_host() - cout)) < 2e-5 * scale
    assert np.max(np.abs(xn.to_host() - cxn)) < 2e-5
    assert np.max(np.abs(istd.to_host() - cistd) / cistd) < 1e-5
    acc_in = rng.standard_normal(rows * F).astype(np.float32)
    acc_g, acc_b = rng.standard_normal(F).astype(np.float32), rng.standard_normal(F).astype(np.float32)
    din, dgam, dbet = dev(hip, acc_in), dev(hip, acc_g), dev(hip, acc_b)
    hip.call("nrs_layernorm_backward", din.ptr, dgam.ptr, dbet.ptr, dev(hip, gr).ptr, dg_.ptr,
             xn.ptr, istd.ptr, rows, F, 1.0)
    rin, rg, rb = acc_in.copy(), acc_g.copy(), acc_b.copy()
    orc.layernorm_backward(gr, g, cxn, cistd, rin, rg, rb, rows, F)
    assert np.max(np.abs(din.to_host() - rin)) < 1e-4 * (1 + np.abs(rin).max())
    tol_p = 1e-5 * np.sqrt(rows) * (1 + np.abs(rg).max())
    assert np.max(np.abs(dgam.to_host() - rg)) < tol_p
    assert np.max(np.abs(dbet.to_host() - rb)) < 1e-5 * np.sqrt(rows) * (1 + np.abs(rb).max())
    # parameter gradients only, overwriting (acc 0); the input gradient is skipped
    d2 = hip.DeviceBuffer(F)
    hip.call("nrs_layernorm_backward", None, d2.ptr, None, dev(hip, gr).ptr, None, xn.ptr, None,
             rows, F, 0.0)
    assert np.max(np.abs(d2.to_host() - (rg - acc_g))) < tol_p


def test_layernorm_param_sums_past_two_million_rows(hip):
    """More rows than 65535 chunks of 32: the chunk height grows. Integer
    gradients make dbeta an exact sum, so a chunk skipped or counted twice
    shows; dgamma is checked against f64."""
    rng = np.random.default_rng(5)
    rows, F = 2_100_000, 2
    x = rng.standard_normal(rows * F).astype(np.float32)
    g = int_matrix(rng, (rows * F,), -3, 3)
    ones, zeros = np.ones(F, np.float32), np.zeros(F, np.float32)
    out, xn, istd = hip.DeviceBuffer(rows * F), hip.DeviceBuffer(rows * F), hip.DeviceBuffer(rows)
    hip.call("nrs_layernorm_forward", out.ptr, xn.ptr, istd.ptr, dev(hip, x).ptr, dev(hip, ones).ptr,
             dev(hip, zeros).ptr, rows, F, 1e-5)
    dg, db = hip.DeviceBuffer(F), hip.DeviceBuffer(F)
    hip.call("nrs_layernorm_backward", None, dg.ptr, db.ptr, dev(hip, g).ptr, None, xn.ptr, None,
             rows, F, 0.0)
    g2 = g.reshape(rows, F).astype(np.float64)
    assert np.array_equal(db.to_host(), g2.sum(axis=0).astype(np.float32))
    want = (g2 * xn.to_host().reshape(rows, F).astype(np.float64)).sum(axis=0)
    assert np.max(np.abs(dg.to_host() - want)) < 1e-6 * np.abs(g2).sum(axis=0).max()


def test_layernorm_backward_zero_rows(hip):
    """No rows: dgamma and dbeta are the empty sums plus acc * old, as the
    reference's ln_reduce gives; 0 when overwriting (acc 0), old values kept
    when accumulating (acc 1). The input gradient has nothing to write."""
    F = 70
    old_g = np.arange(F, dtype=np.float32) - 5
    old_b = np.full(F, np.nan, np.float32)  # never read when overwriting
    dg, db = dev(hip, old_g), dev(hip, old_b)
    hip.call("nrs_layernorm_backward", None, dg.ptr, db.ptr, None, None, None, None, 0, F, 0.0)
    assert np.array_equal(dg.to_host(), np.zeros(F, np.float32))
    assert np.array_equal(db.to_host(), np.zeros(F, np.float32))
    dg2, db2 = dev(hip, old_g), dev(hip, old_g * 2)
    hip.call("nrs_layernorm_backward", None, dg2.ptr, db2.ptr, None, None, None, None, 0, F, 1.0)
    assert np.array_equal(dg2.to_host(), old_g)
    assert np.array_equal(db2.to_host(), old_g * 2)


@pytest.mark.parametrize("rows,F", [(4096, 256), (3, 65), (70, 512), (9, 600)])
def test_add_layernorm_matches_add_then_layernorm(hip, rows, F):
    """The fused residual add + LayerNorm gives the bits of nrs_vadd followed
    by nrs_layernorm_forward (register and re-reading forms)."""
    rng = np.random.default_rng(rows + F)
    a, b = (rng.standard_normal(rows * F).astype(np.float32) for _ in range(2))
    g, be = rng.standard_normal(F).astype(np.float32), rng.standard_normal(F).astype(np.float32)
    da, db_, dg, dbe = dev(hip, a), dev(hip, b), dev(hip, g), dev(hip, be)
    s = hip.DeviceBuffer(rows * F)
    hip.call("nrs_vadd", s.ptr, da.ptr, db_.ptr, rows * F)
    outs = [[hip.DeviceBuffer(rows * F), hip.DeviceBuffer(rows * F), hip.DeviceBuffer(rows)]
            for _ in range(2)]
    o, xn, istd = outs[0]
    hip.call("nrs_layernorm_forward", o.ptr, xn.ptr, istd.ptr, s.ptr, dg.ptr, dbe.ptr, rows, F, 1e-5)
    o2, xn2, istd2 = outs[1]
    hip.call("nrs_add_layernorm_forward", o2.ptr, xn2.ptr, istd2.ptr, da.ptr, db_.ptr, dg.ptr,
             dbe.ptr, rows, F, 1e-5)
    for x, y in zip(outs[0], outs[1]):
        assert np.array_equal(x.to_host(), y.to_host())


@pytest.mark.parametrize("rows,F", [(4096, 256), (3, 65), (70, 512)])
@pytest.mark.parametrize("betas", [(0.0, 0.0, 0.0), (1.0, 0.0, 1.0), (0.0, 1.0, 0.0), (1.0, 1.0, 1.0)])
def test_add_layernorm_backward_two_outputs(hip, rows, F, betas):
    """nrs_add_layernorm_backward gives a's and b's gradients the bits of
    nrs_layernorm_backward's input gradient (each with its own beta) and the
    parameter gradients its bits, in one pass."""
    beta_a, beta_b, beta_p = betas
    rng = np.random.default_rng(rows * 7 + F)
    x = rng.standard_normal(rows * F).astype(np.float32)
    g, be = rng.standard_normal(F).astype(np.float32), rng.standard_normal(F).astype(np.float32)
    gr = rng.standard_normal(rows * F).astype(np.float32)
    old_a, old_b = (rng.standard_normal(rows * F).astype(np.float32) for _ in range(2))
    old_g, old_be = (rng.standard_normal(F).astype(np.float32) for _ in range(2))
    o, xn, istd = hip.DeviceBuffer(rows * F), hip.DeviceBuffer(rows * F), hip.DeviceBuffer(rows)
    dg_ = dev(hip, g)
    hip.call("nrs_layernorm_forward", o.ptr, xn.ptr, istd.ptr, dev(hip, x).ptr, dg_.ptr,
             dev(hip, be).ptr, rows, F, 1e-5)
    dgr = dev(hip, gr)
    # reference: the single-output backward, once per beta
    ra, rb = dev(hip, old_a), dev(hip, old_b)
    rg, rbe = dev(hip, old_g), dev(hip, old_be)
    hip.call("nrs_layernorm_backward", ra.ptr, None, None, dgr.ptr, dg_.ptr, xn.ptr, istd.ptr,
             rows, F, beta_a)
    hip.call("nrs_layernorm_backward", rb.ptr, None, None, dgr.ptr, dg_.ptr, xn.ptr, istd.ptr,
             rows, F, beta_b)
    hip.call("nrs_layernorm_backward", None, rg.ptr, rbe.ptr, dgr.ptr, dg_.ptr, xn.ptr, istd.ptr,
             rows, F, beta_p)
    da, db_ = dev(hip, old_a), dev(hip, old_b)
    dgam, dbet = dev(hip, old_g), dev(hip, old_be)
    print(f"add_layernorm_backward rows {rows} F {F} betas {betas}", flush=True)
    hip.call("nrs_add_layernorm_backward", da.ptr, db_.ptr, dgam.ptr, dbet.ptr, dgr.ptr, dg_.ptr,
             xn.ptr, istd.ptr, rows, F, beta_a, beta_b, beta_p)
    for got, want in ((da, ra), (db_, rb), (dgam, rg), (dbet, rbe)):
        assert np.array_equal(got.to_host(), want.to_host())


def test_add_layernorm_backward_second_output_needs_first(hip):
    buf = hip.DeviceBuffer(16)
    with pytest.raises(hip.NrsError):
        hip.call("nrs_add_layernorm_backward", None, buf.ptr, None, None, buf.ptr, buf.ptr,
                 buf.ptr, buf.ptr, 4, 4, 0.0, 0.0, 0.0)
