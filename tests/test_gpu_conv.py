"""Parity of the conv2d path (primitives and whole-op forward/backward) and
the gradient-plumbing kernels against the CPU oracle, through the C ABI.

Index work (im2col, col2out, out2mm, col2im, maxpool) must match bit for bit;
the reductions match exactly on small-integer data and to the reference
twin-test tolerances (tests/cuda_conv2d_test.rs) on its own inputs.
"""
import numpy as np
import pytest

from kat import close, formula, gemm_tol, int_matrix, kats, rel_err

pytestmark = pytest.mark.gpu

CONV_SHAPES = [  # (n, c_in, c_out, h, w, kh, kw, stride, pad)
    (2, 3, 4, 8, 8, 3, 3, 1, 1),
    (2, 3, 5, 7, 7, 3, 3, 1, 1),
    (1, 2, 3, 9, 6, 3, 2, 2, 1),
    (3, 1, 2, 5, 5, 2, 2, 1, 0),
    (2, 2, 2, 7, 9, 3, 3, 3, 2),
    (4, 16, 32, 12, 12, 3, 3, 1, 1),
    (1, 1, 1, 3, 3, 3, 3, 1, 0),
    (2, 2, 3, 6, 6, 2, 2, 1, 2),     # stride 1, pad > k-1: explicit input-gradient path
    (2, 4, 8, 10, 12, 3, 5, 1, 1),   # kh != kw: flipped-weight padding differs per axis
    # c_in > 4 and more than 32 taps: implicit-GEMM forward and input gradient
    (2, 6, 5, 9, 9, 3, 3, 1, 1),
    (2, 5, 4, 8, 6, 3, 2, 1, 0),
    (1, 8, 3, 7, 7, 3, 3, 2, 1),     # stride 2: explicit input-gradient path
    (2, 7, 9, 11, 13, 5, 5, 1, 2),   # 5x5, pad 2, ragged sizes
    # LDS-slab path edge cases
    (1, 40, 70, 6, 7, 3, 3, 1, 1),   # two output-channel blocks; channels padded to 48
    (1, 160, 20, 5, 5, 3, 3, 1, 1),  # weights exceed LDS: two channel chunks
    (1, 4, 8, 30, 33, 3, 3, 1, 1),   # many bands per image, bands straddling rows
    (2, 16, 24, 11, 10, 3, 3, 2, 1), # stride 2 slab windows
    (2, 40, 12, 5, 6, 1, 1, 1, 0),   # 1x1 kernel
    (2, 12, 17, 9, 13, 2, 4, 2, 1),  # non-square kernel, stride 2
    (2, 1, 70, 9, 9, 3, 3, 1, 1),    # few taps, 70 channels: two forward channel blocks, ragged weight-grad block
    # few-taps weight gradient on the matrix cores (taps <= 15, <= 64 channels, P % 4 == 0)
    (3, 1, 32, 28, 28, 3, 3, 1, 1),  # cfg3 conv1
    (2, 1, 64, 16, 16, 3, 3, 1, 1),  # four channel blocks
    (2, 1, 48, 20, 20, 1, 1, 1, 0),  # three channel blocks, one tap
    (2, 1, 5, 9, 12, 3, 5, 1, 2),    # 15 taps: the bias column is the last MFMA column
    (2, 3, 17, 12, 12, 2, 2, 2, 0),  # three input channels, stride 2
    # "same" 3x3 over rows of whole pixel quads (direct forward, 4 pixels per thread)
    (2, 2, 13, 6, 12, 3, 3, 1, 1),    # two input channels, ragged output-channel block
    (3, 1, 9, 5, 4, 3, 3, 1, 1),      # one quad per row: both row edges in one quad
    # image-resident 3x3 kernels (channels a multiple of 16, padded rows <= 16)
    (3, 32, 64, 14, 14, 3, 3, 1, 1),  # cfg3 conv2 geometry
    (2, 48, 20, 9, 7, 3, 3, 1, 1),    # ragged second output-channel block
    (2, 32, 40, 14, 14, 3, 3, 1, 0),  # pad 0
    (2, 16, 8, 10, 10, 3, 3, 1, 2),   # pad 2
    (2, 16, 32, 12, 12, 3, 3, 1, 0),  # input gradient at pad 2
    # chunk-pipelined "same" 3x3 kernels (images <= 14x14, even width, whole quads)
    (2, 64, 64, 14, 12, 3, 3, 1, 1),  # two input-gradient blocks, four weight-gradient channel blocks
    (5, 32, 128, 8, 6, 3, 3, 1, 1),   # two weight-gradient channel blocks, odd batch (a 1-image slice)
    (2, 96, 64, 10, 10, 3, 3, 1, 1),  # three output blocks each way, six forward chunks
    (3, 16, 64, 4, 4, 3, 3, 1, 1),    # forward only (16 input channels), one row tile per wave
    (1, 32, 64, 2, 8, 3, 3, 1, 1),    # two rows: most row tiles clamped
    # Winograd F(2x2,3x3) forward ("same" 3x3, C % 16 == 0, M % 32 == 0, even width <= 16)
    (2, 16, 32, 7, 8, 3, 3, 1, 1),    # odd height: the last tile row's second row clipped
    (2, 32, 32, 16, 16, 3, 3, 1, 1),  # 8x8 tiles: every tile block full
    (3, 16, 96, 9, 2, 3, 3, 1, 1),    # one tile per row, three output-channel groups
    (2, 48, 32, 15, 14, 3, 3, 1, 1),  # three channel chunks, 56 tiles
]
ids = ["x".join(map(str, s)) for s in CONV_SHAPES]


def D(hip, x, dtype=np.float32):
    return hip.DeviceBuffer.from_host(x, dtype)


@pytest.mark.parametrize("shape", CONV_SHAPES, ids=ids)
def test_conv_primitives_bit_exact(hip, orc, shape):
    n, ci, co, h, w, kh, kw, s, p = shape
    rng = np.random.default_rng(sum(shape))
    x = rng.standard_normal(n * ci * h * w).astype(np.float32)
    oh, ow = orc.conv_out_hw(h, w, kh, kw, s, p)
    P = oh * ow
    ch = ci * kh * kw

    cols = hip.DeviceBuffer(ch * n * P)
    hip.call("nrs_im2col", cols.ptr, D(hip, x), n, ci, h, w, kh, kw, s, p)
    assert np.array_equal(cols.to_host((ch, n * P)), orc.gpu_im2col(x, n, ci, h, w, kh, kw, s, p))

    mm = rng.standard_normal((co, n * P)).astype(np.float32)
    bias = rng.standard_normal(co).astype(np.float32)
    out = hip.DeviceBuffer(n * co * P)
    hip.call("nrs_col2out", out.ptr, D(hip, mm), D(hip, bias), n, co, oh, ow)
    assert np.array_equal(out.to_host(), orc.gpu_col2out(mm, bias, n, co, P))

    g = rng.standard_normal(n * co * P).astype(np.float32)
    gm = hip.DeviceBuffer(co * n * P)
    hip.call("nrs_out2mm", gm.ptr, D(hip, g), n, co, oh, ow)
    assert np.array_equal(gm.to_host((co, n * P)), orc.gpu_out2mm(g, n, co, P))

    dcols = rng.standard_normal((ch, n * P)).astype(np.float32)
    di = hip.DeviceBuffer(n * ci * h * w)
    hip.call("nrs_col2im", di.ptr, D(hip, dcols), n, ci, h, w, kh, kw, s, p, 0.0)
    assert np.array_equal(di.to_host(), orc.gpu_col2im(dcols, n, ci, h, w, kh, kw, s, p))
    # beta = 1 accumulates: dinput_old + col2im
    d0 = rng.standard_normal(n * ci * h * w).astype(np.float32)
    di2 = D(hip, d0)
    hip.call("nrs_col2im", di2.ptr, D(hip, dcols), n, ci, h, w, kh, kw, s, p, 1.0)
    assert np.array_equal(di2.to_host(), orc.gpu_col2im(dcols, n, ci, h, w, kh, kw, s, p) + d0)

    gi = int_matrix(rng, (n * co * P,))
    db = hip.DeviceBuffer(co)
    hip.call("nrs_conv2d_bias_grad", db.ptr, D(hip, gi), n, co, oh, ow, 0.0)
    assert np.array_equal(db.to_host(), orc.gpu_bias_grad(gi, n, co, P))


@pytest.mark.parametrize("shape", CONV_SHAPES, ids=ids)
def test_conv2d_whole_op_exact_integers(hip, orc, shape):
    n, ci, co, h, w, kh, kw, s, p = shape
    rng = np.random.default_rng(1000 + sum(shape))
    x = int_matrix(rng, (n * ci * h * w,), -3, 3)
    wt = int_matrix(rng, (co * ci * kh * kw,), -3, 3)
    b = int_matrix(rng, (co,), -3, 3)
    oh, ow = orc.conv_out_hw(h, w, kh, kw, s, p)
    ref, _, _ = orc.conv2d_forward(x, wt, b, n, ci, co, h, w, kh, kw, s, p)
    out = hip.DeviceBuffer(n * co * oh * ow)
    dx, dw, db = D(hip, x), D(hip, wt), D(hip, b)
    hip.call("nrs_conv2d_forward", out.ptr, dx.ptr, dw.ptr, db.ptr, n, ci, h, w, co, kh, kw, s, p)
    assert np.array_equal(out.to_host(), ref)

    g = int_matrix(rng, (n * co * oh * ow,), -3, 3)
    di_ref, dw_ref, db_ref = orc.conv2d_backward(x, wt, g, n, ci, co, h, w, kh, kw, s, p)
    gi0 = int_matrix(rng, (x.size,))
    gw0 = int_matrix(rng, (wt.size,))
    gb0 = int_matrix(rng, (co,))
    gI, gW, gB = D(hip, gi0), D(hip, gw0), D(hip, gb0)
    hip.call("nrs_conv2d_backward", gI.ptr, gW.ptr, gB.ptr, D(hip, g), dx.ptr, dw.ptr,
             n, ci, h, w, co, kh, kw, s, p)
    assert np.array_equal(gI.to_host(), gi0 + di_ref)
    assert np.array_equal(gW.to_host(), gw0 + dw_ref)
    assert np.array_equal(gB.to_host(), gb0 + db_ref)


def test_conv2d_forward_twin(hip, orc):
    """tests/cuda_conv2d_test.rs:15-43: GPU conv2d vs CPU conv2d_im2col, tol 1e-4."""
    t = kats()["gpu_twin"]["conv2d_forward"]
    n, ci, h, w, co, kh, kw, s, p = (t[k] for k in ("n", "c_in", "in_h", "in_w", "c_out", "kh", "kw", "stride", "pad"))
    x = formula(t["input"], n * ci * h * w)
    wt = formula(t["weight"], co * ci * kh * kw)
    b = formula(t["bias"], co)
    cpu, oh, ow = orc.conv2d_im2col(x, wt, b, n, ci, co, h, w, kh, kw, s, p)
    out = hip.DeviceBuffer(n * co * oh * ow)
    hip.call("nrs_conv2d_forward", out.ptr, D(hip, x), D(hip, wt), D(hip, b),
             n, ci, h, w, co, kh, kw, s, p)
    close(out.to_host(), cpu, t["tol"], "conv")


def test_conv2d_backward_twin(hip, orc):
    """tests/cuda_conv2d_test.rs:46-96: GPU grads vs CPU Conv2d, tol 1e-3."""
    t = kats()["gpu_twin"]["conv2d_backward"]
    n, ci, h, w, co, kh, kw, s, p = (t[k] for k in ("n", "c_in", "in_h", "in_w", "c_out", "kh", "kw", "stride", "pad"))
    x = formula(t["input"], n * ci * h * w)
    wt = formula(t["weight"], co * ci * kh * kw)
    b = formula(t["bias"], co)
    out, oh, ow = orc.conv2d_forward(x, wt, b, n, ci, co, h, w, kh, kw, s, p)
    seed = formula(t["seed"], out.size)
    ci_g, cw_g, cb_g = orc.conv2d_backward(x, wt, seed, n, ci, co, h, w, kh, kw, s, p)
    gI, gW, gB = hip.DeviceBuffer.zeros(x.size), hip.DeviceBuffer.zeros(wt.size), hip.DeviceBuffer.zeros(co)
    hip.call("nrs_conv2d_backward", gI.ptr, gW.ptr, gB.ptr, D(hip, seed), D(hip, x),
             D(hip, wt), n, ci, h, w, co, kh, kw, s, p)
    close(gI.to_host(), ci_g, t["tol"], "input.grad")
    close(gW.to_host(), cw_g, t["tol"], "weight.grad")
    close(gB.to_host(), cb_g, t["tol"], "bias.grad")


def test_conv2d_backward_without_input_grad(hip, orc):
    """dinput = NULL skips the input gradient (conv.rs:304, requires_grad = false)."""
    n, ci, co, h, w, kh, kw, s, p = 2, 1, 4, 6, 6, 3, 3, 1, 1
    rng = np.random.default_rng(77)
    x = int_matrix(rng, (n * ci * h * w,), -3, 3)
    wt = int_matrix(rng, (co * ci * kh * kw,), -3, 3)
    g = int_matrix(rng, (n * co * h * w,), -3, 3)
    _, dw_ref, db_ref = orc.conv2d_backward(x, wt, g, n, ci, co, h, w, kh, kw, s, p)
    gW, gB = hip.DeviceBuffer.zeros(wt.size), hip.DeviceBuffer.zeros(co)
    hip.call("nrs_conv2d_backward", None, gW.ptr, gB.ptr, D(hip, g), D(hip, x),
             D(hip, wt), n, ci, h, w, co, kh, kw, s, p)
    assert np.array_equal(gW.to_host(), dw_ref)
    assert np.array_equal(gB.to_host(), db_ref)


@pytest.mark.parametrize("shape", [
    (3, 32, 64, 14, 14, 3, 3, 1, 1),  # cfg3 conv2 geometry
    (2, 20, 32, 9, 7, 3, 3, 1, 1),    # ragged input-channel block
    (2, 16, 32, 12, 12, 3, 3, 1, 0),  # the flipped convolution pads by 2
    (2, 8, 16, 10, 10, 3, 3, 1, 2),   # ... and by 0
    (2, 32, 16, 7, 8, 3, 3, 1, 1),    # flipped Winograd: odd height, 16 gradient channels
    (2, 64, 24, 16, 16, 3, 3, 1, 1),  # flipped Winograd: 16x16, three 8-channel chunks
], ids=["cfg3-conv2", "ragged", "pad0", "pad2", "wino-odd", "wino-16x16"])
def test_conv2d_backward_input_grad_only(hip, orc, shape):
    """dweight = dbias = NULL: the input gradient alone (a flipped
    convolution of the output gradient: Winograd or image-resident for these
    shapes), accumulated into dinput."""
    n, ci, co, h, w, kh, kw, s, p = shape
    rng = np.random.default_rng(80 + sum(shape))
    x = int_matrix(rng, (n * ci * h * w,), -3, 3)
    wt = int_matrix(rng, (co * ci * kh * kw,), -3, 3)
    oh, ow = orc.conv_out_hw(h, w, kh, kw, s, p)
    g = int_matrix(rng, (n * co * oh * ow,), -3, 3)
    di_ref, _, _ = orc.conv2d_backward(x, wt, g, n, ci, co, h, w, kh, kw, s, p)
    gi0 = int_matrix(rng, (x.size,))
    gI = D(hip, gi0)
    hip.call("nrs_conv2d_backward", gI.ptr, None, None, D(hip, g), D(hip, x),
             D(hip, wt), n, ci, h, w, co, kh, kw, s, p)
    assert np.array_equal(gI.to_host(), gi0 + di_ref)


@pytest.mark.parametrize("shape", [(2, 1, 4, 6, 6, 3, 3, 1, 1), (2, 6, 5, 9, 9, 3, 3, 1, 1)],
                         ids=["few-taps", "gemm"])
def test_conv2d_backward_bias_only(hip, orc, shape):
    """dweight = NULL, dbias given: only the bias (and input) gradients change."""
    n, ci, co, h, w, kh, kw, s, p = shape
    rng = np.random.default_rng(78)
    x = int_matrix(rng, (n * ci * h * w,), -3, 3)
    wt = int_matrix(rng, (co * ci * kh * kw,), -3, 3)
    oh, ow = orc.conv_out_hw(h, w, kh, kw, s, p)
    g = int_matrix(rng, (n * co * oh * ow,), -3, 3)
    di_ref, _, db_ref = orc.conv2d_backward(x, wt, g, n, ci, co, h, w, kh, kw, s, p)
    gI, gB = hip.DeviceBuffer.zeros(x.size), hip.DeviceBuffer.zeros(co)
    hip.call("nrs_conv2d_backward", gI.ptr, None, gB.ptr, D(hip, g), D(hip, x),
             D(hip, wt), n, ci, h, w, co, kh, kw, s, p)
    assert np.array_equal(gI.to_host(), di_ref)
    assert np.array_equal(gB.to_host(), db_ref)


@pytest.mark.parametrize("shape", [(4, 16, 32, 12, 12, 3, 3, 1, 1), (1, 160, 20, 5, 5, 3, 3, 1, 1),
                                   (1, 40, 70, 6, 7, 3, 3, 1, 1)],
                         ids=["16x128", "64x112", "32x128"])
def test_conv2d_backward_no_bias_grad(hip, orc, shape):
    """dbias = NULL with the input and weight gradients in one launch (each
    slab tile configuration): the weight gradient alone lands in dweight."""
    n, ci, co, h, w, kh, kw, s, p = shape
    rng = np.random.default_rng(79)
    x = int_matrix(rng, (n * ci * h * w,), -3, 3)
    wt = int_matrix(rng, (co * ci * kh * kw,), -3, 3)
    oh, ow = orc.conv_out_hw(h, w, kh, kw, s, p)
    g = int_matrix(rng, (n * co * oh * ow,), -3, 3)
    di_ref, dw_ref, _ = orc.conv2d_backward(x, wt, g, n, ci, co, h, w, kh, kw, s, p)
    gI, gW = hip.DeviceBuffer.zeros(x.size), hip.DeviceBuffer.zeros(wt.size)
    hip.call("nrs_conv2d_backward", gI.ptr, gW.ptr, None, D(hip, g), D(hip, x),
             D(hip, wt), n, ci, h, w, co, kh, kw, s, p)
    assert np.array_equal(gI.to_host(), di_ref)
    assert np.array_equal(gW.to_host(), dw_ref)


def test_conv2d_cfg3_layers(hip, orc):
    """cfg3 shapes (batch 128, 1->32 @28x28 and 32->64 @14x14, 3x3 pad 1):
    GPU forward/backward against the restated CPU Conv2d on the same data."""
    rng = np.random.default_rng(3)
    for (n, ci, co, h, w) in ((128, 1, 32, 28, 28), (128, 32, 64, 14, 14)):
        x = rng.uniform(0, 1, n * ci * h * w).astype(np.float32)
        wt = (rng.standard_normal(co * ci * 9) * np.sqrt(2.0 / (ci * 9))).astype(np.float32)
        b = np.zeros(co, np.float32)
        ref, oh, ow = orc.conv2d_forward(x, wt, b, n, ci, co, h, w, 3, 3, 1, 1)
        out = hip.DeviceBuffer(ref.size)
        dx, dw = D(hip, x), D(hip, wt)
        hip.call("nrs_conv2d_forward", out.ptr, dx.ptr, dw.ptr, D(hip, b),
                 n, ci, h, w, co, 3, 3, 1, 1)
        close(out.to_host(), ref, 1e-4, f"cfg3 fwd {ci}->{co}")
        g = rng.standard_normal(ref.size).astype(np.float32)
        di, dwr, dbr = orc.conv2d_backward(x, wt, g, n, ci, co, h, w, 3, 3, 1, 1)
        gI, gW, gB = hip.DeviceBuffer.zeros(x.size), hip.DeviceBuffer.zeros(wt.size), hip.DeviceBuffer.zeros(co)
        hip.call("nrs_conv2d_backward", gI.ptr, gW.ptr, gB.ptr, D(hip, g), dx.ptr, dw.ptr,
                 n, ci, h, w, co, 3, 3, 1, 1)
        close(gI.to_host(), di, 1e-3, "cfg3 dinput")
        # weight/bias grads sum N*P = 100352 / 25088 terms: f64 ground truth
        # with the f32-accumulation bar, for the GPU and the CPU restatement.
        gm = orc.gpu_out2mm(g, n, co, oh * ow).astype(np.float64)
        cols = orc.gpu_im2col(x, n, ci, h, w, 3, 3, 1, 1).astype(np.float64)
        dw64 = gm @ cols.T
        dwab = np.abs(gm) @ np.abs(cols).T
        db64 = gm.sum(axis=1)
        dbab = np.abs(gm).sum(axis=1)
        K = n * oh * ow
        for got in (gW.to_host().reshape(co, -1), dwr.reshape(co, -1)):
            assert rel_err(got, dw64, dwab) <= gemm_tol(K)
        for got in (gB.to_host(), dbr):
            assert rel_err(got, db64, dbab) <= gemm_tol(K)


@pytest.mark.parametrize("shape", [(16, 32, 64, 14, 14), (2, 96, 64, 10, 10), (3, 48, 32, 15, 14),
                                   (2, 16, 32, 16, 16)], ids=lambda s: "x".join(map(str, s)))
def test_conv2d_winograd_forward_vs_f64(hip, orc, shape):
    """The Winograd F(2x2,3x3) forward on general data: within the f32
    accumulation bar gemm_tol(C*9) of the f64 direct sum, on the scale
    sum |x||w| that bounds any summation order, times 8 for the transforms'
    extra roundings (each transformed term is a short +-1 or 1/2 sum of
    inputs and weights). The observed ratio is printed."""
    n, ci, co, h, w = shape
    rng = np.random.default_rng(sum(shape))
    x = rng.standard_normal(n * ci * h * w).astype(np.float32)
    wt = (rng.standard_normal(co * ci * 9) / np.sqrt(ci * 9)).astype(np.float32)
    b = rng.standard_normal(co).astype(np.float32)
    out = hip.DeviceBuffer(n * co * h * w)
    hip.call("nrs_conv2d_forward", out.ptr, D(hip, x), D(hip, wt), D(hip, b), n, ci, h, w, co, 3, 3, 1, 1)
    cols = orc.gpu_im2col(x, n, ci, h, w, 3, 3, 1, 1).astype(np.float64)
    w64 = wt.reshape(co, -1).astype(np.float64)
    y64 = (w64 @ cols + b[:, None]).reshape(co, n, h * w).transpose(1, 0, 2)
    yab = ((np.abs(w64) @ np.abs(cols)) + np.abs(b)[:, None]).reshape(co, n, h * w).transpose(1, 0, 2)
    got = out.to_host((n, co, h * w))
    err = rel_err(got, y64, yab)
    print(f"winograd rel err {err:.3g} (f32 bar {gemm_tol(ci * 9):.3g})")
    assert err <= 8 * gemm_tol(ci * 9)


# ------------------------------------------------------------ plumbing kernels
def test_accumulate_vadd_bias_add_sum_axis0(hip, orc):
    rng = np.random.default_rng(21)
    for n in (1, 3, 1000, 1 << 20, (1 << 20) + 3):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        da = D(hip, a)
        hip.call("nrs_accumulate", da.ptr, D(hip, b), n)
        assert np.array_equal(da.to_host(), a + b)
        out = hip.DeviceBuffer(n)
        hip.call("nrs_vadd", out.ptr, D(hip, a), D(hip, b), n)
        assert np.array_equal(out.to_host(), a + b)
    for rows, cols in ((16, 10), (4096, 1024), (256, 128), (1, 7), (3000, 3)):
        a = rng.standard_normal((rows, cols)).astype(np.float32)
        bias = rng.standard_normal(cols).astype(np.float32)
        out = hip.DeviceBuffer(rows * cols)
        hip.call("nrs_bias_add", out.ptr, D(hip, a), D(hip, bias), rows, cols)
        assert np.array_equal(out.to_host((rows, cols)), orc.graph_add_bias_forward(a, bias))
        ai = int_matrix(rng, (rows, cols))
        s = hip.DeviceBuffer(cols)
        hip.call("nrs_sum_axis0", s.ptr, D(hip, ai), rows, cols, 0.0)
        assert np.array_equal(s.to_host(), orc.sum_axis0(ai))
        s0 = int_matrix(rng, (cols,))
        s2 = D(hip, s0)
        hip.call("nrs_sum_axis0", s2.ptr, D(hip, a), rows, cols, 1.0)
        close(s2.to_host(), orc.sum_axis0(a) + s0, 1e-5 * np.sqrt(rows) * 4, "sum_axis0 float")


@pytest.mark.parametrize("dims", [(2, 3, 6, 8, 2, 2), (128, 32, 28, 28, 2, 2), (1, 2, 7, 7, 3, 2),
                                  (2, 1, 5, 5, 2, 1), (3, 2, 7, 9, 2, 2)])
def test_maxpool_bit_exact(hip, orc, dims):
    n, c, h, w, k, s = dims
    rng = np.random.default_rng(sum(dims))
    x = rng.standard_normal(n * c * h * w).astype(np.float32)
    tie = np.arange(0, x.size - 1, 7)
    x[tie] = x[tie + 1]  # plant ties: the first maximum must win
    out_ref, am_ref = orc.maxpool_forward(x, n, c, h, w, k, s)
    out = hip.DeviceBuffer(out_ref.size)
    am = hip.DeviceBuffer(out_ref.size, np.int32)
    dx = D(hip, x)
    hip.call("nrs_maxpool_forward", out.ptr, am.ptr, dx.ptr, n, c, h, w, k, s)
    assert np.array_equal(out.to_host(), out_ref)
    assert np.array_equal(am.to_host(), am_ref)
    g = int_matrix(rng, out_ref.shape)
    d0 = int_matrix(rng, x.shape)
    di = D(hip, d0)
    hip.call("nrs_maxpool_backward", di.ptr, D(hip, g), am.ptr, n, c, h, w, k, s)
    assert np.array_equal(di.to_host(), orc.maxpool_backward(g, am_ref, x.size, d0))


# ------------------------------------------------ conv2d + maxpool, fused
POOL_SHAPES = [  # (n, c_in, c_out, h, w, kh, kw, stride, pad, pool_k, pool_stride)
    (128, 1, 32, 28, 28, 3, 3, 1, 1, 2, 2),   # cfg3 conv1 -> maxpool: the fused kernels
    (3, 3, 20, 8, 12, 3, 3, 1, 1, 2, 2),      # 3 input channels, ragged channel block
    (2, 2, 9, 6, 4, 3, 3, 1, 1, 2, 2),
    (2, 4, 6, 8, 8, 3, 3, 1, 1, 2, 2),        # 4 input channels: forward runs the two ops
    (2, 1, 5, 7, 9, 3, 3, 1, 1, 2, 2),        # odd sizes: the two ops (and a partial window)
    (2, 2, 4, 9, 9, 3, 3, 1, 1, 3, 3),        # 3x3 pooling
    (2, 3, 4, 8, 8, 5, 5, 1, 2, 2, 2),        # 5x5 conv
]


def _pool_ref(hip, x, w, b, shape, floats, relu=False):
    n, ci, co, h, wd, kh, kw, s, p, pk, ps = shape
    D = hip.DeviceBuffer.from_host
    oh, ow = (h + 2 * p - kh) // s + 1, (wd + 2 * p - kw) // s + 1
    ph, pw = (oh - pk) // ps + 1, (ow - pk) // ps + 1
    y = hip.DeviceBuffer(n * co * oh * ow)
    hip.call("nrs_conv2d_forward", y, D(x), D(w), D(b), n, ci, h, wd, co, kh, kw, s, p)
    a = y
    if relu:
        a = hip.DeviceBuffer(n * co * oh * ow)
        hip.call("nrs_relu_forward", a, y, n * co * oh * ow)
    pooled, am = hip.DeviceBuffer(n * co * ph * pw), hip.DeviceBuffer(n * co * ph * pw, np.int32)
    hip.call("nrs_maxpool_forward", pooled, am, a, n, co, oh, ow, pk, ps)
    return y.to_host(), pooled.to_host(), am.to_host(), (oh, ow, ph, pw)


@pytest.mark.parametrize("shape", POOL_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("floats", [False, True], ids=["ints", "floats"])
@pytest.mark.parametrize("relu", [False, True], ids=["pool", "relu_pool"])
def test_conv2d_maxpool_forward_matches_the_two_ops(hip, orc, shape, floats, relu):
    """nrs_conv2d_maxpool_forward (nrs_conv2d_relu_maxpool_forward with relu)
    gives the pooled values, argmax and (when asked) conv output of
    nrs_conv2d_forward then (nrs_relu_forward then) nrs_maxpool_forward, bit
    for bit (small integers, with ties the first maximum wins; and f32 data).
    The integer case is also checked against the oracle's Conv2d forward, the
    ReLU and its max pooling."""
    n, ci, co, h, wd, kh, kw, s, p, pk, ps = shape
    rng = np.random.default_rng(n * 100 + ci * 10 + co)
    if floats:
        x = rng.standard_normal(n * ci * h * wd).astype(np.float32)
        w = (rng.standard_normal(co * ci * kh * kw) * 0.3).astype(np.float32)
        b = rng.standard_normal(co).astype(np.float32)
    else:
        x = int_matrix(rng, (n * ci * h * wd,), -2, 2)
        w = int_matrix(rng, (co * ci * kh * kw,), -2, 2)
        b = int_matrix(rng, (co,), -2, 2)
    y_ref, pool_ref, am_ref, (oh, ow, ph, pw) = _pool_ref(hip, x, w, b, shape, floats, relu)
    if not floats:
        y64, _, _ = orc.conv2d_forward(x, w, b, n, ci, co, h, wd, kh, kw, s, p)
        a64 = np.where(y64 > 0, y64, 0).astype(np.float32) if relu else y64
        po, ao = orc.maxpool_forward(a64, n, co, oh, ow, pk, ps)
        assert np.array_equal(po, pool_ref) and np.array_equal(ao, am_ref)
    D = hip.DeviceBuffer.from_host
    entry = "nrs_conv2d_relu_maxpool_forward" if relu else "nrs_conv2d_maxpool_forward"
    for with_out in (False, True):
        pooled, am = hip.DeviceBuffer(n * co * ph * pw), hip.DeviceBuffer(n * co * ph * pw, np.int32)
        y = hip.DeviceBuffer(n * co * oh * ow) if with_out else None
        print(f"{entry} {shape} floats={floats} out={with_out}", flush=True)
        hip.call(entry, pooled, am, y, D(x), D(w), D(b), n, ci, h, wd, co, kh, kw, s, p, pk, ps)
        assert np.array_equal(pooled.to_host(), pool_ref)
        assert np.array_equal(am.to_host(), am_ref)
        if with_out:
            assert np.array_equal(y.to_host(), y_ref)


@pytest.mark.parametrize("shape", POOL_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("with_dx", [False, True], ids=["w_b", "x_w_b"])
@pytest.mark.parametrize("relu", [False, True], ids=["pool", "relu_pool"])
def test_maxpool_conv2d_backward_matches_the_two_ops(hip, orc, shape, with_dx, relu):
    """nrs_maxpool_conv2d_backward (weight and bias gradients, and the input
    gradient when asked) equals maxpool_backward into zeros followed by
    nrs_conv2d_backward, bit for bit, accumulating over old values; the
    weight-only form of cfg3 conv1 expands the pooled gradient while loading.
    With relu, nrs_maxpool_relu_conv2d_backward against maxpool_backward,
    then relu_backward on the conv output, then nrs_conv2d_backward. Also
    checked against the oracle's maxpool and conv2d backward on small
    integers."""
    n, ci, co, h, wd, kh, kw, s, p, pk, ps = shape
    rng = np.random.default_rng(n * 7 + ci * 3 + co)
    x = int_matrix(rng, (n * ci * h * wd,), -2, 2)
    w = int_matrix(rng, (co * ci * kh * kw,), -2, 2)
    b = np.zeros(co, np.float32)
    y, pooled, am, (oh, ow, ph, pw) = _pool_ref(hip, x, w, b, shape, False, relu)
    gp = int_matrix(rng, (n * co * ph * pw,), -3, 3)
    D = hip.DeviceBuffer.from_host
    old_x, old_w, old_b = (int_matrix(rng, (m,), -3, 3) for m in (x.size, w.size, co))
    # the two (three) ops
    dam = hip.DeviceBuffer.from_host(am, np.int32)
    g = hip.DeviceBuffer.zeros(n * co * oh * ow)
    hip.call("nrs_maxpool_backward", g, D(gp), dam, n, co, oh, ow, pk, ps)
    if relu:
        gr = hip.DeviceBuffer(n * co * oh * ow)
        hip.call("nrs_relu_backward", gr, g, D(y), n * co * oh * ow, 0.0)
        g = gr
    rx, rw, rb = D(old_x), D(old_w), D(old_b)
    hip.call("nrs_conv2d_backward", rx if with_dx else None, rw, rb, g, D(x), D(w), n, ci, h, wd,
             co, kh, kw, s, p)
    fx, fw, fb = D(old_x), D(old_w), D(old_b)
    print(f"maxpool conv2d backward {shape} dx={with_dx} relu={relu}", flush=True)
    if relu:
        hip.call("nrs_maxpool_relu_conv2d_backward", fx if with_dx else None, fw, fb, D(gp), dam,
                 D(pooled), D(x), D(w), n, ci, h, wd, co, kh, kw, s, p, pk, ps, 1.0)
    else:
        hip.call("nrs_maxpool_conv2d_backward", fx if with_dx else None, fw, fb, D(gp), dam, D(x),
                 D(w), n, ci, h, wd, co, kh, kw, s, p, pk, ps)
    assert np.array_equal(fw.to_host(), rw.to_host())
    assert np.array_equal(fb.to_host(), rb.to_host())
    if with_dx:
        assert np.array_equal(fx.to_host(), rx.to_host())
    # the oracle: maxpool backward into zeros (gated by conv output > 0 with
    # the ReLU), then Conv2d's backward
    g_ref = orc.maxpool_backward(gp, am, n * co * oh * ow)
    if relu:
        g_ref = np.where(y > 0, g_ref, 0).astype(np.float32)
    _, dw_ref, db_ref = orc.conv2d_backward(x, w, g_ref, n, ci, co, h, wd, kh, kw, s, p)
    assert np.array_equal(fw.to_host(), dw_ref.ravel() + old_w)
    assert np.array_equal(fb.to_host(), db_ref.ravel() + old_b)
    assert np.any(dw_ref != 0)  # the pooled gradient reached the weights


FUSED_LOWER_SHAPES = [  # (n, c_lo, c_mid, c_out, h, w): lower "same" 3x3, 2x2 pool, upper "same" 3x3
    (3, 1, 32, 64, 28, 28),   # cfg3's layers: one launch plus the sums
    (128, 1, 32, 64, 28, 28),  # cfg3 at its full batch (integer sums stay below 2^24)
    (2, 2, 32, 64, 12, 16),   # two lower input channels, pooled 6x8
    (2, 1, 64, 64, 8, 8),     # two input-gradient blocks per image, pooled 4x4
    (2, 3, 32, 64, 8, 8),     # three lower channels: the two calls
    (2, 1, 16, 8, 10, 10),    # channel counts off the kernel's blocks: the two calls
    (1, 1, 32, 64, 6, 6),     # pooled 3x3 (odd width): the two calls
]


@pytest.mark.parametrize("shape", FUSED_LOWER_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("floats", [False, True], ids=["ints", "floats"])
@pytest.mark.parametrize("beta_p", [0.0, 1.0])
def test_conv2d_maxpool_relu_conv2d_backward(hip, orc, shape, floats, beta_p):
    """nrs_conv2d_maxpool_relu_conv2d_backward against its definition, the
    upper layer's nrs_conv2d_backward_ex then nrs_maxpool_relu_conv2d_backward
    without the lower input gradient: the pooled gradient and the upper
    layer's weight and bias gradients bit for bit (the same kernels); the
    lower layer's bit for bit on small integers (its sum runs over each
    window's argmax pixel in another order) and within f32 rounding on
    normal data; beta_params 0 over NaN and 1 over old values. The integer
    case is also checked against the oracle's max pool, ReLU gate and
    Conv2d backward."""
    n, clo, cm, co, h, w = shape
    rng = np.random.default_rng(n + 3 * clo + cm + co + h)
    ph, pw = h // 2, w // 2
    if floats:
        x = rng.standard_normal(n * clo * h * w).astype(np.float32)
        w1 = (rng.standard_normal(cm * clo * 9) * 0.3).astype(np.float32)
        b1 = (rng.standard_normal(cm) * 0.1).astype(np.float32)
        w2 = (rng.standard_normal(co * cm * 9) * 0.1).astype(np.float32)
        g = rng.standard_normal(n * co * ph * pw).astype(np.float32)
    else:
        x = int_matrix(rng, (n * clo * h * w,), -2, 2)
        w1 = int_matrix(rng, (cm * clo * 9,), -2, 2)
        b1 = int_matrix(rng, (cm,), -2, 2)
        w2 = int_matrix(rng, (co * cm * 9,), -2, 2)
        g = int_matrix(rng, (n * co * ph * pw,), -2, 2)
    D = hip.DeviceBuffer.from_host
    pooled = hip.DeviceBuffer(n * cm * ph * pw)
    am = hip.DeviceBuffer(n * cm * ph * pw, np.int32)
    y = hip.DeviceBuffer(n * cm * h * w)
    hip.call("nrs_conv2d_relu_maxpool_forward", pooled, am, y, D(x), D(w1), D(b1), n, clo, h, w,
             cm, 3, 3, 1, 1, 2, 2)
    if beta_p:
        olds = [int_matrix(rng, (k,), -3, 3) for k in (w2.size, co, w1.size, cm)]
    else:
        olds = [np.full(k, np.nan, np.float32) for k in (w2.size, co, w1.size, cm)]
    # the definition: the two calls
    rp, rw2, rb2, rw1, rb1 = (hip.DeviceBuffer(n * cm * ph * pw),) + tuple(D(o) for o in olds)
    hip.call("nrs_conv2d_backward_ex", rp, rw2, rb2, D(g), pooled, D(w2), n, cm, ph, pw, co, 3, 3,
             1, 1, 0.0, beta_p)
    hip.call("nrs_maxpool_relu_conv2d_backward", None, rw1, rb1, rp, am, pooled, D(x), D(w1), n,
             clo, h, w, cm, 3, 3, 1, 1, 2, 2, beta_p)
    fp = D(np.full(n * cm * ph * pw, np.nan, np.float32))
    fw2, fb2, fw1, fb1 = (D(o) for o in olds)
    print(f"conv2d maxpool relu conv2d backward {shape} floats={floats} beta={beta_p}", flush=True)
    hip.call("nrs_conv2d_maxpool_relu_conv2d_backward", fp, fw2, fb2, fw1, fb1, D(g), pooled,
             D(w2), am, D(x), D(w1), n, clo, h, w, cm, 3, 3, 1, 1, 2, 2, co, 3, 3, 1, 1, beta_p)
    assert np.array_equal(fp.to_host(), rp.to_host())
    assert np.array_equal(fw2.to_host(), rw2.to_host())
    assert np.array_equal(fb2.to_host(), rb2.to_host())
    got_w1, got_b1, ref_w1, ref_b1 = fw1.to_host(), fb1.to_host(), rw1.to_host(), rb1.to_host()
    if floats:
        # both sum the same products: within a few roundings of their scale
        for got, ref in ((got_w1, ref_w1), (got_b1, ref_b1)):
            scale = np.max(np.abs(ref)) + 1.0
            assert np.max(np.abs(got - ref)) <= 1e-5 * scale
    else:
        assert np.array_equal(got_w1, ref_w1)
        assert np.array_equal(got_b1, ref_b1)
        # the oracle: pooled gradient to the argmax pixels, ReLU gate on the
        # conv output, Conv2d backward
        y_h = y.to_host()
        gu = orc.maxpool_backward(rp.to_host(), am.to_host(), n * cm * h * w)
        gu = np.where(y_h > 0, gu, 0).astype(np.float32)
        _, dw_ref, db_ref = orc.conv2d_backward(x, w1, gu, n, clo, cm, h, w, 3, 3, 1, 1)
        base_w, base_b = (olds[2], olds[3]) if beta_p else (0.0, 0.0)
        assert np.array_equal(got_w1, dw_ref.ravel() + base_w)
        assert np.array_equal(got_b1, db_ref.ravel() + base_b)
        assert np.any(dw_ref != 0)


@pytest.mark.parametrize("shape", [(2, 3, 4, 8, 8, 3, 3, 1, 1), (3, 1, 32, 28, 28, 3, 3, 1, 1),
                                   (3, 32, 64, 14, 14, 3, 3, 1, 1), (2, 6, 5, 9, 9, 3, 3, 1, 1),
                                   (1, 8, 3, 7, 7, 3, 3, 2, 1), (2, 2, 3, 6, 6, 2, 2, 1, 2),
                                   (1, 40, 70, 6, 7, 3, 3, 1, 1), (2, 16, 24, 11, 10, 3, 3, 2, 1)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("beta_p", [0.0, 0.5])
@pytest.mark.parametrize("with_dx", [False, True], ids=["dw_db", "dx_dw_db"])
def test_conv2d_backward_ex_param_beta(hip, orc, shape, beta_p, with_dx):
    """nrs_conv2d_backward_ex: dweight and dbias = gradient + beta_params *
    old on every weight-gradient path (chunk-pipelined, slab pair, few-taps,
    small, slab, split-K GEMM); beta 0 over NaN shows that the old values
    are not read. dinput takes beta_input 1 (it accumulates)."""
    n, ci, co, h, w, kh, kw, s, p = shape
    rng = np.random.default_rng(7 * n + ci + co + h)
    x = int_matrix(rng, (n * ci * h * w,), -2, 2)
    wt = int_matrix(rng, (co * ci * kh * kw,), -2, 2)
    oh, ow = (h + 2 * p - kh) // s + 1, (w + 2 * p - kw) // s + 1
    g = int_matrix(rng, (n * co * oh * ow,), -2, 2)
    di_ref, dw_ref, db_ref = orc.conv2d_backward(x, wt, g, n, ci, co, h, w, kh, kw, s, p)
    if beta_p:
        ow0, ob0 = int_matrix(rng, (wt.size,), -3, 3), int_matrix(rng, (co,), -3, 3)
    else:
        ow0, ob0 = np.full(wt.size, np.nan, np.float32), np.full(co, np.nan, np.float32)
    di0 = int_matrix(rng, (x.size,), -3, 3)
    D = hip.DeviceBuffer.from_host
    ddi, ddw, ddb = D(di0), D(ow0), D(ob0)
    print(f"conv2d backward ex {shape} beta_params={beta_p} dx={with_dx}", flush=True)
    hip.call("nrs_conv2d_backward_ex", ddi if with_dx else None, ddw, ddb, D(g), D(x), D(wt),
             n, ci, h, w, co, kh, kw, s, p, 1.0, beta_p)
    assert np.array_equal(ddw.to_host(), dw_ref.ravel() + (beta_p * ow0 if beta_p else 0))
    assert np.array_equal(ddb.to_host(), db_ref.ravel() + (beta_p * ob0 if beta_p else 0))
    if with_dx:
        assert np.array_equal(ddi.to_host(), di_ref.ravel() + di0)


@pytest.mark.parametrize("shape", [(1, 32, 28, 28, 3, 3, 1, 1), (32, 64, 14, 14, 3, 3, 1, 1),
                                   (40, 70, 6, 7, 3, 3, 1, 1)], ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("beta_p", [0.0, 0.5, 1.0])
def test_conv2d_backward_empty_batch(hip, shape, beta_p):
    """No images: nrs_conv2d_backward_ex, nrs_maxpool_relu_conv2d_backward
    and nrs_conv2d_relu_maxpool_forward return OK; the weight and bias
    gradients become the empty sums plus beta_params * old (zeros over NaN
    under beta 0), as nrs_linear_backward does with no rows."""
    ci, co, h, w, kh, kw, s, p = shape
    rng = np.random.default_rng(ci + co)
    nw = co * ci * kh * kw
    D = hip.DeviceBuffer.from_host
    for entry in ("nrs_conv2d_backward_ex", "nrs_maxpool_relu_conv2d_backward"):
        if beta_p:
            ow0, ob0 = int_matrix(rng, (nw,), -3, 3), int_matrix(rng, (co,), -3, 3)
        else:
            ow0, ob0 = np.full(nw, np.nan, np.float32), np.full(co, np.nan, np.float32)
        ddw, ddb = D(ow0), D(ob0)
        print(f"{entry} N=0 {shape} beta_params={beta_p}", flush=True)
        if entry == "nrs_conv2d_backward_ex":
            hip.call(entry, None, ddw, ddb, None, None, None, 0, ci, h, w, co, kh, kw, s, p, 1.0,
                     beta_p)
        else:
            hip.call(entry, None, ddw, ddb, None, None, None, None, None, 0, ci, h, w, co, kh, kw,
                     s, p, 2, 2, beta_p)
        assert np.array_equal(ddw.to_host(), beta_p * ow0 if beta_p else np.zeros(nw))
        assert np.array_equal(ddb.to_host(), beta_p * ob0 if beta_p else np.zeros(co))
    hip.call("nrs_conv2d_relu_maxpool_forward", None, None, None, None, None, None, 0, ci, h, w,
             co, kh, kw, s, p, 2, 2)


def test_attention_empty_batch(hip):
    """No sequences: both attention entries return OK, on the short and the
    long path, without reading their (null) operands."""
    for seq in (64, 1024):
        print(f"attention batch 0 seq {seq}", flush=True)
        hip.call("nrs_attention_forward", None, None, None, None, None, 0, 4, seq, 32, 128,
                 32 ** -0.5)
        hip.call("nrs_attention_backward", None, None, None, None, None, None, None, None, None,
                 0, 4, seq, 32, 128, 32 ** -0.5, 0.0)


@pytest.mark.parametrize("shape", [(2, 3, 4, 8, 8, 3, 3, 1, 1), (3, 1, 32, 28, 28, 3, 3, 1, 1),
                                   (2, 32, 64, 14, 14, 3, 3, 1, 1), (2, 6, 5, 9, 9, 3, 3, 1, 1),
                                   (1, 8, 3, 7, 7, 3, 3, 2, 1), (2, 2, 3, 6, 6, 2, 2, 1, 2),
                                   (1, 40, 70, 6, 7, 3, 3, 1, 1)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("beta", [0.0, 0.5, 1.0])
@pytest.mark.parametrize("with_w", [False, True], ids=["dx", "dx_dw_db"])
def test_conv2d_backward_beta(hip, orc, shape, beta, with_w):
    """nrs_conv2d_backward_beta: dinput = its gradient + beta * dinput on every
    input-gradient path (pixel quads, direct, slab and the slab pair with the
    weight gradient, implicit GEMM, col2im); beta 0 over NaN shows that the
    old values are not read. Weight and bias gradients accumulate."""
    n, ci, co, h, w, kh, kw, s, p = shape
    rng = np.random.default_rng(n + ci + co + h)
    x = int_matrix(rng, (n * ci * h * w,), -2, 2)
    wt = int_matrix(rng, (co * ci * kh * kw,), -2, 2)
    oh, ow = (h + 2 * p - kh) // s + 1, (w + 2 * p - kw) // s + 1
    g = int_matrix(rng, (n * co * oh * ow,), -2, 2)
    di_ref, dw_ref, db_ref = orc.conv2d_backward(x, wt, g, n, ci, co, h, w, kh, kw, s, p)
    old = int_matrix(rng, (x.size,), -3, 3) if beta else np.full(x.size, np.nan, np.float32)
    ow0, ob0 = int_matrix(rng, (wt.size,), -3, 3), int_matrix(rng, (co,), -3, 3)
    D = hip.DeviceBuffer.from_host
    ddi, ddw, ddb = D(old), D(ow0), D(ob0)
    print(f"conv2d backward beta {shape} beta={beta} w={with_w}", flush=True)
    hip.call("nrs_conv2d_backward_beta", ddi, ddw if with_w else None, ddb if with_w else None,
             D(g), D(x), D(wt), n, ci, h, w, co, kh, kw, s, p, beta)
    want = di_ref.ravel() + (beta * old if beta else 0)
    assert np.array_equal(ddi.to_host(), want)
    if with_w:
        assert np.array_equal(ddw.to_host(), dw_ref.ravel() + ow0)
        assert np.array_equal(ddb.to_host(), db_ref.ravel() + ob0)


def _wino_sweep_shapes():
    """Seeded random shapes of the Winograd and chunk-pipelined 3x3 paths:
    heights 1..16, even widths 2..16, 8..96 input channels (multiples of 8),
    32..96 output channels (multiples of 32), 1..3 images."""
    rng = np.random.default_rng(2026)
    shapes = []
    for _ in range(24):
        h = int(rng.integers(1, 17))
        w = int(rng.choice(np.arange(2, 17, 2)))
        ci = int(rng.choice([8, 16, 24, 32, 48, 64, 96]))
        co = int(rng.choice([32, 64, 96]))
        n = int(rng.integers(1, 4))
        shapes.append((n, ci, co, h, w))
    return shapes


@pytest.mark.parametrize("shape", _wino_sweep_shapes(), ids=lambda s: "x".join(map(str, s)))
def test_conv2d_same3x3_sweep_exact_integers(hip, orc, shape):
    """"Same" 3x3 layers at random eligible sizes (Winograd forward and input
    gradient, chunk-pipelined backward where their blocks fit): forward, the
    input gradient alone (beta 1 over old values), and the whole backward,
    each exact against the oracle on small integers."""
    n, ci, co, h, w = shape
    rng = np.random.default_rng(7 * sum(shape))
    x = int_matrix(rng, (n * ci * h * w,), -3, 3)
    wt = int_matrix(rng, (co * ci * 9,), -3, 3)
    b = int_matrix(rng, (co,), -3, 3)
    ref, _, _ = orc.conv2d_forward(x, wt, b, n, ci, co, h, w, 3, 3, 1, 1)
    out = hip.DeviceBuffer(n * co * h * w)
    dx, dw, db = D(hip, x), D(hip, wt), D(hip, b)
    hip.call("nrs_conv2d_forward", out.ptr, dx.ptr, dw.ptr, db.ptr, n, ci, h, w, co, 3, 3, 1, 1)
    assert np.array_equal(out.to_host(), ref)
    g = int_matrix(rng, (n * co * h * w,), -3, 3)
    di_ref, dw_ref, db_ref = orc.conv2d_backward(x, wt, g, n, ci, co, h, w, 3, 3, 1, 1)
    gi0 = int_matrix(rng, (x.size,))
    gI = D(hip, gi0)
    hip.call("nrs_conv2d_backward", gI.ptr, None, None, D(hip, g), dx.ptr, dw.ptr,
             n, ci, h, w, co, 3, 3, 1, 1)
    assert np.array_equal(gI.to_host(), gi0 + di_ref)
    gI2, gW, gB = hip.DeviceBuffer.zeros(x.size), hip.DeviceBuffer.zeros(wt.size), hip.DeviceBuffer.zeros(co)
    hip.call("nrs_conv2d_backward", gI2.ptr, gW.ptr, gB.ptr, D(hip, g), dx.ptr, dw.ptr,
             n, ci, h, w, co, 3, 3, 1, 1)
    assert np.array_equal(gI2.to_host(), di_ref)
    assert np.array_equal(gW.to_host(), dw_ref)
    assert np.array_equal(gB.to_host(), db_ref)
