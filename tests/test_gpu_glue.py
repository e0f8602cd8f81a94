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


def test_glue_argument_errors(hip):
    b = hip.DeviceBuffer(4)
    with pytest.raises(hip.NrsError):
        hip.call("nrs_transpose", b.ptr, b.ptr, 1, 2, 2)  # aliased
    with pytest.raises(hip.NrsError):
        hip.call("nrs_softmax_forward", b.ptr, b.ptr, 1, 0)
