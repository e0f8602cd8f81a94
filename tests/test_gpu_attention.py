"""The fused attention core (nrs_attention_forward / _backward) through the C
ABI: every head of MultiHeadAttention::forward_batch read and written in place
in [batch*seq, ld] rows (src/cuda/nn/multihead.rs:57-85), each head being
attention_batch (src/cuda/nn/attention.rs:23-32).

References:
  * numpy float64 of the same algebra (scores, scale, max-subtracted softmax,
    P.V and the backward of each step);
  * the oracle's restatement of the reference's CPU ops composed as
    attention_batch composes them (bmm with a transposed K, scale, softmax,
    bmm), per head after slice_cols, for the cfg4 shape.
Bar: |gpu - ref| <= 1e-5 * sqrt(L) * max|ref| + 1e-6, L = max(seq, d_head),
the longest reduction of the products (the north-star f32 accumulation bar);
the gradients also go through exp and the softmax Jacobian, given 4x that.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def heads_view(x, batch, heads, seq, d, ld):
    """[batch*seq, ld] rows -> [batch, heads, seq, d] (head h at columns h*d..)."""
    return x.reshape(batch, seq, ld)[:, :, : heads * d].reshape(batch, seq, heads, d).transpose(0, 2, 1, 3)


def ref_f64(q, k, v, dout, scale):
    q, k, v, dout = (x.astype(np.float64) for x in (q, k, v, dout))
    s = np.matmul(q, k.transpose(0, 1, 3, 2)) * scale
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    p = e / e.sum(axis=-1, keepdims=True)
    o = np.matmul(p, v)
    dp = np.matmul(dout, v.transpose(0, 1, 3, 2))
    ds = p * (dp - (p * dp).sum(axis=-1, keepdims=True)) * scale
    return o, np.matmul(ds, k), np.matmul(ds.transpose(0, 1, 3, 2), q), np.matmul(p.transpose(0, 1, 3, 2), dout)


def check(got, want, L, factor, what):
    tol = factor * 1e-5 * np.sqrt(L) * np.abs(want).max() + 1e-6
    err = np.abs(got - want).max()
    assert err <= tol, f"{what}: max err {err:.3g} > {tol:.3g}"


def run(hip, batch, heads, seq, d, ld, beta, seed):
    rng = np.random.default_rng(seed)
    rows = batch * seq
    q, k, v, dout = (rng.standard_normal((rows, ld)).astype(np.float32) for _ in range(4))
    scale = np.float32(1.0 / np.sqrt(d))
    old = [rng.standard_normal((rows, ld)).astype(np.float32) for _ in range(3)]
    out0 = rng.standard_normal((rows, ld)).astype(np.float32)
    dq_, dk_, dv_, do_ = (hip.DeviceBuffer.from_host(x) for x in (q, k, v, dout))
    out = hip.DeviceBuffer.from_host(out0)
    stats = hip.DeviceBuffer(batch * heads * seq * 2)
    print(f"attention b{batch} h{heads} s{seq} d{d} ld{ld} beta{beta}", flush=True)
    hip.call("nrs_attention_forward", out, stats, dq_, dk_, dv_, batch, heads, seq, d, ld, scale)
    gq, gk, gv = (hip.DeviceBuffer.from_host(x) for x in old)
    hip.call("nrs_attention_backward", gq, gk, gv, do_, out, dq_, dk_, dv_, stats, batch, heads,
             seq, d, ld, scale, beta)
    o64, dq64, dk64, dv64 = ref_f64(*(heads_view(x, batch, heads, seq, d, ld) for x in (q, k, v, dout)),
                                    float(scale))
    L = max(seq, d)
    o = out.to_host((rows, ld))
    check(heads_view(o, batch, heads, seq, d, ld), o64, L, 1, "out")
    # columns outside the heads are left untouched
    if ld > heads * d:
        assert np.array_equal(o[:, heads * d:], out0[:, heads * d:])
    for buf, g64, o_, what in ((gq, dq64, old[0], "dq"), (gk, dk64, old[1], "dk"),
                               (gv, dv64, old[2], "dv")):
        got = buf.to_host((rows, ld))
        base = heads_view(o_, batch, heads, seq, d, ld).astype(np.float64)
        check(heads_view(got, batch, heads, seq, d, ld), g64 + beta * base, L, 4, what)
        if ld > heads * d:
            assert np.array_equal(got[:, heads * d:], o_[:, heads * d:])
    st = stats.to_host((batch, heads, seq, 2))
    return st, (q, k, v, dout, scale)


@pytest.mark.parametrize("shape", [
    (32, 8, 128, 32, 256),   # cfg4: B32 S128 d256 h8 (d_head 32), in place in the projections
    (3, 2, 128, 16, 32),     # d_head 16
    (2, 3, 100, 32, 101),    # ragged seq, row stride past the heads (untouched columns)
    (4, 1, 17, 32, 32),      # attention_batch on [batch, seq, d] (one head)
    (1, 1, 1, 16, 16),       # a single query and key
    (2, 2, 65, 32, 64),
    # past 128: key tiles streamed with an online softmax, dQ parts summed
    (2, 1, 129, 32, 40),     # one key past the first tile
    (1, 2, 256, 16, 32),     # two whole tiles, d_head 16
    (2, 2, 200, 32, 64),     # ragged second tile
    (1, 1, 300, 32, 32),     # three tiles
    (1, 4, 512, 32, 128),    # four tiles, four heads in place
], ids=lambda s: "b{}h{}s{}d{}ld{}".format(*s))
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_attention_fused_vs_f64(hip, shape, beta):
    run(hip, *shape, beta, seed=sum(shape) + int(beta))


def test_attention_stats_are_softmax_max_and_sum(hip):
    """The saved statistics, the softmax in base 2: the row max of
    u = scale * log2(e) * q.k^T and the sum of 2^(u - max) over the row, per
    (item, head, query)."""
    batch, heads, seq, d, ld = 2, 2, 40, 32, 64
    st, (q, k, _, _, scale) = run(hip, batch, heads, seq, d, ld, 0.0, seed=7)
    qh, kh = (heads_view(x, batch, heads, seq, d, ld).astype(np.float64) for x in (q, k))
    u = np.matmul(qh, kh.transpose(0, 1, 3, 2)) * float(scale) / np.log(2.0)
    m = u.max(axis=-1)
    assert np.abs(st[..., 0] - m).max() <= 1e-5 * (1 + np.abs(m).max())
    tot = np.exp2(u - m[..., None]).sum(axis=-1)
    assert np.abs(st[..., 1] - tot).max() <= 1e-5 * tot.max()


@pytest.mark.parametrize("shape", [(2, 8, 128, 32, 256), (1, 2, 320, 32, 64)],
                         ids=["cfg4_heads", "seq320_tiled"])
def test_attention_matches_oracle_composition(hip, orc, shape):
    """cfg4 heads, the first two batch items (and a tiled sequence of 320):
    the oracle's CPU ops composed as MultiHeadAttention runs them (slice_cols
    per head, transpose(k), bmm, scale, softmax, bmm), forward and backward,
    at the reference's 1e-3."""
    batch, heads, seq, d, ld = shape
    st, (q, k, v, dout, scale) = run(hip, batch, heads, seq, d, ld, 0.0, seed=44)
    out = hip.DeviceBuffer(batch * seq * ld)
    stats = hip.DeviceBuffer(batch * heads * seq * 2)
    dq_, dk_, dv_, do_ = (hip.DeviceBuffer.from_host(x) for x in (q, k, v, dout))
    hip.call("nrs_attention_forward", out, stats, dq_, dk_, dv_, batch, heads, seq, d, ld, scale)
    gq, gk, gv = (hip.DeviceBuffer.zeros(batch * seq * ld) for _ in range(3))
    hip.call("nrs_attention_backward", gq, gk, gv, do_, out, dq_, dk_, dv_, stats, batch, heads,
             seq, d, ld, scale, 0.0)
    o, gqh, gkh, gvh = (x.to_host((batch * seq, ld)) for x in (out, gq, gk, gv))
    rows = batch * seq
    for h in range(heads):
        cols = slice(h * d, (h + 1) * d)
        qh, kh, vh, doh = (np.ascontiguousarray(x[:, cols]) for x in (q, k, v, dout))
        kt = orc.transpose(kh, batch, seq, d).reshape(batch, d, seq)
        sc = orc.graph_bmm_forward(qh.reshape(batch, seq, d), kt)
        w = orc.softmax_forward(orc.scale(sc, scale), seq).reshape(batch, seq, seq)
        oh = orc.graph_bmm_forward(w, vh.reshape(batch, seq, d))
        assert np.abs(o[:, cols] - oh.reshape(rows, d)).max() < 1e-3
        gw, gvv = orc.graph_bmm_backward(w, vh.reshape(batch, seq, d), doh.reshape(batch, seq, d))
        gsm = np.zeros(batch * seq * seq, np.float32)
        orc.softmax_backward(w, gw, gsm, seq)
        gsc = np.zeros(batch * seq * seq, np.float32)
        orc.scale_backward(gsm, gsc, scale)
        gq_, gkt = orc.graph_bmm_backward(qh.reshape(batch, seq, d), kt, gsc.reshape(batch, seq, seq))
        gk_ = np.zeros(rows * d, np.float32)
        orc.transpose_backward(gkt, gk_, batch, seq, d)
        assert np.abs(gqh[:, cols] - gq_.reshape(rows, d)).max() < 1e-3
        assert np.abs(gkh[:, cols] - gk_.reshape(rows, d)).max() < 1e-3
        assert np.abs(gvh[:, cols] - gvv.reshape(rows, d)).max() < 1e-3


def test_attention_unsupported_shapes_refused(hip):
    """Shapes outside the fused path are refused before any launch (the host
    layer composes bmm / softmax / bmm for those)."""
    assert hip.load().nrs_attention_supported(32, 8, 128, 32, 256) == 1
    assert hip.load().nrs_attention_supported(2, 8, 4096, 32, 256) == 1
    for shape in ((1, 1, 16385, 32, 32), (1, 1, 8, 24, 24), (1, 2, 8, 32, 40), (1, 1, 8, 64, 64)):
        assert hip.load().nrs_attention_supported(*shape) == 0
        buf = hip.DeviceBuffer(4096)
        with pytest.raises(hip.NrsError, match="unsupported"):
            hip.call("nrs_attention_forward", buf, buf, buf, buf, buf, *shape, 1.0)


def test_attention_tiled_backward_deterministic_and_needs_out(hip):
    """Past 128 the dQ parts of the key tiles are added in a fixed order: two
    backward calls give the same bits; without the forward output the call
    is refused (its row term dout . out is what lets a key tile work alone)."""
    batch, heads, seq, d, ld = 2, 2, 300, 32, 64
    rng = np.random.default_rng(3)
    q, k, v, dout = (hip.DeviceBuffer.from_host(rng.standard_normal((batch * seq, ld)).astype(np.float32))
                     for _ in range(4))
    out, stats = hip.DeviceBuffer(batch * seq * ld), hip.DeviceBuffer(batch * heads * seq * 2)
    scale = np.float32(1.0 / np.sqrt(d))
    hip.call("nrs_attention_forward", out, stats, q, k, v, batch, heads, seq, d, ld, scale)
    res = []
    for _ in range(2):
        g = [hip.DeviceBuffer.zeros(batch * seq * ld) for _ in range(3)]
        hip.call("nrs_attention_backward", *g, dout, out, q, k, v, stats, batch, heads, seq, d, ld,
                 scale, 0.0)
        res.append([x.to_host() for x in g])
    for a, b in zip(*res):
        assert np.array_equal(a, b)
    g = [hip.DeviceBuffer.zeros(batch * seq * ld) for _ in range(3)]
    with pytest.raises(hip.NrsError, match="forward output"):
        hip.call("nrs_attention_backward", *g, dout, None, q, k, v, stats, batch, heads, seq, d,
                 ld, scale, 0.0)
