"""The runtime part of the C ABI on the device: the caching allocator behind
nrs_malloc / nrs_free (class rounding, reuse, errors, release)."""
import ctypes
import gc

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def stats(hip):
    live, idle = ctypes.c_size_t(), ctypes.c_size_t()
    hip.call("nrs_memory_stats", ctypes.byref(live), ctypes.byref(idle))
    return live.value, idle.value


def raw_malloc(hip, nbytes):
    p = ctypes.c_void_p()
    hip.call("nrs_malloc", ctypes.byref(p), nbytes)
    return p.value


def test_allocator_reuses_blocks_of_a_class(hip):
    # no buffer of another test may be collected (and freed) mid-count
    gc.collect()
    gc.disable()
    try:
        _reuse_checks(hip)
    finally:
        gc.enable()


def _reuse_checks(hip):
    hip.call("nrs_empty_cache")
    live0, idle0 = stats(hip)
    assert idle0 == 0
    a = raw_malloc(hip, 4000)                  # class 4096
    assert stats(hip) == (live0 + 4096, 0)
    hip.call("nrs_free", a)
    assert stats(hip) == (live0, 4096)
    b = raw_malloc(hip, 3585)                  # same class: the cached block
    assert b == a and stats(hip) == (live0 + 4096, 0)
    c = raw_malloc(hip, 4097)                  # next class: a new block
    assert c != a
    big = raw_malloc(hip, (3 << 20) + 1)       # 2 MiB steps above 1 MiB: 4 MiB
    assert stats(hip)[0] == live0 + 4096 + 4608 + (4 << 20)
    for p in (b, c, big):
        hip.call("nrs_free", p)
    hip.call("nrs_empty_cache")
    assert stats(hip) == (live0, 0)


def test_allocator_rejects_double_and_foreign_free(hip):
    p = raw_malloc(hip, 100)
    hip.call("nrs_free", p)
    with pytest.raises(hip.NrsError):
        hip.call("nrs_free", p)                # already freed
    q = raw_malloc(hip, 100)
    with pytest.raises(hip.NrsError):
        hip.call("nrs_free", q + 256)          # not the start of a buffer
    hip.call("nrs_free", q)
    hip.call("nrs_free", None)                 # null is a no-op


def test_reused_block_is_ordered_after_queued_reads(hip):
    """A block freed while a queued launch still reads it, then handed out
    again and overwritten: the launch sees the old contents."""
    n = 1 << 20
    x = hip.DeviceBuffer.from_host(np.full(n, 3.0, np.float32))
    y = hip.DeviceBuffer(n)
    old = x.ptr
    hip.call("nrs_scale", y.ptr, x.ptr, 2.0, n, 0.0)
    x.free()
    z = hip.DeviceBuffer.from_host(np.full(n, -1.0, np.float32))
    assert z.ptr == old                        # the same block, reused
    assert np.array_equal(y.to_host(), np.full(n, 6.0, np.float32))
    assert np.array_equal(z.to_host(), np.full(n, -1.0, np.float32))


def _hip_runtime():
    """The HIP runtime libnrs_hip.so is linked against (already mapped into
    this process once the library is loaded)."""
    with open("/proc/self/maps") as f:
        paths = {ln.split()[-1] for ln in f if "libamdhip64.so" in ln}
    assert paths, "libamdhip64 is not loaded"
    return ctypes.CDLL(sorted(paths)[0])


def _hip_stream():
    """A new HIP stream at the default priority, as an integer handle."""
    s = ctypes.c_void_p()
    assert _hip_runtime().hipStreamCreate(ctypes.byref(s)) == 0
    return s.value


def _int_host(rng, shape, lo=-3, hi=3):
    return rng.integers(lo, hi + 1, size=shape).astype(np.float32)


def test_stream_switch_orders_reuse_after_old_stream(hip):
    """nrs_set_stream drains the old stream: a block freed while a long GEMM
    on stream A still reads it, re-allocated and overwritten on stream B,
    and split-K GEMMs on either stream (sharing, and growing, the library's
    partials scratch) all give the results of serial execution."""
    rng = np.random.default_rng(17)
    n = 4096
    xa, xb = _int_host(rng, (n, n)), _int_host(rng, (n, n))
    want = (xa.astype(np.float64) @ xb.astype(np.float64)).astype(np.float32)
    sa, sb = _hip_stream(), _hip_stream()
    prev = hip.load().nrs_get_stream()
    try:
        dx, dy = hip.DeviceBuffer.from_host(xa), hip.DeviceBuffer.from_host(xb)
        dc = hip.DeviceBuffer(n * n)
        hip.call("nrs_set_stream", sa)
        hip.gemm(hip.NN, dc, dx, dy, n, n, n)       # ~1 ms reading dx on stream A
        hip.call("nrs_set_stream", sb)
        old = dx.ptr
        dx.free()
        dz = hip.DeviceBuffer(n * n)
        assert dz.ptr == old                         # the same block, on stream B
        ones = np.full(n * n, -1.0, np.float32)
        hip.call("nrs_memcpy_htod", dz.ptr, ones.ctypes.data, ones.nbytes)
        hip.sync()
        assert np.array_equal(dc.to_host((n, n)), want)

        # split-K partials: a small plan on A, then a larger one on B (scratch grows)
        shapes = ((32, 9, 100352), (64, 576, 100352))
        outs = []
        for shape, s in zip(shapes, (sa, sb)):
            rows, cols, inner = shape
            a, b = _int_host(rng, (rows, inner), -2, 2), _int_host(rng, (cols, inner), -2, 2)
            hip.call("nrs_set_stream", s)
            da, db = hip.DeviceBuffer.from_host(a), hip.DeviceBuffer.from_host(b)
            c = hip.DeviceBuffer(rows * cols)
            hip.gemm_nt_splitk(c, da, db, rows, cols, inner, 0.0)
            outs.append((c, da, db, (a.astype(np.float64) @ b.astype(np.float64).T)))
        hip.sync()
        for (c, _, _, w), (rows, cols, _) in zip(outs, shapes):
            assert np.array_equal(c.to_host((rows, cols)), w.astype(np.float32))
    finally:
        hip.call("nrs_set_stream", prev)
        for s in (sa, sb):
            _hip_runtime().hipStreamDestroy(ctypes.c_void_p(s))


@pytest.mark.parametrize("nbytes,src_off,dst_off", [(16, 0, 0), (4096 * 256 * 4, 0, 0),
                                                    (1000 * 4, 0, 0), (36, 4, 0), (64, 0, 8),
                                                    (7, 1, 3)])
def test_memcpy_dtod_aligned_and_ragged(hip, nbytes, src_off, dst_off):
    """nrs_memcpy_dtod copies exactly `bytes` bytes: the 16-byte copy kernel
    for aligned whole units, the runtime copy otherwise; bytes around the
    destination range stay untouched."""
    rng = np.random.default_rng(nbytes + src_off)
    src = rng.integers(0, 256, nbytes + 64, dtype=np.uint8)
    dst0 = rng.integers(0, 256, nbytes + 64, dtype=np.uint8)
    dsrc = hip.DeviceBuffer.from_host(src.view(np.float32) if src.size % 4 == 0 else
                                      np.pad(src, (0, (-src.size) % 4)).view(np.float32))
    ddst = hip.DeviceBuffer.from_host(dst0.view(np.float32) if dst0.size % 4 == 0 else
                                      np.pad(dst0, (0, (-dst0.size) % 4)).view(np.float32))
    hip.call("nrs_memcpy_dtod", ddst.ptr + dst_off, dsrc.ptr + src_off, nbytes)
    got = ddst.to_host().view(np.uint8)[: dst0.size]
    want = dst0.copy()
    want[dst_off:dst_off + nbytes] = src[src_off:src_off + nbytes]
    assert np.array_equal(got, want)
