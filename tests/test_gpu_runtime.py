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
