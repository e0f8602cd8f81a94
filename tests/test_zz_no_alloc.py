"""nrs_gemm_nt_splitk_noalloc: the split-K weight-gradient GEMM with its
partials in the library's fixed per-GPU scratch array instead of allocated
scratch. It runs the same plan and kernels as nrs_gemm_nt_splitk, so its
results must be bit-identical to it, on consecutive calls that share the
array (the second smaller than the first, so stale partials of the first
would show), and plans whose partials exceed the array are refused."""
import numpy as np
import pytest

from kat import int_matrix

pytestmark = pytest.mark.gpu


def _pair(hip, rows, cols, inner, beta, seed):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((rows, inner)).astype(np.float32)
    b = rng.uniform(-1, 1, (cols, inner)).astype(np.float32)
    c0 = rng.standard_normal((rows, cols)).astype(np.float32)
    dA, dB = hip.DeviceBuffer.from_host(a), hip.DeviceBuffer.from_host(b)
    want = hip.DeviceBuffer.from_host(c0)
    got = hip.DeviceBuffer.from_host(c0)
    hip.gemm_nt_splitk(want, dA, dB, rows, cols, inner, beta)
    hip.call("nrs_gemm_nt_splitk_noalloc", got, dA, dB, rows, cols, inner, beta)
    return got.to_host((rows, cols)), want.to_host((rows, cols))


def test_noalloc_matches_splitk_two_calls(hip):
    # cfg3 conv2 weight gradient (64 x 288 over 25088: 154 slices, 11.4 MB of
    # partials), then the smaller conv1 one (32 x 9 over 100352: 256 slices)
    for shape, beta, seed in (((64, 288, 25088), 1.0, 1), ((32, 9, 100352), 0.0, 2)):
        print(f"noalloc split-K {shape} beta {beta}", flush=True)
        got, want = _pair(hip, *shape, beta, seed)
        assert np.array_equal(got, want), shape


def test_noalloc_cfg5_wgrad_and_unsplit(hip):
    # the largest plan of the BASELINE shapes (64 x 576 over 100352, 12.7 MB
    # of partials), then a plan without split (the scratch is not touched)
    for shape in ((64, 576, 100352), (300, 300, 64)):
        print(f"noalloc split-K {shape}", flush=True)
        got, want = _pair(hip, *shape, 0.5, 3)
        assert np.array_equal(got, want), shape


def test_noalloc_exact_integers(hip):
    rng = np.random.default_rng(5)
    rows, cols, inner = 64, 320, 20000
    a = int_matrix(rng, (rows, inner), -2, 2)
    b = int_matrix(rng, (cols, inner), -2, 2)
    dA, dB = hip.DeviceBuffer.from_host(a), hip.DeviceBuffer.from_host(b)
    dC = hip.DeviceBuffer(rows * cols)
    hip.call("nrs_gemm_nt_splitk_noalloc", dC, dA, dB, rows, cols, inner, 0.0)
    want = (a.astype(np.float64) @ b.astype(np.float64).T).astype(np.float32)
    assert np.array_equal(dC.to_host((rows, cols)), want)


def test_noalloc_refuses_oversized_partials(hip):
    # 960 x 1088 over 4096: 255 tiles of 64 x 64, 4 slices, 16.7 MB of
    # partials > 14 MiB; refused before any launch, and C is left untouched
    rows, cols, inner = 960, 1088, 4096
    dA, dB = hip.DeviceBuffer.zeros(rows * inner), hip.DeviceBuffer.zeros(cols * inner)
    c0 = np.full((rows, cols), 3.0, np.float32)
    dC = hip.DeviceBuffer.from_host(c0)
    with pytest.raises(hip.NrsError, match="exceed"):
        hip.call("nrs_gemm_nt_splitk_noalloc", dC, dA, dB, rows, cols, inner, 0.0)
    assert np.array_equal(dC.to_host((rows, cols)), c0)
