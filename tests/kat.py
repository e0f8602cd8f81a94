"""Helpers shared by the tests: golden-fixture loading and the reference's
deterministic input formulas, evaluated in f32 exactly as the Rust tests do."""
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def kats():
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        return json.load(f)


def formula(spec, n):
    """(i % mod) * scale + offset, or ((i % mod) - sub) * scale, in f32."""
    i = (np.arange(n) % spec["mod"]).astype(np.float32)
    if "sub" in spec:
        return ((i - np.float32(spec["sub"])) * np.float32(spec["scale"])).astype(np.float32)
    return (i * np.float32(spec["scale"]) + np.float32(spec["offset"])).astype(np.float32)


def close(gpu, cpu, tol, what):
    """The reference twin tests' absolute-tolerance check (e.g. cuda_manip_test.rs:30-35)."""
    gpu = np.asarray(gpu, np.float32).ravel()
    cpu = np.asarray(cpu, np.float32).ravel()
    assert gpu.shape == cpu.shape, f"{what}: length mismatch {gpu.size} vs {cpu.size}"
    d = np.abs(gpu - cpu)
    i = int(np.argmax(d)) if d.size else 0
    assert d.size == 0 or d[i] < tol, f"{what} [{i}]: gpu {gpu[i]} cpu {cpu[i]} (tol {tol})"


def gemm_tol(inner):
    """Relative tolerance for f32 accumulation over `inner` terms: 1e-5*sqrt(K)."""
    return 1e-5 * np.sqrt(max(int(inner), 1))


def rel_err(c, c64, absprod):
    """max_ij |c - c64| / sum_t |a||b| -- the scale that bounds any summation order."""
    c = np.asarray(c, np.float64)
    den = np.maximum(absprod, np.finfo(np.float32).tiny)
    return float(np.max(np.abs(c - c64) / den)) if c.size else 0.0


def int_matrix(rng, shape, lo=-8, hi=8):
    """Small-integer f32 data: every product and partial sum is exact in f32
    while |sum| < 2**24, so any summation order gives the exact integer result."""
    return rng.integers(lo, hi + 1, size=shape).astype(np.float32)
