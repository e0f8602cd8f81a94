#!/usr/bin/env python3
"""Benchmark of the MI355X f32 matrix-multiply backend (one GPU).

Headline metric: f32 GEMM TFLOP/s and % of MI355X FP32 MFMA
peak; conv2d fwd+bwd imgs/s.

  * step      = one f32 GEMM C[4096,4096] = A[4096,4096] . B[4096,4096]
                (cfg5, NN, A,B ~ U(-1,1) seeded), inputs resident in HBM;
  * value     = TFLOP/s over the K timed steps (2*M*N*K per step);
  * roofline  = the GEMM kernel's average duration from HIP events recorded
                on the library stream around the timed steps;
  * conv2d    = cfg3 (batch 128: conv1 1->32 3x3 p1, maxpool 2x2, conv2
                32->64 3x3 p1, forward + backward incl. input grads and
                split-K weight grads) in imgs/s, as the metric's second half;
  * cpu_baseline = the reference's CPU path (C restatement of
                ops::simd::matmul_simd, AVX2 + all host threads) timed on a
                bounded row sample of the same GEMM.

Prints ONE JSON line.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA_TFLOPS = 157.3   # MI355X dense FP32 matrix peak
PEAK_HBM_GBS = 8000.0           # MI355X HBM3E


class HipEvents:
    """hipEvent timing on the library stream (the null stream by default)."""

    def __init__(self, stream):
        self.rt = ctypes.CDLL("libamdhip64.so")
        self.stream = ctypes.c_void_p(stream)
        for n in ("hipEventCreate", "hipEventRecord", "hipEventSynchronize",
                  "hipEventElapsedTime", "hipEventDestroy"):
            getattr(self.rt, n).restype = ctypes.c_int

    def event(self):
        e = ctypes.c_void_p()
        assert self.rt.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def record(self, e):
        assert self.rt.hipEventRecord(e, self.stream) == 0

    def elapsed_ms(self, a, b):
        assert self.rt.hipEventSynchronize(b) == 0
        ms = ctypes.c_float()
        assert self.rt.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value


def bench_gemm(hip, n, steps, warmup):
    rng = np.random.default_rng(0)
    a = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    dA, dB = hip.DeviceBuffer.from_host(a), hip.DeviceBuffer.from_host(b)
    dC = hip.DeviceBuffer(n * n)
    for _ in range(warmup):
        hip.gemm(hip.NN, dC, dA, dB, n, n, n)
    hip.sync()
    ev = HipEvents(hip.load().nrs_get_stream())
    e0, e1 = ev.event(), ev.event()
    t0 = time.perf_counter()
    ev.record(e0)
    for _ in range(steps):
        hip.gemm(hip.NN, dC, dA, dB, n, n, n)
    ev.record(e1)
    hip.sync()
    wall = time.perf_counter() - t0
    kernel_ms = ev.elapsed_ms(e0, e1) / steps
    # spot-check the result of the timed launches against f64 on a few rows
    import oracle
    c = dC.to_host((n, n))
    rows = np.arange(0, n, max(1, n // 8))
    c64, ab = oracle.gemm_f64("nn", a, b, n, n, n, rowidx=rows)
    err = float(np.max(np.abs(c[rows] - c64) / np.maximum(ab, 1e-30)))
    return {"wall_ms_per_step": wall * 1e3 / steps, "kernel_ms": kernel_ms, "rel_err": err,
            "a": a, "b": b}


def bench_conv_cfg3(hip, steps, warmup):
    """cfg3 step: conv1 -> maxpool -> conv2, forward + backward (all grads)."""
    rng = np.random.default_rng(3)
    N, H, W = 128, 28, 28
    x = rng.uniform(0, 1, N * 1 * H * W).astype(np.float32)
    w1 = (rng.standard_normal(32 * 1 * 9) * np.sqrt(2.0 / 9)).astype(np.float32)
    w2 = (rng.standard_normal(64 * 32 * 9) * np.sqrt(2.0 / 288)).astype(np.float32)
    b1, b2 = np.zeros(32, np.float32), np.zeros(64, np.float32)
    g2 = rng.standard_normal(N * 64 * 14 * 14).astype(np.float32)
    D = hip.DeviceBuffer.from_host
    dx, dw1, dw2, db1, db2, dg2 = D(x), D(w1), D(w2), D(b1), D(b2), D(g2)
    y1 = hip.DeviceBuffer(N * 32 * 28 * 28)
    p1 = hip.DeviceBuffer(N * 32 * 14 * 14)
    am = hip.DeviceBuffer(N * 32 * 14 * 14, np.int32)
    y2 = hip.DeviceBuffer(N * 64 * 14 * 14)
    gx = hip.DeviceBuffer.zeros(x.size)
    gp1 = hip.DeviceBuffer.zeros(N * 32 * 14 * 14)
    gy1 = hip.DeviceBuffer.zeros(N * 32 * 28 * 28)
    gw1, gw2 = hip.DeviceBuffer.zeros(w1.size), hip.DeviceBuffer.zeros(w2.size)
    gb1, gb2 = hip.DeviceBuffer.zeros(32), hip.DeviceBuffer.zeros(64)

    def step():
        hip.call("nrs_conv2d_forward", y1.ptr, dx.ptr, dw1.ptr, db1.ptr, N, 1, 28, 28, 32, 3, 3, 1, 1)
        hip.call("nrs_maxpool_forward", p1.ptr, am.ptr, y1.ptr, N, 32, 28, 28, 2, 2)
        hip.call("nrs_conv2d_forward", y2.ptr, p1.ptr, dw2.ptr, db2.ptr, N, 32, 14, 14, 64, 3, 3, 1, 1)
        # backward (zero_grad of the activation grads, then accumulate)
        hip.call("nrs_memset_zero", gp1.ptr, gp1.nbytes)
        hip.call("nrs_memset_zero", gy1.ptr, gy1.nbytes)
        hip.call("nrs_conv2d_backward", gp1.ptr, gw2.ptr, gb2.ptr, dg2.ptr, p1.ptr, dw2.ptr,
                 N, 32, 14, 14, 64, 3, 3, 1, 1)
        hip.call("nrs_maxpool_backward", gy1.ptr, gp1.ptr, am.ptr, N, 32, 28, 28, 2, 2)
        hip.call("nrs_conv2d_backward", gx.ptr, gw1.ptr, gb1.ptr, gy1.ptr, dx.ptr, dw1.ptr,
                 N, 1, 28, 28, 32, 3, 3, 1, 1)

    for _ in range(warmup):
        step()
    hip.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    hip.sync()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    return {"ms_per_step": ms, "imgs_per_s": N / (ms / 1e3)}


def cpu_baseline_gemm(a, b, target_s=10.0):
    """oracle matmul_simd (AVX2, all host threads) on a row sample of a.b."""
    import oracle
    threads = oracle.max_threads()
    n = a.shape[0]
    # Calibrate on growing row counts until one run takes >= 1 s, so thread
    # start-up does not dominate the estimate, then time ~target_s of work.
    rows = threads
    while True:
        t0 = time.perf_counter()
        oracle.matmul_simd_rows(a, b, 0, rows)
        dt = time.perf_counter() - t0
        if dt >= 1.0 or rows >= n:
            break
        rows = min(n, rows * 4)
    if dt < target_s and rows < n:
        rows = int(min(n, rows * target_s / max(dt, 1e-6)))
        rows = min(n, max(threads, (rows // threads) * threads))
        t0 = time.perf_counter()
        oracle.matmul_simd_rows(a, b, 0, rows)
        dt = time.perf_counter() - t0
    # The whole GEMM finishes well inside target_s: repeat it.
    reps = 1
    if rows >= n and dt < target_s:
        reps = max(1, int(target_s / max(dt, 1e-6)))
        t0 = time.perf_counter()
        for _ in range(reps):
            oracle.matmul_simd_rows(a, b, 0, rows)
        dt = time.perf_counter() - t0
    flops = 2.0 * rows * b.shape[1] * a.shape[1] * reps
    what = f"rows 0..{rows}" if rows < n else f"{reps} full runs"
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{what} of the {n}^3 GEMM via the C restatement of matmul_simd "
                      f"(src/ops/simd.rs:42-77, AVX2, B transposed per call as the reference "
                      f"does), {dt:.1f} s"}


COPY_BYTES = 256 << 20


def profile_pass(hip, n, steps):
    """Launch sequence profiled with rocprofv3 --pmc: one device-to-device
    copy of COPY_BYTES (a plain copy kernel whose traffic is known: it reads
    and writes COPY_BYTES once), then `steps` NN GEMMs of size n^3."""
    src = hip.DeviceBuffer.zeros(COPY_BYTES // 4)
    dst = hip.DeviceBuffer(COPY_BYTES // 4)
    hip.call("nrs_memcpy_dtod", dst.ptr, src.ptr, COPY_BYTES)
    hip.sync()
    rng = np.random.default_rng(0)
    a = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    dA, dB = hip.DeviceBuffer.from_host(a), hip.DeviceBuffer.from_host(a.T.copy())
    dC = hip.DeviceBuffer(n * n)
    for _ in range(max(1, steps)):
        hip.gemm(hip.NN, dC, dA, dB, n, n, n)
    hip.sync()


def measured_traffic(n):
    """HBM bytes per launch of the n^3 GEMM from the committed counter
    summary (profiles/gemm_nn_4096_traffic.md), or None."""
    path = os.path.join(ROOT, "profiles", "gemm_nn_4096_traffic.md")
    if n != 4096 or not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.strip().startswith("hbm_bytes_per_launch ="):
                return int(float(line.split("=", 1)[1].strip().split()[0]))
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--size", type=int, default=4096)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-conv", action="store_true", help="skip the conv2d leg")
    ap.add_argument("--profile-pass", action="store_true",
                    help="only launch a 256 MiB device copy (counter calibration) and then "
                         "--steps GEMMs, for rocprofv3 --pmc runs; prints nothing else")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the reference has no multi-GPU path and none is built here.", file=sys.stderr)
        sys.exit(2)

    from neuralrs_amd import _abi as hip
    hip.load()
    hip.init(0)
    n = args.size
    if args.profile_pass:
        profile_pass(hip, n, args.steps)
        return
    g = bench_gemm(hip, n, args.steps, args.warmup)
    flops = 2.0 * n * n * n
    value = flops / (g["wall_ms_per_step"] / 1e3) / 1e12
    achieved = flops / (g["kernel_ms"] / 1e3) / 1e12
    traffic = measured_traffic(n)
    out = {
        "metric": "f32 GEMM TFLOP/s + % of MI355X FP32 MFMA peak; conv2d fwd+bwd imgs/sec",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["wall_ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"cfg5 f32 GEMM NN M=N=K={n}, A,B~U(-1,1) seed 0, row-major, "
                               "inputs resident in HBM", "M": n, "N": n, "K": n},
        "pct_fp32_mfma_peak": round(100.0 * value / PEAK_FP32_MFMA_TFLOPS, 2),
        "max_rel_err_vs_f64": g["rel_err"],
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3),
                     "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4), "traffic": traffic,
                     "kernel": "gemm_kernel<256,256,16,2,NN,vec4>",
                     "kernel_ms": round(g["kernel_ms"], 4)},
    }
    if not args.no_conv:
        c = bench_conv_cfg3(hip, max(5, args.steps // 2), args.warmup)
        out["conv2d_fwd_bwd"] = {"value": round(c["imgs_per_s"], 1), "unit": "imgs/s",
                                 "ms_per_step": round(c["ms_per_step"], 4),
                                 "config": "cfg3 batch 128 conv1 1->32, maxpool, conv2 32->64, "
                                           "fwd+bwd with input and weight grads"}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_gemm(g["a"], g["b"])
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
