#!/usr/bin/env python3
"""Benchmark of the MI355X f32 matrix-multiply backend (one GPU).

Headline metric: f32 GEMM TFLOP/s and % of MI355X FP32 MFMA
peak; conv2d fwd+bwd imgs/s.

  * step      = one f32 GEMM C[4096,4096] = A[4096,4096] . B[4096,4096]
                (cfg5, NN, A,B ~ U(-1,1) seeded), inputs resident in HBM;
  * value     = TFLOP/s over the K timed steps (2*M*N*K per step);
  * roofline  = the GEMM kernel's average duration from HIP events recorded
                on the library stream around the timed steps;
  * conv2d    = cfg3 (batch 128: conv1 1->32 3x3 p1, ReLU, maxpool 2x2,
                conv2 32->64 3x3 p1, forward + backward incl. input grads and
                split-K weight grads) in imgs/s, as the metric's second half,
                timed from C++ through the operator surface (bench_host cnn);
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


def event_ms(hip, fn, reps, warmup):
    """Average GPU time of fn() in ms: HIP events on the library stream
    around `reps` calls after `warmup` untimed calls."""
    for _ in range(warmup):
        fn()
    hip.sync()
    ev = HipEvents(hip.load().nrs_get_stream())
    e0, e1 = ev.event(), ev.event()
    ev.record(e0)
    for _ in range(reps):
        fn()
    ev.record(e1)
    return ev.elapsed_ms(e0, e1) / reps


def leg_ms(hip, fn, reps, warmup, rounds=3):
    """A short leg's GPU time in ms: the median of `rounds` event_ms batches
    (one batch of a few-microsecond leg swings by a microsecond between runs)."""
    return float(np.median([event_ms(hip, fn, reps, warmup) for _ in range(rounds)]))


def roofline_us(flops, nbytes):
    """max(FLOP / FP32 MFMA peak, bytes / HBM bandwidth) in microseconds."""
    return max(flops / (PEAK_FP32_MFMA_TFLOPS * 1e12), nbytes / (PEAK_HBM_GBS * 1e9)) * 1e6


def gemm_roof(m, n, k, batch=1):
    """(flops, algorithmic bytes) of C[m,n] = A[m,k] . B[k,n]: each operand
    read once, C written once, f32."""
    return 2.0 * m * n * k * batch, 4.0 * (m * k + k * n + m * n) * batch


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


def bench_conv_cfg3(hip, steps, warmup, closures_only=False):
    """cfg3 step: conv1 -> ReLU -> maxpool -> conv2 (the reference CNN's
    maxpool2d(relu(conv2d(..))), examples/mnist_cuda_cnn.rs:125), forward +
    backward: weight and bias gradients of both layers, input gradient of
    conv2. conv1's input is the image batch, which requires no gradient in
    the reference's training step (examples/mnist_cuda_cnn.rs:261 sets
    requires_grad = false, and src/cuda/nn/conv.rs:304 then skips the input
    gradient); that kernel is timed on its own and reported beside the step.
    The step here issues the C ABI from Python; the same step through the
    C++ operator surface is bench_host cnn (host_step)."""
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

    a1 = hip.DeviceBuffer(N * 32 * 28 * 28)
    ga1 = hip.DeviceBuffer.zeros(N * 32 * 28 * 28)

    # conv1 -> ReLU -> maxpool as one node each way: conv1's output only
    # feeds the pooling, so the fused forward never writes it and the fused
    # backward expands the pooled gradient while loading, gated by the pooled
    # value's sign (nrs_conv2d_relu_maxpool_forward), and conv2's backward
    # gives conv1's weight and bias gradients in its own launch from the
    # pooled gradient it computes (nrs_conv2d_maxpool_relu_conv2d_backward).
    # Gradients are written, not added (beta 0): a training step zeroes them
    # first (zero_grad), and this is that zeroing and the first accumulation
    # in one. The op-by-op sequence, with its zeroing launches, is
    # step_unfused.
    def step():
        hip.call("nrs_conv2d_relu_maxpool_forward", p1.ptr, am.ptr, None, dx.ptr, dw1.ptr,
                 db1.ptr, N, 1, 28, 28, 32, 3, 3, 1, 1, 2, 2)
        hip.call("nrs_conv2d_forward", y2.ptr, p1.ptr, dw2.ptr, db2.ptr, N, 32, 14, 14, 64, 3, 3, 1, 1)
        hip.call("nrs_conv2d_maxpool_relu_conv2d_backward", gp1.ptr, gw2.ptr, gb2.ptr, gw1.ptr,
                 gb1.ptr, dg2.ptr, p1.ptr, dw2.ptr, am.ptr, dx.ptr, dw1.ptr, N, 1, 28, 28, 32,
                 3, 3, 1, 1, 2, 2, 64, 3, 3, 1, 1, 0.0)

    def step_unfused():
        for buf in (gw1, gb1, gw2, gb2):
            hip.call("nrs_memset_zero", buf.ptr, buf.nbytes)
        hip.call("nrs_conv2d_forward", y1.ptr, dx.ptr, dw1.ptr, db1.ptr, N, 1, 28, 28, 32, 3, 3, 1, 1)
        hip.call("nrs_relu_forward", a1.ptr, y1.ptr, a1.n)
        hip.call("nrs_maxpool_forward", p1.ptr, am.ptr, a1.ptr, N, 32, 28, 28, 2, 2)
        hip.call("nrs_conv2d_forward", y2.ptr, p1.ptr, dw2.ptr, db2.ptr, N, 32, 14, 14, 64, 3, 3, 1, 1)
        hip.call("nrs_memset_zero", gp1.ptr, gp1.nbytes)
        hip.call("nrs_memset_zero", ga1.ptr, ga1.nbytes)
        hip.call("nrs_conv2d_backward", gp1.ptr, gw2.ptr, gb2.ptr, dg2.ptr, p1.ptr, dw2.ptr,
                 N, 32, 14, 14, 64, 3, 3, 1, 1)
        hip.call("nrs_maxpool_backward", ga1.ptr, gp1.ptr, am.ptr, N, 32, 28, 28, 2, 2)
        hip.call("nrs_relu_backward", gy1.ptr, ga1.ptr, y1.ptr, gy1.n, 0.0)
        hip.call("nrs_conv2d_backward", None, gw1.ptr, gb1.ptr, gy1.ptr, dx.ptr, dw1.ptr,
                 N, 1, 28, 28, 32, 3, 3, 1, 1)

    def conv_fwd():
        hip.call("nrs_conv2d_forward", y1.ptr, dx.ptr, dw1.ptr, db1.ptr, N, 1, 28, 28, 32, 3, 3, 1, 1)
        hip.call("nrs_conv2d_forward", y2.ptr, p1.ptr, dw2.ptr, db2.ptr, N, 32, 14, 14, 64, 3, 3, 1, 1)

    def conv_bwd():
        hip.call("nrs_conv2d_backward", gp1.ptr, gw2.ptr, gb2.ptr, dg2.ptr, p1.ptr, dw2.ptr,
                 N, 32, 14, 14, 64, 3, 3, 1, 1)
        hip.call("nrs_conv2d_backward", None, gw1.ptr, gb1.ptr, gy1.ptr, dx.ptr, dw1.ptr,
                 N, 1, 28, 28, 32, 3, 3, 1, 1)

    def conv1_input_grad():
        hip.call("nrs_conv2d_backward", gx.ptr, None, None, gy1.ptr, dx.ptr, dw1.ptr,
                 N, 1, 28, 28, 32, 3, 3, 1, 1)

    def conv1_pool_fwd():
        hip.call("nrs_conv2d_relu_maxpool_forward", p1.ptr, am.ptr, None, dx.ptr, dw1.ptr,
                 db1.ptr, N, 1, 28, 28, 32, 3, 3, 1, 1, 2, 2)

    def conv1_pool_bwd():
        hip.call("nrs_maxpool_relu_conv2d_backward", None, gw1.ptr, gb1.ptr, gp1.ptr, am.ptr,
                 p1.ptr, dx.ptr, dw1.ptr, N, 1, 28, 28, 32, 3, 3, 1, 1, 2, 2, 1.0)

    if closures_only:
        return {"conv_fwd_cfg3": conv_fwd, "conv_bwd_cfg3": conv_bwd,
                "conv1_input_grad_cfg3": conv1_input_grad,
                "conv1_maxpool_fwd_cfg3": conv1_pool_fwd, "maxpool_conv1_bwd_cfg3": conv1_pool_bwd}

    def wall_ms(fn):
        for _ in range(warmup):
            fn()
        hip.sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        hip.sync()
        return (time.perf_counter() - t0) * 1e3 / steps

    ms_unfused = wall_ms(step_unfused)
    ms = wall_ms(step)
    fwd_ms = leg_ms(hip, conv_fwd, steps, 3)
    bwd_ms = leg_ms(hip, conv_bwd, steps, 3)
    dx1_ms = leg_ms(hip, conv1_input_grad, steps, 3)
    # rooflines per layer (implicit-GEMM FLOPs; bytes = each tensor read or
    # written once): forward x, W, b, y; input grad g, W, dx; weight+bias
    # grad g, x, dW, db
    roof_f = roof_b = roof_dx1 = 0.0
    for (ci, co, h) in ((1, 32, 28), (32, 64, 14)):
        P, taps = h * h, ci * 9
        fl = 2.0 * co * N * P * taps
        x_b, y_b, w_b = 4.0 * N * ci * P, 4.0 * N * co * P, 4.0 * co * taps
        roof_f += roofline_us(fl, x_b + w_b + 4 * co + y_b)
        dx_roof = roofline_us(fl, y_b + w_b + x_b)
        if ci == 1:
            roof_dx1 = dx_roof  # the image batch's gradient: not part of the step
        else:
            roof_b += dx_roof
        roof_b += roofline_us(fl, y_b + x_b + w_b + 4 * co)
    return {"ms_per_step": ms, "imgs_per_s": N / (ms / 1e3), "ms_per_step_unfused": ms_unfused,
            "conv1_pool_fwd_us": leg_ms(hip, conv1_pool_fwd, steps, 3) * 1e3,
            "pool_conv1_bwd_us": leg_ms(hip, conv1_pool_bwd, steps, 3) * 1e3,
            "fwd_us": fwd_ms * 1e3, "bwd_us": bwd_ms * 1e3,
            "fwd_roof_us": roof_f, "bwd_roof_us": roof_b,
            "conv1_input_grad_us": dx1_ms * 1e3, "conv1_input_grad_roof_us": roof_dx1}


def bench_mlp_cfg2(hip, steps, warmup, closures_only=False):
    """cfg2 training step: x[256,784] -> Linear(784,128) -> ReLU ->
    Linear(128,10) -> cross-entropy seed (softmax - onehot)/256 (the fused
    ce_backward of src/cuda/loss/cross_entropy.rs:39-58) -> backward (dW, db
    of both layers, dh, dx), in two library calls of one launch each:
    nrs_mlp2_forward_seed (both layers forward, the seed, and the hidden
    layer's gradient through the ReLU: all row-local) and nrs_mlp2_backward
    (dW1, db1, dW2, db2 and dx as one short-GEMM launch). The four-call form
    (nrs_gemm with bias and ReLU, nrs_linear_cross_entropy,
    nrs_linear_backward_relu, nrs_linear_backward) is timed beside it. Issued
    from Python here; the same steps issued from C++ (eagerly and as a HIP
    graph) are host_step()."""
    rng = np.random.default_rng(2)
    B, I, Hd, O = 256, 784, 128, 10
    D = hip.DeviceBuffer.from_host
    x = D(rng.standard_normal(B * I).astype(np.float32))
    w1 = D((rng.standard_normal(I * Hd) * np.sqrt(2.0 / I)).astype(np.float32))
    w2 = D((rng.standard_normal(Hd * O) * np.sqrt(2.0 / Hd)).astype(np.float32))
    b1, b2 = hip.DeviceBuffer.zeros(Hd), hip.DeviceBuffer.zeros(O)
    t = np.zeros((B, O), np.float32)
    t[np.arange(B), rng.integers(0, O, B)] = 1.0
    onehot = D(t)
    a, z, gz = hip.DeviceBuffer(B * Hd), hip.DeviceBuffer(B * O), hip.DeviceBuffer(B * O)
    gh, gx = hip.DeviceBuffer(B * Hd), hip.DeviceBuffer(B * I)
    gw1, gw2 = hip.DeviceBuffer.zeros(I * Hd), hip.DeviceBuffer.zeros(Hd * O)
    gb1, gb2 = hip.DeviceBuffer.zeros(Hd), hip.DeviceBuffer.zeros(O)

    def step():
        hip.call("nrs_mlp2_forward_seed", a, z, gz, gh, x, w1, b1, w2, b2, onehot, B, I, Hd, O)
        hip.call("nrs_mlp2_backward", gx, gw1, gb1, gw2, gb2, gh, gz, x, w1, a, B, I, Hd, O,
                 0.0, 1.0)

    def step_four_calls():
        hip.gemm(hip.NN, a, x, w1, B, Hd, I, 0.0, b1, hip.EPI_BIAS_COL | hip.EPI_RELU)
        hip.call("nrs_linear_cross_entropy", z, gz, a, w2, b2, onehot, B, Hd, O)
        hip.call("nrs_linear_backward_relu", gh, gw2, gb2, gz, a, w2, a, B, Hd, O, 0.0, 1.0, 1.0)
        hip.call("nrs_linear_backward", gx, gw1, gb1, gh, x, w1, B, I, Hd, 0.0, 1.0, 1.0)

    if closures_only:
        return {"mlp_step_cfg2": step}
    us = event_ms(hip, step, steps, warmup) * 1e3
    us4 = event_ms(hip, step_four_calls, steps, warmup) * 1e3
    return {"us_per_step": us, "us_per_step_four_calls": us4, "gemm_roof_us": mlp_gemm_roof_us()}


def mlp_gemm_roof_us():
    """Roofline time of cfg2's six GEMMs (each max(FLOP, bytes) bound)."""
    B, I, Hd, O = 256, 784, 128, 10
    roof = 0.0
    for (m, n, k) in ((B, Hd, I), (B, O, Hd), (Hd, O, B), (B, Hd, O), (I, Hd, B), (B, I, Hd)):
        roof += roofline_us(*gemm_roof(m, n, k))
    return roof


def host_step(kind, steps, warmup):
    """Runs neuralrs_amd/bench_host (C++, no Python between launches) for
    `kind` ("mlp": the cfg2 step through the C ABI, eager and replayed as a
    HIP graph; "block": the cfg4 TransformerBlock forward + backward through
    the C++ operator surface; "cnn": the cfg3 step through the operator
    surface) in a child process and returns its JSON, or None when the
    binary is missing or fails."""
    import subprocess
    exe = os.path.join(ROOT, "neuralrs_amd", "bench_host")
    if not os.path.exists(exe):
        return None
    try:
        proc = subprocess.run([exe, kind, str(steps), str(warmup)], capture_output=True,
                              text=True, timeout=300)
    except subprocess.TimeoutExpired:
        return None
    if proc.returncode != 0:
        return None
    for line in reversed(proc.stdout.splitlines()):
        if line.startswith("{"):
            return json.loads(line)
    return None


def bench_attention_cfg4(hip, steps, warmup, closures_only=False):
    """cfg4 attention core as one batched call over batch*heads = 256:
    S = Q.K^T / sqrt(32), P = softmax(S), O = P.V, then the backward bmm
    products dP = dO.V^T, dV = P^T.dO, dS = softmax'(P, dP)/sqrt(32),
    dQ = dS.K, dK = dS^T.Q (fresh outputs; each bmm's two gradients in one
    nrs_bmm_backward call). Plus the block's Linear GEMMs
    (Q/K/V/O projections 4096x256x256 and FFN 256->1024->256, forward and
    both backward products)."""
    rng = np.random.default_rng(4)
    BH, T, Dh = 256, 128, 32
    D = hip.DeviceBuffer.from_host
    q, k, v, do = (D(rng.standard_normal(BH * T * Dh).astype(np.float32)) for _ in range(4))
    S, P, dP, dS = (hip.DeviceBuffer(BH * T * T) for _ in range(4))
    o, dq, dk, dv = (hip.DeviceBuffer(BH * T * Dh) for _ in range(4))
    sc = 1.0 / np.sqrt(Dh)

    # the scale is fused into the softmax (same bits as nrs_scale followed
    # by nrs_softmax_forward / nrs_softmax_backward)
    def fwd():
        hip.bmm(hip.NT, S, q, k, BH, T, T, Dh)
        hip.call("nrs_softmax_forward_scaled", P.ptr, S.ptr, BH * T, T, sc)
        hip.bmm(hip.NN, o, P, v, BH, T, Dh, T)

    # each bmm's backward computes both of its gradients in one call, as the
    # reference's bmm backward closure does (src/cuda/graph/bmm.rs:93-131):
    # O = P.V (NN): dP = dO.V^T, dV = P^T.dO; S = Q.K^T (NT): dQ = dS.K,
    # dK = dS^T.Q
    def bwd():
        hip.bmm_backward(hip.NN, dP, dv, do, P, v, BH, T, T, Dh)
        hip.call("nrs_softmax_backward_scaled", dS.ptr, P.ptr, dP.ptr, BH * T, T, sc, 0.0)
        hip.bmm_backward(hip.NT, dq, dk, dS, q, k, BH, T, Dh, T)

    def bmms_only():
        hip.bmm(hip.NT, S, q, k, BH, T, T, Dh)
        hip.bmm(hip.NN, o, P, v, BH, T, Dh, T)
        hip.bmm_backward(hip.NN, dP, dv, do, P, v, BH, T, T, Dh)
        hip.bmm_backward(hip.NT, dq, dk, dS, q, k, BH, T, Dh, T)

    # the same products with the gradients accumulated into existing
    # buffers (beta = 1), the form the drop-in backward closure uses
    def bmms_accumulate():
        hip.bmm(hip.NT, S, q, k, BH, T, T, Dh)
        hip.bmm(hip.NN, o, P, v, BH, T, Dh, T)
        hip.bmm_backward(hip.NN, dP, dv, do, P, v, BH, T, T, Dh, 1.0)
        hip.bmm_backward(hip.NT, dq, dk, dS, q, k, BH, T, Dh, T, 1.0)

    # the fused attention core (nrs_attention_forward / _backward): every
    # head's softmax(scale Q.K^T).V in one launch, heads read and written in
    # place in the projections' [32*128, 256] rows, scores kept on chip
    Bf, Hf, ldf = 32, 8, 8 * Dh
    fq, fk, fv, fdo = (D(rng.standard_normal(Bf * T * ldf).astype(np.float32)) for _ in range(4))
    fo, fst = hip.DeviceBuffer(Bf * T * ldf), hip.DeviceBuffer(Bf * Hf * T * 2)
    fdq, fdk, fdv = (hip.DeviceBuffer(Bf * T * ldf) for _ in range(3))

    def fused_fwd():
        hip.call("nrs_attention_forward", fo, fst, fq, fk, fv, Bf, Hf, T, Dh, ldf, sc)

    def fused_bwd():
        hip.call("nrs_attention_backward", fdq, fdk, fdv, fdo, fo, fq, fk, fv, fst, Bf, Hf, T,
                 Dh, ldf, sc, 0.0)

    # the heads of the projections [32*128, 8*32] split into [8, 4096, 32]
    # (q, k, v) and the attention output merged back: one launch each, in
    # place of the reference's per-head slice_cols / concat_cols loops
    Rh, Hh = 32 * 128, 8
    wide = [D(rng.standard_normal(Rh * Hh * Dh).astype(np.float32)) for _ in range(3)]
    split = [hip.DeviceBuffer(Rh * Hh * Dh) for _ in range(3)]
    merged = hip.DeviceBuffer(Rh * Hh * Dh)

    def heads():
        for w_, s_ in zip(wide, split):
            hip.call("nrs_split_heads", s_.ptr, w_.ptr, Rh, Hh, Dh, 0.0)
        hip.call("nrs_merge_heads", merged.ptr, split[0].ptr, Rh, Hh, Dh, 0.0)

    # the block's LayerNorm over [4096, 256], forward and backward (input,
    # gamma and beta gradients, accumulated)
    lx = wide[0]
    lg, lb = D(np.ones(Hh * Dh, np.float32)), D(np.zeros(Hh * Dh, np.float32))
    lout, lxn, listd = hip.DeviceBuffer(Rh * Hh * Dh), hip.DeviceBuffer(Rh * Hh * Dh), hip.DeviceBuffer(Rh)
    ldin = hip.DeviceBuffer.zeros(Rh * Hh * Dh)
    ldg, ldb = hip.DeviceBuffer.zeros(Hh * Dh), hip.DeviceBuffer.zeros(Hh * Dh)

    def layernorm():
        hip.call("nrs_layernorm_forward", lout.ptr, lxn.ptr, listd.ptr, lx.ptr, lg.ptr, lb.ptr,
                 Rh, Hh * Dh, 1e-5)
        hip.call("nrs_layernorm_backward", ldin.ptr, ldg.ptr, ldb.ptr, split[1].ptr, lg.ptr,
                 lxn.ptr, listd.ptr, Rh, Hh * Dh, 1.0)

    if closures_only:
        closures = {"attn_bmm6_cfg4": bmms_only, "heads_split_merge_cfg4": heads,
                    "layernorm_cfg4": layernorm, "attn_fused_fwd_cfg4": fused_fwd,
                    "attn_fused_bwd_cfg4": fused_bwd}
    else:
        fwd()
        fwd_us = leg_ms(hip, fwd, steps, warmup) * 1e3
        bwd_us = leg_ms(hip, bwd, steps, warmup) * 1e3
        bmm_us = leg_ms(hip, bmms_only, steps, warmup) * 1e3
        bmm_acc_us = leg_ms(hip, bmms_accumulate, steps, warmup) * 1e3
        fused_fwd()
        ffwd_us = leg_ms(hip, fused_fwd, steps, warmup) * 1e3
        fbwd_us = leg_ms(hip, fused_bwd, steps, warmup) * 1e3
        heads_us = leg_ms(hip, heads, steps, warmup) * 1e3
        heads_roof = roofline_us(0.0, 4 * 8.0 * Rh * Hh * Dh)  # each reads and writes 4 MB
        ln_us = leg_ms(hip, layernorm, steps, warmup) * 1e3
        # forward reads x, writes out and x_norm; backward reads grad and
        # x_norm, writes dinput (+ reads dinput, accumulating); the parameter
        # sums read grad and x_norm: 9 passes of 4 MB
        ln_roof = roofline_us(0.0, 9 * 4.0 * Rh * Hh * Dh)
    bmm_roof = 6 * roofline_us(*gemm_roof(T, T, Dh, BH))  # every product moves 25.2 MB
    # the fused core's bound: the six products' FLOP at MFMA peak (forward
    # 2, backward 4; its HBM traffic, Q/K/V/dO in and O/dQ/dK/dV out, 32 MB,
    # takes less at 8 TB/s); the backward's recomputation of the scores is
    # extra work, not counted
    fused_roof = 6 * 2.0 * BH * T * T * Dh / (PEAK_FP32_MFMA_TFLOPS * 1e12) * 1e6

    # the block's Linear GEMMs: X[4096,256] through 4 projections and the FFN,
    # launched as the operator surface launches them: the Q, K, V projections
    # of one input as one grouped launch and their backward as one pass
    # (nrs_matmul_shared_lhs_backward: six products in one grouped launch and
    # the sums), each other layer's input and weight gradients (dX = dY.W^T,
    # dW = X^T.dY) as one grouped launch
    R, dm, ff = 32 * 128, 256, 1024
    X = D(rng.standard_normal(R * dm).astype(np.float32))
    H = D(rng.standard_normal(R * ff).astype(np.float32))
    Wp = [D((rng.standard_normal(dm * dm) * np.sqrt(1.0 / dm)).astype(np.float32))
          for _ in range(4)]
    W1 = D((rng.standard_normal(dm * ff) * np.sqrt(1.0 / dm)).astype(np.float32))
    W2 = D((rng.standard_normal(ff * dm) * np.sqrt(1.0 / ff)).astype(np.float32))
    Yp = [hip.DeviceBuffer(R * dm) for _ in range(4)]
    Yd, Yf, gXd, gXf = (hip.DeviceBuffer(R * dm), hip.DeviceBuffer(R * ff),
                        hip.DeviceBuffer(R * dm), hip.DeviceBuffer(R * ff))
    gWp = [hip.DeviceBuffer(dm * dm) for _ in range(4)]
    gW1, gW2 = hip.DeviceBuffer(dm * ff), hip.DeviceBuffer(ff * dm)
    shapes = []

    def linears():
        hip.gemm_group([(hip.NN, Yp[i], X, Wp[i], R, dm, dm) for i in range(3)])  # Q, K, V
        hip.gemm(hip.NN, Yp[3], X, Wp[3], R, dm, dm)                              # output proj
        hip.gemm(hip.NN, Yf, X, W1, R, ff, dm)
        hip.gemm(hip.NN, Yd, H, W2, R, dm, ff)
        hip.matmul_shared_lhs_backward(gXd, gWp[:3], Yp[:3], X, Wp[:3], R, dm, dm)
        hip.gemm_group([(hip.NT, gXd, Yp[3], Wp[3], R, dm, dm),
                        (hip.TN, gWp[3], X, Yp[3], dm, dm, R)])
        hip.gemm_group([(hip.NT, gXd, Yf, W1, R, dm, ff), (hip.TN, gW1, X, Yf, dm, ff, R)])
        hip.gemm_group([(hip.NT, gXf, Yd, W2, R, ff, dm), (hip.TN, gW2, H, Yd, ff, dm, R)])

    for _ in range(4):
        shapes += [(R, dm, dm), (R, dm, dm), (dm, dm, R)]
    shapes += [(R, ff, dm), (R, dm, ff), (dm, ff, R), (R, dm, ff), (R, ff, dm), (ff, dm, R)]
    if closures_only:
        closures["linear_gemms_cfg4"] = linears
        return closures
    lin_us = event_ms(hip, linears, steps, warmup) * 1e3
    lin_flops = sum(gemm_roof(*s)[0] for s in shapes)
    lin_roof = sum(roofline_us(*gemm_roof(*s)) for s in shapes)
    return {"fwd_us": fwd_us, "bwd_us": bwd_us, "bmm_us": bmm_us, "bmm_roof_us": bmm_roof,
            "fused_fwd_us": ffwd_us, "fused_bwd_us": fbwd_us, "fused_roof_us": fused_roof,
            "bmm_acc_us": bmm_acc_us, "heads_us": heads_us, "heads_roof_us": heads_roof,
            "ln_us": ln_us, "ln_roof_us": ln_roof,
            "linear_us": lin_us, "linear_tflops": lin_flops / (lin_us * 1e-6) / 1e12,
            "linear_roof_us": lin_roof}


def bench_sweep_cfg5(hip, reps):
    """cfg5 sweep: square NN GEMMs 2048^3 and 8192^3, skinny 32x8192x8192,
    and the split-K weight-gradient NT shape 64x576 over K = 100352. Each is
    spot-checked against f64 on a few rows."""
    import oracle
    rng = np.random.default_rng(5)
    out = {}
    cases = (("nn_2048", hip.NN, 2048, 2048, 2048), ("nn_8192", hip.NN, 8192, 8192, 8192),
             ("skinny_32x8192x8192", hip.NN, 32, 8192, 8192),
             ("wgrad_nt_64x576x100352", hip.NT, 64, 576, 100352))
    for name, layout, m, n, k in cases:
        a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
        b = rng.uniform(-1, 1, (k, n) if layout == hip.NN else (n, k)).astype(np.float32)
        dA, dB, dC = hip.DeviceBuffer.from_host(a), hip.DeviceBuffer.from_host(b), hip.DeviceBuffer(m * n)
        if layout == hip.NN:
            fn = lambda: hip.gemm(hip.NN, dC, dA, dB, m, n, k)
        else:
            fn = lambda: hip.gemm_nt_splitk(dC, dA, dB, m, n, k)
        r = max(2, reps if m * n * k < 2 ** 36 else reps // 10)
        ms = event_ms(hip, fn, r, 2)
        c = dC.to_host((m, n))
        rows = np.arange(0, m, max(1, m // 4))
        c64, ab = oracle.gemm_f64("nn" if layout == hip.NN else "nt", a, b, m, n, k, rowidx=rows)
        err = float(np.max(np.abs(c[rows] - c64) / np.maximum(ab, 1e-30)))
        fl, by = gemm_roof(m, n, k)
        roof = roofline_us(fl, by)
        out[name] = {"us": round(ms * 1e3, 2), "tflops": round(fl / (ms * 1e-3) / 1e12, 2),
                     "bound": "hbm" if by / (PEAK_HBM_GBS * 1e9) > fl / (PEAK_FP32_MFMA_TFLOPS * 1e12) else "mfma",
                     "roofline_frac": round(roof / (ms * 1e3), 4), "max_rel_err_vs_f64": err}
        del dA, dB, dC
    return out


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


def cpu_baseline_extra():
    """BASELINE's CPU plan beside the GEMM baseline: host CPU model, the
    oracle's matmul_simd at 512^3 (cfg1) on all threads and on one, the cfg3
    conv layers forward + backward (C restatement of nn::conv::Conv2d,
    OpenMP over images) on a bounded 16-image sample, in imgs/s, and cfg2's
    six MLP GEMMs on the restated CPU autograd matmul, in us per step."""
    import oracle
    import subprocess
    model, cpu_id = "unknown", {}
    try:
        lscpu = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in lscpu.splitlines():
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "Model name":
                model = v
            elif k in ("CPU family", "Model", "Stepping", "Socket(s)", "Core(s) per socket",
                       "Thread(s) per core", "CPU(s)"):
                cpu_id[k] = v
    except (OSError, subprocess.SubprocessError):
        pass
    if model == "unknown":
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        model = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
    threads = oracle.max_threads()
    rng = np.random.default_rng(1)
    a = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    b = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    out = {"host_cpu": model, "lscpu": cpu_id, "threads": threads,
           "nproc": os.cpu_count()}
    for nt, key in ((0, "matmul_simd_512_gflops"), (1, "matmul_simd_512_gflops_1thread")):
        oracle.matmul_simd(a, b, nt)
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 1.0:
            oracle.matmul_simd(a, b, nt)
            reps += 1
        out[key] = round(2.0 * 512 ** 3 * reps / (time.perf_counter() - t0) / 1e9, 2)
    n = 16
    x = rng.uniform(0, 1, n * 784).astype(np.float32)
    w1 = (rng.standard_normal(32 * 9) * np.sqrt(2.0 / 9)).astype(np.float32)
    w2 = (rng.standard_normal(64 * 288) * np.sqrt(2.0 / 288)).astype(np.float32)
    b1, b2 = np.zeros(32, np.float32), np.zeros(64, np.float32)
    p1 = rng.uniform(0, 1, n * 32 * 196).astype(np.float32)   # pooled conv1 output
    g2 = rng.standard_normal(n * 64 * 196).astype(np.float32)
    g1 = rng.standard_normal(n * 32 * 784).astype(np.float32)

    def layers():
        oracle.conv2d_forward(x, w1, b1, n, 1, 32, 28, 28, 3, 3, 1, 1)
        oracle.conv2d_forward(p1, w2, b2, n, 32, 64, 14, 14, 3, 3, 1, 1)
        oracle.conv2d_backward(p1, w2, g2, n, 32, 64, 14, 14, 3, 3, 1, 1)
        oracle.conv2d_backward(x, w1, g1, n, 1, 32, 28, 28, 3, 3, 1, 1)

    layers()
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 3.0:
        layers()
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    out["conv_cfg3_imgs_per_s"] = round(n / dt, 1)
    # the same sample on one thread
    oracle.set_threads(1)
    layers()
    reps1, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 3.0:
        layers()
        reps1 += 1
    dt1 = (time.perf_counter() - t0) / reps1
    oracle.set_threads(threads)
    out["conv_cfg3_imgs_per_s_1thread"] = round(n / dt1, 1)
    # cfg2's six MLP GEMMs on the reference's CPU autograd matmul (forward
    # and backward loops of autograd/graph/matmul.rs, single-threaded as
    # there), on the same shapes as the GPU step
    B, I, Hd, O = 256, 784, 128, 10
    xm = rng.standard_normal((B, I)).astype(np.float32)
    w1m = (rng.standard_normal((I, Hd)) * np.sqrt(2.0 / I)).astype(np.float32)
    w2m = (rng.standard_normal((Hd, O)) * np.sqrt(2.0 / Hd)).astype(np.float32)
    gz = (rng.standard_normal((B, O)) / B).astype(np.float32)
    gh = rng.standard_normal((B, Hd)).astype(np.float32)

    def mlp_gemms():
        h = oracle.graph_matmul_forward(xm, w1m)
        oracle.graph_matmul_forward(h, w2m)
        oracle.graph_matmul_backward(h, w2m, gz)
        oracle.graph_matmul_backward(xm, w1m, gh)

    mlp_gemms()
    mreps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 3.0:
        mlp_gemms()
        mreps += 1
    mdt = (time.perf_counter() - t0) / mreps
    out["mlp_cfg2_gemms_us_per_step"] = round(mdt * 1e6, 1)
    out["mlp_cfg2_sample"] = (f"cfg2's 6 GEMMs (x.W1, h.W2 and their backward products, "
                              f"156.1 MFLOP) on the C restatement of autograd/graph/matmul.rs, "
                              f"1 thread, {mreps} reps, {mdt * 1e3:.1f} ms each")
    out["conv_cfg3_sample"] = (f"{n} images of cfg3 (conv1 1->32 @28x28, conv2 32->64 @14x14, "
                               f"forward + backward with input, weight and bias grads), "
                               f"{reps} reps, {dt * 1e3:.1f} ms each on {threads} threads; "
                               f"{reps1} reps, {dt1 * 1e3:.1f} ms each on 1 thread")
    return out


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


def counters_pass(hip):
    """Launch sequence for rocprofv3 --pmc over every bench leg: the
    COPY_BYTES device copy (counter calibration), then each leg's launches
    twice, the first call warming up, the second the one to read. A 4 KiB
    device copy goes before each call as a separator, so the dispatch list
    splits by position: after the calibration copy, segment 2i is leg i's
    warm-up and segment 2i + 1 its counted call. Prints the leg names, in
    order, as one JSON line."""
    src = hip.DeviceBuffer.zeros(COPY_BYTES // 4)
    dst = hip.DeviceBuffer(COPY_BYTES // 4)
    mark_a, mark_b = hip.DeviceBuffer.zeros(1024), hip.DeviceBuffer(1024)
    legs = []
    rng = np.random.default_rng(5)
    keep = []
    for name, layout, m, n, k in (("gemm_nn_4096", hip.NN, 4096, 4096, 4096),
                                  ("gemm_nn_2048", hip.NN, 2048, 2048, 2048),
                                  ("gemm_nn_8192", hip.NN, 8192, 8192, 8192),
                                  ("gemm_skinny_32x8192x8192", hip.NN, 32, 8192, 8192),
                                  ("gemm_wgrad_nt_64x576x100352", hip.NT, 64, 576, 100352)):
        a = hip.DeviceBuffer.from_host(rng.uniform(-1, 1, m * k).astype(np.float32))
        b = hip.DeviceBuffer.from_host(rng.uniform(-1, 1, k * n).astype(np.float32))
        c = hip.DeviceBuffer(m * n)
        keep += [a, b, c]
        if layout == hip.NN:
            fn = (lambda a=a, b=b, c=c, m=m, n=n, k=k: hip.gemm(hip.NN, c, a, b, m, n, k))
        else:
            fn = (lambda a=a, b=b, c=c, m=m, n=n, k=k: hip.gemm_nt_splitk(c, a, b, m, n, k))
        legs.append((name, fn))
    legs += list(bench_conv_cfg3(hip, 0, 0, closures_only=True).items())
    legs += list(bench_attention_cfg4(hip, 0, 0, closures_only=True).items())
    legs += list(bench_mlp_cfg2(hip, 0, 0, closures_only=True).items())
    hip.call("nrs_memcpy_dtod", dst.ptr, src.ptr, COPY_BYTES)
    hip.sync()
    for _, fn in legs:
        for _ in range(2):
            hip.call("nrs_memcpy_dtod", mark_b.ptr, mark_a.ptr, 4096)
            fn()
            hip.sync()
    print(json.dumps([name for name, _ in legs]))


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
    ap.add_argument("--no-legs", action="store_true",
                    help="skip the cfg2 / cfg4 / cfg5 legs (MLP step, attention, GEMM sweep)")
    ap.add_argument("--counters-pass", action="store_true",
                    help="only launch every leg twice behind 4 KiB copy separators, after a "
                         "256 MiB copy calibration, for rocprofv3 --pmc runs; prints the leg "
                         "names")
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
    if args.counters_pass:
        counters_pass(hip)
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
                     "kernel": "gemm_kernel 256x256x32 tile, 2x4 waves, NN",
                     "kernel_ms": round(g["kernel_ms"], 4)},
    }
    if not args.no_conv:
        c = bench_conv_cfg3(hip, max(5, args.steps // 2), args.warmup)
        hc = host_step("cnn", 200, 20)
        out["conv2d_fwd_bwd"] = {
            "value": round(hc["imgs_per_s"] if hc else c["imgs_per_s"], 1), "unit": "imgs/s",
            "timing": ("neuralrs_amd/bench_host cnn: the step through the C++ operator surface "
                       "(nn::conv2d_maxpool with ReLU, nn::conv2d, backward_graph, zero_grad), "
                       "HIP events on the stream" if hc else
                       "C ABI calls from Python, wall clock (bench_host missing)"),
            "step_us": round(hc["step_gpu_us"], 2) if hc else None,
            "step_us_op_by_op": round(hc["unfused_step_gpu_us"], 2) if hc else None,
            "c_abi_ms_per_step": round(c["ms_per_step"], 4),
            "c_abi_ms_per_step_unfused": round(c["ms_per_step_unfused"], 4),
            "config": "cfg3 batch 128 conv1 1->32 3x3 p1, ReLU, 2x2 maxpool, conv2 32->64 3x3 p1 "
                      "(the reference CNN's maxpool2d(relu(conv2d(..))), "
                      "examples/mnist_cuda_cnn.rs:125), fwd+bwd: weight and bias grads of both "
                      "layers, input grad of conv2 (the image batch requires no grad, as in "
                      "examples/mnist_cuda_cnn.rs:261); conv1, ReLU and the maxpool as one node "
                      "each way, conv2's backward giving conv1's parameter gradients in its "
                      "launch, op by op in step_us_op_by_op; the conv_* legs time the two conv "
                      "layers' own passes against their rooflines",
            "conv1_maxpool_fwd_us": round(c["conv1_pool_fwd_us"], 2),
            "maxpool_conv1_bwd_us": round(c["pool_conv1_bwd_us"], 2),
            "conv_fwd_us": round(c["fwd_us"], 2), "conv_bwd_us": round(c["bwd_us"], 2),
            "fwd_roofline_us": round(c["fwd_roof_us"], 2),
            "bwd_roofline_us": round(c["bwd_roof_us"], 2),
            "fwd_roofline_frac": round(c["fwd_roof_us"] / c["fwd_us"], 4),
            "bwd_roofline_frac": round(c["bwd_roof_us"] / c["bwd_us"], 4),
            "conv1_input_grad_us": round(c["conv1_input_grad_us"], 2),
            "conv1_input_grad_roofline_frac": round(
                c["conv1_input_grad_roof_us"] / c["conv1_input_grad_us"], 4)}
    if not args.no_legs:
        m = bench_mlp_cfg2(hip, args.steps, 5)
        hm = host_step("mlp", 200, 20)
        out["mlp_cfg2"] = {"python_us_per_step": round(m["us_per_step"], 2),
                           "python_us_per_step_four_calls": round(m["us_per_step_four_calls"], 2),
                           "gemm_roofline_us": round(m["gemm_roof_us"], 3),
                           "library_calls": 2,
                           "config": "cfg2 Linear 784->128 (+bias) -> ReLU -> Linear 128->10 "
                                     "(+bias) -> CE seed -> hidden gradient through the ReLU "
                                     "(nrs_mlp2_forward_seed, one launch), then dW1, db1, dW2, db2 "
                                     "and dx (nrs_mlp2_backward, one launch); batch 256"}
        if hm:
            out["mlp_cfg2"].update({
                "us_per_step": round(hm["eager_gpu_us"], 2),
                "graph_us_per_step": round(hm["graph_gpu_us"], 2),
                "us_per_step_four_calls": round(hm["four_call_gpu_us"], 2),
                "gemm_roofline_frac": round(m["gemm_roof_us"] / hm["eager_gpu_us"], 4),
                "timing": "C++ issue (neuralrs_amd/bench_host mlp), HIP events on the stream"})
        hb = host_step("block", 200, 20)
        if hb:
            gemm_roof = hb["gemm_flop_per_step"] / (PEAK_FP32_MFMA_TFLOPS * 1e12) * 1e6
            out["transformer_block_cfg4"] = {
                "step_us": round(hb["step_gpu_us"], 2), "fwd_us": round(hb["fwd_gpu_us"], 2),
                "gemm_flop_per_step": hb["gemm_flop_per_step"],
                "gemm_roofline_us": round(gemm_roof, 2),
                "gemm_roofline_frac": round(gemm_roof / hb["step_gpu_us"], 4),
                "config": "cfg4 TransformerBlock B32 S128 d256 h8 dff1024 forward + backward "
                          "through the C++ operator surface (libnrs_host.so), from C++",
                "timing": "neuralrs_amd/bench_host block, HIP events on the stream"}
        at = bench_attention_cfg4(hip, args.steps, 5)
        out["attention_cfg4"] = {
            "bmm_us": round(at["bmm_us"], 2), "bmm_roofline_us": round(at["bmm_roof_us"], 2),
            "bmm_roofline_frac": round(at["bmm_roof_us"] / at["bmm_us"], 4),
            "bmm_accumulate_us": round(at["bmm_acc_us"], 2),
            "heads_split3_merge1_us": round(at["heads_us"], 2),
            "heads_roofline_frac": round(at["heads_roof_us"] / at["heads_us"], 4),
            "layernorm_fwd_bwd_us": round(at["ln_us"], 2),
            "layernorm_roofline_frac": round(at["ln_roof_us"] / at["ln_us"], 4),
            "attn_fwd_us": round(at["fwd_us"], 2), "attn_bwd_us": round(at["bwd_us"], 2),
            "fused_fwd_us": round(at["fused_fwd_us"], 2),
            "fused_bwd_us": round(at["fused_bwd_us"], 2),
            "fused_roofline_us": round(at["fused_roof_us"], 2),
            "fused_roofline_frac": round(at["fused_roof_us"] / (at["fused_fwd_us"] + at["fused_bwd_us"]), 4),
            "linear_us": round(at["linear_us"], 2), "linear_tflops": round(at["linear_tflops"], 2),
            "linear_roofline_frac": round(at["linear_roof_us"] / at["linear_us"], 4),
            "config": "cfg4 batch 32 x 8 heads, seq 128, d_head 32: the fused attention core "
                      "(fused_*), the same core as 6 bmm (QK^T, PV and the 4 backward products) "
                      "+ softmax launches (attn_*, bmm_*), 4 proj and 2 FFN Linear GEMMs fwd+bwd"}
        out["gemm_sweep_cfg5"] = bench_sweep_cfg5(hip, args.steps)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_gemm(g["a"], g["b"])
        out["cpu_baseline_extra"] = cpu_baseline_extra()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
