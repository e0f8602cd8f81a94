// Step timings from C++ (no Python between launches), printed as one JSON
// object for bench.py:
//   block: the cfg4 TransformerBlock (B32 S128 d256 h8 dff1024) forward and
//          backward through the C++ operator surface (libnrs_host.so), the
//          path a drop-in caller takes: nn::TransformerBlock::forward,
//          the upstream gradient swapped in (runtime::swap_grad),
//          backward_graph, zero_grad of the parameters;
//   mlp:   the cfg2 MLP training step (784 -> 128 -> ReLU -> 10, batch 256,
//          fused cross-entropy gradient) issued through the C ABI in two
//          calls, timed eagerly and as a replayed HIP graph of the same
//          launches, and the four-call form of the same step eagerly;
//   cnn:   the cfg3 step (batch 128: conv1 1->32 3x3 p1 -> ReLU -> 2x2 max
//          pool -> conv2 32->64 3x3 p1, forward and backward, the image
//          batch requiring no gradient) through the C++ operator surface, as
//          the reference CNN builds it (maxpool2d(relu(conv2d(..)))), op by
//          op and with conv1 + ReLU + pool as one conv2d_maxpool node.
// Usage: bench_host {block|mlp|cnn} [steps] [warmup]
#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "neuralrs.hpp"
#include "nrs_hip.h"

using namespace neuralrs;
using Vec = std::vector<float>;
namespace gpu = neuralrs::hip::runtime;

namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
        std::exit(2);
    }
}

void nrs_check(int rc, const char* what) {
    if (rc != NRS_OK) {
        std::fprintf(stderr, "%s: %s\n", what, nrs_last_error());
        std::exit(2);
    }
}

std::mt19937_64 rng(7);

Vec normal(size_t n, float std) {
    std::normal_distribution<float> d(0.0f, std);
    Vec v(n);
    for (float& x : v) x = d(rng);
    return v;
}

Vec uniform(size_t n, float lo, float hi) {
    std::uniform_real_distribution<float> d(lo, hi);
    Vec v(n);
    for (float& x : v) x = d(rng);
    return v;
}

NodeRef resident(const Vec& v, std::vector<size_t> shape) {
    NodeRef n = Node::create(v, std::move(shape));
    gpu::to_cuda(n);
    return n;
}

// GPU time of `steps` calls of fn on the library stream (HIP events) and the
// host wall time of the same loop, after `warmup` calls.
template <class F>
void time_steps(F&& fn, int steps, int warmup, double& gpu_us, double& wall_us) {
    for (int i = 0; i < warmup; ++i) fn();
    nrs_check(nrs_sync(), "sync");
    hipStream_t s = static_cast<hipStream_t>(nrs_get_stream());
    hipEvent_t e0, e1;
    hip_check(hipEventCreate(&e0), "event");
    hip_check(hipEventCreate(&e1), "event");
    const auto t0 = std::chrono::steady_clock::now();
    hip_check(hipEventRecord(e0, s), "record");
    for (int i = 0; i < steps; ++i) fn();
    hip_check(hipEventRecord(e1, s), "record");
    hip_check(hipEventSynchronize(e1), "event sync");
    const auto t1 = std::chrono::steady_clock::now();
    float ms = 0.0f;
    hip_check(hipEventElapsedTime(&ms, e0, e1), "elapsed");
    gpu_us = 1e3 * ms / steps;
    wall_us = std::chrono::duration<double, std::micro>(t1 - t0).count() / steps;
    hip_check(hipEventDestroy(e0), "event");
    hip_check(hipEventDestroy(e1), "event");
}

int bench_block(int steps, int warmup) {
    const size_t B = 32, S = 128, D = 256, H = 8, F = 1024;
    const float xa = std::sqrt(6.0f / (2 * D)), fa = std::sqrt(6.0f / (D + F));
    NodeRef wq = resident(uniform(D * D, -xa, xa), {D, D}), wk = resident(uniform(D * D, -xa, xa), {D, D});
    NodeRef wv = resident(uniform(D * D, -xa, xa), {D, D}), wo = resident(uniform(D * D, -xa, xa), {D, D});
    NodeRef g1 = resident(Vec(D, 1.0f), {D}), b1 = resident(Vec(D, 0.0f), {D});
    NodeRef g2 = resident(Vec(D, 1.0f), {D}), b2 = resident(Vec(D, 0.0f), {D});
    NodeRef f1w = resident(uniform(D * F, -fa, fa), {D, F}), f1b = resident(Vec(F, 0.0f), {F});
    NodeRef f2w = resident(uniform(F * D, -fa, fa), {F, D}), f2b = resident(Vec(D, 0.0f), {D});
    hip::nn::TransformerBlock tb{hip::nn::MultiHeadAttention(wq, wk, wv, wo, D, H),
                                 hip::nn::LayerNorm(g1, b1, 1e-5f), hip::nn::LayerNorm(g2, b2, 1e-5f),
                                 hip::nn::Linear(f1w, f1b), hip::nn::Linear(f2w, f2b), D, F};
    NodeRef x = resident(normal(B * S * D, 1.0f), {B, S, D});
    const std::vector<NodeRef> params{wq, wk, wv, wo, g1, b1, g2, b2, f1w, f1b, f2w, f2b};
    // upstream gradient: a resident buffer swapped in as the output's
    // gradient and back (set_grad's host copy would synchronise every step;
    // in a network the layer above writes it there)
    DeviceBuffer seed = DeviceBuffer::from_host(normal(B * S * D, 1.0f));
    auto step = [&] {
        NodeRef out = tb.forward(x);
        gpu::swap_grad(out, seed);
        backward_graph(out);
        gpu::swap_grad(out, seed);
        gpu::zero_grad(params);
        x->gpu->grad->zero();
    };
    double gpu_us = 0, wall_us = 0;
    time_steps(step, steps, warmup, gpu_us, wall_us);
    // forward alone
    double f_gpu = 0, f_wall = 0;
    time_steps([&] { NodeRef out = tb.forward(x); }, steps, warmup, f_gpu, f_wall);
    const double flops_fwd = 2.0 * B * S * (4.0 * D * D + 2.0 * D * F) + 2.0 * 2.0 * B * H * S * S * (D / H);
    std::printf("{\"workload\": \"cfg4 TransformerBlock B32 S128 d256 h8 dff1024 through libnrs_host.so\", "
                "\"step_gpu_us\": %.2f, \"step_wall_us\": %.2f, \"fwd_gpu_us\": %.2f, "
                "\"fwd_wall_us\": %.2f, \"gemm_flop_per_step\": %.6e, \"steps\": %d}\n",
                gpu_us, wall_us, f_gpu, f_wall, 3.0 * flops_fwd, steps);
    return 0;
}

int bench_cnn(int steps, int warmup) {
    const size_t N = 128, H = 28, W = 28, C1 = 32, C2 = 64;
    NodeRef x = resident(uniform(N * H * W, 0.0f, 1.0f), {N, 1, H, W});
    x->requires_grad = false;  // examples/mnist_cuda_cnn.rs:261
    NodeRef w1 = resident(normal(C1 * 9, std::sqrt(2.0f / 9.0f)), {C1, 1, 3, 3});
    NodeRef b1 = resident(Vec(C1, 0.0f), {C1});
    NodeRef w2 = resident(normal(C2 * C1 * 9, std::sqrt(2.0f / 288.0f)), {C2, C1, 3, 3});
    NodeRef b2 = resident(Vec(C2, 0.0f), {C2});
    const std::vector<NodeRef> params{w1, b1, w2, b2};
    DeviceBuffer seed = DeviceBuffer::from_host(normal(N * C2 * 14 * 14, 1.0f));
    auto run = [&](bool fused) {
        NodeRef p1 = fused ? hip::nn::conv2d_maxpool(x, w1, b1, 1, 1, true, 2, 2)
                           : hip::nn::maxpool2d(hip::graph::relu(hip::nn::conv2d(x, w1, b1, 1, 1)),
                                                2, 2);
        NodeRef out = hip::nn::conv2d(p1, w2, b2, 1, 1);
        // the upstream gradient swapped in as the output's gradient (no
        // copy: in a network the layer above writes it there), then back
        gpu::swap_grad(out, seed);
        backward_graph(out);
        gpu::swap_grad(out, seed);
        gpu::zero_grad(params);
    };
    double f_gpu = 0, f_wall = 0, u_gpu = 0, u_wall = 0;
    time_steps([&] { run(true); }, steps, warmup, f_gpu, f_wall);
    time_steps([&] { run(false); }, steps, warmup, u_gpu, u_wall);
    std::printf("{\"workload\": \"cfg3 CNN step batch 128 (conv1 -> ReLU -> 2x2 maxpool -> conv2, "
                "fwd + bwd) through libnrs_host.so\", \"step_gpu_us\": %.2f, \"step_wall_us\": %.2f, "
                "\"imgs_per_s\": %.1f, \"unfused_step_gpu_us\": %.2f, \"unfused_step_wall_us\": %.2f, "
                "\"steps\": %d}\n",
                f_gpu, f_wall, N / (f_gpu * 1e-6), u_gpu, u_wall, steps);
    return 0;
}

int bench_mlp(int steps, int warmup) {
    const int64_t Bn = 256, I = 784, Hd = 128, O = 10;
    DeviceBuffer x = DeviceBuffer::from_host(normal(Bn * I, 1.0f));
    DeviceBuffer w1 = DeviceBuffer::from_host(normal(I * Hd, std::sqrt(2.0f / I)));
    DeviceBuffer w2 = DeviceBuffer::from_host(normal(Hd * O, std::sqrt(2.0f / Hd)));
    DeviceBuffer b1(Hd, true), b2(O, true);
    Vec t(Bn * O, 0.0f);
    std::uniform_int_distribution<int> cls(0, O - 1);
    for (int64_t r = 0; r < Bn; ++r) t[r * O + cls(rng)] = 1.0f;
    DeviceBuffer onehot = DeviceBuffer::from_host(t);
    DeviceBuffer a(Bn * Hd, false), z(Bn * O, false), gz(Bn * O, false),
        gh(Bn * Hd, false), gx(Bn * I, false);
    DeviceBuffer gw1(I * Hd, true), gw2(Hd * O, true), gb1(Hd, true), gb2(O, true);
    // the reference's step (Linear, ReLU, Linear, the fused cross-entropy
    // seed (softmax - onehot) / batch, then each layer's backward: dW and db
    // accumulated, dx written) in two library calls of one launch each: the
    // row-local part (both layers forward, the seed, the hidden layer's
    // gradient through the ReLU) and the gradients that sum over the batch
    // (dW1, db1, dW2, db2) with dx.
    auto step = [&] {
        nrs_check(nrs_mlp2_forward_seed(a.ptr(), z.ptr(), gz.ptr(), gh.ptr(), x.ptr(), w1.ptr(),
                                        b1.ptr(), w2.ptr(), b2.ptr(), onehot.ptr(), Bn, I, Hd, O),
                  "mlp2 forward + seed");
        nrs_check(nrs_mlp2_backward(gx.ptr(), gw1.ptr(), gb1.ptr(), gw2.ptr(), gb2.ptr(), gh.ptr(),
                                    gz.ptr(), x.ptr(), w1.ptr(), a.ptr(), Bn, I, Hd, O, 0.0f, 1.0f),
                  "mlp2 backward");
    };
    // the same step in four library calls: layer 1 with bias and ReLU in the
    // product's epilogue; layer 2 with the seed in its epilogue; layer 2's
    // backward with the ReLU backward applied to its input gradient (the mask
    // is the ReLU output: a > 0 exactly where the pre-activation is); layer
    // 1's backward. Each is one launch.
    auto step4 = [&] {
        nrs_check(nrs_gemm(NRS_NN, a.ptr(), x.ptr(), w1.ptr(), Bn, Hd, I, 0.0f, b1.ptr(),
                           NRS_EPI_BIAS_COL | NRS_EPI_RELU), "l1+relu");
        nrs_check(nrs_linear_cross_entropy(z.ptr(), gz.ptr(), a.ptr(), w2.ptr(), b2.ptr(),
                                           onehot.ptr(), Bn, Hd, O), "l2+ce");
        nrs_check(nrs_linear_backward_relu(gh.ptr(), gw2.ptr(), gb2.ptr(), gz.ptr(), a.ptr(),
                                           w2.ptr(), a.ptr(), Bn, Hd, O, 0.0f, 1.0f, 1.0f),
                  "layer 2 bwd + relu bwd");
        nrs_check(nrs_linear_backward(gx.ptr(), gw1.ptr(), gb1.ptr(), gh.ptr(), x.ptr(), w1.ptr(),
                                      Bn, I, Hd, 0.0f, 1.0f, 1.0f), "layer 1 bwd");
    };
    double gpu_us = 0, wall_us = 0, gpu4_us = 0, wall4_us = 0;
    time_steps(step, steps, warmup, gpu_us, wall_us);
    time_steps(step4, steps, warmup, gpu4_us, wall4_us);
    // the same step captured once into a HIP graph and replayed (every
    // launch above is capture-safe once the split-K scratch has grown)
    hipStream_t cap;
    hip_check(hipStreamCreate(&cap), "stream");
    void* prev = nrs_get_stream();
    nrs_check(nrs_set_stream(cap), "set stream");
    hipGraph_t graph;
    hipGraphExec_t exec;
    hip_check(hipStreamBeginCapture(cap, hipStreamCaptureModeThreadLocal), "begin capture");
    step();
    hip_check(hipStreamEndCapture(cap, &graph), "end capture");
    hip_check(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "instantiate");
    double g_gpu = 0, g_wall = 0;
    time_steps([&] { hip_check(hipGraphLaunch(exec, cap), "graph launch"); }, steps, warmup, g_gpu, g_wall);
    hip_check(hipStreamSynchronize(cap), "sync");
    nrs_check(nrs_set_stream(prev), "set stream");
    hip_check(hipGraphExecDestroy(exec), "destroy");
    hip_check(hipGraphDestroy(graph), "destroy");
    hip_check(hipStreamDestroy(cap), "destroy");
    std::printf("{\"workload\": \"cfg2 MLP step 784-128-10 batch 256 through the C ABI\", "
                "\"calls\": 2, \"eager_gpu_us\": %.2f, \"eager_wall_us\": %.2f, "
                "\"graph_gpu_us\": %.2f, \"graph_wall_us\": %.2f, "
                "\"four_call_gpu_us\": %.2f, \"four_call_wall_us\": %.2f, \"steps\": %d}\n",
                gpu_us, wall_us, g_gpu, g_wall, gpu4_us, wall4_us, steps);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s {block|mlp|cnn} [steps] [warmup]\n", argv[0]);
        return 2;
    }
    const int steps = argc > 2 ? std::atoi(argv[2]) : 20;
    const int warmup = argc > 3 ? std::atoi(argv[3]) : 5;
    nrs_check(nrs_init(0), "init");
    if (!std::strcmp(argv[1], "block")) return bench_block(steps, warmup);
    if (!std::strcmp(argv[1], "mlp")) return bench_mlp(steps, warmup);
    if (!std::strcmp(argv[1], "cnn")) return bench_cnn(steps, warmup);
    std::fprintf(stderr, "unknown workload %s\n", argv[1]);
    return 2;
}
