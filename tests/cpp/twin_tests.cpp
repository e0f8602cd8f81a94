// GPU-vs-CPU twin tests of the C++ host layer (neuralrs_amd/csrc/host),
// restating the reference's tests/cuda_*_test.rs: the same deterministic
// inputs `(i % p) * s - o`, the same seeded upstream gradient, backward_graph,
// and the same absolute tolerances. The CPU side is the oracle's C
// restatement of the reference's CPU ops (liboracle.so), composed the way the
// reference's CPU autograd composes them.
//
// Usage: twin_tests [name-substring]. Prints one "PASS <name>" or
// "FAIL <name>: <reason>" line per test; exit status 1 if any failed.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <sstream>
#include <string>
#include <vector>

#include "neuralrs.hpp"

extern "C" {
void orc_graph_matmul_forward(const float*, const float*, float*, int64_t, int64_t, int64_t);
void orc_graph_matmul_backward(const float*, const float*, const float*, float*, float*, int64_t,
                               int64_t, int64_t);
void orc_graph_bmm_forward(const float*, const float*, float*, int64_t, int64_t, int64_t, int64_t);
void orc_graph_bmm_backward(const float*, const float*, const float*, float*, float*, int64_t,
                            int64_t, int64_t, int64_t);
void orc_graph_add_bias_forward(const float*, const float*, float*, int64_t, int64_t);
void orc_graph_add_bias_backward(const float*, float*, float*, int64_t, int64_t);
void orc_conv2d_im2col(const float*, const float*, const float*, float*, int64_t, int64_t, int64_t,
                       int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int);
void orc_conv2d_forward(const float*, const float*, const float*, float*, int64_t, int64_t, int64_t,
                        int64_t, int64_t, int64_t, int64_t, int64_t, int64_t);
void orc_conv2d_backward(const float*, const float*, const float*, float*, float*, float*, int64_t,
                         int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t);
void orc_transpose(const float*, float*, int64_t, int64_t, int64_t);
void orc_transpose_backward(const float*, float*, int64_t, int64_t, int64_t);
void orc_scale(const float*, float*, float, int64_t);
void orc_scale_backward(const float*, float*, float, int64_t);
void orc_softmax_forward(const float*, float*, int64_t, int64_t);
void orc_softmax_backward(const float*, const float*, float*, int64_t, int64_t);
void orc_relu_forward(const float*, float*, int64_t);
float orc_cross_entropy_loss(const float*, const float*, int64_t, int64_t);
void orc_cross_entropy_grad(const float*, const float*, float*, int64_t, int64_t);
void orc_relu_backward(const float*, const float*, float*, int64_t);
void orc_maxpool_forward(const float*, float*, int32_t*, int64_t, int64_t, int64_t, int64_t, int64_t,
                         int64_t);
void orc_maxpool_backward(const float*, const int32_t*, float*, int64_t);
void orc_slice_cols(const float*, float*, int64_t, int64_t, int64_t, int64_t);
void orc_slice_cols_backward(const float*, float*, int64_t, int64_t, int64_t, int64_t);
void orc_concat_part(const float*, float*, int64_t, int64_t, int64_t, int64_t);
void orc_concat_part_backward(const float*, float*, int64_t, int64_t, int64_t, int64_t);
void orc_layernorm_forward(const float*, const float*, const float*, float*, float*, float*,
                           int64_t, int64_t, float);
void orc_layernorm_backward(const float*, const float*, const float*, const float*, float*,
                            float*, float*, int64_t, int64_t);
}

using namespace neuralrs;
namespace gpu = neuralrs::hip::runtime;
using Vec = std::vector<float>;

struct Failure : std::runtime_error {
    explicit Failure(const std::string& m) : std::runtime_error(m) {}
};

// (i % p) as f32 * s + o, evaluated in f32 like the Rust tests.
Vec formula(size_t n, int p, float s, float o) {
    Vec v(n);
    for (size_t i = 0; i < n; ++i) v[i] = static_cast<float>(static_cast<int>(i % p)) * s + o;
    return v;
}

// tests/cuda_assembly_test.rs:9-14 `close`: |gpu - cpu| < tol elementwise.
void close(const Vec& g, const Vec& c, float tol, const std::string& what) {
    if (g.size() != c.size()) {
        std::ostringstream m;
        m << what << ": length mismatch " << g.size() << " vs " << c.size();
        throw Failure(m.str());
    }
    for (size_t i = 0; i < g.size(); ++i)
        if (!(std::fabs(g[i] - c[i]) < tol)) {
            std::ostringstream m;
            m << what << " [" << i << "]: gpu " << g[i] << " cpu " << c[i] << " (tol " << tol << ")";
            throw Failure(m.str());
        }
}

NodeRef resident(const Vec& d, std::vector<size_t> shape) {
    NodeRef n = Node::create(d, std::move(shape));
    gpu::to_cuda(n);
    return n;
}

// ------------------------------------------------------ CPU compositions
struct CpuMatmul {  // autograd::graph::matmul forward + backward
    Vec c, da, db;
    CpuMatmul(const Vec& a, const Vec& b, const Vec& seed, size_t m, size_t k, size_t n)
        : c(m * n), da(m * k, 0.0f), db(k * n, 0.0f) {
        orc_graph_matmul_forward(a.data(), b.data(), c.data(), m, k, n);
        orc_graph_matmul_backward(a.data(), b.data(), seed.data(), da.data(), db.data(), m, k, n);
    }
};

// CPU attention_batch (src/nn/attention.rs:26-39) on [batch, seq, d]; batch = 1
// gives the single-sequence attention (matmul == bmm with one item).
struct CpuAttention {
    Vec out, dq, dk, dv;
    CpuAttention(const Vec& q, const Vec& k, const Vec& v, const Vec& seed, size_t B, size_t S,
                 size_t D) {
        const float s = 1.0f / std::sqrt(static_cast<float>(D));
        Vec kt(B * S * D), scores(B * S * S), scaled(B * S * S), w(B * S * S);
        out.assign(B * S * D, 0.0f);
        orc_transpose(k.data(), kt.data(), B, S, D);
        orc_graph_bmm_forward(q.data(), kt.data(), scores.data(), B, S, D, S);
        orc_scale(scores.data(), scaled.data(), s, B * S * S);
        orc_softmax_forward(scaled.data(), w.data(), B * S, S);
        orc_graph_bmm_forward(w.data(), v.data(), out.data(), B, S, S, D);
        Vec dw(B * S * S, 0.0f), dscaled(B * S * S, 0.0f), dscores(B * S * S, 0.0f),
            dkt(B * S * D, 0.0f);
        dq.assign(B * S * D, 0.0f);
        dk.assign(B * S * D, 0.0f);
        dv.assign(B * S * D, 0.0f);
        orc_graph_bmm_backward(w.data(), v.data(), seed.data(), dw.data(), dv.data(), B, S, S, D);
        orc_softmax_backward(w.data(), dw.data(), dscaled.data(), B * S, S);
        orc_scale_backward(dscaled.data(), dscores.data(), s, B * S * S);
        orc_graph_bmm_backward(q.data(), kt.data(), dscores.data(), dq.data(), dkt.data(), B, S, D, S);
        orc_transpose_backward(dkt.data(), dk.data(), B, S, D);
    }
};

// ------------------------------------------------------------------ tests
// tests/cuda_matmul_resident_test.rs:9-45
void cuda_resident_matmul_backward() {
    const size_t m = 40, k = 56, n = 32;
    Vec a = formula(m * k, 13, 0.1f, -0.6f), b = formula(k * n, 7, 0.2f, -0.6f);
    Vec seed = formula(m * n, 5, 0.2f, 0.1f);
    CpuMatmul cpu(a, b, seed, m, k, n);
    NodeRef ga = resident(a, {m, k}), gb = resident(b, {k, n});
    NodeRef gc = hip::graph::matmul(ga, gb);
    Vec gc_data = gpu::to_host(gc);
    gpu::set_grad(gc, seed);
    backward_graph(gc);
    close(gc_data, cpu.c, 1e-3f, "fwd");
    close(gpu::read_grad(ga), cpu.da, 1e-3f, "a.grad");
    close(gpu::read_grad(gb), cpu.db, 1e-3f, "b.grad");
}

// tests/cuda_linear_test.rs:9-54: add(matmul(x, w), bias)
void cuda_resident_linear_chain() {
    const size_t batch = 16, in_f = 24, out_f = 10;
    Vec x = formula(batch * in_f, 17, 0.1f, -0.8f), w = formula(in_f * out_f, 13, 0.05f, -0.3f);
    Vec bias = formula(out_f, 5, 0.2f, -0.4f), seed = formula(batch * out_f, 7, 0.2f, 0.1f);
    Vec mm(batch * out_f), y(batch * out_f), dmm(batch * out_f, 0.0f), db(out_f, 0.0f);
    Vec dx(batch * in_f, 0.0f), dw(in_f * out_f, 0.0f);
    orc_graph_matmul_forward(x.data(), w.data(), mm.data(), batch, in_f, out_f);
    orc_graph_add_bias_forward(mm.data(), bias.data(), y.data(), batch, out_f);
    orc_graph_add_bias_backward(seed.data(), dmm.data(), db.data(), batch, out_f);
    orc_graph_matmul_backward(x.data(), w.data(), dmm.data(), dx.data(), dw.data(), batch, in_f, out_f);

    NodeRef gx = resident(x, {batch, in_f}), gw = resident(w, {in_f, out_f});
    NodeRef gb = resident(bias, {out_f});
    NodeRef gy = hip::graph::add(hip::graph::matmul(gx, gw), gb);
    Vec gy_data = gpu::to_host(gy);
    gpu::set_grad(gy, seed);
    backward_graph(gy);
    close(gy_data, y, 1e-3f, "fwd");
    close(gpu::read_grad(gx), dx, 1e-3f, "x.grad");
    close(gpu::read_grad(gw), dw, 1e-3f, "w.grad");
    close(gpu::read_grad(gb), db, 1e-3f, "bias.grad");
}

// tests/cuda_ce_test.rs:10-58: cross-entropy of add(matmul(x, w), bias)
// against one-hot rows, loss and gradients through the Linear
void cuda_cross_entropy_through_linear() {
    const size_t batch = 16, in_f = 24, classes = 10;
    Vec x = formula(batch * in_f, 17, 0.1f, -0.8f), w = formula(in_f * classes, 13, 0.05f, -0.3f);
    Vec bias = formula(classes, 5, 0.2f, -0.4f), target(batch * classes, 0.0f);
    for (size_t b = 0; b < batch; ++b) target[b * classes + b % classes] = 1.0f;
    Vec mm(batch * classes), logits(batch * classes), seed(batch * classes);
    Vec dmm(batch * classes, 0.0f), db(classes, 0.0f), dx(batch * in_f, 0.0f), dw(in_f * classes, 0.0f);
    orc_graph_matmul_forward(x.data(), w.data(), mm.data(), batch, in_f, classes);
    orc_graph_add_bias_forward(mm.data(), bias.data(), logits.data(), batch, classes);
    const float cpu_loss = orc_cross_entropy_loss(logits.data(), target.data(), batch, classes);
    orc_cross_entropy_grad(logits.data(), target.data(), seed.data(), batch, classes);
    orc_graph_add_bias_backward(seed.data(), dmm.data(), db.data(), batch, classes);
    orc_graph_matmul_backward(x.data(), w.data(), dmm.data(), dx.data(), dw.data(), batch, in_f, classes);

    NodeRef gx = resident(x, {batch, in_f}), gw = resident(w, {in_f, classes});
    NodeRef gb = resident(bias, {classes}), gt = resident(target, {batch, classes});
    NodeRef glogits = hip::graph::add(hip::graph::matmul(gx, gw), gb);
    const float gpu_loss = hip::loss::cross_entropy(glogits, gt);
    hip::loss::cross_entropy_backward(glogits, gt);
    backward_graph(glogits);
    if (!(std::fabs(gpu_loss - cpu_loss) < 1e-3f))
        throw std::runtime_error("ce loss: gpu " + std::to_string(gpu_loss) + " cpu " +
                                 std::to_string(cpu_loss));
    close(gpu::read_grad(gx), dx, 1e-3f, "x.grad");
    close(gpu::read_grad(gw), dw, 1e-3f, "w.grad");
    close(gpu::read_grad(gb), db, 1e-3f, "bias.grad");
}

// tests/cuda_assembly_test.rs:17-56: nn::Linear (fused bias epilogue here)
void cuda_linear() {
    const size_t batch = 3, in_d = 4, out_d = 5;
    Vec x = formula(batch * in_d, 11, 0.1f, -0.5f), w = formula(in_d * out_d, 13, 0.1f, -0.6f);
    Vec b = formula(out_d, 5, 0.1f, -0.2f), seed = formula(batch * out_d, 6, 0.1f, 0.2f);
    Vec mm(batch * out_d), y(batch * out_d), dmm(batch * out_d, 0.0f), db(out_d, 0.0f);
    Vec dx(batch * in_d, 0.0f), dw(in_d * out_d, 0.0f);
    orc_graph_matmul_forward(x.data(), w.data(), mm.data(), batch, in_d, out_d);
    orc_graph_add_bias_forward(mm.data(), b.data(), y.data(), batch, out_d);
    orc_graph_add_bias_backward(seed.data(), dmm.data(), db.data(), batch, out_d);
    orc_graph_matmul_backward(x.data(), w.data(), dmm.data(), dx.data(), dw.data(), batch, in_d, out_d);

    NodeRef gw = resident(w, {in_d, out_d}), gb = resident(b, {out_d});
    hip::nn::Linear lin(gw, gb);
    NodeRef gx = resident(x, {batch, in_d});
    NodeRef gout = lin.forward(gx);
    Vec gf = gpu::to_host(gout);
    gpu::set_grad(gout, seed);
    backward_graph(gout);
    close(gf, y, 1e-4f, "linear fwd");
    close(gpu::read_grad(gw), dw, 1e-4f, "linear dw");
    close(gpu::read_grad(gb), db, 1e-4f, "linear db");
    close(gpu::read_grad(gx), dx, 1e-4f, "linear dx");
}

// tests/cuda_conv2d_test.rs:15-43
void cuda_conv2d_forward() {
    const size_t n = 2, c_in = 3, in_h = 8, in_w = 8, c_out = 4, kh = 3, kw = 3, stride = 1, pad = 1;
    Vec input = formula(n * c_in * in_h * in_w, 23, 0.05f, -0.5f);
    Vec weight = formula(c_out * c_in * kh * kw, 13, 0.07f, -0.4f);
    Vec bias = formula(c_out, 5, 0.1f, -0.2f);
    const size_t oh = (in_h + 2 * pad - kh) / stride + 1, ow = (in_w + 2 * pad - kw) / stride + 1;
    Vec cpu_out(n * c_out * oh * ow);
    orc_conv2d_im2col(input.data(), weight.data(), bias.data(), cpu_out.data(), n, c_in, c_out,
                      in_h, in_w, kh, kw, stride, pad, 1);
    NodeRef gi = resident(input, {n, c_in, in_h, in_w});
    NodeRef gw = resident(weight, {c_out, c_in, kh, kw});
    NodeRef gb = resident(bias, {c_out});
    NodeRef gout = hip::nn::conv2d(gi, gw, gb, stride, pad);
    if (gout->shape != std::vector<size_t>{n, c_out, oh, ow}) throw Failure("output shape");
    close(gpu::to_host(gout), cpu_out, 1e-4f, "conv");
}

// tests/cuda_conv2d_test.rs:46-96, plus the stride-2 and no-input-grad cases.
void conv_backward_case(size_t n, size_t c_in, size_t in_h, size_t in_w, size_t c_out, size_t k,
                        size_t stride, size_t pad, bool input_grad) {
    Vec input = formula(n * c_in * in_h * in_w, 23, 0.05f, -0.5f);
    Vec weight = formula(c_out * c_in * k * k, 13, 0.07f, -0.4f);
    Vec bias = formula(c_out, 5, 0.1f, -0.2f);
    const size_t oh = (in_h + 2 * pad - k) / stride + 1, ow = (in_w + 2 * pad - k) / stride + 1;
    const size_t out_len = n * c_out * oh * ow;
    Vec seed = formula(out_len, 7, 0.2f, 0.1f);
    Vec cpu_out(out_len), c_ig(input.size(), 0.0f), c_wg(weight.size(), 0.0f), c_bg(c_out, 0.0f);
    orc_conv2d_forward(input.data(), weight.data(), bias.data(), cpu_out.data(), n, c_in, c_out,
                       in_h, in_w, k, k, stride, pad);
    orc_conv2d_backward(input.data(), weight.data(), seed.data(), c_ig.data(), c_wg.data(),
                        c_bg.data(), n, c_in, c_out, in_h, in_w, k, k, stride, pad);
    NodeRef gi = resident(input, {n, c_in, in_h, in_w});
    gi->requires_grad = input_grad;
    NodeRef gw = resident(weight, {c_out, c_in, k, k});
    NodeRef gb = resident(bias, {c_out});
    NodeRef gout = hip::nn::conv2d(gi, gw, gb, stride, pad);
    close(gpu::to_host(gout), cpu_out, 1e-4f, "conv fwd");
    gpu::set_grad(gout, seed);
    backward_graph(gout);
    close(gpu::read_grad(gi), input_grad ? c_ig : Vec(input.size(), 0.0f), 1e-3f, "input.grad");
    close(gpu::read_grad(gw), c_wg, 1e-3f, "weight.grad");
    close(gpu::read_grad(gb), c_bg, 1e-3f, "bias.grad");
}

void cuda_conv2d_backward() { conv_backward_case(2, 3, 7, 7, 5, 3, 1, 1, true); }
void cuda_conv2d_backward_stride2() { conv_backward_case(2, 3, 9, 9, 4, 3, 2, 1, true); }
void cuda_conv2d_backward_no_input_grad() { conv_backward_case(2, 3, 7, 7, 5, 3, 1, 1, false); }

// tests/cuda_manip_test.rs:38-48
void cuda_transpose() {
    const size_t b = 2, r = 3, c = 4;
    Vec input = formula(b * r * c, 11, 0.1f, -0.5f), seed = formula(b * r * c, 7, 0.1f, 0.2f);
    Vec cf(b * r * c), cg(b * r * c, 0.0f);
    orc_transpose(input.data(), cf.data(), b, r, c);
    orc_transpose_backward(seed.data(), cg.data(), b, r, c);
    NodeRef x = resident(input, {b, r, c});
    NodeRef out = hip::graph::transpose(x);
    Vec gf = gpu::to_host(out);
    gpu::set_grad(out, seed);
    backward_graph(out);
    close(gf, cf, 1e-5f, "transpose fwd");
    close(gpu::read_grad(x), cg, 1e-5f, "transpose grad");
}

// tests/cuda_manip_test.rs:64-74
void cuda_softmax() {
    const size_t rows = 4, width = 5;
    Vec input = formula(rows * width, 9, 0.3f, -1.0f), seed = formula(rows * width, 7, 0.1f, 0.2f);
    Vec cf(rows * width), cg(rows * width, 0.0f);
    orc_softmax_forward(input.data(), cf.data(), rows, width);
    orc_softmax_backward(cf.data(), seed.data(), cg.data(), rows, width);
    NodeRef x = resident(input, {rows, width});
    NodeRef out = hip::graph::softmax(x);
    Vec gf = gpu::to_host(out);
    gpu::set_grad(out, seed);
    backward_graph(out);
    close(gf, cf, 1e-4f, "softmax fwd");
    close(gpu::read_grad(x), cg, 1e-4f, "softmax grad");
}

// tests/cuda_manip_test.rs:76-104
void cuda_bmm() {
    const size_t batch = 2, m = 3, k = 4, n = 5;
    Vec a = formula(batch * m * k, 11, 0.1f, -0.5f), bb = formula(batch * k * n, 13, 0.1f, -0.6f);
    Vec seed = formula(batch * m * n, 7, 0.1f, 0.2f);
    Vec cf(batch * m * n), cga(a.size(), 0.0f), cgb(bb.size(), 0.0f);
    orc_graph_bmm_forward(a.data(), bb.data(), cf.data(), batch, m, k, n);
    orc_graph_bmm_backward(a.data(), bb.data(), seed.data(), cga.data(), cgb.data(), batch, m, k, n);
    NodeRef ga = resident(a, {batch, m, k}), gbn = resident(bb, {batch, k, n});
    NodeRef gout = hip::graph::bmm(ga, gbn);
    Vec gf = gpu::to_host(gout);
    gpu::set_grad(gout, seed);
    backward_graph(gout);
    close(gf, cf, 1e-4f, "bmm fwd");
    close(gpu::read_grad(ga), cga, 1e-4f, "bmm grad_a");
    close(gpu::read_grad(gbn), cgb, 1e-4f, "bmm grad_b");
}

void attention_case(size_t B, size_t S, size_t D, bool batched, float tol, Vec q, Vec k, Vec v,
                    Vec seed) {
    CpuAttention cpu(q, k, v, seed, B, S, D);
    std::vector<size_t> shape = batched ? std::vector<size_t>{B, S, D} : std::vector<size_t>{S, D};
    NodeRef gq = resident(q, shape), gk = resident(k, shape), gv = resident(v, shape);
    NodeRef gout = batched ? hip::nn::attention_batch(gq, gk, gv) : hip::nn::attention(gq, gk, gv);
    Vec gf = gpu::to_host(gout);
    gpu::set_grad(gout, seed);
    backward_graph(gout);
    close(gf, cpu.out, tol, "attention fwd");
    close(gpu::read_grad(gq), cpu.dq, tol, "attention dq");
    close(gpu::read_grad(gk), cpu.dk, tol, "attention dk");
    close(gpu::read_grad(gv), cpu.dv, tol, "attention dv");
}

// tests/cuda_composite_test.rs:16-48
void cuda_attention() {
    const size_t S = 4, D = 6;
    attention_case(1, S, D, false, 1e-3f, formula(S * D, 11, 0.1f, -0.5f),
                   formula(S * D, 13, 0.1f, -0.6f), formula(S * D, 7, 0.1f, -0.3f),
                   formula(S * D, 5, 0.1f, 0.2f));
}

// tests/cuda_composite_test.rs:50-82
void cuda_attention_batch() {
    const size_t B = 2, S = 3, D = 4, n = B * S * D;
    attention_case(B, S, D, true, 1e-3f, formula(n, 11, 0.1f, -0.5f), formula(n, 13, 0.1f, -0.6f),
                   formula(n, 7, 0.1f, -0.3f), formula(n, 5, 0.1f, 0.2f));
}

// Panics of the reference ops surface as neuralrs::Panic with its message.
void panics_on_misuse() {
    auto expect_panic = [](auto fn, const std::string& msg) {
        try {
            fn();
        } catch (const Panic& p) {
            if (std::string(p.what()).find(msg) == std::string::npos)
                throw Failure("wrong panic: " + std::string(p.what()));
            return;
        }
        throw Failure("no panic for: " + msg);
    };
    NodeRef host_only = Node::create(Vec(6, 1.0f), {2, 3});
    NodeRef r = resident(Vec(6, 1.0f), {3, 2});
    NodeRef bad = resident(Vec(8, 1.0f), {4, 2});
    expect_panic([&] { hip::graph::matmul(host_only, r); }, "cuda matmul: lhs not on GPU");
    expect_panic([&] { hip::graph::matmul(r, host_only); }, "cuda matmul: rhs not on GPU");
    expect_panic([&] { hip::graph::matmul(r, bad); }, "cuda matmul: inner dims mismatch");
    expect_panic([&] { gpu::to_host(host_only); }, "to_host: node is not on the GPU");
    expect_panic([&] { gpu::read_grad(host_only); }, "read_grad: node not on GPU");
}

// ------------------------------------------------ BASELINE-sized twins
std::mt19937_64& rng() {
    static std::mt19937_64 g(1234);
    return g;
}
// Each BASELINE-sized case starts from its own seed, so its inputs do not
// depend on which cases ran before it.
void reseed(uint64_t s) { rng().seed(s); }
Vec normal(size_t n, float std) {
    std::normal_distribution<float> d(0.0f, std);
    Vec v(n);
    for (float& x : v) x = d(rng());
    return v;
}
Vec uniform(size_t n, float lo, float hi) {
    std::uniform_real_distribution<float> d(lo, hi);
    Vec v(n);
    for (float& x : v) x = d(rng());
    return v;
}

// cfg2: Linear 784->128, ReLU, Linear 128->10, batch 256, He init, zero bias,
// upstream grad (softmax - onehot) / 256 from the CPU logits.
void cfg2_mlp_step() {
    reseed(2);
    const size_t B = 256, I = 784, H = 128, O = 10;
    Vec x = normal(B * I, 1.0f), w1 = normal(I * H, std::sqrt(2.0f / I));
    Vec w2 = normal(H * O, std::sqrt(2.0f / H)), b1(H, 0.0f), b2(O, 0.0f);
    Vec mm1(B * H), h1(B * H), r1(B * H), mm2(B * O), y(B * O);
    orc_graph_matmul_forward(x.data(), w1.data(), mm1.data(), B, I, H);
    orc_graph_add_bias_forward(mm1.data(), b1.data(), h1.data(), B, H);
    orc_relu_forward(h1.data(), r1.data(), B * H);
    orc_graph_matmul_forward(r1.data(), w2.data(), mm2.data(), B, H, O);
    orc_graph_add_bias_forward(mm2.data(), b2.data(), y.data(), B, O);
    Vec seed(B * O), sm(B * O);
    orc_softmax_forward(y.data(), sm.data(), B, O);
    std::uniform_int_distribution<int> cls(0, (int)O - 1);
    for (size_t r = 0; r < B; ++r) {
        const int t = cls(rng());
        for (size_t c = 0; c < O; ++c)
            seed[r * O + c] = (sm[r * O + c] - (static_cast<int>(c) == t ? 1.0f : 0.0f)) / B;
    }
    Vec dmm2(B * O, 0.0f), db2(O, 0.0f), dr1(B * H, 0.0f), dw2(H * O, 0.0f), dh1(B * H, 0.0f);
    Vec dmm1(B * H, 0.0f), db1(H, 0.0f), dx(B * I, 0.0f), dw1(I * H, 0.0f);
    orc_graph_add_bias_backward(seed.data(), dmm2.data(), db2.data(), B, O);
    orc_graph_matmul_backward(r1.data(), w2.data(), dmm2.data(), dr1.data(), dw2.data(), B, H, O);
    orc_relu_backward(h1.data(), dr1.data(), dh1.data(), B * H);
    orc_graph_add_bias_backward(dh1.data(), dmm1.data(), db1.data(), B, H);
    orc_graph_matmul_backward(x.data(), w1.data(), dmm1.data(), dx.data(), dw1.data(), B, I, H);

    NodeRef gx = resident(x, {B, I}), gw1 = resident(w1, {I, H}), gb1 = resident(b1, {H});
    NodeRef gw2 = resident(w2, {H, O}), gb2 = resident(b2, {O});
    hip::nn::Linear l1(gw1, gb1), l2(gw2, gb2);
    NodeRef out = l2.forward(hip::graph::relu(l1.forward(gx)));
    close(gpu::to_host(out), y, 1e-3f, "cfg2 logits");
    gpu::set_grad(out, seed);
    backward_graph(out);
    close(gpu::read_grad(gw1), dw1, 1e-3f, "cfg2 dW1");
    close(gpu::read_grad(gb1), db1, 1e-3f, "cfg2 db1");
    close(gpu::read_grad(gw2), dw2, 1e-3f, "cfg2 dW2");
    close(gpu::read_grad(gb2), db2, 1e-3f, "cfg2 db2");
    close(gpu::read_grad(gx), dx, 1e-3f, "cfg2 dx");
}

// cfg4 per-head attention, heads folded into the batch: [32*8, 128, 32].
void cfg4_attention_heads() {
    reseed(4);
    const size_t B = 256, S = 128, D = 32, n = B * S * D;
    attention_case(B, S, D, true, 1e-3f, normal(n, 1.0f), normal(n, 1.0f), normal(n, 1.0f),
                   normal(n, 0.1f));
}

// cfg3 conv2 layer at a reduced batch: 32 -> 64 channels, 14x14, k3 p1.
void cfg3_conv2_layer() {
    reseed(3);
    const size_t N = 16, C = 32, H = 14, W = 14, CO = 64;
    Vec input = uniform(N * C * H * W, 0.0f, 1.0f), weight = normal(CO * C * 9, std::sqrt(2.0f / 288));
    Vec bias(CO, 0.0f), seed = normal(N * CO * H * W, 1.0f);
    Vec cpu_out(N * CO * H * W), c_ig(input.size(), 0.0f), c_wg(weight.size(), 0.0f), c_bg(CO, 0.0f);
    orc_conv2d_forward(input.data(), weight.data(), bias.data(), cpu_out.data(), N, C, CO, H, W, 3,
                       3, 1, 1);
    orc_conv2d_backward(input.data(), weight.data(), seed.data(), c_ig.data(), c_wg.data(),
                        c_bg.data(), N, C, CO, H, W, 3, 3, 1, 1);
    NodeRef gi = resident(input, {N, C, H, W}), gw = resident(weight, {CO, C, 3, 3});
    NodeRef gb = resident(bias, {CO});
    NodeRef gout = hip::nn::conv2d(gi, gw, gb, 1, 1);
    close(gpu::to_host(gout), cpu_out, 1e-4f, "cfg3 conv2 fwd");
    gpu::set_grad(gout, seed);
    backward_graph(gout);
    close(gpu::read_grad(gi), c_ig, 1e-3f, "cfg3 conv2 input.grad");
    // weight/bias grads sum N*H*W = 3136 terms of O(1): scale the tolerance.
    close(gpu::read_grad(gw), c_wg, 2e-3f, "cfg3 conv2 weight.grad");
    close(gpu::read_grad(gb), c_bg, 2e-3f, "cfg3 conv2 bias.grad");
}

struct Case {
    const char* name;
    void (*fn)();
};

// tests/cuda_manip_test.rs:49-61
void cuda_slice_cols() {
    const size_t rows = 4, total = 6, cs = 2, ce = 5, sw = ce - cs;
    const Vec input = formula(rows * total, 13, 0.1f, -0.6f);
    const Vec seed = formula(rows * sw, 5, 0.1f, 0.3f);
    Vec cf(rows * sw), cg(rows * total, 0.0f);
    orc_slice_cols(input.data(), cf.data(), rows, total, cs, ce);
    orc_slice_cols_backward(seed.data(), cg.data(), rows, total, cs, ce);
    NodeRef x = resident(input, {rows, total});
    NodeRef out = hip::graph::slice_cols(x, cs, ce);
    const Vec gf = gpu::to_host(out);
    gpu::set_grad(out, seed);
    backward_graph(out);
    close(gf, cf, 1e-5f, "slice_cols fwd");
    close(gpu::read_grad(x), cg, 1e-5f, "slice_cols grad");
}

// tests/cuda_manip_test.rs:105-141
void cuda_concat_cols() {
    const size_t rows = 4, w[3] = {2, 3, 1}, total = 6;
    const Vec p[3] = {formula(rows * w[0], 7, 0.1f, -0.3f), formula(rows * w[1], 9, 0.1f, -0.4f),
                      formula(rows * w[2], 5, 0.1f, -0.2f)};
    const Vec seed = formula(rows * total, 6, 0.1f, 0.2f);
    Vec cf(rows * total), cg[3];
    size_t off = 0;
    for (int i = 0; i < 3; ++i) {
        orc_concat_part(p[i].data(), cf.data(), rows, total, off, w[i]);
        cg[i].assign(rows * w[i], 0.0f);
        orc_concat_part_backward(seed.data(), cg[i].data(), rows, total, off, w[i]);
        off += w[i];
    }
    std::vector<NodeRef> parts;
    for (int i = 0; i < 3; ++i) parts.push_back(resident(p[i], {rows, w[i]}));
    NodeRef out = hip::graph::concat_cols(parts);
    const Vec gf = gpu::to_host(out);
    gpu::set_grad(out, seed);
    backward_graph(out);
    close(gf, cf, 1e-5f, "concat fwd");
    for (int i = 0; i < 3; ++i)
        close(gpu::read_grad(parts[i]), cg[i], 1e-5f, "concat grad" + std::to_string(i));
}

// tests/cuda_layers_test.rs:18-62
void cuda_layernorm() {
    const size_t rows = 4, F = 6;
    const float eps = 1e-5f;
    const Vec input = formula(rows * F, 13, 0.2f, -1.0f);
    const Vec gamma = formula(F, 3, 0.3f, 0.5f);
    const Vec beta = formula(F, 4, 0.1f, -0.2f);
    const Vec seed = formula(rows * F, 7, 0.1f, 0.2f);
    Vec cf(rows * F), xn(rows * F), istd(rows), cdin(rows * F, 0.0f), cdg(F, 0.0f), cdb(F, 0.0f);
    orc_layernorm_forward(input.data(), gamma.data(), beta.data(), cf.data(), xn.data(),
                          istd.data(), rows, F, eps);
    orc_layernorm_backward(seed.data(), gamma.data(), xn.data(), istd.data(), cdin.data(),
                           cdg.data(), cdb.data(), rows, F);
    NodeRef gx = resident(input, {rows, F});
    NodeRef gg = resident(gamma, {F});
    NodeRef gb = resident(beta, {F});
    NodeRef out = hip::nn::layernorm(gx, gg, gb, eps);
    const Vec gf = gpu::to_host(out);
    gpu::set_grad(out, seed);
    backward_graph(out);
    close(gf, cf, 1e-4f, "layernorm fwd");
    close(gpu::read_grad(gx), cdin, 1e-4f, "layernorm dinput");
    close(gpu::read_grad(gg), cdg, 1e-4f, "layernorm dgamma");
    close(gpu::read_grad(gb), cdb, 1e-4f, "layernorm dbeta");
}

// CPU TransformerBlock (src/nn/transformer_block.rs, multihead.rs, attention.rs,
// normalization.rs) composed from the oracle's CPU ops, forward and backward.
struct CpuTransformer {
    Vec out, dx, dwq, dwk, dwv, dwo, dg1, db1, dg2, db2, df1w, df1b, df2w, df2b;
    // relu_margin > 0: before the FFN bias is added, each column of f1b is
    // redrawn (from U(-0.1, 0.1)) until no pre-activation of that column lies
    // within relu_margin of zero, so a GPU and a CPU whose roundings differ by
    // less than the margin put every ReLU on the same side.
    CpuTransformer(const Vec& x, const Vec& wq, const Vec& wk, const Vec& wv, const Vec& wo,
                   const Vec& g1, const Vec& b1, const Vec& g2, const Vec& b2, const Vec& f1w,
                   Vec& f1b, const Vec& f2w, const Vec& f2b, const Vec& seed, size_t B,
                   size_t S, size_t D, size_t H, size_t Fd, float eps, float relu_margin = 0.0f) {
        const size_t R = B * S, dh = D / H;
        const float s = 1.0f / std::sqrt(static_cast<float>(dh));
        Vec q(R * D), k(R * D), v(R * D);
        orc_graph_matmul_forward(x.data(), wq.data(), q.data(), R, D, D);
        orc_graph_matmul_forward(x.data(), wk.data(), k.data(), R, D, D);
        orc_graph_matmul_forward(x.data(), wv.data(), v.data(), R, D, D);
        std::vector<Vec> qh(H, Vec(R * dh)), kh(H, Vec(R * dh)), vh(H, Vec(R * dh)),
            kt(H, Vec(R * dh)), w(H, Vec(B * S * S)), oh(H, Vec(R * dh));
        Vec concat(R * D);
        for (size_t h = 0; h < H; ++h) {
            orc_slice_cols(q.data(), qh[h].data(), R, D, h * dh, (h + 1) * dh);
            orc_slice_cols(k.data(), kh[h].data(), R, D, h * dh, (h + 1) * dh);
            orc_slice_cols(v.data(), vh[h].data(), R, D, h * dh, (h + 1) * dh);
            Vec scores(B * S * S), scaled(B * S * S);
            orc_transpose(kh[h].data(), kt[h].data(), B, S, dh);
            orc_graph_bmm_forward(qh[h].data(), kt[h].data(), scores.data(), B, S, dh, S);
            orc_scale(scores.data(), scaled.data(), s, B * S * S);
            orc_softmax_forward(scaled.data(), w[h].data(), B * S, S);
            orc_graph_bmm_forward(w[h].data(), vh[h].data(), oh[h].data(), B, S, S, dh);
            orc_concat_part(oh[h].data(), concat.data(), R, D, h * dh, dh);
        }
        Vec ao(R * D), x1a(R * D), x1(R * D), xn1(R * D), is1(R);
        orc_graph_matmul_forward(concat.data(), wo.data(), ao.data(), R, D, D);
        for (size_t i = 0; i < R * D; ++i) x1a[i] = x[i] + ao[i];
        orc_layernorm_forward(x1a.data(), g1.data(), b1.data(), x1.data(), xn1.data(), is1.data(),
                              R, D, eps);
        Vec h1p(R * Fd), h1(R * Fd), hr(R * Fd), f2p(R * D), f(R * D), x2(R * D), xn2(R * D), is2(R);
        orc_graph_matmul_forward(x1.data(), f1w.data(), h1p.data(), R, D, Fd);
        if (relu_margin > 0.0f) {
            std::uniform_real_distribution<float> draw(-0.1f, 0.1f);
            for (size_t j = 0; j < Fd; ++j)
                for (int tries = 0;; ++tries) {
                    bool clear = true;
                    for (size_t i = 0; i < R && clear; ++i)
                        clear = std::fabs(h1p[i * Fd + j] + f1b[j]) >= relu_margin;
                    if (clear) break;
                    if (tries == 1000) throw Failure("no FFN bias clears the ReLU margin");
                    f1b[j] = draw(rng());
                }
        }
        orc_graph_add_bias_forward(h1p.data(), f1b.data(), h1.data(), R, Fd);
        orc_relu_forward(h1.data(), hr.data(), R * Fd);
        orc_graph_matmul_forward(hr.data(), f2w.data(), f2p.data(), R, Fd, D);
        orc_graph_add_bias_forward(f2p.data(), f2b.data(), f.data(), R, D);
        for (size_t i = 0; i < R * D; ++i) x2[i] = x1[i] + f[i];
        out.assign(R * D, 0.0f);
        orc_layernorm_forward(x2.data(), g2.data(), b2.data(), out.data(), xn2.data(), is2.data(),
                              R, D, eps);
        // backward
        auto z = [](size_t n) { return Vec(n, 0.0f); };
        dx = z(R * D); dwq = z(D * D); dwk = z(D * D); dwv = z(D * D); dwo = z(D * D);
        dg1 = z(D); db1 = z(D); dg2 = z(D); db2 = z(D);
        df1w = z(D * Fd); df1b = z(Fd); df2w = z(Fd * D); df2b = z(D);
        Vec dx2 = z(R * D);
        orc_layernorm_backward(seed.data(), g2.data(), xn2.data(), is2.data(), dx2.data(),
                               dg2.data(), db2.data(), R, D);
        Vec dx1 = dx2, df2p = z(R * D), dhr = z(R * Fd), dh1 = z(R * Fd), dh1p = z(R * Fd);
        orc_graph_add_bias_backward(dx2.data(), df2p.data(), df2b.data(), R, D);
        orc_graph_matmul_backward(hr.data(), f2w.data(), df2p.data(), dhr.data(), df2w.data(), R,
                                  Fd, D);
        orc_relu_backward(h1.data(), dhr.data(), dh1.data(), R * Fd);
        orc_graph_add_bias_backward(dh1.data(), dh1p.data(), df1b.data(), R, Fd);
        orc_graph_matmul_backward(x1.data(), f1w.data(), dh1p.data(), dx1.data(), df1w.data(), R,
                                  D, Fd);
        Vec dx1a = z(R * D);
        orc_layernorm_backward(dx1.data(), g1.data(), xn1.data(), is1.data(), dx1a.data(),
                               dg1.data(), db1.data(), R, D);
        for (size_t i = 0; i < R * D; ++i) dx[i] += dx1a[i];
        Vec dconcat = z(R * D), dq = z(R * D), dk = z(R * D), dv = z(R * D);
        orc_graph_matmul_backward(concat.data(), wo.data(), dx1a.data(), dconcat.data(),
                                  dwo.data(), R, D, D);
        for (size_t h = 0; h < H; ++h) {
            Vec doh = z(R * dh), dw = z(B * S * S), dvh = z(R * dh), dsc = z(B * S * S),
                dscores = z(B * S * S), dqh = z(R * dh), dkt = z(R * dh), dkh = z(R * dh);
            orc_concat_part_backward(dconcat.data(), doh.data(), R, D, h * dh, dh);
            orc_graph_bmm_backward(w[h].data(), vh[h].data(), doh.data(), dw.data(), dvh.data(), B,
                                   S, S, dh);
            orc_softmax_backward(w[h].data(), dw.data(), dsc.data(), B * S, S);
            orc_scale_backward(dsc.data(), dscores.data(), s, B * S * S);
            orc_graph_bmm_backward(qh[h].data(), kt[h].data(), dscores.data(), dqh.data(),
                                   dkt.data(), B, S, dh, S);
            orc_transpose_backward(dkt.data(), dkh.data(), B, S, dh);
            orc_slice_cols_backward(dqh.data(), dq.data(), R, D, h * dh, (h + 1) * dh);
            orc_slice_cols_backward(dkh.data(), dk.data(), R, D, h * dh, (h + 1) * dh);
            orc_slice_cols_backward(dvh.data(), dv.data(), R, D, h * dh, (h + 1) * dh);
        }
        orc_graph_matmul_backward(x.data(), wq.data(), dq.data(), dx.data(), dwq.data(), R, D, D);
        orc_graph_matmul_backward(x.data(), wk.data(), dk.data(), dx.data(), dwk.data(), R, D, D);
        orc_graph_matmul_backward(x.data(), wv.data(), dv.data(), dx.data(), dwv.data(), R, D, D);
    }
};

// tests/cuda_transformer_test.rs:17-89: the whole block, output, input
// gradient and all twelve parameter gradients, tol 3e-3.
void cuda_transformer_block() {
    const size_t B = 2, S = 3, D = 6, H = 2, Fd = 12;
    const float eps = 1e-5f;
    auto mk = [](size_t n, size_t shift) {
        Vec v(n);
        for (size_t i = 0; i < n; ++i)
            v[i] = static_cast<float>(static_cast<int>((i + shift) % 13)) * 0.1f - 0.6f;
        return v;
    };
    const Vec wq = mk(D * D, 1), wk = mk(D * D, 2), wv = mk(D * D, 3), wo = mk(D * D, 4);
    const Vec g1 = mk(D, 5), b1 = mk(D, 6), g2 = mk(D, 7), b2 = mk(D, 8);
    const Vec f1w = mk(D * Fd, 9), f2w = mk(Fd * D, 11), f2b = mk(D, 12);
    Vec f1b = mk(Fd, 10);
    const Vec x = mk(B * S * D, 20), seed = mk(B * S * D, 30);
    CpuTransformer c(x, wq, wk, wv, wo, g1, b1, g2, b2, f1w, f1b, f2w, f2b, seed, B, S, D, H, Fd,
                     eps);
    NodeRef gwq = resident(wq, {D, D}), gwk = resident(wk, {D, D}), gwv = resident(wv, {D, D}),
            gwo = resident(wo, {D, D});
    NodeRef gg1 = resident(g1, {D}), gb1 = resident(b1, {D}), gg2 = resident(g2, {D}),
            gb2 = resident(b2, {D});
    NodeRef gf1w = resident(f1w, {D, Fd}), gf1b = resident(f1b, {Fd}),
            gf2w = resident(f2w, {Fd, D}), gf2b = resident(f2b, {D});
    hip::nn::TransformerBlock tb{hip::nn::MultiHeadAttention(gwq, gwk, gwv, gwo, D, H),
                                 hip::nn::LayerNorm(gg1, gb1, eps),
                                 hip::nn::LayerNorm(gg2, gb2, eps),
                                 hip::nn::Linear(gf1w, gf1b),
                                 hip::nn::Linear(gf2w, gf2b),
                                 D, Fd};
    NodeRef gx = resident(x, {B, S, D});
    NodeRef out = tb.forward(gx);
    const Vec gf = gpu::to_host(out);
    gpu::set_grad(out, seed);
    backward_graph(out);
    close(gf, c.out, 3e-3f, "transformer fwd");
    const NodeRef params[12] = {gwq, gwk, gwv, gwo, gg1, gb1, gg2, gb2, gf1w, gf1b, gf2w, gf2b};
    const Vec* want[12] = {&c.dwq, &c.dwk, &c.dwv, &c.dwo, &c.dg1, &c.db1,
                           &c.dg2, &c.db2, &c.df1w, &c.df1b, &c.df2w, &c.df2b};
    const char* names[12] = {"w_q", "w_k", "w_v", "w_o", "norm1.gamma", "norm1.beta",
                             "norm2.gamma", "norm2.beta", "ff1.w", "ff1.b", "ff2.w", "ff2.b"};
    for (int j = 0; j < 12; ++j)
        close(gpu::read_grad(params[j]), *want[j], 3e-3f, std::string("transformer d") + names[j]);
    close(gpu::read_grad(gx), c.dx, 3e-3f, "transformer dx");
}

// CPU MultiHeadAttention::forward_batch (src/nn/multihead.rs composed from
// the oracle's ops as the reference composes them): projections, per-head
// slice_cols, attention, concat_cols, output projection; forward and backward.
struct CpuMultiHead {
    Vec out, dx, dwq, dwk, dwv, dwo;
    CpuMultiHead(const Vec& x, const Vec& wq, const Vec& wk, const Vec& wv, const Vec& wo,
                 const Vec& seed, size_t B, size_t S, size_t D, size_t H) {
        const size_t R = B * S, dh = D / H;
        Vec q(R * D), k(R * D), v(R * D), concat(R * D, 0.0f);
        orc_graph_matmul_forward(x.data(), wq.data(), q.data(), R, D, D);
        orc_graph_matmul_forward(x.data(), wk.data(), k.data(), R, D, D);
        orc_graph_matmul_forward(x.data(), wv.data(), v.data(), R, D, D);
        std::vector<Vec> qh(H, Vec(R * dh)), kh(H, Vec(R * dh)), vh(H, Vec(R * dh));
        const Vec zero(R * dh, 0.0f);
        for (size_t h = 0; h < H; ++h) {
            orc_slice_cols(q.data(), qh[h].data(), R, D, h * dh, (h + 1) * dh);
            orc_slice_cols(k.data(), kh[h].data(), R, D, h * dh, (h + 1) * dh);
            orc_slice_cols(v.data(), vh[h].data(), R, D, h * dh, (h + 1) * dh);
            CpuAttention a(qh[h], kh[h], vh[h], zero, B, S, dh);
            orc_concat_part(a.out.data(), concat.data(), R, D, h * dh, dh);
        }
        out.assign(R * D, 0.0f);
        orc_graph_matmul_forward(concat.data(), wo.data(), out.data(), R, D, D);
        Vec dconcat(R * D, 0.0f), dq(R * D, 0.0f), dk(R * D, 0.0f), dv(R * D, 0.0f);
        dwo.assign(D * D, 0.0f);
        orc_graph_matmul_backward(concat.data(), wo.data(), seed.data(), dconcat.data(),
                                  dwo.data(), R, D, D);
        for (size_t h = 0; h < H; ++h) {
            Vec doh(R * dh, 0.0f);
            orc_concat_part_backward(dconcat.data(), doh.data(), R, D, h * dh, dh);
            CpuAttention a(qh[h], kh[h], vh[h], doh, B, S, dh);
            orc_slice_cols_backward(a.dq.data(), dq.data(), R, D, h * dh, (h + 1) * dh);
            orc_slice_cols_backward(a.dk.data(), dk.data(), R, D, h * dh, (h + 1) * dh);
            orc_slice_cols_backward(a.dv.data(), dv.data(), R, D, h * dh, (h + 1) * dh);
        }
        dx.assign(R * D, 0.0f);
        dwq.assign(D * D, 0.0f);
        dwk.assign(D * D, 0.0f);
        dwv.assign(D * D, 0.0f);
        orc_graph_matmul_backward(x.data(), wq.data(), dq.data(), dx.data(), dwq.data(), R, D, D);
        orc_graph_matmul_backward(x.data(), wk.data(), dk.data(), dx.data(), dwk.data(), R, D, D);
        orc_graph_matmul_backward(x.data(), wv.data(), dv.data(), dx.data(), dwv.data(), R, D, D);
    }
};

// MultiHeadAttention through the operator surface against the CPU composition:
// batched (x [B, S, D]) or single-sequence (x [S, D], B = 1).
void mha_case(size_t B, size_t S, size_t D, size_t H, bool batched, float tol) {
    const float a = std::sqrt(6.0f / static_cast<float>(2 * D));
    const Vec wq = uniform(D * D, -a, a), wk = uniform(D * D, -a, a), wv = uniform(D * D, -a, a),
              wo = uniform(D * D, -a, a);
    const Vec x = normal(B * S * D, 1.0f), seed = normal(B * S * D, 1.0f);
    CpuMultiHead c(x, wq, wk, wv, wo, seed, B, S, D, H);
    NodeRef gwq = resident(wq, {D, D}), gwk = resident(wk, {D, D}), gwv = resident(wv, {D, D}),
            gwo = resident(wo, {D, D});
    hip::nn::MultiHeadAttention mha(gwq, gwk, gwv, gwo, D, H);
    NodeRef gx = batched ? resident(x, {B, S, D}) : resident(x, {S, D});
    NodeRef out = batched ? mha.forward_batch(gx) : mha.forward(gx);
    close(gpu::to_host(out), c.out, tol, "mha fwd");
    gpu::set_grad(out, seed);
    backward_graph(out);
    close(gpu::read_grad(gx), c.dx, tol, "mha dx");
    close(gpu::read_grad(gwq), c.dwq, tol, "mha dw_q");
    close(gpu::read_grad(gwk), c.dwk, tol, "mha dw_k");
    close(gpu::read_grad(gwv), c.dwv, tol, "mha dw_v");
    close(gpu::read_grad(gwo), c.dwo, tol, "mha dw_o");
}

// single sequence, d_head 16: the fused node with one batch item
void mha_single_sequence_fused() {
    reseed(51);
    mha_case(1, 64, 64, 4, false, 1e-3f);
}

// d_head 8 (outside the fused path): split-heads, one attention_batch of
// heads * batch items (Q.K^T as one NT product), merge-heads
void mha_batch_split_heads() {
    reseed(52);
    mha_case(3, 20, 24, 3, true, 1e-3f);
}

// attention on [seq, d] through the fused node (batch 1, one head)
void attention_fused_2d() {
    reseed(53);
    const size_t S = 50, D = 32, n = S * D;
    attention_case(1, S, D, false, 1e-3f, normal(n, 1.0f), normal(n, 1.0f), normal(n, 1.0f),
                   normal(n, 0.1f));
}

// self-attention with one node as q, k and v: the fused backward's three
// gradients land in one buffer (through temporaries), dq + dk + dv
void attention_batch_self() {
    reseed(54);
    const size_t B = 4, S = 40, D = 32, n = B * S * D;
    const Vec x = normal(n, 1.0f), seed = normal(n, 0.1f);
    CpuAttention cpu(x, x, x, seed, B, S, D);
    NodeRef gx = resident(x, {B, S, D});
    NodeRef out = hip::nn::attention_batch(gx, gx, gx);
    close(gpu::to_host(out), cpu.out, 1e-3f, "self-attention fwd");
    gpu::set_grad(out, seed);
    backward_graph(out);
    Vec want(n);
    for (size_t i = 0; i < n; ++i) want[i] = cpu.dq[i] + cpu.dk[i] + cpu.dv[i];
    close(gpu::read_grad(gx), want, 1e-3f, "self-attention dx");
}

// Gradients over several backward passes (src/autograd/node.rs:113-151
// accumulates into every parent): parents used twice (w in matmul(w, w), h in
// relu(h) and add(r, h)) collect both contributions, a second graph over the
// same leaves adds to their gradients, zero_grad makes them read zero, and a
// third pass starts again from zero.
void grads_accumulate_and_zero() {
    const size_t m = 24, k = 16;
    const Vec x = formula(m * k, 11, 0.1f, -0.5f), w = formula(k * k, 7, 0.08f, -0.25f);
    const Vec seed = formula(k * m, 5, 0.2f, -0.4f);
    Vec p(k * k), h(m * k), r(m * k), s(m * k), t(k * m), u(k * m);
    orc_graph_matmul_forward(w.data(), w.data(), p.data(), k, k, k);
    orc_graph_matmul_forward(x.data(), p.data(), h.data(), m, k, k);
    orc_relu_forward(h.data(), r.data(), m * k);
    for (size_t i = 0; i < m * k; ++i) s[i] = r[i] + h[i];
    orc_transpose(s.data(), t.data(), 1, m, k);
    orc_scale(t.data(), u.data(), 0.5f, k * m);
    Vec dt(k * m, 0.0f), ds(m * k, 0.0f), dh(m * k, 0.0f), dp(k * k, 0.0f), dx(m * k, 0.0f),
        dw(k * k, 0.0f);
    orc_scale_backward(seed.data(), dt.data(), 0.5f, k * m);
    orc_transpose_backward(dt.data(), ds.data(), 1, m, k);
    for (size_t i = 0; i < m * k; ++i) dh[i] += ds[i];      // add: dh += ds (dr = ds)
    orc_relu_backward(h.data(), ds.data(), dh.data(), m * k);  // relu: dh += relu'(h) dr
    orc_graph_matmul_backward(x.data(), p.data(), dh.data(), dx.data(), dp.data(), m, k, k);
    orc_graph_matmul_backward(w.data(), w.data(), dp.data(), dw.data(), dw.data(), k, k, k);

    NodeRef gx = resident(x, {m, k}), gw = resident(w, {k, k});
    auto pass = [&] {
        NodeRef gp = hip::graph::matmul(gw, gw);
        NodeRef gh = hip::graph::matmul(gx, gp);
        NodeRef gs = hip::graph::add(hip::graph::relu(gh), gh);
        NodeRef out =
            hip::graph::reshape(hip::graph::scale(hip::graph::transpose(gs), 0.5f), {k * m});
        gpu::set_grad(out, seed);
        backward_graph(out);
        return gpu::to_host(out);
    };
    close(pass(), u, 1e-3f, "pass 1 fwd");
    close(gpu::read_grad(gx), dx, 1e-3f, "pass 1 x.grad");
    close(gpu::read_grad(gw), dw, 1e-3f, "pass 1 w.grad");
    pass();
    Vec dx2(dx), dw2(dw);
    for (float& v : dx2) v *= 2.0f;
    for (float& v : dw2) v *= 2.0f;
    close(gpu::read_grad(gx), dx2, 2e-3f, "pass 2 x.grad");
    close(gpu::read_grad(gw), dw2, 2e-3f, "pass 2 w.grad");
    gpu::zero_grad({gx, gw});
    close(gpu::read_grad(gx), Vec(m * k, 0.0f), 1e-30f, "zeroed x.grad");
    close(gpu::read_grad(gw), Vec(k * k, 0.0f), 1e-30f, "zeroed w.grad");
    pass();
    close(gpu::read_grad(gx), dx, 1e-3f, "pass 3 x.grad");
    close(gpu::read_grad(gw), dw, 1e-3f, "pass 3 w.grad");
}

// |gpu - cpu| <= abs_tol + rel * max|cpu| elementwise; prints the largest
// error against the scale so the margin is on record.
void close_scaled(const Vec& g, const Vec& c, float abs_tol, float rel, const std::string& what) {
    if (g.size() != c.size()) throw Failure(what + ": length mismatch");
    float cmax = 0.0f, emax = 0.0f;
    for (float v : c) cmax = std::max(cmax, std::fabs(v));
    for (size_t i = 0; i < g.size(); ++i) emax = std::max(emax, std::fabs(g[i] - c[i]));
    const float tol = abs_tol + rel * cmax;
    std::printf("INFO %s: max|err| %.3g, max|cpu| %.3g, bar %.3g\n", what.c_str(), emax, cmax, tol);
    for (size_t i = 0; i < g.size(); ++i)
        if (!(std::fabs(g[i] - c[i]) <= tol)) {
            std::ostringstream m;
            m << what << " [" << i << "]: gpu " << g[i] << " cpu " << c[i] << " (bar " << tol << ")";
            throw Failure(m.str());
        }
}

// cfg4: the whole TransformerBlock at B32 S128 d256 h8 dff1024 through the
// operator surface, x ~ N(0,1), Xavier-uniform projection and FFN weights,
// small random LayerNorm and FFN parameters around the reference's init
// (gamma 1, beta 0), upstream gradient ~ N(0,1). Bar per tensor: the
// reference's absolute 3e-3 (cuda_transformer_test.rs), although the weight
// gradients here are sums over B*S = 4096 rows with magnitudes up to ~200.
void cfg4_transformer_block() {
    reseed(44);
    const size_t B = 32, S = 128, D = 256, H = 8, Fd = 1024, R = B * S;
    const float eps = 1e-5f;
    auto xavier = [](size_t fi, size_t fo) {
        const float a = std::sqrt(6.0f / static_cast<float>(fi + fo));
        return uniform(fi * fo, -a, a);
    };
    auto around = [](size_t n, float centre) {
        Vec v = uniform(n, -0.1f, 0.1f);
        for (float& e : v) e += centre;
        return v;
    };
    const Vec wq = xavier(D, D), wk = xavier(D, D), wv = xavier(D, D), wo = xavier(D, D);
    const Vec g1 = around(D, 1.0f), b1 = around(D, 0.0f), g2 = around(D, 1.0f), b2 = around(D, 0.0f);
    const Vec f1w = xavier(D, Fd), f2w = xavier(Fd, D), f2b = around(D, 0.0f);
    Vec f1b = around(Fd, 0.0f);
    const Vec x = normal(R * D, 1.0f), seed = normal(R * D, 1.0f);
    // ReLU ties: the FFN pre-activations (K = 256 sums of the normalised
    // block input) differ between GPU and CPU by ~1e-6; one that straddles
    // zero flips a ReLU and moves the weight gradients by O(1). The CPU model
    // redraws the FFN bias of any column with a pre-activation within 1e-4 of
    // zero, so no ReLU can flip.
    CpuTransformer c(x, wq, wk, wv, wo, g1, b1, g2, b2, f1w, f1b, f2w, f2b, seed, B, S, D, H, Fd,
                     eps, 1e-4f);
    NodeRef gwq = resident(wq, {D, D}), gwk = resident(wk, {D, D}), gwv = resident(wv, {D, D}),
            gwo = resident(wo, {D, D});
    NodeRef gg1 = resident(g1, {D}), gb1 = resident(b1, {D}), gg2 = resident(g2, {D}),
            gb2 = resident(b2, {D});
    NodeRef gf1w = resident(f1w, {D, Fd}), gf1b = resident(f1b, {Fd}),
            gf2w = resident(f2w, {Fd, D}), gf2b = resident(f2b, {D});
    hip::nn::TransformerBlock tb{hip::nn::MultiHeadAttention(gwq, gwk, gwv, gwo, D, H),
                                 hip::nn::LayerNorm(gg1, gb1, eps),
                                 hip::nn::LayerNorm(gg2, gb2, eps),
                                 hip::nn::Linear(gf1w, gf1b),
                                 hip::nn::Linear(gf2w, gf2b),
                                 D, Fd};
    NodeRef gx = resident(x, {B, S, D});
    NodeRef out = tb.forward(gx);
    const Vec gf = gpu::to_host(out);
    gpu::set_grad(out, seed);
    backward_graph(out);
    const float rel = 0.0f;
    close_scaled(gf, c.out, 3e-3f, rel, "cfg4 block fwd");
    const NodeRef params[12] = {gwq, gwk, gwv, gwo, gg1, gb1, gg2, gb2, gf1w, gf1b, gf2w, gf2b};
    const Vec* want[12] = {&c.dwq, &c.dwk, &c.dwv, &c.dwo, &c.dg1, &c.db1,
                           &c.dg2, &c.db2, &c.df1w, &c.df1b, &c.df2w, &c.df2b};
    const char* names[12] = {"w_q", "w_k", "w_v", "w_o", "norm1.gamma", "norm1.beta",
                             "norm2.gamma", "norm2.beta", "ff1.w", "ff1.b", "ff2.w", "ff2.b"};
    for (int j = 0; j < 12; ++j)
        close_scaled(gpu::read_grad(params[j]), *want[j], 3e-3f, rel,
                     std::string("cfg4 block d") + names[j]);
    close_scaled(gpu::read_grad(gx), c.dx, 3e-3f, rel, "cfg4 block dx");
}

// tests/cuda_assembly_test.rs:86-131: single-head self-attention, seq 4,
// d_model 6, d_k 4, formula inputs, tol 1e-3 (the CPU side: the three
// projections and attention composed from the oracle's ops).
void cuda_self_attention() {
    const size_t S = 4, D = 6, DK = 4;
    const Vec x = formula(S * D, 11, 0.1f, -0.5f), wq = formula(D * DK, 13, 0.1f, -0.6f),
              wk = formula(D * DK, 9, 0.1f, -0.4f), wv = formula(D * DK, 7, 0.1f, -0.3f),
              seed = formula(S * DK, 6, 0.1f, 0.2f);
    Vec q(S * DK), k(S * DK), v(S * DK);
    orc_graph_matmul_forward(x.data(), wq.data(), q.data(), S, D, DK);
    orc_graph_matmul_forward(x.data(), wk.data(), k.data(), S, D, DK);
    orc_graph_matmul_forward(x.data(), wv.data(), v.data(), S, D, DK);
    CpuAttention a(q, k, v, seed, 1, S, DK);
    Vec cdx(S * D, 0.0f), cdq(D * DK, 0.0f), cdk(D * DK, 0.0f), cdv(D * DK, 0.0f);
    orc_graph_matmul_backward(x.data(), wq.data(), a.dq.data(), cdx.data(), cdq.data(), S, D, DK);
    orc_graph_matmul_backward(x.data(), wk.data(), a.dk.data(), cdx.data(), cdk.data(), S, D, DK);
    orc_graph_matmul_backward(x.data(), wv.data(), a.dv.data(), cdx.data(), cdv.data(), S, D, DK);

    NodeRef gwq = resident(wq, {D, DK}), gwk = resident(wk, {D, DK}), gwv = resident(wv, {D, DK});
    hip::nn::SelfAttention sa(gwq, gwk, gwv, D, DK);
    NodeRef gx = resident(x, {S, D});
    NodeRef gout = sa.forward(gx);
    const Vec gf = gpu::to_host(gout);
    gpu::set_grad(gout, seed);
    backward_graph(gout);
    close(gf, a.out, 1e-3f, "self_attn fwd");
    close(gpu::read_grad(gwq), cdq, 1e-3f, "self_attn dw_q");
    close(gpu::read_grad(gwk), cdk, 1e-3f, "self_attn dw_k");
    close(gpu::read_grad(gwv), cdv, 1e-3f, "self_attn dw_v");
    close(gpu::read_grad(gx), cdx, 1e-3f, "self_attn dx");
}

// tests/cuda_assembly_test.rs:133-182: MultiHeadAttention on one sequence,
// seq 4, d_model 6, 2 heads (d_head 3), formula inputs, tol 1e-3.
void cuda_multihead() {
    const size_t S = 4, D = 6, H = 2;
    const Vec x = formula(S * D, 11, 0.1f, -0.5f), wq = formula(D * D, 13, 0.1f, -0.6f),
              wk = formula(D * D, 9, 0.1f, -0.4f), wv = formula(D * D, 7, 0.1f, -0.3f),
              wo = formula(D * D, 5, 0.1f, -0.2f), seed = formula(S * D, 6, 0.1f, 0.2f);
    CpuMultiHead c(x, wq, wk, wv, wo, seed, 1, S, D, H);
    NodeRef gwq = resident(wq, {D, D}), gwk = resident(wk, {D, D}), gwv = resident(wv, {D, D}),
            gwo = resident(wo, {D, D});
    hip::nn::MultiHeadAttention mha(gwq, gwk, gwv, gwo, D, H);
    NodeRef gx = resident(x, {S, D});
    NodeRef gout = mha.forward(gx);
    const Vec gf = gpu::to_host(gout);
    gpu::set_grad(gout, seed);
    backward_graph(gout);
    close(gf, c.out, 1e-3f, "mha fwd");
    close(gpu::read_grad(gwq), c.dwq, 1e-3f, "mha dw_q");
    close(gpu::read_grad(gwk), c.dwk, 1e-3f, "mha dw_k");
    close(gpu::read_grad(gwv), c.dwv, 1e-3f, "mha dw_v");
    close(gpu::read_grad(gwo), c.dwo, 1e-3f, "mha dw_o");
    close(gpu::read_grad(gx), c.dx, 1e-3f, "mha dx");
}

// tests/cuda_maxpool_test.rs:9-39: maxpool2d against the CPU MaxPool2d
// (restated by the oracle), forward 1e-5, input gradient 1e-4.
void maxpool_case(size_t n, size_t c, size_t in_h, size_t in_w, size_t k, size_t stride) {
    const size_t in_len = n * c * in_h * in_w;
    Vec input(in_len);
    for (size_t i = 0; i < in_len; ++i)
        input[i] = static_cast<float>(static_cast<int>((i * 31 + 7) % 97)) * 0.05f - 2.0f;
    const size_t oh = (in_h - k) / stride + 1, ow = (in_w - k) / stride + 1, out_len = n * c * oh * ow;
    Vec cout(out_len), cig(in_len, 0.0f);
    std::vector<int32_t> am(out_len);
    orc_maxpool_forward(input.data(), cout.data(), am.data(), n, c, in_h, in_w, k, stride);
    const Vec seed = formula(out_len, 7, 0.2f, 0.1f);
    orc_maxpool_backward(seed.data(), am.data(), cig.data(), out_len);
    NodeRef gi = resident(input, {n, c, in_h, in_w});
    NodeRef gout = hip::nn::maxpool2d(gi, k, stride);
    if (gout->shape != std::vector<size_t>{n, c, oh, ow}) throw Failure("maxpool: output shape");
    close(gpu::to_host(gout), cout, 1e-5f, "maxpool fwd");
    gpu::set_grad(gout, seed);
    backward_graph(gout);
    close(gpu::read_grad(gi), cig, 1e-4f, "maxpool input.grad");
}
void cuda_maxpool_non_overlapping() { maxpool_case(2, 3, 8, 8, 2, 2); }
void cuda_maxpool_overlapping() { maxpool_case(2, 3, 7, 7, 3, 1); }

// cfg3 end to end at batch 128 through the operator surface, as the reference
// CNN builds it (examples/mnist_cuda_cnn.rs:125: maxpool2d(relu(conv2d(..)))):
// conv1 1->32 3x3 p1 -> ReLU -> 2x2 maxpool -> conv2 32->64 3x3 p1, forward
// and backward (the image batch requires no gradient, as at
// mnist_cuda_cnn.rs:261), against the oracle's Conv2d, ReLU and max pooling
// composed the same way. Run twice on the GPU: op by op (conv2d, relu,
// maxpool2d nodes) and with the first three as one conv2d_maxpool node; the
// two must agree bit for bit except where a conv output lands exactly on a
// ReLU or pooling tie, which the integer check of the GPU tests covers.
void cfg3_cnn_step() {
    reseed(33);
    const size_t N = 128, H = 28, W = 28, C1 = 32, C2 = 64, PH = 14, PW = 14;
    const Vec x = uniform(N * H * W, 0.0f, 1.0f);
    const Vec w1 = normal(C1 * 9, std::sqrt(2.0f / 9.0f)), b1 = normal(C1, 0.1f);
    const Vec w2 = normal(C2 * C1 * 9, std::sqrt(2.0f / 288.0f)), b2 = normal(C2, 0.1f);
    const Vec seed = normal(N * C2 * PH * PW, 1.0f);
    // CPU composition
    Vec y1(N * C1 * H * W), a1(N * C1 * H * W), p1(N * C1 * PH * PW), y2(N * C2 * PH * PW);
    std::vector<int32_t> am(N * C1 * PH * PW);
    orc_conv2d_forward(x.data(), w1.data(), b1.data(), y1.data(), N, 1, C1, H, W, 3, 3, 1, 1);
    orc_relu_forward(y1.data(), a1.data(), y1.size());
    orc_maxpool_forward(a1.data(), p1.data(), am.data(), N, C1, H, W, 2, 2);
    orc_conv2d_forward(p1.data(), w2.data(), b2.data(), y2.data(), N, C1, C2, PH, PW, 3, 3, 1, 1);
    Vec dp1(p1.size(), 0.0f), dw2(w2.size(), 0.0f), db2(C2, 0.0f), da1(a1.size(), 0.0f),
        dy1(y1.size(), 0.0f), dx(x.size(), 0.0f), dw1(w1.size(), 0.0f), db1(C1, 0.0f);
    orc_conv2d_backward(p1.data(), w2.data(), seed.data(), dp1.data(), dw2.data(), db2.data(), N,
                        C1, C2, PH, PW, 3, 3, 1, 1);
    orc_maxpool_backward(dp1.data(), am.data(), da1.data(), dp1.size());
    orc_relu_backward(y1.data(), da1.data(), dy1.data(), y1.size());
    orc_conv2d_backward(x.data(), w1.data(), dy1.data(), dx.data(), dw1.data(), db1.data(), N, 1,
                        C1, H, W, 3, 3, 1, 1);
    Vec fused_out, fused_dw1, fused_db1, fused_dw2, fused_db2;
    for (int fused = 0; fused < 2; ++fused) {
        const char* tag = fused ? "cfg3 cnn (fused conv1+relu+pool)" : "cfg3 cnn (op by op)";
        NodeRef gx = resident(x, {N, 1, H, W});
        gx->requires_grad = false;
        NodeRef gw1 = resident(w1, {C1, 1, 3, 3}), gb1 = resident(b1, {C1});
        NodeRef gw2 = resident(w2, {C2, C1, 3, 3}), gb2 = resident(b2, {C2});
        NodeRef pooled = fused ? hip::nn::conv2d_maxpool(gx, gw1, gb1, 1, 1, true, 2, 2)
                               : hip::nn::maxpool2d(
                                     hip::graph::relu(hip::nn::conv2d(gx, gw1, gb1, 1, 1)), 2, 2);
        close(gpu::to_host(pooled), p1, 1e-4f, std::string(tag) + " pooled");
        NodeRef out = hip::nn::conv2d(pooled, gw2, gb2, 1, 1);
        const Vec gout = gpu::to_host(out);
        close_scaled(gout, y2, 1e-4f, 1e-5f, std::string(tag) + " fwd");
        gpu::set_grad(out, seed);
        backward_graph(out);
        const Vec gdw1 = gpu::read_grad(gw1), gdb1 = gpu::read_grad(gb1),
                  gdw2 = gpu::read_grad(gw2), gdb2 = gpu::read_grad(gb2);
        // the parameter gradients sum N * 196 (conv2) or N * 784 (conv1)
        // terms: an absolute floor plus a relative bar on their scale
        close_scaled(gdw2, dw2, 1e-3f, 1e-5f, std::string(tag) + " conv2 weight.grad");
        close_scaled(gdb2, db2, 1e-3f, 1e-5f, std::string(tag) + " conv2 bias.grad");
        close_scaled(gdw1, dw1, 1e-3f, 1e-5f, std::string(tag) + " conv1 weight.grad");
        close_scaled(gdb1, db1, 1e-3f, 1e-5f, std::string(tag) + " conv1 bias.grad");
        if (fused) {
            close(gout, fused_out, 1e-5f, "cfg3 cnn fused vs op by op fwd");
            close_scaled(gdw1, fused_dw1, 1e-4f, 1e-6f, "cfg3 cnn fused vs op by op conv1 weight.grad");
            close_scaled(gdb1, fused_db1, 1e-4f, 1e-6f, "cfg3 cnn fused vs op by op conv1 bias.grad");
        } else {
            fused_out = gout;
            fused_dw1 = gdw1;
            fused_db1 = gdb1;
        }
    }
}

// The CNN's conv2d over a conv2d_maxpool node with a ReLU: when the conv is
// the pooled node's only consumer and the image needs no gradient, the
// backward pass runs both layers' backwards as one fused call. On small
// integers every gradient equals, bit for bit, the pass that cannot fuse
// (the image asking for its gradient) and the oracle's composition; with a
// second consumer of the pooled node the pass does not fuse and still
// matches the unfused pass.
void cfg3_fused_backward_exact() {
    reseed(47);
    const size_t N = 3, H = 28, W = 28, C1 = 32, C2 = 64, PH = 14, PW = 14;
    auto ints = [](size_t n, int lo, int hi) {
        Vec v(n);
        std::uniform_int_distribution<int> d(lo, hi);
        for (float& e : v) e = (float)d(rng());
        return v;
    };
    const Vec x = ints(N * H * W, -2, 2), w1 = ints(C1 * 9, -2, 2), b1 = ints(C1, -2, 2);
    const Vec w2 = ints(C2 * C1 * 9, -2, 2), b2 = ints(C2, -2, 2), w3 = ints(C2 * C1 * 9, -2, 2);
    const Vec seed = ints(N * C2 * PH * PW, -2, 2);
    auto same = [](const Vec& g, const Vec& c, const std::string& what) {
        if (g.size() != c.size() || std::memcmp(g.data(), c.data(), g.size() * sizeof(float)))
            throw Failure(what + ": bits differ");
    };
    for (int two_consumers = 0; two_consumers < 2; ++two_consumers) {
        Vec ref[5];
        for (int x_grad = 0; x_grad < 2; ++x_grad) {  // x_grad: the pass cannot fuse
            NodeRef gx = resident(x, {N, 1, H, W});
            gx->requires_grad = x_grad != 0;
            NodeRef gw1 = resident(w1, {C1, 1, 3, 3}), gb1 = resident(b1, {C1});
            NodeRef gw2 = resident(w2, {C2, C1, 3, 3}), gb2 = resident(b2, {C2});
            NodeRef pooled = hip::nn::conv2d_maxpool(gx, gw1, gb1, 1, 1, true, 2, 2);
            NodeRef out = hip::nn::conv2d(pooled, gw2, gb2, 1, 1);
            if (two_consumers) {
                NodeRef gw3 = resident(w3, {C2, C1, 3, 3}), gb3 = resident(Vec(C2, 0.0f), {C2});
                out = hip::graph::add(out, hip::nn::conv2d(pooled, gw3, gb3, 1, 1));
            }
            gpu::set_grad(out, seed);
            backward_graph(out);
            const Vec got[5] = {gpu::read_grad(pooled), gpu::read_grad(gw1), gpu::read_grad(gb1),
                                gpu::read_grad(gw2), gpu::read_grad(gb2)};
            const char* names[5] = {"pooled.grad", "conv1 weight.grad", "conv1 bias.grad",
                                    "conv2 weight.grad", "conv2 bias.grad"};
            for (int i = 0; i < 5; ++i) {
                if (!x_grad)
                    ref[i] = got[i];
                else
                    same(ref[i], got[i], std::string(two_consumers ? "two consumers: " : "") +
                                             "fused vs unfused " + names[i]);
            }
        }
        if (two_consumers) continue;
        // the oracle's composition on the same integers
        Vec y1(N * C1 * H * W), a1(y1.size()), p1(N * C1 * PH * PW);
        std::vector<int32_t> am(p1.size());
        orc_conv2d_forward(x.data(), w1.data(), b1.data(), y1.data(), N, 1, C1, H, W, 3, 3, 1, 1);
        orc_relu_forward(y1.data(), a1.data(), y1.size());
        orc_maxpool_forward(a1.data(), p1.data(), am.data(), N, C1, H, W, 2, 2);
        Vec dp1(p1.size(), 0.0f), dw2(w2.size(), 0.0f), db2(C2, 0.0f), da1(a1.size(), 0.0f),
            dy1(y1.size(), 0.0f), dx(x.size(), 0.0f), dw1(w1.size(), 0.0f), db1(C1, 0.0f);
        orc_conv2d_backward(p1.data(), w2.data(), seed.data(), dp1.data(), dw2.data(), db2.data(),
                            N, C1, C2, PH, PW, 3, 3, 1, 1);
        orc_maxpool_backward(dp1.data(), am.data(), da1.data(), dp1.size());
        orc_relu_backward(y1.data(), da1.data(), dy1.data(), y1.size());
        orc_conv2d_backward(x.data(), w1.data(), dy1.data(), dx.data(), dw1.data(), db1.data(), N,
                            1, C1, H, W, 3, 3, 1, 1);
        same(ref[0], dp1, "fused vs oracle pooled.grad");
        same(ref[1], dw1, "fused vs oracle conv1 weight.grad");
        same(ref[2], db1, "fused vs oracle conv1 bias.grad");
        same(ref[3], dw2, "fused vs oracle conv2 weight.grad");
        same(ref[4], db2, "fused vs oracle conv2 bias.grad");
    }
}

// runtime::swap_grad seeds a backward from a gradient already on the device:
// the same bits as set_grad's host copy; swapping back returns the seed and
// the node's own (zero) gradient; a buffer of another length panics.
void swap_grad_seed() {
    reseed(43);
    const size_t N = 4, C = 3, H = 6, W = 6, M = 5;
    const Vec x = normal(N * C * H * W, 1.0f), w = normal(M * C * 9, 0.3f), b = normal(M, 0.1f);
    const Vec seed = normal(N * M * H * W, 1.0f);
    auto same = [](const Vec& g, const Vec& c, const std::string& what) {
        if (g.size() != c.size() || std::memcmp(g.data(), c.data(), g.size() * sizeof(float)))
            throw Failure(what + ": bits differ");
    };
    Vec ref_dx, ref_dw, ref_db;
    for (int swap = 0; swap < 2; ++swap) {
        NodeRef gx = resident(x, {N, C, H, W}), gw = resident(w, {M, C, 3, 3});
        NodeRef gb = resident(b, {M});
        NodeRef out = hip::nn::conv2d(gx, gw, gb, 1, 1);
        DeviceBuffer dseed = DeviceBuffer::from_host(seed);
        if (swap)
            gpu::swap_grad(out, dseed);
        else
            gpu::set_grad(out, seed);
        backward_graph(out);
        const Vec dx = gpu::read_grad(gx), dw = gpu::read_grad(gw), db = gpu::read_grad(gb);
        if (!swap) {
            ref_dx = dx;
            ref_dw = dw;
            ref_db = db;
            continue;
        }
        same(dx, ref_dx, "swap_grad vs set_grad: input.grad");
        same(dw, ref_dw, "swap_grad vs set_grad: weight.grad");
        same(db, ref_db, "swap_grad vs set_grad: bias.grad");
        gpu::swap_grad(out, dseed);
        same(dseed.to_host(), seed, "swap_grad: the seed comes back");
        same(gpu::read_grad(out), Vec(seed.size(), 0.0f),
             "swap_grad: the node's own gradient comes back");
        DeviceBuffer wrong(seed.size() - 1);
        bool panicked = false;
        try {
            gpu::swap_grad(out, wrong);
        } catch (const Panic& p) {
            panicked = std::string(p.what()).find("swap_grad: gradient length mismatch") !=
                       std::string::npos;
        }
        if (!panicked) throw Failure("swap_grad: no panic for a buffer of another length");
    }
}

// The conv2d_maxpool node without the ReLU (a pool over the raw conv
// output), with the image's gradient asked for: against the oracle's Conv2d
// and max pooling composed, and against the conv2d -> maxpool2d graph.
void cuda_conv2d_maxpool_node() {
    reseed(41);
    const size_t N = 3, C = 2, H = 8, W = 12, M = 5, PH = 4, PW = 6;
    const Vec x = normal(N * C * H * W, 1.0f), w = normal(M * C * 9, 0.3f), b = normal(M, 0.1f);
    const Vec seed = normal(N * M * PH * PW, 1.0f);
    Vec y(N * M * H * W), p(N * M * PH * PW);
    std::vector<int32_t> am(p.size());
    orc_conv2d_forward(x.data(), w.data(), b.data(), y.data(), N, C, M, H, W, 3, 3, 1, 1);
    orc_maxpool_forward(y.data(), p.data(), am.data(), N, M, H, W, 2, 2);
    Vec dy(y.size(), 0.0f), dx(x.size(), 0.0f), dw(w.size(), 0.0f), db(M, 0.0f);
    orc_maxpool_backward(seed.data(), am.data(), dy.data(), seed.size());
    orc_conv2d_backward(x.data(), w.data(), dy.data(), dx.data(), dw.data(), db.data(), N, C, M,
                        H, W, 3, 3, 1, 1);
    Vec first_out, first_dx, first_dw;
    for (int fused = 0; fused < 2; ++fused) {
        const char* tag = fused ? "conv2d_maxpool node" : "conv2d -> maxpool2d";
        NodeRef gx = resident(x, {N, C, H, W});
        NodeRef gw = resident(w, {M, C, 3, 3}), gb = resident(b, {M});
        NodeRef out = fused ? hip::nn::conv2d_maxpool(gx, gw, gb, 1, 1, false, 2, 2)
                            : hip::nn::maxpool2d(hip::nn::conv2d(gx, gw, gb, 1, 1), 2, 2);
        if (out->shape != std::vector<size_t>{N, M, PH, PW}) throw Failure("conv2d_maxpool: shape");
        const Vec gout = gpu::to_host(out);
        close(gout, p, 1e-4f, std::string(tag) + " fwd");
        gpu::set_grad(out, seed);
        backward_graph(out);
        const Vec gdx = gpu::read_grad(gx), gdw = gpu::read_grad(gw), gdb = gpu::read_grad(gb);
        close(gdx, dx, 1e-4f, std::string(tag) + " input.grad");
        close(gdw, dw, 1e-3f, std::string(tag) + " weight.grad");
        close(gdb, db, 1e-3f, std::string(tag) + " bias.grad");
        if (fused) {
            close(gout, first_out, 1e-6f, "conv2d_maxpool node vs graph fwd");
            close(gdx, first_dx, 1e-5f, "conv2d_maxpool node vs graph input.grad");
            close(gdw, first_dw, 1e-5f, "conv2d_maxpool node vs graph weight.grad");
        } else {
            first_out = gout;
            first_dx = gdx;
            first_dw = gdw;
        }
    }
}

// The Q, K and V projections' three matmul closures run as one
// nrs_matmul_shared_lhs_backward call (fused) give the bits of the closures
// run one by one (set_fused_backward(false)): the block's input gradient and
// all four weight gradients, at cfg4's shape (one grouped launch) and at a
// small shape (the short-GEMM kernel: the call runs the closures' sequence).
// The fused pass is also checked against the oracle's composition by
// cfg4_transformer_block.
void mha_fused_projection_backward_exact() {
    reseed(55);
    const size_t shapes[2][4] = {{32, 128, 256, 8}, {2, 12, 32, 4}};  // batch, seq, d, heads
    for (const auto& sh : shapes) {
        const size_t B = sh[0], S = sh[1], D = sh[2], Hh = sh[3], n = B * S * D;
        const Vec x = normal(n, 1.0f), seed = normal(n, 0.1f);
        Vec wv[4];
        for (Vec& w : wv) w = normal(D * D, 1.0f / std::sqrt((float)D));
        Vec ref[5];
        for (int fused = 1; fused >= 0; --fused) {
            gpu::set_fused_backward(fused != 0);
            NodeRef gx = resident(x, {B, S, D});
            NodeRef w[4];
            for (int i = 0; i < 4; ++i) w[i] = resident(wv[i], {D, D});
            const hip::nn::MultiHeadAttention mha(w[0], w[1], w[2], w[3], D, Hh);
            NodeRef out = mha.forward_batch(gx);
            gpu::set_grad(out, seed);
            backward_graph(out);
            const Vec got[5] = {gpu::read_grad(gx), gpu::read_grad(w[0]), gpu::read_grad(w[1]),
                                gpu::read_grad(w[2]), gpu::read_grad(w[3])};
            const char* names[5] = {"x.grad", "w_q.grad", "w_k.grad", "w_v.grad", "w_o.grad"};
            for (int i = 0; i < 5; ++i) {
                if (fused) {
                    ref[i] = got[i];
                } else if (ref[i].size() != got[i].size() ||
                           std::memcmp(ref[i].data(), got[i].data(), got[i].size() * sizeof(float))) {
                    gpu::set_fused_backward(true);
                    throw Failure(std::string("fused vs one by one (d ") + std::to_string(D) +
                                  "): " + names[i] + " bits differ");
                }
            }
        }
        gpu::set_fused_backward(true);
    }
}

const Case kCases[] = {
    {"cuda_resident_matmul_backward", cuda_resident_matmul_backward},
    {"cuda_resident_linear_chain", cuda_resident_linear_chain},
    {"cuda_linear", cuda_linear},
    {"cuda_cross_entropy_through_linear", cuda_cross_entropy_through_linear},
    {"cuda_conv2d_forward", cuda_conv2d_forward},
    {"cuda_conv2d_backward", cuda_conv2d_backward},
    {"cuda_conv2d_backward_stride2", cuda_conv2d_backward_stride2},
    {"cuda_conv2d_backward_no_input_grad", cuda_conv2d_backward_no_input_grad},
    {"cuda_transpose", cuda_transpose},
    {"cuda_softmax", cuda_softmax},
    {"cuda_bmm", cuda_bmm},
    {"cuda_attention", cuda_attention},
    {"cuda_attention_batch", cuda_attention_batch},
    {"panics_on_misuse", panics_on_misuse},
    {"cfg2_mlp_step", cfg2_mlp_step},
    {"cfg3_conv2_layer", cfg3_conv2_layer},
    {"cfg4_attention_heads", cfg4_attention_heads},
    {"cuda_slice_cols", cuda_slice_cols},
    {"cuda_concat_cols", cuda_concat_cols},
    {"cuda_layernorm", cuda_layernorm},
    {"cuda_transformer_block", cuda_transformer_block},
    {"cfg4_transformer_block", cfg4_transformer_block},
    {"mha_single_sequence_fused", mha_single_sequence_fused},
    {"mha_batch_split_heads", mha_batch_split_heads},
    {"attention_fused_2d", attention_fused_2d},
    {"attention_batch_self", attention_batch_self},
    {"grads_accumulate_and_zero", grads_accumulate_and_zero},
    {"cuda_self_attention", cuda_self_attention},
    {"cuda_multihead", cuda_multihead},
    {"cuda_maxpool_non_overlapping", cuda_maxpool_non_overlapping},
    {"cuda_maxpool_overlapping", cuda_maxpool_overlapping},
    {"cfg3_cnn_step", cfg3_cnn_step},
    {"cuda_conv2d_maxpool_node", cuda_conv2d_maxpool_node},
    {"swap_grad_seed", swap_grad_seed},
    {"cfg3_fused_backward_exact", cfg3_fused_backward_exact},
    {"mha_fused_projection_backward_exact", mha_fused_projection_backward_exact},
};

int main(int argc, char** argv) {
    const char* filter = argc > 1 ? argv[1] : "";
    if (!std::strcmp(filter, "--list")) {
        for (const Case& c : kCases) std::printf("%s\n", c.name);
        return 0;
    }
    int failed = 0;
    for (const Case& c : kCases) {
        if (!std::strstr(c.name, filter)) continue;
        std::printf("RUN  %s\n", c.name);
        std::fflush(stdout);
        try {
            c.fn();
            gpu::synchronize();
            std::printf("PASS %s\n", c.name);
        } catch (const std::exception& e) {
            ++failed;
            std::printf("FAIL %s: %s\n", c.name, e.what());
        }
        std::fflush(stdout);
    }
    return failed ? 1 : 0;
}
