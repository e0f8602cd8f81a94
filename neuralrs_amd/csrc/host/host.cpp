// Implementation of the C++ host layer (neuralrs.hpp) over the C ABI of
// libnrs_hip.so. Each op follows the reference op it names: same operand
// checks and panic messages, same output shape, same gradient flow.
#include <algorithm>
#include <memory>
#include <utility>

#include "neuralrs.hpp"

#include <cmath>
#include <initializer_list>
#include <unordered_map>
#include <unordered_set>

#include "nrs_hip.h"

namespace neuralrs {

namespace {

// Buffers handed out by acc_target / write_target since the last launch
// check: their memory holds a value only once that launch is enqueued.
std::vector<DeviceBuffer*>& taken_pending() {
    static std::vector<DeviceBuffer*> v;
    return v;
}

// A library call that allocates, copies or clears: the launch of an op is
// checked by check(), which settles the buffers taken for it.
void check_raw(int rc, const char* what) {
    if (rc != NRS_OK) throw Panic(std::string(what) + ": " + nrs_last_error());
}

// The launch of an op: on success the buffers taken for it hold its result;
// on failure nothing was enqueued, so they are pending zeros again.
void check(int rc, const char* what) {
    std::vector<DeviceBuffer*>& t = taken_pending();
    if (rc != NRS_OK) {
        for (DeviceBuffer* b : t) b->zero();
        t.clear();
        throw Panic(std::string(what) + ": " + nrs_last_error());
    }
    t.clear();
}

size_t product(const std::vector<size_t>& s) {
    size_t p = 1;
    for (size_t d : s) p *= d;
    return p;
}

GpuBuffers& gpu_of(const NodeRef& n, const char* msg) {
    if (!n || !n->gpu) throw Panic(msg);
    return *n->gpu;
}

// An op output: empty host data, device data, zeroed device gradient
// (the `Node::new(vec![], shape)` + `GpuBuffers{..}` pattern of every op).
NodeRef make_output(std::vector<size_t> shape, std::vector<NodeRef> parents, DeviceBuffer data) {
    NodeRef out = std::make_shared<Node>();
    const size_t len = product(shape);
    out->shape = std::move(shape);
    out->parents = std::move(parents);
    out->gpu = std::make_unique<GpuBuffers>();
    out->gpu->data = std::move(data);
    out->gpu->grad = std::make_shared<DeviceBuffer>(len, true);
    return out;
}

// accumulate_into (src/cuda/runtime.rs): dst += src over len elements. A
// destination that is still a pending zero takes a copy instead.
void accumulate_into(DeviceBuffer& dst, const float* src, size_t len) {
    if (dst.pending_zero()) {
        check(nrs_memcpy_dtod(dst.write_target(), src, len * sizeof(float)),
              "accumulate copy failed");
        return;
    }
    check(nrs_accumulate(dst.ptr(), src, len), "accumulate launch failed");
}

// The one beta of a launch that stores value + beta * old into several
// distinct buffers: 0 when all of them are pending zeros, else 1 (any pending
// zero among them is cleared first).
float joint_beta(std::initializer_list<DeviceBuffer*> bufs) {
    bool all_pending = true;
    for (DeviceBuffer* b : bufs) all_pending = all_pending && b->pending_zero();
    for (DeviceBuffer* b : bufs) {
        if (all_pending)
            b->write_target();
        else
            b->ptr();
    }
    return all_pending ? 0.0f : 1.0f;
}

// The backward closure of a bmm node (bmm.rs:93-131): both gradients
// accumulated into the parents, in one launch for small items. When a and b
// are the same node the two gradients go to one buffer, one product after the
// other.
void bmm_backward_into(int layout, const NodeRef& a, const NodeRef& b, const float* g,
                       size_t batch, size_t m, size_t k, size_t n, const char* what) {
    GpuBuffers& ag = gpu_of(a, "backward: lhs not on GPU");
    GpuBuffers& bg = gpu_of(b, "backward: rhs not on GPU");
    if (ag.grad != bg.grad) {
        const float beta = joint_beta({ag.grad.get(), bg.grad.get()});
        check(nrs_bmm_backward(layout, ag.grad->write_target(), bg.grad->write_target(), g,
                               ag.data.ptr(), bg.data.ptr(), batch, m, k, n, beta),
              what);
        return;
    }
    float beta = 1.0f;
    float* da = ag.grad->acc_target(beta);
    check(nrs_bmm_backward(layout, da, nullptr, g, ag.data.ptr(), bg.data.ptr(), batch, m, k, n,
                           beta),
          what);
    check(nrs_bmm_backward(layout, nullptr, bg.grad->ptr(), g, ag.data.ptr(), bg.data.ptr(), batch,
                           m, k, n, 1.0f),
          what);
}

// The backward closure of a matmul node (matmul.rs:418-431): dA += dC . B^T
// (matmul_nt) and dB += A^T . dC (matmul_tn), each followed by
// accumulate_into, as one grouped launch. When a and b are the same node the
// two products go to one buffer, one after the other.
void matmul_backward_into(const NodeRef& a, const NodeRef& b, const float* g, size_t m, size_t k,
                          size_t n, const char* what) {
    GpuBuffers& ag = gpu_of(a, "cuda matmul bwd: lhs not on GPU");
    GpuBuffers& bg = gpu_of(b, "cuda matmul bwd: rhs not on GPU");
    float ba = 1.0f, bb = 1.0f;
    float* da = ag.grad->acc_target(ba);
    if (ag.grad == bg.grad) {
        check(nrs_gemm(NRS_NT, da, g, bg.data.ptr(), m, k, n, ba, nullptr, NRS_EPI_NONE), what);
        check(nrs_gemm(NRS_TN, bg.grad->ptr(), ag.data.ptr(), g, k, n, m, 1.0f, nullptr,
                       NRS_EPI_NONE),
              what);
        return;
    }
    float* db = bg.grad->acc_target(bb);
    const nrs_gemm_desc d[2] = {
        {NRS_NT, da, g, bg.data.ptr(), (int64_t)m, (int64_t)k, (int64_t)n, ba, nullptr,
         NRS_EPI_NONE},
        {NRS_TN, db, ag.data.ptr(), g, (int64_t)k, (int64_t)n, (int64_t)m, bb, nullptr,
         NRS_EPI_NONE}};
    check(nrs_gemm_group(d, 2), what);
}

// Gives a matmul output node (a [m, k] . b [k, n]) its backward closure.
void set_matmul_backward(const NodeRef& node, const NodeRef& a, const NodeRef& b, size_t m,
                         size_t k, size_t n) {
    node->backward_fn = [grad = node->gpu->grad, a, b, m, k, n](const std::vector<float>&) {
        matmul_backward_into(a, b, grad->ptr(), m, k, n, "cuda matmul bwd: launch failed");
    };
}

void build_topo(const NodeRef& n, std::unordered_set<const Node*>& visited,
                std::vector<NodeRef>& topo) {
    if (!visited.insert(n.get()).second) return;
    for (const NodeRef& p : n->parents) build_topo(p, visited, topo);
    topo.push_back(n);
}

// The backward pass being run on this thread: each node's consumers in its
// graph, how many of them have yet to run (a node's gradient is complete at
// 0), its position in the topological order (closures run from the last
// position down), and the nodes whose closure has run (on its own, or
// within a fused backward).
struct BackwardPass {
    std::unordered_map<const Node*, int> consumers;
    std::unordered_map<const Node*, int> pending;
    std::unordered_map<const Node*, size_t> pos;
    std::unordered_set<const Node*> done;
};
thread_local BackwardPass* tl_pass = nullptr;
bool g_fused_backward = true;

}  // namespace

// What the backward of a conv2d_maxpool node with a ReLU needs.
struct ReluPoolConv {
    NodeRef input, weight, bias;
    std::shared_ptr<DeviceBuffer> argmax;
    size_t n, c_in, in_h, in_w, c_out, kh, kw, stride, pad, pool_k, pool_stride;
};

// ------------------------------------------------------------ DeviceBuffer
void note_pending_taken(DeviceBuffer* b) { taken_pending().push_back(b); }

DeviceBuffer::DeviceBuffer(size_t len, bool zero) : len_(len), pending_zero_(zero) {
    void* p = nullptr;
    check_raw(nrs_malloc(&p, len * sizeof(float)), "device alloc failed");
    ptr_ = static_cast<float*>(p);
}

void DeviceBuffer::clear_now() const {
    check_raw(nrs_memset_zero(ptr_, len_ * sizeof(float)), "device memset failed");
    pending_zero_ = false;
}

DeviceBuffer DeviceBuffer::from_host(const std::vector<float>& v) {
    DeviceBuffer b(v.size(), false);
    check_raw(nrs_memcpy_htod(b.ptr_, v.data(), v.size() * sizeof(float)), "htod failed");
    return b;
}

DeviceBuffer DeviceBuffer::view_of(const DeviceBuffer& src) {
    DeviceBuffer v;
    v.ptr_ = src.ptr();  // a pending zero is cleared: the view reads memory
    v.len_ = src.len_;
    v.owned_ = false;
    return v;
}

DeviceBuffer::~DeviceBuffer() {
    std::vector<DeviceBuffer*>& t = taken_pending();
    t.erase(std::remove(t.begin(), t.end(), this), t.end());
    if (ptr_ && owned_) nrs_free(ptr_);
}

DeviceBuffer::DeviceBuffer(DeviceBuffer&& o) noexcept
    : ptr_(o.ptr_), len_(o.len_), pending_zero_(o.pending_zero_), owned_(o.owned_) {
    o.ptr_ = nullptr;
    o.len_ = 0;
    o.pending_zero_ = false;
    o.owned_ = true;
}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) {
        if (ptr_ && owned_) nrs_free(ptr_);
        ptr_ = o.ptr_;
        len_ = o.len_;
        pending_zero_ = o.pending_zero_;
        owned_ = o.owned_;
        o.ptr_ = nullptr;
        o.len_ = 0;
        o.pending_zero_ = false;
        o.owned_ = true;
    }
    return *this;
}

std::vector<float> DeviceBuffer::to_host() const {
    std::vector<float> v(len_);
    if (pending_zero_) {
        check_raw(nrs_sync(), "synchronize failed");
        return v;
    }
    check_raw(nrs_memcpy_dtoh(v.data(), ptr_, len_ * sizeof(float)), "dtoh failed");
    return v;
}

void DeviceBuffer::zero() { pending_zero_ = true; }

// -------------------------------------------------------------------- Node
NodeRef Node::create(std::vector<float> data, std::vector<size_t> shape) {
    NodeRef n = std::make_shared<Node>();
    n->grad.assign(data.size(), 0.0f);
    n->data = std::move(data);
    n->shape = std::move(shape);
    return n;
}

size_t Node::numel() const { return product(shape); }

void backward_graph(const NodeRef& root) {
    std::vector<NodeRef> topo;
    std::unordered_set<const Node*> visited;
    build_topo(root, visited, topo);
    BackwardPass pass;
    for (size_t i = 0; i < topo.size(); ++i) {
        pass.pos[topo[i].get()] = i;
        for (const NodeRef& p : topo[i]->parents) ++pass.consumers[p.get()];
    }
    pass.pending = pass.consumers;
    struct Restore {
        BackwardPass* prev;
        ~Restore() { tl_pass = prev; }
    } restore{tl_pass};
    tl_pass = &pass;
    for (auto it = topo.rbegin(); it != topo.rend(); ++it) {
        // a node in `done` was run by a fused backward
        if (!pass.done.count(it->get())) {
            const std::vector<float> grad = (*it)->grad;
            if ((*it)->backward_fn) (*it)->backward_fn(grad);
            pass.done.insert(it->get());
        }
        for (const NodeRef& p : (*it)->parents) --pass.pending[p.get()];
    }
}

namespace hip {

// ----------------------------------------------------------------- runtime
namespace runtime {

void to_cuda(const NodeRef& node) {
    node->gpu = std::make_unique<GpuBuffers>();
    node->gpu->data = DeviceBuffer::from_host(node->data);
    node->gpu->grad = std::make_shared<DeviceBuffer>(node->data.size(), true);
}

std::vector<float> to_host(const NodeRef& node) {
    return gpu_of(node, "to_host: node is not on the GPU").data.to_host();
}

void set_grad(const NodeRef& node, const std::vector<float>& grad) {
    GpuBuffers& g = gpu_of(node, "set_grad: node not on GPU");
    if (grad.size() != g.data.len()) throw Panic("set_grad: gradient length mismatch");
    *g.grad = DeviceBuffer::from_host(grad);
}

void set_fused_backward(bool on) { g_fused_backward = on; }

void swap_grad(const NodeRef& node, DeviceBuffer& buf) {
    GpuBuffers& g = gpu_of(node, "swap_grad: node not on GPU");
    if (buf.len() != g.data.len()) throw Panic("swap_grad: gradient length mismatch");
    std::swap(*g.grad, buf);
}

std::vector<float> read_grad(const NodeRef& node) {
    return gpu_of(node, "read_grad: node not on GPU").grad->to_host();
}

void zero_grad(const std::vector<NodeRef>& params) {
    for (const NodeRef& p : params) gpu_of(p, "zero_grad: node not on GPU").grad->zero();
}

void synchronize() { check(nrs_sync(), "cuda synchronize failed"); }

}  // namespace runtime

// ------------------------------------------------------------------- graph
namespace graph {

NodeRef matmul(const NodeRef& a, const NodeRef& b) {
    GpuBuffers& ag = gpu_of(a, "cuda matmul: lhs not on GPU");
    GpuBuffers& bg = gpu_of(b, "cuda matmul: rhs not on GPU");
    if (a->shape.size() != 2 || b->shape.size() != 2) throw Panic("cuda matmul: operands must be 2-D");
    const size_t m = a->shape[0], k = a->shape[1], n = b->shape[1];
    if (b->shape[0] != k) throw Panic("cuda matmul: inner dims mismatch");
    DeviceBuffer out(m * n, false);
    check(nrs_gemm(NRS_NN, out.ptr(), ag.data.ptr(), bg.data.ptr(), m, n, k, 0.0f, nullptr,
                   NRS_EPI_NONE),
          "cuda matmul: launch failed");
    NodeRef node = make_output({m, n}, {a, b}, std::move(out));
    set_matmul_backward(node, a, b, m, k, n);
    return node;
}

NodeRef bmm(const NodeRef& a, const NodeRef& b) {
    GpuBuffers& ag = gpu_of(a, "cuda bmm: lhs not on GPU");
    GpuBuffers& bg = gpu_of(b, "cuda bmm: rhs not on GPU");
    if (a->shape.size() != 3 || b->shape.size() != 3) throw Panic("cuda bmm: operands must be 3-D");
    const size_t batch = a->shape[0], m = a->shape[1], k = a->shape[2], n = b->shape[2];
    if (b->shape[0] != batch || b->shape[1] != k) throw Panic("cuda bmm: shape mismatch");
    DeviceBuffer out(batch * m * n, false);
    check(nrs_bmm(NRS_NN, out.ptr(), ag.data.ptr(), bg.data.ptr(), batch, m, n, k, 0.0f),
          "cuda bmm: launch failed");
    NodeRef node = make_output({batch, m, n}, {a, b}, std::move(out));
    node->backward_fn = [grad = node->gpu->grad, a, b, batch, m, k, n](const std::vector<float>&) {
        bmm_backward_into(NRS_NN, a, b, grad->ptr(), batch, m, k, n, "cuda bmm bwd");
    };
    return node;
}

NodeRef add(const NodeRef& a, const NodeRef& b) {
    GpuBuffers& ag = gpu_of(a, "cuda add: lhs not on GPU");
    GpuBuffers& bg = gpu_of(b, "cuda add: rhs not on GPU");
    const bool broadcast =
        a->shape.size() == 2 && b->shape.size() == 1 && a->shape[1] == b->shape[0];
    const size_t len = product(a->shape);
    if (!broadcast && product(b->shape) != len) throw Panic("cuda add: shape mismatch");
    DeviceBuffer out(len, false);
    if (broadcast)
        check(nrs_bias_add(out.ptr(), ag.data.ptr(), bg.data.ptr(), a->shape[0], a->shape[1]),
              "cuda add: bias_add launch failed");
    else
        check(nrs_vadd(out.ptr(), ag.data.ptr(), bg.data.ptr(), len), "cuda add: launch failed");
    NodeRef node = make_output(a->shape, {a, b}, std::move(out));
    const size_t rows = broadcast ? a->shape[0] : 0, cols = broadcast ? a->shape[1] : 0;
    node->backward_fn = [grad = node->gpu->grad, a, b, len, broadcast, rows,
                         cols](const std::vector<float>&) {
        accumulate_into(*gpu_of(a, "backward: parent not on GPU").grad, grad->ptr(), len);
        DeviceBuffer& bgrad = *gpu_of(b, "backward: parent not on GPU").grad;
        if (broadcast) {  // bias gradient: column sums (add.rs:91-100, reduce.rs:28-43)
            float beta = 1.0f;
            float* db = bgrad.acc_target(beta);
            check(nrs_sum_axis0(db, grad->ptr(), rows, cols, beta), "sum_axis0 launch failed");
        } else {
            accumulate_into(bgrad, grad->ptr(), len);
        }
    };
    return node;
}

NodeRef transpose(const NodeRef& a) {
    GpuBuffers& ag = gpu_of(a, "cuda transpose: input not on GPU");
    const size_t nd = a->shape.size();
    if (nd < 2) throw Panic("cuda transpose: needs at least 2 dims");
    const size_t rows = a->shape[nd - 2], cols = a->shape[nd - 1], len = product(a->shape);
    const size_t batch = (rows != 0 && cols != 0) ? len / (rows * cols) : 0;
    DeviceBuffer out(len, false);
    check(nrs_transpose(out.ptr(), ag.data.ptr(), batch, rows, cols), "cuda transpose: launch failed");
    std::vector<size_t> shape = a->shape;
    shape[nd - 2] = cols;
    shape[nd - 1] = rows;
    NodeRef node = make_output(shape, {a}, std::move(out));
    node->backward_fn = [grad = node->gpu->grad, a, batch, rows, cols, len](const std::vector<float>&) {
        // the gradient is [.., cols, rows]: transpose back, then accumulate (transpose.rs:53-69)
        DeviceBuffer& agrad = *gpu_of(a, "backward: parent not on GPU").grad;
        if (agrad.pending_zero()) {  // nothing to add to: transpose straight into it
            check(nrs_transpose(agrad.write_target(), grad->ptr(), batch, cols, rows),
                  "cuda transpose bwd: launch");
            return;
        }
        DeviceBuffer tmp(len, false);
        check(nrs_transpose(tmp.ptr(), grad->ptr(), batch, cols, rows), "cuda transpose bwd: launch");
        accumulate_into(agrad, tmp.ptr(), len);
    };
    return node;
}

NodeRef scale(const NodeRef& a, float s) {
    GpuBuffers& ag = gpu_of(a, "cuda scale: input not on GPU");
    const size_t len = product(a->shape);
    DeviceBuffer out(len, false);
    check(nrs_scale(out.ptr(), ag.data.ptr(), s, len, 0.0f), "cuda scale: launch failed");
    NodeRef node = make_output(a->shape, {a}, std::move(out));
    node->backward_fn = [grad = node->gpu->grad, a, s, len](const std::vector<float>&) {
        float beta = 1.0f;
        float* ga = gpu_of(a, "backward: parent not on GPU").grad->acc_target(beta);
        check(nrs_scale(ga, grad->ptr(), s, len, beta), "cuda scale bwd: launch");
    };
    return node;
}

NodeRef softmax(const NodeRef& a) {
    GpuBuffers& ag = gpu_of(a, "cuda softmax: input not on GPU");
    if (a->shape.empty()) throw Panic("cuda softmax: scalar input");
    const size_t width = a->shape.back(), len = product(a->shape);
    const size_t rows = width ? len / width : 0;
    DeviceBuffer out(len, false);
    check(nrs_softmax_forward(out.ptr(), ag.data.ptr(), rows, width), "cuda softmax: launch failed");
    NodeRef node = make_output(a->shape, {a}, std::move(out));
    // The closure lives inside the node, so the node's own output buffer is
    // alive whenever the closure runs.
    const float* y = node->gpu->data.ptr();
    node->backward_fn = [grad = node->gpu->grad, a, y, rows, width](const std::vector<float>&) {
        float beta = 1.0f;
        float* ga = gpu_of(a, "cuda softmax bwd: input not on GPU").grad->acc_target(beta);
        check(nrs_softmax_backward(ga, y, grad->ptr(), rows, width, beta),
              "cuda softmax bwd: launch");
    };
    return node;
}

NodeRef relu(const NodeRef& a) {
    GpuBuffers& ag = gpu_of(a, "cuda relu: input not on GPU");
    const size_t len = product(a->shape);
    DeviceBuffer out(len, false);
    check(nrs_relu_forward(out.ptr(), ag.data.ptr(), len), "cuda relu: launch failed");
    NodeRef node = make_output(a->shape, {a}, std::move(out));
    node->backward_fn = [grad = node->gpu->grad, a, len](const std::vector<float>&) {
        GpuBuffers& g = gpu_of(a, "cuda relu bwd: input not on GPU");
        float beta = 1.0f;
        float* ga = g.grad->acc_target(beta);
        check(nrs_relu_backward(ga, grad->ptr(), g.data.ptr(), len, beta),
              "cuda relu bwd: launch");
    };
    return node;
}

NodeRef slice_cols(const NodeRef& a, size_t col_start, size_t col_end) {
    GpuBuffers& ag = gpu_of(a, "cuda slice_cols: input not on GPU");
    if (a->shape.empty()) throw Panic("cuda slice_cols: scalar input");
    const size_t total = a->shape.back(), len = product(a->shape);
    if (col_start > col_end || col_end > total) throw Panic("cuda slice_cols: bad column range");
    const size_t rows = total ? len / total : 0, w = col_end - col_start;
    DeviceBuffer out(rows * w, false);
    check(nrs_slice_cols(out.ptr(), ag.data.ptr(), rows, total, col_start, w),
          "cuda slice_cols: launch failed");
    std::vector<size_t> shape = a->shape;
    shape.back() = w;
    NodeRef node = make_output(shape, {a}, std::move(out));
    // slice_bwd into a zero temporary plus accumulate_into, as one pass
    node->backward_fn = [grad = node->gpu->grad, a, rows, total, col_start,
                         w](const std::vector<float>&) {
        check(nrs_slice_cols_backward(gpu_of(a, "backward: parent not on GPU").grad->ptr(),
                                      grad->ptr(), rows, total, col_start, w, 1.0f),
              "cuda slice_cols bwd: launch");
    };
    return node;
}

NodeRef concat_cols(const std::vector<NodeRef>& parts) {
    if (parts.empty()) throw Panic("cuda concat_cols: no parts");
    std::vector<size_t> widths;
    size_t total = 0;
    for (const NodeRef& p : parts) {
        gpu_of(p, "cuda concat_cols: part not on GPU");
        if (p->shape.empty()) throw Panic("cuda concat_cols: scalar part");
        widths.push_back(p->shape.back());
        total += widths.back();
    }
    const size_t rows = widths[0] ? product(parts[0]->shape) / widths[0] : 0;
    for (size_t i = 0; i < parts.size(); ++i)
        if (product(parts[i]->shape) != rows * widths[i])
            throw Panic("cuda concat_cols: parts differ in rows");
    DeviceBuffer out(rows * total, false);
    size_t off = 0;
    for (size_t i = 0; i < parts.size(); ++i) {
        check(nrs_concat_cols(out.ptr(), gpu_of(parts[i], "").data.ptr(), rows, total, off,
                              widths[i]),
              "cuda concat_cols: write launch failed");
        off += widths[i];
    }
    std::vector<size_t> shape = parts[0]->shape;
    shape.back() = total;
    NodeRef node = make_output(shape, parts, std::move(out));
    node->backward_fn = [grad = node->gpu->grad, parts, widths, rows,
                         total](const std::vector<float>&) {
        size_t off = 0;
        for (size_t i = 0; i < parts.size(); ++i) {
            check(nrs_concat_cols_backward(gpu_of(parts[i], "backward: part not on GPU").grad->ptr(),
                                           grad->ptr(), rows, total, off, widths[i], 1.0f),
                  "cuda concat_cols bwd: launch");
            off += widths[i];
        }
    };
    return node;
}

NodeRef scaled_softmax(const NodeRef& a, float s) {
    GpuBuffers& ag = gpu_of(a, "cuda softmax: input not on GPU");
    if (a->shape.empty()) throw Panic("cuda softmax: scalar input");
    const size_t width = a->shape.back(), len = product(a->shape);
    const size_t rows = width ? len / width : 0;
    DeviceBuffer out(len, false);
    check(nrs_softmax_forward_scaled(out.ptr(), ag.data.ptr(), rows, width, s),
          "cuda softmax: launch failed");
    NodeRef node = make_output(a->shape, {a}, std::move(out));
    const float* y = node->gpu->data.ptr();
    node->backward_fn = [grad = node->gpu->grad, a, y, rows, width, s](const std::vector<float>&) {
        float beta = 1.0f;
        float* ga = gpu_of(a, "cuda softmax bwd: input not on GPU").grad->acc_target(beta);
        check(nrs_softmax_backward_scaled(ga, y, grad->ptr(), rows, width, s, beta),
              "cuda softmax bwd: launch");
    };
    return node;
}

NodeRef reshape(const NodeRef& a, std::vector<size_t> shape) {
    GpuBuffers& ag = gpu_of(a, "cuda reshape: input not on GPU");
    const size_t len = product(a->shape);
    if (product(shape) != len) throw Panic("cuda reshape: element count mismatched");
    DeviceBuffer out(len, false);
    check(nrs_memcpy_dtod(out.ptr(), ag.data.ptr(), len * sizeof(float)),
          "cuda reshape: launch failed");
    NodeRef node = make_output(std::move(shape), {a}, std::move(out));
    node->backward_fn = [grad = node->gpu->grad, a, len](const std::vector<float>&) {
        accumulate_into(*gpu_of(a, "backward: parent not on GPU").grad, grad->ptr(), len);
    };
    return node;
}

}  // namespace graph

// -------------------------------------------------------------------- loss
namespace loss {
namespace {
// (batch, classes) of the logits (src/cuda/loss/cross_entropy.rs:62-67)
std::pair<size_t, size_t> batch_classes(const NodeRef& n) {
    if (n->shape.size() == 2) return {n->shape[0], n->shape[1]};
    if (n->shape.empty()) throw Panic("cuda ce: scalar logits");
    return {1, n->shape[0]};
}
}  // namespace

float cross_entropy(const NodeRef& pred, const NodeRef& target) {
    const auto [batch, classes] = batch_classes(pred);
    GpuBuffers& p = gpu_of(pred, "cuda ce: logits not on GPU");
    GpuBuffers& t = gpu_of(target, "cuda ce: target not on GPU");
    DeviceBuffer row_loss(batch, false);
    check(nrs_cross_entropy_forward(row_loss.ptr(), p.data.ptr(), t.data.ptr(), batch, classes),
          "cuda ce: forward launch failed");
    const std::vector<float> host = row_loss.to_host();
    float total = 0.0f;
    for (float v : host) total += v;
    return total / (float)batch;
}

void cross_entropy_backward(const NodeRef& pred, const NodeRef& target) {
    const auto [batch, classes] = batch_classes(pred);
    GpuBuffers& p = gpu_of(pred, "cuda ce: logits not on GPU");
    GpuBuffers& t = gpu_of(target, "cuda ce: target not on GPU");
    check(nrs_cross_entropy_backward(p.grad->write_target(), p.data.ptr(), t.data.ptr(), batch,
                                     classes),
          "cuda ce: backward launch failed");
}

}  // namespace loss

// ---------------------------------------------------------------------- nn
namespace nn {

namespace {

// The backward of conv2d over a conv2d_maxpool node with a ReLU (the
// reference CNN's conv2d(maxpool2d(relu(conv2d(x))))) together with that
// node's, as one nrs_conv2d_maxpool_relu_conv2d_backward call: when this conv
// is the pooled node's only consumer in the running pass, the pooled node's
// gradient is still a pending zero (so this conv's input gradient is all of
// it), the lower conv's input needs no gradient (conv.rs:304 skips it) and
// the gradients written are distinct buffers. The pass then skips the pooled
// node's closure. Returns false, having changed nothing, otherwise.
bool fused_relu_pool_backward(const NodeRef& input, const NodeRef& weight, const NodeRef& bias,
                              const DeviceBuffer& grad, size_t c_out, size_t kh, size_t kw,
                              size_t stride, size_t pad) {
    const ReluPoolConv* lo = input->relu_pool_conv.get();
    if (!lo || !tl_pass || !g_fused_backward || !input->requires_grad ||
        lo->input->requires_grad)
        return false;
    const auto it = tl_pass->consumers.find(input.get());
    if (it == tl_pass->consumers.end() || it->second != 1) return false;
    GpuBuffers& pg = gpu_of(input, "conv2d bwd: input not on GPU");
    GpuBuffers& wg = gpu_of(weight, "conv2d bwd: weight not on GPU");
    GpuBuffers& bg = gpu_of(bias, "conv2d bwd: bias not on GPU");
    GpuBuffers& xg = gpu_of(lo->input, "conv2d bwd: input not on GPU");
    GpuBuffers& lwg = gpu_of(lo->weight, "conv2d bwd: weight not on GPU");
    GpuBuffers& lbg = gpu_of(lo->bias, "conv2d bwd: bias not on GPU");
    if (!pg.grad->pending_zero()) return false;
    DeviceBuffer* outs[5] = {pg.grad.get(), wg.grad.get(), bg.grad.get(), lwg.grad.get(),
                             lbg.grad.get()};
    for (int i = 0; i < 5; ++i)
        for (int j = i + 1; j < 5; ++j)
            if (outs[i] == outs[j]) return false;
    // the four parameter gradients are written when all are pending zeros,
    // else added (the pending ones cleared first), as each closure would
    const float beta_p = joint_beta({outs[1], outs[2], outs[3], outs[4]});
    check(nrs_conv2d_maxpool_relu_conv2d_backward(
              pg.grad->write_target(), wg.grad->write_target(), bg.grad->write_target(),
              lwg.grad->write_target(), lbg.grad->write_target(), grad.ptr(), pg.data.ptr(),
              wg.data.ptr(), reinterpret_cast<const int32_t*>(lo->argmax->ptr()),
              xg.data.ptr(), lwg.data.ptr(), lo->n, lo->c_in, lo->in_h, lo->in_w, lo->c_out,
              lo->kh, lo->kw, lo->stride, lo->pad, lo->pool_k, lo->pool_stride, c_out, kh, kw,
              stride, pad, beta_p),
          "cuda conv2d bwd: launch failed");
    tl_pass->done.insert(input.get());
    return true;
}

}  // namespace

NodeRef conv2d(const NodeRef& input, const NodeRef& weight, const NodeRef& bias, size_t stride,
               size_t pad) {
    GpuBuffers& ig = gpu_of(input, "cuda conv2d: input not on GPU");
    GpuBuffers& wg = gpu_of(weight, "cuda conv2d: weight not on GPU");
    GpuBuffers& bg = gpu_of(bias, "cuda conv2d: bias not on GPU");
    if (input->shape.size() != 4 || weight->shape.size() != 4)
        throw Panic("cuda conv2d: input and weight must be 4-D");
    const size_t n = input->shape[0], c_in = input->shape[1], in_h = input->shape[2],
                 in_w = input->shape[3];
    const size_t c_out = weight->shape[0], kh = weight->shape[2], kw = weight->shape[3];
    if (weight->shape[1] != c_in) throw Panic("cuda conv2d: channel mismatch");
    if (product(bias->shape) != c_out) throw Panic("cuda conv2d: bias length mismatch");
    if (stride == 0 || in_h + 2 * pad < kh || in_w + 2 * pad < kw)
        throw Panic("cuda conv2d: bad stride/padding for the kernel size");
    const size_t out_h = (in_h + 2 * pad - kh) / stride + 1;
    const size_t out_w = (in_w + 2 * pad - kw) / stride + 1;
    DeviceBuffer out(n * c_out * out_h * out_w, false);
    check(nrs_conv2d_forward(out.ptr(), ig.data.ptr(), wg.data.ptr(), bg.data.ptr(), n, c_in, in_h,
                             in_w, c_out, kh, kw, stride, pad),
          "cuda conv2d: launch failed");
    NodeRef node = make_output({n, c_out, out_h, out_w}, {input, weight, bias}, std::move(out));
    node->backward_fn = [grad = node->gpu->grad, input, weight, bias, n, c_in, in_h, in_w, c_out,
                         kh, kw, stride, pad](const std::vector<float>&) {
        if (fused_relu_pool_backward(input, weight, bias, *grad, c_out, kh, kw, stride, pad))
            return;
        GpuBuffers& ig = gpu_of(input, "conv2d bwd: input not on GPU");
        GpuBuffers& wg = gpu_of(weight, "conv2d bwd: weight not on GPU");
        GpuBuffers& bg = gpu_of(bias, "conv2d bwd: bias not on GPU");
        // the input gradient is written when it is still a pending zero
        // (beta 0), else added; conv.rs:304 skips it for an input that
        // requires no gradient
        float beta = 1.0f;
        float* dinput = input->requires_grad ? ig.grad->acc_target(beta) : nullptr;
        // the parameter gradients likewise: written when both are pending
        // zeros (after zero_grad), else added
        const float beta_p = joint_beta({wg.grad.get(), bg.grad.get()});
        check(nrs_conv2d_backward_ex(dinput, wg.grad->write_target(), bg.grad->write_target(),
                                     grad->ptr(), ig.data.ptr(), wg.data.ptr(), n, c_in, in_h,
                                     in_w, c_out, kh, kw, stride, pad, beta, beta_p),
              "cuda conv2d bwd: launch failed");
    };
    return node;
}

NodeRef maxpool2d(const NodeRef& input, size_t kernel, size_t stride) {
    GpuBuffers& ig = gpu_of(input, "cuda maxpool: input not on GPU");
    if (input->shape.size() != 4) throw Panic("cuda maxpool: input must be 4-D");
    const size_t n = input->shape[0], c = input->shape[1], in_h = input->shape[2],
                 in_w = input->shape[3];
    if (kernel == 0 || stride == 0 || in_h < kernel || in_w < kernel)
        throw Panic("cuda maxpool: bad window");
    const size_t out_h = (in_h - kernel) / stride + 1, out_w = (in_w - kernel) / stride + 1;
    const size_t total = n * c * out_h * out_w;
    DeviceBuffer out(total, false);
    // the winners' flat input indices (int32, same element size as f32)
    auto argmax = std::make_shared<DeviceBuffer>(total, false);
    check(nrs_maxpool_forward(out.ptr(), reinterpret_cast<int32_t*>(argmax->write_target()),
                              ig.data.ptr(), n, c, in_h, in_w, kernel, stride),
          "cuda maxpool: forward launch failed");
    NodeRef node = make_output({n, c, out_h, out_w}, {input}, std::move(out));
    node->backward_fn = [grad = node->gpu->grad, input, argmax, n, c, in_h, in_w, kernel,
                         stride](const std::vector<float>&) {
        GpuBuffers& ig = gpu_of(input, "cuda maxpool bwd: input not on GPU");
        check(nrs_maxpool_backward(ig.grad->ptr(), grad->ptr(),
                                   reinterpret_cast<const int32_t*>(argmax->ptr()), n, c, in_h,
                                   in_w, kernel, stride),
              "cuda maxpool bwd: launch failed");
    };
    return node;
}

NodeRef conv2d_maxpool(const NodeRef& input, const NodeRef& weight, const NodeRef& bias,
                       size_t stride, size_t pad, bool relu, size_t pool_k, size_t pool_stride) {
    GpuBuffers& ig = gpu_of(input, "cuda conv2d: input not on GPU");
    GpuBuffers& wg = gpu_of(weight, "cuda conv2d: weight not on GPU");
    GpuBuffers& bg = gpu_of(bias, "cuda conv2d: bias not on GPU");
    if (input->shape.size() != 4 || weight->shape.size() != 4)
        throw Panic("cuda conv2d: input and weight must be 4-D");
    const size_t n = input->shape[0], c_in = input->shape[1], in_h = input->shape[2],
                 in_w = input->shape[3];
    const size_t c_out = weight->shape[0], kh = weight->shape[2], kw = weight->shape[3];
    if (weight->shape[1] != c_in) throw Panic("cuda conv2d: channel mismatch");
    if (product(bias->shape) != c_out) throw Panic("cuda conv2d: bias length mismatch");
    if (stride == 0 || in_h + 2 * pad < kh || in_w + 2 * pad < kw)
        throw Panic("cuda conv2d: bad stride/padding for the kernel size");
    const size_t out_h = (in_h + 2 * pad - kh) / stride + 1;
    const size_t out_w = (in_w + 2 * pad - kw) / stride + 1;
    if (pool_k == 0 || pool_stride == 0 || out_h < pool_k || out_w < pool_k)
        throw Panic("cuda maxpool: bad window");
    const size_t ph = (out_h - pool_k) / pool_stride + 1, pw = (out_w - pool_k) / pool_stride + 1;
    const size_t total = n * c_out * ph * pw;
    DeviceBuffer pooled(total, false);
    auto argmax = std::make_shared<DeviceBuffer>(total, false);
    int32_t* am = reinterpret_cast<int32_t*>(argmax->write_target());
    check(relu ? nrs_conv2d_relu_maxpool_forward(pooled.ptr(), am, nullptr, ig.data.ptr(),
                                                 wg.data.ptr(), bg.data.ptr(), n, c_in, in_h, in_w,
                                                 c_out, kh, kw, stride, pad, pool_k, pool_stride)
               : nrs_conv2d_maxpool_forward(pooled.ptr(), am, nullptr, ig.data.ptr(),
                                            wg.data.ptr(), bg.data.ptr(), n, c_in, in_h, in_w,
                                            c_out, kh, kw, stride, pad, pool_k, pool_stride),
          "cuda conv2d maxpool: launch failed");
    NodeRef node = make_output({n, c_out, ph, pw}, {input, weight, bias}, std::move(pooled));
    if (relu)
        node->relu_pool_conv = std::make_shared<const ReluPoolConv>(
            ReluPoolConv{input, weight, bias, argmax, n, c_in, in_h, in_w, c_out, kh, kw, stride,
                         pad, pool_k, pool_stride});
    Node* self = node.get();
    node->backward_fn = [grad = node->gpu->grad, self, input, weight, bias, argmax, relu, n, c_in,
                         in_h, in_w, c_out, kh, kw, stride, pad, pool_k,
                         pool_stride](const std::vector<float>&) {
        GpuBuffers& ig = gpu_of(input, "conv2d bwd: input not on GPU");
        GpuBuffers& wg = gpu_of(weight, "conv2d bwd: weight not on GPU");
        GpuBuffers& bg = gpu_of(bias, "conv2d bwd: bias not on GPU");
        float* dinput = input->requires_grad ? ig.grad->ptr() : nullptr;  // conv.rs:304
        const int32_t* am = reinterpret_cast<const int32_t*>(argmax->ptr());
        // the ReLU's gate reads the node's own pooled values (its data); the
        // parameter gradients are written when both are pending zeros
        if (relu) {
            const float beta_p = joint_beta({wg.grad.get(), bg.grad.get()});
            check(nrs_maxpool_relu_conv2d_backward(
                      dinput, wg.grad->write_target(), bg.grad->write_target(), grad->ptr(), am,
                      self->gpu->data.ptr(), ig.data.ptr(), wg.data.ptr(), n, c_in, in_h, in_w,
                      c_out, kh, kw, stride, pad, pool_k, pool_stride, beta_p),
                  "cuda conv2d bwd: launch failed");
        } else {
            check(nrs_maxpool_conv2d_backward(dinput, wg.grad->ptr(), bg.grad->ptr(), grad->ptr(),
                                              am, ig.data.ptr(), wg.data.ptr(), n, c_in, in_h,
                                              in_w, c_out, kh, kw, stride, pad, pool_k,
                                              pool_stride),
                  "cuda conv2d bwd: launch failed");
        }
    };
    return node;
}

namespace {

// The backward of a Linear node (its matmul closure and the bias's
// sum_axis0, linear.rs:22-25) given the gradient g of its output. With
// `mask` (the input x is a ReLU output whose gradient only ever receives
// masked contributions, see linear_node), the input gradient is masked by
// x > 0 in the same launch: relu_grad (relu.rs:30-45) of the ReLU's output
// gradient, i.e. the gradient of the ReLU's input.
void linear_backward_into(const NodeRef& x, const NodeRef& w, const NodeRef& b, const float* g,
                          size_t batch, size_t in_f, size_t out_f, const float* mask = nullptr) {
    GpuBuffers& xg = gpu_of(x, "cuda matmul bwd: lhs not on GPU");
    GpuBuffers& wg = gpu_of(w, "cuda matmul bwd: rhs not on GPU");
    GpuBuffers& bg = gpu_of(b, "backward: parent not on GPU");
    if (xg.grad == wg.grad || xg.grad == bg.grad || wg.grad == bg.grad) {
        // parents sharing a gradient: the products one after the other
        matmul_backward_into(x, w, g, batch, in_f, out_f, "cuda linear bwd: launch");
        if (mask)  // every contribution to x's gradient is masked: mask the sum
            check(nrs_relu_backward(xg.grad->ptr(), xg.grad->ptr(), mask, batch * in_f, 0.0f),
                  "cuda relu bwd: launch");
        float beta = 1.0f;
        float* db = bg.grad->acc_target(beta);
        check(nrs_sum_axis0(db, g, batch, out_f, beta), "cuda linear bwd: bias launch");
        return;
    }
    // dx += g . W^T, dW += x^T . g and db += column sums of g, one grouped
    // launch (the bias gradient rides the weight gradient)
    float bx = 1.0f, bw = 1.0f, bb = 1.0f;
    float* dx = xg.grad->acc_target(bx);
    float* dw = wg.grad->acc_target(bw);
    float* db = bg.grad->acc_target(bb);
    check(mask ? nrs_linear_backward_relu(dx, dw, db, g, xg.data.ptr(), wg.data.ptr(), mask, batch,
                                          in_f, out_f, bx, bw, bb)
               : nrs_linear_backward(dx, dw, db, g, xg.data.ptr(), wg.data.ptr(), batch, in_f,
                                     out_f, bx, bw, bb),
          "cuda linear bwd: launch");
}

// How a Linear node meets a ReLU:
//   kPlain      x . W + bias;
//   kReluOut    relu(x . W + bias), ReLU in the GEMM epilogue; the node's
//               backward masks its output gradient by the output (> 0
//               exactly where the pre-activation is);
//   kReluOutPre the same node whose only consumer is a kReluIn Linear: the
//               gradient arrives masked, so the backward uses it as is;
//   kReluIn     x . W + bias whose input x is a kReluOutPre node: its
//               backward writes x's gradient masked by x > 0 in the
//               input-gradient product's epilogue (nrs_linear_backward_relu).
enum class ReluLink { kPlain, kReluOut, kReluOutPre, kReluIn };

NodeRef linear_node(const Linear& l, const NodeRef& input, ReluLink link) {
    const bool relu = link == ReluLink::kReluOut || link == ReluLink::kReluOutPre;
    GpuBuffers& xg = gpu_of(input, "cuda matmul: lhs not on GPU");
    GpuBuffers& wg = gpu_of(l.weights, "cuda matmul: rhs not on GPU");
    GpuBuffers& bg = gpu_of(l.bias, "cuda add: rhs not on GPU");
    if (input->shape.size() != 2 || l.weights->shape.size() != 2)
        throw Panic("cuda matmul: operands must be 2-D");
    const size_t batch = input->shape[0], in_f = input->shape[1], out_f = l.weights->shape[1];
    if (l.weights->shape[0] != in_f) throw Panic("cuda matmul: inner dims mismatch");
    if (product(l.bias->shape) != out_f) throw Panic("cuda add: bias length mismatch");
    // x . W + bias in one GEMM: bias added in the epilogue (matmul + add).
    DeviceBuffer out(batch * out_f, false);
    check(nrs_gemm(NRS_NN, out.ptr(), xg.data.ptr(), wg.data.ptr(), batch, out_f, in_f, 0.0f,
                   bg.data.ptr(), NRS_EPI_BIAS_COL | (relu ? NRS_EPI_RELU : 0)),
          "cuda linear: launch failed");
    NodeRef x = input, w = l.weights, b = l.bias;
    NodeRef node = make_output({batch, out_f}, {x, w, b}, std::move(out));
    if (!relu) {
        const float* mask = link == ReluLink::kReluIn ? xg.data.ptr() : nullptr;
        node->backward_fn = [grad = node->gpu->grad, x, w, b, batch, in_f, out_f,
                             mask](const std::vector<float>&) {
            linear_backward_into(x, w, b, grad->ptr(), batch, in_f, out_f, mask);
        };
        return node;
    }
    if (link == ReluLink::kReluOutPre) {
        node->backward_fn = [grad = node->gpu->grad, x, w, b, batch, in_f,
                             out_f](const std::vector<float>&) {
            linear_backward_into(x, w, b, grad->ptr(), batch, in_f, out_f);
        };
        return node;
    }
    // relu.rs:30-45 masks by the pre-activation; the output is positive
    // exactly where it is, so the mask is read from the node's own output
    const float* y = node->gpu->data.ptr();
    node->backward_fn = [grad = node->gpu->grad, x, w, b, y, batch, in_f,
                         out_f](const std::vector<float>&) {
        DeviceBuffer gm(batch * out_f, false);
        check(nrs_relu_backward(gm.ptr(), grad->ptr(), y, batch * out_f, 0.0f),
              "cuda relu bwd: launch");
        linear_backward_into(x, w, b, gm.ptr(), batch, in_f, out_f);
    };
    return node;
}

}  // namespace

NodeRef Linear::forward(const NodeRef& input) const {
    return linear_node(*this, input, ReluLink::kPlain);
}

namespace {

// The products of one matmul_shared_lhs call, for their joint backward.
struct SharedLhs {
    NodeRef x;
    std::vector<NodeRef> ws;
    std::vector<std::weak_ptr<Node>> outs;
    size_t m, k, n;
};

// The matmul closures of every product of `s` (matmul.rs:418-431) as one
// nrs_matmul_shared_lhs_backward call, when the running pass holds every
// product, none has run yet and every product's gradient is complete (all
// its consumers have run); the input-gradient parts are added in the order
// the closures would run (the last topological position first), so the bits
// are those of the closures. The pass then skips the other products'
// closures. Returns false, having changed nothing, otherwise (and for shared
// gradient buffers, e.g. a weight used twice).
bool fused_shared_lhs_backward(const SharedLhs& s) {
    const size_t count = s.outs.size();
    if (!tl_pass || !g_fused_backward || count < 2 || count > 3) return false;
    std::vector<NodeRef> outs;
    for (const std::weak_ptr<Node>& wp : s.outs) {
        NodeRef o = wp.lock();
        if (!o || !o->gpu || tl_pass->done.count(o.get()) || !tl_pass->pos.count(o.get()))
            return false;
        const auto r = tl_pass->pending.find(o.get());
        if (r != tl_pass->pending.end() && r->second != 0) return false;
        outs.push_back(std::move(o));
    }
    GpuBuffers& xg = gpu_of(s.x, "cuda matmul bwd: lhs not on GPU");
    std::vector<GpuBuffers*> wg;
    for (const NodeRef& w : s.ws) wg.push_back(&gpu_of(w, "cuda matmul bwd: rhs not on GPU"));
    for (size_t i = 0; i < count; ++i) {
        if (wg[i]->grad == xg.grad) return false;
        for (size_t j = i + 1; j < count; ++j)
            if (wg[i]->grad == wg[j]->grad) return false;
    }
    size_t order[3] = {0, 1, 2};
    std::sort(order, order + count, [&](size_t a, size_t b) {
        return tl_pass->pos.at(outs[a].get()) > tl_pass->pos.at(outs[b].get());
    });
    float beta_x = 1.0f;
    float* dx = xg.grad->acc_target(beta_x);
    float* dw[3];
    const float* g[3];
    const float* w[3];
    float beta_w[3];
    for (size_t j = 0; j < count; ++j) {
        const size_t i = order[j];
        beta_w[j] = 1.0f;
        dw[j] = wg[i]->grad->acc_target(beta_w[j]);
        g[j] = outs[i]->gpu->grad->ptr();
        w[j] = wg[i]->data.ptr();
    }
    check(nrs_matmul_shared_lhs_backward(dx, dw, g, xg.data.ptr(), w, (int)count, s.m, s.k, s.n,
                                         beta_x, beta_w),
          "cuda matmul bwd: launch failed");
    for (const NodeRef& o : outs) tl_pass->done.insert(o.get());
    return true;
}

// x . w for each of several weights, in one grouped launch: the Q, K and V
// projections of one input (multihead.rs:64-66). Each result is a node of
// its own with graph::matmul's checks and output; their backward closures
// run together when the pass allows (fused_shared_lhs_backward), else each
// is graph::matmul's.
std::vector<NodeRef> matmul_shared_lhs(const NodeRef& x, const std::vector<NodeRef>& ws) {
    GpuBuffers& xg = gpu_of(x, "cuda matmul: lhs not on GPU");
    if (x->shape.size() != 2) throw Panic("cuda matmul: operands must be 2-D");
    if (ws.empty() || ws.size() > NRS_GEMM_GROUP_MAX) throw Panic("cuda matmul: bad group");
    const size_t m = x->shape[0], k = x->shape[1];
    std::vector<DeviceBuffer> outs;
    std::vector<nrs_gemm_desc> d;
    for (const NodeRef& w : ws) {
        GpuBuffers& wg = gpu_of(w, "cuda matmul: rhs not on GPU");
        if (w->shape.size() != 2) throw Panic("cuda matmul: operands must be 2-D");
        if (w->shape[0] != k) throw Panic("cuda matmul: inner dims mismatch");
        const size_t n = w->shape[1];
        outs.emplace_back(m * n, false);
        d.push_back({NRS_NN, outs.back().ptr(), xg.data.ptr(), wg.data.ptr(), (int64_t)m,
                     (int64_t)n, (int64_t)k, 0.0f, nullptr, NRS_EPI_NONE});
    }
    check(nrs_gemm_group(d.data(), (int)d.size()), "cuda matmul: launch failed");
    std::vector<NodeRef> nodes;
    for (size_t i = 0; i < ws.size(); ++i)
        nodes.push_back(make_output({m, ws[i]->shape[1]}, {x, ws[i]}, std::move(outs[i])));
    bool same_n = true;
    for (const NodeRef& w : ws) same_n = same_n && w->shape[1] == ws[0]->shape[1];
    std::shared_ptr<SharedLhs> group;
    if (same_n && ws.size() >= 2 && ws.size() <= 3) {
        group = std::make_shared<SharedLhs>(SharedLhs{x, ws, {}, m, k, ws[0]->shape[1]});
        for (const NodeRef& node : nodes) group->outs.push_back(node);
    }
    for (size_t i = 0; i < ws.size(); ++i) {
        const size_t n = ws[i]->shape[1];
        const NodeRef& w = ws[i];
        nodes[i]->backward_fn = [grad = nodes[i]->gpu->grad, group, x, w, m, k,
                                 n](const std::vector<float>&) {
            if (group && fused_shared_lhs_backward(*group)) return;
            matmul_backward_into(x, w, grad->ptr(), m, k, n, "cuda matmul bwd: launch failed");
        };
    }
    return nodes;
}

// q . k^T per item without materialising k^T: [b, m, d] x [b, n, d] -> [b, m, n]
// (or 2-D [m, d] x [n, d] -> [m, n]): the bmm(q, transpose(k)) / matmul(q,
// transpose(k)) of attention.rs:15,28 as one NT product. Its backward is the
// bmm closure for that layout: dq += g . k, dk += g^T . q.
NodeRef bmm_nt(const NodeRef& q, const NodeRef& k) {
    GpuBuffers& qg = gpu_of(q, "cuda bmm: lhs not on GPU");
    GpuBuffers& kg = gpu_of(k, "cuda bmm: rhs not on GPU");
    const bool two_d = q->shape.size() == 2;
    if (q->shape.size() != k->shape.size() || (!two_d && q->shape.size() != 3))
        throw Panic("cuda bmm: operands must be 3-D");
    const size_t batch = two_d ? 1 : q->shape[0];
    const size_t m = q->shape[two_d ? 0 : 1], d = q->shape.back(), n = k->shape[two_d ? 0 : 1];
    if (k->shape.back() != d || (!two_d && k->shape[0] != batch))
        throw Panic("cuda bmm: shape mismatch");
    DeviceBuffer out(batch * m * n, false);
    check(nrs_bmm(NRS_NT, out.ptr(), qg.data.ptr(), kg.data.ptr(), batch, m, n, d, 0.0f),
          "cuda bmm: launch failed");
    std::vector<size_t> shape = two_d ? std::vector<size_t>{m, n} : std::vector<size_t>{batch, m, n};
    NodeRef node = make_output(std::move(shape), {q, k}, std::move(out));
    node->backward_fn = [grad = node->gpu->grad, q, k, batch, m, d, n](const std::vector<float>&) {
        bmm_backward_into(NRS_NT, q, k, grad->ptr(), batch, m, d, n, "cuda bmm bwd");
    };
    return node;
}

// [rows, heads * w] -> [heads, rows, w] (given `shape`, e.g. [heads * batch,
// seq, w]): the per-head slice_cols of MultiHeadAttention (multihead.rs:72-78)
// in one launch; its backward is merge_heads accumulating into x's gradient.
NodeRef split_heads(const NodeRef& x, size_t rows, size_t heads, size_t w,
                    std::vector<size_t> shape) {
    GpuBuffers& xg = gpu_of(x, "cuda slice_cols: input not on GPU");
    DeviceBuffer out(rows * heads * w, false);
    check(nrs_split_heads(out.ptr(), xg.data.ptr(), rows, heads, w, 0.0f),
          "cuda slice_cols: launch failed");
    NodeRef node = make_output(std::move(shape), {x}, std::move(out));
    node->backward_fn = [grad = node->gpu->grad, x, rows, heads, w](const std::vector<float>&) {
        float beta = 1.0f;
        float* gx = gpu_of(x, "backward: parent not on GPU").grad->acc_target(beta);
        check(nrs_merge_heads(gx, grad->ptr(), rows, heads, w, beta),
              "cuda slice_cols bwd: launch");
    };
    return node;
}

// [heads, rows, w] -> [rows, heads * w]: the concat_cols of the heads
// (multihead.rs:81) in one launch; its backward is split_heads accumulating.
NodeRef merge_heads(const NodeRef& x, size_t rows, size_t heads, size_t w,
                    std::vector<size_t> shape) {
    GpuBuffers& xg = gpu_of(x, "cuda concat_cols: part not on GPU");
    DeviceBuffer out(rows * heads * w, false);
    check(nrs_merge_heads(out.ptr(), xg.data.ptr(), rows, heads, w, 0.0f),
          "cuda concat_cols: write launch failed");
    NodeRef node = make_output(std::move(shape), {x}, std::move(out));
    node->backward_fn = [grad = node->gpu->grad, x, rows, heads, w](const std::vector<float>&) {
        float beta = 1.0f;
        float* gx = gpu_of(x, "backward: part not on GPU").grad->acc_target(beta);
        check(nrs_split_heads(gx, grad->ptr(), rows, heads, w, beta),
              "cuda concat_cols bwd: launch");
    };
    return node;
}

// softmax(scale * q . k^T) . v for every (item, head) in one node: q, k, v
// and the output are [batch * seq, ld] rows (any leading shape of that many
// elements) with head h in columns [h*dh, (h+1)*dh). Same values as
// attention_batch per head (attention.rs:23-32); the scores stay on chip and
// the backward recomputes them from the saved softmax statistics.
NodeRef fused_attention(const NodeRef& q, const NodeRef& k, const NodeRef& v, size_t batch,
                        size_t heads, size_t seq, size_t dh, size_t ld, float scale) {
    GpuBuffers& qg = gpu_of(q, "attention: q not on GPU");
    GpuBuffers& kg = gpu_of(k, "attention: k not on GPU");
    GpuBuffers& vg = gpu_of(v, "attention: v not on GPU");
    const size_t len = product(q->shape);
    DeviceBuffer out(len, false);
    auto stats = std::make_shared<DeviceBuffer>(batch * heads * seq * 2, false);
    check(nrs_attention_forward(out.ptr(), stats->ptr(), qg.data.ptr(), kg.data.ptr(),
                                vg.data.ptr(), batch, heads, seq, dh, ld, scale),
          "attention: launch failed");
    NodeRef node = make_output(q->shape, {q, k, v}, std::move(out));
    Node* self = node.get();  // the output (read by the backward of long sequences)
    node->backward_fn = [grad = node->gpu->grad, self, q, k, v, stats, len, batch, heads, seq, dh,
                         ld, scale](const std::vector<float>&) {
        GpuBuffers& qg = gpu_of(q, "attention bwd: q not on GPU");
        GpuBuffers& kg = gpu_of(k, "attention bwd: k not on GPU");
        GpuBuffers& vg = gpu_of(v, "attention bwd: v not on GPU");
        const float* o = self->gpu->data.ptr();
        if (qg.grad != kg.grad && kg.grad != vg.grad && qg.grad != vg.grad) {
            const float beta = joint_beta({qg.grad.get(), kg.grad.get(), vg.grad.get()});
            check(nrs_attention_backward(qg.grad->write_target(), kg.grad->write_target(),
                                         vg.grad->write_target(), grad->ptr(), o, qg.data.ptr(),
                                         kg.data.ptr(), vg.data.ptr(), stats->ptr(), batch, heads,
                                         seq, dh, ld, scale, beta),
                  "attention bwd: launch");
            return;
        }
        // q, k or v are one node: the gradients go to temporaries, then add up
        DeviceBuffer tq(len, false), tk(len, false), tv(len, false);
        check(nrs_attention_backward(tq.ptr(), tk.ptr(), tv.ptr(), grad->ptr(), o, qg.data.ptr(),
                                     kg.data.ptr(), vg.data.ptr(), stats->ptr(), batch, heads, seq,
                                     dh, ld, scale, 0.0f),
              "attention bwd: launch");
        accumulate_into(*qg.grad, tq.ptr(), len);
        accumulate_into(*kg.grad, tk.ptr(), len);
        accumulate_into(*vg.grad, tv.ptr(), len);
    };
    return node;
}

}  // namespace

NodeRef attention(const NodeRef& q, const NodeRef& k, const NodeRef& v) {
    if (q->shape.size() != 2) throw Panic("attention: q must be [seq, d]");
    const size_t seq = q->shape[0], d = q->shape[1];
    const float s = 1.0f / std::sqrt(static_cast<float>(d));
    if (k->shape == q->shape && v->shape == q->shape && nrs_attention_supported(1, 1, seq, d, d))
        return fused_attention(q, k, v, 1, 1, seq, d, d, s);
    // the composition of attention.rs:15-19 with q . k^T as one NT product and
    // scale + softmax as one node
    NodeRef weights = graph::scaled_softmax(bmm_nt(q, k), s);
    return graph::matmul(weights, v);
}

NodeRef attention_batch(const NodeRef& q, const NodeRef& k, const NodeRef& v) {
    if (q->shape.size() != 3) throw Panic("attention_batch: q must be [batch, seq, d]");
    const size_t batch = q->shape[0], seq = q->shape[1], d = q->shape[2];
    const float s = 1.0f / std::sqrt(static_cast<float>(d));
    if (k->shape == q->shape && v->shape == q->shape &&
        nrs_attention_supported(batch, 1, seq, d, d))
        return fused_attention(q, k, v, batch, 1, seq, d, d, s);
    NodeRef weights = graph::scaled_softmax(bmm_nt(q, k), s);  // attention.rs:28-30
    return graph::bmm(weights, v);
}

// `a` in another shape without a copy: the node shares a's device memory and
// its gradient, so its consumers' gradients land in a's gradient directly and
// it has no backward of its own. Only for reshapes internal to a composite
// node (the flattening inside MultiHeadAttention and TransformerBlock), which
// no caller can reach: graph::reshape copies, as the reference does
// (src/cuda/graph/reshape.rs:31-70), and keeps the two gradients apart.
static NodeRef reshape_view(const NodeRef& a, std::vector<size_t> shape) {
    GpuBuffers& ag = gpu_of(a, "cuda reshape: input not on GPU");
    if (product(shape) != product(a->shape)) throw Panic("cuda reshape: element count mismatched");
    NodeRef out = std::make_shared<Node>();
    out->shape = std::move(shape);
    out->parents = {a};
    out->gpu = std::make_unique<GpuBuffers>();
    out->gpu->data = DeviceBuffer::view_of(ag.data);
    out->gpu->grad = ag.grad;
    return out;
}

// Shared by forward (batch 1) and forward_batch: the projections of the
// flattened input, every head's attention at once, the output projection.
static NodeRef multihead(const MultiHeadAttention& mha, const NodeRef& flat, size_t batch,
                         size_t seq, size_t d) {
    if (mha.num_heads == 0 || mha.d_model % mha.num_heads != 0)
        throw Panic("multihead: d_model % heads != 0");
    const size_t heads = mha.num_heads, dh = mha.d_model / heads, rows = batch * seq;
    if (heads * dh != d) throw Panic("multihead: input width is not d_model");
    const std::vector<NodeRef> qkv = matmul_shared_lhs(flat, {mha.w_q, mha.w_k, mha.w_v});
    const NodeRef &q = qkv[0], &k = qkv[1], &v = qkv[2];
    NodeRef concat;
    if (nrs_attention_supported(batch, heads, seq, dh, d)) {
        // heads read and written in place in the [rows, d_model] projections
        concat = fused_attention(q, k, v, batch, heads, seq, dh, d,
                                 1.0f / std::sqrt(static_cast<float>(dh)));
    } else {
        // the heads as one batch of heads * batch items, one attention_batch
        const std::vector<size_t> hs{heads * batch, seq, dh};
        NodeRef att = attention_batch(split_heads(q, rows, heads, dh, hs),
                                      split_heads(k, rows, heads, dh, hs),
                                      split_heads(v, rows, heads, dh, hs));
        concat = merge_heads(att, rows, heads, dh, {rows, d});
    }
    return graph::matmul(concat, mha.w_o);
}

NodeRef SelfAttention::forward(const NodeRef& x) const {
    // self_attention.rs:31-36: q, k, v = x . w_q, x . w_k, x . w_v (one grouped
    // launch, three matmul nodes), then attention
    if (x->shape.size() != 2) throw Panic("self attention: x must be [seq, d_model]");
    const std::vector<NodeRef> qkv = matmul_shared_lhs(x, {w_q, w_k, w_v});
    return attention(qkv[0], qkv[1], qkv[2]);
}

NodeRef MultiHeadAttention::forward(const NodeRef& x) const {
    if (x->shape.size() != 2) throw Panic("multihead: x must be [seq, d_model]");
    return multihead(*this, x, 1, x->shape[0], x->shape[1]);
}

NodeRef MultiHeadAttention::forward_batch(const NodeRef& x) const {
    if (x->shape.size() != 3) throw Panic("multihead: x must be [batch, seq, d_model]");
    const size_t batch = x->shape[0], seq = x->shape[1], d = x->shape[2];
    NodeRef out = multihead(*this, reshape_view(x, {batch * seq, d}), batch, seq, d);
    return graph::reshape(out, {batch, seq, d});
}

namespace {

// norm(add(a, b)) as one node: the residual add and the LayerNorm of
// transformer_block.rs:32-33, 41-42, with the sum never written out. The
// add node is internal to the block, so no graph node a caller can reach is
// lost. Its backward is the LayerNorm's, whose input gradient goes to both
// a and b (add.rs's backward): stored to or added into both gradients by one
// launch when the four gradients are distinct buffers, else through a
// temporary.
NodeRef add_layernorm(const NodeRef& a, const NodeRef& b, const LayerNorm& norm) {
    GpuBuffers& ag = gpu_of(a, "cuda add: lhs not on GPU");
    GpuBuffers& bgb = gpu_of(b, "cuda add: rhs not on GPU");
    GpuBuffers& gg = gpu_of(norm.gamma, "cuda layernorm: gamma not on GPU");
    GpuBuffers& betag = gpu_of(norm.beta, "cuda layernorm: beta not on GPU");
    if (product(b->shape) != product(a->shape)) throw Panic("cuda add: shape mismatch");
    if (a->shape.empty()) throw Panic("cuda layernorm: scalar input");
    const size_t F = a->shape.back(), len = product(a->shape);
    const size_t rows = F ? len / F : 0;
    if (F == 0 || product(norm.gamma->shape) != F || product(norm.beta->shape) != F)
        throw Panic("cuda layernorm: gamma/beta length mismatch");
    DeviceBuffer out(len, false);
    auto xn = std::make_shared<DeviceBuffer>(len, false);
    auto istd = std::make_shared<DeviceBuffer>(rows, false);
    check(nrs_add_layernorm_forward(out.ptr(), xn->ptr(), istd->ptr(), ag.data.ptr(),
                                    bgb.data.ptr(), gg.data.ptr(), betag.data.ptr(), rows, F,
                                    norm.eps),
          "cuda layernorm: forward launch failed");
    NodeRef gamma = norm.gamma, beta = norm.beta;
    NodeRef node = make_output(a->shape, {a, b, gamma, beta}, std::move(out));
    node->backward_fn = [grad = node->gpu->grad, a, b, gamma, beta, xn, istd, rows, F,
                         len](const std::vector<float>&) {
        GpuBuffers& ag = gpu_of(a, "cuda layernorm bwd: input not on GPU");
        GpuBuffers& bgb = gpu_of(b, "cuda layernorm bwd: input not on GPU");
        GpuBuffers& gg = gpu_of(gamma, "cuda layernorm bwd: gamma not on GPU");
        GpuBuffers& betag = gpu_of(beta, "cuda layernorm bwd: beta not on GPU");
        const bool distinct = ag.grad != bgb.grad && ag.grad != gg.grad &&
                              ag.grad != betag.grad && bgb.grad != gg.grad &&
                              bgb.grad != betag.grad && gg.grad != betag.grad;
        if (distinct) {
            // the input gradient stored to (or added into) both a's and b's
            // gradients in one pass
            float beta_a = 1.0f, beta_b = 1.0f;
            float* da = ag.grad->acc_target(beta_a);
            float* db = bgb.grad->acc_target(beta_b);
            const float acc = gg.grad != betag.grad ? joint_beta({gg.grad.get(), betag.grad.get()})
                                                    : 1.0f;
            check(nrs_add_layernorm_backward(da, db, gg.grad->ptr(), betag.grad->ptr(), grad->ptr(),
                                             gg.data.ptr(), xn->ptr(), istd->ptr(), rows, F,
                                             beta_a, beta_b, acc),
                  "cuda layernorm bwd: launch");
            return;
        }
        DeviceBuffer tmp(len, false);
        check(nrs_layernorm_backward(tmp.ptr(), nullptr, nullptr, grad->ptr(), gg.data.ptr(),
                                     xn->ptr(), istd->ptr(), rows, F, 0.0f),
              "cuda layernorm bwd: launch");
        const float accp =
            gg.grad != betag.grad ? joint_beta({gg.grad.get(), betag.grad.get()}) : 1.0f;
        check(nrs_layernorm_backward(nullptr, gg.grad->ptr(), betag.grad->ptr(), grad->ptr(),
                                     gg.data.ptr(), xn->ptr(), istd->ptr(), rows, F, accp),
              "cuda layernorm bwd: launch");
        accumulate_into(*ag.grad, tmp.ptr(), len);
        accumulate_into(*bgb.grad, tmp.ptr(), len);
    };
    return node;
}

}  // namespace

NodeRef TransformerBlock::forward(const NodeRef& x) const {
    if (x->shape.size() != 3) throw Panic("transformer block: x must be [batch, seq, d_model]");
    const size_t batch = x->shape[0], seq = x->shape[1], d = x->shape[2];
    if (d != mha.d_model) throw Panic("multihead: input width is not d_model");
    // mha.forward_batch(x) without its reshapes: the attention output stays
    // [batch*seq, d] (add_layernorm takes it as is); norm1(add(x, attn_out))
    // and norm2(add(x1, ff_out)) each as one node, relu(ff1(x1)) as one node
    // with ReLU in the GEMM epilogue. The reshapes, sums and pre-activation
    // are internal to the block, so no node a caller can reach is lost.
    NodeRef attn_out = multihead(mha, reshape_view(x, {batch * seq, d}), batch, seq, d);
    NodeRef x1 = add_layernorm(x, attn_out, norm1);
    // h is internal and ff2 its only consumer: ff2's backward writes h's
    // gradient already masked by the ReLU, and h's backward uses it as is
    NodeRef h = linear_node(ff1, reshape_view(x1, {batch * seq, d}), ReluLink::kReluOutPre);
    NodeRef ff_out = linear_node(ff2, h, ReluLink::kReluIn);
    return add_layernorm(x1, ff_out, norm2);
}

NodeRef layernorm(const NodeRef& input, const NodeRef& gamma, const NodeRef& beta, float eps) {
    GpuBuffers& ig = gpu_of(input, "cuda layernorm: input not on GPU");
    GpuBuffers& gg = gpu_of(gamma, "cuda layernorm: gamma not on GPU");
    GpuBuffers& bg = gpu_of(beta, "cuda layernorm: beta not on GPU");
    if (input->shape.empty()) throw Panic("cuda layernorm: scalar input");
    const size_t F = input->shape.back(), len = product(input->shape);
    const size_t rows = F ? len / F : 0;
    if (F == 0 || product(gamma->shape) != F || product(beta->shape) != F)
        throw Panic("cuda layernorm: gamma/beta length mismatch");
    DeviceBuffer out(len, false);
    auto xn = std::make_shared<DeviceBuffer>(len, false);
    auto istd = std::make_shared<DeviceBuffer>(rows, false);
    check(nrs_layernorm_forward(out.ptr(), xn->ptr(), istd->ptr(), ig.data.ptr(), gg.data.ptr(),
                                bg.data.ptr(), rows, F, eps),
          "cuda layernorm: forward launch failed");
    NodeRef node = make_output(input->shape, {input, gamma, beta}, std::move(out));
    node->backward_fn = [grad = node->gpu->grad, input, gamma, beta, xn, istd, rows,
                         F](const std::vector<float>&) {
        GpuBuffers& ig = gpu_of(input, "cuda layernorm bwd: input not on GPU");
        GpuBuffers& gg = gpu_of(gamma, "cuda layernorm bwd: gamma not on GPU");
        GpuBuffers& bg = gpu_of(beta, "cuda layernorm bwd: beta not on GPU");
        // one beta for the three gradients, unless gamma and beta are one node
        const bool distinct = ig.grad != gg.grad && ig.grad != bg.grad && gg.grad != bg.grad;
        const float acc =
            distinct ? joint_beta({ig.grad.get(), gg.grad.get(), bg.grad.get()}) : 1.0f;
        check(nrs_layernorm_backward(ig.grad->ptr(), gg.grad->ptr(), bg.grad->ptr(), grad->ptr(),
                                     gg.data.ptr(), xn->ptr(), istd->ptr(), rows, F, acc),
              "cuda layernorm bwd: launch");
    };
    return node;
}

}  // namespace nn
}  // namespace hip
}  // namespace neuralrs
