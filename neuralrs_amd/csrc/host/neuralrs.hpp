// C++ host layer of the MI355X backend: the reference's resident GPU operator
// API (Tensor/Node device placement, resident matmul, bmm, Linear, Conv2d and
// the attention composition), restated over the C ABI of libnrs_hip.so.
//
// The reference is Rust. Its GPU path is the `cuda` module behind
// `--features cuda` (Cargo.toml:23-26, src/lib.rs:53-54). This header keeps
// the same shape so the same call sites read the same:
//   Node / GpuBuffers / backward_graph   src/autograd/node.rs:38-126
//   runtime::{to_cuda, to_host, set_grad, read_grad, zero_grad, synchronize}
//                                        src/cuda/runtime.rs:39-124
//   graph::{matmul, bmm, add, transpose, scale, softmax, relu, slice_cols,
//          concat_cols, scaled_softmax}
//                                        src/cuda/graph/*.rs
//   nn::{conv2d, maxpool2d, Linear, attention, attention_batch, layernorm,
//        SelfAttention, MultiHeadAttention, TransformerBlock}
//                                        src/cuda/nn/*.rs
// Rc<RefCell<Node>> becomes std::shared_ptr<Node>; a panic ("cuda matmul: lhs
// not on GPU") becomes a thrown neuralrs::Panic with the same message. Like
// the reference it is single-threaded, device 0, one stream.
//
// Differences that change no result: backward closures write straight into
// the parents' gradients through the kernels' beta = 1 epilogues instead of
// allocating a temporary and launching accumulate (src/cuda/runtime.rs:67-83);
// Linear::forward is one GEMM with a fused bias epilogue instead of matmul
// followed by add (src/cuda/nn/linear.rs:22-25).
#pragma once

#include <cstddef>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace neuralrs {

// A reference panic (`.expect(...)`, `assert_eq!`) surfaces as this exception.
struct Panic : std::runtime_error {
    explicit Panic(const std::string& m) : std::runtime_error(m) {}
};

// src/device.rs:3-7. The reference calls the GPU variant CUDA(usize); here the
// GPU is the HIP device (always index 0, like src/cuda/backend.rs:21).
enum class Device { CPU, GPU };

// Owning f32 device allocation: the reference's CudaSlice<f32>.
//
// A zeroed buffer (alloc_zeros, memset_zeros) is zero in value at once but its
// memory is cleared only when first needed: ptr() clears it first, while a
// kernel that writes every element as value + beta * old takes the pointer
// from acc_target(), which hands out beta 0 instead of clearing (and a kernel
// that overwrites every element takes write_target()). Gradient buffers are
// created zeroed and their first contribution is usually such a kernel, so a
// backward pass mostly skips the clearing launches.
class DeviceBuffer;
// Records that `b` stopped being a pending zero for a launch that is about to
// be enqueued: a failed launch (a thrown Panic) makes it a pending zero again,
// since nothing was written to its memory.
void note_pending_taken(DeviceBuffer* b);

class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t len, bool zero = true);  // stream.alloc_zeros
    static DeviceBuffer from_host(const std::vector<float>& v);  // stream.clone_htod
    // The memory of `src` without owning it (not freed by this buffer): the
    // data of a node internal to a composite op that shows another node's
    // values in another shape. `src` must outlive the view.
    static DeviceBuffer view_of(const DeviceBuffer& src);
    ~DeviceBuffer();
    DeviceBuffer(DeviceBuffer&& o) noexcept;
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept;
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;

    // Device memory holding the buffer's value (a pending zero is cleared
    // first).
    float* ptr() const {
        if (pending_zero_) clear_now();
        return ptr_;
    }
    // For a launch that stores value + beta * old in every element: sets
    // beta (0 while the buffer is a pending zero, else 1) and returns memory
    // that holds the buffer's value once the launch is enqueued.
    float* acc_target(float& beta) {
        beta = pending_zero_ ? 0.0f : 1.0f;
        take_pending();
        return ptr_;
    }
    // For a launch that overwrites every element without reading it.
    float* write_target() {
        take_pending();
        return ptr_;
    }
    bool pending_zero() const { return pending_zero_; }
    size_t len() const { return len_; }
    std::vector<float> to_host() const;  // stream.clone_dtoh (synchronises)
    void zero();                          // stream.memset_zeros

private:
    void take_pending() {
        if (pending_zero_) {
            pending_zero_ = false;
            note_pending_taken(this);
        }
    }
    void clear_now() const;
    float* ptr_ = nullptr;
    size_t len_ = 0;
    mutable bool pending_zero_ = false;
    bool owned_ = true;
};

// src/autograd/node.rs:49-53: device data plus a shared, swappable gradient.
struct GpuBuffers {
    DeviceBuffer data;
    std::shared_ptr<DeviceBuffer> grad;
};

struct Node;
using NodeRef = std::shared_ptr<Node>;
struct ReluPoolConv;

// src/autograd/node.rs:38-47.
struct Node {
    std::vector<float> data;
    std::vector<float> grad;
    std::vector<size_t> shape;
    std::vector<NodeRef> parents;
    std::function<void(const std::vector<float>&)> backward_fn;
    bool requires_grad = true;
    std::unique_ptr<GpuBuffers> gpu;  // Option<GpuBuffers>
    // Host-only, no counterpart in the reference: set by
    // hip::nn::conv2d_maxpool with a ReLU. A conv2d over this node that is
    // its only consumer in a backward pass runs both backwards in one call
    // (same results) and the pass then skips this node's closure.
    std::shared_ptr<const ReluPoolConv> relu_pool_conv;

    // Node::new (src/autograd/node.rs:61-74).
    static NodeRef create(std::vector<float> data, std::vector<size_t> shape);
    // Node::device (src/autograd/node.rs:77-82).
    Device device() const { return gpu ? Device::GPU : Device::CPU; }
    size_t numel() const;
};

// Topological backward over the whole graph (src/autograd/node.rs:113-151).
void backward_graph(const NodeRef& root);

namespace hip {

namespace runtime {
// src/cuda/runtime.rs:39-51: H->D copy of data and a zeroed device gradient.
void to_cuda(const NodeRef& node);
// src/cuda/runtime.rs:57-63.
std::vector<float> to_host(const NodeRef& node);
// src/cuda/runtime.rs:87-93: replaces the gradient buffer with a copy of grad.
void set_grad(const NodeRef& node, const std::vector<float>& grad);
// set_grad's replacement of the gradient buffer for a gradient that is
// already on the device: exchanges the node's gradient with `buf` (same
// length), no copy. Backward closures hold the node's gradient object, so
// they read what was swapped in; swapping back returns the buffer.
void swap_grad(const NodeRef& node, DeviceBuffer& buf);
// Whether backward_graph runs a closure together with its neighbours' where
// that saves launches (a conv over a ReLU + max-pool node, the Q, K and V
// projections' three matmul closures): the same results either way. On by
// default; off runs every closure on its own.
void set_fused_backward(bool on);
// src/cuda/runtime.rs:96-103.
std::vector<float> read_grad(const NodeRef& node);
// src/cuda/runtime.rs:108-117.
void zero_grad(const std::vector<NodeRef>& params);
// src/cuda/runtime.rs:122-124.
void synchronize();
}  // namespace runtime

namespace graph {
// src/cuda/graph/matmul.rs:386-436: [m,k] x [k,n] -> [m,n].
NodeRef matmul(const NodeRef& a, const NodeRef& b);
// src/cuda/graph/bmm.rs:65-131: [b,m,k] x [b,k,n] -> [b,m,n].
NodeRef bmm(const NodeRef& a, const NodeRef& b);
// src/cuda/graph/add.rs:41-110: same-shape add, or [rows,cols] + bias[cols].
NodeRef add(const NodeRef& a, const NodeRef& b);
// src/cuda/graph/transpose.rs:26-72: swaps the last two dims.
NodeRef transpose(const NodeRef& a);
// src/cuda/graph/scale.rs:22-58.
NodeRef scale(const NodeRef& a, float s);
// src/cuda/graph/softmax.rs:38-85: softmax over the last dim.
NodeRef softmax(const NodeRef& a);
// src/cuda/graph/relu.rs:30-80.
NodeRef relu(const NodeRef& a);
// src/cuda/graph/slice_cols.rs:37-86: columns [col_start, col_end) of the last dim.
NodeRef slice_cols(const NodeRef& a, size_t col_start, size_t col_end);
// src/cuda/graph/concat_cols.rs:35-95: the parts side by side along the last dim.
NodeRef concat_cols(const std::vector<NodeRef>& parts);
// graph::scale then graph::softmax as one node (same values and gradients,
// one pass each way), as attention applies them (src/cuda/nn/attention.rs:17-18).
NodeRef scaled_softmax(const NodeRef& a, float s);
// src/cuda/graph/reshape.rs:31-70: the same values in a new shape (copied into
// a new buffer, as the reference does; the gradient is accumulated back).
NodeRef reshape(const NodeRef& a, std::vector<size_t> shape);
}  // namespace graph

namespace loss {
// src/cuda/loss/cross_entropy.rs:74-91: cross-entropy of resident logits
// ([batch, classes], or [classes] as one row) against a resident one-hot
// target, averaged over the batch (per-row losses on the device, summed on
// the host in row order).
float cross_entropy(const NodeRef& pred, const NodeRef& target);
// src/cuda/loss/cross_entropy.rs:100-127: writes (softmax - target) / batch
// into the logits' gradient; backward_graph then propagates it.
void cross_entropy_backward(const NodeRef& pred, const NodeRef& target);
}  // namespace loss

namespace nn {
// src/cuda/nn/conv.rs:244-328: input [N,c_in,H,W], weight [c_out,c_in,kh,kw],
// bias [c_out] -> [N,c_out,oh,ow]. The input gradient is skipped when
// input->requires_grad is false (conv.rs:304).
NodeRef conv2d(const NodeRef& input, const NodeRef& weight, const NodeRef& bias, size_t stride,
               size_t pad);

// src/cuda/nn/maxpool.rs:60-66: kernel x kernel windows with `stride`, no
// padding, on [N,C,H,W]; the backward adds each window's gradient to its
// first maximum.
NodeRef maxpool2d(const NodeRef& input, size_t kernel, size_t stride);

// maxpool2d(conv2d(input, weight, bias, stride, pad), pool_k, pool_stride),
// or with relu maxpool2d(relu(conv2d(..)), ..) as the reference CNN builds it
// (examples/mnist_cuda_cnn.rs:125,127), as one node for a conv output that
// only feeds the pooling: same values and gradients, and the conv output and
// its ReLU are never materialised on the fused shapes ("same" 3x3 stride 1
// over c_in <= 3 channels with 2x2 stride-2 pooling: one launch each way).
NodeRef conv2d_maxpool(const NodeRef& input, const NodeRef& weight, const NodeRef& bias,
                       size_t stride, size_t pad, bool relu, size_t pool_k, size_t pool_stride);

// src/cuda/nn/linear.rs:11-26: weights [in,out], bias [out].
struct Linear {
    NodeRef weights;
    NodeRef bias;
    Linear(NodeRef w, NodeRef b) : weights(std::move(w)), bias(std::move(b)) {}
    NodeRef forward(const NodeRef& input) const;  // [batch,in] -> [batch,out]
};

// src/cuda/nn/attention.rs:10-32: softmax(Q K^T / sqrt(d)) V. One fused node
// (scores kept on chip) when q, k, v have one shape, seq <= 128 and d 16 or
// 32; otherwise Q.K^T as one NT product, scale + softmax, and the last product.
NodeRef attention(const NodeRef& q, const NodeRef& k, const NodeRef& v);
NodeRef attention_batch(const NodeRef& q, const NodeRef& k, const NodeRef& v);
// src/cuda/nn/normalization.rs:87-160: per-row layer norm over the last dim
// with gamma/beta [features].
NodeRef layernorm(const NodeRef& input, const NodeRef& gamma, const NodeRef& beta, float eps);

// src/cuda/nn/self_attention.rs:10-37: single-head self-attention over
// resident projections w_q, w_k, w_v [d_model, d_k]: x [seq, d_model] ->
// attention(x w_q, x w_k, x w_v) [seq, d_k] (the three projections of one
// input share one grouped launch).
struct SelfAttention {
    NodeRef w_q, w_k, w_v;
    size_t d_model, d_k;
    SelfAttention(NodeRef q, NodeRef k, NodeRef v, size_t d, size_t dk)
        : w_q(std::move(q)), w_k(std::move(k)), w_v(std::move(v)), d_model(d), d_k(dk) {}
    NodeRef forward(const NodeRef& x) const;
};

// src/cuda/nn/normalization.rs (LayerNorm): resident gamma/beta [features].
struct LayerNorm {
    NodeRef gamma, beta;
    float eps;
    LayerNorm(NodeRef g, NodeRef b, float e) : gamma(std::move(g)), beta(std::move(b)), eps(e) {}
    NodeRef forward(const NodeRef& x) const { return layernorm(x, gamma, beta, eps); }
};

// src/cuda/nn/multihead.rs:10-85: projections w_* [d_model, d_model], every
// head's attention, heads joined, w_o. The reference slices each head out of
// the projections, runs attention per head and concatenates; here all heads
// run in one fused attention node that reads and writes them in place (or,
// for shapes outside the fused path, split/merge-heads nodes around one
// attention_batch of heads * batch items). Same values and gradients.
struct MultiHeadAttention {
    NodeRef w_q, w_k, w_v, w_o;
    size_t d_model, num_heads;
    MultiHeadAttention(NodeRef q, NodeRef k, NodeRef v, NodeRef o, size_t d, size_t heads)
        : w_q(std::move(q)), w_k(std::move(k)), w_v(std::move(v)), w_o(std::move(o)),
          d_model(d), num_heads(heads) {}
    NodeRef forward(const NodeRef& x) const;        // [seq, d_model]
    NodeRef forward_batch(const NodeRef& x) const;  // [batch, seq, d_model]
};

// src/cuda/nn/transformer_block.rs:9-45: post-norm block, x + MHA(x) -> norm1
// -> x1 + ff2(relu(ff1(x1))) -> norm2.
struct TransformerBlock {
    MultiHeadAttention mha;
    LayerNorm norm1, norm2;
    Linear ff1, ff2;
    size_t d_model, d_ff;
    NodeRef forward(const NodeRef& x) const;  // [batch, seq, d_model]
};
}  // namespace nn

}  // namespace hip
}  // namespace neuralrs
