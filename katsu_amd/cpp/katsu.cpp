// katsu.cpp -- the C++ mirror of katsu-core (see katsu.hpp).  Every function
// cites the reference code it follows (paths relative to the reference
// repository root, crates/katsu-core/src/).
#include "katsu.hpp"

#include <cmath>
#include <new>
#include <stdexcept>
#include <unordered_map>
#include <unordered_set>

#include "../../include/katsu_hip.h"

namespace katsu {

struct TensorNode {
    std::vector<float> data;
    std::vector<size_t> shape;
    // RefCell<Option<Vec<f32>>>: `borrows` counts live GradRef guards.
    mutable std::optional<std::vector<float>> grad;
    mutable int borrows = 0;
    std::vector<Tensor> parents;
    Op op;
};

namespace {

TensorError err(TensorError::Kind k) { return TensorError{k}; }
TensorError invalid_conv(const char *m) {
    TensorError e{TensorError::Kind::InvalidConv};
    e.message = m;
    return e;
}
TensorError data_length(size_t expected, size_t actual) {
    TensorError e{TensorError::Kind::DataLength};
    e.a = expected;
    e.b = actual;
    return e;
}
TensorError device(int status) {
    TensorError e{TensorError::Kind::Device};
    e.status = status;
    return e;
}

#define KATSU_TRY(var, expr)                         \
    auto var##_r = (expr);                           \
    if (!var##_r.ok()) return var##_r.error();       \
    auto var = std::move(var##_r).value()

// zeros_buffer, tensor.rs:120-125: a failed reservation is Allocation.
Result<std::vector<float>> zeros_buffer(size_t count) {
    try {
        return std::vector<float>(count, 0.0f);
    } catch (const std::bad_alloc &) {
        return err(TensorError::Kind::Allocation);
    } catch (const std::length_error &) {
        return err(TensorError::Kind::Allocation);
    }
}

bool checked_mul(size_t a, size_t b, size_t *out) { return !__builtin_mul_overflow(a, b, out); }
bool checked_add(size_t a, size_t b, size_t *out) { return !__builtin_add_overflow(a, b, out); }

}  // namespace

// tensor.rs:32-67.
std::string TensorError::to_string() const {
    switch (kind) {
        case Kind::InvalidConv: return std::string("invalid Conv2D: ") + message;
        case Kind::MissingForward: return "Conv2D backward requires a successful forward";
        case Kind::NonScalarBackward:
            return "backward requires one element; use sum() or backward_with(seed)";
        case Kind::GradientBorrowed: return "release gradient borrows before backward or zero_grad";
        case Kind::ShapeOverflow: return "shape exceeds addressable tensor storage";
        case Kind::DataLength:
            return "expected " + std::to_string(a) + " elements, got " + std::to_string(b);
        case Kind::ShapeMismatch:
            return "elementwise operations require identical shapes (no broadcasting)";
        case Kind::RankMismatch:
            return "matmul requires rank 2, got " + std::to_string(a) + " and " + std::to_string(b);
        case Kind::MatmulMismatch:
            return "matmul inner dimensions differ: " + std::to_string(a) + " and " +
                   std::to_string(b);
        case Kind::Allocation: return "tensor allocation failed";
        case Kind::Device:
            return std::string("device kernel failed: ") + katsu_hip_strerror(status);
    }
    return "unknown tensor error";
}

// element_count, tensor.rs:127-138: zero dims give 0; the product must not
// overflow and must stay below isize::MAX / size_of::<f32>().
Result<size_t> element_count(const std::vector<size_t> &shape) {
    for (size_t d : shape)
        if (d == 0) return size_t(0);
    size_t count = 1;
    for (size_t d : shape)
        if (!checked_mul(count, d, &count)) return err(TensorError::Kind::ShapeOverflow);
    if (count > (SIZE_MAX >> 1) / sizeof(float)) return err(TensorError::Kind::ShapeOverflow);
    return count;
}

// ---------------------------------------------------------------------------
// GradRef: the Ref guard of Tensor::grad (tensor.rs:199-205).

GradRef::GradRef(const TensorNode *n) : node_(n) { ++node_->borrows; }
GradRef::~GradRef() {
    if (node_) --node_->borrows;
}
const std::optional<std::vector<float>> &GradRef::operator*() const { return node_->grad; }

// ---------------------------------------------------------------------------
// Tensor.

Tensor Tensor::node(std::vector<float> data, std::vector<size_t> shape, Op op,
                    std::vector<Tensor> parents) {
    auto n = std::make_shared<TensorNode>();
    n->data = std::move(data);
    n->shape = std::move(shape);
    n->op = op;
    n->parents = std::move(parents);
    return Tensor(std::move(n));
}

// tensor.rs:149-158.
Result<Tensor> Tensor::create(std::vector<float> data, const std::vector<size_t> &shape) {
    KATSU_TRY(expected, element_count(shape));
    if (data.size() != expected) return data_length(expected, data.size());
    return node(std::move(data), shape, Op{}, {});
}

// tensor.rs:160-166.
Result<Tensor> Tensor::zeros(const std::vector<size_t> &shape) {
    KATSU_TRY(count, element_count(shape));
    KATSU_TRY(data, zeros_buffer(count));
    return node(std::move(data), shape, Op{}, {});
}

const std::vector<size_t> &Tensor::shape() const { return node_->shape; }
const std::vector<float> &Tensor::data() const { return node_->data; }
Op Tensor::op() const { return node_->op; }
const std::vector<Tensor> &Tensor::parents() const { return node_->parents; }

// tensor.rs:199-205: fails while the engine holds the gradient mutably
// (which it never does between calls in this single-threaded mirror).
Result<GradRef> Tensor::grad() const {
    if (node_->borrows < 0) return err(TensorError::Kind::GradientBorrowed);
    return GradRef(node_.get());
}

// tensor.rs:208-215: clears this node only.
Status Tensor::zero_grad() const {
    if (node_->borrows != 0) return err(TensorError::Kind::GradientBorrowed);
    node_->grad.reset();
    return Unit{};
}

Result<Tensor> Tensor::add(const Tensor &rhs) const { return elementwise(rhs, Op::Kind::Add); }
Result<Tensor> Tensor::mul(const Tensor &rhs) const { return elementwise(rhs, Op::Kind::Mul); }

// tensor.rs:226-240: identical shapes, no broadcasting.
Result<Tensor> Tensor::elementwise(const Tensor &rhs, Op::Kind op) const {
    if (shape() != rhs.shape()) return err(TensorError::Kind::ShapeMismatch);
    KATSU_TRY(out, zeros_buffer(numel()));
    const float *a = data().data(), *b = rhs.data().data();
    for (size_t i = 0; i < out.size(); ++i) out[i] = op == Op::Kind::Add ? a[i] + b[i] : a[i] * b[i];
    return node(std::move(out), shape(), Op{op}, {*this, rhs});
}

// tensor.rs:242-247: a sequential f32 fold (0 for an empty tensor).
Result<Tensor> Tensor::sum() const {
    KATSU_TRY(out, zeros_buffer(1));
    float acc = 0.0f;
    for (float v : data()) acc += v;
    out[0] = acc;
    return node(std::move(out), {}, Op{Op::Kind::Sum}, {*this});
}

// tensor.rs:249-280, seam S1: the product runs on the GPU.
Result<Tensor> Tensor::matmul(const Tensor &rhs) const {
    if (rank() != 2 || rhs.rank() != 2) {
        TensorError e{TensorError::Kind::RankMismatch};
        e.a = rank();
        e.b = rhs.rank();
        return e;
    }
    const size_t m = shape()[0], k = shape()[1], n = rhs.shape()[1];
    if (k != rhs.shape()[0]) {
        TensorError e{TensorError::Kind::MatmulMismatch};
        e.a = k;
        e.b = rhs.shape()[0];
        return e;
    }
    KATSU_TRY(count, element_count({m, n}));
    KATSU_TRY(out, zeros_buffer(count));
    if (!out.empty() && k != 0) {
        const int rc = katsu_hip_gemm_f32(data().data(), rhs.data().data(), out.data(), m, n, k,
                                          0, 0, 0.0f);
        if (rc != KATSU_OK) return device(rc);
    }
    return node(std::move(out), {m, n}, Op{Op::Kind::Matmul}, {*this, rhs});
}

// tensor.rs:286-306: iterative DFS, parents before children, deduplicated
// by node identity.
std::vector<Tensor> Tensor::topological_order() const {
    std::vector<Tensor> order;
    std::unordered_set<const TensorNode *> visited;
    std::vector<std::pair<Tensor, bool>> stack{{*this, false}};
    while (!stack.empty()) {
        auto [node, expanded] = stack.back();
        stack.pop_back();
        if (expanded) {
            order.push_back(node);
            continue;
        }
        if (!visited.insert(node.node_.get()).second) continue;
        stack.push_back({node, true});
        const auto &ps = node.parents();
        for (auto it = ps.rbegin(); it != ps.rend(); ++it) stack.push_back({*it, false});
    }
    return order;
}

// tensor.rs:308-314.
Status Tensor::backward() const {
    if (numel() != 1) return err(TensorError::Kind::NonScalarBackward);
    return backward_with({1.0f});
}

namespace {
Result<std::pair<std::vector<float>, std::vector<float>>> backward_buffers(
    const Tensor &input, const Tensor &weights, const std::vector<float> &grad, size_t stride,
    size_t padding);
}  // namespace

struct Engine {
    using Pending = std::unordered_map<const TensorNode *, std::vector<float>>;

    // Op::backward, tensor.rs:365-449.
    static Status op_backward(const Tensor &node, const std::vector<float> &g, Pending &pending) {
        const Op op = node.op();
        const auto &ps = node.parents();
        switch (op.kind) {
            case Op::Kind::Leaf: break;
            case Op::Kind::Conv2D: {
                // tensor.rs:374-391, seam S4: fresh dx, dw from the GPU, then
                // added into the pending buffers one parent after the other.
                KATSU_TRY(grads, backward_buffers(ps[0], ps[1], g, op.stride, op.padding));
                const std::vector<float> *both[2] = {&grads.first, &grads.second};
                for (int side = 0; side < 2; ++side) {
                    std::vector<float> &target = pending.at(ps[side].node_.get());
                    const std::vector<float> &src = *both[side];
                    for (size_t i = 0; i < target.size() && i < src.size(); ++i) target[i] += src[i];
                }
                break;
            }
            case Op::Kind::Add:
            case Op::Kind::Mul:
                // tensor.rs:392-409: both edges, even when they are one node.
                for (int side = 0; side < 2; ++side) {
                    std::vector<float> &target = pending.at(ps[side].node_.get());
                    const std::vector<float> &other = ps[1 - side].data();
                    for (size_t i = 0; i < target.size() && i < g.size(); ++i)
                        target[i] += op.kind == Op::Kind::Add ? g[i] : g[i] * other[i];
                }
                break;
            case Op::Kind::Sum: {
                // tensor.rs:410-417.
                for (float &v : pending.at(ps[0].node_.get())) v += g[0];
                break;
            }
            case Op::Kind::Matmul: {
                // tensor.rs:418-445, seam S2: dA += G.B^T, then dB += A^T.G, on
                // the GPU with beta = 1 into the pending buffers (the same
                // buffer when A and B are one node, hence the order).
                const Tensor &a = ps[0], &b = ps[1];
                const size_t m = a.shape()[0], k = a.shape()[1], n = b.shape()[1];
                if (g.empty() || k == 0) break;
                std::vector<float> &da = pending.at(a.node_.get());
                int rc = katsu_hip_gemm_f32(g.data(), b.data().data(), da.data(), m, k, n, 0, 1,
                                            1.0f);
                if (rc != KATSU_OK) return device(rc);
                std::vector<float> &db = pending.at(b.node_.get());
                rc = katsu_hip_gemm_f32(a.data().data(), g.data(), db.data(), k, n, m, 1, 0, 1.0f);
                if (rc != KATSU_OK) return device(rc);
                break;
            }
        }
        return Unit{};
    }
};

// tensor.rs:316-362: fresh adjoints per call; every gradient slot is
// checked before any is published, so a failure publishes nothing.
Status Tensor::backward_with(const std::vector<float> &seed) const {
    if (seed.size() != numel()) return data_length(numel(), seed.size());
    const std::vector<Tensor> order = topological_order();
    Engine::Pending pending;
    for (const Tensor &n : order) {
        KATSU_TRY(buf, zeros_buffer(n.numel()));
        pending.emplace(n.node_.get(), std::move(buf));
    }
    pending.at(node_.get()) = seed;
    for (auto it = order.rbegin(); it != order.rend(); ++it) {
        const TensorNode *id = it->node_.get();
        std::vector<float> upstream = std::move(pending.at(id));
        pending.erase(id);
        Status st = Engine::op_backward(*it, upstream, pending);
        if (!st.ok()) return st;
        pending.emplace(id, std::move(upstream));
    }
    for (const Tensor &n : order)
        if (n.node_->borrows != 0) return err(TensorError::Kind::GradientBorrowed);
    for (const Tensor &n : order) {
        std::vector<float> &gradient = pending.at(n.node_.get());
        auto &stored = n.node_->grad;
        if (stored) {
            for (size_t i = 0; i < stored->size() && i < gradient.size(); ++i)
                (*stored)[i] += gradient[i];
        } else {
            stored = std::move(gradient);
        }
    }
    return Unit{};
}

// ---------------------------------------------------------------------------
// Conv2D.

namespace {

// validate_weights, conv2d.rs:156-166.
Status validate_weights(const std::vector<size_t> &shape, size_t stride) {
    bool zero = false;
    for (size_t d : shape) zero |= d == 0;
    if (shape.size() != 4 || zero) return invalid_conv("weights must have positive OIHW dimensions");
    if (stride == 0) return invalid_conv("stride must be positive");
    return Unit{};
}

// Geometry::new, conv2d.rs:183-224, filling the library's katsu_conv_geom.
Result<katsu_conv_geom> geometry(const Tensor &input, const Tensor &weights, size_t stride,
                                 size_t padding) {
    Status v = validate_weights(weights.shape(), stride);
    if (!v.ok()) return v.error();
    if (input.rank() != 4) return invalid_conv("input must be rank 4 (NCHW)");
    const auto &x = input.shape();
    const auto &k = weights.shape();
    if (x[1] != k[1] || x[2] == 0 || x[3] == 0)
        return invalid_conv("input channels must match weights; H and W must be positive");
    {
        KATSU_TRY(c, element_count({x[1], x[2], x[3]}));
        (void)c;
    }
    size_t pad2;
    if (!checked_mul(padding, 2, &pad2)) return err(TensorError::Kind::ShapeOverflow);
    auto output_dim = [&](size_t size, size_t kernel) -> Result<size_t> {
        size_t padded, q;
        if (!checked_add(size, pad2, &padded)) return err(TensorError::Kind::ShapeOverflow);
        if (padded < kernel) return invalid_conv("kernel exceeds padded input");
        if (!checked_add((padded - kernel) / stride, 1, &q))
            return err(TensorError::Kind::ShapeOverflow);
        return q;
    };
    KATSU_TRY(oh, output_dim(x[2], k[2]));
    KATSU_TRY(ow, output_dim(x[3], k[3]));
    {
        KATSU_TRY(c1, element_count({k[0], oh, ow}));
        KATSU_TRY(c2, element_count({x[0], k[0], oh, ow}));
        (void)c1;
        (void)c2;
    }
    return katsu_conv_geom{x[0], x[1], x[2], x[3], k[0], k[2], k[3], stride, padding, oh, ow};
}

// backward_buffers, conv2d.rs:269-292, seam S4: fresh dx and dw, both from
// the GPU in one call (beta = 0).
Result<std::pair<std::vector<float>, std::vector<float>>> backward_buffers(
    const Tensor &input, const Tensor &weights, const std::vector<float> &grad, size_t stride,
    size_t padding) {
    KATSU_TRY(g, geometry(input, weights, stride, padding));
    KATSU_TRY(expected, element_count({g.n, g.k, g.oh, g.ow}));
    if (grad.size() != expected) return data_length(expected, grad.size());
    KATSU_TRY(dx, zeros_buffer(input.numel()));
    KATSU_TRY(dw, zeros_buffer(weights.numel()));
    const int rc = katsu_hip_conv2d_bwd_f32(input.data().data(), weights.data().data(),
                                            grad.data(), dx.data(), dw.data(), &g, 0.0f);
    if (rc != KATSU_OK) return device(rc);
    return std::make_pair(std::move(dx), std::move(dw));
}

}  // namespace

// Conv2D::new, conv2d.rs:25-33 (default seed 42).
Result<Conv2D> Conv2D::create(size_t in_channels, size_t out_channels,
                              std::pair<size_t, size_t> kernel_size, size_t stride,
                              size_t padding) {
    return new_seeded(in_channels, out_channels, kernel_size, stride, padding, 42);
}

// conv2d.rs:35-61: SplitMix64 (the published generator), uniform =
// (z >> 40) / 2^24, w = (2 uniform - 1) / sqrt(fan_in), all in f32.
Result<Conv2D> Conv2D::new_seeded(size_t in_channels, size_t out_channels,
                                  std::pair<size_t, size_t> kernel_size, size_t stride,
                                  size_t padding, uint64_t seed) {
    const std::vector<size_t> shape{out_channels, in_channels, kernel_size.first,
                                    kernel_size.second};
    Status v = validate_weights(shape, stride);
    if (!v.ok()) return v.error();
    size_t pad2;
    if (!checked_mul(padding, 2, &pad2)) return err(TensorError::Kind::ShapeOverflow);
    KATSU_TRY(count, element_count(shape));
    KATSU_TRY(data, zeros_buffer(count));
    KATSU_TRY(fan_in, element_count({shape[1], shape[2], shape[3]}));
    const float bound = 1.0f / std::sqrt((float)fan_in);
    uint64_t state = seed;
    for (float &value : data) {
        state += 0x9e3779b97f4a7c15ull;
        uint64_t z = state;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z ^= z >> 31;
        const float uniform = (float)(z >> 40) / 16777216.0f;
        value = (2.0f * uniform - 1.0f) * bound;
    }
    KATSU_TRY(w, Tensor::create(std::move(data), shape));
    return from_weights(std::move(w), stride, padding);
}

// conv2d.rs:63-74: keeps the weights' identity and graph.
Result<Conv2D> Conv2D::from_weights(Tensor weights, size_t stride, size_t padding) {
    Status v = validate_weights(weights.shape(), stride);
    if (!v.ok()) return v.error();
    size_t pad2;
    if (!checked_mul(padding, 2, &pad2)) return err(TensorError::Kind::ShapeOverflow);
    return Conv2D(std::move(weights), stride, padding);
}

// conv2d.rs:95-115, seam S3: the cache is replaced only after success.
Result<Tensor> Conv2D::forward(const Tensor &input) const {
    KATSU_TRY(g, geometry(input, weights_, stride_, padding_));
    const std::vector<size_t> shape{g.n, g.k, g.oh, g.ow};
    KATSU_TRY(count, element_count(shape));
    KATSU_TRY(data, zeros_buffer(count));
    if (!data.empty()) {
        const int rc = katsu_hip_conv2d_fwd_f32(input.data().data(), weights_.data().data(),
                                                data.data(), &g);
        if (rc != KATSU_OK) return device(rc);
    }
    Op op{Op::Kind::Conv2D, stride_, padding_};
    Tensor out = Tensor::node(std::move(data), shape, op, {input, weights_});
    *last_forward_ = std::make_pair(input, out);
    return out;
}

// conv2d.rs:117-138: the local VJP of the last forward, as leaf tensors.
Result<std::pair<Tensor, Tensor>> Conv2D::backward(const Tensor &grad_output) const {
    if (!*last_forward_) return err(TensorError::Kind::MissingForward);
    const auto &[input, output] = **last_forward_;
    if (grad_output.shape() != output.shape())
        return invalid_conv("grad_output must match the output NCHW shape");
    KATSU_TRY(bufs, backward_buffers(input, weights_, grad_output.data(), stride_, padding_));
    KATSU_TRY(dx, Tensor::create(std::move(bufs.first), input.shape()));
    KATSU_TRY(dw, Tensor::create(std::move(bufs.second), weights_.shape()));
    return std::make_pair(dx, dw);
}

// conv2d.rs:140-148: the same node as the last output (no copy).
std::optional<Tensor> Conv2D::get_activation_map() const {
    if (!*last_forward_) return std::nullopt;
    return (*last_forward_)->second;
}

// conv2d.rs:150-153.
void Conv2D::clear_cache() const { last_forward_->reset(); }

}  // namespace katsu
