// katsu.cpp -- the C++ mirror of katsu-core (see katsu.hpp).  Every function
// cites the reference code it follows (paths relative to the reference
// repository root, crates/katsu-core/src/).
#include "katsu.hpp"

#include <atomic>
#include <cmath>
#include <new>
#include <stdexcept>
#include <unordered_map>
#include <unordered_set>
#include <utility>

#include "../../include/katsu_hip.h"

namespace katsu {

// A block of device memory from the library's pool, returned on destruction.
class DeviceBuf {
   public:
    DeviceBuf() = default;
    DeviceBuf(const DeviceBuf &) = delete;
    DeviceBuf &operator=(const DeviceBuf &) = delete;
    DeviceBuf(DeviceBuf &&o) noexcept : p_(std::exchange(o.p_, nullptr)), n_(o.n_) {}
    DeviceBuf &operator=(DeviceBuf &&o) noexcept {
        if (this != &o) {
            release();
            p_ = std::exchange(o.p_, nullptr);
            n_ = o.n_;
        }
        return *this;
    }
    ~DeviceBuf() { release(); }
    // count floats; a zero count holds no memory.  Returns a katsu_status.
    int allocate(size_t count) {
        release();
        n_ = count;
        if (count == 0) return KATSU_OK;
        void *p = nullptr;
        const int rc = katsu_hip_malloc(&p, count * sizeof(float));
        p_ = (float *)p;
        return rc;
    }
    float *get() const { return p_; }
    size_t size() const { return n_; }

   private:
    void release() {
        if (p_) (void)katsu_hip_free(p_);
        p_ = nullptr;
    }
    float *p_ = nullptr;
    size_t n_ = 0;
};

struct TensorNode {
    std::vector<size_t> shape;
    size_t count = 0;
    // The data: on the device once uploaded or computed there; on the host
    // when created from host values or once downloaded.
    mutable DeviceBuf dev;
    mutable bool on_device = false;
    mutable std::optional<std::vector<float>> host;
    // RefCell<Option<Vec<f32>>>: the gradient lives on the device; `grad_host`
    // is its downloaded copy, refreshed on grad() after a backward changed
    // it.  `borrows` counts live GradRef guards.
    mutable std::optional<DeviceBuf> grad;
    mutable std::optional<std::vector<float>> grad_host;
    mutable bool grad_host_stale = false;
    mutable int borrows = 0;
    std::vector<Tensor> parents;
    Op op;
};

DeviceFault::DeviceFault(int st)
    : std::runtime_error(std::string("device download failed: ") + katsu_hip_strerror(st)),
      status(st) {}

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

void *stream() { return katsu_hip_stream(); }

// A device buffer of `count` floats (uninitialised), or Device/Allocation.
Result<DeviceBuf> device_buffer(size_t count) {
    DeviceBuf b;
    const int rc = b.allocate(count);
    if (rc == KATSU_E_OOM) return err(TensorError::Kind::Allocation);
    if (rc != KATSU_OK) return device(rc);
    return b;
}


bool checked_mul(size_t a, size_t b, size_t *out) { return !__builtin_mul_overflow(a, b, out); }
bool checked_add(size_t a, size_t b, size_t *out) { return !__builtin_add_overflow(a, b, out); }

}  // namespace

// The fault-injection hook of the all-or-nothing publication test exists
// only in test builds (KATSU_TESTING); elsewhere publication never fails on
// purpose.
namespace testing {
#ifdef KATSU_TESTING
static std::atomic<int> publish_countdown{-1};
void fail_publish_after(int n) { publish_countdown.store(n); }
// True once the countdown set by fail_publish_after reaches zero.
static bool publish_fault() {
    int n = publish_countdown.load();
    while (n >= 0) {
        const int next = n == 0 ? -1 : n - 1;
        if (publish_countdown.compare_exchange_weak(n, next)) return n == 0;
    }
    return false;
}
#else
static constexpr bool publish_fault() { return false; }
#endif
}  // namespace testing

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
        case Kind::MissingGradient:
            return "Grad-CAM requires a backward that reached the activation map";
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
const std::optional<std::vector<float>> &GradRef::operator*() const { return node_->grad_host; }

// ---------------------------------------------------------------------------
// Tensor.

Tensor Tensor::node(std::vector<float> data, std::vector<size_t> shape, Op op,
                    std::vector<Tensor> parents) {
    auto n = std::make_shared<TensorNode>();
    n->count = data.size();
    n->host = std::move(data);
    n->shape = std::move(shape);
    n->op = op;
    n->parents = std::move(parents);
    return Tensor(std::move(n));
}

namespace {
// A node whose data was computed on the device.
Tensor device_node(DeviceBuf data, std::vector<size_t> shape, Op op, std::vector<Tensor> parents,
                   size_t count) {
    auto n = std::make_shared<TensorNode>();
    n->count = count;
    n->dev = std::move(data);
    n->on_device = true;
    n->shape = std::move(shape);
    n->op = op;
    n->parents = std::move(parents);
    return Tensor::from_node(std::move(n));
}
}  // namespace

Tensor Tensor::from_node(std::shared_ptr<TensorNode> n) { return Tensor(std::move(n)); }

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
size_t Tensor::numel() const { return node_->count; }

const std::vector<float> &Tensor::data() const {
    TensorNode &n = *node_;
    if (!n.host) {
        std::vector<float> h(n.count);
        const int rc = katsu_hip_download(h.data(), n.dev.get(), n.count, stream());
        if (rc != KATSU_OK) throw DeviceFault(rc);
        n.host = std::move(h);
    }
    return *n.host;
}

Result<const float *> Tensor::device_data() const {
    TensorNode &n = *node_;
    if (!n.on_device) {
        KATSU_TRY(b, device_buffer(n.count));
        const int rc = katsu_hip_upload(b.get(), n.host->data(), n.count, stream());
        if (rc != KATSU_OK) return device(rc);
        n.dev = std::move(b);
        n.on_device = true;
    }
    return (const float *)n.dev.get();
}

Op Tensor::op() const { return node_->op; }
const std::vector<Tensor> &Tensor::parents() const { return node_->parents; }

// tensor.rs:199-205: fails while the engine holds the gradient mutably
// (which it never does between calls in this single-threaded mirror).  The
// device gradient is downloaded here when a backward has changed it.
Result<GradRef> Tensor::grad() const {
    TensorNode &n = *node_;
    if (n.borrows < 0) return err(TensorError::Kind::GradientBorrowed);
    if (n.grad_host_stale) {
        if (n.borrows != 0) return err(TensorError::Kind::GradientBorrowed);
        std::vector<float> h(n.grad->size());
        const int rc = katsu_hip_download(h.data(), n.grad->get(), h.size(), stream());
        if (rc != KATSU_OK) return device(rc);
        n.grad_host = std::move(h);
        n.grad_host_stale = false;
    }
    return GradRef(node_.get());
}

// tensor.rs:208-215: clears this node only.
Status Tensor::zero_grad() const {
    if (node_->borrows != 0) return err(TensorError::Kind::GradientBorrowed);
    node_->grad.reset();
    node_->grad_host.reset();
    node_->grad_host_stale = false;
    return Unit{};
}

Result<Tensor> Tensor::add(const Tensor &rhs) const { return elementwise(rhs, Op::Kind::Add); }
Result<Tensor> Tensor::mul(const Tensor &rhs) const { return elementwise(rhs, Op::Kind::Mul); }

// tensor.rs:226-240: identical shapes, no broadcasting; on the GPU.
Result<Tensor> Tensor::elementwise(const Tensor &rhs, Op::Kind op) const {
    if (shape() != rhs.shape()) return err(TensorError::Kind::ShapeMismatch);
    KATSU_TRY(a, device_data());
    KATSU_TRY(b, rhs.device_data());
    KATSU_TRY(out, device_buffer(numel()));
    const int rc = op == Op::Kind::Add
                       ? katsu_hip_add_f32_dev(a, b, out.get(), numel(), 0.0f, stream())
                       : katsu_hip_mul_f32_dev(a, b, out.get(), numel(), 0.0f, stream());
    if (rc != KATSU_OK) return device(rc);
    return device_node(std::move(out), shape(), Op{op}, {*this, rhs}, numel());
}

// tensor.rs:242-247: the sum of all elements (0 for an empty tensor), on the
// GPU in a fixed tree.
Result<Tensor> Tensor::sum() const {
    KATSU_TRY(x, device_data());
    KATSU_TRY(out, device_buffer(1));
    const int rc = katsu_hip_sum_f32_dev(x, numel(), out.get(), 0.0f, stream());
    if (rc != KATSU_OK) return device(rc);
    return device_node(std::move(out), {}, Op{Op::Kind::Sum}, {*this}, 1);
}

// tensor.rs:249-280, seam S1.
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
    KATSU_TRY(a, device_data());
    KATSU_TRY(b, rhs.device_data());
    KATSU_TRY(out, device_buffer(count));
    // beta = 0 writes every element; k == 0 gives the zero buffer of :264.
    const int rc = katsu_hip_gemm_f32_dev(a, b, out.get(), m, n, k, 0, 0, 0.0f, stream());
    if (rc != KATSU_OK) return device(rc);
    return device_node(std::move(out), {m, n}, Op{Op::Kind::Matmul}, {*this, rhs}, count);
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
Result<katsu_conv_geom> geometry(const Tensor &input, const Tensor &weights, size_t stride,
                                 size_t padding);
}  // namespace

struct Engine {
    // The adjoint buffer of one node in one backward pass, on the device.
    // `zero` marks a buffer that no adjoint has reached yet: it holds no
    // values, and the first adjoint is written into it (beta = 0) instead of
    // added to a zero fill, which saves a fill and a read of every buffer.
    struct Slot {
        DeviceBuf buf;
        bool zero = true;
        float beta() const { return zero ? 0.0f : 1.0f; }
    };
    using Pending = std::unordered_map<const TensorNode *, Slot>;

    // Op::backward, tensor.rs:365-449: every adjoint accumulated into the
    // device pending buffers in the reference's order.
    static Status op_backward(const Tensor &node, const float *g, Pending &pending) {
        const Op op = node.op();
        const auto &ps = node.parents();
        void *st = stream();
        auto slot = [&](int side) -> Slot & { return pending.at(ps[side].node_.get()); };
        int rc = KATSU_OK;
        switch (op.kind) {
            case Op::Kind::Leaf: break;
            case Op::Kind::Conv2D: {
                // tensor.rs:374-391, seam S4: dx into pending[input], then dw into
                // pending[weights], each fresh adjoint added once as the
                // reference's += of the fresh buffers does.
                KATSU_TRY(geo, geometry(ps[0], ps[1], op.stride, op.padding));
                KATSU_TRY(x, ps[0].device_data());
                KATSU_TRY(w, ps[1].device_data());
                Slot &sx = slot(0), &sw = slot(1);
                if (&sx != &sw && sx.zero == sw.zero) {
                    rc = katsu_hip_conv2d_bwd_f32_dev(x, w, g, sx.buf.get(), sw.buf.get(), &geo,
                                                      sx.beta(), nullptr, 0, st);
                } else {
                    rc = katsu_hip_conv2d_bwd_data_f32_dev(g, w, sx.buf.get(), &geo, sx.beta(), st);
                    sx.zero = false;
                    if (rc == KATSU_OK)
                        rc = katsu_hip_conv2d_bwd_filter_f32_dev(x, g, sw.buf.get(), &geo,
                                                                 sw.beta(), nullptr, 0, st);
                }
                sx.zero = sw.zero = false;
                break;
            }
            case Op::Kind::Add:
                // tensor.rs:392-397: both edges, even when they are one node.
                for (int side = 0; side < 2 && rc == KATSU_OK; ++side) {
                    Slot &t = slot(side);
                    rc = katsu_hip_accumulate_f32_dev(g, t.buf.get(), node.numel(), t.beta(), st);
                    t.zero = false;
                }
                break;
            case Op::Kind::Mul:
                // tensor.rs:398-409: pending[side] += g * other.
                for (int side = 0; side < 2 && rc == KATSU_OK; ++side) {
                    KATSU_TRY(other, ps[1 - side].device_data());
                    Slot &t = slot(side);
                    rc = katsu_hip_mul_f32_dev(g, other, t.buf.get(), node.numel(), t.beta(), st);
                    t.zero = false;
                }
                break;
            case Op::Kind::Sum: {
                // tensor.rs:410-417.
                Slot &t = slot(0);
                rc = katsu_hip_add_scalar_f32_dev(g, t.buf.get(), ps[0].numel(), t.beta(), st);
                t.zero = false;
                break;
            }
            case Op::Kind::Matmul: {
                // tensor.rs:418-445, seam S2: dA += G.B^T, then dB += A^T.G, into
                // the pending buffers (the same buffer when A and B are one
                // node: the entry point then runs them in that order, else as
                // one launch).  dB's beta is read after dA's slot is marked
                // written, so a shared slot accumulates.
                const Tensor &a = ps[0], &b = ps[1];
                const size_t m = a.shape()[0], k = a.shape()[1], n = b.shape()[1];
                if (node.numel() == 0 || k == 0) break;
                KATSU_TRY(ad, a.device_data());
                KATSU_TRY(bd, b.device_data());
                Slot &sa = slot(0);
                const float beta_a = sa.beta();
                sa.zero = false;
                Slot &sb = slot(1);
                const float beta_b = sb.beta();
                sb.zero = false;
                rc = katsu_hip_matmul_vjp_f32_dev(ad, bd, g, sa.buf.get(), sb.buf.get(), m, k, n,
                                                  beta_a, beta_b, st);
                break;
            }
        }
        if (rc != KATSU_OK) return device(rc);
        return Unit{};
    }

    // tensor.rs:316-362: fresh adjoints per call; every gradient slot is
    // checked before any is published, so a failure publishes nothing.  `seed`
    // writes the root's adjoint into its pending buffer.
    template <class SeedFn>
    static Status backward_pass(const Tensor &root, const std::vector<Tensor> &order, SeedFn seed) {
        void *st = stream();
        Engine::Pending pending;
        for (const Tensor &n : order) {
            KATSU_TRY(buf, device_buffer(n.numel()));
            pending.emplace(n.node_.get(), Engine::Slot{std::move(buf), true});
        }
        {
            Engine::Slot &r = pending.at(root.node_.get());
            const int rc = seed(r.buf.get(), st);
            if (rc != KATSU_OK) return device(rc);
            r.zero = false;
        }
        for (auto it = order.rbegin(); it != order.rend(); ++it) {
            Engine::Slot &up = pending.at(it->node_.get());
            if (up.zero) {  // no adjoint reached this node: its upstream is zeros
                const int rc = katsu_hip_fill_f32_dev(up.buf.get(), it->numel(), 0.0f, st);
                if (rc != KATSU_OK) return device(rc);
                up.zero = false;
            }
            Status s = Engine::op_backward(*it, up.buf.get(), pending);
            if (!s.ok()) return s;
        }
        for (const Tensor &n : order)
            if (n.node_->borrows != 0) return err(TensorError::Kind::GradientBorrowed);
        // All or nothing (tensor.rs:341-360): each new gradient is formed in
        // the pass's own pending buffer (stored + pending, the same bits as
        // the reference's `old += new`), and the stored gradients are replaced
        // only once every launch has succeeded.
        for (const Tensor &n : order) {
            const auto &stored = n.node_->grad;
            if (!stored) continue;
            DeviceBuf &gradient = pending.at(n.node_.get()).buf;
            const int rc = testing::publish_fault()
                               ? KATSU_E_LAUNCH
                               : katsu_hip_accumulate_f32_dev(stored->get(), gradient.get(),
                                                              n.numel(), 1.0f, st);
            if (rc != KATSU_OK) return device(rc);
        }
        for (const Tensor &n : order) {
            n.node_->grad = std::move(pending.at(n.node_.get()).buf);
            n.node_->grad_host_stale = true;
        }
        return Unit{};
    }
};

Status Tensor::backward_with(const std::vector<float> &seed) const {
    if (seed.size() != numel()) return data_length(numel(), seed.size());
    // A one-element seed (backward()) is written by a kernel, so the pass
    // never waits on the host; longer seeds are copied in.
    return Engine::backward_pass(*this, topological_order(), [&](float *dst, void *st) {
        return seed.size() == 1 ? katsu_hip_fill_f32_dev(dst, 1, seed[0], st)
                                : katsu_hip_upload(dst, seed.data(), seed.size(), st);
    });
}

Status Tensor::backward_with(const Tensor &seed) const {
    if (seed.numel() != numel()) return data_length(numel(), seed.numel());
    KATSU_TRY(src, seed.device_data());
    return Engine::backward_pass(*this, topological_order(), [&](float *dst, void *st) {
        return katsu_hip_accumulate_f32_dev(src, dst, numel(), 0.0f, st);
    });
}

// The config-5 head on the device (see katsu.hpp).
Result<Tensor> mean_pool_hw(const Tensor &y) {
    if (y.rank() != 4) return invalid_conv("input must be rank 4 (NCHW)");
    const auto &s = y.shape();
    KATSU_TRY(rows, element_count({s[0], s[1]}));
    KATSU_TRY(cols, element_count({s[2], s[3]}));
    KATSU_TRY(src, y.device_data());
    KATSU_TRY(out, device_buffer(rows));
    if (rows > 0) {
        const int rc = cols == 0 ? katsu_hip_fill_f32_dev(out.get(), rows, 0.0f, stream())
                                 : katsu_hip_mean_rows_f32_dev(src, rows, cols, out.get(),
                                                               stream());
        if (rc != KATSU_OK) return device(rc);
    }
    return device_node(std::move(out), {s[0], s[1]}, Op{}, {}, rows);
}

Result<Tensor> spread_hw(const Tensor &dp, const std::vector<size_t> &shape) {
    if (shape.size() != 4 || dp.rank() != 2 || dp.shape()[0] != shape[0] ||
        dp.shape()[1] != shape[1])
        return err(TensorError::Kind::ShapeMismatch);
    KATSU_TRY(rows, element_count({shape[0], shape[1]}));
    KATSU_TRY(cols, element_count({shape[2], shape[3]}));
    KATSU_TRY(count, element_count(shape));
    KATSU_TRY(src, dp.device_data());
    KATSU_TRY(out, device_buffer(count));
    if (count > 0) {
        const int rc = katsu_hip_broadcast_rows_f32_dev(src, rows, cols, 1.0f / (float)cols,
                                                        out.get(), 0.0f, stream());
        if (rc != KATSU_OK) return device(rc);
    }
    return device_node(std::move(out), shape, Op{}, {}, count);
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
// the GPU in one call (beta = 0), kept on the device.
Result<std::pair<DeviceBuf, DeviceBuf>> backward_buffers(const Tensor &input,
                                                         const Tensor &weights,
                                                         const Tensor &grad, size_t stride,
                                                         size_t padding) {
    KATSU_TRY(g, geometry(input, weights, stride, padding));
    KATSU_TRY(expected, element_count({g.n, g.k, g.oh, g.ow}));
    if (grad.numel() != expected) return data_length(expected, grad.numel());
    KATSU_TRY(x, input.device_data());
    KATSU_TRY(w, weights.device_data());
    KATSU_TRY(gy, grad.device_data());
    KATSU_TRY(dx, device_buffer(input.numel()));
    KATSU_TRY(dw, device_buffer(weights.numel()));
    const int rc = katsu_hip_conv2d_bwd_f32_dev(x, w, gy, dx.get(), dw.get(), &g, 0.0f, nullptr,
                                                0, stream());
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
    KATSU_TRY(x, input.device_data());
    KATSU_TRY(w, weights_.device_data());
    KATSU_TRY(y, device_buffer(count));
    const int rc = katsu_hip_conv2d_fwd_f32_dev(x, w, y.get(), &g, stream());
    if (rc != KATSU_OK) return device(rc);
    Op op{Op::Kind::Conv2D, stride_, padding_};
    Tensor out = device_node(std::move(y), shape, op, {input, weights_}, count);
    *last_forward_ = std::make_pair(input, out);
    return out;
}

// conv2d.rs:117-138: the local VJP of the last forward, as leaf tensors.
Result<std::pair<Tensor, Tensor>> Conv2D::backward(const Tensor &grad_output) const {
    if (!*last_forward_) return err(TensorError::Kind::MissingForward);
    const auto &[input, output] = **last_forward_;
    if (grad_output.shape() != output.shape())
        return invalid_conv("grad_output must match the output NCHW shape");
    KATSU_TRY(bufs, backward_buffers(input, weights_, grad_output, stride_, padding_));
    Tensor dx = device_node(std::move(bufs.first), input.shape(), Op{}, {}, input.numel());
    Tensor dw = device_node(std::move(bufs.second), weights_.shape(), Op{}, {}, weights_.numel());
    return std::make_pair(dx, dw);
}

// conv2d.rs:140-148: the same node as the last output (no copy).
std::optional<Tensor> Conv2D::get_activation_map() const {
    if (!*last_forward_) return std::nullopt;
    return (*last_forward_)->second;
}

// conv2d.rs:150-153.
void Conv2D::clear_cache() const { last_forward_->reset(); }

// Grad-CAM over get_activation_map() and its gradient, on the device.
// With to_input_size, the maps are then resized to the input image
// ("redimensionar para a imagem original", docs/conv2d.md).
Result<Tensor> Conv2D::grad_cam(bool to_input_size) const {
    if (!*last_forward_) return err(TensorError::Kind::MissingForward);
    const auto &[input, map] = **last_forward_;
    const TensorNode &n = *map.node_;
    if (!n.grad) return err(TensorError::Kind::MissingGradient);
    const auto &s = map.shape();
    KATSU_TRY(act, map.device_data());
    KATSU_TRY(count, element_count({s[0], s[2], s[3]}));
    KATSU_TRY(out, device_buffer(count));
    int rc = katsu_hip_gradcam_f32_dev(act, n.grad->get(), s[0], s[1], s[2] * s[3], out.get(),
                                       stream());
    if (rc != KATSU_OK) return device(rc);
    if (!to_input_size) return device_node(std::move(out), {s[0], s[2], s[3]}, Op{}, {}, count);
    const auto &is = input.shape();
    KATSU_TRY(rcount, element_count({is[0], is[2], is[3]}));
    KATSU_TRY(resized, device_buffer(rcount));
    rc = katsu_hip_resize_bilinear_f32_dev(out.get(), s[0], s[2], s[3], is[2], is[3],
                                           resized.get(), stream());
    if (rc != KATSU_OK) return device(rc);
    return device_node(std::move(resized), {is[0], is[2], is[3]}, Op{}, {}, rcount);
}

}  // namespace katsu
