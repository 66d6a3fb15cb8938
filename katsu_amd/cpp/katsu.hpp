// katsu.hpp -- C++ mirror of katsu-core's public API (Tensor, Op, TensorError,
// Conv2D), whose four kernel seams call the gfx950 library through the C ABI
// of include/katsu_hip.h.
//
// The reference (paths relative to its repository root):
//   crates/katsu-core/src/lib.rs:4-8       re-exports Tensor, TensorError, Op, Conv2D
//   crates/katsu-core/src/tensor.rs        Tensor, autograd engine, TensorError
//   crates/katsu-core/src/conv2d.rs        Conv2D layer, Geometry
//
// Names, argument meaning and error behaviour follow the reference.  Rust's
// `Result<T, TensorError>` becomes katsu::Result<T>; `Rc` handles become
// shared_ptr handles (a copy shares the node, as `clone()` does); the
// `RefCell` around a gradient becomes a borrow counter with the same
// GradientBorrowed failures.  Two names differ because they are C++
// keywords or conventions: `Tensor::new` is `Tensor::create`, `Conv2D::new`
// is `Conv2D::create`.
//
// Tensor data lives on the GPU.  A tensor made from host data (create,
// zeros, the seeded weights) keeps that host copy and uploads it on its first
// use by a kernel; every op result, adjoint and gradient is produced and kept
// in device memory, and data() / grad() download it on first access (node
// data is immutable, tensor.rs:96, so the host copy never goes stale).  The
// matmul and its VJPs, both convolution passes, the elementwise ops, sum,
// their VJPs, and the engine's pending buffers all run on the GPU through the
// C ABI; only shape checks and graph bookkeeping stay on the host.  A device
// failure is reported as TensorError::Device, a variant the reference lacks
// (it has no device); data(), which cannot return an error, throws
// katsu::DeviceFault if its download fails.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <variant>
#include <vector>

namespace katsu {

// Thrown by Tensor::data() when the download of a device result fails.
struct DeviceFault : std::runtime_error {
    int status;
    explicit DeviceFault(int st);
};

// tensor.rs:9-30, plus Device for a failed library call and MissingGradient
// for Grad-CAM on an activation map that no backward has reached.
struct TensorError {
    enum class Kind {
        ShapeOverflow,
        InvalidConv,
        MissingForward,
        NonScalarBackward,
        GradientBorrowed,
        DataLength,
        ShapeMismatch,
        RankMismatch,
        MatmulMismatch,
        Allocation,
        Device,
        MissingGradient,
    };
    Kind kind;
    const char *message = "";  // InvalidConv
    size_t a = 0, b = 0;       // DataLength {expected, actual}, RankMismatch {left, right},
                               // MatmulMismatch {left_columns, right_rows}
    int status = 0;            // Device: the katsu_status of the failed call

    // The texts of tensor.rs:32-67.
    std::string to_string() const;
};

// Result<T, TensorError>: a value or an error.
template <class T>
class Result {
   public:
    Result(T value) : v_(std::move(value)) {}
    Result(TensorError e) : v_(std::move(e)) {}
    bool ok() const { return v_.index() == 0; }
    explicit operator bool() const { return ok(); }
    T &value() & { return std::get<0>(v_); }
    T &&value() && { return std::get<0>(std::move(v_)); }
    const T &value() const & { return std::get<0>(v_); }
    const TensorError &error() const { return std::get<1>(v_); }
    bool is(TensorError::Kind k) const { return !ok() && error().kind == k; }

   private:
    std::variant<T, TensorError> v_;
};

struct Unit {};
using Status = Result<Unit>;

// tensor.rs:84-93.
struct Op {
    enum class Kind { Leaf, Add, Mul, Matmul, Conv2D, Sum };
    Kind kind = Kind::Leaf;
    size_t stride = 0, padding = 0;  // Conv2D only
    bool operator==(const Op &o) const {
        return kind == o.kind && stride == o.stride && padding == o.padding;
    }
    bool operator!=(const Op &o) const { return !(*this == o); }
};

class Tensor;
class Conv2D;
struct TensorNode;

// A shared borrow of a node's gradient (Ref<'_, Option<Vec<f32>>>): while it
// lives, backward and zero_grad on that node fail with GradientBorrowed.
class GradRef {
   public:
    GradRef(const GradRef &) = delete;
    GradRef &operator=(const GradRef &) = delete;
    GradRef(GradRef &&o) noexcept : node_(std::exchange(o.node_, nullptr)) {}
    ~GradRef();
    // The Option: empty before the first backward reaches this node.
    const std::optional<std::vector<float>> &operator*() const;
    const std::optional<std::vector<float>> *operator->() const { return &**this; }

   private:
    friend class Tensor;
    explicit GradRef(const TensorNode *n);
    const TensorNode *node_;
};

// tensor.rs:95-107: a shared handle; copies preserve node identity.
class Tensor {
   public:
    // Tensor::new (tensor.rs:149-158): takes the data, checks its length.
    static Result<Tensor> create(std::vector<float> data, const std::vector<size_t> &shape);
    static Result<Tensor> zeros(const std::vector<size_t> &shape);

    const std::vector<size_t> &shape() const;
    // The values (downloaded from the device on first access).
    const std::vector<float> &data() const;
    size_t rank() const { return shape().size(); }
    size_t numel() const;
    // The device copy of the data (uploading host data on first use), or a
    // Device error; null for an empty tensor.  Valid while the node lives.
    Result<const float *> device_data() const;
    Op op() const;
    const std::vector<Tensor> &parents() const;

    Result<GradRef> grad() const;
    Status zero_grad() const;

    Result<Tensor> add(const Tensor &rhs) const;
    Result<Tensor> mul(const Tensor &rhs) const;
    Result<Tensor> sum() const;
    Result<Tensor> matmul(const Tensor &rhs) const;  // seam S1 (GPU)

    Status backward() const;
    Status backward_with(const std::vector<float> &seed) const;
    // backward_with for a seed already on the device (any tensor with this
    // tensor's element count; its values are read, its graph is not).
    Status backward_with(const Tensor &seed) const;

    bool same_node(const Tensor &o) const { return node_ == o.node_; }

    // Crate-internal (Tensor::node, tensor.rs:182-190), and its device form.
    static Tensor node(std::vector<float> data, std::vector<size_t> shape, Op op,
                       std::vector<Tensor> parents);
    static Tensor from_node(std::shared_ptr<TensorNode> n);

   private:
    explicit Tensor(std::shared_ptr<TensorNode> n) : node_(std::move(n)) {}
    Result<Tensor> elementwise(const Tensor &rhs, Op::Kind op) const;
    std::vector<Tensor> topological_order() const;
    friend struct Engine;
    friend class Conv2D;
    std::shared_ptr<TensorNode> node_;
};

// conv2d.rs:14-20.
class Conv2D {
   public:
    // Conv2D::new (seed 42) and new_seeded (conv2d.rs:22-61).
    static Result<Conv2D> create(size_t in_channels, size_t out_channels,
                                 std::pair<size_t, size_t> kernel_size, size_t stride,
                                 size_t padding);
    static Result<Conv2D> new_seeded(size_t in_channels, size_t out_channels,
                                     std::pair<size_t, size_t> kernel_size, size_t stride,
                                     size_t padding, uint64_t seed);
    static Result<Conv2D> from_weights(Tensor weights, size_t stride, size_t padding);

    const Tensor &weights() const { return weights_; }
    size_t in_channels() const { return weights_.shape()[1]; }
    size_t out_channels() const { return weights_.shape()[0]; }
    std::pair<size_t, size_t> kernel_size() const {
        return {weights_.shape()[2], weights_.shape()[3]};
    }
    size_t stride() const { return stride_; }
    size_t padding() const { return padding_; }

    Result<Tensor> forward(const Tensor &input) const;                          // seam S3
    Result<std::pair<Tensor, Tensor>> backward(const Tensor &grad_output) const;  // seam S4
    std::optional<Tensor> get_activation_map() const;
    void clear_cache() const;
    // Grad-CAM of the last forward's activation map, after a backward has
    // given it a gradient (the method docs/conv2d.md outlines; the reference
    // provides only the raw map): channel weights = spatial means of the
    // gradient, ReLU of the weighted channel sum, each map divided by its
    // maximum: [N, OH, OW] maps; with to_input_size, each map resized
    // bilinearly to the input image, [N, H, W].
    Result<Tensor> grad_cam(bool to_input_size = false) const;

   private:
    Conv2D(Tensor w, size_t stride, size_t padding)
        : weights_(std::move(w)), stride_(stride), padding_(padding),
          last_forward_(std::make_shared<std::optional<std::pair<Tensor, Tensor>>>()) {}
    Tensor weights_;
    size_t stride_, padding_;
    // RefCell<Option<(Tensor, Tensor)>>: the last successful forward.
    std::shared_ptr<std::optional<std::pair<Tensor, Tensor>>> last_forward_;
};

// tensor.rs:127-138 (crate-internal, exposed for the tests).
Result<size_t> element_count(const std::vector<size_t> &shape);

// The stem workload's head, which katsu-core has no op
// for, on the device: mean_pool_hw(y) is the [N, C] leaf of per-channel means
// of an NCHW tensor; spread_hw(dp, shape) is the [N, C, H, W] leaf
// dy[n][c][h][w] = dp[n][c] / (H*W), the pool's VJP, to seed
// y.backward_with(dy).
Result<Tensor> mean_pool_hw(const Tensor &y);
Result<Tensor> spread_hw(const Tensor &dp, const std::vector<size_t> &shape);

#ifdef KATSU_TESTING
namespace testing {
// Test support for the all-or-nothing publication of backward_with
// (tensor.rs:341-360), compiled only into test builds (KATSU_TESTING): the
// engine's publication step reports a failed device call
// (TensorError::Device) after n more successful accumulation launches; n < 0
// (the default) never.  Forces the condition from the host, so no kernel
// misbehaves.
void fail_publish_after(int n);
}  // namespace testing
#endif

}  // namespace katsu
