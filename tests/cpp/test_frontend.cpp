// test_frontend.cpp -- the reference's 19 integration tests, ported one to
// one onto the C++ front end (katsu_amd/cpp/katsu.hpp), whose matmul and
// convolutions run on the GPU through the C ABI.
//
// Each test names the reference test it ports (paths relative to the
// reference repository root, crates/katsu-core/tests/).  Usage:
//   test_frontend            run every test
//   test_frontend NAME...    run the named tests
// Output: one line per test, "PASS name" or "FAIL name: reason"; the exit
// status is the number of failures.
#include <cmath>
#include <cstdio>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <limits>
#include <string>
#include <vector>

#include "../../katsu_amd/cpp/katsu.hpp"

using katsu::Conv2D;
using katsu::Op;
using katsu::Tensor;
using katsu::TensorError;
using Kind = TensorError::Kind;

namespace {

struct Failure {
    std::string what;
};

#define CHECK(cond)                                                                          \
    do {                                                                                     \
        if (!(cond)) throw Failure{std::string(__FILE__ ":") + std::to_string(__LINE__) +    \
                                   ": " #cond};                                              \
    } while (0)

// `?`: unwrap a Result or fail the test with the error's text.
template <class R>
auto unwrap(R &&r, int line) {
    if (!r.ok()) throw Failure{"line " + std::to_string(line) + ": " + r.error().to_string()};
    return std::forward<R>(r).value();
}
#define TRY(expr) unwrap((expr), __LINE__)

// matches!(expr, Err(Kind::..))
#define CHECK_ERR(expr, kind) CHECK((expr).is(kind))

std::vector<float> grad(const Tensor &t) {
    auto g = TRY(t.grad());
    CHECK(g->has_value());
    return **g;
}

bool grad_is_none(const Tensor &t) {
    auto g = TRY(t.grad());
    return !g->has_value();
}

using V = std::vector<float>;
const size_t USIZE_MAX = std::numeric_limits<size_t>::max();
const size_t ISIZE_MAX = USIZE_MAX >> 1;

// tests/conv2d.rs:5-13: |x - y| <= tol * (1 + max(|x|, |y|)).
void close(const V &a, const V &b, float tol) {
    CHECK(a.size() == b.size());
    for (size_t i = 0; i < a.size(); ++i)
        if (!(std::fabs(a[i] - b[i]) <= tol * (1.0f + std::fmax(std::fabs(a[i]), std::fabs(b[i])))))
            throw Failure{"element " + std::to_string(i) + ": " + std::to_string(a[i]) +
                          " != " + std::to_string(b[i])};
}

// ---- tests/tensor.rs --------------------------------------------------------

void validates_data_and_storage_size() {  // tensor.rs:4-17
    CHECK_ERR(Tensor::create({1.0f}, {2}), Kind::DataLength);
    CHECK_ERR(Tensor::zeros({USIZE_MAX, 2}), Kind::ShapeOverflow);
    CHECK_ERR(Tensor::zeros({ISIZE_MAX}), Kind::ShapeOverflow);
}

void scalar_and_empty_shapes() {  // tensor.rs:20-25
    CHECK(TRY(Tensor::create({3.0f}, {})).rank() == 0);
    CHECK(TRY(Tensor::zeros({})).data() == V{0.0f});
    CHECK(TRY(Tensor::zeros({USIZE_MAX, 0})).numel() == 0);
}

void addition_preserves_inputs() {  // tensor.rs:28-38
    auto a = TRY(Tensor::create({1.0f, 2.0f}, {2}));
    auto b = TRY(Tensor::create({3.0f, 4.0f}, {2}));
    CHECK(TRY(a.add(b)).data() == (V{4.0f, 6.0f}));
    CHECK(a.data() == (V{1.0f, 2.0f}));
    CHECK_ERR(a.add(TRY(Tensor::zeros({1, 2}))), Kind::ShapeMismatch);
}

void rectangular_matmul() {  // tensor.rs:41-48
    auto a = TRY(Tensor::create({1, 2, 3, 4, 5, 6}, {2, 3}));
    auto b = TRY(Tensor::create({7, 8, 9, 10, 11, 12}, {3, 2}));
    auto c = TRY(a.matmul(b));
    CHECK(c.shape() == (std::vector<size_t>{2, 2}));
    CHECK(c.data() == (V{58, 64, 139, 154}));
}

void rejects_invalid_matmul() {  // tensor.rs:51-62
    auto a = TRY(Tensor::zeros({2, 3}));
    CHECK_ERR(a.matmul(TRY(Tensor::zeros({2, 2}))), Kind::MatmulMismatch);
    CHECK_ERR(a.matmul(TRY(Tensor::zeros({3}))), Kind::RankMismatch);
}

void empty_matmul_and_output_overflow() {  // tensor.rs:65-86
    auto c = TRY(TRY(Tensor::zeros({2, 0})).matmul(TRY(Tensor::zeros({0, 3}))));
    CHECK(c.shape() == (std::vector<size_t>{2, 3}));
    CHECK(c.data() == V(6, 0.0f));
    CHECK(TRY(TRY(Tensor::zeros({0, 2})).matmul(TRY(Tensor::zeros({2, 3})))).shape() ==
          (std::vector<size_t>{0, 3}));
    CHECK(TRY(TRY(Tensor::zeros({USIZE_MAX, 0})).matmul(TRY(Tensor::zeros({0, 0})))).numel() ==
          0);
    CHECK_ERR(TRY(Tensor::zeros({USIZE_MAX, 0})).matmul(TRY(Tensor::zeros({0, 2}))),
              Kind::ShapeOverflow);
}

// ---- tests/autograd.rs ------------------------------------------------------

void squared_error_shared_nodes_and_repeated_backward() {  // autograd.rs:8-28
    auto a = TRY(Tensor::create({1, 2}, {2}));
    auto b = TRY(Tensor::create({3, 4}, {2}));
    auto s = TRY(a.add(b));
    auto loss = TRY(TRY(s.mul(s)).sum());
    CHECK(s.op() == Op{Op::Kind::Add});
    CHECK(s.parents().size() == 2);
    CHECK(grad_is_none(a));
    TRY(loss.backward());
    CHECK(loss.data() == V{52});
    CHECK(grad(a) == (V{8, 12}));
    CHECK(grad(b) == (V{8, 12}));
    CHECK(grad(s) == (V{8, 12}));
    TRY(loss.backward());
    CHECK(grad(a) == (V{16, 24}));
    TRY(a.zero_grad());
    TRY(loss.backward());
    CHECK(grad(a) == (V{8, 12}));
    CHECK(grad(b) == (V{24, 36}));
}

void diamond_and_clone_identity() {  // autograd.rs:31-39
    auto x = TRY(Tensor::create({2}, {}));
    Tensor alias = x;
    auto square = TRY(x.mul(alias));
    TRY(TRY(square.add(TRY(square.mul(x)))).backward());  // x^2 + x^3
    CHECK(grad(alias) == V{16});
    CHECK(grad(square) == V{3});
}

void explicit_seed_and_errors_are_atomic() {  // autograd.rs:42-60
    auto x = TRY(Tensor::create({2, 3}, {2}));
    auto y = TRY(x.mul(x));
    CHECK_ERR(y.backward(), Kind::NonScalarBackward);
    CHECK_ERR(y.backward_with({1}), Kind::DataLength);
    {
        auto borrowed = TRY(x.grad());
        CHECK_ERR(y.backward_with({2, 4}), Kind::GradientBorrowed);
        CHECK(grad_is_none(y));
    }
    TRY(y.backward_with({2, 4}));
    CHECK(grad(x) == (V{8, 24}));
}

void matmul_finite_differences() {  // autograd.rs:63-95
    const V av{0.2f, -0.4f, 0.7f, 0.3f, 0.8f, -0.1f};
    const V bv{0.1f, 0.5f, -0.3f, 0.6f, 0.9f, -0.2f};
    auto eval = [](V a, V b) {
        auto y = TRY(TRY(Tensor::create(a, {2, 3})).matmul(TRY(Tensor::create(b, {3, 2}))));
        return TRY(TRY(y.mul(y)).sum()).data()[0];
    };
    auto a = TRY(Tensor::create(av, {2, 3}));
    auto b = TRY(Tensor::create(bv, {3, 2}));
    auto y = TRY(a.matmul(b));
    TRY(TRY(TRY(y.mul(y)).sum()).backward());
    for (int side = 0; side < 2; ++side) {
        const V analytical = side == 0 ? grad(a) : grad(b);
        for (int i = 0; i < 6; ++i) {
            V ap = av, am = av, bp = bv, bm = bv;
            const float eps = 0.001f;
            if (side == 0) {
                ap[i] += eps;
                am[i] -= eps;
            } else {
                bp[i] += eps;
                bm[i] -= eps;
            }
            const float numerical = (eval(ap, bp) - eval(am, bm)) / (2.0f * eps);
            CHECK(std::fabs(analytical[i] - numerical) < 0.001f);
        }
    }
}

void matmul_same_parent_accumulates_both_edges() {  // autograd.rs:98-103
    auto a = TRY(Tensor::create({1, 2, 3, 4}, {2, 2}));
    TRY(TRY(TRY(a.matmul(a)).sum()).backward());
    CHECK(grad(a) == (V{7, 11, 9, 13}));
}

void empty_graph_operations() {  // autograd.rs:106-116
    auto a = TRY(Tensor::zeros({2, 0}));
    auto b = TRY(Tensor::zeros({0, 3}));
    TRY(TRY(TRY(a.matmul(b)).sum()).backward());
    CHECK(grad(a).empty());
    CHECK(grad(b).empty());
    auto x = TRY(Tensor::zeros({0}));
    TRY(TRY(TRY(TRY(x.mul(x)).add(x)).sum()).backward());
    CHECK(grad(x).empty());
}

// ---- tests/conv2d.rs --------------------------------------------------------

V iota1(int n) {
    V v;
    for (int i = 1; i <= n; ++i) v.push_back((float)i);
    return v;
}

void known_forward_and_overlap_gradients() {  // conv2d.rs:16-43
    auto x = TRY(Tensor::create(iota1(9), {1, 1, 3, 3}));
    auto layer = TRY(Conv2D::from_weights(TRY(Tensor::create({1, 2, 3, 4}, {1, 1, 2, 2})), 1, 0));
    CHECK(!layer.get_activation_map().has_value());
    auto y = TRY(layer.forward(x));
    CHECK(y.shape() == (std::vector<size_t>{1, 1, 2, 2}));
    CHECK(y.data() == (V{37, 47, 67, 77}));
    auto g = TRY(Tensor::create(V(4, 1.0f), y.shape()));
    auto [dx, dw] = TRY(layer.backward(g));
    CHECK(dx.data() == (V{1, 3, 2, 4, 10, 6, 3, 7, 4}));
    CHECK(dw.data() == (V{12, 16, 24, 28}));
    CHECK(grad_is_none(x));  // the local VJP publishes no gradients
    TRY(TRY(y.sum()).backward());
    close(grad(x), dx.data(), 0.0f);
    close(grad(layer.weights()), dw.data(), 0.0f);
    auto map = layer.get_activation_map();
    CHECK(map.has_value());
    CHECK(grad(*map) == V(4, 1.0f));
    layer.clear_cache();
    CHECK(!layer.get_activation_map().has_value());
    CHECK_ERR(layer.backward(g), Kind::MissingForward);
    // the original handle stays valid after the cache is released
    TRY(TRY(y.sum()).backward());
    CHECK(grad(x)[0] == 2.0f);
}

void finite_differences_input_and_weights() {  // conv2d.rs:46-87
    const std::pair<size_t, size_t> cases[] = {{1, 0}, {1, 1}, {2, 1}};
    for (auto [stride, padding] : cases) {
        const std::vector<size_t> xs{2, 2, 3, 4}, ws{2, 2, 2, 3};
        V xv, wv;
        for (int i = 0; i < 48; ++i) xv.push_back((float)(i % 11) * 0.07f - 0.3f);
        for (int i = 0; i < 24; ++i) wv.push_back((float)(i % 7) * 0.09f - 0.2f);
        auto x = TRY(Tensor::create(xv, xs));
        auto layer = TRY(Conv2D::from_weights(TRY(Tensor::create(wv, ws)), stride, padding));
        auto y = TRY(layer.forward(x));
        V seed;
        for (size_t i = 0; i < y.numel(); ++i) seed.push_back((float)(i % 5) * 0.13f - 0.2f);
        auto [dx, dw] = TRY(layer.backward(TRY(Tensor::create(seed, y.shape()))));
        TRY(y.backward_with(seed));
        close(grad(x), dx.data(), 1e-6f);
        close(grad(layer.weights()), dw.data(), 1e-6f);
        auto eval = [&](V data, V weights) {
            auto conv = TRY(Conv2D::from_weights(TRY(Tensor::create(weights, ws)), stride, padding));
            auto out = TRY(conv.forward(TRY(Tensor::create(data, xs))));
            float acc = 0.0f;
            for (size_t i = 0; i < out.numel(); ++i) acc += out.data()[i] * seed[i];
            return acc;
        };
        for (int side = 0; side < 2; ++side) {
            const V analytical = side == 0 ? dx.data() : dw.data();
            for (size_t i = 0; i < analytical.size(); ++i) {
                V xp = xv, xm = xv, wp = wv, wm = wv;
                const float eps = 0.001f;
                if (side == 0) {
                    xp[i] += eps;
                    xm[i] -= eps;
                } else {
                    wp[i] += eps;
                    wm[i] -= eps;
                }
                const float numerical = (eval(xp, wp) - eval(xm, wm)) / (2.0f * eps);
                close({analytical[i]}, {numerical}, 3e-4f);
            }
        }
    }
}

void reused_layer_keeps_independent_graphs() {  // conv2d.rs:90-106
    auto layer = TRY(Conv2D::from_weights(TRY(Tensor::create({2}, {1, 1, 1, 1})), 1, 0));
    auto a = TRY(Tensor::create({3}, {1, 1, 1, 1}));
    auto b = TRY(Tensor::create({5}, {1, 1, 1, 1}));
    auto ya = TRY(layer.forward(a));
    auto yb = TRY(layer.forward(b));
    TRY(TRY(TRY(ya.add(yb)).sum()).backward());
    CHECK(grad(layer.weights()) == V{8});
    CHECK(grad(a) == V{2});
    CHECK(grad(b) == V{2});
    auto [unused, dw] = TRY(layer.backward(TRY(Tensor::create({1}, yb.shape()))));
    (void)unused;
    CHECK(dw.data() == V{5});
    // an invalid forward keeps the last successful cache
    CHECK(!layer.forward(TRY(Tensor::zeros({1}))).ok());
    CHECK(layer.get_activation_map()->data() == V{10});
}

void shared_operand_and_chained_convolution() {  // conv2d.rs:109-116
    auto x = TRY(Tensor::create({2}, {1, 1, 1, 1}));
    auto layer = TRY(Conv2D::from_weights(x, 1, 0));
    auto y = TRY(layer.forward(x));                       // x^2
    TRY(TRY(TRY(layer.forward(y)).sum()).backward());      // x^3
    CHECK(grad(x) == V{12});
}

void invalid_shapes_and_overflow() {  // conv2d.rs:119-142
    CHECK(!Conv2D::create(0, 1, {3, 3}, 1, 0).ok());
    CHECK(!Conv2D::create(1, 1, {0, 3}, 1, 0).ok());
    CHECK(!Conv2D::create(1, 1, {1, 1}, 0, 0).ok());
    CHECK(!Conv2D::from_weights(TRY(Tensor::zeros({1, 1, 1})), 1, 0).ok());
    CHECK(!Conv2D::create(1, 1, {1, 1}, 1, USIZE_MAX).ok());
    auto layer = TRY(Conv2D::create(1, 1, {3, 3}, 1, 0));
    CHECK_ERR(layer.backward(TRY(Tensor::zeros({1}))), Kind::MissingForward);
    CHECK(!layer.forward(TRY(Tensor::zeros({1, 2, 3, 3}))).ok());
    CHECK(!layer.forward(TRY(Tensor::zeros({1, 1, 2, 2}))).ok());
    CHECK(!layer.forward(TRY(Tensor::zeros({1, 1, 0, 2}))).ok());
    TRY(layer.forward(TRY(Tensor::zeros({1, 1, 3, 3}))));
    // same numel, wrong rank
    CHECK(!layer.backward(TRY(Tensor::zeros({1}))).ok());
    auto huge_pad = TRY(Conv2D::create(1, 1, {1, 1}, 1, USIZE_MAX / 2));
    CHECK_ERR(huge_pad.forward(TRY(Tensor::zeros({0, 1, 2, 2}))), Kind::ShapeOverflow);
}

void empty_batch_and_seeded_initialization() {  // conv2d.rs:145-169
    auto layer = TRY(Conv2D::new_seeded(3, 2, {3, 3}, 1, 1, 7));
    auto same = TRY(Conv2D::new_seeded(3, 2, {3, 3}, 1, 1, 7));
    auto other = TRY(Conv2D::new_seeded(3, 2, {3, 3}, 1, 1, 8));
    CHECK(layer.weights().data() == same.weights().data());
    CHECK(layer.weights().data() != other.weights().data());
    for (float w : layer.weights().data()) CHECK(std::fabs(w) <= 1.0f / std::sqrt(27.0f));
    auto x = TRY(Tensor::zeros({0, 3, 4, 5}));
    auto y = TRY(layer.forward(x));
    CHECK(y.shape() == (std::vector<size_t>{0, 2, 4, 5}));
    TRY(TRY(y.sum()).backward());
    CHECK(grad(x).empty());
    for (float w : grad(layer.weights())) CHECK(w == 0.0f);
}

// ---- beyond the reference's tests: the device engine's own features -----------

// The stem workload's chain on the device: pool, matmul
// head, sum, backward into the pooled leaf, spread, and the conv backward
// seeded with it.  The chain's gradients must equal the layer's local VJP of
// the same seed bit for bit (same kernels, written into fresh buffers), the
// pool must match a host mean, and dP must be the row sums of the head.
void stem_chain_on_device() {
    const size_t N = 2, C = 3, K = 4, J = 5;
    V xs(N * C * 9 * 11);
    for (size_t i = 0; i < xs.size(); ++i) xs[i] = (float)((i * 37) % 101) / 101.0f;
    auto x = TRY(Tensor::create(xs, {N, C, 9, 11}));
    auto layer = TRY(Conv2D::new_seeded(C, K, {3, 3}, 2, 1, 5));
    auto y = TRY(layer.forward(x));
    const size_t OH = y.shape()[2], OW = y.shape()[3];
    auto p = TRY(katsu::mean_pool_hw(y));
    CHECK(p.shape() == (std::vector<size_t>{N, K}));
    const V &yd = y.data();
    for (size_t r = 0; r < N * K; ++r) {
        double acc = 0;
        for (size_t i = 0; i < OH * OW; ++i) acc += yd[r * OH * OW + i];
        CHECK(std::fabs(p.data()[r] - acc / (OH * OW)) <= 1e-6 * (1 + std::fabs(acc)));
    }
    V hs(K * J);
    for (size_t i = 0; i < hs.size(); ++i) hs[i] = 0.25f * (float)((int)(i % 7) - 3);
    auto h = TRY(Tensor::create(hs, {K, J}));
    TRY(TRY(TRY(p.matmul(h)).sum()).backward());
    const V dp = grad(p);
    for (size_t n = 0; n < N; ++n)
        for (size_t k = 0; k < K; ++k) {
            float row = 0;
            for (size_t j = 0; j < J; ++j) row += hs[k * J + j];
            CHECK(dp[n * K + k] == row);  // sums of quarter-integers: exact
        }
    auto dp_t = TRY(Tensor::create(dp, {N, K}));
    auto dy = TRY(katsu::spread_hw(dp_t, y.shape()));
    for (size_t i = 0; i < dy.numel(); ++i)
        CHECK(dy.data()[i] == dp[i / (OH * OW)] * (1.0f / (float)(OH * OW)));
    TRY(y.backward_with(dy));
    auto [dx, dw] = TRY(layer.backward(dy));
    CHECK(grad(x) == dx.data());
    CHECK(grad(layer.weights()) == dw.data());
}

// Grad-CAM on the repository example's shapes (a seeded 3->8 layer, loss
// sum(y*y)), against the same formula evaluated on the host from the map and
// its downloaded gradient.
void grad_cam_on_device() {
    auto layer = TRY(Conv2D::new_seeded(3, 8, {3, 3}, 1, 1, 123));
    CHECK_ERR(layer.grad_cam(), Kind::MissingForward);
    V xs(2 * 3 * 12 * 10);
    for (size_t i = 0; i < xs.size(); ++i) xs[i] = (float)(i % 256) / 255.0f;
    auto x = TRY(Tensor::create(xs, {2, 3, 12, 10}));
    auto y = TRY(layer.forward(x));
    CHECK_ERR(layer.grad_cam(), Kind::MissingGradient);
    TRY(TRY(TRY(y.mul(y)).sum()).backward());
    auto cam = TRY(layer.grad_cam());
    CHECK(cam.shape() == (std::vector<size_t>{2, 12, 10}));
    const V &a = y.data();
    const V g = grad(y);
    const size_t C = 8, HW = 120;
    for (size_t n = 0; n < 2; ++n) {
        std::vector<double> ref(HW, 0.0);
        double mx = 0;
        for (size_t p = 0; p < HW; ++p) {
            double v = 0;
            for (size_t c = 0; c < C; ++c) {
                double alpha = 0;
                for (size_t q = 0; q < HW; ++q) alpha += g[(n * C + c) * HW + q];
                v += alpha / HW * a[(n * C + c) * HW + p];
            }
            ref[p] = v > 0 ? v : 0;
            mx = std::fmax(mx, ref[p]);
        }
        for (size_t p = 0; p < HW; ++p) {
            const double want = mx > 0 ? ref[p] / mx : 0;
            CHECK(std::fabs(cam.data()[n * HW + p] - want) <= 1e-5);
        }
    }
}

// Grad-CAM resized to the input image on a stride-2 layer ([2,3,12,10] ->
// maps [2,6,5] -> [2,12,10]): the resized maps equal the bilinear
// half-pixel-centre formula, evaluated in double on the host from the
// unresized maps; the unresized call is unchanged by the option.
void grad_cam_resized_to_input() {
    auto layer = TRY(Conv2D::new_seeded(3, 8, {3, 3}, 2, 1, 321));
    V xs(2 * 3 * 12 * 10);
    for (size_t i = 0; i < xs.size(); ++i) xs[i] = (float)((i * 37) % 251) / 125.0f - 1.0f;
    auto x = TRY(Tensor::create(xs, {2, 3, 12, 10}));
    auto y = TRY(layer.forward(x));
    CHECK(y.shape() == (std::vector<size_t>{2, 8, 6, 5}));
    TRY(TRY(TRY(y.mul(y)).sum()).backward());
    auto small = TRY(layer.grad_cam());
    auto big = TRY(layer.grad_cam(true));
    CHECK(small.shape() == (std::vector<size_t>{2, 6, 5}));
    CHECK(big.shape() == (std::vector<size_t>{2, 12, 10}));
    const V &s = small.data(), &b = big.data();
    const size_t IH = 6, IW = 5, OH = 12, OW = 10;
    double worst = 0;
    for (size_t n = 0; n < 2; ++n)
        for (size_t oy = 0; oy < OH; ++oy)
            for (size_t ox = 0; ox < OW; ++ox) {
                const double sy = std::fmax((oy + 0.5) * IH / OH - 0.5, 0.0);
                const double sx = std::fmax((ox + 0.5) * IW / OW - 0.5, 0.0);
                const size_t y0 = std::min((size_t)sy, IH - 1), x0 = std::min((size_t)sx, IW - 1);
                const size_t y1 = std::min(y0 + 1, IH - 1), x1 = std::min(x0 + 1, IW - 1);
                const double fy = sy - y0, fx = sx - x0;
                const float *m = s.data() + n * IH * IW;
                const double want = (1 - fy) * ((1 - fx) * m[y0 * IW + x0] + fx * m[y0 * IW + x1]) +
                                    fy * ((1 - fx) * m[y1 * IW + x0] + fx * m[y1 * IW + x1]);
                worst = std::fmax(worst, std::fabs(b[(n * OH + oy) * OW + ox] - want));
            }
    CHECK(worst <= 1e-6);
}

// backward_with publishes all gradients or none (tensor.rs:341-360): a device
// failure after the first node's accumulation leaves every stored gradient
// as it was; the next pass accumulates into all of them.
void publish_is_all_or_nothing() {
    auto a = TRY(Tensor::create({1, 2, 3, 4}, {2, 2}));
    auto b = TRY(Tensor::create({5, 6, 7, 8}, {2, 2}));
    auto loss = TRY(TRY(a.matmul(b)).sum());
    TRY(loss.backward());
    const V ga = grad(a), gb = grad(b);
    katsu::testing::fail_publish_after(1);
    auto failed = loss.backward();
    katsu::testing::fail_publish_after(-1);
    CHECK(!failed.ok());
    CHECK(failed.is(Kind::Device));
    CHECK(grad(a) == ga);
    CHECK(grad(b) == gb);
    TRY(loss.backward());
    V ga2(ga.size()), gb2(gb.size());
    for (size_t i = 0; i < ga.size(); ++i) ga2[i] = 2 * ga[i];
    for (size_t i = 0; i < gb.size(); ++i) gb2[i] = 2 * gb[i];
    CHECK(grad(a) == ga2);  // small integers: exact
    CHECK(grad(b) == gb2);
}

void known_stride_and_padding() {  // conv2d.rs:172-179
    auto x = TRY(Tensor::create(iota1(9), {1, 1, 3, 3}));
    auto layer = TRY(Conv2D::from_weights(TRY(Tensor::create({1, 2, 3, 4}, {1, 1, 2, 2})), 2, 1));
    auto y = TRY(layer.forward(x));
    CHECK(y.shape() == (std::vector<size_t>{1, 1, 2, 2}));
    CHECK(y.data() == (V{4, 18, 36, 77}));
}

struct Case {
    const char *name;
    void (*fn)();
};

const Case kCases[] = {
    {"validates_data_and_storage_size", validates_data_and_storage_size},
    {"scalar_and_empty_shapes", scalar_and_empty_shapes},
    {"addition_preserves_inputs", addition_preserves_inputs},
    {"rectangular_matmul", rectangular_matmul},
    {"rejects_invalid_matmul", rejects_invalid_matmul},
    {"empty_matmul_and_output_overflow", empty_matmul_and_output_overflow},
    {"squared_error_shared_nodes_and_repeated_backward",
     squared_error_shared_nodes_and_repeated_backward},
    {"diamond_and_clone_identity", diamond_and_clone_identity},
    {"explicit_seed_and_errors_are_atomic", explicit_seed_and_errors_are_atomic},
    {"matmul_finite_differences", matmul_finite_differences},
    {"matmul_same_parent_accumulates_both_edges", matmul_same_parent_accumulates_both_edges},
    {"empty_graph_operations", empty_graph_operations},
    {"known_forward_and_overlap_gradients", known_forward_and_overlap_gradients},
    {"finite_differences_input_and_weights", finite_differences_input_and_weights},
    {"reused_layer_keeps_independent_graphs", reused_layer_keeps_independent_graphs},
    {"shared_operand_and_chained_convolution", shared_operand_and_chained_convolution},
    {"invalid_shapes_and_overflow", invalid_shapes_and_overflow},
    {"empty_batch_and_seeded_initialization", empty_batch_and_seeded_initialization},
    {"known_stride_and_padding", known_stride_and_padding},
    {"stem_chain_on_device", stem_chain_on_device},
    {"grad_cam_on_device", grad_cam_on_device},
    {"grad_cam_resized_to_input", grad_cam_resized_to_input},
    {"publish_is_all_or_nothing", publish_is_all_or_nothing},
};

}  // namespace

// `test_frontend --seeded-weights C K R S SEED`: the weights of
// Conv2D::new_seeded(C, K, (R, S), 1, 0, SEED) as the hexadecimal bits of
// each f32, one per line (host-side only: no device call).
static int dump_seeded(char **argv) {
    const size_t c = std::strtoull(argv[0], nullptr, 10), k = std::strtoull(argv[1], nullptr, 10),
                 r = std::strtoull(argv[2], nullptr, 10), s = std::strtoull(argv[3], nullptr, 10);
    const uint64_t seed = std::strtoull(argv[4], nullptr, 10);
    auto layer = Conv2D::new_seeded(c, k, {r, s}, 1, 0, seed);
    if (!layer.ok()) {
        std::printf("ERROR %s\n", layer.error().to_string().c_str());
        return 1;
    }
    for (float v : layer.value().weights().data()) {
        uint32_t bits;
        std::memcpy(&bits, &v, sizeof bits);
        std::printf("%08x\n", bits);
    }
    return 0;
}

int main(int argc, char **argv) {
    if (argc == 7 && std::strcmp(argv[1], "--seeded-weights") == 0) return dump_seeded(argv + 2);
    int failures = 0;
    for (const Case &c : kCases) {
        if (argc > 1) {
            bool want = false;
            for (int i = 1; i < argc; ++i) want |= std::strcmp(argv[i], c.name) == 0;
            if (!want) continue;
        }
        try {
            c.fn();
            std::printf("PASS %s\n", c.name);
        } catch (const Failure &f) {
            std::printf("FAIL %s: %s\n", c.name, f.what.c_str());
            ++failures;
        }
        std::fflush(stdout);
    }
    return failures;
}
