// frontend_bench.cpp -- end-to-end steps through the C++ front end (the
// reference's public API, katsu.hpp) with device-resident tensors:
//
//   conv:   y = layer.forward(x); y.sum().backward()   (config 3: the upstream
//           gradient of sum() is all-ones, as the benchmark config states)
//   matmul: c = a.matmul(b);     c.sum().backward()    (config 2, n = 1024)
//   stem:   the config-5 chain: stem conv, mean pool, matmul head, sum,
//           backward, spread of dP over HW, backward of the stem
//
// Inputs are created from host values once; every step leaves x.grad and the
// weights' gradient on the device (zero_grad between steps), so no step
// crosses PCIe.  Prints one JSON line.
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/katsu_hip.h"
#include "katsu.hpp"

using namespace katsu;

namespace {

std::vector<float> uniform(uint64_t seed, size_t n) {
    std::vector<float> v(n);
    uint64_t s = seed;
    for (float &x : v) {
        s += 0x9e3779b97f4a7c15ull;
        uint64_t z = s;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z ^= z >> 31;
        x = 2.0f * ((float)(z >> 40) / 16777216.0f) - 1.0f;
    }
    return v;
}

template <class T>
T must(Result<T> r, const char *what) {
    if (!r.ok()) {
        std::fprintf(stderr, "frontend_bench: %s: %s\n", what, r.error().to_string().c_str());
        std::exit(1);
    }
    return std::move(r).value();
}

double now() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

}  // namespace

int main(int argc, char **argv) {
    int steps = 20;
    for (int i = 1; i + 1 < argc; ++i)
        if (!std::strcmp(argv[i], "--steps")) steps = std::atoi(argv[i + 1]);
    void *st = katsu_hip_stream();
    if (!st) {
        std::fprintf(stderr, "frontend_bench: no device\n");
        return 1;
    }

    // Config 3 through Conv2D.
    const size_t N = 32, C = 64, H = 56, W = 56, K = 64;
    Tensor x = must(Tensor::create(uniform(1, N * C * H * W), {N, C, H, W}), "x");
    Tensor w = must(Tensor::create(uniform(2, K * C * 9), {K, C, 3, 3}), "w");
    Conv2D layer = must(Conv2D::from_weights(w, 1, 1), "layer");
    auto conv_step = [&]() {
        Tensor y = must(layer.forward(x), "forward");
        Tensor loss = must(y.sum(), "sum");
        must(Result<Unit>(loss.backward()), "backward");
        must(Result<Unit>(x.zero_grad()), "zero_grad");
        must(Result<Unit>(w.zero_grad()), "zero_grad");
    };
    for (int i = 0; i < 3; ++i) conv_step();
    katsu_hip_sync(st);
    double t0 = now();
    for (int i = 0; i < steps; ++i) conv_step();
    katsu_hip_sync(st);
    const double conv_ms = (now() - t0) / steps * 1e3;
    const double conv_flop = 3.0 * 2.0 * N * K * H * W * C * 9;

    // Config 2 (n = 1024) through Tensor::matmul.
    const size_t n = 1024;
    Tensor a = must(Tensor::create(uniform(1, n * n), {n, n}), "a");
    Tensor b = must(Tensor::create(uniform(2, n * n), {n, n}), "b");
    auto mm_step = [&]() {
        Tensor c = must(a.matmul(b), "matmul");
        must(Result<Unit>(must(c.sum(), "sum").backward()), "backward");
        must(Result<Unit>(a.zero_grad()), "zero_grad");
        must(Result<Unit>(b.zero_grad()), "zero_grad");
    };
    for (int i = 0; i < 3; ++i) mm_step();
    katsu_hip_sync(st);
    t0 = now();
    for (int i = 0; i < steps; ++i) mm_step();
    katsu_hip_sync(st);
    const double mm_ms = (now() - t0) / steps * 1e3;
    const double mm_flop = 3.0 * 2.0 * n * n * n;

    // Config 5: the stem and its head.  y = conv(x) [64,64,112,112]; P = mean
    // over HW; L = sum(P . H) with H [64,1000]; backward into P; dY = dP/HW
    // spread over HW; y.backward_with(dY) gives dX and dW.
    Tensor xs = must(Tensor::create(uniform(1, 64 * 3 * 224 * 224), {64, 3, 224, 224}), "x5");
    Tensor ws = must(Tensor::create(uniform(2, 64 * 3 * 49), {64, 3, 7, 7}), "w5");
    Tensor hs = must(Tensor::create(uniform(4, 64 * 1000), {64, 1000}), "h5");
    Conv2D stem = must(Conv2D::from_weights(ws, 2, 3), "stem");
    auto stem_step = [&]() {
        Tensor y = must(stem.forward(xs), "stem forward");
        Tensor pooled = must(mean_pool_hw(y), "pool");
        must(Result<Unit>(must(must(pooled.matmul(hs), "head").sum(), "sum").backward()),
             "head backward");
        std::vector<float> dp = **must(pooled.grad(), "dP");
        Tensor dpt = must(Tensor::create(std::move(dp), {64, 64}), "dP tensor");
        Tensor dy = must(spread_hw(dpt, y.shape()), "spread");
        must(Result<Unit>(y.backward_with(dy)), "stem backward");
        must(Result<Unit>(xs.zero_grad()), "zero_grad");
        must(Result<Unit>(ws.zero_grad()), "zero_grad");
        must(Result<Unit>(hs.zero_grad()), "zero_grad");
    };
    for (int i = 0; i < 2; ++i) stem_step();
    katsu_hip_sync(st);
    const int stem_steps = steps > 10 ? steps / 2 : steps;
    t0 = now();
    for (int i = 0; i < stem_steps; ++i) stem_step();
    katsu_hip_sync(st);
    const double stem_ms = (now() - t0) / stem_steps * 1e3;
    const double stem_flop = 3.0 * 2.0 * 64 * 64 * 112 * 112 * 3 * 49 + 3.0 * 2.0 * 64 * 64 * 1000;

    std::printf(
        "{\"conv_c3\": {\"ms_per_step\": %.4f, \"tflops\": %.3f, \"steps\": %d, "
        "\"step\": \"forward + sum + backward through Conv2D, device-resident\"}, "
        "\"matmul_1024\": {\"ms_per_step\": %.4f, \"tflops\": %.3f, \"steps\": %d, "
        "\"step\": \"matmul + sum + backward through Tensor, device-resident\"}, "
        "\"stem_chain_c5\": {\"ms_per_step\": %.4f, \"tflops\": %.3f, \"steps\": %d, "
        "\"step\": \"stem forward, mean pool, matmul head, sum, backward, spread, "
        "stem backward; device-resident\"}}\n",
        conv_ms, conv_flop / (conv_ms * 1e-3) / 1e12, steps, mm_ms,
        mm_flop / (mm_ms * 1e-3) / 1e12, steps, stem_ms, stem_flop / (stem_ms * 1e-3) / 1e12,
        stem_steps);
    return 0;
}
