// katsu_hip.hip -- C ABI (include/katsu_hip.h) over the gfx950 MFMA engine.
//
// Replaces the reference's kernel seams (paths relative to the reference
// repository root):
//   katsu_hip_gemm_f32*                 tensor.rs:264-273 (fwd), 424-444 (VJPs)
//   katsu_hip_conv2d_fwd_f32*           conv2d.rs:98-103
//   katsu_hip_conv2d_bwd_data_f32*      conv2d.rs:288 (dx half of backward_buffers)
//   katsu_hip_conv2d_bwd_filter_f32*    conv2d.rs:289 (dw half of backward_buffers)
//   katsu_hip_conv2d_geometry           conv2d.rs:183-224 (Geometry::new checks)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "../../include/katsu_hip.h"
#include "igemm.hpp"
#include "direct.hpp"
#include "elementwise.hpp"
#include "gemm.hpp"
#include "hostcopy.hpp"
#include "pointwise.hpp"
#include "smallc.hpp"
#include "stemdx.hpp"
#include "tiny.hpp"

namespace katsu {
namespace {

constexpr int64_t kI32Max = 0x7fffffff;

// ---------------------------------------------------------------------------
// Small helper kernels.

// out = beta * out, used when a reduction is empty (k == 0 or batch == 0).
__global__ void __launch_bounds__(256) scale_kernel(float *p, int64_t n, float beta) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step)
        p[i] = (beta == 0.f) ? 0.f : beta * p[i];
}

// ---------------------------------------------------------------------------
// Library state.

struct Buffer {
    void *ptr = nullptr;
    size_t bytes = 0;
};

// Device buffers handed out by katsu_hip_malloc: freed blocks are kept for
// reuse (hipFree synchronises the device) and returned to HIP at shutdown.
struct Pool {
    std::multimap<size_t, void *> free;       // block size -> block
    std::unordered_map<void *, size_t> live;  // block -> size
};

struct State {
    std::mutex mu;
    bool ready = false;
    int device = -1;
    hipStream_t stream = nullptr;
    Buffer staging[5];
    HostCopy copy;  // the host-pointer entry points' pinned staging ring
    Pool pool;
};

State &state() {
    static State s;
    return s;
}

// Device allocations this library has made (every successful hipMalloc of
// the scratch buffers, the staging buffers and the caller pool), for callers
// that check that a code path allocates nothing.
std::atomic<uint64_t> g_device_allocs{0};

int map_hip(hipError_t e) {
    if (e == hipSuccess) return KATSU_OK;
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) return KATSU_E_OOM;
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) return KATSU_E_NODEVICE;
    return KATSU_E_LAUNCH;
}

// Library-owned scratch of the device entry points: the dW split partials
// (when the caller passes no workspace), the GEMM's split-K partials, the
// sum's chunk partials and Grad-CAM's channel weights, one buffer per
// purpose.  The buffers are shared by every stream, so a call may run under
// HIP graph capture on another stream than the eager call that sized them
// (no allocation is then needed); calls that overlap in time on two streams
// race on them.  A buffer that must grow is replaced, and the old block is
// kept until katsu_hip_shutdown, because a graph captured earlier still
// addresses it.  Its own mutex: the host-pointer entry points hold State::mu
// while their device calls take scratch.
enum class ScratchKind : int { Dw = 0, Gemm = 1, Sum = 2, Cam = 3, Count = 4 };

struct ScratchPool {
    std::mutex mu;
    Buffer live[(int)ScratchKind::Count];
    std::vector<void *> retired;
};

ScratchPool &scratch_pool() {
    static ScratchPool p;
    return p;
}

int scratch_get(ScratchKind kind, hipStream_t, size_t bytes, float **out) {
    ScratchPool &p = scratch_pool();
    std::lock_guard<std::mutex> lock(p.mu);
    Buffer &b = p.live[(int)kind];
    if (b.bytes < bytes) {
        void *ptr = nullptr;
        const size_t want = std::max<size_t>(bytes, 256);
        const hipError_t e = hipMalloc(&ptr, want);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return map_hip(e);
        }
        g_device_allocs.fetch_add(1, std::memory_order_relaxed);
        if (b.ptr) p.retired.push_back(b.ptr);
        b.ptr = ptr;
        b.bytes = want;
    }
    *out = (float *)b.ptr;
    return KATSU_OK;
}

void scratch_release_all() {
    ScratchPool &p = scratch_pool();
    std::lock_guard<std::mutex> lock(p.mu);
    for (Buffer &b : p.live) {
        if (b.ptr) (void)hipFree(b.ptr);
        b = Buffer{};
    }
    for (void *q : p.retired) (void)hipFree(q);
    p.retired.clear();
}

// Where a dW (or GEMM) launch takes its partial slices: the caller's
// workspace when it passes one (checked against the plan), else the
// library's scratch for the stream when `lib` allows it.
struct WsSource {
    void *ws = nullptr;
    size_t bytes = 0;
    bool lib = false;  // NULL workspace: use library scratch (else an error)
};

int ws_take(const WsSource &src, size_t need, hipStream_t st, float **out) {
    *out = nullptr;
    if (need == 0) return KATSU_OK;
    if (src.ws) {
        if (src.bytes < need) return KATSU_E_INVALID;
        *out = (float *)src.ws;
        return KATSU_OK;
    }
    if (!src.lib) return KATSU_E_INVALID;
    return scratch_get(ScratchKind::Dw, st, need, out);
}

int init_locked(State &s) {
    if (s.ready) return KATSU_OK;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return KATSU_E_NODEVICE;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return KATSU_E_NODEVICE;
    if (hipSetDevice(dev) != hipSuccess) return KATSU_E_NODEVICE;
    // Default priority, non-blocking with respect to the null stream.
    if (hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking) != hipSuccess)
        return KATSU_E_NODEVICE;
    s.device = dev;
    s.ready = true;
    return KATSU_OK;
}

int ensure(Buffer &b, size_t bytes) {
    if (b.bytes >= bytes) return KATSU_OK;
    if (b.ptr) {
        (void)hipFree(b.ptr);
        b.ptr = nullptr;
        b.bytes = 0;
    }
    size_t want = std::max<size_t>(bytes, 256);
    hipError_t e = hipMalloc(&b.ptr, want);
    if (e != hipSuccess) {
        b.ptr = nullptr;
        return map_hip(e);
    }
    g_device_allocs.fetch_add(1, std::memory_order_relaxed);
    b.bytes = want;
    return KATSU_OK;
}

int launch_status() { return map_hip(hipGetLastError()); }

int launch_scale(float *p, int64_t n, float beta, hipStream_t st) {
    if (n <= 0 || beta == 1.f) return KATSU_OK;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
    scale_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(p, n, beta);
    return launch_status();
}

bool beta_ok(float beta) { return beta == 0.f || beta == 1.f; }
bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// ---------------------------------------------------------------------------
// Tile configurations.  BM spans the output's "row" dimension (oc, c, or m),
// BN the contiguous one (pixels, or n).
template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct Cfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
};
using CfgS = Cfg<16, 256, 16, 16, 64>;   // rows <= 16 (tiny channel counts)
using CfgM = Cfg<64, 128, 16, 32, 64>;   // rows <= 64
using CfgL = Cfg<128, 128, 16, 64, 64>;  // large
using CfgW = Cfg<64, 64, 32, 32, 32>;    // dW: oc x (c,r,s), long split reductions
using Cfg64 = Cfg<64, 64, 16, 32, 32>;   // mid-size GEMMs (enough tiles for 256 CUs)
using Cfg32 = Cfg<32, 32, 32, 16, 16>;   // small GEMMs

template <class C, class Prob>
int run(const Prob &p, int64_t blocks, hipStream_t st) {
    if (blocks <= 0) return KATSU_OK;
    if (blocks > kI32Max) return KATSU_E_INVALID;
    igemm_kernel<C::BM, C::BN, C::BK, C::WM, C::WN, Prob>
        <<<dim3((unsigned)blocks), dim3(kThreads), 0, st>>>(p);
    return launch_status();
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// GEMM.

template <class C, bool A_KM, bool B_KM>
int gemm_cfg(const float *a, int64_t a_si, int64_t a_sk, const float *b, int64_t b_si,
             int64_t b_sk, float *c, int64_t m, int64_t n, int64_t k, float beta,
             hipStream_t st) {
    GemmProb<A_KM, B_KM> p;
    p.a = {a, a_si, a_sk, (int)m};
    p.b = {b, b_si, b_sk, (int)n};
    p.c = {c, n, (int)m, (int)n, beta};
    p.K = (int)k;
    p.tiles_m = (int)cdiv(m, C::BM);
    p.tiles_n = (int)cdiv(n, C::BN);
    p.group = 8;
    return run<C>(p, (int64_t)p.tiles_m * p.tiles_n, st);
}

template <class C>
int gemm_dispatch(const float *a, const float *b, float *c, int64_t m, int64_t n, int64_t k,
                  int ta, int tb, float beta, hipStream_t st) {
    // op(A)[i][kk]: A stored [m][k] -> (si=k, sk=1), contiguous along k (IMAJOR);
    //               A stored [k][m] -> (si=1, sk=m), contiguous along i (KMAJOR).
    // op(B)[kk][j]: B stored [k][n] -> (si=1, sk=n), KMAJOR;
    //               B stored [n][k] -> (si=k, sk=1), IMAJOR.
    if (!ta && !tb) return gemm_cfg<C, false, true>(a, k, 1, b, 1, n, c, m, n, k, beta, st);
    if (!ta && tb) return gemm_cfg<C, false, false>(a, k, 1, b, k, 1, c, m, n, k, beta, st);
    if (ta && !tb) return gemm_cfg<C, true, true>(a, 1, m, b, 1, n, c, m, n, k, beta, st);
    return gemm_cfg<C, true, false>(a, 1, m, b, k, 1, c, m, n, k, beta, st);
}

int launch_split_reduce(const float *ws, float *dw, int64_t elems, int64_t pstride, int splits,
                        float beta, hipStream_t st);
State &state();

// Raises a kernel's dynamic LDS limit above 64 KiB (defined below).
template <auto Kernel>
int lds_optin(size_t bytes);

template <int BM, int BN, int BK, bool TA, bool TB, int WG>
int gemm_fast_launch(const GemmArgs &g, int64_t blocks, hipStream_t st) {
    using Geo = GemmGeo<BM, BN, BK, TA, TB>;
    constexpr auto kern = gemm_kernel<BM, BN, BK, TA, TB, WG>;
    const int rc = lds_optin<kern>(WG * Geo::kBytes);
    if (rc != KATSU_OK) return rc;
    kern<<<dim3((unsigned)blocks), dim3(256 * WG), WG * Geo::kBytes, st>>>(g);
    return launch_status();
}

template <int BM, int BN, int BK, int WG>
int gemm_fast_t(const GemmArgs &g, int64_t blocks, int ta, int tb, hipStream_t st) {
    if (!ta && !tb) return gemm_fast_launch<BM, BN, BK, false, false, WG>(g, blocks, st);
    if (!ta && tb) return gemm_fast_launch<BM, BN, BK, false, true, WG>(g, blocks, st);
    if (ta && !tb) return gemm_fast_launch<BM, BN, BK, true, false, WG>(g, blocks, st);
    return gemm_fast_launch<BM, BN, BK, true, true, WG>(g, blocks, st);
}

template <int BM, int BN, int BK>
int gemm_fast_wg(const GemmArgs &g, int64_t blocks, int wg, int ta, int tb, hipStream_t st) {
    return wg == 2 ? gemm_fast_t<BM, BN, BK, 2>(g, blocks, ta, tb, st)
                   : gemm_fast_t<BM, BN, BK, 1>(g, blocks, ta, tb, st);
}

// Tile choice: the largest square tile (128, 64, 32) that gives every CU a
// block without splitting K; otherwise 64-tiles with split-K up to about
// one block per CU, at least 128 of K per split so the k-loop hides its load
// latency.  A split adds a reduce kernel, so it is the last resort.
#ifndef KATSU_GEMM_TARGET
#define KATSU_GEMM_TARGET 256
#define KATSU_GEMM_KMIN64 128
#endif
#ifndef KATSU_GEMM_BK64
#define KATSU_GEMM_BK64 64
#endif
#ifndef KATSU_GEMM_WG2_BELOW
#define KATSU_GEMM_WG2_BELOW 512
#endif

// The dedicated GEMM (gemm.hpp) for aligned problems: the tile, the split of
#ifndef KATSU_GEMM_BK32
#define KATSU_GEMM_BK32 64  // k-tile depth of the 32 x 32 GEMM tiles
#endif
// K and the launch arguments (C not bound yet).  False = not applicable.
struct GemmFastPlan {
    GemmArgs g{};
    int T = 0;
    int64_t blocks = 0, splits = 1, pstride = 0;
};

bool gemm_fast_plan(const float *a, const float *b, const float *c, int64_t M, int64_t N,
                    int64_t K, int ta, int tb, float beta, GemmFastPlan *pl) {
    if (M % 4 || N % 4 || K % 4 || !aligned16(a) || !aligned16(b) || !aligned16(c)) return false;
    if (M * K * 4 >= (int64_t)kMaxBufBytes || K * N * 4 >= (int64_t)kMaxBufBytes ||
        M * N >= kI32Max)
        return false;
    auto tiles_of = [&](int64_t t) { return cdiv(M, t) * cdiv(N, t); };
    int T = 0;
    int64_t tiles = 0, splits = 1;
    for (int t : {128, 64, 32}) {
        if (tiles_of(t) >= 256) {
            T = t;
            tiles = tiles_of(t);
            break;
        }
    }
    if (T == 0) {
        T = 64;
        tiles = tiles_of(64);
        splits = std::max<int64_t>(
            1, std::min<int64_t>(cdiv(KATSU_GEMM_TARGET, tiles), K / KATSU_GEMM_KMIN64));
    }
    const int64_t kq = T == 128 ? 16 : T == 64 ? KATSU_GEMM_BK64 : KATSU_GEMM_BK32;  // k depth
    const int64_t kchunk = (cdiv(K, splits) + kq - 1) / kq * kq;
    splits = cdiv(K, kchunk);
    GemmArgs &g = pl->g;
    g.a = a;
    g.b = b;
    g.M = (int)M;
    g.N = (int)N;
    g.K = (int)K;
    g.lda = (int)(ta ? M : K);
    g.ldb = (int)(tb ? K : N);
    g.ldc = (int)N;
    g.beta = beta;
    g.tiles_m = (int)cdiv(M, T);
    g.tiles_n = (int)cdiv(N, T);
    g.splits = (int)splits;
    g.kchunk = (int)kchunk;
    g.a_bytes = (uint32_t)(M * K * 4);
    g.b_bytes = (uint32_t)(K * N * 4);
    pl->T = T;
    pl->splits = splits;
    pl->pstride = M * N;
    pl->blocks = tiles * splits;
    return true;
}

// The register-direct GEMM (gemm.hpp, gemm_rd_*): 64 x 64 tiles whose four
// waves each take a quarter of K, for problems of about one tile per CU
// with K = 4 * 16 * kRdNkb (1024^3).
#ifndef KATSU_GEMM_RD
#define KATSU_GEMM_RD 1
#endif
#ifndef KATSU_GEMM_RD_D
#define KATSU_GEMM_RD_D 3
#endif
#ifndef KATSU_GEMM_RD_VJP_D
#define KATSU_GEMM_RD_VJP_D 2
#endif
#ifndef KATSU_GEMM_RD_KS
#define KATSU_GEMM_RD_KS 4
#endif
#ifndef KATSU_GEMM_RD_VJP_KS
#define KATSU_GEMM_RD_VJP_KS 4
#endif
#ifndef KATSU_GEMM_RD_VJP_PAIR
#define KATSU_GEMM_RD_VJP_PAIR 1  // square VJPs: a block takes a dA tile, then a dB tile
#endif
#ifndef KATSU_GEMM_RD_VJP_OCC
#define KATSU_GEMM_RD_VJP_OCC 1  // blocks per CU the VJP kernel is built for
#endif
// K = 1024: KS waves of 1024 / KS each, in blocks of 16.
constexpr int kRdK = 1024;
constexpr int kRdKs = KATSU_GEMM_RD_KS, kRdNkb = kRdK / 16 / kRdKs;
constexpr int kRdVjpKs = KATSU_GEMM_RD_VJP_KS, kRdVjpNkb = kRdK / 16 / kRdVjpKs;

bool gemm_rd_plan(const float *a, const float *b, const float *c, int64_t M, int64_t N,
                  int64_t K, int ta, int tb, float beta, GemmArgs *g) {
    if (!KATSU_GEMM_RD || M % 64 || N % 64 || K != kRdK || !aligned16(a) ||
        !aligned16(b) || !aligned16(c))
        return false;
    if (M * K * 4 >= (int64_t)kMaxBufBytes || K * N * 4 >= (int64_t)kMaxBufBytes ||
        M * N >= kI32Max)
        return false;
    const int64_t tiles = (M / 64) * (N / 64);
    if (tiles < 128 || tiles > 512) return false;
    *g = GemmArgs{};
    g->a = a;
    g->b = b;
    g->M = (int)M;
    g->N = (int)N;
    g->K = (int)K;
    g->lda = (int)(ta ? M : K);
    g->ldb = (int)(tb ? K : N);
    g->ldc = (int)N;
    g->beta = beta;
    g->tiles_m = (int)(M / 64);
    g->tiles_n = (int)(N / 64);
    // Groups of four tile rows per patch (1024^2: each XCD's 32 tiles read
    // 4 row and 8 column panels, 3 MB), else plain column order.
    g->gm = g->tiles_m % 4 == 0 ? 4 : g->tiles_m;
    g->splits = 1;
    g->kchunk = 0;  // set by the kernel's KS
    g->a_bytes = (uint32_t)(M * K * 4);
    g->b_bytes = (uint32_t)(K * N * 4);
    return true;
}

template <bool TA, bool TB>
int gemm_rd_launch(const GemmArgs &g, hipStream_t st) {
    constexpr auto kern = gemm_rd_kernel<TA, TB, kRdKs, kRdNkb, KATSU_GEMM_RD_D, 1>;
    constexpr size_t lds = kRdKs * 64 * 64 * 4;
    const int rc = lds_optin<kern>(lds);
    if (rc != KATSU_OK) return rc;
    kern<<<dim3((unsigned)(g.tiles_m * g.tiles_n)), dim3(64 * kRdKs), lds, st>>>(g);
    return launch_status();
}

// The planned GEMM into c, with a fixed-order reduce of the partial slices
// when K is split.
bool gemm_fast(const float *a, const float *b, float *c, int64_t M, int64_t N, int64_t K, int ta,
               int tb, float beta, hipStream_t st, int *rc) {
    {
        GemmArgs g;
        if (gemm_rd_plan(a, b, c, M, N, K, ta, tb, beta, &g)) {
            g.c = c;
            *rc = !ta ? (!tb ? gemm_rd_launch<false, false>(g, st) : gemm_rd_launch<false, true>(g, st))
                      : (!tb ? gemm_rd_launch<true, false>(g, st) : gemm_rd_launch<true, true>(g, st));
            return true;
        }
    }
    GemmFastPlan pl;
    if (!gemm_fast_plan(a, b, c, M, N, K, ta, tb, beta, &pl)) return false;
    GemmArgs g = pl.g;
    float *ws = nullptr;
    if (pl.splits > 1 &&
        (*rc = scratch_get(ScratchKind::Gemm, st, (size_t)(pl.splits * pl.pstride) * sizeof(float),
                           &ws)) != KATSU_OK)
        return true;
    g.c = pl.splits > 1 ? ws : c;
    g.split_stride = pl.splits > 1 ? pl.pstride : 0;
    // Fewer blocks than two per CU: two wave groups per block, so every SIMD
    // still holds two waves.
    const int wg = pl.blocks < KATSU_GEMM_WG2_BELOW ? 2 : 1;
    *rc = pl.T == 128  ? gemm_fast_wg<128, 128, 16>(g, pl.blocks, wg, ta, tb, st)
          : pl.T == 64 ? gemm_fast_wg<64, 64, KATSU_GEMM_BK64>(g, pl.blocks, wg, ta, tb, st)
                       : gemm_fast_wg<32, 32, KATSU_GEMM_BK32>(g, pl.blocks, wg, ta, tb, st);
    if (*rc == KATSU_OK && pl.splits > 1)
        *rc = launch_split_reduce(ws, c, M * N, pl.pstride, (int)pl.splits, beta, st);
    return true;
}

// dA and dB of the matmul VJP in one launch (gemm_vjp_kernel).
template <int BM, int BN, int BK, int WG>
int gemm_vjp_launch(const GemmArgs &nt, const GemmArgs &tn, int64_t nb0, int64_t nb1,
                    hipStream_t st) {
    using GeoNT = GemmGeo<BM, BN, BK, false, true>;
    using GeoTN = GemmGeo<BM, BN, BK, true, false>;
    constexpr size_t lds = WG * std::max(GeoNT::kBytes, GeoTN::kBytes);
    constexpr auto kern = gemm_vjp_kernel<BM, BN, BK, WG>;
    const int rc = lds_optin<kern>(lds);
    if (rc != KATSU_OK) return rc;
    kern<<<dim3((unsigned)(nb0 + nb1)), dim3(256 * WG), lds, st>>>(nt, tn, (int)nb0);
    return launch_status();
}

int gemm_dev(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int ta,
             int tb, float beta, hipStream_t st) {
    if (!beta_ok(beta) || (ta != 0 && ta != 1) || (tb != 0 && tb != 1)) return KATSU_E_INVALID;
    // Empty problems first, whatever their other dimensions (the reference
    // accepts [usize::MAX, 0] . [0, 0], tests/tensor.rs:65-86).
    if (m == 0 || n == 0) return KATSU_OK;
    if (!c) return KATSU_E_INVALID;
    if (k == 0) {
        uint64_t mn;
        if (__builtin_mul_overflow((uint64_t)m, (uint64_t)n, &mn) || mn > (uint64_t)INT64_MAX)
            return KATSU_E_INVALID;
        return launch_scale(c, (int64_t)mn, beta, st);
    }
    if ((int64_t)m > kI32Max || (int64_t)n > kI32Max || (int64_t)k > kI32Max)
        return KATSU_E_INVALID;
    if (!a || !b) return KATSU_E_INVALID;
    {
        int rc = KATSU_OK;
        if (gemm_fast(a, b, c, (int64_t)m, (int64_t)n, (int64_t)k, ta, tb, beta, st, &rc))
            return rc;
    }
    // The generic engine: the largest tile that still gives every CU a
    // block; tiny row counts take the 16-row tile.
    const int64_t M = (int64_t)m, N = (int64_t)n;
    auto tiles = [&](int64_t bm, int64_t bn) { return cdiv(M, bm) * cdiv(N, bn); };
    if (m >= 128 && n >= 128 && tiles(128, 128) >= 256)
        return gemm_dispatch<CfgL>(a, b, c, m, n, k, ta, tb, beta, st);
    if (m <= 16) return gemm_dispatch<CfgS>(a, b, c, m, n, k, ta, tb, beta, st);
    if (m <= 64 && tiles(64, 128) >= 256)
        return gemm_dispatch<CfgM>(a, b, c, m, n, k, ta, tb, beta, st);
    if (tiles(64, 64) >= 256) return gemm_dispatch<Cfg64>(a, b, c, m, n, k, ta, tb, beta, st);
    return gemm_dispatch<Cfg32>(a, b, c, m, n, k, ta, tb, beta, st);
}

// Matmul VJP (tensor.rs:418-445): da = beta_a*da + g b^T, then
// db = beta_b*db + a^T g; a null da or db skips that product.  When both are
// wanted, their buffers do not overlap, and both plan the same unsplit tile,
// the two products run as one launch; otherwise as two launches in that
// order.
int matmul_vjp_dev(const float *a, const float *b, const float *g, float *da, float *db,
                   size_t m, size_t k, size_t n, float beta_a, float beta_b, hipStream_t st) {
    if (!beta_ok(beta_a) || !beta_ok(beta_b)) return KATSU_E_INVALID;
    // An empty problem (C empty or k == 0, where the reference returns before
    // either product, tensor.rs:421-423) goes to the two calls below, which
    // write beta*da and beta*db and check nothing else.
    const bool empty = m == 0 || n == 0 || k == 0;
    if (!empty && ((int64_t)m > kI32Max || (int64_t)n > kI32Max || (int64_t)k > kI32Max))
        return KATSU_E_INVALID;
    const int64_t M = (int64_t)m, N = (int64_t)n, K = (int64_t)k;
    const bool apart = da && db && (da + M * K <= db || db + K * N <= da);
    if (apart && !empty && a && b && g) {
        GemmArgs ra, rb;
        if (gemm_rd_plan(g, b, da, M, K, N, 0, 1, beta_a, &ra) &&
            gemm_rd_plan(a, g, db, K, N, M, 1, 0, beta_b, &rb) &&
            (ra.tiles_m * ra.tiles_n) % 8 == 0) {
            ra.c = da;
            rb.c = db;
            const int nb0 = ra.tiles_m * ra.tiles_n, nb1 = rb.tiles_m * rb.tiles_n;
            if (KATSU_GEMM_RD_VJP_PAIR && nb0 == nb1) {
                // One block per tile index: its dA tile, then its dB tile.
                constexpr auto pk =
                    gemm_rd_vjp_pair_kernel<kRdVjpKs, kRdVjpNkb, KATSU_GEMM_RD_VJP_D>;
                constexpr size_t lds = kRdVjpKs * 64 * 64 * 4;
                const int rc = lds_optin<pk>(lds);
                if (rc != KATSU_OK) return rc;
                pk<<<dim3((unsigned)nb0), dim3(64 * kRdVjpKs), lds, st>>>(ra, rb);
                return launch_status();
            }
            constexpr auto kern =
                gemm_rd_vjp_kernel<kRdVjpKs, kRdVjpNkb, KATSU_GEMM_RD_VJP_D, KATSU_GEMM_RD_VJP_OCC>;
            constexpr size_t lds = kRdVjpKs * 64 * 64 * 4;
            const int rc = lds_optin<kern>(lds);
            if (rc != KATSU_OK) return rc;
            kern<<<dim3((unsigned)(nb0 + nb1)), dim3(64 * kRdVjpKs), lds, st>>>(ra, rb, nb0);
            return launch_status();
        }
        GemmFastPlan pa, pb;
        if (gemm_fast_plan(g, b, da, M, K, N, 0, 1, beta_a, &pa) &&
            gemm_fast_plan(a, g, db, K, N, M, 1, 0, beta_b, &pb) && pa.T == pb.T &&
            pa.splits == 1 && pb.splits == 1 && pa.blocks % 8 == 0 &&
            pa.blocks + pb.blocks <= kI32Max) {
            pa.g.c = da;
            pb.g.c = db;
            pa.g.split_stride = pb.g.split_stride = 0;
            // Wave groups by the combined grid (two blocks per CU from the
            // pair where each alone would take two groups): the k-sum order
            // can then differ from the separate launches', within the f32
            // bound and the same on every call.
            const bool two = pa.blocks + pb.blocks < KATSU_GEMM_WG2_BELOW;
            const int64_t b0 = pa.blocks, b1 = pb.blocks;
            if (pa.T == 128)
                return two ? gemm_vjp_launch<128, 128, 16, 2>(pa.g, pb.g, b0, b1, st)
                           : gemm_vjp_launch<128, 128, 16, 1>(pa.g, pb.g, b0, b1, st);
            if (pa.T == 64)
                return two ? gemm_vjp_launch<64, 64, KATSU_GEMM_BK64, 2>(pa.g, pb.g, b0, b1, st)
                           : gemm_vjp_launch<64, 64, KATSU_GEMM_BK64, 1>(pa.g, pb.g, b0, b1, st);
            return two ? gemm_vjp_launch<32, 32, KATSU_GEMM_BK32, 2>(pa.g, pb.g, b0, b1, st)
                       : gemm_vjp_launch<32, 32, KATSU_GEMM_BK32, 1>(pa.g, pb.g, b0, b1, st);
        }
    }
    int rc = KATSU_OK;
    if (da) rc = gemm_dev(g, b, da, m, k, n, 0, 1, beta_a, st);
    if (rc == KATSU_OK && db) rc = gemm_dev(a, g, db, k, n, m, 1, 0, beta_b, st);
    return rc;
}

// ---------------------------------------------------------------------------
// Convolution geometry (the checks of Geometry::new, conv2d.rs:183-224, plus
// the 32-bit index limits of the kernels).

bool mul_ok(uint64_t a, uint64_t b, uint64_t *out) { return !__builtin_mul_overflow(a, b, out); }

int geometry_fill(katsu_conv_geom *g) {
    if (!g) return KATSU_E_INVALID;
    if (g->c == 0 || g->k == 0 || g->r == 0 || g->s == 0 || g->stride == 0)
        return KATSU_E_INVALID;  // validate_weights, conv2d.rs:156-166
    if (g->h == 0 || g->w == 0) return KATSU_E_INVALID;  // conv2d.rs:190
    uint64_t pad2;
    if (!mul_ok(g->pad, 2, &pad2)) return KATSU_E_INVALID;
    uint64_t ph, pw;
    if (__builtin_add_overflow(g->h, pad2, &ph) || __builtin_add_overflow(g->w, pad2, &pw))
        return KATSU_E_INVALID;
    if (ph < g->r || pw < g->s) return KATSU_E_INVALID;  // kernel exceeds padded input
    const uint64_t oh = (ph - g->r) / g->stride + 1, ow = (pw - g->s) / g->stride + 1;
    // element_count (tensor.rs:129-140) of C*H*W, K*OH*OW and N*K*OH*OW
    // (conv2d.rs:196, 214-215): a product of non-zero dimensions must not
    // overflow and must stay within isize::MAX / 4 floats.
    auto count_ok = [](std::initializer_list<uint64_t> dims) {
        uint64_t c = 1;
        for (uint64_t v : dims) {
            if (v == 0) return true;
            if (!mul_ok(c, v, &c)) return false;
        }
        return c <= (uint64_t)INT64_MAX / sizeof(float);
    };
    if (!count_ok({g->c, g->h, g->w}) || !count_ok({g->k, oh, ow}) ||
        !count_ok({g->n, g->k, oh, ow}))
        return KATSU_E_INVALID;
    g->oh = oh;
    g->ow = ow;
    return KATSU_OK;
}

// Checked problem sizes used by the launchers.
struct ConvDims {
    int N, C, H, W, K, R, S, st, pad, OH, OW;
    int HW, CHW, OHW, KOHW, RS, CRS;
    int64_t npix_out, npix_in;  // N*OH*OW, N*H*W
};

int conv_dims(const katsu_conv_geom *g, ConvDims *d) {
    if (!g) return KATSU_E_INVALID;
    katsu_conv_geom t = *g;
    if (geometry_fill(&t) != KATSU_OK) return KATSU_E_INVALID;
    if (t.oh != g->oh || t.ow != g->ow) return KATSU_E_INVALID;
    // Per-image and per-filter element counts must fit the kernels' 32-bit
    // index math; so must the pixel counts that index GEMM columns.
    uint64_t hw, chw, ohw, kohw, rs, crs, kcrs, npo, npi;
    if (!mul_ok(t.h, t.w, &hw) || !mul_ok(hw, t.c, &chw) || !mul_ok(t.oh, t.ow, &ohw) ||
        !mul_ok(ohw, t.k, &kohw) || !mul_ok(t.r, t.s, &rs) || !mul_ok(rs, t.c, &crs) ||
        !mul_ok(crs, t.k, &kcrs) || !mul_ok(ohw, t.n, &npo) || !mul_ok(hw, t.n, &npi))
        return KATSU_E_INVALID;
    const uint64_t lim = (uint64_t)kI32Max;
    if (chw > lim || kohw > lim || kcrs > lim || npo > lim || npi > lim || t.pad > lim ||
        t.stride > lim || t.h + 2 * t.pad > lim || t.w + 2 * t.pad > lim)
        return KATSU_E_INVALID;
    d->N = (int)t.n;
    d->C = (int)t.c;
    d->H = (int)t.h;
    d->W = (int)t.w;
    d->K = (int)t.k;
    d->R = (int)t.r;
    d->S = (int)t.s;
    d->st = (int)t.stride;
    d->pad = (int)t.pad;
    d->OH = (int)t.oh;
    d->OW = (int)t.ow;
    d->HW = (int)hw;
    d->CHW = (int)chw;
    d->OHW = (int)ohw;
    d->KOHW = (int)kohw;
    d->RS = (int)rs;
    d->CRS = (int)crs;
    d->npix_out = (int64_t)npo;
    d->npix_in = (int64_t)npi;
    return KATSU_OK;
}

FastDiv fdiv(int64_t d) { return make_fastdiv((uint32_t)std::max<int64_t>(1, d)); }

// ---------------------------------------------------------------------------
// Direct (halo-tile) kernels: planning and launch.  A planner returns false
// when its kernel variant does not fit the problem (kernel size, halo
// columns or rows, LDS, too few blocks to fill the chip); the caller then
// tries the next variant and finally the implicit-GEMM engine, which takes
// every shape.

constexpr size_t kLdsMax = 163840;         // bytes of LDS a gfx950 workgroup may use
constexpr int64_t kMinDirectBlocks = 256;  // one per CU at least

// Rows of output touched by any tile of `tile_px` consecutive pixels.
int64_t tile_row_span(int64_t tile_px, int64_t OW, int64_t OH) {
    int64_t span;
    if (tile_px % OW == 0) span = tile_px / OW;
    else if (OW % tile_px == 0) span = 1;
    else span = (tile_px + OW - 2) / OW + 1;
    return std::min(span, OH);
}

// Dynamic LDS above 64 KiB must be opted into, once per kernel function
// (a function-local static: thread-safe one-time initialisation).
template <auto Kernel>
int lds_optin(size_t bytes) {
    if (bytes <= 65536) return KATSU_OK;
    static const hipError_t e = hipFuncSetAttribute(
        (const void *)Kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    return e == hipSuccess ? KATSU_OK : KATSU_E_LAUNCH;
}

// A "forward-shaped" problem: out[n][co] = sum_ci,taps in[n][ci] * w'.
// For the super-pixel data gradient (WMODE 2) the extra fields describe the
// layer (C, R, S, padding), the super-filter's first offsets and the
// full-resolution output; they are unused otherwise.
struct DirectFwdProblem {
    const float *in, *w;
    float *out;
    int64_t N, CI, H, W, CO, R, S, st, pady, padx, OH, OW;
    float beta;
    int64_t g_c = 0, g_r = 0, g_s = 0, g_pad = 0, g_amin = 0, g_bmin = 0, fh = 0, fw = 0;
};


// A planned direct forward-shaped launch: arguments, grid, weight path.
struct DirectFwdPlan {
    bool ok = false;
    DirectArgs a;
    int64_t blocks = 0;
    bool wvec = false;
};

template <int KT, int F, int CB, int R, int S, int ROWS, int PITCH, int WMODE, bool S2 = false,
          bool RF = false, int PD = 0, int KG = 1>
bool direct_fwd_plan(const DirectFwdProblem &P, DirectFwdPlan *pl) {
    using Geo = DirectFwdGeo<KT, F, CB, R, S, ROWS, PITCH, WMODE, KG>;
    if (P.R != R || P.S != S) return false;
    // Halo filter: the layer's, or for the phase form its G offsets.
    constexpr int HR = WMODE == 3 ? Dxs2Taps<R, S, PD>::DR : R;
    constexpr int HS = WMODE == 3 ? Dxs2Taps<R, S, PD>::DS : S;
    if (RF && P.OW > 16) return false;  // one output row per 16-lane fragment
    // Split halo rows: every tap's column must stay inside its half row.
    if (S2 && (P.st != 2 || (P.OW - 1) + (S - 1) / 2 >= PITCH / 2)) return false;
    static_assert(Geo::kBytes <= kLdsMax, "LDS");
    constexpr int WPX = 4 / (KT / 16);
    const int64_t OHW = P.OH * P.OW;
    const int64_t ncols = (P.OW - 1) * P.st + HS;
    if (ncols > Geo::HCOLS) return false;
    // Buffer resources address one image of `in` and all of `w` in bytes.
    const int64_t in_img = P.CI * P.H * P.W;
    const int64_t w_elems = WMODE == 2 ? P.CI * P.g_c * P.g_r * P.g_s : P.CO * P.CI * R * S;
    if (in_img * 4 >= (int64_t)kMaxBufBytes || w_elems * 4 >= (int64_t)kMaxBufBytes) return false;
    const int64_t co_blocks = cdiv(P.CO, KT);
    const int64_t tpmax = (int64_t)WPX * F * 16;
    // The fewest tiles that fit, but enough blocks to fill the chip; tile
    // lengths rounded to whole 16-byte output runs when that still fits.
    // Row fragments: tiles of whole rows, one row per fragment.
    const int64_t frag_rows = (int64_t)WPX * F;
    int64_t tiles_img = RF ? std::max(cdiv(P.OH, frag_rows), cdiv(kMinDirectBlocks, co_blocks * P.N))
                           : std::max(cdiv(OHW, tpmax), cdiv(kMinDirectBlocks, co_blocks * P.N));
    for (int attempt = 0; attempt < 64; ++attempt, ++tiles_img) {
        auto rows_of = [&](int64_t px) { return (tile_row_span(px, P.OW, P.OH) - 1) * P.st + HR; };
        int64_t tile_px;
        if (RF) {
            const int64_t rows = cdiv(P.OH, tiles_img);
            if (rows > frag_rows) continue;
            if (2 * rows < frag_rows) return false;  // fragments would be under half used
            tile_px = rows * P.OW;
        } else {
            const int64_t even = cdiv(OHW, tiles_img);
            if (even > tpmax) continue;
            if (2 * even < tpmax) return false;  // fragments would be under half full
            // A length rounded to whole 16-byte runs first, else the even split
            // (which can be whole rows where the rounded one is not).
            tile_px = (even + 3) / 4 * 4;
            if (tile_px > tpmax || rows_of(tile_px) > ROWS) tile_px = even;
        }
        if (rows_of(tile_px) > ROWS) continue;
        const int64_t ntiles = cdiv(OHW, tile_px);
        const int64_t blocks = co_blocks * P.N * ntiles;
        if (blocks < kMinDirectBlocks || blocks > kI32Max) return false;
        DirectArgs &a = pl->a;
        a.in = P.in;
        a.w = P.w;
        a.out = P.out;
        a.N = (int)P.N;
        a.CI = (int)P.CI;
        a.H = (int)P.H;
        a.W = (int)P.W;
        a.CO = (int)P.CO;
        a.OH = (int)P.OH;
        a.OW = (int)P.OW;
        a.st = (int)P.st;
        a.pady = (int)P.pady;
        a.padx = (int)P.padx;
        a.OHW = (int)OHW;
        a.HW = (int)(P.H * P.W);
        a.in_img = in_img;
        a.out_img = WMODE >= 2 ? P.g_c * P.fh * P.fw : P.CO * OHW;
        a.tile_px = (int)tile_px;
        a.tiles_img = (int)ntiles;
        a.co_blocks = (int)co_blocks;
        a.ncols = (int)ncols;
        a.w_bytes = (uint32_t)(w_elems * 4);
        a.out_vec = (tile_px % 4 == 0 && OHW % 4 == 0 && aligned16(P.out)) ? 1 : 0;
        a.beta = P.beta;
        a.fd_ow = fdiv(P.OW);
        a.g_c = (int)P.g_c;
        a.g_r = (int)P.g_r;
        a.g_s = (int)P.g_s;
        a.g_pad = (int)P.g_pad;
        a.g_amin = (int)P.g_amin;
        a.g_bmin = (int)P.g_bmin;
        a.g_crs = (int)(P.g_c * P.g_r * P.g_s);
        a.fh = (int)P.fh;
        a.fw = (int)P.fw;
        a.band_px = a.band_off = 0;
        // 16-byte weight loads: every float4 of a chunk row must lie inside
        // the row, which holds when rows start and end on multiples of 4.
        pl->wvec = WMODE != 2 && (WMODE == 0 ? P.CI % 4 == 0 : P.CO % 4 == 0) && aligned16(P.w);
        pl->blocks = blocks;
        pl->ok = true;
        return true;
    }
    return false;
}

template <int KT, int F, int CB, int R, int S, int ROWS, int PITCH, int WMODE, int EPI,
          bool S2 = false, bool RF = false, int PD = 0, int KG = 1>
int direct_fwd_run(const DirectFwdPlan &pl, hipStream_t st) {
    using Geo = DirectFwdGeo<KT, F, CB, R, S, ROWS, PITCH, WMODE, KG>;
    int rc;
    if (pl.wvec) {
        constexpr auto kern = direct_fwd_kernel<KT, F, CB, R, S, ROWS, PITCH, WMODE, EPI,
                                                WMODE != 2, S2, RF, PD, KG>;
        if ((rc = lds_optin<kern>(Geo::kBytes)) != KATSU_OK) return rc;
        kern<<<dim3((unsigned)pl.blocks), dim3(256 * KG), Geo::kBytes, st>>>(pl.a);
    } else {
        constexpr auto kern =
            direct_fwd_kernel<KT, F, CB, R, S, ROWS, PITCH, WMODE, EPI, false, S2, RF, PD, KG>;
        if ((rc = lds_optin<kern>(Geo::kBytes)) != KATSU_OK) return rc;
        kern<<<dim3((unsigned)pl.blocks), dim3(256 * KG), Geo::kBytes, st>>>(pl.a);
    }
    return launch_status();
}

// Direct forward-shaped variants: block tile (KT output channels x F
// fragments per wave), input-channel chunk, filter, halo rows and pitch.
template <int KT_, int F_, int CB_, int R_, int S_, int ROWS_, int PITCH_, bool S2_ = false,
          bool RF_ = false, int PD_ = 0, int KG_ = 1>
struct FwdVariant {
    static constexpr int KT = KT_, F = F_, CB = CB_, R = R_, S = S_, ROWS = ROWS_, PITCH = PITCH_;
    static constexpr bool S2 = S2_;  // stride-2 halo rows split by column parity
    static constexpr bool RF = RF_;  // one output row (<= 16 pixels) per fragment
    static constexpr int PD = PD_;   // phase form: the layer's padding
    static constexpr int KG = KG_;   // forward launches: groups of four waves per block
};
// 3x3 stride 1 (forward and data gradient): 64 x 208-pixel tiles.
#ifndef KATSU_FWDV
#define KATSU_FWDV 64, 13, 8, 3, 3, 7, 64
#endif
using FwdV = FwdVariant<KATSU_FWDV>;
// The same tile with halo rows 8 floats longer, for output rows of 8 (mod
// 16) pixels (56 at config 3): a fragment that runs from one row's end into
// the next then reads 16 distinct LDS banks, as a fragment inside a row
// does, instead of meeting the other channel group of its half-wave on the
// same banks.  The loads and the sums are those of FwdV, so are the bits.
#ifndef KATSU_FWD_PITCH8
#define KATSU_FWD_PITCH8 1
#endif
using FwdVP = FwdVariant<FwdV::KT, FwdV::F, FwdV::CB, FwdV::R, FwdV::S, FwdV::ROWS, FwdV::PITCH + 8>;
inline bool fwd_pitch8(int64_t ow) { return KATSU_FWD_PITCH8 && ow % 16 == 8; }
// 3x3 stride 2 forward: 64 x 64-pixel tiles, 32-float halo rows split by
// column parity.
#ifndef KATSU_FWD_S2_VARIANT
#define KATSU_FWD_S2_VARIANT 64, 4, 8, 3, 3, 12, 32, true
#endif
using FwdS2 = FwdVariant<KATSU_FWD_S2_VARIANT>;
// 3x3 stride 2 forward on rows of at most 16 pixels: 64 channels x 7 rows,
// one row per fragment.
#ifndef KATSU_FWD_S2R_VARIANT
#define KATSU_FWD_S2R_VARIANT 64, 7, 16, 3, 3, 16, 32, true, true, 0, 2
#endif
using FwdS2R = FwdVariant<KATSU_FWD_S2R_VARIANT>;
// Stride-2 data gradient by super-pixels: a 4x4 super-filter (7x7 layers
// such as the stem) with few channels, and a 2x2 one (3x3 layers).
using DxSp4 = FwdVariant<16, 13, 4, 4, 4, 11, 128>;
using DxSp2 = FwdVariant<64, 7, 16, 2, 2, 8, 32>;
#ifndef KATSU_DX_SP2R_VARIANT
#define KATSU_DX_SP2R_VARIANT 64, 7, 16, 2, 2, 8, 32, false, true
#endif
using DxSp2R = FwdVariant<KATSU_DX_SP2R_VARIANT>;  // super-pixel rows of at most 16
// Stride-2 data gradient by phases (WMODE 3), 3x3 filter with padding 1:
// 16 channels x 8 super-pixel rows of at most 16, 16 G channels per stage.
#ifndef KATSU_DX_PH_VARIANT
#define KATSU_DX_PH_VARIANT 16, 2, 16, 3, 3, 8, 32, false, true, 1
#endif
using DxPh = FwdVariant<KATSU_DX_PH_VARIANT>;

#define KATSU_FWD_VARIANT FwdV::KT, FwdV::F, FwdV::CB, FwdV::R, FwdV::S, FwdV::ROWS, FwdV::PITCH

// The variant's wave groups apply to forward launches (WMODE 0) only: the
// stride-1 dX shares its kernel body with the one-launch backward, whose dX
// blocks run four waves, and both must give the same bits.
template <class V, int WMODE, int EPI>
bool try_direct(const DirectFwdProblem &P, hipStream_t st, int *rc) {
    constexpr int KG = WMODE == 0 ? V::KG : 1;
    DirectFwdPlan pl;
    if (P.CO < V::KT / 2 ||
        !direct_fwd_plan<V::KT, V::F, V::CB, V::R, V::S, V::ROWS, V::PITCH, WMODE, V::S2, V::RF,
                         V::PD, KG>(P, &pl))
        return false;
    *rc = direct_fwd_run<V::KT, V::F, V::CB, V::R, V::S, V::ROWS, V::PITCH, WMODE, EPI, V::S2,
                         V::RF, V::PD, KG>(pl, st);
    return true;
}

// The stride-1 forward (WMODE 0) or dX (WMODE 1) with tiles of F and F-1
// fragments (direct_fwd_mix_kernel) when the plain plan's tiles are whole
// fragments short of F: an image's ceil(OHW/16) fragments over its
// tiles_img tiles, the first ones F, the rest F-1, with the F tiles fewer
// than one per CU slot of the grid's first half.  False = not applicable
// (the plain launch runs).
#ifndef KATSU_FWD_MIX
#define KATSU_FWD_MIX 1
#endif
template <class V, int WMODE>
bool try_direct_mix(const DirectFwdProblem &P, hipStream_t st, int *rc) {
    static_assert(WMODE == 0 || WMODE == 1, "stride-1 forward and dX");
    DirectFwdPlan pl;
    if (!KATSU_FWD_MIX || P.CO < V::KT / 2 ||
        !direct_fwd_plan<V::KT, V::F, V::CB, V::R, V::S, V::ROWS, V::PITCH, WMODE>(P, &pl))
        return false;
    const DirectArgs &a = pl.a;
    if (a.OHW % 16 != 0 || a.tiles_img < 2) return false;
    const int64_t q = a.OHW / 16, T = a.tiles_img;
    const int64_t fs = q / T, nbig = q - fs * T;
    if (fs + 1 != V::F || nbig == 0) return false;
    const int64_t n1 = (int64_t)a.co_blocks * a.N * nbig, n2 = pl.blocks - n1;
    if (2 * n1 > pl.blocks || n2 != (int64_t)a.co_blocks * a.N * (T - nbig)) return false;
    // Halo rows of the larger tile (whole fragments, any start column).
    if ((tile_row_span(16 * V::F, a.OW, a.OH) - 1) * a.st + V::R > V::ROWS) return false;
    DirectArgs a1 = a, a2 = a;
    a1.tile_px = a1.band_px = 16 * V::F;
    a1.tiles_img = (int)nbig;
    a1.band_off = 0;
    a2.tile_px = a2.band_px = 16 * (V::F - 1);
    a2.tiles_img = (int)(T - nbig);
    a2.band_off = (int)(16 * V::F * nbig);
    a1.out_vec = a2.out_vec = (a.OHW % 4 == 0 && aligned16(P.out)) ? 1 : 0;
    using Geo = DirectFwdGeo<V::KT, V::F, V::CB, V::R, V::S, V::ROWS, V::PITCH, WMODE>;
    if (pl.wvec) {
        constexpr auto kern =
            direct_fwd_mix_kernel<V::KT, V::F, V::CB, V::R, V::S, V::ROWS, V::PITCH, true, WMODE>;
        if ((*rc = lds_optin<kern>(Geo::kBytes)) != KATSU_OK) return true;
        kern<<<dim3((unsigned)pl.blocks), dim3(256), Geo::kBytes, st>>>(a1, a2, (int)n1);
    } else {
        constexpr auto kern =
            direct_fwd_mix_kernel<V::KT, V::F, V::CB, V::R, V::S, V::ROWS, V::PITCH, false, WMODE>;
        if ((*rc = lds_optin<kern>(Geo::kBytes)) != KATSU_OK) return true;
        kern<<<dim3((unsigned)pl.blocks), dim3(256), Geo::kBytes, st>>>(a1, a2, (int)n1);
    }
    *rc = launch_status();
    return true;
}

// Forward-shaped direct launch; false = no variant applies.
template <int WMODE>
bool direct_fwd(const DirectFwdProblem &P, hipStream_t st, int *rc) {
    if (P.st == 1 && P.CO >= FwdV::KT) {
        const bool p8 = fwd_pitch8(P.OW);
        if constexpr (WMODE <= 1)
            if (p8 ? try_direct_mix<FwdVP, WMODE>(P, st, rc) : try_direct_mix<FwdV, WMODE>(P, st, rc))
                return true;
        return p8 ? try_direct<FwdVP, WMODE, 0>(P, st, rc) : try_direct<FwdV, WMODE, 0>(P, st, rc);
    }
    if (WMODE == 0 && P.st == 2) {
        if (P.OW <= 16 && try_direct<FwdS2R, 0, 0>(P, st, rc)) return true;
        return try_direct<FwdS2, 0, 0>(P, st, rc);
    }
    return false;
}

// The stride-2 data gradient in phase form (direct.hpp, WMODE 3): input G,
// C output channels over the super-pixel grid, all four phases per block.
bool dx_phases_problem(const ConvDims &d, const float *gy, const float *w, float *dx, float beta,
                       DirectFwdProblem *P) {
    using Tp = Dxs2Taps<DxPh::R, DxPh::S, DxPh::PD>;
    if (d.st != 2 || d.R != DxPh::R || d.S != DxPh::S || d.pad != DxPh::PD || d.C < 16)
        return false;
    *P = DirectFwdProblem{gy, w, dx, d.N, d.K, d.OH, d.OW, d.C, d.R, d.S, 1, -Tp::DYMIN,
                          -Tp::DXMIN, (d.H + 1) / 2, (d.W + 1) / 2, beta};
    P->g_c = d.C;
    P->fh = d.H;
    P->fw = d.W;
    return true;
}

bool dx_phases_plan(const ConvDims &d, const float *gy, const float *w, float *dx, float beta,
                    DirectFwdPlan *pl) {
    DirectFwdProblem P;
    return dx_phases_problem(d, gy, w, dx, beta, &P) && P.CO >= DxPh::KT / 2 &&
           direct_fwd_plan<DxPh::KT, DxPh::F, DxPh::CB, DxPh::R, DxPh::S, DxPh::ROWS, DxPh::PITCH,
                           3, DxPh::S2, DxPh::RF, DxPh::PD>(P, pl);
}

bool dx_phases(const ConvDims &d, const float *gy, const float *w, float *dx, float beta,
               hipStream_t st, int *rc) {
    DirectFwdProblem P;
    return dx_phases_problem(d, gy, w, dx, beta, &P) && try_direct<DxPh, 3, 3>(P, st, rc);
}

// The stride-2 data gradient as a stride-1 problem over super-pixels (see
// direct.hpp, WMODE 2): input G, 4C output channels, super-filter offsets
// [amin, amax] per axis.
bool dx_superpixel(const ConvDims &d, const float *gy, const float *w, float *dx, float beta,
                   hipStream_t st, int *rc) {
    if (d.st != 2) return false;
    auto range = [&](int64_t R, int64_t *lo, int64_t *hi) {
        *lo = INT64_MAX;
        *hi = INT64_MIN;
        for (int64_t p = 0; p < 2; ++p)
            for (int64_t r = 0; r < R; ++r) {
                const int64_t e = p + d.pad - r;
                if (e % 2 != 0) continue;
                *lo = std::min(*lo, e / 2);
                *hi = std::max(*hi, e / 2);
            }
    };
    int64_t amin, amax, bmin, bmax;
    range(d.R, &amin, &amax);
    range(d.S, &bmin, &bmax);
    DirectFwdProblem P{gy, w, dx, d.N, d.K, d.OH, d.OW, 4 * d.C, amax - amin + 1,
                       bmax - bmin + 1, 1, -amin, -bmin, (d.H + 1) / 2, (d.W + 1) / 2, beta};
    P.g_c = d.C;
    P.g_r = d.R;
    P.g_s = d.S;
    P.g_pad = d.pad;
    P.g_amin = amin;
    P.g_bmin = bmin;
    P.fh = d.H;
    P.fw = d.W;
    if (P.R == DxSp4::R && P.S == DxSp4::S && P.CO <= 16) return try_direct<DxSp4, 2, 1>(P, st, rc);
    if (P.R == DxSp2::R && P.S == DxSp2::S) {
        if (P.OW <= 16 && try_direct<DxSp2R, 2, 1>(P, st, rc)) return true;
        return try_direct<DxSp2, 2, 1>(P, st, rc);
    }
    return false;
}

// The data gradient as a forward problem (stride 1 only): G convolved with
// the transposed, flipped filter, padding R-1-pad (rows) / S-1-pad (columns).
bool dx_as_forward(const ConvDims &d, const float *gy, const float *w, float *dx, float beta,
                   DirectFwdProblem *P) {
    if (d.st != 1 || d.pad > d.R - 1 || d.pad > d.S - 1) return false;
    *P = DirectFwdProblem{gy, w, dx, d.N, d.K, d.OH, d.OW, d.C, d.R, d.S, 1,
                          d.R - 1 - d.pad, d.S - 1 - d.pad, d.H, d.W, beta};
    return true;
}

// Filter gradient.  Plan first (the workspace size is part of the API), then launch.
struct DirectDwPlan {
    bool ok = false;
    int variant = -1;
    DirectDwArgs a;
    int64_t blocks = 0;
    int splits = 0;
    int64_t pstride = 0;  // floats between partials
    size_t ws_bytes = 0;
    size_t lds_bytes = 0;
    bool full = false;  // every tile row is a multiple of 4 pixels wide
};

// Fixed-order sum of split-K partials into dw.  G split groups per float4
// column, U loads in flight per thread: the smallest G in {8, 16, 32} that
// keeps each thread's chain at 8 loads, else G = 32 with 16 in flight (a
// wave then still reads whole 128-byte runs of eight partials).
template <int G, int U>
int split_reduce_g(const float *ws, float *dw, int64_t elems, int64_t pstride, int splits,
                   float beta, hipStream_t st) {
    dw_split_reduce<G, U><<<dim3((unsigned)cdiv(elems, (256 / G) * 4)), dim3(256), 0, st>>>(
        ws, dw, elems, pstride, splits, beta);
    return launch_status();
}

int launch_split_reduce(const float *ws, float *dw, int64_t elems, int64_t pstride, int splits,
                        float beta, hipStream_t st) {
    const int64_t chain = cdiv(splits, 8);
    if (chain <= 8) return split_reduce_g<8, 8>(ws, dw, elems, pstride, splits, beta, st);
    if (chain <= 16) return split_reduce_g<16, 8>(ws, dw, elems, pstride, splits, beta, st);
    if (chain <= 32) return split_reduce_g<32, 8>(ws, dw, elems, pstride, splits, beta, st);
    return split_reduce_g<32, 16>(ws, dw, elems, pstride, splits, beta, st);
}

template <int ST, int KT, int CT, int R, int S, int ROWS, int PITCH, int GPC, int WKF>
bool direct_dw_plan(const ConvDims &d, int64_t target_blocks, DirectDwPlan *pl) {
    using Geo = DirectDwGeo<KT, CT, R, S, ROWS, PITCH, GPC>;
    if (d.R != R || d.S != S || (ST != 0 && d.st != ST)) return false;
    const int64_t tmax = Geo::GMAX;  // G tile capacity (pixels)
    const int64_t ncols = (int64_t)(d.OW - 1) * d.st + S;
    if (ncols > PITCH || R > ROWS) return false;
    // Buffer resources address one image of x and of G in bytes.
    if ((int64_t)d.CHW * 4 >= (int64_t)kMaxBufBytes || (int64_t)d.KOHW * 4 >= (int64_t)kMaxBufBytes)
        return false;
    // Whole output rows per tile when a row fits, else balanced row segments.
    int64_t trows = 1, seg_w = d.OW;
    if (d.OW <= tmax) {
        trows = std::min<int64_t>(tmax / d.OW, (ROWS - R) / d.st + 1);
        trows = std::max<int64_t>(1, std::min<int64_t>(trows, d.OH));
    } else {
        seg_w = cdiv(d.OW, cdiv(d.OW, tmax));
    }
    // LDS: two stages of [KT][gpitch] G + [CT][CPITCH] x; the epilogue's
    // [KT][PPITCH] transpose reuses them.
    const int64_t gcap = (trows * seg_w + 3) / 4 * 4;
    const int64_t gpitch = gcap % 4 == 0 ? gcap + 2 : gcap;  // == 2 (mod 4)
    const int64_t stage = KT * gpitch + Geo::XS;
    // The stages (or the epilogue's transpose), then the block's flag word.
    const int64_t flag = std::max<int64_t>(2 * stage, (int64_t)KT * Geo::PPITCH);
    const int64_t lds = (flag + 4) * 4;
    if (lds > kLdsMax) return false;
    const int64_t segs = cdiv(d.OW, seg_w);
    const int64_t tiles_img = cdiv(d.OH, trows) * segs;
    const int64_t tiles_total = (int64_t)d.N * tiles_img;
    const int64_t kb = cdiv(d.K, KT), cb = cdiv(d.C, CT);
    int64_t splits = std::max<int64_t>(1, cdiv(target_blocks, kb * cb));
    splits = std::min(splits, tiles_total);
    const int64_t tps = cdiv(tiles_total, splits);
    splits = cdiv(tiles_total, tps);
    const int64_t blocks = kb * cb * splits;
    if (blocks < kMinDirectBlocks / 2 || blocks > kI32Max) return false;
    const int64_t elems = (int64_t)d.K * d.CRS;
    DirectDwArgs &a = pl->a;
    a.x = nullptr;
    a.g = nullptr;
    a.out = nullptr;
    a.N = d.N;
    a.C = d.C;
    a.H = d.H;
    a.W = d.W;
    a.K = d.K;
    a.OH = d.OH;
    a.OW = d.OW;
    a.st = d.st;
    a.pad = d.pad;
    a.OHW = d.OHW;
    a.HW = d.HW;
    a.CRS = d.CRS;
    a.x_img = d.CHW;
    a.g_img = d.KOHW;
    a.trows = (int)trows;
    a.seg_w = (int)seg_w;
    a.segs = (int)segs;
    a.tiles_img = (int)tiles_img;
    a.tiles_total = (int)tiles_total;
    a.tiles_per_split = (int)tps;
    a.k_blocks = (int)kb;
    a.c_blocks = (int)cb;
    a.ncols = (int)ncols;
    a.gpitch = (int)gpitch;
    a.gcap = (int)gcap;
    a.stage = (int)stage;
    a.out_vec = d.CRS % 4 == 0 ? 1 : 0;
    a.split_stride = 0;
    a.beta = 0.f;
    a.fd_tiles_img = fdiv(tiles_img);
    a.fd_segs = fdiv(segs);
    a.flag = (int)flag;
    pl->ok = true;
    pl->blocks = blocks;
    pl->splits = (int)splits;
    pl->lds_bytes = (size_t)lds;
    pl->full = segs == 1 ? d.OW % 4 == 0
                         : seg_w % 4 == 0 && (d.OW - (segs - 1) * seg_w) % 4 == 0;
    pl->pstride = (elems + 3) / 4 * 4;
    pl->ws_bytes = splits > 1 ? (size_t)splits * (size_t)pl->pstride * sizeof(float) : 0;
    return true;
}

// Variant table, in order of preference: id, the stride it requires (0: any),
// block tile (KT output x CT input channels), filter R x S, halo rows and
// row pitch of the x tile, G tile capacity in 64-pixel chunks, oc fragments
// per wave, and the target block count that sets the split over output
// pixels.  Variant 1 takes stride-2 layers with small images: four output
// rows per tile on 32-float halo rows.
#ifndef KATSU_DW_VARIANTS
#define KATSU_DW_VARIANTS(X)                    \
    X(1, 2, 64, 16, 3, 3, 10, 32, 1, 1, 512)    \
    X(0, 0, 64, 32, 3, 3, 3, 64, 1, 2, 512)
#endif

// The first variant that plans (only `variant` when it is given), with its
// target block count divided by `tb_div`.
DirectDwPlan direct_dw_plan_any(const ConvDims &d, int variant = -1, int tb_div = 1) {
    DirectDwPlan pl;
#define KATSU_DW_TRY(id, ST, KT, CT, R, S, ROWS, PITCH, GPC, WKF, TB)                      \
    if (pl.variant < 0 && (variant < 0 || variant == id) && d.K >= KT &&                     \
        direct_dw_plan<ST, KT, CT, R, S, ROWS, PITCH, GPC, WKF>(d, TB / tb_div, &pl))        \
        pl.variant = id;
    KATSU_DW_VARIANTS(KATSU_DW_TRY)
#undef KATSU_DW_TRY
    pl.ok = pl.variant >= 0;
    return pl;
}

template <int KT, int CT, int R, int S, int ROWS, int PITCH, int GPC, int WKF, bool FULL>
int dw_kernel_launch(const DirectDwPlan &pl, hipStream_t st) {
    constexpr auto kern = direct_dw_kernel<KT, CT, R, S, ROWS, PITCH, GPC, WKF, FULL>;
    const int rc = lds_optin<kern>(kLdsMax);
    if (rc != KATSU_OK) return rc;
    kern<<<dim3((unsigned)pl.blocks), dim3(256), pl.lds_bytes, st>>>(pl.a);
    return launch_status();
}

// Binds the operands of a planned direct dW launch.
void dw_bind(DirectDwPlan *pl, const float *x, const float *gy, float *dw, float beta, float *ws) {
    DirectDwArgs &a = pl->a;
    const bool direct = pl->splits == 1;
    a.x = x;
    a.g = gy;
    a.out = direct ? dw : ws;
    a.split_stride = direct ? 0 : pl->pstride;
    a.beta = direct ? beta : 0.f;
    if (!aligned16(a.out)) a.out_vec = 0;
}

int direct_dw_launch(DirectDwPlan pl, const float *x, const float *gy, float *dw, float beta,
                     float *ws, hipStream_t st) {
    dw_bind(&pl, x, gy, dw, beta, ws);
    int rc = KATSU_E_INVALID;
    switch (pl.variant) {
#define KATSU_DW_CASE(id, ST, KT, CT, R, S, ROWS, PITCH, GPC, WKF, TB)                   \
    case id:                                                                              \
        rc = pl.full ? dw_kernel_launch<KT, CT, R, S, ROWS, PITCH, GPC, WKF, true>(pl, st)   \
                     : dw_kernel_launch<KT, CT, R, S, ROWS, PITCH, GPC, WKF, false>(pl, st); \
        break;
        KATSU_DW_VARIANTS(KATSU_DW_CASE)
#undef KATSU_DW_CASE
        default: return KATSU_E_INVALID;
    }
    if (rc != KATSU_OK || pl.splits == 1) return rc;
    return launch_split_reduce(ws, dw, (int64_t)pl.a.K * pl.a.CRS, pl.pstride, pl.splits, beta,
                               st);
}

// dX and dW in one launch (direct_bwd_kernel): the direct dX plan and a
// direct dW variant with the same filter size.
template <class XV, int XWMODE, int XEPI, int KT, int CT, int R, int S, int ROWS, int PITCH,
          int GPC, int WKF, bool FULL, bool XWVEC>
int bwd_fused_kernel_launch(const DirectFwdPlan &xp, const DirectDwPlan &wp, hipStream_t st) {
    using XGeo = DirectFwdGeo<XV::KT, XV::F, XV::CB, XV::R, XV::S, XV::ROWS, XV::PITCH, XWMODE>;
    constexpr auto kern = direct_bwd_kernel<XV::KT, XV::F, XV::CB, R, S, XV::ROWS, XV::PITCH,
                                            XWVEC, KT, CT, ROWS, PITCH, GPC, WKF, FULL, XWMODE,
                                            XEPI, XV::RF, XV::PD>;
    const int rc = lds_optin<kern>(kLdsMax);
    if (rc != KATSU_OK) return rc;
    const size_t lds = std::max(XGeo::kBytes, wp.lds_bytes);
    kern<<<dim3((unsigned)(xp.blocks + wp.blocks)), dim3(256), lds, st>>>(xp.a, wp.a,
                                                                         (int)wp.blocks);
    return launch_status();
}

template <class XV, int XWMODE, int XEPI, int KT, int CT, int R, int S, int ROWS, int PITCH,
          int GPC, int WKF>
int bwd_fused_dx(const DirectFwdPlan &xp, const DirectDwPlan &wp, hipStream_t st) {
    if (wp.full)
        return xp.wvec ? bwd_fused_kernel_launch<XV, XWMODE, XEPI, KT, CT, R, S, ROWS, PITCH, GPC,
                                                 WKF, true, true>(xp, wp, st)
                       : bwd_fused_kernel_launch<XV, XWMODE, XEPI, KT, CT, R, S, ROWS, PITCH, GPC,
                                                 WKF, true, false>(xp, wp, st);
    return xp.wvec ? bwd_fused_kernel_launch<XV, XWMODE, XEPI, KT, CT, R, S, ROWS, PITCH, GPC, WKF,
                                             false, true>(xp, wp, st)
                   : bwd_fused_kernel_launch<XV, XWMODE, XEPI, KT, CT, R, S, ROWS, PITCH, GPC, WKF,
                                             false, false>(xp, wp, st);
}

// Two-size stride-1 dX tiles for the shared launch (direct_bwd_band_kernel):
// per band of two plain tiles' rows, a first tile of ceil(rows/2) rows and a
// second of the rest, when the image is whole bands,
// the tiles fit kBandF1 and kBandF2 fragments and the halo rows, and there
// is one first-tile block per dW block (one per CU slot at the start).
#ifndef KATSU_FUSED_BAND
#define KATSU_FUSED_BAND 1
#endif
constexpr int kBandF1 = 14, kBandF2 = 11;

bool band_plans(const DirectFwdPlan &xp, const DirectDwPlan &wp, DirectArgs *a1, DirectArgs *a2,
                int64_t *n1, int64_t *n2) {
    const DirectArgs &a = xp.a;
    if (!KATSU_FUSED_BAND || a.st != 1) return false;
    const int band_px = 2 * a.tile_px;
    if (band_px % a.OW != 0) return false;
    const int band_rows = band_px / a.OW;
    const int r1 = (band_rows + 1) / 2, r2 = band_rows - r1;
    if (r2 < 1 || a.OH % band_rows != 0 || r1 * a.OW > 16 * kBandF1 ||
        r2 * a.OW > 16 * kBandF2 || r1 - 1 + FwdV::R > FwdV::ROWS)
        return false;
    const int bands = a.OH / band_rows;
    const int64_t nb = (int64_t)a.co_blocks * a.N * bands;
    if (nb != wp.blocks || 2 * nb != xp.blocks) return false;
    // The first tiles lie together at the top of the image and the second
    // ones below them, so each set's neighbouring tiles share their halo
    // rows while they run at the same time (one fetch into L2).
    *a1 = a;
    *a2 = a;
    a1->tiles_img = a2->tiles_img = bands;
    a1->tile_px = a1->band_px = r1 * a.OW;
    a1->band_off = 0;
    a2->tile_px = a2->band_px = r2 * a.OW;
    a2->band_off = bands * r1 * a.OW;
    const bool v4 = (r1 * a.OW) % 4 == 0 && (r2 * a.OW) % 4 == 0 && a.OHW % 4 == 0;
    a1->out_vec = a2->out_vec = a.out_vec && v4 ? 1 : 0;
    *n1 = *n2 = nb;
    return true;
}

template <class XV, int KT, int CT, int R, int S, int ROWS, int PITCH, int GPC, int WKF,
          bool FULL, bool XWVEC>
int bwd_band_kernel_launch(const DirectArgs &a1, const DirectArgs &a2, int64_t n1, int64_t n2,
                           const DirectDwPlan &wp, hipStream_t st) {
    using XGeo = DirectFwdGeo<XV::KT, kBandF1, XV::CB, R, S, XV::ROWS, XV::PITCH, 1>;
    constexpr auto kern =
        direct_bwd_band_kernel<XV::KT, kBandF1, kBandF2, XV::CB, R, S, XV::ROWS, XV::PITCH,
                               XWVEC, KT, CT, ROWS, PITCH, GPC, WKF, FULL>;
    const int rc = lds_optin<kern>(kLdsMax);
    if (rc != KATSU_OK) return rc;
    const size_t lds = std::max(XGeo::kBytes, wp.lds_bytes);
    kern<<<dim3((unsigned)(wp.blocks + n1 + n2)), dim3(256), lds, st>>>(a1, a2, wp.a,
                                                                      (int)wp.blocks, (int)n1);
    return launch_status();
}

// The stride-1 dX blocks of a shared launch, FwdV's tile at XV's halo pitch:
// two-size tiles when band_plans applies, else the plain tiles.
template <class XV, int KT, int CT, int R, int S, int ROWS, int PITCH, int GPC, int WKF>
int bwd_fused_s1(const DirectFwdPlan &xp, const DirectDwPlan &wp, hipStream_t st) {
    DirectArgs a1, a2;
    int64_t n1, n2;
    if (band_plans(xp, wp, &a1, &a2, &n1, &n2)) {
        if (wp.full)
            return xp.wvec ? bwd_band_kernel_launch<XV, KT, CT, R, S, ROWS, PITCH, GPC, WKF, true,
                                                    true>(a1, a2, n1, n2, wp, st)
                           : bwd_band_kernel_launch<XV, KT, CT, R, S, ROWS, PITCH, GPC, WKF, true,
                                                    false>(a1, a2, n1, n2, wp, st);
        return xp.wvec ? bwd_band_kernel_launch<XV, KT, CT, R, S, ROWS, PITCH, GPC, WKF, false,
                                                true>(a1, a2, n1, n2, wp, st)
                       : bwd_band_kernel_launch<XV, KT, CT, R, S, ROWS, PITCH, GPC, WKF, false,
                                                false>(a1, a2, n1, n2, wp, st);
    }
    return bwd_fused_dx<XV, 1, 0, KT, CT, R, S, ROWS, PITCH, GPC, WKF>(xp, wp, st);
}

// The dX blocks of a shared launch: the stride-1 form (FwdV or FwdVP, WMODE
// 1) with a stride-1 dW variant, the stride-2 phase form (DxPh, WMODE 3)
// with a stride-2 one.
template <int ST, int KT, int CT, int R, int S, int ROWS, int PITCH, int GPC, int WKF>
int bwd_fused_variant(const DirectFwdPlan &xp, const DirectDwPlan &wp, hipStream_t st) {
    if constexpr (ST != 2 && R == FwdV::R && S == FwdV::S) {
        return fwd_pitch8(xp.a.OW)
                   ? bwd_fused_s1<FwdVP, KT, CT, R, S, ROWS, PITCH, GPC, WKF>(xp, wp, st)
                   : bwd_fused_s1<FwdV, KT, CT, R, S, ROWS, PITCH, GPC, WKF>(xp, wp, st);
    }
    else if constexpr (ST == 2 && R == DxPh::R && S == DxPh::S)
        return bwd_fused_dx<DxPh, 3, 3, KT, CT, R, S, ROWS, PITCH, GPC, WKF>(xp, wp, st);
    return KATSU_E_INVALID;
}

// Whether a dW variant can share a launch with the direct dX kernel of the
// layer's stride (see bwd_fused_variant).
#ifndef KATSU_FUSE_S2
#define KATSU_FUSE_S2 1
#endif
bool dw_variant_fusable(int variant, int64_t stride) {
#define KATSU_DW_FUSABLE(id, st, kt, ct, r, s, rows, pitch, gpc, wkf, tb)            \
    if (variant == id)                                                               \
        return stride == 2 ? KATSU_FUSE_S2 && st == 2 && r == DxPh::R && s == DxPh::S \
                           : st != 2 && r == FwdV::R && s == FwdV::S;
    KATSU_DW_VARIANTS(KATSU_DW_FUSABLE)
#undef KATSU_DW_FUSABLE
    return false;
}

int bwd_fused_launch(const DirectFwdPlan &xp, DirectDwPlan wp, const float *x, const float *gy,
                     float *dw, float beta, float *ws, hipStream_t st) {
    dw_bind(&wp, x, gy, dw, beta, ws);
    int rc = KATSU_E_INVALID;
    switch (wp.variant) {
#define KATSU_DW_FUSED(id, ST, KT, CT, R, S, ROWS, PITCH, GPC, WKF, TB)          \
    case id: rc = bwd_fused_variant<ST, KT, CT, R, S, ROWS, PITCH, GPC, WKF>(xp, wp, st); break;
        KATSU_DW_VARIANTS(KATSU_DW_FUSED)
#undef KATSU_DW_FUSED
        default: return KATSU_E_INVALID;
    }
    if (rc != KATSU_OK || wp.splits == 1) return rc;
    return launch_split_reduce(ws, dw, (int64_t)wp.a.K * wp.a.CRS, wp.pstride, wp.splits, beta,
                               st);
}

// ---------------------------------------------------------------------------
// 1x1 convolutions without padding (pw_kernel): every output pixel reads one
// input pixel, so the three passes are plain GEMMs over gathered pixels.

bool pw_ok(const ConvDims &d) {
    return d.R == 1 && d.S == 1 && d.pad == 0 && d.npix_out > 0 && d.npix_out < kI32Max;
}

PwArgs pw_args(const ConvDims &d, int64_t m, int64_t n, int64_t k) {
    PwArgs a{};
    a.M = (int)m;
    a.N = (int)n;
    a.K = (int)k;
    a.C = d.C;
    a.H = d.H;
    a.W = d.W;
    a.KO = d.K;
    a.OW = d.OW;
    a.OHW = d.OHW;
    a.HW = d.HW;
    a.st = d.st;
    a.x_img = d.CHW;
    a.g_img = d.KOHW;
    a.fd_ohw = fdiv(d.OHW);
    a.fd_ow = fdiv(d.OW);
    a.splits = 1;
    a.kchunk = (int)((k + 31) / 32 * 32);
    a.x_bytes = (uint32_t)std::min<int64_t>((int64_t)d.N * d.CHW * 4, kMaxBufBytes);
    a.w_bytes = (uint32_t)std::min<int64_t>((int64_t)d.K * d.C * 4, kMaxBufBytes);
    a.g_bytes = (uint32_t)std::min<int64_t>((int64_t)d.N * d.KOHW * 4, kMaxBufBytes);
    return a;
}

#ifndef KATSU_PW_PF
#define KATSU_PW_PF 2  // k-tiles in flight in pw_kernel's dX and dW (1: one, through LDS stages)
#endif
constexpr int kPwPf = KATSU_PW_PF;

// Whether the 1x1 dX and dW take the buffer-load ring (pw_block, PF > 1):
// every operand within the buffer range, and the dX's reduction (K output
// channels) at least PF k-tiles deep.
bool pw_ring(const ConvDims &d) {
    return kPwPf > 1 && cdiv(d.K, 32) >= kPwPf &&
           (int64_t)d.N * d.CHW * 4 < (int64_t)kMaxBufBytes &&
           (int64_t)d.N * d.KOHW * 4 < (int64_t)kMaxBufBytes &&
           (int64_t)d.K * d.C * 4 < (int64_t)kMaxBufBytes;
}

// 64-row tiles when they still give every CU a block, else 32.
int pw_bm(int64_t m, int64_t n, int64_t splits) {
    return cdiv(m, 64) * cdiv(n, 64) * splits >= kMinDirectBlocks ? 64 : 32;
}

template <int MODE, int BM, int V, int PF>
int pw_launch(PwArgs a, hipStream_t st) {
    a.tiles_m = (int)cdiv(a.M, BM);
    a.tiles_n = (int)cdiv(a.N, PwGeo<BM>::BN);
    const int64_t blocks = (int64_t)a.tiles_m * a.tiles_n * a.splits;
    if (blocks <= 0) return KATSU_OK;
    if (blocks > kI32Max) return KATSU_E_INVALID;
    pw_kernel<MODE, BM, V, PF><<<dim3((unsigned)blocks), dim3(256), PwGeo<BM>::kBytes, st>>>(a);
    return launch_status();
}

// Vector loads of pw_kernel: 1 = the A operand 16 bytes at a time (forward
// and dX: the weight, rows of length C % 4 = 0 from a 16-byte aligned base;
// dW: G along pixels, planes of OH*OW % 4 = 0 floats from a 16-byte aligned
// base); 3 = the dX's G too (the same plane condition).
int pw_vec(const PwArgs &a, int mode) {
    const bool gv = a.OHW % 4 == 0 && aligned16(a.g);
    if (mode == 2) return gv ? 1 : 0;
    if (a.C % 4 != 0 || !aligned16(a.w)) return 0;
    return mode == 1 && gv ? 3 : 1;
}

template <int MODE, int V, int PF>
int pw_run_v(const PwArgs &a, hipStream_t st) {
    return pw_bm(a.M, a.N, a.splits) == 64 ? pw_launch<MODE, 64, V, PF>(a, st)
                                             : pw_launch<MODE, 32, V, PF>(a, st);
}

template <int MODE, int PF>
int pw_run_pf(const PwArgs &a, hipStream_t st) {
    const int v = pw_vec(a, MODE);
    if (MODE == 1 && v == 3) return pw_run_v<MODE, MODE == 1 ? 3 : 0, PF>(a, st);
    if (v == 1) return pw_run_v<MODE, 1, PF>(a, st);
    return pw_run_v<MODE, 0, PF>(a, st);
}

// ring: pw_ring(d) for the layer (dX and dW only).
template <int MODE>
int pw_run(const PwArgs &a, bool ring, hipStream_t st) {
    if constexpr (MODE != 0 && kPwPf > 1)
        if (ring) return pw_run_pf<MODE, kPwPf>(a, st);
    return pw_run_pf<MODE, 1>(a, st);
}

#ifndef KATSU_PW_RD
#define KATSU_PW_RD 1
#endif

// The register-direct forward (pw_rd_fwd_kernel): C = 64, 128 or 256, w rows
// 16-byte aligned, operands within the buffer range, at least one block per CU.
template <int NKB>
int pw_rd_fwd_launch(PwArgs a, hipStream_t st) {
    a.tiles_m = (int)cdiv(a.M, 64);
    a.tiles_n = (int)cdiv(a.N, 64);
    const int64_t blocks = (int64_t)a.tiles_m * a.tiles_n;
    pw_rd_fwd_kernel<NKB><<<dim3((unsigned)blocks), dim3(256), 4 * 64 * 64 * sizeof(float), st>>>(a);
    return launch_status();
}

bool pw_rd_fwd_ok(const ConvDims &d, const float *x, const float *w) {
    const int64_t xb = (int64_t)d.N * d.CHW * 4, wb = (int64_t)d.K * d.C * 4;
    return KATSU_PW_RD && (d.C == 64 || d.C == 128 || d.C == 256) && aligned16(w) &&
           xb < (int64_t)kMaxBufBytes && wb < (int64_t)kMaxBufBytes &&
           cdiv(d.K, 64) * cdiv(d.npix_out, 64) >= kMinDirectBlocks;
}

int pw_fwd(const float *x, const float *w, float *y, const ConvDims &d, hipStream_t st) {
    PwArgs a = pw_args(d, d.K, d.npix_out, d.C);
    a.x = x;
    a.w = w;
    a.out = y;
    a.beta = 0.f;
    if (pw_rd_fwd_ok(d, x, w)) {
        a.x_bytes = (uint32_t)((int64_t)d.N * d.CHW * 4);
        a.w_bytes = (uint32_t)((int64_t)d.K * d.C * 4);
        return d.C == 64    ? pw_rd_fwd_launch<1>(a, st)
               : d.C == 128 ? pw_rd_fwd_launch<2>(a, st)
                            : pw_rd_fwd_launch<4>(a, st);
    }
    return pw_run<0>(a, false, st);
}

// Whether the 1x1 dX epilogue may write whole 2 x 4 blocks of dx (pw_block,
// PwArgs::quad): every output pixel's stride-2 block lies inside the image
// and a lane's pixel pair shares a row.
int pw_quad(const ConvDims &d, const float *dx, float beta) {
    return d.st == 2 && d.H == 2 * d.OH && d.W == 2 * d.OW && d.OW % 2 == 0 && beta == 0.f &&
           aligned16(dx);
}

int pw_dx(const float *gy, const float *w, float *dx, const ConvDims &d, float beta,
          hipStream_t st) {
    PwArgs a = pw_args(d, d.C, d.npix_out, d.K);
    a.g = gy;
    a.w = w;
    a.out = dx;
    a.beta = beta;
    a.quad = pw_quad(d, dx, beta);
    return pw_run<1>(a, pw_ring(d), st);
}

// dW: the pixel reduction split so the launch has about two blocks per CU,
// each split at least 256 pixels long.
struct PwDwPlan {
    bool ok = false;
    int splits = 1, kchunk = 32;
    int64_t pstride = 0;
    size_t ws_bytes = 0;
};

PwDwPlan pw_dw_plan(const ConvDims &d) {
    PwDwPlan pl;
    if (!pw_ok(d)) return pl;
    const int64_t kred = d.npix_out;
    const int64_t tiles = cdiv(d.K, 32) * cdiv(d.C, 64);
    int64_t splits = std::max<int64_t>(1, cdiv(2 * kMinDirectBlocks, tiles));
    splits = std::min(splits, std::max<int64_t>(1, kred / 256));
    // With the ring, slices of whole rounds of kPwPf k-tiles.
    const int64_t q = pw_ring(d) ? 32 * kPwPf : 32;
    const int64_t kchunk = cdiv(cdiv(kred, splits), q) * q;
    splits = cdiv(kred, kchunk);
    pl.ok = true;
    pl.splits = (int)splits;
    pl.kchunk = (int)kchunk;
    pl.pstride = ((int64_t)d.K * d.C + 3) / 4 * 4;
    pl.ws_bytes = splits > 1 ? (size_t)splits * (size_t)pl.pstride * sizeof(float) : 0;
    return pl;
}

int pw_dw(const float *x, const float *gy, float *dw, const ConvDims &d, const PwDwPlan &pl,
          float beta, float *ws, hipStream_t st) {
    PwArgs a = pw_args(d, d.K, d.C, d.npix_out);
    a.x = x;
    a.g = gy;
    const bool direct = pl.splits == 1;
    a.out = direct ? dw : ws;
    a.beta = direct ? beta : 0.f;
    a.splits = pl.splits;
    a.kchunk = pl.kchunk;
    a.split_stride = direct ? 0 : pl.pstride;
    const int rc = pw_run<2>(a, pw_ring(d), st);
    if (rc != KATSU_OK || direct) return rc;
    return launch_split_reduce(ws, dw, (int64_t)d.K * d.C, pl.pstride, pl.splits, beta, st);
}

// dX and dW of a 1x1 layer in one launch (pw_bwd_kernel), then the reduce:
// the same plans as the two separate calls, so the same bits.  False = the
// dW block count is not a multiple of 8 (the shared grid would move the dX
// blocks' XCD placement): the caller runs the separate calls.
template <int BMX, int BMW, int VX, int VW, int PF>
int pw_bwd_launch(PwArgs ax, PwArgs aw, hipStream_t st) {
    ax.tiles_m = (int)cdiv(ax.M, BMX);
    ax.tiles_n = (int)cdiv(ax.N, PwGeo<BMX>::BN);
    aw.tiles_m = (int)cdiv(aw.M, BMW);
    aw.tiles_n = (int)cdiv(aw.N, PwGeo<BMW>::BN);
    const int64_t bx = (int64_t)ax.tiles_m * ax.tiles_n, bw = (int64_t)aw.tiles_m * aw.tiles_n * aw.splits;
    if (bx + bw > kI32Max) return KATSU_E_INVALID;
    const size_t lds = std::max(PwGeo<BMX>::kBytes, PwGeo<BMW>::kBytes);
    pw_bwd_kernel<BMX, BMW, VX, VW, PF>
        <<<dim3((unsigned)(bx + bw)), dim3(256), lds, st>>>(ax, aw, (int)bw);
    return launch_status();
}

template <int VX, int VW, int PF>
int pw_bwd_bm(int bmx, int bmw, const PwArgs &ax, const PwArgs &aw, hipStream_t st) {
    return bmx == 64 ? (bmw == 64 ? pw_bwd_launch<64, 64, VX, VW, PF>(ax, aw, st)
                                  : pw_bwd_launch<64, 32, VX, VW, PF>(ax, aw, st))
                     : (bmw == 64 ? pw_bwd_launch<32, 64, VX, VW, PF>(ax, aw, st)
                                  : pw_bwd_launch<32, 32, VX, VW, PF>(ax, aw, st));
}

template <int VX, int PF>
int pw_bwd_vw(int bmx, int bmw, const PwArgs &ax, const PwArgs &aw, hipStream_t st) {
    return pw_vec(aw, 2) == 1 ? pw_bwd_bm<VX, 1, PF>(bmx, bmw, ax, aw, st)
                              : pw_bwd_bm<VX, 0, PF>(bmx, bmw, ax, aw, st);
}

template <int PF>
int pw_bwd_pf(int bmx, int bmw, const PwArgs &ax, const PwArgs &aw, hipStream_t st) {
    const int vx = pw_vec(ax, 1);
    return vx == 3   ? pw_bwd_vw<3, PF>(bmx, bmw, ax, aw, st)
           : vx == 1 ? pw_bwd_vw<1, PF>(bmx, bmw, ax, aw, st)
                     : pw_bwd_vw<0, PF>(bmx, bmw, ax, aw, st);
}

bool pw_bwd(const float *x, const float *w, const float *gy, float *dx, float *dw,
            const ConvDims &d, const PwDwPlan &pl, float beta, float *ws, hipStream_t st,
            int *rc) {
    PwArgs ax = pw_args(d, d.C, d.npix_out, d.K);
    ax.g = gy;
    ax.w = w;
    ax.out = dx;
    ax.beta = beta;
    ax.quad = pw_quad(d, dx, beta);
    PwArgs aw = pw_args(d, d.K, d.C, d.npix_out);
    aw.x = x;
    aw.g = gy;
    const bool direct = pl.splits == 1;
    aw.out = direct ? dw : ws;
    aw.beta = direct ? beta : 0.f;
    aw.splits = pl.splits;
    aw.kchunk = pl.kchunk;
    aw.split_stride = direct ? 0 : pl.pstride;
    const int bmx = pw_bm(ax.M, ax.N, 1), bmw = pw_bm(aw.M, aw.N, aw.splits);
    if (cdiv(aw.M, bmw) * cdiv(aw.N, 64) * aw.splits % 8 != 0) return false;
    *rc = pw_ring(d) ? pw_bwd_pf<kPwPf>(bmx, bmw, ax, aw, st)
                     : pw_bwd_pf<1>(bmx, bmw, ax, aw, st);
    if (*rc == KATSU_OK && !direct)
        *rc = launch_split_reduce(ws, dw, (int64_t)d.K * d.C, pl.pstride, pl.splits, beta, st);
    return true;
}

// ---------------------------------------------------------------------------
// The stem forward (stem_fwd_kernel): three input channels, 7x7, rows of at
// most 112 output pixels.

constexpr int kStemF = 7, kStemPitch = 256;

template <int ST>
int stem_fwd_launch(const StemArgs &a, unsigned blocks, hipStream_t st) {
    using Geo = StemGeo<3, 7, 7, kStemPitch>;
    constexpr auto kern = stem_fwd_kernel<3, 7, 7, kStemF, kStemPitch, ST>;
    const int rc = lds_optin<kern>(Geo::kBytes);
    if (rc != KATSU_OK) return rc;
    kern<<<dim3(blocks), dim3(512), Geo::kBytes, st>>>(a);
    return launch_status();
}

bool stem_fwd(const float *x, const float *w, float *y, const ConvDims &d, hipStream_t st,
              int *rc) {
    using Geo = StemGeo<3, 7, 7, kStemPitch>;
    if (d.C != 3 || d.R != 7 || d.S != 7) return false;
    // Whole rows of 64..112 pixels, stride 1 or 2 (every lane's halo columns,
    // 16*kStemF of them, then fit the row pitch).
    if (d.OW < 64 || d.OW > 16 * kStemF || d.st > 2) return false;
    if ((int64_t)d.CHW * 4 >= (int64_t)kMaxBufBytes ||
        (int64_t)d.K * d.CRS * 4 >= (int64_t)kMaxBufBytes)
        return false;
    const int64_t co_blocks = cdiv(d.K, 64);
    // About one block per CU: rows per block, even (two groups).
    int64_t rb = std::max<int64_t>(2, cdiv(co_blocks * d.N * d.OH, kMinDirectBlocks));
    rb += rb & 1;
    const int64_t blocks_img = cdiv(d.OH, rb);
    const int64_t blocks = co_blocks * d.N * blocks_img;
    if (blocks > kI32Max) return false;
    StemArgs a;
    a.x = x;
    a.w = w;
    a.y = y;
    a.N = d.N;
    a.C = d.C;
    a.H = d.H;
    a.W = d.W;
    a.K = d.K;
    a.OH = d.OH;
    a.OW = d.OW;
    a.st = d.st;
    a.pad = d.pad;
    a.x_img = d.CHW;
    a.y_img = d.KOHW;
    a.rows_per_block = (int)rb;
    a.blocks_img = (int)blocks_img;
    a.co_blocks = (int)co_blocks;
    a.ncols = (d.OW - 1) * d.st + d.S;
    a.w_bytes = (uint32_t)((int64_t)d.K * d.CRS * 4);
    *rc = d.st == 2 ? stem_fwd_launch<2>(a, (unsigned)blocks, st)
                    : stem_fwd_launch<1>(a, (unsigned)blocks, st);
    return true;
}

// ---------------------------------------------------------------------------
// Few-channel layers on the vector ALUs (tiny.hpp).

// Output-channel bucket of the forward, and the row kernels' LDS: the
// transposed filter plus the forward's input rows, or dX's G rows.
int tiny_kb(const ConvDims &d) { return d.K <= 4 ? 4 : d.K <= 8 ? 8 : 16; }
int64_t tiny_xw(const ConvDims &d) { return (int64_t)(d.OW - 1) * d.st + d.S; }
int64_t tiny_fwd_lds(const ConvDims &d) {
    return (((int64_t)d.CRS * tiny_kb(d) + 3) / 4 * 4 + (int64_t)d.C * d.R * tiny_xw(d)) * 4;
}
int64_t tiny_dx_lds(const ConvDims &d) {
    return ((int64_t)d.K * d.RS * 4 + (int64_t)d.K * d.R * d.OW) * 4;
}

// The row kernels (tiny_*_kernel): any filter up to 32 x 8, any stride.
bool tiny_rows_ok(const ConvDims &d) {
    return d.C <= kTinyC && d.K <= kTinyK && (int64_t)d.K * d.CRS <= kTinyW && d.S <= 8 &&
           d.R <= 32 && (int64_t)d.CHW * 4 < (int64_t)kMaxBufBytes &&
           (int64_t)d.KOHW * 4 < (int64_t)kMaxBufBytes &&
           tiny_fwd_lds(d) <= 65536 && tiny_dx_lds(d) <= 65536 &&
           (int64_t)d.N * std::max(d.OH, d.H) <= kI32Max;
}
bool tiny3_ok(const ConvDims &d);
// Few-channel layers: the register forms where they apply, else the row kernels.
bool tiny_ok(const ConvDims &d) { return tiny3_ok(d) || tiny_rows_ok(d); }

// The register forms (tiny3_*): 3x3 filters, stride 1 or 2, output rows of at
// least 4 pixels (the dW walk wraps a row at most once per step).  Their
// grids are (images x pixel parts [x channels]), kept in 32 bits.
#ifndef KATSU_TINY3_KG
#define KATSU_TINY3_KG 4  // forward outputs per thread
#endif
#ifndef KATSU_TINY3_STEPS
#define KATSU_TINY3_STEPS 16  // dW MFMA k-steps (4 pixels each) per wave and tile
#endif
#ifndef KATSU_TINY3_DW_BLOCKS
#define KATSU_TINY3_DW_BLOCKS 512  // at most this many dW partials
#endif
constexpr size_t kTiny3DwLds = 4 * 3 * 64 * 4 * sizeof(float);  // 4 waves x NF <= 3 tiles
int tiny3_nf(const ConvDims &d) { return (int)cdiv((int64_t)d.C * 9, 16); }
bool tiny3_ok(const ConvDims &d) {
    return d.C <= kTinyC && d.K <= kTinyK && d.R == 3 && d.S == 3 && (d.st == 1 || d.st == 2) &&
           d.OW >= 4 &&
           (int64_t)d.CHW * 4 < (int64_t)kMaxBufBytes &&
           (int64_t)d.KOHW * 4 < (int64_t)kMaxBufBytes &&
           (int64_t)d.N * cdiv((int64_t)d.H * d.W, 256) * d.C <= kI32Max &&
           (int64_t)d.N * cdiv((int64_t)d.OH * d.OW, 256) <= kI32Max;
}
int64_t tiny3_dw_pb(const ConvDims &d) {
    return cdiv((int64_t)d.OH * d.OW, 16 * KATSU_TINY3_STEPS);
}
int64_t tiny3_dw_blocks(const ConvDims &d) {
    return std::min<int64_t>((int64_t)d.N * tiny3_dw_pb(d), KATSU_TINY3_DW_BLOCKS);
}

TinyArgs tiny_args(const ConvDims &d) {
    TinyArgs a{};
    a.N = d.N;
    a.C = d.C;
    a.H = d.H;
    a.W = d.W;
    a.K = d.K;
    a.R = d.R;
    a.S = d.S;
    a.OH = d.OH;
    a.OW = d.OW;
    a.st = d.st;
    a.pad = d.pad;
    return a;
}

template <int KG>
int tiny3_fwd_launch(const TinyArgs &a, const float *w, const ConvDims &d, hipStream_t st) {
    const int64_t pb = cdiv((int64_t)d.OH * d.OW, 256);
    tiny3_fwd_kernel<KG><<<dim3((unsigned)(d.N * pb), (unsigned)cdiv(d.K, KG)), dim3(256), 0,
                           st>>>(a, w, (int)pb);
    return launch_status();
}

int tiny_fwd(const float *x, const float *w, float *y, const ConvDims &d, hipStream_t st) {
    TinyArgs a = tiny_args(d);
    a.x = x;
    a.w = w;
    a.out = y;
    if (tiny3_ok(d)) {
        const int kg = std::min(KATSU_TINY3_KG, d.K);
        return kg >= 4 ? tiny3_fwd_launch<4>(a, w, d, st)
               : kg >= 2 ? tiny3_fwd_launch<2>(a, w, d, st)
                         : tiny3_fwd_launch<1>(a, w, d, st);
    }
    a.xw = (int)tiny_xw(d);
    const dim3 grid((unsigned)((int64_t)d.N * d.OH));
    const size_t lds = (size_t)tiny_fwd_lds(d);
    switch (tiny_kb(d)) {
        case 4: tiny_fwd_kernel<4><<<grid, dim3(256), lds, st>>>(a, w); break;
        case 8: tiny_fwd_kernel<8><<<grid, dim3(256), lds, st>>>(a, w); break;
        default: tiny_fwd_kernel<16><<<grid, dim3(256), lds, st>>>(a, w); break;
    }
    return launch_status();
}

// dX register form: KB output channels summed per thread (the K bucket),
// stride 1 or 2; ndx blocks of pixel parts pb, or 0 when it does not apply.
template <int ST>
int tiny3_dx_launch_st(const TinyArgs &a, const float *w, const ConvDims &d, hipStream_t st) {
    const int64_t pb = cdiv((int64_t)d.H * d.W, 256);
    const dim3 grid((unsigned)((KATSU_TINY3_DX_ALLC ? 1 : d.C) * d.N * pb));
    switch (tiny_kb(d)) {
        case 4: tiny3_dx_kernel<4, ST><<<grid, dim3(256), 0, st>>>(a, w, (int)pb); break;
        case 8: tiny3_dx_kernel<8, ST><<<grid, dim3(256), 0, st>>>(a, w, (int)pb); break;
        default: tiny3_dx_kernel<16, ST><<<grid, dim3(256), 0, st>>>(a, w, (int)pb); break;
    }
    return launch_status();
}

int tiny_dx(const float *gy, const float *w, float *dx, const ConvDims &d, float beta,
            hipStream_t st) {
    TinyArgs a = tiny_args(d);
    a.g = gy;
    a.w = w;
    a.out = dx;
    a.beta = beta;
    if (tiny3_ok(d))
        return d.st == 1 ? tiny3_dx_launch_st<1>(a, w, d, st) : tiny3_dx_launch_st<2>(a, w, d, st);
    tiny_dx_kernel<<<dim3((unsigned)((int64_t)d.N * d.H)), dim3(256), (size_t)tiny_dx_lds(d),
                     st>>>(a, w);
    return launch_status();
}

// Both register-form passes in one launch: the dX blocks (channel x image x
// pixel part), then the dW partial blocks.
template <int KB, int ST, int NF>
int tiny3_bwd_launch_t(const TinyArgs &a, const float *w, const ConvDims &d, int64_t dwblocks,
                       size_t lds, hipStream_t st) {
    const int64_t pbx = cdiv((int64_t)d.H * d.W, 256);
    const int64_t ndx = (int64_t)(KATSU_TINY3_DX_ALLC ? 1 : d.C) * d.N * pbx;
    if (ndx + dwblocks > kI32Max) return KATSU_E_INVALID;
    tiny3_bwd_kernel<KB, ST, NF, KATSU_TINY3_STEPS>
        <<<dim3((unsigned)(ndx + dwblocks)), dim3(256), lds, st>>>(a, w, (int)ndx, (int)pbx,
                                                                  (int)tiny3_dw_pb(d));
    return launch_status();
}

template <int KB, int ST>
int tiny3_bwd_launch_kb(const TinyArgs &a, const float *w, const ConvDims &d, int64_t dwblocks,
                        size_t lds, hipStream_t st) {
    switch (tiny3_nf(d)) {
        case 1: return tiny3_bwd_launch_t<KB, ST, 1>(a, w, d, dwblocks, lds, st);
        case 2: return tiny3_bwd_launch_t<KB, ST, 2>(a, w, d, dwblocks, lds, st);
        default: return tiny3_bwd_launch_t<KB, ST, 3>(a, w, d, dwblocks, lds, st);
    }
}

template <int ST>
int tiny3_bwd_launch_st(const TinyArgs &a, const float *w, const ConvDims &d, int64_t dwblocks,
                        size_t lds, hipStream_t st) {
    switch (tiny_kb(d)) {
        case 4: return tiny3_bwd_launch_kb<4, ST>(a, w, d, dwblocks, lds, st);
        case 8: return tiny3_bwd_launch_kb<8, ST>(a, w, d, dwblocks, lds, st);
        default: return tiny3_bwd_launch_kb<16, ST>(a, w, d, dwblocks, lds, st);
    }
}

// dW: one partial per block of output rows, about one block per CU.
struct TinyDwPlan {
    bool ok = false;
    int64_t blocks = 0, rows_per_block = 0, pstride = 0, xw = 0;
    size_t lds = 0, ws_bytes = 0;
};

TinyDwPlan tiny_dw_plan(const ConvDims &d) {
    TinyDwPlan pl;
    if (!tiny_ok(d)) return pl;
    const int64_t rows = (int64_t)d.N * d.OH;
    const int64_t xw = (int64_t)(d.OW - 1) * d.st + d.S;
    const int64_t lds = ((int64_t)d.K * d.OW + (int64_t)d.C * d.R * xw) * 4;
    pl.pstride = ((int64_t)d.K * d.CRS + 3) / 4 * 4;
    if (rows <= 0) return pl;
    if (tiny3_ok(d)) {
        pl.blocks = tiny3_dw_blocks(d);
        pl.lds = kTiny3DwLds;
        pl.ws_bytes = (size_t)pl.blocks * (size_t)pl.pstride * sizeof(float);
        pl.ok = true;
        return pl;
    }
    if (lds > 65536) return pl;
    pl.rows_per_block = cdiv(rows, kMinDirectBlocks);
    pl.blocks = cdiv(rows, pl.rows_per_block);
    pl.xw = xw;
    pl.lds = (size_t)lds;
    pl.ws_bytes = (size_t)pl.blocks * (size_t)pl.pstride * sizeof(float);
    pl.ok = true;
    return pl;
}

int tiny_dw(const float *x, const float *gy, float *dw, const ConvDims &d, const TinyDwPlan &pl,
            float beta, float *ws, hipStream_t st) {
    TinyArgs a = tiny_args(d);
    a.x = x;
    a.g = gy;
    a.out2 = ws;
    a.rows_per_block = (int)pl.rows_per_block;
    a.xw = (int)pl.xw;
    a.pstride = pl.pstride;
    if (tiny3_ok(d)) {
        const int pb = (int)tiny3_dw_pb(d);
        const dim3 grid((unsigned)pl.blocks);
        switch (tiny3_nf(d)) {
            case 1:
                tiny3_dw_kernel<1, KATSU_TINY3_STEPS><<<grid, dim3(256), pl.lds, st>>>(a, pb);
                break;
            case 2:
                tiny3_dw_kernel<2, KATSU_TINY3_STEPS><<<grid, dim3(256), pl.lds, st>>>(a, pb);
                break;
            default:
                tiny3_dw_kernel<3, KATSU_TINY3_STEPS><<<grid, dim3(256), pl.lds, st>>>(a, pb);
                break;
        }
    } else {
        tiny_dw_kernel<<<dim3((unsigned)pl.blocks), dim3(256), pl.lds, st>>>(a);
    }
    const int rc = launch_status();
    if (rc != KATSU_OK) return rc;
    return launch_split_reduce(ws, dw, (int64_t)d.K * d.CRS, pl.pstride, (int)pl.blocks, beta,
                               st);
}

int tiny3_bwd_launch(const TinyArgs &a, const float *w, const ConvDims &d, const TinyDwPlan &pl,
                     hipStream_t st) {
    return d.st == 1 ? tiny3_bwd_launch_st<1>(a, w, d, pl.blocks, pl.lds, st)
                     : tiny3_bwd_launch_st<2>(a, w, d, pl.blocks, pl.lds, st);
}

// ---------------------------------------------------------------------------
// Forward.

template <class C>
int fwd_cfg(const float *x, const float *w, float *y, const ConvDims &d, hipStream_t st) {
    FwdProb p;
    p.a = {w, d.CRS, 1, d.K};
    FwdColView &b = p.b;
    b.x = x;
    b.H = d.H;
    b.W = d.W;
    b.HW = d.HW;
    b.S = d.S;
    b.RS = d.RS;
    b.OW = d.OW;
    b.OHW = d.OHW;
    b.npix = (int)d.npix_out;
    b.stride = d.st;
    b.pad = d.pad;
    b.chw = d.CHW;
    b.fd_ohw = fdiv(d.OHW);
    b.fd_ow = fdiv(d.OW);
    b.fd_rs = fdiv(d.RS);
    b.fd_s = fdiv(d.S);
    FwdEpi &e = p.c;
    e.y = y;
    e.K = d.K;
    e.OHW = d.OHW;
    e.npix = (int)d.npix_out;
    e.kohw = (int64_t)d.KOHW;
    e.fd_ohw = fdiv(d.OHW);
    e.x = x;
    e.w = w;
    e.C = d.C;
    e.H = d.H;
    e.W = d.W;
    e.R = d.R;
    e.S = d.S;
    e.OW = d.OW;
    e.stride = d.st;
    e.pad = d.pad;
    e.chw = d.CHW;
    p.CRS = d.CRS;
    p.tiles_m = (int)cdiv(d.K, C::BM);
    const int64_t tiles_n = cdiv(d.npix_out, C::BN);
    return run<C>(p, tiles_n * p.tiles_m, st);
}

int conv_fwd_dev(const float *x, const float *w, float *y, const katsu_conv_geom *g,
                 hipStream_t st) {
    ConvDims d;
    if (conv_dims(g, &d) != KATSU_OK) return KATSU_E_INVALID;
    if (d.npix_out == 0) return KATSU_OK;
    if (!x || !w || !y) return KATSU_E_INVALID;
    {
        DirectFwdProblem P{x, w, y, d.N, d.C, d.H, d.W, d.K, d.R, d.S, d.st, d.pad, d.pad,
                           d.OH, d.OW, 0.f};
        int rc = KATSU_OK;
        if (direct_fwd<0>(P, st, &rc)) return rc;
        if (stem_fwd(x, w, y, d, st, &rc)) return rc;
    }
    if (pw_ok(d)) return pw_fwd(x, w, y, d, st);
    if (tiny_ok(d)) return tiny_fwd(x, w, y, d, st);
    // The largest tile that still gives every CU a block (rows x pixels).
    const int64_t px = d.npix_out;
    if (d.K <= 16) return fwd_cfg<CfgS>(x, w, y, d, st);
    if (d.K > 64 && cdiv(d.K, 128) * cdiv(px, 128) >= kMinDirectBlocks)
        return fwd_cfg<CfgL>(x, w, y, d, st);
    if (cdiv(d.K, 64) * cdiv(px, 128) >= kMinDirectBlocks) return fwd_cfg<CfgM>(x, w, y, d, st);
    if (cdiv(d.K, 64) * cdiv(px, 64) >= kMinDirectBlocks) return fwd_cfg<Cfg64>(x, w, y, d, st);
    return fwd_cfg<Cfg32>(x, w, y, d, st);
}

// ---------------------------------------------------------------------------
// Backward data.

template <class C>
int dx_cfg(const float *gy, const float *w, float *dx, const ConvDims &d, float beta,
           hipStream_t st) {
    DxProb p;
    std::memset(&p, 0, sizeof(p));
    DxWView &a = p.a;
    a.w = w;
    a.C = d.C;
    a.RS = d.RS;
    a.S = d.S;
    a.CRS = d.CRS;
    a.stride = d.st;
    DxColView &b = p.b;
    b.g = gy;
    b.OH = d.OH;
    b.OW = d.OW;
    b.OHW = d.OHW;
    b.kohw = d.KOHW;
    DxEpi &e = p.c;
    e.dx = dx;
    e.C = d.C;
    e.HW = d.HW;
    e.W = d.W;
    e.stride = d.st;
    e.chw = d.CHW;
    e.beta = beta;
    e.g = gy;
    e.w = w;
    e.K = d.K;
    e.OH = d.OH;
    e.OW = d.OW;
    e.R = d.R;
    e.S = d.S;
    e.pad = d.pad;
    e.kohw = d.KOHW;
    p.tiles_m = (int)cdiv(d.C, C::BM);

    // Enumerate the stride phases; launch at most kMaxPhases per kernel.
    const int st2 = d.st * d.st;
    int rc = KATSU_OK;
    int64_t tiles = 0;
    p.nphases = 0;
    for (int q = 0; q < st2 && rc == KATSU_OK; ++q) {
        const int py = q / d.st, px = q % d.st;
        DxPhase P;
        P.py = py;
        P.px = px;
        P.Ha = py < d.H ? (d.H - py + d.st - 1) / d.st : 0;
        P.Wa = px < d.W ? (d.W - px + d.st - 1) / d.st : 0;
        P.r0 = (int)(((int64_t)py + d.pad) % d.st);
        P.s0 = (int)(((int64_t)px + d.pad) % d.st);
        P.dy = (int)(((int64_t)py + d.pad - P.r0) / d.st);
        P.dx = (int)(((int64_t)px + d.pad - P.s0) / d.st);
        P.Ru = P.r0 < d.R ? (d.R - P.r0 + d.st - 1) / d.st : 0;
        P.Su = P.s0 < d.S ? (d.S - P.s0 + d.st - 1) / d.st : 0;
        const int64_t npix = (int64_t)d.N * P.Ha * P.Wa;
        if (npix == 0) continue;
        P.npix = (int)npix;
        P.kred = d.K * P.Ru * P.Su;
        P.tiles_n = (int)cdiv(npix, C::BN);
        P.fd_hawa = fdiv((int64_t)P.Ha * P.Wa);
        P.fd_wa = fdiv(P.Wa);
        P.fd_rusu = fdiv((int64_t)P.Ru * P.Su);
        P.fd_su = fdiv(P.Su);
        P.tile_begin = (int)tiles;
        p.ph[p.nphases++] = P;
        tiles += (int64_t)P.tiles_n * p.tiles_m;
        if (tiles > kI32Max) return KATSU_E_INVALID;
        if (p.nphases == kMaxPhases || q == st2 - 1) {
            rc = run<C>(p, tiles, st);
            p.nphases = 0;
            tiles = 0;
        }
    }
    if (rc == KATSU_OK && p.nphases > 0) rc = run<C>(p, tiles, st);
    return rc;
}

// The stem's data gradient by rolling rows (stemdx.hpp): 3 input channels,
// 64 output channels, 7x7, stride 2, padding 3.  Bands of `rows` flattened
// super-rows per column tile, about one wave per SIMD; one block per CU (its
// LDS request keeps a second block off the CU, so the waves spread over all
// SIMDs).
#ifndef KATSU_STEM_DX
#define KATSU_STEM_DX 1
#endif
#ifndef KATSU_STEM_DX_XCD_WAVES
#define KATSU_STEM_DX_XCD_WAVES 128
#endif
#ifndef KATSU_STEM_DX_PF
#define KATSU_STEM_DX_PF 8
#endif
#ifndef KATSU_STEM_DX_LDS
#define KATSU_STEM_DX_LDS 98304
#endif
#ifndef KATSU_STEM_DX_OCC
#define KATSU_STEM_DX_OCC 1
#endif
bool stem_dx(const ConvDims &d, const float *gy, const float *w, float *dx, float beta,
             hipStream_t st, int *rc) {
    if (!KATSU_STEM_DX || d.C != kStemDxC || d.K != kStemDxK || d.R != 7 || d.S != 7 ||
        d.st != 2 || d.pad != 3)
        return false;
    const int64_t g_bytes = d.npix_out * d.K * 4, dx_bytes = d.npix_in * d.C * 4;
    if (g_bytes >= (int64_t)kMaxBufBytes || dx_bytes >= (int64_t)kMaxBufBytes) return false;
    StemDxArgs a;
    a.g = gy;
    a.w = w;
    a.dx = dx;
    a.N = (int)d.N;
    a.H = (int)d.H;
    a.W = (int)d.W;
    a.OH = (int)d.OH;
    a.OW = (int)d.OW;
    a.tiles = (int)cdiv(d.OW, 16);
    const int64_t total = (int64_t)d.N * d.OH;
    // At most KATSU_STEM_DX_XCD_WAVES waves (one per SIMD) on each of the 8
    // XCDs, each XCD holding whole bands.
    const int64_t bands_max = 8 * std::max<int64_t>(1, KATSU_STEM_DX_XCD_WAVES / a.tiles);
    a.rows = (int)cdiv(total, bands_max);
    a.bands = (int)cdiv(total, a.rows);
    a.wpx = (int)cdiv(a.bands, 8) * a.tiles;
    a.g_bytes = (uint32_t)g_bytes;
    a.dx_bytes = (uint32_t)dx_bytes;
    a.beta = beta;
    const int64_t blocks = 8 * cdiv(a.wpx, 4);
    constexpr auto kern = stem_dx_kernel<KATSU_STEM_DX_PF, KATSU_STEM_DX_OCC>;
    constexpr size_t lds = std::max<size_t>(KATSU_STEM_DX_LDS, 3 * 16 * 4 * 64 * sizeof(float));
    if ((*rc = lds_optin<kern>(lds)) != KATSU_OK) return true;
    kern<<<dim3((unsigned)blocks), dim3(256), lds, st>>>(a);
    *rc = launch_status();
    return true;
}

int conv_bwd_data_dev(const float *gy, const float *w, float *dx, const katsu_conv_geom *g,
                      float beta, hipStream_t st) {
    if (!beta_ok(beta)) return KATSU_E_INVALID;
    ConvDims d;
    if (conv_dims(g, &d) != KATSU_OK) return KATSU_E_INVALID;
    if (d.npix_in == 0) return KATSU_OK;
    if (!gy || !w || !dx) return KATSU_E_INVALID;
    DirectFwdProblem P;
    int rc = KATSU_OK;
    if (dx_as_forward(d, gy, w, dx, beta, &P) && direct_fwd<1>(P, st, &rc)) return rc;
    if (dx_phases(d, gy, w, dx, beta, st, &rc)) return rc;
    if (stem_dx(d, gy, w, dx, beta, st, &rc)) return rc;
    if (dx_superpixel(d, gy, w, dx, beta, st, &rc)) return rc;
    if (pw_ok(d)) return pw_dx(gy, w, dx, d, beta, st);
    if (tiny_ok(d)) return tiny_dx(gy, w, dx, d, beta, st);
    if (d.C <= 16) return dx_cfg<CfgS>(gy, w, dx, d, beta, st);
    if (d.C <= 64) return dx_cfg<CfgM>(gy, w, dx, d, beta, st);
    return dx_cfg<CfgL>(gy, w, dx, d, beta, st);
}

// ---------------------------------------------------------------------------
// Backward filter.

// The stem's filter gradient (stem_dw_kernel): 3 channels, 7x7, stride 2.
struct StemDwPlan {
    bool ok = false;
    StemDwArgs a;
    int64_t blocks = 0;
    int splits = 0;
    size_t ws_bytes = 0;
};

StemDwPlan stem_dw_plan(const ConvDims &d) {
    StemDwPlan pl;
    using Geo = StemDwGeo<3, 7, 7>;
    if (d.C != 3 || d.R != 7 || d.S != 7 || d.st != 2) return pl;
    if ((int64_t)d.CHW * 4 >= (int64_t)kMaxBufBytes ||
        (int64_t)d.KOHW * 4 >= (int64_t)kMaxBufBytes)
        return pl;
    const int64_t tiles_row = cdiv(d.OW, Geo::TW);
    const int64_t tiles_total = (int64_t)d.N * d.OH * tiles_row;
    if (tiles_total > kI32Max) return pl;
    const int64_t co_blocks = cdiv(d.K, 64);
    // About two blocks per CU, each with an equal share of the tiles.
    int64_t splits = std::max<int64_t>(1, 2 * kMinDirectBlocks / co_blocks);
    const int64_t tpb = cdiv(tiles_total, splits);
    splits = cdiv(tiles_total, tpb);
    StemDwArgs &a = pl.a;
    a.x = nullptr;
    a.g = nullptr;
    a.part = nullptr;
    a.N = d.N;
    a.C = d.C;
    a.H = d.H;
    a.W = d.W;
    a.K = d.K;
    a.OH = d.OH;
    a.OW = d.OW;
    a.pad = d.pad;
    a.x_img = d.CHW;
    a.g_img = d.KOHW;
    a.tiles_row = (int)tiles_row;
    a.tiles_total = (int)tiles_total;
    a.tiles_per_block = (int)tpb;
    a.co_blocks = (int)co_blocks;
    a.pstride = ((int64_t)d.K * d.CRS + 3) / 4 * 4;
    pl.ok = true;
    pl.splits = (int)splits;
    pl.blocks = co_blocks * splits;
    pl.ws_bytes = (size_t)splits * (size_t)a.pstride * sizeof(float);
    return pl;
}

int stem_dw_launch(StemDwPlan pl, const float *x, const float *gy, float *dw, float beta,
                   float *ws, hipStream_t st) {
    using Geo = StemDwGeo<3, 7, 7>;
    pl.a.x = x;
    pl.a.g = gy;
    pl.a.part = ws;
    constexpr auto kern = stem_dw_kernel<3, 7, 7, 2>;
    int rc = lds_optin<kern>(Geo::kBytes);
    if (rc != KATSU_OK) return rc;
    kern<<<dim3((unsigned)pl.blocks), dim3(256), Geo::kBytes, st>>>(pl.a);
    if ((rc = launch_status()) != KATSU_OK) return rc;
    return launch_split_reduce(ws, dw, (int64_t)pl.a.K * 147, pl.a.pstride, pl.splits, beta, st);
}

struct DwPlan {
    int tiles_m, tiles_n, splits, kchunk;
    int64_t pstride;  // floats between partials (a multiple of 4)
    size_t ws_bytes;
    DirectDwPlan direct;  // used when direct.ok
    PwDwPlan pw;          // used when pw.ok (1x1, no padding)
    StemDwPlan stem;      // used when stem.ok
    TinyDwPlan tiny;      // used when tiny.ok
};

template <class C>
DwPlan dw_plan(const ConvDims &d) {
    DwPlan pl;
    pl.tiles_m = (int)cdiv(d.K, C::BM);
    pl.tiles_n = (int)cdiv(d.CRS, C::BN);
    const int64_t tiles = (int64_t)pl.tiles_m * pl.tiles_n;
    const int64_t npix = d.npix_out;
    // Aim for ~4 workgroups per CU (256 CUs) but keep every split at least
    // 8 k-tiles long so the partial traffic stays small next to the GEMM.
    const int64_t target = 1024;
    int64_t splits = std::max<int64_t>(1, cdiv(target, tiles));
    splits = std::min<int64_t>(splits, std::max<int64_t>(1, npix / (8 * C::BK)));
    int64_t kchunk = cdiv(cdiv(npix, splits), C::BK) * C::BK;
    if (kchunk <= 0) kchunk = C::BK;
    splits = std::max<int64_t>(1, cdiv(npix, kchunk));
    pl.splits = (int)splits;
    pl.kchunk = (int)kchunk;
    pl.pstride = ((int64_t)d.K * d.CRS + 3) / 4 * 4;
    pl.ws_bytes = splits > 1 ? (size_t)splits * (size_t)pl.pstride * sizeof(float) : 0;
    return pl;
}

DwPlan dw_plan_any(const ConvDims &d) {
    DirectDwPlan dp = direct_dw_plan_any(d);
    if (dp.ok) {
        DwPlan pl{};
        pl.ws_bytes = dp.ws_bytes;
        pl.direct = dp;
        return pl;
    }
    const PwDwPlan pp = pw_dw_plan(d);
    if (pp.ok) {
        DwPlan pl{};
        pl.ws_bytes = pp.ws_bytes;
        pl.pw = pp;
        return pl;
    }
    const StemDwPlan sp = stem_dw_plan(d);
    if (sp.ok) {
        DwPlan pl{};
        pl.ws_bytes = sp.ws_bytes;
        pl.stem = sp;
        return pl;
    }
    const TinyDwPlan tp = tiny_dw_plan(d);
    if (tp.ok) {
        DwPlan pl{};
        pl.ws_bytes = tp.ws_bytes;
        pl.tiny = tp;
        return pl;
    }
    return dw_plan<CfgW>(d);
}

template <class C>
int dw_cfg(const float *x, const float *gy, float *dw, const ConvDims &d, float beta,
           float *ws, hipStream_t st) {
    const DwPlan pl = dw_plan<C>(d);
    DwProb p;
    DwGView &a = p.a;
    a.g = gy;
    a.K = d.K;
    a.OHW = d.OHW;
    a.kohw = d.KOHW;
    a.fd_ohw = fdiv(d.OHW);
    DwColView &b = p.b;
    b.x = x;
    b.H = d.H;
    b.W = d.W;
    b.HW = d.HW;
    b.S = d.S;
    b.RS = d.RS;
    b.CRS = d.CRS;
    b.OW = d.OW;
    b.OHW = d.OHW;
    b.stride = d.st;
    b.pad = d.pad;
    b.chw = d.CHW;
    b.fd_rs = fdiv(d.RS);
    b.fd_s = fdiv(d.S);
    b.fd_ohw = fdiv(d.OHW);
    b.fd_ow = fdiv(d.OW);
    const bool direct = pl.splits == 1;
    p.c.out = direct ? dw : ws;
    p.c.K = d.K;
    p.c.CRS = d.CRS;
    p.c.split_stride = direct ? 0 : pl.pstride;
    p.c.beta = direct ? beta : 0.f;
    p.c.split = 0;
    p.c.x = x;
    p.c.g = gy;
    p.c.C = d.C;
    p.c.H = d.H;
    p.c.W = d.W;
    p.c.OH = d.OH;
    p.c.OW = d.OW;
    p.c.R = d.R;
    p.c.S = d.S;
    p.c.stride = d.st;
    p.c.pad = d.pad;
    p.tiles_m = pl.tiles_m;
    p.tiles_n = pl.tiles_n;
    p.splits = pl.splits;
    p.kchunk = pl.kchunk;
    p.npix = (int)d.npix_out;
    int rc = run<C>(p, (int64_t)pl.tiles_m * pl.tiles_n * pl.splits, st);
    if (rc != KATSU_OK || direct) return rc;
    return launch_split_reduce(ws, dw, (int64_t)d.K * d.CRS, pl.pstride, pl.splits, beta, st);
}

int conv_bwd_filter_dev(const float *x, const float *gy, float *dw, const katsu_conv_geom *g,
                        float beta, const WsSource &src, hipStream_t st) {
    if (!beta_ok(beta)) return KATSU_E_INVALID;
    ConvDims d;
    if (conv_dims(g, &d) != KATSU_OK) return KATSU_E_INVALID;
    if (!dw) return KATSU_E_INVALID;
    if (d.npix_out == 0) return launch_scale(dw, (int64_t)d.K * d.CRS, beta, st);
    if (!x || !gy) return KATSU_E_INVALID;
    const DwPlan pl = dw_plan_any(d);
    float *wsp = nullptr;
    int rc = ws_take(src, pl.ws_bytes, st, &wsp);
    if (rc != KATSU_OK) return rc;
    if (pl.direct.ok) return direct_dw_launch(pl.direct, x, gy, dw, beta, wsp, st);
    if (pl.pw.ok) return pw_dw(x, gy, dw, d, pl.pw, beta, wsp, st);
    if (pl.stem.ok) return stem_dw_launch(pl.stem, x, gy, dw, beta, wsp, st);
    if (pl.tiny.ok) return tiny_dw(x, gy, dw, d, pl.tiny, beta, wsp, st);
    return dw_cfg<CfgW>(x, gy, dw, d, beta, wsp, st);
}

// The workspace that covers every path of the filter gradient and of the
// one-call backward for this geometry (what the workspace query reports).
size_t bwd_ws_bytes(const ConvDims &d) {
    if (d.npix_out == 0) return 0;
    size_t b = dw_plan_any(d).ws_bytes;
    if (tiny_ok(d)) {
        const TinyDwPlan tp = tiny_dw_plan(d);
        if (tp.ok) b = std::max(b, tp.ws_bytes);
    }
    return b;
}

#ifndef KATSU_FUSED_DW_TBDIV
#define KATSU_FUSED_DW_TBDIV 2
#endif

// Whether two buffers of na and nb floats share any byte.
bool overlap(const float *a, size_t na, const float *b, size_t nb) {
    if (!a || !b || na == 0 || nb == 0) return false;
    const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
    return a0 < b0 + nb * sizeof(float) && b0 < a0 + na * sizeof(float);
}

// Both backward passes (backward_buffers, conv2d.rs:265-292).  When dX and
// dW both take their direct kernels they run as one launch; otherwise dX then
// dW, as two.  dx and dw either do not overlap or are the same buffer (an
// engine's pending buffer when input and weights are one node: the two
// passes then run one after the other, dX first).
int conv_bwd_dev(const float *x, const float *w, const float *gy, float *dx, float *dw,
                 const katsu_conv_geom *g, float beta, const WsSource &src, hipStream_t st) {
    if (!beta_ok(beta)) return KATSU_E_INVALID;
    ConvDims d;
    if (conv_dims(g, &d) != KATSU_OK) return KATSU_E_INVALID;
    if (!dw || (d.npix_in > 0 && !dx)) return KATSU_E_INVALID;
    const size_t nx = (size_t)d.npix_in * d.C, nw = (size_t)d.K * d.CRS;
    if (dx != dw && overlap(dx, nx, dw, nw)) return KATSU_E_INVALID;
    if (dx == dw && nx != nw) return KATSU_E_INVALID;
    DirectFwdProblem P;
    DirectFwdPlan xp;
    DwPlan wpl;
    const bool xplan =
        d.st == 2 ? dx_phases_plan(d, gy, w, dx, beta, &xp)
                  : dx_as_forward(d, gy, w, dx, beta, &P) && P.CO >= FwdV::KT &&
                        direct_fwd_plan<KATSU_FWD_VARIANT, 1>(P, &xp);
    const bool fused = dx != dw && d.npix_out > 0 && x && w && gy && xplan &&
                       (wpl = dw_plan_any(d)).direct.ok &&
                       dw_variant_fusable(wpl.direct.variant, d.st);
    if (!fused && dx != dw && d.npix_in > 0 && d.npix_out > 0 && x && w && gy && tiny_ok(d)) {
        // Few channels: dX rows and dW partials in one launch, then the reduce.
        const TinyDwPlan tp = tiny_dw_plan(d);
        if (tp.ok) {
            float *wsp = nullptr;
            int rc = ws_take(src, tp.ws_bytes, st, &wsp);
            if (rc != KATSU_OK) return rc;
            TinyArgs a = tiny_args(d);
            a.x = x;
            a.g = gy;
            a.out = dx;
            a.out2 = wsp;
            a.beta = beta;
            a.rows_per_block = (int)tp.rows_per_block;
            a.xw = (int)tp.xw;
            a.pstride = tp.pstride;
            if (tiny3_ok(d)) {
                rc = tiny3_bwd_launch(a, w, d, tp, st);
            } else {
                const int64_t ndx = (int64_t)d.N * d.H;
                const size_t lds = std::max((size_t)tiny_dx_lds(d), tp.lds);
                tiny_bwd_kernel<<<dim3((unsigned)(ndx + tp.blocks)), dim3(256), lds, st>>>(
                    a, w, (int)ndx);
                rc = launch_status();
            }
            if (rc != KATSU_OK) return rc;
            return launch_split_reduce(wsp, dw, (int64_t)d.K * d.CRS, tp.pstride, (int)tp.blocks,
                                       beta, st);
        }
    }
    if (!fused && dx != dw && d.npix_in > 0 && d.npix_out > 0 && x && w && gy && pw_ok(d)) {
        // 1x1: dX and the dW partials in one launch, then the reduce.
        const PwDwPlan pp = pw_dw_plan(d);
        if (pp.ok) {
            float *wsp = nullptr;
            int rc = ws_take(src, pp.ws_bytes, st, &wsp);
            if (rc != KATSU_OK) return rc;
            if (pw_bwd(x, w, gy, dx, dw, d, pp, beta, wsp, st, &rc)) return rc;
        }
    }
    if (!fused) {
        // One buffer for both: it receives beta*buf + dX + dW, dX added first.
        const int rc = conv_bwd_data_dev(gy, w, dx, g, beta, st);
        if (rc != KATSU_OK) return rc;
        return conv_bwd_filter_dev(x, gy, dw, g, dx == dw ? 1.f : beta, src, st);
    }
    // The shared launch takes the dW split with half the blocks: each dW
    // block then lasts about as long as two dX blocks, the dW blocks go
    // first, and half as many partials are written and summed.  The
    // workspace it needs is at most the standalone plan's, which the
    // workspace query reports.
    DirectDwPlan wp = direct_dw_plan_any(d, wpl.direct.variant, KATSU_FUSED_DW_TBDIV);
    if (!wp.ok || wp.ws_bytes > wpl.ws_bytes) wp = wpl.direct;
    float *wsp = nullptr;
    const int rc = ws_take(src, wp.ws_bytes, st, &wsp);
    if (rc != KATSU_OK) return rc;
    return bwd_fused_launch(xp, wp, x, gy, dw, beta, wsp, st);
}

// ---------------------------------------------------------------------------
// The allocation-free backward: its dW partials live in `scratch`, a
// file-scope device array of which every GPU holds its own copy.  In host
// code the array's name is only a stand-in, so its address on the current
// device is looked up once per device (hipGetSymbolAddress) and that
// pointer is what the kernels receive.  Every plan of this library needs at
// most 37.7 MB of partials (about 512 blocks of one 64 x 288 tile each),
// which the array covers.  Calls on one GPU share it: calls that overlap in
// time on that GPU race.  Nothing in it needs to start at zero (every
// partial element the reduce reads is written first).

constexpr size_t kStaticScratchBytes = (size_t)40 << 20;
constexpr int kMaxDevices = 64;

__device__ __align__(256) float scratch[kStaticScratchBytes / sizeof(float)];

struct StaticScratch {
    std::mutex mu;
    void *ptr[kMaxDevices] = {};
};

StaticScratch &static_scratch_state() {
    static StaticScratch s;
    return s;
}

// This device's copy of `scratch` (set up on the first call per device).
int static_scratch(void **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return KATSU_E_NODEVICE;
    }
    StaticScratch &s = static_scratch_state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (!s.ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            return e == hipSuccess ? KATSU_E_LAUNCH : map_hip(e);
        }
        s.ptr[dev] = p;
    }
    *out = s.ptr[dev];
    return KATSU_OK;
}

// ---------------------------------------------------------------------------
// Device engine: buffers and the elementwise kernels.

// Pool block sizes: 512-byte granules below 1 MiB, 2 MiB granules above.
size_t pool_round(size_t bytes) {
    const size_t g = bytes < (1u << 20) ? 512 : (2u << 20);
    return (std::max<size_t>(bytes, 1) + g - 1) / g * g;
}

int pool_alloc(State &s, size_t bytes, void **out) {
    const size_t want = pool_round(bytes);
    auto it = s.pool.free.lower_bound(want);
    if (it != s.pool.free.end() && it->first <= 2 * want) {
        *out = it->second;
        s.pool.live.emplace(it->second, it->first);
        s.pool.free.erase(it);
        return KATSU_OK;
    }
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
        // Return the cached blocks to HIP and try once more.
        (void)hipGetLastError();
        for (auto &kv : s.pool.free) (void)hipFree(kv.second);
        s.pool.free.clear();
        e = hipMalloc(&p, want);
        if (e != hipSuccess) return map_hip(e);
    }
    g_device_allocs.fetch_add(1, std::memory_order_relaxed);
    s.pool.live.emplace(p, want);
    *out = p;
    return KATSU_OK;
}

// Grid for a streaming kernel over n elements: enough blocks to cover the
// chip several times over, no more than the work needs.
unsigned ew_blocks(int64_t n) {
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(cdiv(n, 256), 256 * 16));
}

template <EwOp OP>
int ew_binary_launch(const float *a, const float *b, float *c, size_t n, float beta,
                     hipStream_t st) {
    if (!beta_ok(beta)) return KATSU_E_INVALID;
    if (n == 0) return KATSU_OK;
    if (!a || !b || !c) return KATSU_E_INVALID;
    const int64_t N = (int64_t)n;
    if (aligned16(a) && aligned16(b) && aligned16(c))
        ew_binary<OP, true><<<ew_blocks(cdiv(N, 4)), 256, 0, st>>>(a, b, c, N, beta);
    else
        ew_binary<OP, false><<<ew_blocks(N), 256, 0, st>>>(a, b, c, N, beta);
    return launch_status();
}

// ---------------------------------------------------------------------------
// Host-pointer wrappers: stage through the pool, run, copy back, synchronise.

int h2d(Buffer &b, const float *src, size_t count, hipStream_t st) {
    const size_t bytes = count * sizeof(float);
    int rc = ensure(b, bytes);
    if (rc != KATSU_OK) return rc;
    if (bytes == 0) return KATSU_OK;
    return map_hip(state().copy.h2d(b.ptr, src, bytes, st));
}

// Device to host after the work ordered on st, returning once dst holds it.
int d2h(float *dst, const Buffer &b, size_t count, hipStream_t st) {
    const size_t bytes = count * sizeof(float);
    return bytes ? map_hip(state().copy.d2h(dst, b.ptr, bytes, st)) : KATSU_OK;
}

// beta*C for an empty reduction on a host buffer (beta is 0 or 1).
int host_scale(float *c, size_t count, float beta) {
    if (beta == 0.f && count) std::memset(c, 0, count * sizeof(float));
    return KATSU_OK;
}

int d2h_sync(float *dst, const Buffer &b, size_t count, hipStream_t st) {
    const int rc = d2h(dst, b, count, st);
    return rc != KATSU_OK ? rc : map_hip(hipStreamSynchronize(st));
}

}  // namespace
}  // namespace katsu

using namespace katsu;

extern "C" {

const char *katsu_hip_version(void) { return "katsu-mi355x 0.1.0 (gfx950, fp32 MFMA)"; }

const char *katsu_hip_strerror(int status) {
    switch (status) {
        case KATSU_OK: return "ok";
        case KATSU_E_INVALID: return "invalid argument or shape";
        case KATSU_E_NODEVICE: return "no HIP device available";
        case KATSU_E_OOM: return "device allocation failed";
        case KATSU_E_LAUNCH: return "kernel launch, copy or synchronisation failed";
        case KATSU_E_SCRATCH:
            return "the problem needs more scratch than the allocation-free entry point holds";
        default: return "unknown katsu status";
    }
}

int katsu_hip_init(void) {
    State &s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    return init_locked(s);
}

void katsu_hip_shutdown(void) {
    State &s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (!s.ready) return;
    (void)hipStreamSynchronize(s.stream);
    s.copy.release();
    for (Buffer &b : s.staging) {
        if (b.ptr) (void)hipFree(b.ptr);
        b = Buffer{};
    }
    (void)hipDeviceSynchronize();  // scratch may be in use on other streams
    scratch_release_all();
    for (auto &kv : s.pool.free) (void)hipFree(kv.second);
    for (auto &kv : s.pool.live) (void)hipFree(kv.first);
    s.pool = Pool{};
    (void)hipStreamDestroy(s.stream);
    s.stream = nullptr;
    s.ready = false;
}

int katsu_hip_conv2d_geometry(katsu_conv_geom *g) { return geometry_fill(g); }

int katsu_hip_gemm_f32_dev(const float *a, const float *b, float *c, size_t m, size_t n,
                           size_t k, int trans_a, int trans_b, float beta, void *stream) {
    return gemm_dev(a, b, c, m, n, k, trans_a, trans_b, beta, (hipStream_t)stream);
}

int katsu_hip_matmul_vjp_f32_dev(const float *a, const float *b, const float *g, float *da,
                                 float *db, size_t m, size_t k, size_t n, float beta_a,
                                 float beta_b, void *stream) {
    return matmul_vjp_dev(a, b, g, da, db, m, k, n, beta_a, beta_b, (hipStream_t)stream);
}

int katsu_hip_gemm_f32(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                       int trans_a, int trans_b, float beta) {
    if (!beta_ok(beta) || (trans_a != 0 && trans_a != 1) || (trans_b != 0 && trans_b != 1))
        return KATSU_E_INVALID;
    if (m == 0 || n == 0) return KATSU_OK;
    if (!c || (k > 0 && (!a || !b))) return KATSU_E_INVALID;
    size_t mn, mk, kn;
    if (!mul_ok(m, n, (uint64_t *)&mn) || !mul_ok(m, k, (uint64_t *)&mk) ||
        !mul_ok(k, n, (uint64_t *)&kn))
        return KATSU_E_INVALID;
    // An empty reduction computes nothing: C = beta*C on the caller's buffer.
    if (k == 0) return host_scale(c, mn, beta);
    State &s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    int rc = init_locked(s);
    if (rc) return rc;
    if (k > 0) {
        if ((rc = h2d(s.staging[0], a, mk, s.stream))) return rc;
        if ((rc = h2d(s.staging[1], b, kn, s.stream))) return rc;
    }
    if (beta != 0.f) {
        if ((rc = h2d(s.staging[2], c, mn, s.stream))) return rc;
    } else if ((rc = ensure(s.staging[2], mn * sizeof(float)))) {
        return rc;
    }
    rc = gemm_dev((const float *)s.staging[0].ptr, (const float *)s.staging[1].ptr,
                  (float *)s.staging[2].ptr, m, n, k, trans_a, trans_b, beta, s.stream);
    if (rc) return rc;
    return d2h_sync(c, s.staging[2], mn, s.stream);
}

int katsu_hip_conv2d_fwd_f32_dev(const float *x, const float *w, float *y,
                                 const katsu_conv_geom *g, void *stream) {
    return conv_fwd_dev(x, w, y, g, (hipStream_t)stream);
}

int katsu_hip_conv2d_fwd_f32(const float *x, const float *w, float *y,
                             const katsu_conv_geom *g) {
    ConvDims d;
    if (conv_dims(g, &d) != KATSU_OK) return KATSU_E_INVALID;
    const size_t nx = (size_t)d.npix_in * d.C, nw = (size_t)d.K * d.CRS,
                 ny = (size_t)d.npix_out * d.K;
    if (ny == 0) return KATSU_OK;
    if (!x || !w || !y) return KATSU_E_INVALID;
    State &s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    int rc = init_locked(s);
    if (rc) return rc;
    if ((rc = h2d(s.staging[0], x, nx, s.stream))) return rc;
    if ((rc = h2d(s.staging[1], w, nw, s.stream))) return rc;
    if ((rc = ensure(s.staging[2], ny * sizeof(float)))) return rc;
    rc = conv_fwd_dev((const float *)s.staging[0].ptr, (const float *)s.staging[1].ptr,
                      (float *)s.staging[2].ptr, g, s.stream);
    if (rc) return rc;
    return d2h_sync(y, s.staging[2], ny, s.stream);
}

int katsu_hip_conv2d_bwd_data_f32_dev(const float *gy, const float *w, float *dx,
                                      const katsu_conv_geom *g, float beta, void *stream) {
    return conv_bwd_data_dev(gy, w, dx, g, beta, (hipStream_t)stream);
}

int katsu_hip_conv2d_bwd_data_f32(const float *gy, const float *w, float *dx,
                                  const katsu_conv_geom *g, float beta) {
    if (!beta_ok(beta)) return KATSU_E_INVALID;
    ConvDims d;
    if (conv_dims(g, &d) != KATSU_OK) return KATSU_E_INVALID;
    const size_t nx = (size_t)d.npix_in * d.C, nw = (size_t)d.K * d.CRS,
                 ny = (size_t)d.npix_out * d.K;
    if (nx == 0) return KATSU_OK;
    if (!gy || !w || !dx) return KATSU_E_INVALID;
    State &s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    int rc = init_locked(s);
    if (rc) return rc;
    if ((rc = h2d(s.staging[0], gy, ny, s.stream))) return rc;
    if ((rc = h2d(s.staging[1], w, nw, s.stream))) return rc;
    if (beta != 0.f) {
        if ((rc = h2d(s.staging[2], dx, nx, s.stream))) return rc;
    } else if ((rc = ensure(s.staging[2], nx * sizeof(float)))) {
        return rc;
    }
    rc = conv_bwd_data_dev((const float *)s.staging[0].ptr, (const float *)s.staging[1].ptr,
                           (float *)s.staging[2].ptr, g, beta, s.stream);
    if (rc) return rc;
    return d2h_sync(dx, s.staging[2], nx, s.stream);
}

int katsu_hip_conv2d_bwd_filter_workspace(const katsu_conv_geom *g, size_t *bytes) {
    if (!bytes) return KATSU_E_INVALID;
    ConvDims d;
    if (conv_dims(g, &d) != KATSU_OK) return KATSU_E_INVALID;
    *bytes = bwd_ws_bytes(d);
    return KATSU_OK;
}

int katsu_hip_conv2d_bwd_filter_f32_dev(const float *x, const float *gy, float *dw,
                                        const katsu_conv_geom *g, float beta, void *workspace,
                                        size_t workspace_bytes, void *stream) {
    return conv_bwd_filter_dev(x, gy, dw, g, beta, WsSource{workspace, workspace_bytes, true},
                               (hipStream_t)stream);
}

int katsu_hip_conv2d_bwd_f32_dev(const float *x, const float *w, const float *gy, float *dx,
                                 float *dw, const katsu_conv_geom *g, float beta, void *workspace,
                                 size_t workspace_bytes, void *stream) {
    return conv_bwd_dev(x, w, gy, dx, dw, g, beta, WsSource{workspace, workspace_bytes, true},
                        (hipStream_t)stream);
}

int katsu_hip_conv2d_bwd_f32_dev_noalloc(const float *x, const float *w, const float *gy,
                                         float *dx, float *dw, const katsu_conv_geom *g,
                                         float beta, void *stream) {
    if (!beta_ok(beta)) return KATSU_E_INVALID;
    ConvDims d;
    if (conv_dims(g, &d) != KATSU_OK) return KATSU_E_INVALID;
    if (bwd_ws_bytes(d) > kStaticScratchBytes) return KATSU_E_SCRATCH;
    void *ws = nullptr;
    const int rc = static_scratch(&ws);
    if (rc != KATSU_OK) return rc;
    return conv_bwd_dev(x, w, gy, dx, dw, g, beta, WsSource{ws, kStaticScratchBytes, false},
                        (hipStream_t)stream);
}

size_t katsu_hip_noalloc_scratch_bytes(void) { return kStaticScratchBytes; }

uint64_t katsu_hip_device_allocations(void) {
    return g_device_allocs.load(std::memory_order_relaxed);
}

int katsu_hip_conv2d_bwd_f32(const float *x, const float *w, const float *gy, float *dx,
                             float *dw, const katsu_conv_geom *g, float beta) {
    if (!beta_ok(beta)) return KATSU_E_INVALID;
    ConvDims d;
    if (conv_dims(g, &d) != KATSU_OK) return KATSU_E_INVALID;
    const size_t nx = (size_t)d.npix_in * d.C, nw = (size_t)d.K * d.CRS,
                 ny = (size_t)d.npix_out * d.K;
    if (!dw || (nx > 0 && !dx)) return KATSU_E_INVALID;
    if (ny > 0 && (!x || !w || !gy)) return KATSU_E_INVALID;
    // dx and dw: apart, or one buffer (one pending buffer for input and
    // weights that are one node), which is staged once so the device passes
    // see the aliasing and add dX before dW.
    const bool same = dx == dw;
    if ((same && nx != nw) || (!same && overlap(dx, nx, dw, nw))) return KATSU_E_INVALID;
    if (ny == 0) return host_scale(dw, nw, beta);  // empty batch: dx is empty, dw = beta*dw
    State &s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    int rc = init_locked(s);
    if (rc) return rc;
    if ((rc = h2d(s.staging[0], x, nx, s.stream))) return rc;
    if ((rc = h2d(s.staging[1], w, nw, s.stream))) return rc;
    if ((rc = h2d(s.staging[2], gy, ny, s.stream))) return rc;
    if (beta != 0.f) {
        if ((rc = h2d(s.staging[3], dx, nx, s.stream))) return rc;
        if (!same && (rc = h2d(s.staging[4], dw, nw, s.stream))) return rc;
    } else {
        if ((rc = ensure(s.staging[3], nx * sizeof(float)))) return rc;
        if (!same && (rc = ensure(s.staging[4], nw * sizeof(float)))) return rc;
    }
    float *ddx = (float *)s.staging[3].ptr;
    float *ddw = same ? ddx : (float *)s.staging[4].ptr;
    rc = conv_bwd_dev((const float *)s.staging[0].ptr, (const float *)s.staging[1].ptr,
                      (const float *)s.staging[2].ptr, ddx, ddw, g, beta,
                      WsSource{nullptr, 0, true}, s.stream);
    if (rc) return rc;
    if (same) return d2h_sync(dx, s.staging[3], nx, s.stream);
    if ((rc = d2h(dx, s.staging[3], nx, s.stream))) return rc;
    return d2h_sync(dw, s.staging[4], nw, s.stream);
}

int katsu_hip_conv2d_bwd_filter_f32(const float *x, const float *gy, float *dw,
                                    const katsu_conv_geom *g, float beta) {
    if (!beta_ok(beta)) return KATSU_E_INVALID;
    ConvDims d;
    if (conv_dims(g, &d) != KATSU_OK) return KATSU_E_INVALID;
    const size_t nx = (size_t)d.npix_in * d.C, nw = (size_t)d.K * d.CRS,
                 ny = (size_t)d.npix_out * d.K;
    if (!dw) return KATSU_E_INVALID;
    if (ny > 0 && (!x || !gy)) return KATSU_E_INVALID;
    if (ny == 0) return host_scale(dw, nw, beta);  // empty batch: dw = beta*dw
    State &s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    int rc = init_locked(s);
    if (rc) return rc;
    if ((rc = h2d(s.staging[0], x, nx, s.stream))) return rc;
    if ((rc = h2d(s.staging[1], gy, ny, s.stream))) return rc;
    if (beta != 0.f) {
        if ((rc = h2d(s.staging[2], dw, nw, s.stream))) return rc;
    } else if ((rc = ensure(s.staging[2], nw * sizeof(float)))) {
        return rc;
    }
    rc = conv_bwd_filter_dev((const float *)s.staging[0].ptr, (const float *)s.staging[1].ptr,
                             (float *)s.staging[2].ptr, g, beta, WsSource{nullptr, 0, true},
                             s.stream);
    if (rc) return rc;
    return d2h_sync(dw, s.staging[2], nw, s.stream);
}

void *katsu_hip_stream(void) {
    State &s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    return init_locked(s) == KATSU_OK ? (void *)s.stream : nullptr;
}

int katsu_hip_malloc(void **ptr, size_t bytes) {
    if (!ptr) return KATSU_E_INVALID;
    *ptr = nullptr;
    if (bytes == 0) return KATSU_OK;
    State &s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    int rc = init_locked(s);
    if (rc) return rc;
    return pool_alloc(s, bytes, ptr);
}

int katsu_hip_free(void *ptr) {
    if (!ptr) return KATSU_OK;
    State &s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    auto it = s.pool.live.find(ptr);
    if (it == s.pool.live.end()) return KATSU_E_INVALID;
    s.pool.free.emplace(it->second, it->first);
    s.pool.live.erase(it);
    return KATSU_OK;
}

int katsu_hip_upload(void *dst, const float *src, size_t count, void *stream) {
    if (count == 0) return KATSU_OK;
    if (!dst || !src) return KATSU_E_INVALID;
    hipStream_t st = (hipStream_t)stream;
    int rc = map_hip(hipMemcpyAsync(dst, src, count * sizeof(float), hipMemcpyHostToDevice, st));
    if (rc) return rc;
    return map_hip(hipStreamSynchronize(st));
}

int katsu_hip_download(float *dst, const void *src, size_t count, void *stream) {
    if (count == 0) return KATSU_OK;
    if (!dst || !src) return KATSU_E_INVALID;
    hipStream_t st = (hipStream_t)stream;
    int rc = map_hip(hipMemcpyAsync(dst, src, count * sizeof(float), hipMemcpyDeviceToHost, st));
    if (rc) return rc;
    return map_hip(hipStreamSynchronize(st));
}

int katsu_hip_sync(void *stream) { return map_hip(hipStreamSynchronize((hipStream_t)stream)); }

int katsu_hip_add_f32_dev(const float *a, const float *b, float *c, size_t n, float beta,
                          void *stream) {
    return ew_binary_launch<EwOp::Add>(a, b, c, n, beta, (hipStream_t)stream);
}

int katsu_hip_mul_f32_dev(const float *a, const float *b, float *c, size_t n, float beta,
                          void *stream) {
    return ew_binary_launch<EwOp::Mul>(a, b, c, n, beta, (hipStream_t)stream);
}

int katsu_hip_accumulate_f32_dev(const float *x, float *y, size_t n, float beta,
                                 void *stream) {
    if (!beta_ok(beta)) return KATSU_E_INVALID;
    if (n == 0) return KATSU_OK;
    if (!x || !y) return KATSU_E_INVALID;
    const int64_t N = (int64_t)n;
    if (aligned16(x) && aligned16(y))
        ew_accumulate<true><<<ew_blocks(cdiv(N, 4)), 256, 0, (hipStream_t)stream>>>(x, y, N, beta);
    else
        ew_accumulate<false><<<ew_blocks(N), 256, 0, (hipStream_t)stream>>>(x, y, N, beta);
    return launch_status();
}

int katsu_hip_fill_f32_dev(float *x, size_t n, float value, void *stream) {
    if (n == 0) return KATSU_OK;
    if (!x) return KATSU_E_INVALID;
    const int64_t N = (int64_t)n;
    if (aligned16(x))
        ew_fill<true><<<ew_blocks(cdiv(N, 4)), 256, 0, (hipStream_t)stream>>>(x, N, value);
    else
        ew_fill<false><<<ew_blocks(N), 256, 0, (hipStream_t)stream>>>(x, N, value);
    return launch_status();
}

int katsu_hip_add_scalar_f32_dev(const float *s_, float *y, size_t n, float beta,
                                 void *stream) {
    if (!beta_ok(beta)) return KATSU_E_INVALID;
    if (n == 0) return KATSU_OK;
    if (!s_ || !y) return KATSU_E_INVALID;
    const int64_t N = (int64_t)n;
    if (aligned16(y))
        ew_add_scalar<true><<<ew_blocks(cdiv(N, 4)), 256, 0, (hipStream_t)stream>>>(s_, y, N,
                                                                                   beta);
    else
        ew_add_scalar<false><<<ew_blocks(N), 256, 0, (hipStream_t)stream>>>(s_, y, N, beta);
    return launch_status();
}

int katsu_hip_sum_f32_dev(const float *x, size_t n, float *out, float beta, void *stream) {
    if (!beta_ok(beta) || !out || (n > 0 && !x)) return KATSU_E_INVALID;
    hipStream_t st = (hipStream_t)stream;
    if (n == 0) {  // the empty fold: out = beta*out + 0
        if (beta == 0.f) ew_fill<false><<<1, 256, 0, st>>>(out, 1, 0.f);
        return launch_status();
    }
    // A fixed number of chunks for a given n (at most 1024), so the tree is
    // the same on every call.
    const int64_t N = (int64_t)n;
    const int64_t chunk = std::max<int64_t>(4096, cdiv(N, 1024));
    const int parts = (int)cdiv(N, chunk);
    float *part = nullptr;
    {
        const int rc = scratch_get(ScratchKind::Sum, st, (size_t)parts * sizeof(float), &part);
        if (rc) return rc;
    }
    if (chunk % 4 == 0 && aligned16(x))
        sum_partials<true><<<parts, 256, 0, st>>>(x, N, chunk, part);
    else
        sum_partials<false><<<parts, 256, 0, st>>>(x, N, chunk, part);
    sum_finish<<<1, 256, 0, st>>>(part, parts, out, beta);
    return launch_status();
}

int katsu_hip_mean_rows_f32_dev(const float *y, size_t rows, size_t cols, float *out,
                                void *stream) {
    if (rows == 0) return KATSU_OK;
    if (!y || !out || cols == 0) return KATSU_E_INVALID;
    if (rows > kI32Max) return KATSU_E_INVALID;
    if (cols % 4 == 0 && aligned16(y))
        mean_rows<true><<<(unsigned)cdiv((int64_t)rows, 4), 256, 0, (hipStream_t)stream>>>(
            y, (int64_t)rows, (int64_t)cols, out);
    else
        mean_rows<false><<<(unsigned)cdiv((int64_t)rows, 4), 256, 0, (hipStream_t)stream>>>(
            y, (int64_t)rows, (int64_t)cols, out);
    return launch_status();
}

int katsu_hip_broadcast_rows_f32_dev(const float *g, size_t rows, size_t cols, float scale,
                                     float *dy, float beta, void *stream) {
    if (!beta_ok(beta)) return KATSU_E_INVALID;
    if (rows == 0 || cols == 0) return KATSU_OK;
    if (!g || !dy) return KATSU_E_INVALID;
    // Parts of at most 4096 elements (or float4s) per block, rows times parts
    // blocks in all.
    const bool vec = cols % 4 == 0 && aligned16(dy);
    const int64_t w = vec ? (int64_t)cols / 4 : (int64_t)cols;
    const int64_t bpr = cdiv(w, 4096), per = cdiv(w, bpr);
    if ((int64_t)rows * bpr > kI32Max) return KATSU_E_INVALID;
    const unsigned blocks = (unsigned)((int64_t)rows * bpr);
    if (vec)
        broadcast_rows<true><<<blocks, 256, 0, (hipStream_t)stream>>>(g, (int64_t)cols, (int)bpr,
                                                                      per, scale, dy, beta);
    else
        broadcast_rows<false><<<blocks, 256, 0, (hipStream_t)stream>>>(g, (int64_t)cols, (int)bpr,
                                                                       per, scale, dy, beta);
    return launch_status();
}

int katsu_hip_gradcam_f32_dev(const float *act, const float *grad, size_t n, size_t c,
                              size_t hw, float *cam, void *stream) {
    if (n == 0 || hw == 0) return KATSU_OK;
    if (!act || !grad || !cam || c == 0) return KATSU_E_INVALID;
    hipStream_t st = (hipStream_t)stream;
    const int64_t N = (int64_t)n, C = (int64_t)c, HW = (int64_t)hw;
    if (N > kI32Max) return KATSU_E_INVALID;
    float *alpha = nullptr;
    {
        const int rc = scratch_get(ScratchKind::Cam, st, (size_t)(N * C) * sizeof(float), &alpha);
        if (rc) return rc;
    }
    if (HW % 4 == 0 && aligned16(grad))
        mean_rows<true><<<(unsigned)cdiv(N * C, 4), 256, 0, st>>>(grad, N * C, HW, alpha);
    else
        mean_rows<false><<<(unsigned)cdiv(N * C, 4), 256, 0, st>>>(grad, N * C, HW, alpha);
    cam_combine<<<ew_blocks(N * HW), 256, 0, st>>>(act, alpha, N, C, HW, cam);
    normalize_rows_by_max<<<(unsigned)N, 256, 0, st>>>(cam, HW);
    return launch_status();
}

int katsu_hip_resize_bilinear_f32_dev(const float *src, size_t n, size_t ih, size_t iw,
                                      size_t oh, size_t ow, float *dst, void *stream) {
    if (n == 0 || oh == 0 || ow == 0) return KATSU_OK;
    if (!src || !dst || ih == 0 || iw == 0) return KATSU_E_INVALID;
    // Per-image offsets and pixel indices are 32-bit.
    if (ih > kI32Max / iw || oh > kI32Max / ow || n > (size_t)kI32Max)
        return KATSU_E_INVALID;
    const int64_t total = (int64_t)n * (int64_t)(oh * ow);
    resize_bilinear<<<ew_blocks(total), 256, 0, (hipStream_t)stream>>>(
        src, (int64_t)n, (int)ih, (int)iw, (int)oh, (int)ow, dst);
    return launch_status();
}

}  // extern "C"
