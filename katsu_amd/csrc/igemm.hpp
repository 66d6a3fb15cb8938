// igemm.hpp -- fp32 MFMA tile engine for gfx950 (CDNA4) shared by every
// contraction on the path: matmul NN/NT/TN and the three implicit-GEMM
// convolution passes.
//
// A launch computes C[i][j] = sum_k A[i][k] * B[k][j] over tiles of
// BM x BN with a k-loop of BK.  Each operand is a *view* that knows how to
// produce element (k, i) from the caller's tensors (a row-major matrix, an
// OIHW filter, or an on-the-fly im2col of an NCHW tensor -- nothing is
// materialised in HBM).  Tiles are staged through LDS, double-buffered, and
// consumed by v_mfma_f32_16x16x4_f32 (64 lanes, 2048 FLOP, 32 cycles).
//
// MFMA 16x16x4 f32 lane layout (wave64):
//   A fragment: lane l holds A[i = l%16][k = l/16]
//   B fragment: lane l holds B[k = l/16][j = l%16]
//   D: lane l, register v holds D[i = 4*(l/16) + v][j = l%16]
// The j dimension of every problem is the contiguous one of its output, so
// each store writes 16 consecutive floats per row.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "exact.hpp"

namespace katsu {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 waves of 64

// Division by a runtime constant d (1 <= d < 2^31) for n < 2^31:
// q = (umulhi(n, m) + n) >> s with s = ceil(log2 d) and
// m = floor(2^32 (2^s - d) / d) + 1 (Granlund & Montgomery, 1994).
struct FastDiv {
    uint32_t d, m, s;
    __device__ __forceinline__ int div(int n) const {
        return (int)((__umulhi((uint32_t)n, m) + (uint32_t)n) >> s);
    }
};

inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f;
    f.d = d;
    uint32_t s = 0;
    while ((1ull << s) < d) ++s;
    f.s = s;
    f.m = (uint32_t)(((1ull << 32) * ((1ull << s) - d)) / d + 1);
    return f;
}

// Blocks are dispatched round-robin over the 8 XCDs (block b runs on XCD
// b % 8).  Renumber so that each XCD receives a contiguous range of logical
// tiles; neighbouring tiles share operand rows/halos, which then hit the
// same XCD's L2.
__device__ __forceinline__ int xcd_swizzle(int b, int nb) {
    const int per = nb >> 3, rem = nb & 7;
    const int x = b & 7, idx = b >> 3;
    return x * per + (x < rem ? x : rem) + idx;
}

// LDS tile of one operand, BI (i or j extent) by BK.
// KMAJOR: stored [k][i] (i contiguous), used when the global tensor is
//         contiguous along i; row pitch = BI + pad with pitch % 32 == 16 so
//         the two k-rows a half-wave reads land in disjoint banks.
// IMAJOR: stored [i][k] (k contiguous), used when the global tensor is
//         contiguous along k; pitch = 2 * odd so 16 rows x 2 k-columns of a
//         half-wave read cover 32 distinct banks.
template <bool KMAJOR, int BI, int BK>
struct SmemTile {
    static constexpr int kPitch = KMAJOR ? (BI % 32 == 0 ? BI + 16 : BI)
                                         : (((BK / 2) % 2 == 1) ? BK : BK + 2);
    static constexpr int kSize = KMAJOR ? BK * kPitch : BI * kPitch;
    __device__ __forceinline__ static int idx(int k, int i) {
        return KMAJOR ? k * kPitch + i : i * kPitch + k;
    }
};

// Moves one operand tile global -> registers -> LDS.
//   KMAJOR: thread t owns column i = t % BI and rows k = t / BI + q*(256/BI)
//   IMAJOR: thread t owns row-element k = t % BK and i = t / BK + q*(256/BK)
// so consecutive lanes walk the contiguous global dimension (coalesced).
template <class View, int BI, int BK>
struct TileLoader {
    static constexpr bool KM = View::kKMajor;
    static_assert(KM ? (kThreads % BI == 0) : (kThreads % BK == 0), "tile/threads mismatch");
    static constexpr int E = BI * BK / kThreads;
    static_assert(E >= 1, "tile too small");
    static constexpr int STEP = KM ? kThreads / BI : kThreads / BK;
    using Tile = SmemTile<KM, BI, BK>;

    typename View::IState is[KM ? 1 : E];
    int ti, tk;

    __device__ __forceinline__ void init(const View &v, int i0, int tid) {
        if constexpr (KM) {
            ti = tid % BI;
            tk = tid / BI;
            is[0] = v.prep_i(i0 + ti);
        } else {
            tk = tid % BK;
            ti = tid / BK;
#pragma unroll
            for (int q = 0; q < E; ++q) is[q] = v.prep_i(i0 + ti + q * STEP);
        }
    }

    __device__ __forceinline__ void fetch(const View &v, int k0, int kend, float (&r)[E]) const {
        if constexpr (KM) {
#pragma unroll
            for (int q = 0; q < E; ++q) {
                const auto ks = v.prep_k(k0 + tk + q * STEP, kend);
                r[q] = v.get(is[0], ks);
            }
        } else {
            const auto ks = v.prep_k(k0 + tk, kend);
#pragma unroll
            for (int q = 0; q < E; ++q) r[q] = v.get(is[q], ks);
        }
    }

    __device__ __forceinline__ void store(float *s, const float (&r)[E]) const {
        if constexpr (KM) {
#pragma unroll
            for (int q = 0; q < E; ++q) s[Tile::idx(tk + q * STEP, ti)] = r[q];
        } else {
#pragma unroll
            for (int q = 0; q < E; ++q) s[Tile::idx(tk, ti + q * STEP)] = r[q];
        }
    }
};

// Per-block plan produced by a problem: tile origin and k range.
struct BlockPlan {
    int tm, tn;      // tile coordinates
    int kbeg, kend;  // reduction range of this block
};

// The engine.  Prob supplies:
//   using AView, BView, Epi;  Prob::plan(int t, AView&, BView&, Epi&, BlockPlan&)
//   (plan may specialise the views per block, e.g. per stride phase).
template <int BM, int BN, int BK, int WM, int WN, class Prob>
__global__ void __launch_bounds__(kThreads) igemm_kernel(const Prob prob) {
    static_assert(BK % 4 == 0, "BK must be a multiple of the MFMA k (4)");
    static_assert((BM / WM) * (BN / WN) == kThreads / 64, "4 waves per block");
    static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile is made of 16x16 MFMA tiles");
    constexpr int FM = WM / 16, FN = WN / 16;
    constexpr int WAVES_N = BN / WN;

    using AL = TileLoader<typename Prob::AView, BM, BK>;
    using BL = TileLoader<typename Prob::BView, BN, BK>;
    using AT = typename AL::Tile;
    using BT = typename BL::Tile;

    __shared__ float sA[2][AT::kSize];
    __shared__ float sB[2][BT::kSize];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wi0 = (wave / WAVES_N) * WM;
    const int wj0 = (wave % WAVES_N) * WN;

    typename Prob::AView av;
    typename Prob::BView bv;
    typename Prob::Epi epi;
    BlockPlan bp;
    prob.plan(xcd_swizzle(blockIdx.x, gridDim.x), av, bv, epi, bp);
    const int i0 = bp.tm * BM;
    const int j0 = bp.tn * BN;

    floatx4 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};

    if (bp.kbeg < bp.kend) {
        AL al;
        BL bl;
        al.init(av, i0, tid);
        bl.init(bv, j0, tid);
        float ra[AL::E], rb[BL::E];
        al.fetch(av, bp.kbeg, bp.kend, ra);
        bl.fetch(bv, bp.kbeg, bp.kend, rb);
        al.store(sA[0], ra);
        bl.store(sB[0], rb);
        __syncthreads();

        int cur = 0;
        for (int k0 = bp.kbeg; k0 < bp.kend; k0 += BK) {
            const bool more = k0 + BK < bp.kend;
            if (more) {
                al.fetch(av, k0 + BK, bp.kend, ra);
                bl.fetch(bv, k0 + BK, bp.kend, rb);
            }
            const float *A = sA[cur];
            const float *B = sB[cur];
#pragma unroll
            for (int ks = 0; ks < BK / 4; ++ks) {
                const int kk = ks * 4 + (lane >> 4);
                float af[FM], bf[FN];
#pragma unroll
                for (int a = 0; a < FM; ++a) af[a] = A[AT::idx(kk, wi0 + a * 16 + (lane & 15))];
#pragma unroll
                for (int b = 0; b < FN; ++b) bf[b] = B[BT::idx(kk, wj0 + b * 16 + (lane & 15))];
#pragma unroll
                for (int a = 0; a < FM; ++a)
#pragma unroll
                    for (int b = 0; b < FN; ++b)
                        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[a], bf[b], acc[a][b],
                                                                         0, 0, 0);
            }
            if (more) {
                al.store(sA[cur ^ 1], ra);
                bl.store(sB[cur ^ 1], rb);
            }
            __syncthreads();
            cur ^= 1;
        }
    }

#pragma unroll
    for (int b = 0; b < FN; ++b) {
        const int j = j0 + wj0 + b * 16 + (lane & 15);
        const auto js = epi.prep_j(j);
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int i = i0 + wi0 + a * 16 + 4 * (lane >> 4) + v;
                epi.store(js, i, acc[a][b][v]);
            }
    }
}

// ---------------------------------------------------------------------------
// Epilogue helper: out = acc (beta == 0, out not read) or beta*out + acc.
__device__ __forceinline__ void store_beta(float *p, float v, float beta) {
    *p = (beta == 0.f) ? v : beta * *p + v;
}
// The same for the direct convolution kernels' output stream (written once,
// read by a later kernel): a non-temporal store, which drained faster at the
// end of a block there (config 3: forward and dX about 1 us faster), as do
// the 1x1 dX's whole 2 x 4 blocks (pointwise.hpp) and the direct dW's
// 16-byte partial runs.  It is slower for scattered single floats and for
// the GEMM's tiles, which keep ordinary stores.
__device__ __forceinline__ void store_beta_nt(float *p, float v, float beta) {
    __builtin_nontemporal_store((beta == 0.f) ? v : beta * *p + v, p);
}
__device__ __forceinline__ void store4_beta_nt(floatx4 *p, floatx4 v, float beta) {
    if (beta != 0.f) v += *p;
    __builtin_nontemporal_store(v, p);
}

// ---------------------------------------------------------------------------
// Matrix view: element (k, i) at base[i*si + k*sk], zero outside i < I, k < kend.
template <bool KMAJOR>
struct MatView {
    static constexpr bool kKMajor = KMAJOR;
    const float *base;
    int64_t si, sk;
    int I;
    struct IState { const float *p; bool v; };
    struct KState { int64_t off; bool v; };
    __device__ __forceinline__ IState prep_i(int i) const { return {base + (int64_t)i * si, i < I}; }
    __device__ __forceinline__ KState prep_k(int k, int kend) const { return {(int64_t)k * sk, k < kend}; }
    __device__ __forceinline__ float get(const IState &a, const KState &b) const {
        return (a.v && b.v) ? a.p[b.off] : 0.f;
    }
};

struct MatEpi {
    float *c;
    int64_t ldc;
    int M, N;
    float beta;
    struct JState { float *p; bool v; };
    __device__ __forceinline__ JState prep_j(int j) const { return {c + j, j < N}; }
    __device__ __forceinline__ void store(const JState &s, int i, float v) const {
        if (s.v && i < M) store_beta(s.p + (int64_t)i * ldc, v, beta);
    }
};

// C = beta*C + op(A) op(B).  AView/BView layouts are chosen per transpose case.
template <bool A_KM, bool B_KM>
struct GemmProb {
    using AView = MatView<A_KM>;
    using BView = MatView<B_KM>;
    using Epi = MatEpi;
    AView a;
    BView b;
    Epi c;
    int K;
    int tiles_m, tiles_n;
    int group;  // tile rows per group in the grouped ordering
    __device__ __forceinline__ void plan(int t, AView &av, BView &bv, Epi &ep, BlockPlan &bp) const {
        av = a;
        bv = b;
        ep = c;
        // Grouped ordering: walk `group` tile rows column by column so that a
        // contiguous range of t (one XCD) touches few A row-panels and few B
        // column-panels.
        const int per_group = group * tiles_n;
        const int g = t / per_group;
        const int first = g * group;
        const int rows = min(group, tiles_m - first);
        const int r = t - g * per_group;
        bp.tm = first + r % rows;
        bp.tn = r / rows;
        bp.kbeg = 0;
        bp.kend = K;
    }
};

// ---------------------------------------------------------------------------
// Convolution views.  Index arithmetic is 32-bit inside one image (the host
// rejects images of 2^31 elements or more); image bases are 64-bit pointers.

// Forward, B operand: im2col(X).  k = (c, r, s) in OIHW order, i = output
// pixel (n, oy, ox).  Padded taps read as zero.
struct FwdColView {
    static constexpr bool kKMajor = true;  // consecutive output pixels -> consecutive x (stride 1)
    const float *x;
    int H, W, HW, S, RS, OW, OHW, npix, stride, pad;
    int64_t chw;
    FastDiv fd_ohw, fd_ow, fd_rs, fd_s;
    struct IState { const float *p; int iy0, ix0, off; bool v; };
    struct KState { int coff, r, s; bool v; };
    __device__ __forceinline__ IState prep_i(int j) const {
        const int n = fd_ohw.div(j);
        const int rem = j - n * OHW;
        const int oy = fd_ow.div(rem);
        const int ox = rem - oy * OW;
        IState st;
        st.p = x + (int64_t)n * chw;
        st.iy0 = oy * stride - pad;
        st.ix0 = ox * stride - pad;
        st.off = st.iy0 * W + st.ix0;
        st.v = j < npix;
        return st;
    }
    __device__ __forceinline__ KState prep_k(int k, int kend) const {
        const int c = fd_rs.div(k);
        const int rs = k - c * RS;
        const int r = fd_s.div(rs);
        const int s = rs - r * S;
        return {c * HW + r * W + s, r, s, k < kend};
    }
    __device__ __forceinline__ float get(const IState &a, const KState &b) const {
        const int iy = a.iy0 + b.r, ix = a.ix0 + b.s;
        const bool ok = a.v && b.v && (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W;
        return ok ? a.p[b.coff + a.off] : 0.f;
    }
};

// Forward epilogue: C[i = oc][j = pixel] -> y[n][oc][oy][ox].  A non-finite
// sum may hold a weight times a padded zero, which the reference skips: it
// is recomputed over the visited products (exact.hpp).
struct FwdEpi {
    float *y;
    int K, OHW, npix;
    int64_t kohw;
    FastDiv fd_ohw;
    const float *x, *w;  // the operands, for the recomputation
    int C, H, W, R, S, OW, stride, pad;
    int64_t chw;
    struct JState { float *p; int n, pix; bool v; };
    __device__ __forceinline__ JState prep_j(int j) const {
        const int n = fd_ohw.div(j);
        return {y + (int64_t)n * kohw + (j - n * OHW), n, j - n * OHW, j < npix};
    }
    __device__ __forceinline__ void store(const JState &s, int i, float v) const {
        if (!(s.v && i < K)) return;
        if (!__builtin_isfinite(v))
            v = exact_fwd_inl(x + (int64_t)s.n * chw, w, C, H, W, R, S, stride, pad, i, s.pix / OW,
                          s.pix % OW);
        s.p[(int64_t)i * OHW] = v;
    }
};

struct FwdProb {
    using AView = MatView<false>;  // W as [oc][c*r*s], contiguous along k
    using BView = FwdColView;
    using Epi = FwdEpi;
    AView a;
    BView b;
    Epi c;
    int CRS, tiles_m;
    __device__ __forceinline__ void plan(int t, AView &av, BView &bv, Epi &ep, BlockPlan &bp) const {
        av = a;
        bv = b;
        ep = c;
        bp.tm = t % tiles_m;  // the oc tiles of one pixel tile are neighbours (same XCD)
        bp.tn = t / tiles_m;
        bp.kbeg = 0;
        bp.kend = CRS;
    }
};

// ---------------------------------------------------------------------------
// Backward data (dX).  The input plane is split into stride x stride phases
// (py, px); inside a phase every input pixel (iy, ix) = (py + st*a, px + st*b)
// receives exactly the taps r = r0 + st*u, s = s0 + st*v with
// r0 = (py + pad) % st, and the output row oy = a + dy - u with
// dy = (py + pad - r0) / st (similarly for columns).  Each phase is a dense
// GEMM: i = c, j = (n, a, b), k = (oc, u, v) -- no zero-stuffed taps.
struct DxPhase {
    int py, px, r0, s0, dy, dx;
    int Ha, Wa, Ru, Su;
    int npix, kred;       // N*Ha*Wa and K*Ru*Su
    int tiles_n;          // pixel tiles of this phase
    int tile_begin;       // first logical tile of this phase
    FastDiv fd_hawa, fd_wa, fd_rusu, fd_su;
};

constexpr int kMaxPhases = 16;

// A operand: element (k = (oc,u,v), i = c) = W[oc][c][r0+st*u][s0+st*v].
struct DxWView {
    static constexpr bool kKMajor = false;
    const float *w;
    int C, RS, S, CRS, stride, r0, s0, RuSu, Su;
    FastDiv fd_rusu, fd_su;
    struct IState { const float *p; bool v; };
    struct KState { int off; bool v; };
    __device__ __forceinline__ IState prep_i(int c) const { return {w + c * RS, c < C}; }
    __device__ __forceinline__ KState prep_k(int k, int kend) const {
        const int oc = fd_rusu.div(k);
        const int uv = k - oc * RuSu;
        const int u = fd_su.div(uv);
        const int v = uv - u * Su;
        return {oc * CRS + (r0 + stride * u) * S + s0 + stride * v, k < kend};
    }
    __device__ __forceinline__ float get(const IState &a, const KState &b) const {
        return (a.v && b.v) ? a.p[b.off] : 0.f;
    }
};

// B operand: element (k = (oc,u,v), j = (n,a,b)) = G[n][oc][a+dy-u][b+dx-v].
struct DxColView {
    static constexpr bool kKMajor = true;  // consecutive b -> consecutive ox
    const float *g;
    int OH, OW, OHW, dy, dx, Wa, HaWa, npix, RuSu, Su;
    int64_t kohw;
    FastDiv fd_hawa, fd_wa, fd_rusu, fd_su;
    struct IState { const float *p; int oy0, ox0, off; bool v; };
    struct KState { int off, u, v; bool ok; };
    __device__ __forceinline__ IState prep_i(int j) const {
        const int n = fd_hawa.div(j);
        const int rem = j - n * HaWa;
        const int a = fd_wa.div(rem);
        const int b = rem - a * Wa;
        IState st;
        st.p = g + (int64_t)n * kohw;
        st.oy0 = a + dy;
        st.ox0 = b + dx;
        st.off = st.oy0 * OW + st.ox0;
        st.v = j < npix;
        return st;
    }
    __device__ __forceinline__ KState prep_k(int k, int kend) const {
        const int oc = fd_rusu.div(k);
        const int uv = k - oc * RuSu;
        const int u = fd_su.div(uv);
        const int v = uv - u * Su;
        return {oc * OHW - u * OW - v, u, v, k < kend};
    }
    __device__ __forceinline__ float get(const IState &a, const KState &b) const {
        const int oy = a.oy0 - b.u, ox = a.ox0 - b.v;
        const bool ok = a.v && b.ok && (unsigned)oy < (unsigned)OH && (unsigned)ox < (unsigned)OW;
        return ok ? a.p[b.off + a.off] : 0.f;
    }
};

// dX epilogue: C[i = c][j = (n,a,b)] -> dx[n][c][py+st*a][px+st*b].  A
// non-finite sum may hold a weight times a zero outside G, which the
// reference skips: it is recomputed over the visited products (exact.hpp).
struct DxEpi {
    float *dx;
    int C, HW, W, stride, py, px, Wa, HaWa, npix;
    int64_t chw;
    FastDiv fd_hawa, fd_wa;
    float beta;
    const float *g, *w;  // the operands, for the recomputation
    int K, OH, OW, R, S, pad;
    int64_t kohw;
    struct JState { float *p; int n, iy, ix; bool v; };
    __device__ __forceinline__ JState prep_j(int j) const {
        const int n = fd_hawa.div(j);
        const int rem = j - n * HaWa;
        const int a = fd_wa.div(rem);
        const int b = rem - a * Wa;
        const int iy = py + stride * a, ix = px + stride * b;
        return {dx + (int64_t)n * chw + iy * W + ix, n, iy, ix, j < npix};
    }
    __device__ __forceinline__ void store(const JState &s, int i, float v) const {
        if (!(s.v && i < C)) return;
        if (!__builtin_isfinite(v))
            v = exact_dx_inl(g + (int64_t)s.n * kohw, w, K, C, OH, OW, R, S, stride, pad, i, s.iy,
                         s.ix);
        store_beta(s.p + (int64_t)i * HW, v, beta);
    }
};

struct DxProb {
    using AView = DxWView;
    using BView = DxColView;
    using Epi = DxEpi;
    AView a;   // phase fields filled per block
    BView b;
    Epi c;
    int tiles_m;
    int nphases;
    DxPhase ph[kMaxPhases];
    __device__ __forceinline__ void plan(int t, AView &av, BView &bv, Epi &ep, BlockPlan &bp) const {
        int p = 0;
        while (p + 1 < nphases && t >= ph[p + 1].tile_begin) ++p;
        const DxPhase &P = ph[p];
        const int lt = t - P.tile_begin;
        av = a;
        bv = b;
        ep = c;
        av.r0 = P.r0;
        av.s0 = P.s0;
        av.RuSu = P.Ru * P.Su;
        av.Su = P.Su;
        av.fd_rusu = P.fd_rusu;
        av.fd_su = P.fd_su;
        bv.dy = P.dy;
        bv.dx = P.dx;
        bv.Wa = P.Wa;
        bv.HaWa = P.Ha * P.Wa;
        bv.npix = P.npix;
        bv.RuSu = P.Ru * P.Su;
        bv.Su = P.Su;
        bv.fd_hawa = P.fd_hawa;
        bv.fd_wa = P.fd_wa;
        bv.fd_rusu = P.fd_rusu;
        bv.fd_su = P.fd_su;
        ep.py = P.py;
        ep.px = P.px;
        ep.Wa = P.Wa;
        ep.HaWa = P.Ha * P.Wa;
        ep.npix = P.npix;
        ep.fd_hawa = P.fd_hawa;
        ep.fd_wa = P.fd_wa;
        bp.tm = lt % tiles_m;
        bp.tn = lt / tiles_m;
        bp.kbeg = 0;
        bp.kend = P.kred;
    }
};

// ---------------------------------------------------------------------------
// Backward filter (dW): i = oc, j = (c, r, s), k = output pixel (n, oy, ox).
// The k range is split over workgroups; each split writes a full partial
// tile, and a second kernel sums the partials in split order.

// A operand: element (k = pixel, i = oc) = G[n][oc][oy][ox].
struct DwGView {
    static constexpr bool kKMajor = false;  // contiguous along pixels
    const float *g;
    int K, OHW;
    int64_t kohw;
    FastDiv fd_ohw;
    struct IState { int off; bool v; };
    struct KState { const float *p; bool v; };
    __device__ __forceinline__ IState prep_i(int oc) const { return {oc * OHW, oc < K}; }
    __device__ __forceinline__ KState prep_k(int k, int kend) const {
        const int n = fd_ohw.div(k);
        return {g + (int64_t)n * kohw + (k - n * OHW), k < kend};
    }
    __device__ __forceinline__ float get(const IState &a, const KState &b) const {
        return (a.v && b.v) ? b.p[a.off] : 0.f;
    }
};

// B operand: element (k = pixel, j = (c,r,s)) = X[n][c][oy*st+r-pad][ox*st+s-pad].
struct DwColView {
    static constexpr bool kKMajor = false;  // contiguous along pixels (stride 1)
    const float *x;
    int H, W, HW, S, RS, CRS, OW, OHW, stride, pad;
    int64_t chw;
    FastDiv fd_rs, fd_s, fd_ohw, fd_ow;
    struct IState { int coff, r, s; bool v; };
    struct KState { const float *p; int iy0, ix0, off; bool v; };
    __device__ __forceinline__ IState prep_i(int j) const {
        const int c = fd_rs.div(j);
        const int rs = j - c * RS;
        const int r = fd_s.div(rs);
        const int s = rs - r * S;
        return {c * HW + r * W + s, r, s, j < CRS};
    }
    __device__ __forceinline__ KState prep_k(int k, int kend) const {
        const int n = fd_ohw.div(k);
        const int rem = k - n * OHW;
        const int oy = fd_ow.div(rem);
        const int ox = rem - oy * OW;
        KState st;
        st.p = x + (int64_t)n * chw;
        st.iy0 = oy * stride - pad;
        st.ix0 = ox * stride - pad;
        st.off = st.iy0 * W + st.ix0;
        st.v = k < kend;
        return st;
    }
    __device__ __forceinline__ float get(const IState &a, const KState &b) const {
        const int iy = b.iy0 + a.r, ix = b.ix0 + a.s;
        const bool ok = a.v && b.v && (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W;
        return ok ? b.p[a.coff + b.off] : 0.f;
    }
};

// dW epilogue: C[i = oc][j = crs] -> out[split][oc][crs] (partials, beta 0)
// or straight into dw with beta when there is a single split.  A non-finite
// partial may hold G times a padded zero, which the reference skips: it is
// recomputed over the split's pixels [kbeg, kend) (exact.hpp).
struct DwEpi {
    float *out;
    int K, CRS;
    int64_t split_stride;  // K*CRS, or 0 when writing dw directly
    float beta;
    int split;             // set per block
    const float *x, *g;    // the operands, for the recomputation
    int C, H, W, OH, OW, R, S, stride, pad;
    int kbeg, kend;        // set per block
    struct JState { float *p; int j; bool v; };
    __device__ __forceinline__ JState prep_j(int j) const {
        return {out + (int64_t)split * split_stride + j, j, j < CRS};
    }
    __device__ __forceinline__ void store(const JState &s, int i, float v) const {
        if (!(s.v && i < K)) return;
        if (!__builtin_isfinite(v)) {
            const int rs = R * S, c = s.j / rs, t = s.j - c * rs;
            v = exact_dw_inl(x, g, C, H, W, K, OH, OW, stride, pad, i, c, t / S, t % S, kbeg, kend);
        }
        store_beta(s.p + (int64_t)i * CRS, v, beta);
    }
};

struct DwProb {
    using AView = DwGView;
    using BView = DwColView;
    using Epi = DwEpi;
    AView a;
    BView b;
    Epi c;
    int tiles_m, tiles_n, splits, kchunk, npix;
    __device__ __forceinline__ void plan(int t, AView &av, BView &bv, Epi &ep, BlockPlan &bp) const {
        av = a;
        bv = b;
        ep = c;
        const int tiles = tiles_m * tiles_n;
        const int split = t / tiles;
        const int r = t - split * tiles;
        bp.tm = r % tiles_m;
        bp.tn = r / tiles_m;
        bp.kbeg = split * kchunk;
        bp.kend = min(npix, bp.kbeg + kchunk);
        ep.split = split;
        ep.kbeg = bp.kbeg;
        ep.kend = bp.kend;
    }
};

}  // namespace katsu
