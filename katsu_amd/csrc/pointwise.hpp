// pointwise.hpp -- 1x1 convolutions (any stride, no padding) as fp32 MFMA
// GEMMs whose pixel operand is addressed in place: the forward
// (conv2d.rs:95-115) and both backward passes (backward_buffers,
// conv2d.rs:265-292) of Conv2D for R = S = 1.  With one tap, every output
// pixel (oy, ox) reads exactly input pixel (oy*s, ox*s), so
//
//   MODE 0  forward  y[n][o][p]  = sum_c w[o][c] x[n][c][oy*s][ox*s]
//           i = o (M = K), j = output pixel over the batch (N*OH*OW), k = c
//   MODE 1  dX       dx[n][c][oy*s][ox*s] = sum_o w[o][c] G[n][o][p]
//           i = c (M = C), j = output pixel, k = o; the other s*s - 1 input
//           pixels of the s x s block that (oy, ox) owns receive no tap and
//           are written as zeros in the same epilogue
//   MODE 2  dW       dw[o][c] = sum_{n,p} G[n][o][p] x[n][c][oy*s][ox*s]
//           i = o (M = K), j = c (N = C), k = output pixel, split over k
//           into fixed partial slices (summed by dw_split_reduce)
//
// Block tile BM x 64 x 32 (BM 64 or 32), four waves in a 2 x 2 grid of
// (BM/2) x 32 wave tiles.  Both operands are staged through registers into
// LDS as [k][i] and [k][j] (i and j contiguous), double-buffered, and read
// FM (FN) fragments at a time: fragment a's MFMA row m is tile row FM*m + a.
// Each thread loads elements along the operand's coalesced dimension: pixel
// columns for the gathered x and G operands of MODE 0 and 1 (fixed per
// thread, so their addresses are decoded once), pixels along k in MODE 2
// (one pixel per thread per k-tile), the weight's contiguous dimension
// otherwise.
#pragma once

#include "direct.hpp"

namespace katsu {

struct PwArgs {
    const float *x, *w, *g;
    float *out;          // y (MODE 0), dx (MODE 1), dw or the partial slices (MODE 2)
    int M, N, K;         // GEMM sizes as above
    int C, H, W, KO, OW, OHW, HW, st;
    int64_t x_img, g_img;  // C*H*W and KO*OH*OW
    int tiles_m, tiles_n, splits, kchunk;  // kchunk: a multiple of 32
    int64_t split_stride;  // floats between partial slices, or 0 when writing the output
    float beta;            // out = beta*out + result when writing the output directly
    FastDiv fd_ohw, fd_ow;
    int quad;  // MODE 1: stride 2 onto H = 2*OH, W = 2*OW, OW even, beta 0, dx 16-byte aligned
    uint32_t x_bytes, w_bytes, g_bytes;  // buffer-resource sizes (buffer-load forms)
};

template <int BM>
struct PwGeo {
    static constexpr int BN = 64, BK = 32;
    static constexpr int PA = BM + 4, PB = BN + 4;  // [k][i] and [k][j] row pitches
    static constexpr int SA = BK * PA, SB = BK * PB;
    static constexpr int STAGE = SA + SB;
    static constexpr size_t kBytes = 2 * (size_t)STAGE * sizeof(float);
};

// A value the compiler may not reason about: a buffer offset selected
// between an address and kOOB stays one unconditional load, instead of
// being split into a branch around the load.
__device__ __forceinline__ int vopaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Block `bid` of the `nb` blocks of pass g (pw_kernel, or one of the two
// passes of pw_bwd_kernel).
// V: 0 scalar loads; bit 0 the A operand 16 bytes at a time (the weight in
// MODE 0 and 1: C % 4 = 0, w 16-byte aligned; G along four adjacent pixels
// in MODE 2: OH*OW % 4 = 0, G 16-byte aligned); V = 3 also G 16 bytes at a
// time in MODE 1 (same condition), each thread then taking four adjacent
// pixel columns.
template <int MODE, int BM, int V, int PF = 1>
__device__ __forceinline__ void pw_block(const PwArgs &g, int bid, int nb) {
    constexpr bool AV = (V & 1) != 0, BV = MODE == 1 && (V & 2) != 0;
    using Geo = PwGeo<BM>;
    constexpr int BN = Geo::BN, BK = Geo::BK;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 16, FN = WN / 16;
    constexpr int NA = BM * BK / 256, NB = BN * BK / 256;  // elements per thread per k-tile
    static_assert(BM == 32 || BM == 64, "BM");

    extern __shared__ float smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wi0 = (wave >> 1) * WM, wj0 = (wave & 1) * WN;
    const int l16 = lane & 15, lg = lane >> 4;

    const int t = xcd_swizzle(bid, nb);
    const int split = t / (g.tiles_m * g.tiles_n);
    const int tile = t - split * (g.tiles_m * g.tiles_n);
    const int i0 = (tile % g.tiles_m) * BM, j0 = (tile / g.tiles_m) * BN;
    const int kb = split * g.kchunk;
    const int ke = min(kb + g.kchunk, g.K);

    // Element e = q*256 + tid of a tile.  "Fast" dimension = the one that
    // varies across consecutive threads.
    //   MODE 0: A (o, c) c-fast; B (c, pixel) pixel-fast
    //   MODE 1: A (c, o) c-fast (i-fast); B (o, pixel) pixel-fast
    //   MODE 2: A (o, pixel) pixel-fast (k-fast); B (pixel, c) pixel-fast (k-fast)
    // Pixel columns of MODE 0 and 1: this thread's column is j0 + tid % 64
    // (with BV, columns j0 + 4*(tid % 16) .. +3, all in one image).
    int64_t colx = 0, colg = 0;
    bool colok = false;
    if (MODE != 2) {
        const int j = j0 + (BV ? 4 * (tid & 15) : (tid & 63));
        colok = j < g.N;
        const int jj = colok ? j : 0;
        const int n = g.fd_ohw.div(jj);
        const int p = jj - n * g.OHW;
        const int oy = g.fd_ow.div(p);
        const int ox = p - oy * g.OW;
        colx = (int64_t)n * g.x_img + (int64_t)oy * g.st * g.W + (int64_t)ox * g.st;
        colg = (int64_t)n * g.g_img + p;
    }

    float va[NA], vb[NB];
    auto load = [&](int k0) __attribute__((always_inline)) {
        if (MODE != 2) {
            // A: the weight, w[o][c] with c contiguous; 16 bytes at a time
            // (four k of one row in MODE 0, four rows i of one k in MODE 1)
            // when the host found C % 4 == 0 and w 16-byte aligned.
            if (AV) {
#pragma unroll
                for (int q = 0; q < NA / 4; ++q) {
                    const int e = q * 256 + tid;
                    int i, k;
                    if (MODE == 0) { i = i0 + e / (BK / 4); k = k0 + 4 * (e % (BK / 4)); }
                    else { i = i0 + 4 * (e % (BM / 4)); k = k0 + e / (BM / 4); }
                    const int64_t off = MODE == 0 ? (int64_t)i * g.C + k : (int64_t)k * g.C + i;
                    const floatx4 v = (i < g.M && k < ke)
                                          ? *reinterpret_cast<const floatx4 *>(g.w + off)
                                          : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int r = 0; r < 4; ++r) va[4 * q + r] = v[r];
                }
            } else {
#pragma unroll
                for (int q = 0; q < NA; ++q) {
                    const int e = q * 256 + tid;
                    if (MODE == 0) {
                        const int i = i0 + e / BK, k = k0 + e % BK;
                        va[q] = (i < g.M && k < ke) ? g.w[(int64_t)i * g.C + k] : 0.f;
                    } else {
                        const int i = i0 + e % BM, k = k0 + e / BM;
                        va[q] = (i < g.M && k < ke) ? g.w[(int64_t)k * g.C + i] : 0.f;
                    }
                }
            }
            // B: pixel columns, x[n][c][oy*s][ox*s] (MODE 0) or G[n][o][p].
            if (BV) {
#pragma unroll
                for (int q = 0; q < NB / 4; ++q) {
                    const int k = k0 + q * 16 + (tid >> 4);
                    const floatx4 v =
                        (colok && k < ke)
                            ? *reinterpret_cast<const floatx4 *>(g.g + colg + (int64_t)k * g.OHW)
                            : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int r = 0; r < 4; ++r) vb[4 * q + r] = v[r];
                }
            } else {
#pragma unroll
                for (int q = 0; q < NB; ++q) {
                    const int k = k0 + q * 4 + (tid >> 6);
                    vb[q] = (colok && k < ke) ? (MODE == 0 ? g.x[colx + (int64_t)k * g.HW]
                                                           : g.g[colg + (int64_t)k * g.OHW])
                                              : 0.f;
                }
            }
        } else {
            // One pixel per thread per k-tile: k = k0 + tid % 32.
            const int k = k0 + (tid & (BK - 1));
            const bool kok = k < ke;
            const int kk = kok ? k : 0;
            const int n = g.fd_ohw.div(kk);
            const int p = kk - n * g.OHW;
            const int oy = g.fd_ow.div(p);
            const int ox = p - oy * g.OW;
            const int64_t gb = (int64_t)n * g.g_img + p;
            const int64_t xb = (int64_t)n * g.x_img + (int64_t)oy * g.st * g.W + (int64_t)ox * g.st;
            if (AV) {  // G[n][o][p..p+3]: pixels k4 .. k4+3 of one image
                const int k4 = k0 + 4 * (tid & (BK / 4 - 1));
                const bool k4ok = k4 < ke;
                const int kk4 = k4ok ? k4 : 0;
                const int n4 = g.fd_ohw.div(kk4);
                const int64_t gb4 = (int64_t)n4 * g.g_img + (kk4 - n4 * g.OHW);
#pragma unroll
                for (int q = 0; q < NA / 4; ++q) {
                    const int i = i0 + q * (1024 / BK) + (tid / (BK / 4));
                    const floatx4 v =
                        (k4ok && i < g.M)
                            ? *reinterpret_cast<const floatx4 *>(g.g + gb4 + (int64_t)i * g.OHW)
                            : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int r = 0; r < 4; ++r) va[4 * q + r] = v[r];
                }
            } else {
#pragma unroll
                for (int q = 0; q < NA; ++q) {  // G[n][o][p]
                    const int i = i0 + q * (256 / BK) + (tid / BK);
                    va[q] = (kok && i < g.M) ? g.g[gb + (int64_t)i * g.OHW] : 0.f;
                }
            }
#pragma unroll
            for (int q = 0; q < NB; ++q) {  // x[n][c][oy*s][ox*s]
                const int j = j0 + q * (256 / BK) + (tid / BK);
                vb[q] = (kok && j < g.N) ? g.x[xb + (int64_t)j * g.HW] : 0.f;
            }
        }
    };
    auto store = [&](float *st) __attribute__((always_inline)) {
        float *sa = st, *sb = st + Geo::SA;
#pragma unroll
        for (int q = 0; q < NA; ++q) {
            int i, k;
            if (AV && MODE == 2) {
                i = (q / 4) * (1024 / BK) + tid / (BK / 4);
                k = 4 * (tid & (BK / 4 - 1)) + q % 4;
            } else if (AV) {
                const int e = (q / 4) * 256 + tid, r = q % 4;
                if (MODE == 0) { i = e / (BK / 4); k = 4 * (e % (BK / 4)) + r; }
                else { i = 4 * (e % (BM / 4)) + r; k = e / (BM / 4); }
            } else {
                const int e = q * 256 + tid;
                if (MODE == 0) { i = e / BK; k = e % BK; }
                else if (MODE == 1) { i = e % BM; k = e / BM; }
                else { i = q * (256 / BK) + tid / BK; k = tid & (BK - 1); }
            }
            sa[k * Geo::PA + i] = va[q];
        }
#pragma unroll
        for (int q = 0; q < NB; ++q) {
            int j, k;
            if (BV) { j = 4 * (tid & 15) + q % 4; k = (q / 4) * 16 + (tid >> 4); }
            else if (MODE != 2) { j = tid & 63; k = q * 4 + (tid >> 6); }
            else { j = q * (256 / BK) + tid / BK; k = tid & (BK - 1); }
            sb[k * Geo::PB + j] = vb[q];
        }
    };

    floatx4 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};

    // Step s of 16-deep block kq: lane group lg takes k = 16*kq + 4*lg + s.
    auto compute = [&](const float *st) __attribute__((always_inline)) {
        const float *sa = st, *sb = st + Geo::SA;
#pragma unroll
        for (int kq = 0; kq < BK / 16; ++kq)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int k = 16 * kq + 4 * lg + s;
                const auto av = *reinterpret_cast<const typename FloatN<FM>::T *>(
                    sa + k * Geo::PA + wi0 + FM * l16);
                const auto bv = *reinterpret_cast<const typename FloatN<FN>::T *>(
                    sb + k * Geo::PB + wj0 + FN * l16);
#pragma unroll
                for (int a = 0; a < FM; ++a)
#pragma unroll
                    for (int b = 0; b < FN; ++b)
                        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                            lane_of<FM>(av, a), lane_of<FN>(bv, b), acc[a][b], 0, 0, 0);
            }
    };

    if constexpr (PF > 1) {
        // Buffer loads with PF k-tiles in flight (MODE 1 and 2): tile t's
        // registers are stored to LDS stage t % 2 and refilled with tile
        // t + PF before tile t's MFMAs.  Every load is issued whatever k
        // (kOOB past the slice, reading zeros), so the loop is the same on
        // every pass and each store waits only for its own tile; the k-tiles
        // past the slice's end up to a multiple of PF add zeros.
        static_assert(MODE != 0 && PF % 2 == 0, "ring: dX and dW, an even depth");
        const __amdgpu_buffer_rsrc_t rw = buf_rsrc(g.w, g.w_bytes);
        const __amdgpu_buffer_rsrc_t rgg = buf_rsrc(g.g, g.g_bytes);
        const __amdgpu_buffer_rsrc_t rx = buf_rsrc(g.x, g.x_bytes);
        auto bload = [&](int k0, float (&xa)[NA], float (&xb)[NB])
                         __attribute__((always_inline)) {
            if (MODE == 1) {
                // A: w[o = k][c = i], four channels per 16-byte load (AV).
                if (AV) {
#pragma unroll
                    for (int q = 0; q < NA / 4; ++q) {
                        const int e = q * 256 + tid;
                        const int i = i0 + 4 * (e % (BM / 4)), k = k0 + e / (BM / 4);
                        const int off = vopaque((i < g.M && k < ke) ? (k * g.C + i) * 4 : kOOB);
                        const floatx4 v = __builtin_bit_cast(
                            floatx4, __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 0));
#pragma unroll
                        for (int r = 0; r < 4; ++r) xa[4 * q + r] = v[r];
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < NA; ++q) {
                        const int e = q * 256 + tid;
                        const int i = i0 + e % BM, k = k0 + e / BM;
                        const int off = vopaque((i < g.M && k < ke) ? (k * g.C + i) * 4 : kOOB);
                        xa[q] = __builtin_bit_cast(
                            float, __builtin_amdgcn_raw_buffer_load_b32(rw, off, 0, 0));
                    }
                }
                // B: G[n][o = k][p], four pixels per 16-byte load (BV).
                if (BV) {
#pragma unroll
                    for (int q = 0; q < NB / 4; ++q) {
                        const int k = k0 + q * 16 + (tid >> 4);
                        const int off = vopaque(
                            (colok && k < ke) ? (int)(colg + (int64_t)k * g.OHW) * 4 : kOOB);
                        const floatx4 v = __builtin_bit_cast(
                            floatx4, __builtin_amdgcn_raw_buffer_load_b128(rgg, off, 0, 0));
#pragma unroll
                        for (int r = 0; r < 4; ++r) xb[4 * q + r] = v[r];
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < NB; ++q) {
                        const int k = k0 + q * 4 + (tid >> 6);
                        const int off = vopaque(
                            (colok && k < ke) ? (int)(colg + (int64_t)k * g.OHW) * 4 : kOOB);
                        xb[q] = __builtin_bit_cast(
                            float, __builtin_amdgcn_raw_buffer_load_b32(rgg, off, 0, 0));
                    }
                }
            } else {
                // One pixel per thread per k-tile, k = k0 + tid % 32.
                const int k = k0 + (tid & (BK - 1));
                const bool kok = k < ke;
                const int kk = kok ? k : 0;
                const int n = g.fd_ohw.div(kk);
                const int p = kk - n * g.OHW;
                const int oy = g.fd_ow.div(p);
                const int ox = p - oy * g.OW;
                const int gb = (int)((int64_t)n * g.g_img + p);
                const int xb0 = (int)((int64_t)n * g.x_img + (int64_t)(oy * g.W + ox) * g.st);
                if (AV) {  // G[n][o][p..p+3]: pixels k4 .. k4+3 of one image
                    const int k4 = k0 + 4 * (tid & (BK / 4 - 1));
                    const bool k4ok = k4 < ke;
                    const int kk4 = k4ok ? k4 : 0;
                    const int n4 = g.fd_ohw.div(kk4);
                    const int gb4 = (int)((int64_t)n4 * g.g_img + (kk4 - n4 * g.OHW));
#pragma unroll
                    for (int q = 0; q < NA / 4; ++q) {
                        const int i = i0 + q * (1024 / BK) + (tid / (BK / 4));
                        const int off = vopaque((k4ok && i < g.M) ? (gb4 + i * g.OHW) * 4 : kOOB);
                        const floatx4 v = __builtin_bit_cast(
                            floatx4, __builtin_amdgcn_raw_buffer_load_b128(rgg, off, 0, 0));
#pragma unroll
                        for (int r = 0; r < 4; ++r) xa[4 * q + r] = v[r];
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < NA; ++q) {  // G[n][o][p]
                        const int i = i0 + q * (256 / BK) + (tid / BK);
                        const int off = vopaque((kok && i < g.M) ? (gb + i * g.OHW) * 4 : kOOB);
                        xa[q] = __builtin_bit_cast(
                            float, __builtin_amdgcn_raw_buffer_load_b32(rgg, off, 0, 0));
                    }
                }
#pragma unroll
                for (int q = 0; q < NB; ++q) {  // x[n][c][oy*s][ox*s]
                    const int j = j0 + q * (256 / BK) + (tid / BK);
                    const int off = vopaque((kok && j < g.N) ? (xb0 + j * g.HW) * 4 : kOOB);
                    xb[q] = __builtin_bit_cast(
                        float, __builtin_amdgcn_raw_buffer_load_b32(rx, off, 0, 0));
                }
            }
        };
        if (kb < ke) {
            const int T = (ke - kb + BK - 1) / BK;
            float ra[PF][NA], rb[PF][NB];
#pragma unroll
            for (int d = 0; d < PF; ++d) bload(kb + d * BK, ra[d], rb[d]);
            for (int t0 = 0; t0 < T; t0 += PF) {
#pragma unroll
                for (int d = 0; d < PF; ++d) {
                    float *stg = smem + (d & 1) * Geo::STAGE;
#pragma unroll
                    for (int q = 0; q < NA; ++q) va[q] = ra[d][q];
#pragma unroll
                    for (int q = 0; q < NB; ++q) vb[q] = rb[d][q];
                    store(stg);
                    __syncthreads();
                    bload(kb + (t0 + d + PF) * BK, ra[d], rb[d]);
                    // The refill is issued before the tile's LDS reads and MFMAs.
                    __builtin_amdgcn_sched_barrier(0);
                    compute(stg);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    } else if (kb < ke) {
        float *st0 = smem, *st1 = smem + Geo::STAGE;
        load(kb);
        store(st0);
        __syncthreads();
        for (int k0 = kb; k0 < ke; k0 += 2 * BK) {
            const bool m1 = k0 + BK < ke, m2 = k0 + 2 * BK < ke;
            if (m1) load(k0 + BK);
            compute(st0);
            if (m1) store(st1);
            __syncthreads();
            if (!m1) break;
            if (m2) load(k0 + 2 * BK);
            compute(st1);
            if (m2) store(st0);
            __syncthreads();
        }
    }

    // Epilogue: fragment (a, b), register v is tile row FM*(4*lg + v) + a,
    // tile column FN*l16 + b.
    const bool direct = g.split_stride == 0;
    if constexpr (MODE == 1 && FN == 2) {
        if (g.quad) {
            // A lane's two columns are output pixels (oy, ox), (oy, ox + 1)
            // with ox even: their 2 x 2 input blocks form a 2 x 4 block of
            // dx, written as two 16-byte stores (taps at even columns of
            // the first row, zeros elsewhere).
            const int j = j0 + wj0 + 2 * l16;
            if (j < g.N) {
                const int n = g.fd_ohw.div(j), p = j - n * g.OHW;
                const int oy = g.fd_ow.div(p), ox = p - oy * g.OW;
                float *col = g.out + (int64_t)n * g.x_img + (int64_t)(2 * oy) * g.W + 2 * ox;
#pragma unroll
                for (int a = 0; a < FM; ++a)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int i = i0 + wi0 + FM * (4 * lg + v) + a;
                        if (i >= g.M) continue;
                        float *blk = col + (int64_t)i * g.HW;
                        // Streamed past the caches: nothing in this launch
                        // reads dx back.
                        __builtin_nontemporal_store(floatx4{acc[a][0][v], 0.f, acc[a][1][v], 0.f},
                                                    reinterpret_cast<floatx4 *>(blk));
                        __builtin_nontemporal_store(floatx4{0.f, 0.f, 0.f, 0.f},
                                                    reinterpret_cast<floatx4 *>(blk + g.W));
                    }
            }
            return;
        }
    }
#pragma unroll
    for (int b = 0; b < FN; ++b) {
        const int j = j0 + wj0 + FN * l16 + b;
        if (j >= g.N) continue;
        if (MODE == 2) {
            float *out = direct ? g.out : g.out + (int64_t)split * g.split_stride;
#pragma unroll
            for (int a = 0; a < FM; ++a)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int i = i0 + wi0 + FM * (4 * lg + v) + a;
                    if (i >= g.M) continue;
                    float *p = out + (int64_t)i * g.N + j;
                    *p = (direct && g.beta != 0.f) ? *p + acc[a][b][v] : acc[a][b][v];
                }
            continue;
        }
        const int n = g.fd_ohw.div(j);
        const int p = j - n * g.OHW;
        if (MODE == 0) {
            float *col = g.out + (int64_t)n * g.g_img + p;
#pragma unroll
            for (int a = 0; a < FM; ++a)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int i = i0 + wi0 + FM * (4 * lg + v) + a;
                    if (i < g.M) store_beta(col + (int64_t)i * g.OHW, acc[a][b][v], g.beta);
                }
        } else {
            // The s x s input block of output pixel (oy, ox), clipped to the
            // image: the tap's value at its corner, zeros elsewhere (kept as
            // they are when accumulating).
            const int oy = g.fd_ow.div(p);
            const int ox = p - oy * g.OW;
            const int iy = oy * g.st, ix = ox * g.st;
            const int hy = min(g.st, g.H - iy), hx = min(g.st, g.W - ix);
            float *col = g.out + (int64_t)n * g.x_img + (int64_t)iy * g.W + ix;
#pragma unroll
            for (int a = 0; a < FM; ++a)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int i = i0 + wi0 + FM * (4 * lg + v) + a;
                    if (i >= g.M) continue;
                    float *blk = col + (int64_t)i * g.HW;
                    store_beta(blk, acc[a][b][v], g.beta);
                    if (g.beta == 0.f) {
                        for (int dy = 0; dy < hy; ++dy)
                            for (int dx = 0; dx < hx; ++dx)
                                if (dy | dx) blk[dy * g.W + dx] = 0.f;
                    }
                }
        }
    }
}

// The forward of a 1x1 layer whose input channels split into four 16-deep
// multiples (C = 64 * NKB), register-direct: a block is one 64 x 64 tile of
// (output channel, output pixel), and wave w takes input channels
// [16 NKB w, 16 NKB (w + 1)).  Each wave loads its operands straight into
// MFMA operand registers, every load of its k-range in flight at once (no LDS
// stage, no barrier before the epilogue):
//   A = w[o][c], c contiguous: one 16-byte load per 16-row fragment gives a
//       lane w[o][c0 + 4 g4 .. +3], its four k-steps (lane group g4 = l/16);
//   B = x[n][c][oy s][ox s]: fragment b is output pixels j0 + 16 b + l%16,
//       one 4-byte load per k-step, channel c0 + 4 g4 + step.
// So MFMA k-row g4 of step s is channel c0 + 4 g4 + s in both operands.  The
// four waves' sums go through LDS and are added in wave order; wave w then
// stores output channels i0 + 16 w .. +15, a row of 64 consecutive pixels per
// store.
template <int NKB>
__device__ __forceinline__ void pw_rd_fwd_block(const PwArgs &g, int bid, int nb) {
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, g4 = lane >> 4;
    const int tile = xcd_swizzle(bid, nb);
    const int i0 = (tile % g.tiles_m) * 64, j0 = (tile / g.tiles_m) * 64;
    const int c0 = w * NKB * 16;

    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(g.w, g.w_bytes);
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(g.x, g.x_bytes);
    // Lane parts of the byte offsets (kOOB past the last row or pixel).
    int vw[4], vx[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int i = i0 + 16 * q + l16;
        vw[q] = i < g.M ? (i * g.C + 4 * g4) * 4 : kOOB;
        const int j = j0 + 16 * q + l16;
        if (j < g.N) {
            const int n = g.fd_ohw.div(j), p = j - n * g.OHW;
            const int oy = g.fd_ow.div(p), ox = p - oy * g.OW;
            vx[q] = (int)((int64_t)n * g.x_img + (int64_t)(oy * g.W + ox) * g.st +
                          (int64_t)4 * g4 * g.HW) * 4;
        } else {
            vx[q] = kOOB;
        }
    }
    const int hw4 = g.HW * 4;

    floatx4 fa[NKB][4];
    float fb[NKB][4][4];  // [k-block][fragment][step]
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
        const int c = c0 + 16 * kb;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            fa[kb][q] = __builtin_bit_cast(
                floatx4, __builtin_amdgcn_raw_buffer_load_b128(rw, vw[q], c * 4, 0));
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                fb[kb][q][s] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(rx, vx[q], (c + s) * hw4, 0));
    }
    // Every load issued before the first MFMA: left alone, the scheduler
    // sinks each load to its first use and waits for it there.
    __builtin_amdgcn_sched_barrier(0);
    floatx4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[kb][a][s], fb[kb][b][s],
                                                                     acc[a][b], 0, 0, 0);

    // Value (a, b, v) of wave p (tile row 16a + 4 g4 + v, column 16b + l16) at
    // part[p][((a*4 + v)*4 + b)*64 + 16 (g4 ^ b) + l16]: the xor puts both the
    // writes (fixed b) and the reads (fixed g4) of a wave on 64 distinct words.
    extern __shared__ float part[];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                part[(w * 64 + (a * 4 + v) * 4 + b) * 64 + ((g4 ^ b) << 4) + l16] = acc[a][b][v];
    __syncthreads();
    const int j = j0 + lane;
    if (j >= g.N) return;
    const int n = g.fd_ohw.div(j), p = j - n * g.OHW;
    float *col = g.out + (int64_t)n * g.g_img + p;
    const int b = lane >> 4;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int i = i0 + 16 * w + r;
        if (i >= g.M) break;
        const int v = r & 3, rg = r >> 2;  // row r = 4 rg + v of fragment a = w
        const int idx = ((w * 4 + v) * 4 + b) * 64 + ((rg ^ b) << 4) + l16;
        float t = part[idx];
#pragma unroll
        for (int q = 1; q < 4; ++q) t += part[q * 64 * 64 + idx];
        col[(int64_t)i * g.OHW] = t;
    }
}

template <int NKB>
__global__ void __launch_bounds__(256, 2) pw_rd_fwd_kernel(const PwArgs g) {
    pw_rd_fwd_block<NKB>(g, blockIdx.x, gridDim.x);
}

template <int MODE, int BM, int V, int PF>
__global__ void __launch_bounds__(256, 2) pw_kernel(const PwArgs g) {
    pw_block<MODE, BM, V, PF>(g, blockIdx.x, gridDim.x);
}

// dX and the dW partials of a 1x1 layer in one launch (conv2d.rs:265-292):
// blocks [0, nbw) are dW blocks (the longer ones, dispatched first), the
// rest dX blocks; nbw is a multiple of 8, so each pass keeps its XCD
// placement.
template <int BMX, int BMW, int VX, int VW, int PF>
__global__ void __launch_bounds__(256, 2) pw_bwd_kernel(const PwArgs dx, const PwArgs dw,
                                                        int nbw) {
    if ((int)blockIdx.x < nbw)
        pw_block<2, BMW, VW, PF>(dw, blockIdx.x, nbw);
    else
        pw_block<1, BMX, VX, PF>(dx, blockIdx.x - nbw, gridDim.x - nbw);
}

}  // namespace katsu
