// stemdx.hpp -- the data gradient of the stem layer (3 input channels, 64
// output channels, 7x7 filter, stride 2, padding 3): backward_buffers' dx
// (conv2d.rs:288),
//   dx[n][c][iy][ix] = sum over (k, r, s) of w[k][c][r][s] * G[n][k][oy][ox],
//   oy = (iy + 3 - r) / 2, ox = (ix + 3 - s) / 2, over the taps where both
//   divisions are exact and (oy, ox) lies inside the G map.
//
// Phase view.  Input pixel (2Y + py, 2X + px) takes G row Y + dy - 1 with tap
// r = 5 - 2dy (py = 0; dy = 3 has no tap) or r = 6 - 2dy (py = 1), and G
// column X + dx - 1 with s = 5 - 2dx (px = 0; no tap at dx = 3) or 6 - 2dx
// (px = 1), for dy, dx in 0..3.
//
// GEMM view of one G row gy and 16 super-columns X0 .. X0+15 (one wave):
//   D[(j, dy)][X] += sum over (k, dx) of w[k][c][r(py,dy)][s(px,dx)] * G[k][gy][X + dx - 1]
// with j = (c, py, px) one of 12 phase combinations, px = j / 6,
// c = (j % 6) / 2, py = j % 2.  The 48 rows (j, dy) are three MFMA fragments:
// fragment f holds combinations 4f .. 4f+3, row 4q + dy of the fragment being
// combination 4f + q at offset dy.  Fragment 0 holds only px = 0 rows and so
// skips dx = 3.  The zero rows (py = 0 at dy = 3, px = 0 at dx = 3 in
// fragment 1) make 1.2x the useful products (the super-pixel form's 12 of 16
// rows and 49 of 64 taps make 1.74x).
//
// Rolling rows.  G row gy adds to output super-row Y = gy + 1 - dy, and dy is
// the accumulator register (D layout: lane l, register v holds row
// 4(l/16) + v), so register v of a fragment accumulates output row gy + 1 - v.
// After G row gy, register 3 (row gy - 2) has all four of its G rows: it is
// stored, and the registers shift one place (3 <- 2 <- 1 <- 0 <- 0) for G row
// gy + 1.  Every output value is summed in the accumulators and written once;
// no partial sum goes through memory or LDS.
//
// The filter is held in registers for the whole kernel (176 values a lane,
// gathered once into an LDS table in fragment order); G comes straight from memory, lane X reading G
// columns X-1 .. X+2 of four channels per k-step, PF k-steps ahead, with
// out-of-map columns read as zero by the buffer range check.  The loop has no
// LDS access and no barrier.
//
// Work.  Super-rows are flattened over images (row n*OH + Y); band b is rows
// [b*rows, (b+1)*rows) of column tile t, one wave each (wave index b*T + t,
// the bands of one XCD consecutive).
// A band that crosses an image boundary is two segments; a segment of output
// rows [Ya, Yb) walks G rows Ya-1 .. Yb+1 (those inside the map), so each
// segment recomputes at most three G rows of its neighbours.
//
// Non-finite data: a padded or absent tap is a zero operand here, which the
// reference never multiplies (0 * Inf would be NaN).  An output whose sum is
// not finite is recomputed over the reference's visited taps (exact.hpp)
// before it is stored; finite sums are unaffected.
#pragma once

#include "direct.hpp"

namespace katsu {

struct StemDxArgs {
    const float *g, *w;
    float *dx;
    int N, H, W, OH, OW;
    int tiles;   // cdiv(OW, 16): column tiles of 16 super-columns
    int bands;   // cdiv(N*OH, rows)
    int rows;    // flattened super-rows per band
    int wpx;     // waves per XCD: cdiv(bands, 8) * tiles
    uint32_t g_bytes, dx_bytes;
    float beta;
};

constexpr int kStemDxK = 64, kStemDxC = 3;

// A row that holds a non-finite value: every element stored as the fast
// path would store it, except that a non-finite one is first recomputed over
// the reference's visited taps.  Out of line: taken only for non-finite
// data, and a call keeps the recomputation's loops out of the MFMA loop.
__device__ __noinline__ void stem_dx_put_exact(const float *g, const float *w, float *dx, int H,
                                               int W, int OH, int OW, float beta, int n, int Y,
                                               int X, int kq, float v0, float v1, float v2) {
    const float *g_img = g + (int64_t)n * kStemDxK * OH * OW;
    float *dst = dx + (int64_t)n * kStemDxC * H * W;
    for (int f = 0; f < 3; ++f) {
        float v = f == 0 ? v0 : (f == 1 ? v1 : v2);
        const int j = 4 * f + kq, px = j / 6, c = (j % 6) / 2, py = j & 1;
        const int iy = 2 * Y + py, ix = 2 * X + px;
        if (ix >= W || iy >= H) continue;
        if (!__builtin_isfinite(v))
            v = exact_dx_inl(g_img, w, kStemDxK, kStemDxC, OH, OW, 7, 7, 2, 3, c, iy, ix);
        store_beta(dst + ((int64_t)c * H + iy) * W + ix, v, beta);
    }
}

template <int PF, int OCC>
__global__ void __launch_bounds__(256, OCC) stem_dx_kernel(const StemDxArgs a) {
    constexpr int KG = kStemDxK / 4;  // k-steps of a G row
    static_assert(KG % PF == 0, "prefetch ring divides the k-steps");
    // The A fragments laid out in LDS as the lanes read them: entry
    // ((f*KG + kg)*4 + dx)*64 + lane.  Each thread gathers its 48 entries
    // from w with every load in flight at once (a load-store loop would pay
    // one load latency per entry), then each wave reads its 176 values at
    // consecutive addresses.
    extern __shared__ float at[];
    {
        constexpr int NE = 3 * KG * 4 * 64 / 256;
        float v[NE];
#pragma unroll
        for (int e = 0; e < NE; ++e) {
            const int entry = e * 256 + (int)threadIdx.x;
            const int l = entry & 63, d = (entry >> 6) & 3, kg = (entry >> 8) % KG,
                      f = (entry >> 8) / KG;
            const int i = l & 15, kk = l >> 4, q = i >> 2, dy = i & 3;
            const int j = 4 * f + q, px = j / 6, c = (j % 6) / 2, py = j & 1;
            const int r = py ? 6 - 2 * dy : 5 - 2 * dy, sx = px ? 6 - 2 * d : 5 - 2 * d;
            v[e] = (r >= 0 && sx >= 0)
                       ? a.w[(((4 * kg + kk) * kStemDxC + c) * 7 + r) * 7 + sx]
                       : 0.f;
        }
#pragma unroll
        for (int e = 0; e < NE; ++e) at[e * 256 + threadIdx.x] = v[e];
    }
    __syncthreads();

    const int lane = threadIdx.x & 63;
    // Blocks go to the 8 XCDs in turn (block b to XCD b % 8); XCD x takes
    // waves [x*wpx, (x+1)*wpx), whole bands, so the column tiles of a band,
    // which read overlapping G lines at the same time, share one L2.  The
    // wave index is made wave-uniform for the compiler (the band's offsets
    // are then scalars, as the loads' soffset operand needs).
    const int local = (blockIdx.x >> 3) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (local >= a.wpx) return;
    const int gw = (blockIdx.x & 7) * a.wpx + local;
    const int band = gw / a.tiles, t = gw - band * a.tiles;
    if (band >= a.bands) return;

    // A fragments: lane l holds A[i = l%16][k = l/16], row i = 4q + dy.
    float A[3][KG][4];
#pragma unroll
    for (int f = 0; f < 3; ++f)
#pragma unroll
        for (int kg = 0; kg < KG; ++kg)
#pragma unroll
            for (int d = 0; d < 4; ++d)
                if (f > 0 || d < 3) A[f][kg][d] = at[((f * KG + kg) * 4 + d) * 64 + lane];

    const int OHW = a.OH * a.OW;
    const int X0 = 16 * t, X = X0 + (lane & 15), kq = lane >> 4;
    // B loads: lane part of the byte offset per dx (kOOB outside the row).
    int vo[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const int col = X + d - 1;
        vo[d] = (unsigned)col < (unsigned)a.OW ? (kq * OHW + col) * 4 : kOOB;
    }
    const auto rs = buf_rsrc(a.g, a.g_bytes);
    const int kgs = 16 * OHW;  // bytes between k-steps (4 channels)
    // Stores: lane l, register 3 of fragment f is combination 4f + l/16 at
    // super-column X: buffer stores whose lane part of the offset is kOOB
    // for a column past the image (dropped by the range check), so a row is
    // always three stores and no branch.
    const auto rd = buf_rsrc(a.dx, a.dx_bytes);
    int sv[3], spy[3];
#pragma unroll
    for (int f = 0; f < 3; ++f) {
        const int j = 4 * f + kq, px = j / 6, c = (j % 6) / 2, py = j & 1;
        const int ix = 2 * X + px;
        sv[f] = ix < a.W ? ((c * a.H + py) * a.W + ix) * 4 : kOOB;
        spy[f] = py;
    }
    // A row's store offsets: output row Y of image n, nothing stored (every
    // lane kOOB) for ok = false, a row outside the segment.
    struct RowAt {
        int off[3], so;
    };
    auto row_at = [&](int n, int Y, bool ok) {
        RowAt r;
        const int Ys = max(Y, 0);
        r.so = (n * kStemDxC * a.H + 2 * Ys) * a.W * 4;
#pragma unroll
        for (int f = 0; f < 3; ++f) r.off[f] = (ok && 2 * Ys + spy[f] < a.H) ? sv[f] : kOOB;
        return r;
    };
    // dx's present values where beta = 1; zeros (kOOB: no memory read) for
    // beta = 0, whose output is never read.
    const int boob = a.beta != 0.f ? 0 : kOOB;
    auto load_old = [&](const RowAt &r, float *o) {
#pragma unroll
        for (int f = 0; f < 3; ++f)
            o[f] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(rd, r.off[f] | boob, r.so, 0));
    };
    // The sum of an output is summed from +0, so it is never -0 and 0 + v
    // is v: beta = 0 and beta = 1 share the add.
    auto store_row = [&](int n, int Y, const RowAt &r, const float *o, float v0, float v1,
                         float v2) {
        const float v[3] = {v0, v1, v2};
        bool bad = false;
#pragma unroll
        for (int f = 0; f < 3; ++f) bad |= r.off[f] != kOOB && !__builtin_isfinite(v[f]);
        if (__builtin_amdgcn_ballot_w64(bad)) {
            stem_dx_put_exact(a.g, a.w, a.dx, a.H, a.W, a.OH, a.OW, a.beta, n, Y, X, kq, v0, v1,
                              v2);
            return;
        }
#pragma unroll
        for (int f = 0; f < 3; ++f)
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, o[f] + v[f]), rd,
                                                  r.off[f], r.so, 0);
    };

    const int total = a.N * a.OH;
    int rho = band * a.rows;
    const int rho1 = min(rho + a.rows, total);
    while (rho < rho1) {
        const int n = rho / a.OH, Ya = rho - n * a.OH;
        const int Yb = min(a.OH, Ya + (rho1 - rho));
        rho += Yb - Ya;
        const int g0 = max(Ya - 1, 0), g1 = min(Yb + 2, a.OH);
        // Uniform byte offset of (image n, k-step 0, row gy).
        int so = (n * kStemDxK * a.OH + g0) * a.OW * 4;
        floatx4 acc[3];
#pragma unroll
        for (int f = 0; f < 3; ++f) acc[f] = floatx4{0.f, 0.f, 0.f, 0.f};
        float b[PF][4];
#pragma unroll
        for (int p = 0; p < PF; ++p)
#pragma unroll
            for (int d = 0; d < 4; ++d)
                b[p][d] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(rs, vo[d], so + p * kgs, 0));
        // The first k-steps are waited for here, once per segment, so that
        // at the row loop's head only the loads of the loop itself are
        // pending (each k-step then waits just for its own operands).
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        for (int gy = g0; gy < g1; ++gy, so += a.OW * 4) {
            // The next G row, or this one again after the segment's last
            // row (those loads are discarded): every load of an in-map
            // column stays inside G.
            const int nrow = gy + 1 < g1 ? a.OW * 4 : 0;
            // The row this G row completes, and its present values, loaded
            // now so that they arrive while the row computes.
            const RowAt ra = row_at(n, gy - 2, gy - 2 >= Ya);
            float old[3];
            load_old(ra, old);
            __builtin_amdgcn_sched_group_barrier(0x020, 3, 0);
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) {
                float cur[4];
#pragma unroll
                for (int d = 0; d < 4; ++d) cur[d] = b[kg % PF][d];
                // The ring slot refills with k-step kg + PF.
                const int nso = kg + PF < KG ? so + (kg + PF) * kgs
                                             : so + nrow + (kg + PF - KG) * kgs;
#pragma unroll
                for (int d = 0; d < 4; ++d)
                    b[kg % PF][d] = __builtin_bit_cast(
                        float, __builtin_amdgcn_raw_buffer_load_b32(rs, vo[d], nso, 0));
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    if (d < 3)
                        acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(A[0][kg][d], cur[d], acc[0],
                                                                      0, 0, 0);
                    acc[1] =
                        __builtin_amdgcn_mfma_f32_16x16x4f32(A[1][kg][d], cur[d], acc[1], 0, 0, 0);
                    acc[2] =
                        __builtin_amdgcn_mfma_f32_16x16x4f32(A[2][kg][d], cur[d], acc[2], 0, 0, 0);
                }
                // Keep each step's refill loads with its MFMAs (the scheduler
                // otherwise sinks them, shortening the prefetch distance).
                __builtin_amdgcn_sched_group_barrier(0x020, 4, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 11, 0);
            }
            store_row(n, gy - 2, ra, old, acc[0][3], acc[1][3], acc[2][3]);
#pragma unroll
            for (int f = 0; f < 3; ++f)
                acc[f] = floatx4{0.f, acc[f][0], acc[f][1], acc[f][2]};
        }
        // Rows the map's last G rows completed: g1 - 2 (register 3) and
        // g1 - 1 (register 2), when they belong to the segment.
        {
            const RowAt r2 = row_at(n, g1 - 2, g1 - 2 >= Ya && g1 - 2 < Yb);
            const RowAt r1 = row_at(n, g1 - 1, g1 - 1 >= Ya && g1 - 1 < Yb);
            float o2[3], o1[3];
            load_old(r2, o2);
            load_old(r1, o1);
            store_row(n, g1 - 2, r2, o2, acc[0][3], acc[1][3], acc[2][3]);
            store_row(n, g1 - 1, r1, o1, acc[0][2], acc[1][2], acc[2][2]);
        }
    }
}

}  // namespace katsu
