// smallc.hpp -- the forward of convolutions with three input channels and a
// 7x7 filter, any stride and padding (the stem layer of config 5):
// Conv2D::forward (conv2d.rs:95-115), y = sum over (c, r, s) of
// w[o][c][r][s] * x[c][oy*st - pad + r][ox*st - pad + s].
//
// GEMM view: i = output channel (64 per block), j = output pixel (one image
// row per step), k = (c, r, s) in the filter's own order, padded from 147 to
// 148.  k-step t takes k = 4t .. 4t+3, lane group lg (lanes 16lg..16lg+15)
// taking k = 4t + lg; the lane's halo offset of that tap is a per-lane
// register (the four taps of a step can straddle filter rows), so a B read is
// the lane's pixel column plus that offset.  37 k-steps per row: the padding
// costs 148/147 of the MFMAs (s padded to 8 would cost 8/7, three channels in
// quads, as the general direct kernel stages them, 4/3).
//
// A block is 512 threads: two groups of four waves that share the filter in
// LDS (64 x 148 floats, staged once) and each walk their own output rows
// (group g takes rows r0 + g, r0 + g + 2, ...) through a double-buffered
// halo of 7 input rows per channel.  Wave q of a group owns output channels
// 16q .. 16q+15 and the whole row (F fragments of 16 pixels).  A row's output
// is stored straight from the accumulators after the barrier that ends its
// step, so the stores drain while the next row computes.
#pragma once

#include "direct.hpp"

namespace katsu {

struct StemArgs {
    const float *x, *w;
    float *y;
    int N, C, H, W, K, OH, OW, st, pad;
    int64_t x_img, y_img;  // C*H*W, K*OH*OW
    int rows_per_block;    // even: the two groups take alternate rows
    int blocks_img;        // cdiv(OH, rows_per_block)
    int co_blocks;         // cdiv(K, 64)
    int ncols;             // (OW - 1)*st + S: halo columns (<= PITCH)
    uint32_t w_bytes;
};

template <int CC, int R, int S, int PITCH>
struct StemGeo {
    static constexpr int CRS = CC * R * S;
    static constexpr int WK = (CRS + 3) / 4 * 4;  // k extent of a filter row: (c, r, s) flat
    static constexpr int WP = WK + 2;            // == 2 (mod 4): a half-wave's A reads on 32 banks
    static constexpr int WS = (64 * WP + 255) / 256 * 256;
    static constexpr int CP = R * PITCH;         // halo channel pitch
    static constexpr int HS = CC * CP;           // one halo stage
    static constexpr int TOTAL = WS + 4 * HS;    // filter + two groups x two stages
    static constexpr size_t kBytes = (size_t)TOTAL * sizeof(float);
    static_assert(PITCH % 64 == 0, "stem geometry");
};

template <int CC, int R, int S, int F, int PITCH, int ST>
__global__ void __launch_bounds__(512, 1) stem_fwd_kernel(const StemArgs a) {
    static_assert((16 * F - 1) * ST + S <= PITCH, "every lane's taps inside its halo row");
    using Geo = StemGeo<CC, R, S, PITCH>;
    constexpr int CRS = Geo::CRS;
    constexpr int NK = Geo::WK / 4;  // k-steps of a row
    constexpr int LPR = PITCH / 64;

    extern __shared__ float smem[];
    const int tid = threadIdx.x;
    const int grp = tid >> 8, wq = (tid >> 6) & 3, lane = tid & 63;
    const int l16 = lane & 15, lg = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index in the block

    const int b = blockIdx.x;
    const int cb = b % a.co_blocks;
    const int rest = b / a.co_blocks;
    const int n = rest / a.blocks_img;
    const int r0 = (rest - n * a.blocks_img) * a.rows_per_block;
    const int co0 = cb * 64;
    const int nsteps = a.rows_per_block / 2;  // rows per group

    float *ws = smem;
    float *hs0 = smem + Geo::WS + grp * 2 * Geo::HS;
    float *hs1 = hs0 + Geo::HS;

    const __amdgpu_buffer_rsrc_t rx =
        buf_rsrc(a.x + (int64_t)n * a.x_img, (uint32_t)(a.x_img * 4));
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(a.w, a.w_bytes);

    // The filter: row o of the LDS copy holds w[co0 + o] as stored, k =
    // (c*R + r)*S + s, zeros for k >= C*R*S and for channels past K.
    {
        constexpr int NI = Geo::WS / 64;
        for (int i = wv; i < NI; i += 8) {
            const int e = i * 64 + lane;
            const int row = e / Geo::WP, col = e - (e / Geo::WP) * Geo::WP;
            const int co = co0 + row;
            const bool ok = row < 64 && co < a.K && col < CRS;
            lds_dma_b32(rw, ws + i * 64, ok ? (co * CRS + col) * 4 : kOOB);
        }
    }
    // Halo of output row oy: channel c, row r, column col at c*CP + r*PITCH +
    // col; image column col - pad, zeros outside the image (and for rows past
    // the output, whose results are not stored).  Wave q of a group stages
    // columns 64q .. 64q+63 of every (c, r) row: one LDS-direct load each,
    // with the lane's column offset fixed and the row offsets compile-time.
    static_assert(LPR == 4, "one 64-column chunk per wave of a group");
    const int q = wv & 3;
    int colq;
    {
        const int col = q * 64 + lane;
        const int ix = col - a.pad;
        colq = (col < a.ncols && (unsigned)ix < (unsigned)a.W) ? ix * 4 : kOOB;
    }
    const int rowbytes = a.W * 4, chanbytes = a.H * a.W * 4;
    auto stage = [&](float *hs, int oy) __attribute__((always_inline)) {
        const int iy0 = oy * a.st - a.pad;
        const bool rowok = oy < a.OH;
#pragma unroll
        for (int c = 0; c < CC; ++c)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int iy = iy0 + r;
                const bool ok = rowok && (unsigned)iy < (unsigned)a.H;
                // colq may be kOOB: kOOB plus a row offset (< 1 GiB) stays out of range.
                lds_dma_b32(rx, hs + c * Geo::CP + r * PITCH + q * 64,
                            ok ? c * chanbytes + iy * rowbytes + colq : kOOB);
            }
    };

    // Per-lane bases.  k-step t takes k = 4t + lg: B reads the halo at the
    // lane's pixel column plus the tap's offset toff[t] (per lane: the four
    // lane groups' taps straddle filter rows); the padding k >= C*R*S reads
    // tap 0, times a zero weight.  A reads the lane's output channel row at
    // 4t + lg.
    // Fragment f adds the constant 16 f ST; lanes past the row's end read
    // inside the halo row (the pitch holds all 16 F columns) and are not
    // stored.
    const int pix0 = l16 * ST;
    int toff[NK];
#pragma unroll
    for (int t = 0; t < NK; ++t) {
        const int k = 4 * t + lg;
        const int c = k / (R * S), rs = k - c * (R * S), r = rs / S, sx = rs - r * S;
        toff[t] = k < CRS ? c * Geo::CP + r * PITCH + sx : 0;
    }
    const int abase = (wq * 16 + l16) * Geo::WP + lg;

    floatx4 acc[F];
#pragma unroll
    for (int f = 0; f < F; ++f) acc[f] = floatx4{0.f, 0.f, 0.f, 0.f};

    auto fetch = [&](const float *hs, const int kk, float (&bv)[F], float &av)
        __attribute__((always_inline)) {
        av = ws[abase + 4 * kk];
        const float *hb = hs + pix0 + toff[kk];
#pragma unroll
        for (int f = 0; f < F; ++f) bv[f] = hb[16 * f * ST];
    };
    auto mma = [&](const float (&bv)[F], const float av) __attribute__((always_inline)) {
#pragma unroll
        for (int f = 0; f < F; ++f)
            acc[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv[f], acc[f], 0, 0, 0);
    };
    auto compute = [&](const float *hs) __attribute__((always_inline)) {
        float b0[F], b1[F];
        float a0, a1;
        fetch(hs, 0, b0, a0);
        asm volatile("" ::: "memory");
#pragma unroll
        for (int kk = 0; kk < NK; kk += 2) {
            if (kk + 1 < NK) fetch(hs, kk + 1, b1, a1);
            mma(b0, a0);
            order_reads_then_mfma<F + 1, F>();
            if (kk + 2 < NK) fetch(hs, kk + 2, b0, a0);
            if (kk + 1 < NK) mma(b1, a1);
            order_reads_then_mfma<F + 1, F>();
        }
    };
    // Fragment f, register v: output channel 4*lg + v of the wave's 16,
    // pixel 16f + l16 of the row.  A non-finite sum may hold a product the
    // reference skips (the zero weight of a padding k times real x, or a
    // weight times the halo's padding): the lane notes it, and after the last row
    // re-reads its own outputs and recomputes the non-finite ones over the
    // visited products (exact.hpp), keeping that code out of the row loop.
    float *ybase = a.y + (int64_t)n * a.y_img;
    bool held = false;
    auto store_row = [&](int oy) __attribute__((always_inline)) {
        if (oy < a.OH) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int co = co0 + wq * 16 + 4 * lg + v;
                if (co >= a.K) continue;
                float *yrow = ybase + ((int64_t)co * a.OH + oy) * a.OW;
#pragma unroll
                for (int f = 0; f < F; ++f) {
                    const int ox = f * 16 + l16;
                    if (ox < a.OW) {
                        held |= !__builtin_isfinite(acc[f][v]);
                        yrow[ox] = acc[f][v];
                    }
                }
            }
        }
#pragma unroll
        for (int f = 0; f < F; ++f) acc[f] = floatx4{0.f, 0.f, 0.f, 0.f};
    };

    // Rows of this group: r0 + grp + 2t, t < nsteps.  Both groups run every
    // step (a row past the image computes on zeros and stores nothing), so
    // the block's barriers stay matched.
    stage(hs0, r0 + grp);
    wait_lds_dma();
    __syncthreads();
    for (int t = 0; t < nsteps; t += 2) {
        const int oy = r0 + grp + 2 * t;
        if (t + 1 < nsteps) stage(hs1, oy + 2);
        compute(hs0);
        wait_lds_dma();
        __syncthreads();
        store_row(oy);
        if (t + 1 >= nsteps) break;
        if (t + 2 < nsteps) stage(hs0, oy + 4);
        compute(hs1);
        wait_lds_dma();
        __syncthreads();
        store_row(oy + 2);
    }
    if (held) {
        for (int t = 0; t < nsteps; ++t) {
            const int oy = r0 + grp + 2 * t;
            if (oy >= a.OH) break;
            for (int v = 0; v < 4; ++v) {
                const int co = co0 + wq * 16 + 4 * lg + v;
                if (co >= a.K) continue;
                float *yrow = ybase + ((int64_t)co * a.OH + oy) * a.OW;
                for (int f = 0; f < F; ++f) {
                    const int ox = f * 16 + l16;
                    if (ox < a.OW && !__builtin_isfinite(yrow[ox]))
                        yrow[ox] = exact_fwd_inl(a.x + (int64_t)n * a.x_img, a.w, a.C, a.H, a.W, R, S,
                                             a.st, a.pad, co, oy, ox);
                }
            }
        }
    }
}

}  // namespace katsu

namespace katsu {

// ---------------------------------------------------------------------------
// The filter gradient of the same layers (backward_buffers, conv2d.rs:289):
// dw[o][c][r][s] = sum over (n, oy, ox) of G[n][o][oy][ox] *
// x[n][c][oy*ST - pad + r][ox*ST - pad + s].
//
// GEMM view: i = o (64 per block), j = (c, r, s) in the filter's own order
// (C*R*S = 147 columns, padded to 160), k = output pixel.  A tile is 56
// output pixels of one row (TW); a k-step takes four of them, lane group lg
// taking pixel 4t + lg.  Wave (wm, wn) owns channels 32wm..32wm+31 and
// columns 80wn..80wn+79: 2 A and 5 B fragments, 10 MFMAs per k-step.  A
// lane's B address is a per-lane base (its column's (c, r, s) offset in the
// halo plus lg*ST) plus 4t*ST; its A address a per-lane base plus 4t.
//
// A block (four waves, two per CU) walks a contiguous range of tiles
// through double-buffered stages of G (64 rows of 56, pitch 58) and the x
// halo (3 channels x 7 rows of 128 columns, pitch 136), all staged by
// LDS-direct loads, and writes one partial dw[o][c*R*S] slice; the slices
// are summed by dw_split_reduce in a fixed order.  The blocks sharing a CU
// run out of phase, so one's staging overlaps the other's MFMAs.
struct StemDwArgs {
    const float *x, *g;
    float *part;          // partial slices [split][K][C*R*S], pitch pstride
    int N, C, H, W, K, OH, OW, pad;
    int64_t x_img, g_img;  // C*H*W, K*OH*OW
    int tiles_row;         // cdiv(OW, TW)
    int tiles_total;       // N*OH*tiles_row
    int tiles_per_block;
    int co_blocks;
    int64_t pstride;
};

template <int CC, int R, int S>
struct StemDwGeo {
    static constexpr int TW = 56;               // output pixels per tile
    static constexpr int GP = TW + 2;           // == 2 (mod 4): A reads on 32 banks per half-wave
    static constexpr int GS = 64 * GP;          // G stage
    static constexpr int XP = 136;              // halo row pitch (128 staged columns)
    static constexpr int CPX = R * XP;          // halo channel pitch
    static constexpr int XS = CC * CPX;         // halo stage
    static constexpr int STAGE = GS + XS;
    static constexpr size_t kBytes = 2 * (size_t)STAGE * sizeof(float);
    static constexpr int NCOL = CC * R * S;     // filter columns
    static_assert(NCOL <= 160, "five 16-column fragments per wave half");
};

template <int CC, int R, int S, int ST>
__global__ void __launch_bounds__(256, 2) stem_dw_kernel(const StemDwArgs a) {
    using Geo = StemDwGeo<CC, R, S>;
    constexpr int TW = Geo::TW;
    constexpr int NT = TW / 4;  // k-steps per tile
    static_assert((TW - 1) * ST + S <= 128, "halo columns of a tile fit the staged 128");

    extern __shared__ float smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int l16 = lane & 15, lg = lane >> 4;
    const int wq = __builtin_amdgcn_readfirstlane(tid >> 6), wm = wq & 1, wn = wq >> 1;

    const int b = blockIdx.x;
    const int cb = b % a.co_blocks;
    const int split = b / a.co_blocks;
    const int co0 = cb * 64;
    const int tb = split * a.tiles_per_block;
    const int te = min(tb + a.tiles_per_block, a.tiles_total);

    float *st0 = smem;
    float *st1 = smem + Geo::STAGE;

    // Tile coordinates, advanced one tile at a time: image n, row oy,
    // first pixel x0 of the row.
    struct Pos { int n, oy, x0; };
    auto advance = [&](Pos p) __attribute__((always_inline)) {
        p.x0 += TW;
        if (p.x0 >= a.tiles_row * TW) {
            p.x0 = 0;
            if (++p.oy == a.OH) {
                p.oy = 0;
                ++p.n;
            }
        }
        return p;
    };
    Pos p0;
    {
        const int rowi = tb / a.tiles_row;
        p0.n = rowi / a.OH;
        p0.oy = rowi - p0.n * a.OH;
        p0.x0 = (tb - rowi * a.tiles_row) * TW;
    }

    // Staging of the tile at p (nothing but zeros when ok is false): G rows
    // o of pixels [x0, x0+56) of row oy; halo rows oy*ST - pad + r, columns
    // x0*ST - pad + col, col < 128.
    auto stage = [&](float *stg, const Pos &p, bool tok) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rg =
            buf_rsrc(a.g + (int64_t)p.n * a.g_img, (uint32_t)(a.g_img * 4));
        const __amdgpu_buffer_rsrc_t rx =
            buf_rsrc(a.x + (int64_t)p.n * a.x_img, (uint32_t)(a.x_img * 4));
        // G: 16 rows per wave; lanes past the 56 columns idle.
        const int px = p.x0 + lane;
        const bool pok = tok && px < a.OW;
        const int gb = (co0 * a.OH + p.oy) * a.OW + px;
        const int gstep = a.OH * a.OW;
        if (lane < TW) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int o = wq * 16 + i;
                const bool ok = pok && co0 + o < a.K;
                lds_dma_b32(rg, stg + o * Geo::GP, ok ? (gb + o * gstep) * 4 : kOOB);
            }
        }
        // Halo: wave q stages column chunk q & 1 of the (c, r) rows with
        // index parity q >> 1.
        const int col = (wq & 1) * 64 + lane;
        const int ix = p.x0 * ST - a.pad + col;
        const int colb = (tok && (unsigned)ix < (unsigned)a.W) ? ix * 4 : kOOB;
        const int iy0 = p.oy * ST - a.pad;
        float *xs = stg + Geo::GS + (wq & 1) * 64;
#pragma unroll
        for (int i = 0; i < CC * R; ++i) {
            if ((i & 1) != (wq >> 1)) continue;
            const int c = i / R, r = i - (i / R) * R;
            const int iy = iy0 + r;
            const bool ok = (unsigned)iy < (unsigned)a.H;
            // colb may be kOOB: kOOB plus a row offset (< 1 GiB) stays out of range.
            lds_dma_b32(rx, xs + c * Geo::CPX + r * Geo::XP,
                        ok ? (c * a.H + iy) * a.W * 4 + colb : kOOB);
        }
    };

    // Per-lane bases.  B column j = 80wn + 16f + l16 is (c, r, s) of the
    // filter; padding columns (j >= C*R*S) read column 0 and are not stored.
    int boff[5];
#pragma unroll
    for (int f = 0; f < 5; ++f) {
        int j = wn * 80 + f * 16 + l16;
        j = j < Geo::NCOL ? j : 0;
        const int c = j / (R * S), rs = j - c * (R * S);
        const int r = rs / S, s = rs - r * S;
        boff[f] = Geo::GS + c * Geo::CPX + r * Geo::XP + s + lg * ST;
    }
    const int abase = (wm * 32 + l16) * Geo::GP + lg;

    floatx4 acc[2][5];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int f = 0; f < 5; ++f) acc[i][f] = floatx4{0.f, 0.f, 0.f, 0.f};

    auto fetch = [&](const float *stg, int t, float (&av)[2], float (&bv)[5])
        __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; ++i) av[i] = stg[abase + i * 16 * Geo::GP + 4 * t];
#pragma unroll
        for (int f = 0; f < 5; ++f) bv[f] = stg[boff[f] + 4 * t * ST];
    };
    auto mma = [&](const float (&av)[2], const float (&bv)[5]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int f = 0; f < 5; ++f)
                acc[i][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[f], acc[i][f], 0, 0, 0);
    };
    auto compute = [&](const float *stg) __attribute__((always_inline)) {
        float a0[2], a1[2], b0[5], b1[5];
        fetch(stg, 0, a0, b0);
        asm volatile("" ::: "memory");
#pragma unroll
        for (int t = 0; t < NT; t += 2) {
            if (t + 1 < NT) fetch(stg, t + 1, a1, b1);
            mma(a0, b0);
            order_reads_then_mfma<7, 10>();
            if (t + 2 < NT) fetch(stg, t + 2, a0, b0);
            if (t + 1 < NT) mma(a1, b1);
            order_reads_then_mfma<7, 10>();
        }
    };

    if (tb < te) {
        Pos cur = p0;
        stage(st0, cur, true);
        wait_lds_dma();
        __syncthreads();
        for (int tile = tb; tile < te; tile += 2) {
            Pos nxt = advance(cur);
            if (tile + 1 < te) stage(st1, nxt, true);
            compute(st0);
            wait_lds_dma();
            __syncthreads();
            if (tile + 1 >= te) break;
            cur = advance(nxt);
            if (tile + 2 < te) stage(st0, cur, true);
            compute(st1);
            wait_lds_dma();
            __syncthreads();
        }
    }

    // D layout: fragment (i, f), register v is channel wm*32 + 16i + 4lg + v,
    // column 80wn + 16f + l16.  A non-finite partial may hold a product the
    // reference skips (G times the halo's padding, or a zeroed G column past
    // the row end times real x): it is recomputed over the block's pixels,
    // one contiguous range of the batch (exact.hpp).
    float *part = a.part + (int64_t)split * a.pstride;
    auto fix = [&](float v, int o, int j) __attribute__((always_inline)) {
        if (__builtin_isfinite(v) || tb >= te) return v;
        const int rb = tb / a.tiles_row, re = (te - 1) / a.tiles_row;
        const int64_t pbeg = (int64_t)rb * a.OW + (tb - rb * a.tiles_row) * TW;
        const int64_t pend =
            (int64_t)re * a.OW + min(((te - 1) - re * a.tiles_row) * TW + TW, a.OW);
        const int c = j / (R * S), rs = j - c * (R * S);
        return exact_dw_inl(a.x, a.g, a.C, a.H, a.W, a.K, a.OH, a.OW, ST, a.pad, o, c, rs / S, rs % S,
                        pbeg, pend);
    };
#pragma unroll
    for (int f = 0; f < 5; ++f) {
        const int j = wn * 80 + f * 16 + l16;
        if (j >= Geo::NCOL) continue;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int o = wm * 32 + i * 16 + 4 * lg + v;
                if (co0 + o < a.K)
                    part[(int64_t)(co0 + o) * Geo::NCOL + j] = fix(acc[i][f][v], co0 + o, j);
            }
    }
}

}  // namespace katsu
