// direct.hpp -- direct (halo-tile) convolution kernels for gfx950.
//
// These kernels cover the convolution passes whose input rows fit an LDS
// halo tile.  Unlike the generic implicit-GEMM engine (igemm.hpp), which
// gathers every im2col element with its own index arithmetic, a block here
// stages whole input rows once -- a [channels][rows][64*CC] tile with the
// zero padding materialised in LDS -- and every one of the R*S taps reads
// that tile at a per-lane offset computed once per block plus a tap offset.
// The tile geometry (row pitch 64*CC, ROWS rows per channel) is a template
// parameter, so every tap, channel and pipeline-stage offset is an LDS
// instruction immediate: the MFMA loop is LDS reads and MFMAs only.
//
// Global loads go through buffer resources: a lane whose element lies in the
// padding or past a tensor edge gets an out-of-range offset and reads zero,
// so staging has no branches.  Tiles are staged by LDS-direct loads; weight
// rows are fetched 16 bytes per lane when the host has checked their
// alignment (WVEC).
// Block outputs are transposed through LDS and written as contiguous
// 16-byte runs.
//
//   direct_fwd_kernel   out[n][co][p] = sum_{ci,r,s} in[n][ci][tap(p,r,s)] * w'(co,ci,r,s)
//                       forward (WMODE 0: w' = w) and, for stride 1, the
//                       data gradient (WMODE 1: in = G, w' = w transposed
//                       and flipped)
//   direct_dw_kernel    dw partials over a range of output pixels
//   dw_split_reduce     fixed-order sum of the dw partials
//
// MFMA v_mfma_f32_16x16x4_f32 lane layout (wave64), as in igemm.hpp:
//   A: lane l holds A[i = l%16][k = l/16]; B: lane l holds B[k = l/16][j = l%16]
//   D: lane l, register v holds D[i = 4*(l/16) + v][j = l%16]
#pragma once

#include "exact.hpp"
#include "igemm.hpp"

namespace katsu {

// Wave-group forward blocks (KG > 1) read the fragments of k-step kk+1
// during step kk's MFMAs when they have at most this many fragments per
// wave, else one step at a time.
#ifndef KATSU_FWD_KG_PIPE_F
#define KATSU_FWD_KG_PIPE_F 8
#endif

// Scheduling fence for a software-pipelined k-step: the LDS reads of the
// next step (NREAD of them) are issued before the MFMAs of the current step
// (NMFMA), so the reads' latency overlaps the MFMAs.  Without it the
// scheduler tends to issue the reads after the MFMAs, and the next step then
// stalls on them.  The empty asm with a memory clobber keeps the load/store
// optimizer from fusing reads of different steps into one ds_read2, which
// would pull a read into the step that consumes it.
template <int NREAD, int NMFMA>
__device__ __forceinline__ void order_reads_then_mfma() {
    __builtin_amdgcn_sched_group_barrier(0x100, NREAD, 0);  // DS reads
    __builtin_amdgcn_sched_group_barrier(0x008, NMFMA, 0);  // MFMA
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
}
// The same with nv LDS-direct loads of the next stage issued first (nv is a
// constant after unrolling, at most 4).
template <int NREAD, int NMFMA>
__device__ __forceinline__ void order_step(int nv) {
    if (nv == 0) {
        order_reads_then_mfma<NREAD, NMFMA>();
        return;
    }
    if (nv == 1) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM reads
    if (nv == 2) __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);
    if (nv == 3) __builtin_amdgcn_sched_group_barrier(0x020, 3, 0);
    if (nv >= 4) __builtin_amdgcn_sched_group_barrier(0x020, 4, 0);
    order_reads_then_mfma<NREAD, NMFMA>();
}

// ---------------------------------------------------------------------------
// Buffer-resource loads.  Range checking of a raw buffer (stride 0) returns
// zero for any byte offset >= the resource size, so `kOOB` (with resources
// kept below 1 GiB by the host) turns a load into a zero without a branch.
constexpr int kOOB = 0x40000000;
constexpr uint32_t kMaxBufBytes = 0x40000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const float *p, uint32_t bytes) {
    // 0x00020000: the gfx9 data-format word of an untyped 32-bit buffer.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p), (short)0, (int)bytes,
                                             0x00020000);
}
__device__ __forceinline__ float buf_load(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ floatx4 buf_load4(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// LDS-direct buffer loads: lane l's 4 (or 16) bytes land at dst + 4*l (or
// 16*l) without passing through registers; an out-of-range lane writes zeros.
// dst must be uniform across the wave.  Completion is tracked by vmcnt, so a
// stage written this way is waited for with wait_lds_dma() before the barrier
// that publishes it.
typedef __attribute__((address_space(3))) void lds_void;
__device__ __forceinline__ void lds_dma_b32(__amdgpu_buffer_rsrc_t r, float *dst, int off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)dst, 4, off, 0, 0, 0);
}
__device__ __forceinline__ void lds_dma_b128(__amdgpu_buffer_rsrc_t r, float *dst, int off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)dst, 16, off, 0, 0, 0);
}
__device__ __forceinline__ void wait_lds_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }


// ---------------------------------------------------------------------------
// Forward / data-gradient kernel.
//
// GEMM view per block: i = output channel (KT of them), j = output pixel
// (a contiguous range of one image), k = (input channel, tap).  Waves split
// the KT channels into 16-row slices and the pixel range into WPX parts of
// F fragments of 16 pixels each.  Input channels are consumed CB at a time
// through a two-stage LDS pipeline.
//
// Four weight modes (WMODE) make the same kernel serve four problems:
//   0  forward:  w' = w[CO][CI][R][S] as stored
//   1  dX, stride 1: in = G, w'[co][ci][r][s] = w[ci][co][R-1-r][S-1-s]
//   2  dX, stride 2, by super-pixels: in = G, output channel co' = 4c + 2py + px
//      is input pixel (2Y+py, 2X+px) of channel c at super-pixel (Y, X), and
//      w'[co'][k][a][b] = w[k][c][r][s] with r = py + pad - 2(amin + a),
//      s = px + pad - 2(bmin + b), zero where (r, s) falls outside the filter.
//      The conv over super-pixels is stride 1 with filter R' x S' and
//      padding (-amin, -bmin); the epilogue (EPI 1) scatters co' back to
//      channel c, pixel (2Y+py, 2X+px).
//   3  dX, stride 2, by phases: in = G, output channel co = c, one
//      accumulator set per phase (py, px) of super-pixel (Y, X).  Phase
//      (py, px) at G offset (dy, dx) takes tap r = py + PD - 2dy,
//      s = px + PD - 2dx of w[k][c][r][s] (stored as in WMODE 1: CB rows of
//      KT*R*S floats); each G fragment is read once per offset and multiplied
//      by the weights of every phase that uses the offset, so no MFMA works
//      on a tap outside the filter, as the mixed-phase rows of WMODE 2 do.
//      The halo is that of a stride-1 problem over super-pixels with the
//      offset filter (Dxs2Taps::DR x DS) and padding (-DYMIN, -DXMIN); the
//      epilogue (EPI 3) writes pixel (2Y+py, 2X+px) of channel c.
struct DirectArgs {
    const float *in;   // [N][CI][H][W]
    const float *w;    // layer weights (see WMODE)
    float *out;        // [N][CO][OH][OW]; EPI 1: [N][CO/4][fh][fw]
    int N, CI, H, W, CO, OH, OW, st, pady, padx;
    int OHW, HW;
    int64_t in_img, out_img;  // CI*H*W, output floats per image
    int tile_px;       // output pixels per tile (one image)
    int tiles_img;     // tiles per image
    int co_blocks;     // ceil(CO / KT)
    int ncols;         // halo columns: (OW-1)*st + S  (<= PITCH)
    uint32_t w_bytes;  // size of w
    int out_vec;       // 1: tile_px and OHW are multiples of 4 (16-byte output runs)
    float beta;        // out = beta*out + result (beta in {0, 1})
    FastDiv fd_ow;     // division by OW
    // WMODE 2 / EPI 1: the layer's C, R, S, padding, the super-filter's
    // offsets, C*R*S, and the full-resolution output size.
    int g_c, g_r, g_s, g_pad, g_amin, g_bmin, g_crs, fh, fw;
    // BAND tiles (direct_bwd_band_kernel): tile t of an image starts at
    // pixel t*band_px + band_off (plain tiles: t*tile_px).
    int band_px, band_off;
};

// The (G offset, phase) pairs of the phase-form stride-2 data gradient of an
// R x S filter with padding PD, ordered by offset.  Along one axis, phase a
// and tap k meet at G offset d = (a + PD - k) / 2 when a + PD - k is even,
// so each tap belongs to exactly one (offset, phase) pair: NP = R*S.
// Lowest (hi = false) or highest G offset along an axis with K taps.
constexpr int dxs2_bound(int K, int PD, bool hi) {
    int m = hi ? -(1 << 20) : 1 << 20;
    for (int a = 0; a < 2; ++a)
        for (int k = 0; k < K; ++k) {
            const int e = a + PD - k;
            if (e % 2 == 0 && (hi ? e / 2 > m : e / 2 < m)) m = e / 2;
        }
    return m;
}
struct Dxs2Tab {
    int n;
    int off[64], ph[64], tap[64];  // offset (dy-DYMIN)*DS + dx-DXMIN, phase 2py+px, tap r*S+s
};
constexpr Dxs2Tab dxs2_pairs(int R, int S, int PD) {
    const int dymin = dxs2_bound(R, PD, false), dxmin = dxs2_bound(S, PD, false);
    const int ds = dxs2_bound(S, PD, true) - dxmin + 1;
    const int no = (dxs2_bound(R, PD, true) - dymin + 1) * ds;
    Dxs2Tab t{};
    for (int o = 0; o < no; ++o)
        for (int p = 0; p < 4; ++p) {
            const int r = (p >> 1) + PD - 2 * (dymin + o / ds);
            const int c = (p & 1) + PD - 2 * (dxmin + o % ds);
            if (r >= 0 && r < R && c >= 0 && c < S) {
                t.off[t.n] = o;
                t.ph[t.n] = p;
                t.tap[t.n] = r * S + c;
                ++t.n;
            }
        }
    return t;
}
template <int R, int S, int PD>
struct Dxs2Taps {
    static constexpr int DYMIN = dxs2_bound(R, PD, false), DXMIN = dxs2_bound(S, PD, false);
    static constexpr int DR = dxs2_bound(R, PD, true) - DYMIN + 1;
    static constexpr int DS = dxs2_bound(S, PD, true) - DXMIN + 1;
    static constexpr int NO = DR * DS;  // G offsets
    static constexpr Dxs2Tab tab = dxs2_pairs(R, S, PD);
    static constexpr int NP = tab.n;
    static_assert(NO <= 16 && NP == R * S, "every tap in exactly one (offset, phase) pair");
};

// LDS layout (floats) of the forward kernel (KG: groups of four waves, see
// direct_fwd_block).
template <int KT, int F, int CB, int R, int S, int ROWS, int PITCH, int WMODE, int KG = 1>
struct DirectFwdGeo {
    static constexpr int RS = R * S;
    // Halo rows: 32 floats (staged in pairs), or PITCH >= 64 floats of which
    // the first HCOLS are staged (whole 64-float loads; the rest of a row is
    // never read).  A pitch congruent to the output row length mod 16 keeps a
    // 16-pixel fragment that runs from one row's end into the next on 16
    // distinct address residues mod 16, as a fragment inside one row is.
    static_assert(PITCH == 32 || (PITCH >= 64 && PITCH % 8 == 0), "halo row pitch");
    static_assert(PITCH != 32 || ROWS % 2 == 0, "32-float rows are staged in pairs");
    static constexpr int HCOLS = PITCH >= 64 ? PITCH / 64 * 64 : PITCH;
    static constexpr int CPITCH = (ROWS * PITCH + 31) / 32 * 32 + 16;  // == 16 (mod 32)
    static constexpr int XS = CB * CPITCH;              // input tile
    // Weight tile, kept in the global order of its rows:
    //   WMODE 0, 2: KT rows (co) of CB*RS floats, pitch CB*RS + 4
    //   WMODE 1, 3: CB rows (ci) of KT*RS floats, pitch == 16 (mod 32)
    // Pitches are multiples of 4 floats so 16-byte DMA lands on row
    // boundaries.  The region is a whole number of 1024*KG floats, so each
    // of the 4*KG waves issues the same number of loads for it (16-byte or
    // 4-byte), without a per-wave branch; loads past the last row read zeros.
    static constexpr bool WBYCI = WMODE == 1 || WMODE == 3;  // weight rows per input channel
    static constexpr int WROWS = WBYCI ? CB : KT;
    static constexpr int WLEN = WBYCI ? KT * RS : CB * RS;
    static constexpr int WPITCH = WBYCI ? WLEN + ((16 - WLEN % 32) + 32) % 32 : WLEN + 4;
    static constexpr int WS = (WROWS * WPITCH + 1024 * KG - 1) / (1024 * KG) * (1024 * KG);
    static_assert(WLEN % 4 == 0 && WPITCH % 4 == 0, "weight rows of whole float4");
    static constexpr int STAGE = XS + WS;
    // Output transpose buffer (reuses the stages after the last chunk).
    static constexpr int TPMAX = (4 / (KT / 16)) * F * 16;  // pixels per tile, at most
    static constexpr int YPITCH = TPMAX + 4;
    static constexpr int NPH = WMODE == 3 ? 4 : 1;  // accumulator sets (phases)
    static_assert(NPH * KT * YPITCH <= 2 * STAGE, "output tile must fit the LDS stages");
    // One word past the stages: the block's flag for a non-finite result.
    static constexpr int FLAG = 2 * STAGE;
    static constexpr size_t kBytes = (2 * (size_t)STAGE + 4) * sizeof(float);
    // WMODE 2 weight slots per lane (4-byte wave loads spread over 4 waves).
    static constexpr int WSLOTS = (WS / 64 + 3) / 4;
};

// Block `bid` of `nb` (the kernel below, or the dX half of the fused
// backward launch).
//
// S2 (stride-2 forward): each staged halo row holds its even columns in the
// first half of the row and its odd columns in the second.  A fragment's 16
// pixels then read 16 consecutive floats for every tap instead of every
// other float, which would put two lanes on each LDS bank.
//
// RF (row fragments, output rows of at most 16 pixels): fragment f of wave
// part wpx is output row wpx*F + f of the tile, lane l%16 its column (lanes
// past the row end repeat the last column and are dropped).  A fragment of
// 16 consecutive pixels would wrap onto the next row, whose lanes then share
// LDS banks with the first row's; one row per fragment keeps the 16 lanes on
// 16 consecutive floats.  Tiles are whole rows.
// The epilogue of a forward-shaped block that holds a non-finite sum: every
// output is stored as in the fast epilogue, except that a non-finite one is
// first recomputed over the reference's visited products (exact.hpp) where
// the MFMA sum may hold a product the reference skips: an output whose
// window reaches the halo's padding (WMODE 0, 1, 3), or any output of the
// gathered super-filter (WMODE 2, whose absent taps are zeros multiplied by
// real G).  (oy, ox) is the output pixel of the kernel's own problem, (iy,
// ix) the full-resolution dX pixel of the stride-2 forms.  Taken only for
// non-finite data, so it is written for clarity, not speed.
template <int KT, int R, int S, int WMODE, int EPI, int PD, int NW = 4>
__device__ __forceinline__ void direct_fwd_epilogue_exact(const DirectArgs &a, const float *ys,
                                                       int ypitch, float *outb, int n, int p0,
                                                       int np, int co0, int wave, int lane) {
    const float *in_img = a.in + (int64_t)n * a.in_img;
    auto fix = [&](float v, int co, int oy, int ox, int iy, int ix) {
        if (__builtin_isfinite(v)) return v;
        if (WMODE == 2)
            return exact_dx(in_img, a.w, a.CI, a.g_c, a.H, a.W, a.g_r, a.g_s, 2, a.g_pad,
                            co >> 2, iy, ix);
        constexpr int WR = WMODE == 3 ? Dxs2Taps<R, S, PD>::DR : R;
        constexpr int WS = WMODE == 3 ? Dxs2Taps<R, S, PD>::DS : S;
        const int y0 = oy * a.st - a.pady, x0 = ox * a.st - a.padx;
        if (y0 >= 0 && y0 + WR <= a.H && x0 >= 0 && x0 + WS <= a.W) return v;
        if (WMODE == 0)
            return exact_fwd(in_img, a.w, a.CI, a.H, a.W, R, S, a.st, a.pady, co, oy, ox);
        if (WMODE == 1)
            return exact_dx(in_img, a.w, a.CI, a.CO, a.H, a.W, R, S, 1, R - 1 - a.pady, co, oy,
                            ox);
        return exact_dx(in_img, a.w, a.CI, a.CO, a.H, a.W, R, S, 2, PD, co, iy, ix);
    };
    for (int row = wave; row < KT; row += NW) {
        const int co = co0 + row;
        if (co >= a.CO) break;
        if (EPI == 3) {
            float *dst = outb + (int64_t)co * a.fh * a.fw;
            for (int py = 0; py < 2; ++py)
                for (int e = lane; e < 2 * np; e += 64) {
                    const int p = p0 + (e >> 1), px = e & 1;
                    const int Y = a.fd_ow.div(p), X = p - Y * a.OW;
                    const int iy = 2 * Y + py, ix = 2 * X + px;
                    if (iy < a.fh && ix < a.fw)
                        store_beta(dst + iy * a.fw + ix,
                                   fix(ys[((2 * py + px) * KT + row) * ypitch + (e >> 1)], co, Y,
                                       X, iy, ix),
                                   a.beta);
                }
        } else if (EPI == 1) {
            const int c = co >> 2, py = (co >> 1) & 1, px = co & 1;
            float *dst = outb + (int64_t)c * a.fh * a.fw;
            for (int p = lane; p < np; p += 64) {
                const int Y = a.fd_ow.div(p0 + p), X = p0 + p - Y * a.OW;
                const int iy = 2 * Y + py, ix = 2 * X + px;
                if (iy < a.fh && ix < a.fw)
                    store_beta(dst + iy * a.fw + ix, fix(ys[row * ypitch + p], co, Y, X, iy, ix),
                               a.beta);
            }
        } else {
            float *dst = outb + (int64_t)co * a.OHW + p0;
            for (int p = lane; p < np; p += 64) {
                const int oy = a.fd_ow.div(p0 + p);
                store_beta(dst + p, fix(ys[row * ypitch + p], co, oy, p0 + p - oy * a.OW, 0, 0),
                           a.beta);
            }
        }
    }
}

//
// KG (groups of four waves, forward and stride-1 dX only): the block runs
// 4*KG waves, and wave group g takes channel quads g, g+KG, ... of every
// stage, so each group covers the whole tile over 1/KG of the reduction.
// The LDS stages are shared, so a block of 8 waves needs no more LDS than
// one of 4, and two blocks per CU keep four waves per SIMD (against two):
// MFMA issue from more waves per SIMD hides the gaps between one wave's
// back-to-back MFMAs.  The groups' sums are added in group order in the
// epilogue's LDS transpose.
template <int KT, int F, int CB, int R, int S, int ROWS, int PITCH, int WMODE, int EPI,
          bool WVEC, bool S2 = false, bool RF = false, int PD = 0, int KG = 1, bool BAND = false>
__device__ __forceinline__ void direct_fwd_block(const DirectArgs &a, int bid, int nb) {
    using Geo = DirectFwdGeo<KT, F, CB, R, S, ROWS, PITCH, WMODE, KG>;
    constexpr int RS = R * S;
    constexpr int NW = 4 * KG;              // waves
    constexpr int WOC = KT / 16;            // waves of a group along output channels
    constexpr int CPW = CB / NW;            // input channels staged per wave
    static_assert(CB % NW == 0 && (CB / 4) % KG == 0, "whole channel quads per wave group");
    static_assert(KG == 1 || WMODE <= 1, "wave groups: forward and stride-1 dX");
    constexpr int RPL = PITCH >= 64 ? 1 : 64 / PITCH;   // halo rows per wave load
    constexpr int LPR = PITCH >= 64 ? PITCH / 64 : 1;   // wave loads per halo row
    static_assert(KT % 16 == 0 && 4 % WOC == 0, "KT must be 16, 32 or 64");
    static_assert(CB % 4 == 0, "CB must be a multiple of 4");
    static_assert(WMODE != 2 || !WVEC, "gathered weights load 4 bytes per lane");
    static_assert(!S2 || (WMODE == 0 && PITCH % 2 == 0), "split columns: forward only");
    static_assert((WMODE == 3) == (EPI == 3), "the phase form has its own epilogue");
    constexpr int HALF = PITCH / 2;

    extern __shared__ float smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int w4 = KG == 1 ? wave : wave & 3, kg = KG == 1 ? 0 : wave >> 2;  // wave in group, group
    const int woc = w4 % WOC, wpx = w4 / WOC;

    const int t = xcd_swizzle(bid, nb);
    const int cob = t % a.co_blocks;
    const int rest = t / a.co_blocks;
    const int n = rest / a.tiles_img;
    const int p0 = BAND ? (rest - n * a.tiles_img) * a.band_px + a.band_off
                        : (rest - n * a.tiles_img) * a.tile_px;
    const int p1 = min(p0 + a.tile_px, a.OHW);
    const int oy0 = a.fd_ow.div(p0);
    const int iy0 = oy0 * a.st - a.pady;
    const int co0 = cob * KT;

    // Per-lane LDS offset of each fragment's pixel, channel group l/16 folded in.
    int pix[F];
#pragma unroll
    for (int f = 0; f < F; ++f) {
        int p = RF ? p0 + (wpx * F + f) * a.OW + min(lane & 15, a.OW - 1)
                   : p0 + (wpx * F + f) * 16 + (lane & 15);
        p = p < p1 ? p : p0;
        const int oy = a.fd_ow.div(p);
        const int ox = p - oy * a.OW;
        pix[f] = (KG == 1 ? lane >> 4 : 4 * kg + (lane >> 4)) * Geo::CPITCH +
                 (oy - oy0) * a.st * PITCH + (S2 ? ox : ox * a.st);
    }
    // Per-lane A-fragment base: row co = woc*16 + l%16, channel 4*kg + l/16.
    const int abase = Geo::WBYCI
        ? (4 * kg + (lane >> 4)) * Geo::WPITCH + (woc * 16 + (lane & 15)) * RS
        : (woc * 16 + (lane & 15)) * Geo::WPITCH + (4 * kg + (lane >> 4)) * RS;
    int abase_l = abase;  // LEAN: moves with the stage

    // ---- staging: LDS-direct loads ------------------------------------------
    // Input halo: wave w stages channels w + NW*j (j < CPW), one 64-float run
    // per load (a row chunk, or two 32-float rows).  Weights: 16-byte loads
    // when every float4 of a row lies inside the row (WVEC), else 4-byte
    // loads (WMODE 2: gathered through a per-lane table).  Padding, rows past
    // the image and channels past the count read as zeros.
    const __amdgpu_buffer_rsrc_t rin =
        buf_rsrc(a.in + (int64_t)n * a.in_img, (uint32_t)(a.in_img * 4));
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(a.w, a.w_bytes);
    const int lrow = PITCH >= 64 ? 0 : lane / PITCH;  // the lane's row within a load
    int colb[LPR];  // byte offset of the lane's column within a row, or kOOB
#pragma unroll
    for (int c = 0; c < LPR; ++c) {
        const int q = c * 64 + (PITCH >= 64 ? lane : lane % PITCH);  // LDS position
        const int col = S2 ? (q < HALF ? 2 * q : 2 * (q - HALF) + 1) : q;
        const int ix = col - a.padx;
        colb[c] = (col < a.ncols && (unsigned)ix < (unsigned)a.W) ? ix * 4 : kOOB;
    }
    const int wv = __builtin_amdgcn_readfirstlane(wave);  // uniform wave index

    // WMODE 2: per lane and weight slot, the float offset of the element for
    // input channel 0 (the chunk adds ci0 * C*R*S), or -1 for a zero.
    int wtab[WMODE == 2 ? Geo::WSLOTS : 1];
    if (WMODE == 2) {
#pragma unroll
        for (int q = 0; q < Geo::WSLOTS; ++q) {
            const int e = (q * 4 + wv) * 64 + lane;
            const int row = e / Geo::WPITCH, col = e - (e / Geo::WPITCH) * Geo::WPITCH;
            const int ci = col / RS, tap = col - (col / RS) * RS;
            const int co = co0 + row;
            const int c = co >> 2, py = (co >> 1) & 1, px = co & 1;
            const int r = py + a.g_pad - 2 * (a.g_amin + tap / S);
            const int sx = px + a.g_pad - 2 * (a.g_bmin + tap % S);
            const bool ok = row < KT && col < Geo::WLEN && co < a.CO &&
                            (unsigned)r < (unsigned)a.g_r && (unsigned)sx < (unsigned)a.g_s;
            wtab[q] = ok ? ci * a.g_crs + (c * a.g_r + r) * a.g_s + sx : -1;
        }
    }

    // Per-lane byte offsets of the stage loads for the chunk at ci0 = 0; a
    // chunk adds a uniform delta.  A kOOB-based offset (< 2^31 with the
    // image below 1 GiB) stays out of range after the delta.  Kept in
    // registers, or with wave groups (LEAN: 128 VGPRs at four waves per
    // SIMD) recomputed at each load (halo_off, wload), a few VALU operations
    // per load.
    constexpr bool LEAN = KG > 1;
    uint32_t in_off[LEAN ? 1 : CPW][LEAN ? 1 : ROWS / RPL][LPR];
    if (!LEAN) {
#pragma unroll
        for (int j = 0; j < CPW; ++j)
#pragma unroll
            for (int r = 0; r < ROWS; r += RPL) {
                const int iy = iy0 + r + lrow;
                const bool ok = (unsigned)iy < (unsigned)a.H;
#pragma unroll
                for (int c = 0; c < LPR; ++c)
                    in_off[j][r / RPL][c] =
                        ok ? (uint32_t)(((wv + NW * j) * a.H + iy) * a.W * 4) + (uint32_t)colb[c]
                           : (uint32_t)kOOB;
            }
    }
    auto halo_off = [&](int j, int r, int c) __attribute__((always_inline)) {
        const int iy = iy0 + r + lrow;
        const bool ok = (unsigned)iy < (unsigned)a.H;
        return ok ? (uint32_t)(((wv + NW * j) * a.H + iy) * a.W * 4) + (uint32_t)colb[c]
                  : (uint32_t)kOOB;
    };
    // Weights (WMODE 0, 1): wave load i = NW*q + wv of the weight region; the
    // lane's row and column in it, the offset at ci0 = 0, and whether the row
    // exists apart from the chunk's channel count.
    constexpr int WE = WVEC ? 4 : 1;                  // floats per lane per load
    constexpr int WNI = Geo::WS / (64 * WE);          // wave loads
    constexpr int WNQ = (WNI + NW - 1) / NW;
    constexpr int WNQK = WMODE == 2 || LEAN ? 1 : WNQ;
    uint32_t w_off[WNQK];
    int w_col[WNQK], w_row[WNQK];
    bool w_ok[WNQK];
    if (WMODE != 2 && !LEAN) {
#pragma unroll
        for (int q = 0; q < WNQ; ++q) {
            const int e = ((q * NW + wv) * 64 + lane) * WE;
            const int row = e / Geo::WPITCH, col = e - (e / Geo::WPITCH) * Geo::WPITCH;
            w_row[q] = row;
            w_col[q] = col;
            if (WMODE == 0) {
                const int co = co0 + row;
                w_ok[q] = row < KT && co < a.CO;
                w_off[q] = (uint32_t)((co * a.CI * RS + col) * 4);
            } else {
                const int lim = min(KT, a.CO - co0) * RS;
                w_ok[q] = row < CB && col < lim;
                w_off[q] = (uint32_t)(((row * a.CO + co0) * RS + col) * 4);
            }
        }
    }
    // LEAN: weight load q's offset at ci0 = 0 and its checks, as above.
    auto wload = [&](int q, uint32_t &off, int &col, int &row, bool &ok)
        __attribute__((always_inline)) {
        const int e = ((q * NW + wv) * 64 + lane) * WE;
        row = e / Geo::WPITCH;
        col = e - row * Geo::WPITCH;
        if (WMODE == 0) {
            const int co = co0 + row;
            ok = row < KT && co < a.CO;
            off = (uint32_t)((co * a.CI * RS + col) * 4);
        } else {
            const int lim = min(KT, a.CO - co0) * RS;
            ok = row < CB && col < lim;
            off = (uint32_t)(((row * a.CO + co0) * RS + col) * 4);
        }
    };

    // Load i of a stage (NSTG per wave): halo loads first, then weight loads.
    // Issued one or two per k-step inside the previous chunk's MFMA loop
    // (stage_step), so the wave does not stall on a burst of them at the
    // chunk boundary.  ci0 >= CI makes every load read zeros, which is how
    // the last chunk's loop runs.
    constexpr int NHALO = CPW * (ROWS / RPL) * LPR;
    constexpr int NWL = WMODE == 2 ? Geo::WS / 256 : Geo::WS / (64 * NW * WE);
    constexpr int NSTG = NHALO + NWL;
    constexpr int NKW = (CB / 4 / KG) * RS;  // k-steps of a wave per stage
    static_assert(NSTG <= 4 * NKW, "at most 4 loads per k-step");
    static_assert(WMODE == 2 ? (Geo::WS / 64) % 4 == 0 : WNI % NW == 0, "equal loads per wave");
    auto stage_part = [&](float *stage, int ci0, int i) __attribute__((always_inline)) {
        if (i < NHALO) {
            const int j = i / ((ROWS / RPL) * LPR);
            const int r = (i / LPR) % (ROWS / RPL) * RPL, c = i % LPR;
            // A channel past CI gets bit 31 set: out of range (the resource
            // is below 1 GiB) whatever the sum wraps to.  Computed, not
            // selected, so the load is not split into branches on the
            // (uniform) channel test.
            const uint32_t din = (uint32_t)ci0 * (uint32_t)(a.H * a.W * 4);
            const uint32_t oob = (uint32_t)(ci0 + wv + NW * j >= a.CI) << 31;
            uint32_t off;
            if constexpr (LEAN)
                off = halo_off(j, r, c);
            else
                off = in_off[j][r / RPL][c];
            lds_dma_b32(rin, stage + (wv + NW * j) * Geo::CPITCH + r * PITCH + c * 64,
                        (int)((off + din) | oob));
            return;
        }
        const int q = i - NHALO, wi = q * NW + wv;  // this wave's load q: wave load wi
        float *wst = stage + Geo::XS;
        if (WMODE == 2) {
            lds_dma_b32(rw, wst + wi * 64, wtab[q] >= 0 ? (wtab[q] + ci0 * a.g_crs) * 4 : kOOB);
            return;
        }
        // WMODE 0: the chunk's valid columns; WMODE 1, 3: the chunk's channels.
        const uint32_t dw = WMODE == 0 ? (uint32_t)(ci0 * RS * 4) : (uint32_t)(ci0 * a.CO * RS * 4);
        const int lim = WMODE == 0 ? min(CB, a.CI - ci0) * RS : 0;
        int off;
        if constexpr (LEAN) {
            uint32_t o;
            int col, row;
            bool wok;
            wload(q, o, col, row, wok);
            const bool ok = WMODE == 0 ? (wok && col < lim) : (wok && ci0 + row < a.CI);
            off = ok ? (int)(o + dw) : kOOB;
        } else {
            const bool ok = WMODE == 0 ? (w_ok[q] && w_col[q] < lim)
                                       : (w_ok[q] && ci0 + w_row[q] < a.CI);
            off = ok ? (int)(w_off[q] + dw) : kOOB;
        }
        if (WVEC)
            lds_dma_b128(rw, wst + wi * 256, off);
        else
            lds_dma_b32(rw, wst + wi * 64, off);
    };
    auto stage_in = [&](float *stage, int ci0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NSTG; ++i) stage_part(stage, ci0, i);
    };
    // The loads of k-step kk of NK: parts [kk*per, kk*per + per), per the
    // fewest that finishes them within the loop.
    auto stage_step = [&](float *stage, int ci0, int kk, int nk) __attribute__((always_inline)) {
        const int per = (NSTG + nk - 1) / nk;
#pragma unroll
        for (int i = kk * per; i < kk * per + per; ++i)
            if (i < NSTG) stage_part(stage, ci0, i);
    };
    auto nsteploads = [](int kk, int nk) {
        const int per = (NSTG + nk - 1) / nk;
        return max(0, min(per, NSTG - kk * per));
    };

    floatx4 acc[F];
#pragma unroll
    for (int f = 0; f < F; ++f) acc[f] = floatx4{0.f, 0.f, 0.f, 0.f};

    // One k-step kk = (the wave's channel quad cs, tap): the A fragment and
    // the F B fragments it multiplies.  The group's first quad is in the
    // lane bases; its quads are KG apart.  All offsets are compile-time
    // after unrolling.
    auto fetch = [&](const float *base, const int kk, float (&b)[F], float &av)
        __attribute__((always_inline)) {
        const int cs = kk / RS * KG, tap = kk % RS;
        const int r = tap / S, s = tap % S;
        const float *ws = base + Geo::XS + (LEAN ? abase_l : abase);
        av = WMODE == 1 ? ws[cs * 4 * Geo::WPITCH + (RS - 1 - tap)] : ws[cs * 4 * RS + tap];
        const int toff = cs * 4 * Geo::CPITCH + r * PITCH + (S2 ? (s & 1) * HALF + (s >> 1) : s);
#pragma unroll
        for (int f = 0; f < F; ++f) b[f] = base[pix[f] + toff];
    };
    auto mma = [&](const float (&b)[F], const float av) __attribute__((always_inline)) {
#pragma unroll
        for (int f = 0; f < F; ++f)
            acc[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b[f], acc[f], 0, 0, 0);
    };
    // WMODE 3: one accumulator set per phase; acc (above) is phase 0's.
    floatx4 acc3[WMODE == 3 ? 3 : 1][F];
#pragma unroll
    for (int p = 0; p < (WMODE == 3 ? 3 : 1); ++p)
#pragma unroll
        for (int f = 0; f < F; ++f) acc3[p][f] = floatx4{0.f, 0.f, 0.f, 0.f};
    // Micro-step m of a stage = (channel quad m / NP, pair m % NP); the F
    // G fragments of an offset are read at its first pair into one of two
    // buffers (alternating by offset), the pair's weight fragment every step.
    auto compute3 = [&](const float *base, float *nxt, int ci0n) __attribute__((always_inline)) {
      if constexpr (WMODE == 3) {
        using Tp = Dxs2Taps<R, S, PD>;
        constexpr int NP = Tp::NP, NM = (CB / 4) * NP;
        float bb[2][F];
        float aa[2];
        const float *ws = base + Geo::XS + abase;
        auto fetch_b = [&](int m, float (&b)[F]) __attribute__((always_inline)) {
            const int cs = m / NP, o = Tp::tab.off[m % NP];
            const int toff = cs * 4 * Geo::CPITCH + (o / Tp::DS) * PITCH + o % Tp::DS;
#pragma unroll
            for (int f = 0; f < F; ++f) b[f] = base[pix[f] + toff];
        };
        auto fetch_a = [&](int m, float &av) __attribute__((always_inline)) {
            av = ws[(m / NP) * 4 * Geo::WPITCH + Tp::tab.tap[m % NP]];
        };
        auto gofs = [](int m) { return (m / NP) * Tp::NO + Tp::tab.off[m % NP]; };
        fetch_b(0, bb[0]);
        fetch_a(0, aa[0]);
        asm volatile("" ::: "memory");
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const int g = gofs(m);
            const bool nb1 = m + 1 < NM && gofs(m + 1) != g;
            if (m + 1 < NM) {
                if (nb1) fetch_b(m + 1, bb[(g + 1) & 1]);
                fetch_a(m + 1, aa[(m + 1) & 1]);
            }
            const int ph = Tp::tab.ph[m % NP];
#pragma unroll
            for (int f = 0; f < F; ++f) {
                if (ph == 0)
                    acc[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(aa[m & 1], bb[g & 1][f], acc[f],
                                                                  0, 0, 0);
                else
                    acc3[ph > 0 ? ph - 1 : 0][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        aa[m & 1], bb[g & 1][f], acc3[ph > 0 ? ph - 1 : 0][f], 0, 0, 0);
            }
            stage_step(nxt, ci0n, m, NM);
            if (nb1)
                order_step<F + 1, F>(nsteploads(m, NM));
            else
                order_step<1, F>(nsteploads(m, NM));
        }
      }
    };

    // Software pipeline over the k-steps of one stage: the fragments of step
    // kk+1 are read while step kk's MFMAs run.
    // The next chunk's loads go into `nxt` as it runs (ci0n = its first
    // channel, or CI for none).
    auto compute = [&](const float *base, float *nxt, int ci0n) __attribute__((always_inline)) {
        if (WMODE == 3) {
            compute3(base, nxt, ci0n);
            return;
        }
        constexpr int NK = NKW;
        if constexpr (KG > 1 && F > KATSU_FWD_KG_PIPE_F) {
            // Wide tiles: one register set keeps the wave within the VGPRs
            // of its occupancy, and the other waves of the SIMD hide its
            // LDS latency.
            float b0[F], a0;
#pragma unroll
            for (int kk = 0; kk < NK; ++kk) {
                fetch(base, kk, b0, a0);
                mma(b0, a0);
                stage_step(nxt, ci0n, kk, NK);
                order_step<F + 1, F>(nsteploads(kk, NK));
            }
            return;
        }
        float b0[F], b1[F];
        float a0, a1;
        fetch(base, 0, b0, a0);
        asm volatile("" ::: "memory");  // keep step 0's reads apart from step 1's
#pragma unroll
        for (int kk = 0; kk < NK; kk += 2) {
            if (kk + 1 < NK) fetch(base, kk + 1, b1, a1);
            mma(b0, a0);
            stage_step(nxt, ci0n, kk, NK);
            order_step<F + 1, F>(nsteploads(kk, NK));
            if (kk + 2 < NK) fetch(base, kk + 2, b0, a0);
            if (kk + 1 < NK) {
                mma(b1, a1);
                stage_step(nxt, ci0n, kk + 1, NK);
            }
            order_step<F + 1, F>(kk + 1 < NK ? nsteploads(kk + 1, NK) : 0);
        }
    };

    // Two-stage pipeline: while chunk ch is consumed from one stage, chunk
    // ch+1 streams into the other.  The loop is unrolled by two so each
    // stage's base is a constant.
    const int nch = (a.CI + CB - 1) / CB;
    float *st0 = smem;
    float *st1 = smem + Geo::STAGE;
    if (tid == 0) smem[Geo::FLAG] = 0.f;  // published by the barriers below
    stage_in(st0, 0);
    wait_lds_dma();
    __syncthreads();
    if constexpr (LEAN) {
        // One loop body: the lane bases move to the other stage after each
        // chunk, which keeps the accumulators in place across the loop's
        // back edge (the unrolled form needs registers to carry them).
        for (int ch = 0; ch < nch; ++ch) {
            const bool odd = ch & 1;
            compute(smem, odd ? st0 : st1, ch + 1 < nch ? (ch + 1) * CB : a.CI);
            wait_lds_dma();
            __syncthreads();
            const int d = odd ? -Geo::STAGE : Geo::STAGE;
#pragma unroll
            for (int f = 0; f < F; ++f) pix[f] += d;
            abase_l += d;
        }
    }
    for (int ch = 0; ch < (LEAN ? 0 : nch); ch += 2) {
        compute(st0, st1, ch + 1 < nch ? (ch + 1) * CB : a.CI);
        wait_lds_dma();
        __syncthreads();
        if (ch + 1 >= nch) break;
        compute(st1, st0, ch + 2 < nch ? (ch + 2) * CB : a.CI);
        wait_lds_dma();
        __syncthreads();
    }

    // Epilogue: transpose the KT x tile block through LDS (the stages are
    // free after the last barrier), then write each output channel's pixel
    // run -- contiguous in NCHW -- as 16-byte stores (EPI 0), or scatter each
    // super-pixel channel to its full-resolution positions (EPI 1).
    // Phase ph of WMODE 3 takes rows ph*KT .. ph*KT + KT-1 of ys.
    // With wave groups, group 0 stores its sums and each later group adds
    // its own in turn (a barrier apart), keeping the result in registers.
    float *ys = smem;
    auto put = [&](int ph, floatx4 (&ac)[F], const bool add) __attribute__((always_inline)) {
        float *yp = ys + ph * KT * Geo::YPITCH;
        auto one = [&](floatx4 &q, const int v, const int e) __attribute__((always_inline)) {
            if (KG == 1) {
                yp[e] = q[v];
                return;
            }
            if (add) q[v] = yp[e] + q[v];
            yp[e] = q[v];
        };
        if (RF) {
            // Pixel p0 + row*OW + col sits at ys column row*OW + col.
            if ((lane & 15) < a.OW) {
#pragma unroll
                for (int f = 0; f < F; ++f)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        one(ac[f], v, (woc * 16 + 4 * (lane >> 4) + v) * Geo::YPITCH +
                                          (wpx * F + f) * a.OW + (lane & 15));
            }
        } else {
#pragma unroll
            for (int f = 0; f < F; ++f)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    one(ac[f], v, (woc * 16 + 4 * (lane >> 4) + v) * Geo::YPITCH +
                                      (wpx * F + f) * 16 + (lane & 15));
        }
    };
#pragma unroll
    for (int g = 1; g < KG; ++g) {
        if (g == 1 && kg == 0) put(0, acc, false);
        __syncthreads();
        if (kg == g) put(0, acc, true);
    }
    // A non-finite sum may hold a product the reference skips: the block
    // notes whether any of its sums is non-finite (a test of the last
    // group's registers, which hold the finished sums) in one LDS word, and
    // only a block that has one takes the epilogue that recomputes them; the
    // others store as fast as they would without the test.
    if (kg == KG - 1) {
        bool bad = false;
#pragma unroll
        for (int f = 0; f < F; ++f) bad |= !all_finite4(acc[f][0], acc[f][1], acc[f][2], acc[f][3]);
        if (WMODE == 3) {
#pragma unroll
            for (int p = 0; p < (WMODE == 3 ? 3 : 1); ++p)
#pragma unroll
                for (int f = 0; f < F; ++f)
                    bad |= !all_finite4(acc3[p][f][0], acc3[p][f][1], acc3[p][f][2], acc3[p][f][3]);
        }
        if (bad) smem[Geo::FLAG] = 1.f;
    }
    if (KG == 1) {
        put(0, acc, false);
        if (WMODE == 3) {
#pragma unroll
            for (int ph = 1; ph < 4; ++ph) put(ph, acc3[ph > 0 ? ph - 1 : 0], false);
        }
    }
    __syncthreads();
    float *outb = a.out + (int64_t)n * a.out_img;
    const int np = p1 - p0;
    if (smem[Geo::FLAG] != 0.f) {
        direct_fwd_epilogue_exact<KT, R, S, WMODE, EPI, PD, NW>(a, ys, Geo::YPITCH, outb, n, p0,
                                                                np, co0, wave, lane);
        return;
    }
    if (EPI == 3) {
        // Element e of a channel's run: super-pixel p0 + e/2, column phase e&1;
        // consecutive lanes write consecutive pixels of a full-resolution row.
        for (int row = wave; row < KT; row += NW) {
            const int co = co0 + row;
            if (co >= a.CO) break;
            float *dst = outb + (int64_t)co * a.fh * a.fw;
            for (int py = 0; py < 2; ++py)
                for (int e = lane; e < 2 * np; e += 64) {
                    const int p = p0 + (e >> 1), px = e & 1;
                    const int Y = a.fd_ow.div(p);
                    const int iy = 2 * Y + py, ix = 2 * (p - Y * a.OW) + px;
                    if (iy < a.fh && ix < a.fw)
                        store_beta_nt(dst + iy * a.fw + ix,
                                   ys[((2 * py + px) * KT + row) * Geo::YPITCH + (e >> 1)], a.beta);
                }
        }
    } else if (EPI == 1) {
        for (int row = wave; row < KT; row += NW) {
            const int co = co0 + row;
            if (co >= a.CO) break;
            const int c = co >> 2, py = (co >> 1) & 1, px = co & 1;
            float *dst = outb + (int64_t)c * a.fh * a.fw;
            for (int p = lane; p < np; p += 64) {
                const int Y = a.fd_ow.div(p0 + p);
                const int X = p0 + p - Y * a.OW;
                const int iy = 2 * Y + py, ix = 2 * X + px;
                if (iy < a.fh && ix < a.fw)
                    store_beta_nt(dst + iy * a.fw + ix, ys[row * Geo::YPITCH + p], a.beta);
            }
        }
    } else if (a.out_vec) {
        const int n4 = np >> 2;
        for (int row = wave; row < KT; row += NW) {
            const int co = co0 + row;
            if (co >= a.CO) break;
            float *dst = outb + (int64_t)co * a.OHW + p0;
            for (int c4 = lane; c4 < n4; c4 += 64) {
                const floatx4 v =
                    *reinterpret_cast<const floatx4 *>(ys + row * Geo::YPITCH + c4 * 4);
                store4_beta_nt(reinterpret_cast<floatx4 *>(dst + c4 * 4), v, a.beta);
            }
        }
    } else {
        for (int row = wave; row < KT; row += NW) {
            const int co = co0 + row;
            if (co >= a.CO) break;
            float *dst = outb + (int64_t)co * a.OHW + p0;
            for (int p = lane; p < np; p += 64)
                store_beta_nt(dst + p, ys[row * Geo::YPITCH + p], a.beta);
        }
    }
}

// Waves per SIMD the forward kernel is compiled for: two blocks per CU, or
// with wave groups as many as the block's LDS lets share a CU.
template <int KT, int F, int CB, int R, int S, int ROWS, int PITCH, int WMODE, int KG>
constexpr int direct_fwd_waves_per_simd() {
    return KG == 1 ? 2
                   : KG * (2 * DirectFwdGeo<KT, F, CB, R, S, ROWS, PITCH, WMODE, KG>::kBytes <=
                                   160 * 1024
                               ? 2
                               : 1);
}

template <int KT, int F, int CB, int R, int S, int ROWS, int PITCH, int WMODE, int EPI,
          bool WVEC, bool S2 = false, bool RF = false, int PD = 0, int KG = 1>
__global__ void __launch_bounds__(
    256 * KG, (direct_fwd_waves_per_simd<KT, F, CB, R, S, ROWS, PITCH, WMODE, KG>()))
    direct_fwd_kernel(const DirectArgs a) {
    direct_fwd_block<KT, F, CB, R, S, ROWS, PITCH, WMODE, EPI, WVEC, S2, RF, PD, KG>(a, blockIdx.x,
                                                                               gridDim.x);
}

// ---------------------------------------------------------------------------
// Filter-gradient kernel.
//
// GEMM view: i = output channel (KT per block), j = input channel (CT per
// block), k = output pixel; one accumulator tile per tap.  A block walks a
// range of pixel tiles (its split of the reduction), staging G[KT][tile] and
// the X halo [CT][ROWS][64*CC] for each tile through a two-stage LDS
// pipeline, and writes one partial dw[KT][CT][R][S] at the end.  Waves split
// KT x CT into 16 x 16 slices.
//
// A tile is `trows` whole output rows, or one segment of `seg_w` columns of
// a row: either way its G pixels are contiguous in memory.  A k-step takes
// four consecutive columns of one tile row, so the step geometry is uniform
// (scalar) and only the lane's column is per-lane.
struct DirectDwArgs {
    const float *x;    // [N][C][H][W]
    const float *g;    // [N][K][OH][OW]
    float *out;        // partials [split][K][C*R*S], or dw itself when splits == 1
    int N, C, H, W, K, OH, OW, st, pad;
    int OHW, HW, CRS;
    int64_t x_img, g_img;
    int trows;           // output rows per tile (1 when tiles are row segments)
    int seg_w;           // columns per tile (OW when tiles are whole rows)
    int segs;            // tiles per row band: cdiv(OW, seg_w)
    int tiles_img, tiles_total, tiles_per_split;
    int k_blocks, c_blocks;
    int ncols;
    int gpitch;          // LDS row pitch of the G tile, == 2 (mod 4), >= gcap
    int gcap;            // G floats staged per row: trows*seg_w rounded up to 4
    int stage;           // floats per LDS stage: KT*gpitch + CT*CPITCH
    int out_vec;         // 1: partial rows are 16-byte aligned runs
    int64_t split_stride;  // floats between partials, or 0 when writing dw directly
    float beta;            // applied only when writing dw directly
    FastDiv fd_tiles_img, fd_segs;
    int flag;              // LDS float index of the block's non-finite flag (past the stages)
};

// Compile-time part of the dW LDS layout; the G tile's pitch is chosen per
// problem (the tightest pitch == 2 mod 4, which keeps the A reads of a
// half-wave on 32 distinct banks).
template <int KT, int CT, int R, int S, int ROWS, int PITCH_, int GPC>
struct DirectDwGeo {
    static constexpr int PITCH = PITCH_;              // halo row pitch: 32 or a multiple of 64
    static_assert(PITCH == 32 || PITCH % 64 == 0, "halo row pitch");
    static_assert(PITCH != 32 || ROWS % 2 == 0, "32-float rows are staged in pairs");
    static constexpr int CPITCH = ROWS * PITCH + 2;   // == 2 (mod 32)
    static constexpr int XS = CT * CPITCH;
    static constexpr int PPITCH = CT * R * S + 4;     // partial transpose buffer
    static constexpr int GMAX = 64 * GPC;             // G floats per row, at most
};

// WKF: 16-row output-channel fragments per wave.  A wave owns
// (16*WKF) oc x 16 c x R*S taps; each k-step reads WKF A and R*S B
// fragments for WKF*R*S MFMAs.  FULL: every tile row is a multiple of 4
// pixels wide, so no k-step holds a pixel past the end of its row.
// The epilogue of a dW block that holds a non-finite partial: every element
// is stored as in the fast epilogue, except that a non-finite one is first
// recomputed over the block's output pixels [pbeg, pend) (exact.hpp).  Taken
// only for non-finite data.
template <int KT, int RS, int S>
__device__ __forceinline__ void direct_dw_epilogue_exact(const DirectDwArgs &a, const float *ps,
                                                      int ppitch, float *ob, int k0, int c0,
                                                      int len, int64_t pbeg, int64_t pend,
                                                      int wave, int lane) {
    for (int row = wave; row < KT; row += 4) {
        const int k = k0 + row;
        if (k >= a.K) break;
        float *dst = ob + (int64_t)k * a.CRS + c0 * RS;
        for (int e = lane; e < len; e += 64) {
            float v = ps[row * ppitch + e];
            if (!__builtin_isfinite(v)) {
                const int ce = e / RS, tap = e - (e / RS) * RS;
                v = exact_dw(a.x, a.g, a.C, a.H, a.W, a.K, a.OH, a.OW, a.st, a.pad, k, c0 + ce,
                             tap / S, tap % S, pbeg, pend);
            }
            if (a.split_stride == 0)
                store_beta(dst + e, v, a.beta);
            else
                dst[e] = v;
        }
    }
}

template <int KT, int CT, int R, int S, int ROWS, int PITCH, int GPC, int WKF, bool FULL>
__device__ __forceinline__ void direct_dw_block(const DirectDwArgs &a, int bid, int nb) {
    using Geo = DirectDwGeo<KT, CT, R, S, ROWS, PITCH, GPC>;
    constexpr int RPL = PITCH >= 64 ? 1 : 64 / PITCH;  // halo rows per 64-lane load
    constexpr int LPR = PITCH >= 64 ? PITCH / 64 : 1;  // 64-lane loads per halo row
    constexpr int RS = R * S;
    constexpr int WK = KT / (16 * WKF);  // waves along output channels
    constexpr int CPW = CT / 4;          // input channels staged per wave
    static_assert(KT % (16 * WKF) == 0 && CT % 16 == 0 && WK * (CT / 16) == 4,
                  "4 waves of (16*WKF) x 16 slices");

    extern __shared__ float smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wk = wave % WK, wc = wave / WK;

    const int t = xcd_swizzle(bid, nb);
    const int kb = t % a.k_blocks;
    const int rest = t / a.k_blocks;
    const int cb = rest % a.c_blocks;
    const int split = rest / a.c_blocks;
    const int k0 = kb * KT, c0 = cb * CT;
    const int tb = split * a.tiles_per_split;
    const int te = min(tb + a.tiles_per_split, a.tiles_total);
    const int gs_floats = KT * a.gpitch;  // the G part of a stage

    const int lrow = PITCH >= 64 ? 0 : lane / PITCH;  // the lane's row within a load
    int colb[LPR];
#pragma unroll
    for (int c = 0; c < LPR; ++c) {
        const int col = c * 64 + (PITCH >= 64 ? lane : lane % PITCH);
        const int ix = col - a.pad;
        colb[c] = (col < a.ncols && (unsigned)ix < (unsigned)a.W) ? ix * 4 : kOOB;
    }

    struct TileGeo { int n, oy0, tr, cx0, cx1, np; };
    auto geo = [&](int tile) __attribute__((always_inline)) {
        TileGeo tg;
        tg.n = a.fd_tiles_img.div(tile);
        const int ti = tile - tg.n * a.tiles_img;
        const int band = a.fd_segs.div(ti);
        tg.oy0 = band * a.trows;
        tg.tr = min(a.trows, a.OH - tg.oy0);
        tg.cx0 = (ti - band * a.segs) * a.seg_w;
        tg.cx1 = min(tg.cx0 + a.seg_w, a.OW);
        tg.np = tg.tr * (tg.cx1 - tg.cx0);
        return tg;
    };

    // LDS-direct staging of a tile: X halo channel w + 4j of wave w at
    // (w + 4j)*CPITCH + r*PITCH + c*64 (lane l at +l: a row chunk, or two
    // 32-float rows); G row k at k*gpitch, lanes below gcap only, so a row
    // never spills into the next (gpitch >= gcap).
    const int wvu = __builtin_amdgcn_readfirstlane(wave);
    auto stage_dma = [&](float *base, const TileGeo &tg) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rx =
            buf_rsrc(a.x + (int64_t)tg.n * a.x_img, (uint32_t)(a.x_img * 4));
        const __amdgpu_buffer_rsrc_t rg =
            buf_rsrc(a.g + (int64_t)tg.n * a.g_img, (uint32_t)(a.g_img * 4));
        const int iy0 = tg.oy0 * a.st - a.pad;
#pragma unroll
        for (int j = 0; j < CPW; ++j) {
            const int ci = c0 + wvu + 4 * j;
#pragma unroll
            for (int r = 0; r < ROWS; r += RPL) {
                const int iy = iy0 + r + lrow;
                const bool rok = ci < a.C && (unsigned)iy < (unsigned)a.H;
                const int rowb = (ci * a.H + iy) * a.W * 4;
#pragma unroll
                for (int c = 0; c < LPR; ++c)
                    lds_dma_b32(rx, base + gs_floats + (wvu + 4 * j) * Geo::CPITCH + r * PITCH + c * 64,
                                rok ? rowb + colb[c] : kOOB);
            }
        }
        const int p0 = tg.oy0 * a.OW + tg.cx0;
#pragma unroll
        for (int i = 0; i < KT / 4; ++i) {
            const int row = wvu + 4 * i;
            const int k = k0 + row;
#pragma unroll
            for (int c = 0; c < GPC; ++c) {
                const int px = c * 64 + lane;
                if (px < a.gcap)
                    lds_dma_b32(rg, base + row * a.gpitch + c * 64,
                                (k < a.K && px < tg.np) ? (k * a.OHW + p0 + px) * 4 : kOOB);
            }
        }
    };

    floatx4 acc[WKF][RS];
#pragma unroll
    for (int f = 0; f < WKF; ++f)
#pragma unroll
        for (int i = 0; i < RS; ++i) acc[f][i] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int arow = (wk * 16 * WKF + (lane & 15)) * a.gpitch;
    const int bch = gs_floats + (wc * 16 + (lane & 15)) * Geo::CPITCH;
    const int lq = lane >> 4;  // the lane's pixel within a k-step

    // One stage: k-steps over (tile row, 4-column group), two register sets
    // so the fragments of step s+1 are read while step s's MFMAs run.  With
    // FULL every lane's pixel is valid and its addresses are a per-lane base
    // plus a uniform step offset.  Otherwise a lane past the end of its tile row reads the
    // row's last pixel (finite data) and its G values are zeroed at MFMA time,
    // so it contributes nothing; the mask is applied after the next step's
    // reads are issued, keeping the LDS latency off the MFMA path.
    auto compute = [&](const float *base, const TileGeo &tg) __attribute__((always_inline)) {
        const int wseg = tg.cx1 - tg.cx0;
        const int cpr = (wseg + 3) >> 2;
        const int nsteps = tg.tr * cpr;
        int fr = 0, fc = 0;  // (tile row, column group) of the next step to fetch
        auto fetch = [&](float (&av)[WKF], float (&b)[RS], bool &ok)
            __attribute__((always_inline)) {
            const int row = min(fr, tg.tr - 1);  // a fetch past the last step re-reads it
            const int col = tg.cx0 + fc * 4 + lq;
            ok = FULL || col < tg.cx1;
            const int cc = FULL ? col : min(col, tg.cx1 - 1);
            const float *gsrc = base + arow + row * wseg + (cc - tg.cx0);
#pragma unroll
            for (int f = 0; f < WKF; ++f) av[f] = gsrc[f * 16 * a.gpitch];
            const float *xs = base + bch + row * a.st * Geo::PITCH + cc * a.st;
#pragma unroll
            for (int tap = 0; tap < RS; ++tap) b[tap] = xs[(tap / S) * Geo::PITCH + tap % S];
            if (++fc == cpr) {
                fc = 0;
                ++fr;
            }
        };
        auto mma = [&](const float (&av)[WKF], const float (&b)[RS], const bool ok)
            __attribute__((always_inline)) {
#pragma unroll
            for (int f = 0; f < WKF; ++f) {
                const float am = FULL || ok ? av[f] : 0.f;
#pragma unroll
                for (int tap = 0; tap < RS; ++tap)
                    acc[f][tap] =
                        __builtin_amdgcn_mfma_f32_16x16x4f32(am, b[tap], acc[f][tap], 0, 0, 0);
            }
        };
        auto run = [&](auto &&fetchf, const int nst) __attribute__((always_inline)) {
            float a0[WKF], a1[WKF], b0[RS], b1[RS];
            bool k0ok, k1ok;
            fetchf(a0, b0, k0ok);
            asm volatile("" ::: "memory");  // keep step 0's reads apart from step 1's
            for (int s = 0; s < nst; s += 2) {
                fetchf(a1, b1, k1ok);
                mma(a0, b0, k0ok);
                order_reads_then_mfma<WKF + RS, WKF * RS>();
                if (s + 1 >= nst) break;
                fetchf(a0, b0, k0ok);
                mma(a1, b1, k1ok);
                order_reads_then_mfma<WKF + RS, WKF * RS>();
            }
        };
        if (FULL && tg.tr == 1 && a.st == 1) {
            // One output row at stride 1 (config 3): the lane's G and x
            // addresses move 4 pixels per step, every tap offset an
            // immediate, with no row or column counters in the loop.
            const float *gp[WKF];
#pragma unroll
            for (int f = 0; f < WKF; ++f) gp[f] = base + arow + f * 16 * a.gpitch + lq;
            const float *xp = base + bch + (tg.cx0 + lq);
            const int nst = (tg.cx1 - tg.cx0) >> 2;
            if (nst == 14) {
                // 56-pixel rows: the steps unrolled, each read at an
                // immediate offset from the lane's base addresses.
                auto sfetch = [&](const int s, float (&av)[WKF], float (&b)[RS])
                    __attribute__((always_inline)) {
#pragma unroll
                    for (int f = 0; f < WKF; ++f) av[f] = gp[f][4 * s];
#pragma unroll
                    for (int tap = 0; tap < RS; ++tap)
                        b[tap] = xp[(tap / S) * Geo::PITCH + tap % S + 4 * s];
                };
                constexpr int NST = 14;
                float a0[WKF], a1[WKF], b0[RS], b1[RS];
                sfetch(0, a0, b0);
                asm volatile("" ::: "memory");  // keep step 0's reads apart from step 1's
#pragma unroll
                for (int s = 0; s < NST; s += 2) {
                    sfetch(s + 1, a1, b1);
                    mma(a0, b0, true);
                    order_reads_then_mfma<WKF + RS, WKF * RS>();
                    if (s + 2 < NST) sfetch(s + 2, a0, b0);
                    mma(a1, b1, true);
                    order_reads_then_mfma<WKF + RS, WKF * RS>();
                }
            } else {
                auto rfetch = [&](float (&av)[WKF], float (&b)[RS], bool &ok)
                    __attribute__((always_inline)) {
                    ok = true;
#pragma unroll
                    for (int f = 0; f < WKF; ++f) {
                        av[f] = *gp[f];
                        gp[f] += 4;
                    }
#pragma unroll
                    for (int tap = 0; tap < RS; ++tap)
                        b[tap] = xp[(tap / S) * Geo::PITCH + tap % S];
                    xp += 4;
                };
                run(rfetch, nst);
            }
        } else if (!FULL && a.segs == 1 && tg.np == 56 && a.OW >= 4) {
            // 56-pixel tiles of whole rows (config 4a: 4 rows of 14) over
            // flattened pixels: 14 steps, every lane valid.  The lane's x
            // offset of each step (its pixel's row and column) is computed
            // once per tile, and its G reads take immediate offsets.
            constexpr int NST = 14;
            int xo[NST];
#pragma unroll
            for (int s = 0; s < NST; ++s) {
                const int q = 4 * s + lq, row = q / a.OW, col = q - row * a.OW;
                xo[s] = (row * Geo::PITCH + col) * a.st;
            }
            const float *gp = base + arow + lq;
            const float *xb = base + bch;
            auto sfetch = [&](const int s, float (&av)[WKF], float (&b)[RS])
                __attribute__((always_inline)) {
#pragma unroll
                for (int f = 0; f < WKF; ++f) av[f] = gp[f * 16 * a.gpitch + 4 * s];
                const float *xs = xb + xo[s];
#pragma unroll
                for (int tap = 0; tap < RS; ++tap) b[tap] = xs[(tap / S) * Geo::PITCH + tap % S];
            };
            float a0[WKF], a1[WKF], b0[RS], b1[RS];
            sfetch(0, a0, b0);
            asm volatile("" ::: "memory");  // keep step 0's reads apart from step 1's
#pragma unroll
            for (int s = 0; s < NST; s += 2) {
                sfetch(s + 1, a1, b1);
                mma(a0, b0, true);
                order_reads_then_mfma<WKF + RS, WKF * RS>();
                if (s + 2 < NST) sfetch(s + 2, a0, b0);
                mma(a1, b1, true);
                order_reads_then_mfma<WKF + RS, WKF * RS>();
            }
        } else if (!FULL && a.segs == 1 && a.OW >= 4) {
            // Tiles of whole rows whose width is not a multiple of 4: steps
            // over the tile's flattened pixels (G is stored contiguous by
            // pixel), so only the tile's last step has idle lanes.  Each lane
            // keeps its pixel's (row, column) for the X reads.
            int q = lq, prow = lq / a.OW, pcol = lq - (lq / a.OW) * a.OW;
            auto ffetch = [&](float (&av)[WKF], float (&b)[RS], bool &ok)
                __attribute__((always_inline)) {
                ok = q < tg.np;
                const int row = min(prow, tg.tr - 1), col = ok ? pcol : a.OW - 1;
                const float *gsrc = base + arow + min(q, tg.np - 1);
#pragma unroll
                for (int f = 0; f < WKF; ++f) av[f] = gsrc[f * 16 * a.gpitch];
                const float *xs = base + bch + row * a.st * Geo::PITCH + col * a.st;
#pragma unroll
                for (int tap = 0; tap < RS; ++tap)
                    b[tap] = xs[(tap / S) * Geo::PITCH + tap % S];
                q += 4;
                pcol += 4;
                if (pcol >= a.OW) {
                    pcol -= a.OW;
                    ++prow;
                }
            };
            run(ffetch, (tg.np + 3) >> 2);
        } else {
            run(fetch, nsteps);
        }
    };
    // Cleared before the stage loop's barriers; a block without tiles has
    // zero sums and never sets it.
    if (tid == 0) smem[a.flag] = 0.f;
    if (tb < te) {
        float *st0 = smem;
        float *st1 = smem + a.stage;
        TileGeo cur = geo(tb);
        stage_dma(st0, cur);
        wait_lds_dma();
        __syncthreads();
        for (int tile = tb; tile < te; tile += 2) {
            TileGeo nxt = cur;
            if (tile + 1 < te) {
                nxt = geo(tile + 1);
                stage_dma(st1, nxt);
            }
            compute(st0, cur);
            wait_lds_dma();
            __syncthreads();
            if (tile + 1 >= te) break;
            cur = nxt;
            if (tile + 2 < te) {
                nxt = geo(tile + 2);
                stage_dma(st0, nxt);
            }
            compute(st1, cur);
            wait_lds_dma();
            __syncthreads();
            cur = nxt;
        }
    }

    // Epilogue: D[i = oc][j = c] per tap, transposed through LDS into the
    // partial's row order [oc][c][tap], then written as contiguous runs of
    // CT*RS floats per output channel.  A non-finite partial may hold a
    // product the reference skips (a G value times the halo's padding, or a
    // masked lane's zero times real x): as in the forward's epilogue, the
    // block notes one in an LDS word (the accumulators are tested before the
    // transpose), and only then takes the epilogue that recomputes them.
    float *ps = smem;
    {
        bool bad = false;
#pragma unroll
        for (int f = 0; f < WKF; ++f)
#pragma unroll
            for (int tap = 0; tap < RS; ++tap)
                bad |= !all_finite4(acc[f][tap][0], acc[f][tap][1], acc[f][tap][2], acc[f][tap][3]);
        if (bad) smem[a.flag] = 1.f;
    }
#pragma unroll
    for (int f = 0; f < WKF; ++f)
#pragma unroll
        for (int tap = 0; tap < RS; ++tap)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                ps[(wk * 16 * WKF + f * 16 + 4 * (lane >> 4) + v) * Geo::PPITCH +
                   (wc * 16 + (lane & 15)) * RS + tap] = acc[f][tap][v];
    __syncthreads();
    float *ob = a.out + (int64_t)split * a.split_stride;
    const int len = min(CT, a.C - c0) * RS;  // valid floats of a row
    if (smem[a.flag] != 0.f) {
        // The block's output pixels are one contiguous range of the batch.
        const TileGeo g0 = geo(tb), g1 = geo(te - 1);
        const int64_t pbeg = ((int64_t)g0.n * a.OH + g0.oy0) * a.OW + g0.cx0;
        const int64_t pend = ((int64_t)g1.n * a.OH + g1.oy0 + g1.tr - 1) * a.OW + g1.cx1;
        direct_dw_epilogue_exact<KT, RS, S>(a, ps, Geo::PPITCH, ob, k0, c0, len, pbeg, pend,
                                            wave, lane);
        return;
    }
    for (int row = wave; row < KT; row += 4) {
        const int k = k0 + row;
        if (k >= a.K) break;
        float *dst = ob + (int64_t)k * a.CRS + c0 * RS;
        const float *src = ps + row * Geo::PPITCH;
        if (a.out_vec && len == CT * RS) {
            for (int c4 = lane; c4 < CT * RS / 4; c4 += 64) {
                floatx4 v = *reinterpret_cast<const floatx4 *>(src + c4 * 4);
                floatx4 *d = reinterpret_cast<floatx4 *>(dst + c4 * 4);
                if (a.split_stride == 0 && a.beta != 0.f) v += *d;
                __builtin_nontemporal_store(v, d);  // read back by the next kernel only
            }
        } else {
            for (int e = lane; e < len; e += 64) {
                if (a.split_stride == 0)
                    store_beta(dst + e, src[e], a.beta);
                else
                    dst[e] = src[e];
            }
        }
    }
}

template <int KT, int CT, int R, int S, int ROWS, int PITCH, int GPC, int WKF, bool FULL>
__global__ void __launch_bounds__(256, 2) direct_dw_kernel(const DirectDwArgs a) {
    direct_dw_block<KT, CT, R, S, ROWS, PITCH, GPC, WKF, FULL>(a, blockIdx.x, gridDim.x);
}

// Both backward passes in one launch: blocks [0, nbw) compute the dW
// partials, the rest dX (the forward kernel on G with the transposed,
// flipped filter).  The dW blocks are the longer ones and are dispatched
// first; dX blocks fill the CUs beside them and as they retire, so the two
// passes share one ramp and one tail.  Dynamic LDS is the larger of the two
// needs.
template <int XKT, int XF, int XCB, int R, int S, int XROWS, int XPITCH, bool XWVEC, int KT,
          int CT, int ROWS, int PITCH, int GPC, int WKF, bool FULL, int XWMODE = 1, int XEPI = 0,
          bool XRF = false, int XPD = 0>
__global__ void __launch_bounds__(256, 2) direct_bwd_kernel(const DirectArgs dx,
                                                            const DirectDwArgs dw, int nbw) {
    if ((int)blockIdx.x < nbw)
        direct_dw_block<KT, CT, R, S, ROWS, PITCH, GPC, WKF, FULL>(dw, blockIdx.x, nbw);
    else
        direct_fwd_block<XKT, XF, XCB, R, S, XROWS, XPITCH, XWMODE, XEPI, XWVEC, false, XRF, XPD>(
            dx, blockIdx.x - nbw, gridDim.x - nbw);
}

// The forward with tiles of two fragment counts: an image's first tiles have
// F fragments, the rest F-1, laid out with BAND offsets (a1: the F tiles,
// a2: the others).  The F tiles are the grid's first n1 blocks, which the
// dispatcher hands out one per CU before any CU takes a second block, so no
// CU holds two of them: a CU's two blocks then hold at most 2F-1 fragment
// columns, where equal tiles of F fragments (of which the image's pixels
// fill F-1/4 on average) hold 2F.
// WMODE 1: the stride-1 dX (the same kernel on G with the flipped filter);
// tile shape does not change any output's sum order, so dX has the bits of
// the plain tiles and of the one-launch backward.
template <int KT, int F, int CB, int R, int S, int ROWS, int PITCH, bool WVEC, int WMODE = 0>
__global__ void __launch_bounds__(256, 2)
    direct_fwd_mix_kernel(const DirectArgs a1, const DirectArgs a2, int n1) {
    if ((int)blockIdx.x < n1)
        direct_fwd_block<KT, F, CB, R, S, ROWS, PITCH, WMODE, 0, WVEC, false, false, 0, 1, true>(
            a1, blockIdx.x, n1);
    else
        direct_fwd_block<KT, F - 1, CB, R, S, ROWS, PITCH, WMODE, 0, WVEC, false, false, 0, 1,
                         true>(a2, blockIdx.x - n1, (int)gridDim.x - n1);
}

// The one-launch backward with the stride-1 dX tiles in two sizes: each
// image holds as many larger first tiles as smaller second ones (BAND
// offsets place each set).  Blocks [nbw, nbw + nx1) take the first tiles
// (dx1, XF1 fragments per wave) and are dispatched beside the dW blocks at
// the start; the rest take the second tiles (dx2, XF2), which the CU slots
// pick up as the first ones retire.  A CU thus runs one dW block beside a
// larger then a smaller dX block, and its two slots end closer together
// than with two equal dX blocks, which outlast the dW block.  Tile shape
// does not change any output's sum order, so dX has the bits of the
// separate call.
template <int XKT, int XF1, int XF2, int XCB, int R, int S, int XROWS, int XPITCH, bool XWVEC,
          int KT, int CT, int ROWS, int PITCH, int GPC, int WKF, bool FULL>
__global__ void __launch_bounds__(256, 2)
    direct_bwd_band_kernel(const DirectArgs dx1, const DirectArgs dx2, const DirectDwArgs dw,
                           int nbw, int nx1) {
    const int b = blockIdx.x;
    if (b < nbw)
        direct_dw_block<KT, CT, R, S, ROWS, PITCH, GPC, WKF, FULL>(dw, b, nbw);
    else if (b - nbw < nx1)
        direct_fwd_block<XKT, XF1, XCB, R, S, XROWS, XPITCH, 1, 0, XWVEC, false, false, 0, 1,
                         true>(dx1, b - nbw, nx1);
    else
        direct_fwd_block<XKT, XF2, XCB, R, S, XROWS, XPITCH, 1, 0, XWVEC, false, false, 0, 1,
                         true>(dx2, b - nbw - nx1, (int)gridDim.x - nbw - nx1);
}

// dw[e] = beta*dw[e] + sum_s part[s][e].  Thread (e4, grp) sums splits
// grp, grp+G, ... in order for four consecutive elements; the G group sums
// are then added in group order.  The summation tree is fixed by (splits,
// G), so the result is identical on every run.  Partial rows are pstride
// floats apart (pstride % 4 == 0, so the float4 loads stay aligned).
template <int G, int U>
__global__ void __launch_bounds__(256) dw_split_reduce(const float *__restrict__ part,
                                                       float *__restrict__ dw, int64_t elems,
                                                       int64_t pstride, int splits, float beta) {
    constexpr int E4 = 256 / G;  // float4 columns per block
    __shared__ float4 red[G][E4];
    const int col = threadIdx.x % E4, grp = threadIdx.x / E4;
    const int64_t e = ((int64_t)blockIdx.x * E4 + col) * 4;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e + 3 < elems) {
        // U loads in flight per thread, then added in split order.
        for (int k0 = grp; k0 < splits; k0 += U * G) {
            float4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int k = k0 + u * G;
                v[u] = k < splits
                    ? *reinterpret_cast<const float4 *>(part + (int64_t)k * pstride + e)
                    : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (k0 + u * G < splits) {
                    s.x += v[u].x;
                    s.y += v[u].y;
                    s.z += v[u].z;
                    s.w += v[u].w;
                }
            }
        }
    } else if (e < elems) {
        for (int k = grp; k < splits; k += G) {
            const float *pk = part + (int64_t)k * pstride + e;
            s.x += pk[0];
            if (e + 1 < elems) s.y += pk[1];
            if (e + 2 < elems) s.z += pk[2];
        }
    }
    red[grp][col] = s;
    __syncthreads();
    if (grp != 0 || e >= elems) return;
    float4 tot = red[0][col];
#pragma unroll
    for (int q = 1; q < G; ++q) {
        const float4 v = red[q][col];
        tot.x += v.x;
        tot.y += v.y;
        tot.z += v.z;
        tot.w += v.w;
    }
    const float tv[4] = {tot.x, tot.y, tot.z, tot.w};
    for (int i = 0; i < 4 && e + i < elems; ++i) store_beta(dw + e + i, tv[i], beta);
}

}  // namespace katsu
