// tiny.hpp -- convolutions with few channels (C <= 4 inputs, K <= 16
// outputs, K*C*R*S <= 256), such as config 1's repo example ([1,3,224,224]
// with [8,3,3,3] filters).  Their passes are too small and too narrow for
// the matrix cores (a 16-row MFMA would be half empty at K = 8, and a pass
// is 22 MFLOP), so they run on the vector ALUs, one thread per pixel:
//
//   tiny_fwd_kernel  y[n][k][oy][ox] for every k at one output pixel, summed
//                    over (c, r, s) in the reference's visit order
//                    (conv2d.rs:232-262: ic, ky, kx ascending, padded taps
//                    skipped), each term multiplied and added with separate
//                    roundings, so the result equals the reference's bit for bit;
//   tiny_dx_kernel   dx[n][c][iy][ix] for every c at one input pixel, summed
//                    in the order the reference's scatter (conv2d.rs:286-290)
//                    adds into it: oc ascending, then the output pixels
//                    (oy, ox) ascending, i.e. ky and kx descending; also bit
//                    for bit;
//   tiny_dw_kernel   one partial dw[k][c][r][s] per block over a range of
//                    output rows (one thread per filter element, the rows
//                    staged in LDS), summed by dw_split_reduce in a fixed
//                    order.  The reference's dw is one sequential sum over
//                    every output pixel, which no parallel order reproduces;
//                    this one lies within the f32 summation bound of it.
#pragma once

#include <type_traits>

#include "direct.hpp"

namespace katsu {

struct TinyArgs {
    const float *x, *w, *g;
    float *out;           // y, dx, or the dw partial slices (dw kernel)
    float *out2;          // dw partial slices when one launch writes dx and dw
    int N, C, H, W, K, R, S, OH, OW, st, pad;
    float beta;           // dx: out = beta*out + result (beta in {0, 1})
    int rows_per_block;   // dw: output rows (over the batch) per block
    int xw;               // fwd, dw: staged input columns per row, (OW-1)*st + S
    int64_t pstride;      // dw: floats between partial slices
};

constexpr int kTinyC = 4, kTinyK = 16, kTinyW = 256;  // channel limits; filter elements

// Stages `total` floats into dst[0 .. total) with LDS-direct loads, element
// e from byte offset off(e) of r (kOOB for a zero): every wave load is in
// flight at once, and the caller waits once (wait_lds_dma) before its barrier.
template <class Off>
__device__ __forceinline__ void tiny_stage(__amdgpu_buffer_rsrc_t r, float *dst, int total,
                                           Off off) {
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    for (int base = wv * 64; base < total; base += 256) {
        const int e = base + lane;
        if (e < total) lds_dma_b32(r, dst + base, off(e));
    }
}


// Block b computes output row b of the batch (n = b / OH, oy = b % OH): it
// stages the R input rows under it for every channel (columns
// ox*st - pad ..., zeros outside the image) and the filter in LDS, then each
// thread takes output pixels ox = t, t + 256, ...
// The forward and dX kernels multiply and add with separate roundings (the
// library is built with fp-contract=fast-honor-pragmas), as the reference's
// `+= a * b` does.  The filter sits in LDS transposed to [tap][channel] and
// zero-padded to the channel bucket (KB outputs, 4 inputs), so a tap's
// weights are one or more 16-byte broadcast reads and the channels past the
// layer's are computed and not stored.

// Block b computes output row b of the batch (n = b / OH, oy = b % OH): it
// stages the R input rows under it for every channel (columns
// ox*st - pad ..., zeros outside the image), then each thread takes output
// pixels ox = t, t + 256, ...
template <int KB>
__global__ void __launch_bounds__(256)
    tiny_fwd_kernel(const TinyArgs a, const float *__restrict__ w) {
#pragma clang fp contract(off)
    extern __shared__ float sm[];
    const int crs = a.C * a.R * a.S;
    float *wt = sm;                             // [crs][KB]
    float *xs = sm + ((crs * KB + 3) & ~3);     // [C][R][xw]
    const int t = threadIdx.x;
    for (int i = t; i < crs * KB; i += 256) {
        const int tap = i / KB, k = i - tap * KB;
        wt[i] = k < a.K ? w[k * crs + tap] : 0.f;
    }
    const int n = blockIdx.x / a.OH, oy = blockIdx.x - (blockIdx.x / a.OH) * a.OH;
    const int iy0 = oy * a.st - a.pad;
    const int64_t chw = (int64_t)a.C * a.H * a.W;
    tiny_stage(buf_rsrc(a.x + n * chw, (uint32_t)(chw * 4)), xs, a.C * a.R * a.xw, [&](int e) {
        const int cr = e / a.xw, col = e - cr * a.xw;
        const int c = cr / a.R, iy = iy0 + (cr - c * a.R), ix = col - a.pad;
        return ((unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W)
                   ? ((c * a.H + iy) * a.W + ix) * 4
                   : kOOB;
    });
    wait_lds_dma();
    __syncthreads();
    const int64_t ohw = (int64_t)a.OH * a.OW;
    float *yrow = a.out + (int64_t)n * a.K * ohw + (int64_t)oy * a.OW;
    for (int ox = t; ox < a.OW; ox += 256) {
        float acc[KB];
#pragma unroll
        for (int k = 0; k < KB; ++k) acc[k] = 0.f;
        // Column taps inside the image, as a mask (the reference skips the
        // others, and so does this sum).
        unsigned smask = 0;
#pragma unroll
        for (int s = 0; s < 8; ++s)
            smask |= (s < a.S && (unsigned)(ox * a.st + s - a.pad) < (unsigned)a.W) ? 1u << s : 0u;
        for (int c = 0; c < a.C; ++c)
            for (int r = 0; r < a.R; ++r) {
                // Rows outside the image are skipped, as the reference skips them.
                if ((unsigned)(iy0 + r) >= (unsigned)a.H) continue;
                const float *xr = xs + (c * a.R + r) * a.xw + ox * a.st;
                const float *wr = wt + (c * a.R + r) * a.S * KB;
#pragma unroll
                for (int s = 0; s < 8; ++s) {
                    if (s >= a.S) continue;
                    float wv[KB];
#pragma unroll
                    for (int q = 0; q < KB / 4; ++q) {
                        const floatx4 v = *reinterpret_cast<const floatx4 *>(wr + s * KB + 4 * q);
                        wv[4 * q] = v[0];
                        wv[4 * q + 1] = v[1];
                        wv[4 * q + 2] = v[2];
                        wv[4 * q + 3] = v[3];
                    }
                    const float xv = xr[s];
                    if (!(smask >> s & 1u)) continue;
#pragma unroll
                    for (int k = 0; k < KB; ++k) acc[k] = acc[k] + xv * wv[k];
                }
            }
#pragma unroll
        for (int k = 0; k < KB; ++k)
            if (k < a.K) yrow[k * ohw + ox] = acc[k];
    }
}

// Block b computes input row b of the batch (n = b / H, iy = b % H): it
// stages, for every k, the output row oy that each tap row r reaches
// (oy*st = iy + pad - r; zeros where there is none), then each thread takes
// input pixels ix = t, t + 256, ...
__device__ __forceinline__ void tiny_dx_block(const TinyArgs &a, const float *__restrict__ w,
                                              float *sm, int bid) {
#pragma clang fp contract(off)
    const int crs = a.C * a.R * a.S, rs = a.R * a.S, krs = a.K * rs;
    float *wt = sm;                 // [k][r][s][4]: the 4 input channels' weights
    float *gs = sm + krs * 4;       // [K][R][OW]
    const int t = threadIdx.x;
    for (int i = t; i < krs * 4; i += 256) {
        const int krs_i = i >> 2, c = i & 3;
        const int k = krs_i / rs, rsi = krs_i - k * rs;
        wt[i] = c < a.C ? w[k * crs + c * rs + rsi] : 0.f;
    }
    const int n = bid / a.H, iy = bid - (bid / a.H) * a.H;
    const int64_t ohw = (int64_t)a.OH * a.OW;
    // Tap row r reaches output row (iy + pad - r)/st when that divides.
    unsigned rmask = 0;
    for (int r = 0; r < a.R; ++r) {
        const int ty = iy + a.pad - r;
        const bool ok = ty >= 0 && ty % a.st == 0 && ty / a.st < a.OH;
        rmask |= ok ? 1u << r : 0u;
    }
    tiny_stage(buf_rsrc(a.g + n * a.K * ohw, (uint32_t)(a.K * ohw * 4)), gs, a.K * a.R * a.OW,
               [&](int e) {
                   const int kr = e / a.OW, ox = e - kr * a.OW;
                   const int k = kr / a.R, r = kr - k * a.R;
                   const int ty = iy + a.pad - r;
                   return (rmask >> r & 1u) ? (int)((k * ohw + (ty / a.st) * a.OW + ox) * 4) : kOOB;
               });
    wait_lds_dma();
    __syncthreads();
    const int64_t hw = (int64_t)a.H * a.W;
    float *dxrow = a.out + (int64_t)n * a.C * hw + (int64_t)iy * a.W;
    for (int ix = t; ix < a.W; ix += 256) {
        // Tap column s reaches output column (ix + pad - s)/st when that divides.
        int sidx[8];
        unsigned smask = 0;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int tx = ix + a.pad - s;
            const bool ok = s < a.S && tx >= 0 && tx % a.st == 0 && tx / a.st < a.OW;
            smask |= ok ? 1u << s : 0u;
            sidx[s] = ok ? tx / a.st : 0;
        }
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int k = 0; k < a.K; ++k)
            for (int r = a.R - 1; r >= 0; --r) {
                if (!(rmask >> r & 1u)) continue;
                const float *gr = gs + (k * a.R + r) * a.OW;
                const float *wr = wt + (k * rs + r * a.S) * 4;
#pragma unroll
                for (int s = 7; s >= 0; --s) {
                    if (s >= a.S) continue;
                    const floatx4 wv = *reinterpret_cast<const floatx4 *>(wr + 4 * s);
                    if (!(smask >> s & 1u)) continue;
                    const float gv = gr[sidx[s]];
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[c] = acc[c] + gv * wv[c];
                }
            }
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (c < a.C)
                dxrow[c * hw + ix] = a.beta == 0.f ? acc[c] : dxrow[c * hw + ix] + acc[c];
    }
}

// Block b sums output rows [b*rpb, (b+1)*rpb) of the batch (row = n*OH + oy):
// per row it stages G[n][0..K)[oy][0..OW) and the R input rows of every
// channel under it (columns ox*st - pad .. , zeros outside the image), then
// thread t = ((k*C + c)*R + r)*S + s adds G[k][ox] * x[c][r][ox*st + s] over
// the row's pixels.
__device__ __forceinline__ void tiny_dw_block(const TinyArgs &a, float *sm, int bid) {
    const int t = threadIdx.x;
    const int kcrs = a.K * a.C * a.R * a.S;
    float *gs = sm;                   // [K][OW]
    float *xs = sm + a.K * a.OW;      // [C][R][xw]
    const int rows = a.N * a.OH;
    const int r0 = bid * a.rows_per_block;
    const int r1 = min(r0 + a.rows_per_block, rows);
    int k = 0, c = 0, r = 0, s = 0;
    if (t < kcrs) {
        s = t % a.S;
        r = (t / a.S) % a.R;
        c = (t / (a.S * a.R)) % a.C;
        k = t / (a.S * a.R * a.C);
    }
    const int64_t ohw = (int64_t)a.OH * a.OW;
    const int64_t chw = (int64_t)a.C * a.H * a.W;
    float acc = 0.f;
    int n = r0 / a.OH, oy = r0 - n * a.OH;
    for (int row = r0; row < r1; ++row) {
        tiny_stage(buf_rsrc(a.g + n * a.K * ohw, (uint32_t)(a.K * ohw * 4)), gs, a.K * a.OW,
                   [&](int e) {
                       const int kk = e / a.OW, ox = e - kk * a.OW;
                       return (int)((kk * ohw + (int64_t)oy * a.OW + ox) * 4);
                   });
        const int iy0 = oy * a.st - a.pad;
        tiny_stage(buf_rsrc(a.x + n * chw, (uint32_t)(chw * 4)), xs, a.C * a.R * a.xw,
                   [&](int e) {
                       const int cr = e / a.xw, col = e - cr * a.xw;
                       const int cc = cr / a.R, iy = iy0 + (cr - cc * a.R), ix = col - a.pad;
                       return ((unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W)
                                  ? ((cc * a.H + iy) * a.W + ix) * 4
                                  : kOOB;
                   });
        wait_lds_dma();
        __syncthreads();
        if (t < kcrs && (unsigned)(iy0 + r) < (unsigned)a.H) {
            // Only the pixels whose tap lies inside the image: the reference
            // skips the others (conv2d.rs:240-255), so a non-finite G there
            // never meets the padding's zeros.
            const int gap = a.pad - s, span = a.W - 1 + a.pad - s;
            const int lo = gap > 0 ? (gap + a.st - 1) / a.st : 0;
            const int hi = span < 0 ? -1 : min(a.OW - 1, span / a.st);
            const float *gk = gs + k * a.OW;
            const float *xr = xs + (c * a.R + r) * a.xw + s;
            for (int ox = lo; ox <= hi; ++ox) acc += gk[ox] * xr[ox * a.st];
        }
        __syncthreads();
        if (++oy == a.OH) {
            oy = 0;
            ++n;
        }
    }
    if (t < kcrs) a.out2[(int64_t)bid * a.pstride + t] = acc;
}

__global__ void __launch_bounds__(256)
    tiny_dx_kernel(const TinyArgs a, const float *__restrict__ w) {
    extern __shared__ float sm[];
    tiny_dx_block(a, w, sm, blockIdx.x);
}

__global__ void __launch_bounds__(256) tiny_dw_kernel(const TinyArgs a) {
    extern __shared__ float sm[];
    tiny_dw_block(a, sm, blockIdx.x);
}

// Both backward passes in one launch: blocks [0, N*H) are dX rows, the
// rest dW partials; dynamic LDS is the larger need.
__global__ void __launch_bounds__(256)
    tiny_bwd_kernel(const TinyArgs a, const float *__restrict__ w, int ndx) {
    extern __shared__ float sm[];
    if ((int)blockIdx.x < ndx)
        tiny_dx_block(a, w, sm, blockIdx.x);
    else
        tiny_dw_block(a, sm, blockIdx.x - ndx);
}

// ---------------------------------------------------------------------------
// Register forms for 3x3 filters (config 1's layer).  The row kernels above
// put one block on each image row, which leaves most SIMDs with one wave
// and serialises each block's staging, barrier and compute.  These instead
// give every thread one output element group and no barrier: each thread
// issues all of its loads at once (buffer loads; a padded or absent tap gets
// an out-of-range offset and reads zero without a branch), then sums.  The
// weights are uniform across the block and read as such.  The sums keep the
// orders above, and a padded tap is skipped by a select (acc unchanged), as
// the reference skips it, so the forward and dX equal the reference bit for
// bit whatever the data, NaN and Inf included.

// Forward: thread = (output pixel p of image n, outputs k0 .. k0+KG-1).
// Block b covers pixels [256*(b % pb), +256) of image b / pb; blockIdx.y
// is the output group.  The block's weights go to LDS as [c][r][s][KG]
// (zeros past C and K) while the input loads are in flight.  With finite
// weights a padded tap's zero input adds an exact +-0 to a sum that is never
// -0 (it starts at +0, and round-to-nearest never turns a sum of other
// values into -0), so it leaves the sum as skipping it would; a non-finite
// weight makes the block skip padded taps explicitly.
template <int KG>
__global__ void __launch_bounds__(256)
    tiny3_fwd_kernel(const TinyArgs a, const float *__restrict__ w, int pb) {
#pragma clang fp contract(off)
    constexpr int R = 3, S = 3, CC = kTinyC, NW = CC * R * S * KG;
    static_assert(NW <= 256, "one weight per thread");
    __shared__ float wt[NW];
    __shared__ int nonfinite;
    const int t = threadIdx.x;
    if (t == 0) nonfinite = 0;
    const int n = blockIdx.x / pb, pblk = blockIdx.x - n * pb;
    const int k0 = blockIdx.y * KG;
    const int crs = a.C * R * S;
    // Thread t < NW fetches weight (tap t / KG, output k0 + t % KG), tap =
    // (c*R + r)*S + s; the load is issued first and used after the input
    // loads, so the two round trips overlap.
    const int wq = t % KG, wtap = t / KG;
    const bool wok = t < NW && wtap < crs && k0 + wq < a.K;
    float wraw = w[wok ? (k0 + wq) * crs + wtap : 0];
    const int ohw = a.OH * a.OW;
    const int p0 = pblk * 256 + t;
    const bool live = p0 < ohw;
    const int p = live ? p0 : ohw - 1;
    const int oy = p / a.OW, ox = p - oy * a.OW;
    const int iy0 = oy * a.st - a.pad, ix0 = ox * a.st - a.pad;
    const int hw = a.H * a.W;
    const int64_t chw = (int64_t)a.C * hw;
    const auto rx = buf_rsrc(a.x + n * chw, (uint32_t)(chw * 4));
    bool rok[R], cok[S];
#pragma unroll
    for (int r = 0; r < R; ++r) rok[r] = (unsigned)(iy0 + r) < (unsigned)a.H;
#pragma unroll
    for (int s = 0; s < S; ++s) cok[s] = (unsigned)(ix0 + s) < (unsigned)a.W;
    const int base = iy0 * a.W + ix0;
    float xv[CC][R][S];
#pragma unroll
    for (int c = 0; c < CC; ++c)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const bool v = c < a.C && rok[r] && cok[s];
                xv[c][r][s] = buf_load(rx, v ? (c * hw + base + r * a.W + s) * 4 : kOOB);
            }
    // An unconditional use here keeps the weight load ahead of the input
    // loads (the compiler would otherwise sink it into the store below).
    asm volatile("" : "+v"(wraw));
    __syncthreads();  // nonfinite = 0 is visible before any thread sets it
    if (t < NW) {
        const float wv = wok ? wraw : 0.f;
        wt[t] = wv;
        if (!__builtin_isfinite(wv)) nonfinite = 1;
    }
    __syncthreads();
    const bool skip = nonfinite != 0;
    float acc[KG];
#pragma unroll
    for (int q = 0; q < KG; ++q) acc[q] = 0.f;
    if (!skip) {
#pragma unroll
        for (int c = 0; c < CC; ++c) {
            if (c >= a.C) continue;
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const float *wp = wt + ((c * R + r) * S + s) * KG;
#pragma unroll
                    for (int q = 0; q < KG; ++q) acc[q] = acc[q] + xv[c][r][s] * wp[q];
                }
        }
    } else {
        // A padded tap's product is replaced by +0, which leaves acc as it is.
#pragma unroll
        for (int c = 0; c < CC; ++c) {
            if (c >= a.C) continue;
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const float *wp = wt + ((c * R + r) * S + s) * KG;
                    const bool v = rok[r] && cok[s];
#pragma unroll
                    for (int q = 0; q < KG; ++q) {
                        const float prod = xv[c][r][s] * wp[q];
                        acc[q] = acc[q] + (v ? prod : 0.f);
                    }
                }
        }
    }
    if (!live) return;
    float *yp = a.out + ((int64_t)n * a.K + k0) * ohw + p;
#pragma unroll
    for (int q = 0; q < KG; ++q)
        if (k0 + q < a.K) yp[(int64_t)q * ohw] = acc[q];
}

// dX: thread = (input pixel p of image n, channel c).  Block b covers
// pixels [256*(b % pb), +256) of image (b / pb) % N, channel b / (pb*N).
// Tap r reaches output row (iy + pad - r)/ST when that divides and lies
// inside; the sum runs over k ascending, then r and s descending (the order
// the reference's scatter adds into dx).  The block's weights w[k][c][.][.]
// go to LDS as [k][r][s]; absent taps read G as zero, which (as in the
// forward) leaves the sum unchanged unless a weight is non-finite, when the
// block skips them explicitly.
template <int KB, int ST>
__device__ __forceinline__ void tiny3_dx_block(const TinyArgs &a, const float *__restrict__ w,
                                               float *wt, int pb, int bid) {
#pragma clang fp contract(off)
    constexpr int R = 3, S = 3, NW = KB * R * S;
    static_assert(NW <= 256, "one weight per thread");
    int *nonfinite = reinterpret_cast<int *>(wt + NW);
    const int t = threadIdx.x;
    if (t == 0) *nonfinite = 0;
    const int npb = a.N * pb;
    const int c = bid / npb, rem = bid - c * npb;
    const int n = rem / pb, pblk = rem - n * pb;
    const int crs = a.C * R * S;
    // Thread t < NW fetches w[k][c][r][s] for k = t / (R*S); the load is
    // issued first and used after the G loads, so the round trips overlap.
    const int wk = t / (R * S), wrs = t - wk * (R * S);
    const bool wok = t < NW && wk < a.K;
    float wraw = w[wok ? wk * crs + c * (R * S) + wrs : 0];
    const int hw = a.H * a.W;
    const int p0 = pblk * 256 + t;
    const bool live = p0 < hw;
    const int p = live ? p0 : hw - 1;
    const int iy = p / a.W, ix = p - iy * a.W;
    const int ohw = a.OH * a.OW;
    bool rok[R], cok[S];
    int oyo[R], oxo[S];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int u = iy + a.pad - r;
        rok[r] = u >= 0 && u % ST == 0 && u / ST < a.OH;
        oyo[r] = (u / ST) * a.OW;
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int u = ix + a.pad - s;
        cok[s] = u >= 0 && u % ST == 0 && u / ST < a.OW;
        oxo[s] = u / ST;
    }
    const int64_t kohw = (int64_t)a.K * ohw;
    const auto rg = buf_rsrc(a.g + n * kohw, (uint32_t)(kohw * 4));
    float gv[KB][R][S];
#pragma unroll
    for (int k = 0; k < KB; ++k)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const bool v = k < a.K && rok[r] && cok[s];
                gv[k][r][s] = buf_load(rg, v ? (k * ohw + oyo[r] + oxo[s]) * 4 : kOOB);
            }
    // An unconditional use here keeps the weight load ahead of the G loads
    // (the compiler would otherwise sink it into the store below).
    asm volatile("" : "+v"(wraw));
    __syncthreads();  // *nonfinite = 0 is visible before any thread sets it
    if (t < NW) {
        const float wv = wok ? wraw : 0.f;
        wt[t] = wv;
        if (!__builtin_isfinite(wv)) *nonfinite = 1;
    }
    __syncthreads();
    const bool skip = *nonfinite != 0;
    float acc = 0.f;
    if (!skip) {
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            if (k >= a.K) continue;
#pragma unroll
            for (int r = R - 1; r >= 0; --r)
#pragma unroll
                for (int s = S - 1; s >= 0; --s)
                    acc = acc + gv[k][r][s] * wt[(k * R + r) * S + s];
        }
    } else {
        // An absent tap's product is replaced by +0, which leaves acc as it is.
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            if (k >= a.K) continue;
#pragma unroll
            for (int r = R - 1; r >= 0; --r)
#pragma unroll
                for (int s = S - 1; s >= 0; --s) {
                    const float prod = gv[k][r][s] * wt[(k * R + r) * S + s];
                    acc = acc + (rok[r] && cok[s] ? prod : 0.f);
                }
        }
    }
    if (!live) return;
    float *dp = a.out + ((int64_t)n * a.C + c) * hw + p;
    *dp = a.beta == 0.f ? acc : *dp + acc;
}

// dX with every input channel per thread: thread = input pixel p of image
// b / pb (pixels [256*(b % pb), +256)), C accumulators, each summed in the
// order above.  A block reads G once for all channels.  Weights go to LDS as
// [k][r][s][4] (zeros past C and K).
template <int KB, int ST>
__device__ __forceinline__ void tiny3_dxa_block(const TinyArgs &a, const float *__restrict__ w,
                                                float *wt, int pb, int bid) {
#pragma clang fp contract(off)
    constexpr int R = 3, S = 3, CC = kTinyC, NW = KB * R * S * CC, NL = (NW + 255) / 256;
    int *nonfinite = reinterpret_cast<int *>(wt + NW);
    const int t = threadIdx.x;
    if (t == 0) *nonfinite = 0;
    const int n = bid / pb, pblk = bid - n * pb;
    const int crs = a.C * R * S;
    // Weight slot e = ((k*R + r)*S + s)*CC + c; loads issued first, used
    // after the G loads.
    float wraw[NL];
    bool wok[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int e = t + 256 * j;
        const int c = e % CC, krs = e / CC, k = krs / (R * S), rs = krs - k * (R * S);
        wok[j] = e < NW && k < a.K && c < a.C;
        wraw[j] = w[wok[j] ? k * crs + c * (R * S) + rs : 0];
    }
    const int hw = a.H * a.W;
    const int p0 = pblk * 256 + t;
    const bool live = p0 < hw;
    const int p = live ? p0 : hw - 1;
    const int iy = p / a.W, ix = p - iy * a.W;
    const int ohw = a.OH * a.OW;
    bool rok[R], cok[S];
    int oyo[R], oxo[S];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int u = iy + a.pad - r;
        rok[r] = u >= 0 && u % ST == 0 && u / ST < a.OH;
        oyo[r] = (u / ST) * a.OW;
    }
#pragma unroll
    for (int s2 = 0; s2 < S; ++s2) {
        const int u = ix + a.pad - s2;
        cok[s2] = u >= 0 && u % ST == 0 && u / ST < a.OW;
        oxo[s2] = u / ST;
    }
    const int64_t kohw = (int64_t)a.K * ohw;
    const auto rg = buf_rsrc(a.g + n * kohw, (uint32_t)(kohw * 4));
    float gv[KB][R][S];
#pragma unroll
    for (int k = 0; k < KB; ++k)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int s2 = 0; s2 < S; ++s2) {
                const bool v = k < a.K && rok[r] && cok[s2];
                gv[k][r][s2] = buf_load(rg, v ? (k * ohw + oyo[r] + oxo[s2]) * 4 : kOOB);
            }
#pragma unroll
    for (int j = 0; j < NL; ++j) asm volatile("" : "+v"(wraw[j]));
    __syncthreads();  // *nonfinite = 0 is visible before any thread sets it
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int e = t + 256 * j;
        if (e < NW) {
            const float wv = wok[j] ? wraw[j] : 0.f;
            wt[e] = wv;
            if (!__builtin_isfinite(wv)) *nonfinite = 1;
        }
    }
    __syncthreads();
    const bool skip = *nonfinite != 0;
    float acc[CC];
#pragma unroll
    for (int c = 0; c < CC; ++c) acc[c] = 0.f;
    auto sum = [&](auto masked) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            if (k >= a.K) continue;
#pragma unroll
            for (int r = R - 1; r >= 0; --r)
#pragma unroll
                for (int s2 = S - 1; s2 >= 0; --s2) {
                    const floatx4 wv =
                        *reinterpret_cast<const floatx4 *>(wt + ((k * R + r) * S + s2) * CC);
                    const bool v = rok[r] && cok[s2];
#pragma unroll
                    for (int c = 0; c < CC; ++c) {
                        if (c >= a.C) continue;
                        const float prod = gv[k][r][s2] * wv[c];
                        // Masked: an absent tap's product is replaced by +0.
                        acc[c] = acc[c] + (decltype(masked)::value && !v ? 0.f : prod);
                    }
                }
        }
    };
    if (skip)
        sum(std::true_type{});
    else
        sum(std::false_type{});
    if (!live) return;
    float *dp = a.out + (int64_t)n * a.C * hw + p;
#pragma unroll
    for (int c = 0; c < CC; ++c) {
        if (c >= a.C) continue;
        dp[(int64_t)c * hw] = a.beta == 0.f ? acc[c] : dp[(int64_t)c * hw] + acc[c];
    }
}

#ifndef KATSU_TINY3_DX_ALLC
#define KATSU_TINY3_DX_ALLC 1  // dX threads take every input channel
#endif

template <int KB, int ST>
__global__ void __launch_bounds__(256)
    tiny3_dx_kernel(const TinyArgs a, const float *__restrict__ w, int pb) {
    __shared__ float wt[KB * 9 * kTinyC + 1];  // weights, then the non-finite flag
    if (KATSU_TINY3_DX_ALLC)
        tiny3_dxa_block<KB, ST>(a, w, wt, pb, blockIdx.x);
    else
        tiny3_dx_block<KB, ST>(a, w, wt, pb, blockIdx.x);
}

// dW partials on the matrix cores: per block, dw[k][crs] = sum over its
// output pixels of G[k][p] * X[crs][p] (crs = (c*3 + r)*3 + s, X the input
// tap under pixel p), a 16 x (16*NF) tile fed 4 pixels per
// v_mfma_f32_16x16x4_f32.  Block b of nb takes tiles b, b + nb, ... (tile
// t: pixels [TP*(t % pb), +TP) of image t / pb, TP = 16*STEPS); wave v the
// quarter [TP/4*v, +TP/4) of each, lane l (l/16 = pixel slot q, l%16 = i)
// loading G[k = i] and the taps crs = 16f + i of pixels 4j + q, j < STEPS,
// all in flight at once.  A padded or absent tap reads zero, which leaves a
// finite sum as skipping it would; the four waves' tiles are added in wave
// order through LDS, and a non-finite result is recomputed over the block's
// pixels in the reference's order with padded taps skipped (exact_dw).  The
// partial row goes to out2[b*pstride + k*crs_n + crs] for dw_split_reduce.
template <int NF, int STEPS>
__device__ __forceinline__ void tiny3_dw_block(const TinyArgs &a, float *sm, int pb, int nb,
                                               int bid) {
    constexpr int TP = 16 * STEPS;
    const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int ohw = a.OH * a.OW, hw = a.H * a.W;
    const int64_t chw = (int64_t)a.C * hw, kohw = (int64_t)a.K * ohw;
    const int crs_n = a.C * 9;
    int toff[NF], tr[NF], ts[NF];
    bool tval[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        const int crs = f * 16 + i;
        tval[f] = crs < crs_n;
        const int c = crs / 9, rs = crs - c * 9;
        tr[f] = rs / 3;
        ts[f] = rs - tr[f] * 3;
        toff[f] = c * hw;
    }
    floatx4 acc[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) acc[f] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int ntiles = a.N * pb;
    for (int t = bid; t < ntiles; t += nb) {
        const int n = t / pb, part = t - n * pb;
        const int pbeg = part * TP + wv * (TP / 4);
        const int pend = min(part * TP + TP, ohw);
        const auto rx = buf_rsrc(a.x + n * chw, (uint32_t)(chw * 4));
        const auto rg = buf_rsrc(a.g + n * kohw, (uint32_t)(kohw * 4));
        int p = pbeg + q;
        int oy = p / a.OW, ox = p - (p / a.OW) * a.OW;
        float av[STEPS], bv[STEPS][NF];
#pragma unroll
        for (int j = 0; j < STEPS; ++j) {
            const bool pin = p < pend;
            av[j] = buf_load(rg, pin && i < a.K ? (i * ohw + oy * a.OW + ox) * 4 : kOOB);
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                const int iy = oy * a.st - a.pad + tr[f], ix = ox * a.st - a.pad + ts[f];
                const bool v = pin && tval[f] && (unsigned)iy < (unsigned)a.H &&
                               (unsigned)ix < (unsigned)a.W;
                bv[j][f] = buf_load(rx, v ? (toff[f] + iy * a.W + ix) * 4 : kOOB);
            }
            p += 4;
            ox += 4;  // OW >= 4 (checked by the host): at most one wrap
            if (ox >= a.OW) {
                ox -= a.OW;
                ++oy;
            }
        }
#pragma unroll
        for (int j = 0; j < STEPS; ++j)
#pragma unroll
            for (int f = 0; f < NF; ++f)
                acc[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], bv[j][f], acc[f], 0, 0, 0);
    }
    // The four waves' tiles, added in wave order: element e = (f*64 + l)*4 + v
    // of a tile is D[k = 4*(l/16) + v][crs = 16f + l%16].
    floatx4 *red = reinterpret_cast<floatx4 *>(sm);
#pragma unroll
    for (int f = 0; f < NF; ++f) red[(wv * NF + f) * 64 + lane] = acc[f];
    __syncthreads();
    const float *rs4 = sm;
    for (int e = threadIdx.x; e < NF * 256; e += 256) {
        const int f = e >> 8, l = (e >> 2) & 63, v = e & 3;
        const int k = 4 * (l >> 4) + v, crs = 16 * f + (l & 15);
        float sum = rs4[e];
#pragma unroll
        for (int w = 1; w < 4; ++w) sum = sum + rs4[w * NF * 256 + e];
        if (k >= a.K || crs >= crs_n) continue;
        if (!__builtin_isfinite(sum)) {
            const int c = crs / 9, r = (crs - c * 9) / 3, s2 = crs - c * 9 - r * 3;
            sum = 0.f;
            for (int t = bid; t < ntiles; t += nb) {
                const int n = t / pb, part = t - n * pb;
                const int64_t b0 = (int64_t)n * ohw + (int64_t)part * TP;
                const int64_t b1 = (int64_t)n * ohw + min(part * TP + TP, ohw);
                sum = sum + exact_dw(a.x, a.g, a.C, a.H, a.W, a.K, a.OH, a.OW, a.st, a.pad, k, c,
                                     r, s2, b0, b1);
            }
        }
        a.out2[(int64_t)bid * a.pstride + (int64_t)k * crs_n + crs] = sum;
    }
}

template <int NF, int STEPS>
__global__ void __launch_bounds__(256) tiny3_dw_kernel(const TinyArgs a, int pb) {
    extern __shared__ float sm[];
    tiny3_dw_block<NF, STEPS>(a, sm, pb, (int)gridDim.x, blockIdx.x);
}

// Both backward passes in one launch: blocks [0, ndx) are dX, the rest dW
// partials.
template <int KB, int ST, int NF, int STEPS>
__global__ void __launch_bounds__(256)
    tiny3_bwd_kernel(const TinyArgs a, const float *__restrict__ w, int ndx, int pbx, int pbw) {
    extern __shared__ float sm[];
    if ((int)blockIdx.x < ndx) {
        if (KATSU_TINY3_DX_ALLC)
            tiny3_dxa_block<KB, ST>(a, w, sm, pbx, blockIdx.x);
        else
            tiny3_dx_block<KB, ST>(a, w, sm, pbx, blockIdx.x);
    }
    else
        tiny3_dw_block<NF, STEPS>(a, sm, pbw, (int)gridDim.x - ndx, blockIdx.x - ndx);
}

}  // namespace katsu
