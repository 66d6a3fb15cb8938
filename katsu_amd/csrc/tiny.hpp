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

}  // namespace katsu
