// exact.hpp -- single convolution outputs recomputed the reference's way.
//
// The MFMA kernels multiply what the reference never touches: the zeros of a
// padded halo (conv2d.rs:240-255 skips padded taps), the zero taps of a
// gathered stride-2 super-filter, and the zeroed lanes and columns that pad
// a tile to whole fragments.  With finite operands each such product is an
// exact 0 and changes nothing.  With a non-finite operand it can be 0 * Inf
// = NaN where the reference's sum is Inf or finite (docs/api.md:34: NaN and
// Inf follow f32 arithmetic over the visited products).  A sum that contains
// such a product is itself non-finite, so a finite MFMA result is already the
// reference's (within the f32 summation bound), and only a non-finite one
// may differ.  The kernels' epilogues therefore test each value they store
// and recompute a non-finite one here: over exactly the reference's visited
// products, in its order (multiply and add rounded separately, as Rust's
// `+= a * b`), from the operands in global memory.  This runs only for
// non-finite data.
//
//   exact_fwd  y[n][co][oy][ox]   (Conv2D::forward, conv2d.rs:95-115)
//   exact_dx   dx[n][c][iy][ix]   (backward_buffers' dx, conv2d.rs:288)
//   exact_dw   dw[k][c][r][s] over a contiguous range of output pixels
//              (backward_buffers' dw, conv2d.rs:289; a split partial)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace katsu {

// Sum over ci, r, s ascending of the valid taps (the visit order,
// conv2d.rs:232-262).  x_img: image n of x, [CI][H][W]; w: [CO][CI][R][S].
__device__ __forceinline__ float exact_fwd_inl(const float *__restrict__ x_img,
                                        const float *__restrict__ w, int CI, int H, int W, int R,
                                        int S, int st, int pad, int co, int oy, int ox) {
#pragma clang fp contract(off)
    float acc = 0.f;
    const int iy0 = oy * st - pad, ix0 = ox * st - pad;
    const float *wc = w + (int64_t)co * CI * R * S;
    for (int ci = 0; ci < CI; ++ci)
        for (int r = 0; r < R; ++r) {
            const int iy = iy0 + r;
            if ((unsigned)iy >= (unsigned)H) continue;
            for (int s = 0; s < S; ++s) {
                const int ix = ix0 + s;
                if ((unsigned)ix >= (unsigned)W) continue;
                acc = acc + x_img[((int64_t)ci * H + iy) * W + ix] * wc[(ci * R + r) * S + s];
            }
        }
    return acc;
}

// The reference scatters dx[x] += g[y] * w[w] in visit order (oc, oy, ox
// ascending for a fixed input element), so the taps arrive with r and s
// descending.  g_img: image n of G, [K][OH][OW]; w: [K][C][R][S].
__device__ __forceinline__ float exact_dx_inl(const float *__restrict__ g_img,
                                       const float *__restrict__ w, int K, int C, int OH, int OW,
                                       int R, int S, int st, int pad, int c, int iy, int ix) {
#pragma clang fp contract(off)
    float acc = 0.f;
    for (int k = 0; k < K; ++k) {
        const float *gk = g_img + (int64_t)k * OH * OW;
        const float *wk = w + ((int64_t)k * C + c) * R * S;
        for (int r = R - 1; r >= 0; --r) {
            const int ty = iy + pad - r;
            if (ty < 0 || ty % st != 0 || ty / st >= OH) continue;
            const int oy = ty / st;
            for (int s = S - 1; s >= 0; --s) {
                const int tx = ix + pad - s;
                if (tx < 0 || tx % st != 0 || tx / st >= OW) continue;
                acc = acc + gk[oy * OW + tx / st] * wk[r * S + s];
            }
        }
    }
    return acc;
}

// dw[k][c][r][s] summed over output pixels p in [pbeg, pend) of the batch
// (p = (n*OH + oy)*OW + ox), ascending, padded taps skipped.  x: [N][C][H][W],
// g: [N][K][OH][OW].
__device__ __forceinline__ float exact_dw_inl(const float *__restrict__ x, const float *__restrict__ g,
                                       int C, int H, int W, int K, int OH, int OW, int st,
                                       int pad, int k, int c, int r, int s, int64_t pbeg,
                                       int64_t pend) {
#pragma clang fp contract(off)
    float acc = 0.f;
    if (pbeg >= pend) return acc;
    const int64_t ohw = (int64_t)OH * OW;
    int64_t n = pbeg / ohw;
    int rem = (int)(pbeg - n * ohw);
    int oy = rem / OW, ox = rem - (rem / OW) * OW;
    for (int64_t p = pbeg; p < pend; ++p) {
        const int iy = oy * st + r - pad, ix = ox * st + s - pad;
        if ((unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W)
            acc = acc + g[(n * K + k) * ohw + (int64_t)oy * OW + ox] *
                            x[((n * C + c) * H + iy) * (int64_t)W + ix];
        if (++ox == OW) {
            ox = 0;
            if (++oy == OH) {
                oy = 0;
                ++n;
            }
        }
    }
    return acc;
}

// Out-of-line forms, for epilogues that call them from a second pass with
// little live state (a call there costs no registers of the MFMA loop); the
// inline forms suit epilogues with few registers in use.
__device__ __noinline__ float exact_fwd(const float *x_img, const float *w, int CI, int H, int W,
                                        int R, int S, int st, int pad, int co, int oy, int ox) {
    return exact_fwd_inl(x_img, w, CI, H, W, R, S, st, pad, co, oy, ox);
}
__device__ __noinline__ float exact_dx(const float *g_img, const float *w, int K, int C, int OH,
                                       int OW, int R, int S, int st, int pad, int c, int iy,
                                       int ix) {
    return exact_dx_inl(g_img, w, K, C, OH, OW, R, S, st, pad, c, iy, ix);
}
__device__ __noinline__ float exact_dw(const float *x, const float *g, int C, int H, int W, int K,
                                       int OH, int OW, int st, int pad, int k, int c, int r, int s,
                                       int64_t pbeg, int64_t pend) {
    return exact_dw_inl(x, g, C, H, W, K, OH, OW, st, pad, k, c, r, s, pbeg, pend);
}

__device__ __forceinline__ bool all_finite4(float a, float b, float c, float d) {
    return __builtin_isfinite(a) && __builtin_isfinite(b) && __builtin_isfinite(c) &&
           __builtin_isfinite(d);
}

}  // namespace katsu
