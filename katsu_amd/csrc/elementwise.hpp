// elementwise.hpp -- the HBM-bound kernels of the device-resident engine:
// the elementwise ops and sum of Tensor (tensor.rs:217-247), their VJPs
// (tensor.rs:392-417), the accumulation of gradients into pending buffers
// (tensor.rs:327-360) and the mean-pool chain of the stem workload.
//
// Every kernel streams its operands once with 16-byte accesses where the
// pointers and length allow, a grid-stride loop sized to the CU count, and
// no LDS except in the reductions.  Reductions are deterministic: a fixed
// assignment of elements to lanes and a fixed combination tree, so a result
// is identical run to run (it differs from the reference's sequential fold
// only within the f32 summation bound).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace katsu {

enum class EwOp { Add, Mul };

// c = beta*c + (a OP b), beta in {0, 1}.  With beta = 1 the two roundings are
// those of `pending[i] += g[i] * other[i]` (tensor.rs:392-409).
template <EwOp OP, bool VEC>
__global__ void __launch_bounds__(256) ew_binary(const float *__restrict__ a,
                                                 const float *__restrict__ b, float *c,
                                                 int64_t n, float beta) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    auto f = [](float x, float y) { return OP == EwOp::Add ? x + y : x * y; };
    if (VEC) {
        const int64_t n4 = n >> 2;
        for (int64_t q = i; q < n4; q += stride) {
            const float4 x = reinterpret_cast<const float4 *>(a)[q];
            const float4 y = reinterpret_cast<const float4 *>(b)[q];
            float4 r = make_float4(f(x.x, y.x), f(x.y, y.y), f(x.z, y.z), f(x.w, y.w));
            float4 *d = reinterpret_cast<float4 *>(c) + q;
            if (beta != 0.f) {
                const float4 o = *d;
                r = make_float4(o.x + r.x, o.y + r.y, o.z + r.z, o.w + r.w);
            }
            *d = r;
        }
        if (i == 0) {  // the last n % 4 elements
            for (int64_t e = n4 << 2; e < n; ++e) {
                const float r = f(a[e], b[e]);
                c[e] = beta != 0.f ? c[e] + r : r;
            }
        }
        return;
    }
    for (; i < n; i += stride) {
        const float r = f(a[i], b[i]);
        c[i] = beta != 0.f ? c[i] + r : r;
    }
}

// y[i] = beta*y[i] + x[i]: an adjoint added into a pending buffer (Add's VJP,
// and the publication of pending into an existing gradient,
// tensor.rs:341-360); beta = 0 copies into a buffer still known to be zero.
template <bool VEC>
__global__ void __launch_bounds__(256) ew_accumulate(const float *__restrict__ x, float *y,
                                                     int64_t n, float beta) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (VEC) {
        const int64_t n4 = n >> 2;
        for (int64_t q = i; q < n4; q += stride) {
            float4 r = reinterpret_cast<const float4 *>(x)[q];
            float4 *d = reinterpret_cast<float4 *>(y) + q;
            if (beta != 0.f) {
                const float4 o = *d;
                r = make_float4(o.x + r.x, o.y + r.y, o.z + r.z, o.w + r.w);
            }
            *d = r;
        }
        i += n4 << 2;  // the last n % 4 elements, one per thread of the first block
        if (i >= n || i >= (n4 << 2) + 4) return;
    }
    for (; i < n; i += stride) y[i] = beta != 0.f ? y[i] + x[i] : x[i];
}

// x[i] = v (fresh zero buffers: a kernel, not a memset, so it can sit in a
// captured graph).
template <bool VEC>
__global__ void __launch_bounds__(256) ew_fill(float *x, int64_t n, float v) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (VEC) {
        const int64_t n4 = n >> 2;
        for (int64_t q = i; q < n4; q += stride)
            reinterpret_cast<float4 *>(x)[q] = make_float4(v, v, v, v);
        i += n4 << 2;
        if (i >= n || i >= (n4 << 2) + 4) return;
    }
    for (; i < n; i += stride) x[i] = v;
}

// y[i] = beta*y[i] + s[0]: Sum's VJP (tensor.rs:410-417) with the scalar
// adjoint on the device.
template <bool VEC>
__global__ void __launch_bounds__(256) ew_add_scalar(const float *__restrict__ s, float *y,
                                                     int64_t n, float beta) {
    const float v = s[0];
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (VEC) {
        const int64_t n4 = n >> 2;
        for (int64_t q = i; q < n4; q += stride) {
            float4 *d = reinterpret_cast<float4 *>(y) + q;
            float4 r = make_float4(v, v, v, v);
            if (beta != 0.f) {
                const float4 o = *d;
                r = make_float4(o.x + v, o.y + v, o.z + v, o.w + v);
            }
            *d = r;
        }
        i += n4 << 2;
        if (i >= n || i >= (n4 << 2) + 4) return;
    }
    for (; i < n; i += stride) y[i] = beta != 0.f ? y[i] + v : v;
}

// Block sum of one value per thread, in a fixed tree (wave shuffles, then
// the four wave sums in order).
__device__ __forceinline__ float block_sum_256(float v) {
    __shared__ float part[4];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off, 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) part[wave] = v;
    __syncthreads();
    float t = 0.f;
    if (threadIdx.x == 0) t = ((part[0] + part[1]) + part[2]) + part[3];
    __syncthreads();
    return t;
}

// Sum, pass 1: block b sums elements [b*chunk, (b+1)*chunk), each thread a
// strided subsequence in order, then the block tree.
// VEC (chunk a multiple of 4, x 16-byte aligned): each thread takes
// float4s and adds their elements in order, then the tail of the last chunk.
template <bool VEC>
__global__ void __launch_bounds__(256) sum_partials(const float *__restrict__ x, int64_t n,
                                                    int64_t chunk, float *part) {
    const int64_t lo = (int64_t)blockIdx.x * chunk;
    const int64_t hi = lo + chunk < n ? lo + chunk : n;
    float v = 0.f;
    int64_t i = lo + threadIdx.x;
    if (VEC) {
        const int64_t h4 = (hi - lo) >> 2;
        const float4 *x4 = reinterpret_cast<const float4 *>(x + lo);
        for (int64_t q = threadIdx.x; q < h4; q += 256) {
            const float4 e = x4[q];
            v += e.x;
            v += e.y;
            v += e.z;
            v += e.w;
        }
        i = lo + (h4 << 2) + threadIdx.x;
    }
    for (; i < hi; i += 256) v += x[i];
    const float t = block_sum_256(v);
    if (threadIdx.x == 0) part[blockIdx.x] = t;
}

// Sum, pass 2: out[0] = beta*out[0] + sum of the `count` partials, in order
// per thread, then the block tree.
__global__ void __launch_bounds__(256) sum_finish(const float *__restrict__ part, int count,
                                                  float *out, float beta) {
    float v = 0.f;
    for (int i = threadIdx.x; i < count; i += 256) v += part[i];
    const float t = block_sum_256(v);
    if (threadIdx.x == 0) out[0] = beta != 0.f ? out[0] + t : t;
}

// out[r] = (sum_h y[r][h]) / hw: one wave per row (the stem's global
// average pool, N*C rows of OH*OW); VEC (hw a multiple of 4, y 16-byte
// aligned): float4 loads, their elements added in order.
template <bool VEC>
__global__ void __launch_bounds__(256) mean_rows(const float *__restrict__ y, int64_t rows,
                                                 int64_t hw, float *out) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float *row = y + r * hw;
    float v = 0.f;
    if (VEC) {
        const float4 *row4 = reinterpret_cast<const float4 *>(row);
        for (int64_t i = lane; i < (hw >> 2); i += 64) {
            const float4 e = row4[i];
            v += e.x;
            v += e.y;
            v += e.z;
            v += e.w;
        }
    } else {
        for (int64_t i = lane; i < hw; i += 64) v += row[i];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off, 64);
    if (lane == 0) out[r] = v / (float)hw;
}

// dy[r][h] = beta*dy[r][h] + g[r]*scale: the mean-pool's VJP.  Block b
// writes part b % bpr (per_block elements, or float4s when VEC: hw a
// multiple of 4, dy 16-byte aligned) of row b / bpr.
template <bool VEC>
__global__ void __launch_bounds__(256) broadcast_rows(const float *__restrict__ g, int64_t hw,
                                                      int bpr, int64_t per_block, float scale,
                                                      float *dy, float beta) {
    const int b = blockIdx.x;
    const int64_t r = b / bpr;
    const float v = g[r] * scale;
    float *row = dy + r * hw;
    const int64_t w = VEC ? hw >> 2 : hw;  // elements (or float4s) of the row
    const int64_t lo = (int64_t)(b - (b / bpr) * bpr) * per_block;
    const int64_t hi = lo + per_block < w ? lo + per_block : w;
    for (int64_t i = lo + threadIdx.x; i < hi; i += 256) {
        if (VEC) {
            float4 *d = reinterpret_cast<float4 *>(row) + i;
            float4 o = make_float4(v, v, v, v);
            if (beta != 0.f) {
                const float4 p = *d;
                o = make_float4(p.x + v, p.y + v, p.z + v, p.w + v);
            }
            *d = o;
        } else {
            row[i] = beta != 0.f ? row[i] + v : v;
        }
    }
}

}  // namespace katsu

namespace katsu {

// Grad-CAM, step 2: cam[n][p] = max(0, sum_c alpha[n][c] * act[n][c][p]),
// channels summed in order; one thread per pixel.
__global__ void __launch_bounds__(256) cam_combine(const float *__restrict__ act,
                                                   const float *__restrict__ alpha, int64_t N,
                                                   int64_t C, int64_t HW, float *cam) {
    const int64_t total = N * HW;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t n = i / HW, p = i - n * HW;
        const float *a = act + n * C * HW + p;
        const float *al = alpha + n * C;
        float v = 0.f;
        for (int64_t c = 0; c < C; ++c) v += al[c] * a[c * HW];
        cam[i] = v > 0.f ? v : 0.f;
    }
}

// Grad-CAM, step 3: each row divided by its maximum (a row with no positive
// value stays zero); one block per row.
__global__ void __launch_bounds__(256) normalize_rows_by_max(float *x, int64_t cols) {
    __shared__ float part[4];
    float *row = x + (int64_t)blockIdx.x * cols;
    float m = 0.f;
    for (int64_t i = threadIdx.x; i < cols; i += 256) m = fmaxf(m, row[i]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_down(m, off, 64));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    if (m <= 0.f) return;
    const float inv = 1.f / m;
    for (int64_t i = threadIdx.x; i < cols; i += 256) row[i] *= inv;
}

// Grad-CAM, step 4: each [IH, IW] map resized to [OH, OW] bilinearly with
// half-pixel centres.  Output row oy samples source row
// sy = max(0, (oy + 0.5) * IH/OH - 0.5); it blends rows floor(sy) and
// floor(sy) + 1 (clamped to the last row) with weights 1 - f and f,
// f = sy - floor(sy); columns likewise.  Each blend is rounded as written,
// (1 - f) * a + f * b with no fused multiply-add, and a neighbour whose
// weight is exactly 0 is left out (so a non-finite pixel reaches only the
// outputs that use it).  Equal sizes copy every pixel as it is.
__device__ __forceinline__ float blend_lin(float a, float b, float f) {
#pragma clang fp contract(off)
    if (f == 0.f) return a;
    if (f == 1.f) return b;
    return (1.f - f) * a + f * b;
}

__global__ void __launch_bounds__(256) resize_bilinear(const float *__restrict__ src, int64_t N,
                                                       int IH, int IW, int OH, int OW,
                                                       float *__restrict__ dst) {
#pragma clang fp contract(off)
    const int64_t ohw = (int64_t)OH * OW, total = N * ohw;
    const bool same = IH == OH && IW == OW;
    const float sh = (float)IH / (float)OH, sw = (float)IW / (float)OW;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        if (same) {
            dst[i] = src[i];
            continue;
        }
        const int64_t n = i / ohw;
        const int p = (int)(i - n * ohw), oy = p / OW, ox = p - (p / OW) * OW;
        const float sy = fmaxf(((float)oy + 0.5f) * sh - 0.5f, 0.f);
        const float sx = fmaxf(((float)ox + 0.5f) * sw - 0.5f, 0.f);
        const int y0 = min((int)sy, IH - 1), x0 = min((int)sx, IW - 1);
        const int y1 = min(y0 + 1, IH - 1), x1 = min(x0 + 1, IW - 1);
        const float fy = fminf(sy - (float)y0, 1.f), fx = fminf(sx - (float)x0, 1.f);
        const float *s = src + n * IH * IW;
        const float top = blend_lin(s[y0 * IW + x0], s[y0 * IW + x1], fx);
        const float bot = blend_lin(s[y1 * IW + x0], s[y1 * IW + x1], fx);
        dst[i] = blend_lin(top, bot, fy);
    }
}

}  // namespace katsu
