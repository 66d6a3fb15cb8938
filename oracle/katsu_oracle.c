/*
 * katsu_oracle.c -- CPU restatement of Katsu's dense-contraction path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker and the timed
 * CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product path (katsu_amd/) never does.
 *
 * Every function restates one piece of the reference's Rust source
 * (paths relative to the reference repository root):
 *   crates/katsu-core/src/tensor.rs   -- element_count, matmul, Matmul VJP, sum
 *   crates/katsu-core/src/conv2d.rs   -- SplitMix64 init, Geometry, visit,
 *                                        forward, backward_buffers
 * The loop order, the `+=` into a fresh zero buffer (or into an existing
 * pending buffer for the VJPs) and the skipping of padded taps follow the
 * reference exactly.  Built with -O3 -ffp-contract=off and no -ffast-math,
 * every `acc += a*b` is fl(acc + fl(a*b)) as in Rust (which never contracts
 * to FMA), so for the same inputs the results are bit-identical to the Rust
 * arithmetic.
 *
 * Parity pins (each one is a test under tests/):
 *   ko_element_count   -- tests/tensor.rs:4-25 overflow/empty cases
 *   ko_conv_geometry   -- tests/conv2d.rs:119-142,145-169,172-179 and the
 *                         docs/conv2d.md:12-15 formula
 *   ko_conv2d_forward  -- KATs tests/conv2d.rs:22,177; f64 torch conv2d;
 *                         brute force; exact small-integer cases
 *   ko_conv2d_backward -- KATs tests/conv2d.rs:25-26,97-104,114; finite
 *                         differences tests/conv2d.rs:46-87; f64 torch grads
 *   ko_matmul          -- KAT tests/tensor.rs:41-48; f64 numpy; exactness
 *   ko_matmul_vjp      -- KAT tests/autograd.rs:98-103 (aliased pending);
 *                         finite differences tests/autograd.rs:63-95;
 *                         closed forms under G=1
 *   ko_splitmix_fill   -- published SplitMix64 output for seed 0;
 *                         tests/conv2d.rs:145-155 invariants
 *   ko_sum             -- sequential f32 fold, exact small-integer cases
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

/* KO_MUTANT (default 0) plants one known mistake; tests/test_oracle.py builds
 * each mutant separately to show that the pins above catch it. */
#ifndef KO_MUTANT
#define KO_MUTANT 0
#endif

/* Status codes mirror the TensorError variants the path can raise
 * (crates/katsu-core/src/tensor.rs:9-30). */
enum {
    KO_OK = 0,
    KO_SHAPE_OVERFLOW = 1,
    KO_INVALID_CONV = 2,
};

/* Geometry record: the fields of `struct Geometry` (conv2d.rs:168-180). */
enum {
    KO_G_BATCH, KO_G_CIN, KO_G_COUT, KO_G_H, KO_G_W, KO_G_KH, KO_G_KW,
    KO_G_OH, KO_G_OW, KO_G_STRIDE, KO_G_PADDING, KO_G_LEN
};

/* tensor.rs:127-138: zero dims give an empty tensor; otherwise the
 * checked product must also stay below isize::MAX / sizeof(f32). */
int ko_element_count(const uint64_t *shape, size_t rank, uint64_t *out) {
    for (size_t i = 0; i < rank; ++i) {
        if (shape[i] == 0) {
            *out = 0;
            return KO_OK;
        }
    }
    uint64_t count = 1;
    for (size_t i = 0; i < rank; ++i) {
        if (__builtin_mul_overflow(count, shape[i], &count)) return KO_SHAPE_OVERFLOW;
    }
    if (count > ((uint64_t)INT64_MAX) / sizeof(float)) return KO_SHAPE_OVERFLOW;
    *out = count;
    return KO_OK;
}

/* conv2d.rs:156-166 */
static int ko_validate_weights(const uint64_t *wshape, size_t wrank, uint64_t stride) {
    if (wrank != 4) return KO_INVALID_CONV;
    for (size_t i = 0; i < 4; ++i)
        if (wshape[i] == 0) return KO_INVALID_CONV;
    if (stride == 0) return KO_INVALID_CONV;
    return KO_OK;
}

/* conv2d.rs:198-206: floor((size + 2p - kernel) / stride) + 1, every step checked. */
static int ko_output_dim(uint64_t size, uint64_t kernel, uint64_t pad2, uint64_t stride,
                         uint64_t *out) {
    uint64_t padded;
    if (__builtin_add_overflow(size, pad2, &padded)) return KO_SHAPE_OVERFLOW;
    if (padded < kernel) return KO_INVALID_CONV; /* "kernel exceeds padded input" */
    uint64_t q = (padded - kernel) / stride;
    if (__builtin_add_overflow(q, (uint64_t)1, out)) return KO_SHAPE_OVERFLOW;
    return KO_OK;
}

/* Geometry::new, conv2d.rs:183-224, with the checks in the reference's order. */
int ko_conv_geometry(const uint64_t *xshape, size_t xrank, const uint64_t *wshape,
                     size_t wrank, uint64_t stride, uint64_t padding, uint64_t *geo) {
    int st = ko_validate_weights(wshape, wrank, stride);
    if (st) return st;
    if (xrank != 4) return KO_INVALID_CONV;
    if (xshape[1] != wshape[1] || xshape[2] == 0 || xshape[3] == 0) return KO_INVALID_CONV;
    uint64_t tmp;
    st = ko_element_count(xshape + 1, 3, &tmp);
    if (st) return st;
    uint64_t pad2;
    if (__builtin_mul_overflow(padding, (uint64_t)2, &pad2)) return KO_SHAPE_OVERFLOW;
    uint64_t oh, ow;
    st = ko_output_dim(xshape[2], wshape[2], pad2, stride, &oh);
    if (st) return st;
    st = ko_output_dim(xshape[3], wshape[3], pad2, stride, &ow);
    if (st) return st;
    uint64_t s3[3] = {wshape[0], oh, ow};
    st = ko_element_count(s3, 3, &tmp);
    if (st) return st;
    uint64_t s4[4] = {xshape[0], wshape[0], oh, ow};
    st = ko_element_count(s4, 4, &tmp);
    if (st) return st;
    geo[KO_G_BATCH] = xshape[0];
    geo[KO_G_CIN] = xshape[1];
    geo[KO_G_COUT] = wshape[0];
    geo[KO_G_H] = xshape[2];
    geo[KO_G_W] = xshape[3];
    geo[KO_G_KH] = wshape[2];
    geo[KO_G_KW] = wshape[3];
    geo[KO_G_OH] = oh;
    geo[KO_G_OW] = ow;
    geo[KO_G_STRIDE] = stride;
    geo[KO_G_PADDING] = padding;
    return KO_OK;
}

/* One tap coordinate: p = o*stride + k in padded space; valid when
 * p - pad lies in [0, size) (checked_sub + bound, conv2d.rs:242 and 250). */
static inline int ko_tap(uint64_t p, uint64_t pad, uint64_t size, uint64_t *out) {
#if KO_MUTANT == 4
    if (p < pad) { *out = p + size - pad; return *out < size; }
    if (p - pad >= size) { *out = p - pad - size; return *out < size; }
#endif
    if (p < pad || p - pad >= size) return 0;
    *out = p - pad;
    return 1;
}

/* Geometry::visit, conv2d.rs:232-262, expanded once per caller so the
 * closure bodies (conv2d.rs:101-103 and 287-290) stay inline.  Padded taps
 * are skipped, never multiplied by zero (conv2d.rs:241-254). */
#define KO_VISIT(geo, BODY)                                                          \
    do {                                                                             \
        const uint64_t B_ = geo[KO_G_BATCH], CI_ = geo[KO_G_CIN], CO_ = geo[KO_G_COUT]; \
        const uint64_t H_ = geo[KO_G_H], W_ = geo[KO_G_W], KH_ = geo[KO_G_KH];       \
        const uint64_t KW_ = geo[KO_G_KW], OH_ = geo[KO_G_OH], OW_ = geo[KO_G_OW];   \
        const uint64_t S_ = geo[KO_G_STRIDE], P_ = geo[KO_G_PADDING];                \
        for (uint64_t n = 0; n < B_; ++n)                                            \
            for (uint64_t oc = 0; oc < CO_; ++oc)                                    \
                for (uint64_t oy = 0; oy < OH_; ++oy)                                \
                    for (uint64_t ox = 0; ox < OW_; ++ox) {                          \
                        const uint64_t yi = ((n * CO_ + oc) * OH_ + oy) * OW_ + ox;  \
                        for (uint64_t ic = 0; ic < CI_; ++ic)                        \
                            for (uint64_t ky = 0; ky < KH_; ++ky) {                  \
                                uint64_t iy;                                         \
                                if (!ko_tap(oy * S_ + ky, P_, H_, &iy)) continue;    \
                                const uint64_t xbase = ((n * CI_ + ic) * H_ + iy) * W_; \
                                const uint64_t wbase = ((oc * CI_ + ic) * KH_ + ky) * KW_; \
                                for (uint64_t kx = 0; kx < KW_; ++kx) {              \
                                    uint64_t ix;                                     \
                                    if (!ko_tap(ox * S_ + kx, P_, W_, &ix)) continue; \
                                    const uint64_t xi = xbase + ix;                  \
                                    const uint64_t wi = wbase + kx;                  \
                                    BODY;                                            \
                                }                                                    \
                            }                                                        \
                    }                                                                \
    } while (0)

static uint64_t ko_geo_input_numel(const uint64_t *g) {
    return g[KO_G_BATCH] * g[KO_G_CIN] * g[KO_G_H] * g[KO_G_W];
}
static uint64_t ko_geo_weight_numel(const uint64_t *g) {
    return g[KO_G_COUT] * g[KO_G_CIN] * g[KO_G_KH] * g[KO_G_KW];
}
static uint64_t ko_geo_output_numel(const uint64_t *g) {
    return g[KO_G_BATCH] * g[KO_G_COUT] * g[KO_G_OH] * g[KO_G_OW];
}

/* Conv2D::forward, conv2d.rs:95-115: fresh zero output, then
 * data[yi] += x[xi] * w[wi] in visit order (reduction ic -> ky -> kx). */
void ko_conv2d_forward(const float *x, const float *w, float *y, const uint64_t *geo) {
    memset(y, 0, ko_geo_output_numel(geo) * sizeof(float));
#if KO_MUTANT == 1
    KO_VISIT(geo, { y[yi] += x[xi] * w[((oc * CI_ + ic) * KH_ + (KH_ - 1 - ky)) * KW_ + (KW_ - 1 - kx)]; (void)wi; });
#else
    KO_VISIT(geo, { y[yi] += x[xi] * w[wi]; });
#endif
}

/* backward_buffers, conv2d.rs:269-292: fresh zero dx and dw, one visit pass,
 * dx[xi] += g[yi]*w[wi] then dw[wi] += g[yi]*x[xi]. */
void ko_conv2d_backward(const float *x, const float *w, const float *g, float *dx, float *dw,
                        const uint64_t *geo) {
    memset(dx, 0, ko_geo_input_numel(geo) * sizeof(float));
    memset(dw, 0, ko_geo_weight_numel(geo) * sizeof(float));
    KO_VISIT(geo, {
#if KO_MUTANT == 2
        dx[xi] += g[yi] * x[xi];
#else
        dx[xi] += g[yi] * w[wi];
#endif
        dw[wi] += g[yi] * x[xi];
    });
}

/* The dX half of the same visit pass (conv2d.rs:288 only).  Each dx element
 * receives exactly the terms, in exactly the order, that ko_conv2d_backward
 * gives it, so the result is bit-identical; it exists so a sampled parity
 * check or the CPU baseline can time the two halves separately. */
void ko_conv2d_backward_data(const float *w, const float *g, float *dx, const uint64_t *geo) {
    memset(dx, 0, ko_geo_input_numel(geo) * sizeof(float));
    KO_VISIT(geo, { dx[xi] += g[yi] * w[wi]; });
}

/* The dW half (conv2d.rs:289 only); bit-identical to ko_conv2d_backward's dw. */
void ko_conv2d_backward_filter(const float *x, const float *g, float *dw, const uint64_t *geo) {
    memset(dw, 0, ko_geo_weight_numel(geo) * sizeof(float));
    KO_VISIT(geo, { dw[wi] += g[yi] * x[xi]; });
}

/* Tensor::matmul, tensor.rs:264-273: fresh zero C; skipped when C is empty
 * or k == 0; loop i -> p -> j with C[i*n+j] += A[i*k+p] * B[p*n+j]. */
void ko_matmul(const float *a, const float *b, float *c, uint64_t m, uint64_t k, uint64_t n) {
    memset(c, 0, m * n * sizeof(float));
    if (m * n == 0 || k == 0) return;
    for (uint64_t i = 0; i < m; ++i)
        for (uint64_t p = 0; p < k; ++p)
            for (uint64_t j = 0; j < n; ++j) c[i * n + j] += a[i * k + p] * b[p * n + j];
}

/* Op::backward Matmul arm, tensor.rs:418-445.  da and db are the pending
 * buffers and are accumulated into (not overwritten); they may be the same
 * buffer when A and B are the same node, which is why dA runs to completion
 * before dB starts (tensor.rs:425-444). */
void ko_matmul_vjp(const float *a, const float *b, const float *g, float *da, float *db,
                   uint64_t m, uint64_t k, uint64_t n) {
    if (m * n == 0 || k == 0) return; /* g.is_empty() || k == 0, tensor.rs:421-423 */
    for (uint64_t i = 0; i < m; ++i)
        for (uint64_t p = 0; p < k; ++p)
            for (uint64_t j = 0; j < n; ++j)
#if KO_MUTANT == 3
                da[i * k + p] += g[i * n + j] * b[j * k + p];
#else
                da[i * k + p] += g[i * n + j] * b[p * n + j];
#endif
    for (uint64_t i = 0; i < m; ++i)
        for (uint64_t p = 0; p < k; ++p)
            for (uint64_t j = 0; j < n; ++j) db[p * n + j] += a[i * k + p] * g[i * n + j];
}

/* Tensor::sum, tensor.rs:242-247: sequential f32 fold. */
float ko_sum(const float *x, uint64_t n) {
    float acc = 0.0f;
    for (uint64_t i = 0; i < n; ++i) acc += x[i];
    return acc;
}

/* One SplitMix64 step (conv2d.rs:52-56), the published algorithm by
 * Steele, Lea and Flood / Vigna. */
uint64_t ko_splitmix_next(uint64_t *state) {
    *state += 0x9e3779b97f4a7c15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

/* Conv2D::new_seeded weight fill, conv2d.rs:46-59:
 * uniform = (z >> 40) / 2^24 (exact in f32), w = (2*uniform - 1) * bound,
 * bound = 1 / sqrt(fan_in) evaluated in f32 (conv2d.rs:48). */
void ko_splitmix_fill(uint64_t seed, uint64_t fan_in, float *out, uint64_t count) {
    const float bound = 1.0f / sqrtf((float)fan_in);
    uint64_t state = seed;
    for (uint64_t i = 0; i < count; ++i) {
        const uint64_t z = ko_splitmix_next(&state);
        const float uniform = (float)(z >> 40) / 16777216.0f;
        out[i] = (2.0f * uniform - 1.0f) * bound;
    }
}
