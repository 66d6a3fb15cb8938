/*
 * katsu_hip.h -- C ABI of the MI355X (gfx950) dense-contraction path.
 *
 * This library replaces the four crate-internal kernel seams of Katsu's
 * katsu-core (paths relative to the reference repository root):
 *
 *   S1  matmul forward     crates/katsu-core/src/tensor.rs:264-273
 *   S2  matmul VJPs        crates/katsu-core/src/tensor.rs:424-444
 *   S3  conv forward       crates/katsu-core/src/conv2d.rs:98-103
 *   S4  conv backward      crates/katsu-core/src/conv2d.rs:284-290
 *                          (reached from conv2d.rs:127 and tensor.rs:375)
 *
 * Layouts are the reference's: row-major matrices, NCHW activations, OIHW
 * weights, all contiguous f32.  Every entry point returns a katsu_status;
 * nothing aborts or throws across the ABI.
 *
 * Two families of entry points:
 *   - host-pointer ("drop-in") entry points take the caller's host buffers,
 *     as the reference's slices are, copy them to the device, run on the
 *     library's stream and return once the outputs are written back.  Copies
 *     of 1 MiB or more go through a ring of four pinned 8 MiB host chunks
 *     (allocated on first use, freed by katsu_hip_shutdown), the CPU side of
 *     each chunk split over four threads (environment: KATSU_COPY_THREADS,
 *     KATSU_COPY_CHUNK_MB); the caller's buffers stay pageable;
 *   - *_dev entry points take device pointers and a hipStream_t (passed as
 *     void*, 0 = the null stream) and return right after the launch.
 *
 * Threading: the reference engine is single-threaded (Rc handles,
 * tensor.rs:95-99).  The library's host-side state is guarded by mutexes, so
 * it is safe to call from several threads; the host-pointer entry points
 * share one stream and one staging pool.
 *
 * Library scratch: the *_dev entry points that need device scratch (the dW
 * split partials when no workspace is passed, the GEMM's split-K partials,
 * the sum's chunk partials, Grad-CAM's channel weights) take it from one
 * buffer per purpose that the library keeps and shares across all streams
 * and graphs: an eager call sizes it, and a later capture of the same call
 * on any stream uses it without allocating.  Calls (or graph replays) that
 * overlap in time on different streams race on it; callers that run such
 * calls concurrently order them, or pass their own workspace where the
 * entry point takes one.  A buffer that must grow is replaced and the old
 * block is kept (not freed) until katsu_hip_shutdown, so a graph captured
 * earlier keeps valid addresses.
 *
 * Size limits: empty problems (an output with no elements, or an empty
 * reduction) return KATSU_OK whatever their other dimensions.  Otherwise the
 * kernels index in 32 bits and these entry points return KATSU_E_INVALID
 * (launching nothing) when a bound is exceeded:
 *   matmul:       m, n, k <= 2^31 - 1;
 *   convolutions: C*H*W, K*OH*OW, K*C*R*S, N*H*W, N*OH*OW, pad, stride,
 *                 H + 2*pad and W + 2*pad <= 2^31 - 1.
 */
#ifndef KATSU_HIP_H
#define KATSU_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum katsu_status {
    KATSU_OK = 0,
    KATSU_E_INVALID = 1,  /* bad argument or shape; nothing was launched */
    KATSU_E_NODEVICE = 2, /* no HIP device, or device/runtime init failed */
    KATSU_E_OOM = 3,      /* device allocation failed */
    KATSU_E_LAUNCH = 4,   /* kernel launch, copy or synchronisation failed */
    KATSU_E_SCRATCH = 5,  /* more scratch than the allocation-free entry point holds */
} katsu_status;

/* Convolution geometry, the fields of the reference's `struct Geometry`
 * (conv2d.rs:168-180).  n: batch, c: in channels, h/w: input size,
 * k: out channels, r/s: kernel height/width, stride/pad: equal on both axes
 * (conv2d.rs:11-12), oh/ow: output size.  Callers fill n..pad and either
 * fill oh/ow or call katsu_hip_conv2d_geometry. */
typedef struct katsu_conv_geom {
    uint64_t n, c, h, w, k, r, s, stride, pad, oh, ow;
} katsu_conv_geom;

/* Version string of this library. */
const char *katsu_hip_version(void);

/* Human-readable text for a katsu_status. */
const char *katsu_hip_strerror(int status);

/* Selects the first HIP device and creates the library stream.  Called
 * implicitly by every entry point that needs the device; idempotent. */
int katsu_hip_init(void);

/* Frees the staging pool and workspace and destroys the stream. */
void katsu_hip_shutdown(void);

/* Completes *g: checks it the way Geometry::new does (conv2d.rs:183-224:
 * positive OIHW dims and stride, positive H and W, kernel within the padded
 * input, no size overflow) and writes oh = (h + 2*pad - r)/stride + 1 and
 * ow likewise.  Batch 0 is accepted.  Returns KATSU_E_INVALID otherwise. */
int katsu_hip_conv2d_geometry(katsu_conv_geom *g);

/* ---- S1/S2: matmul ------------------------------------------------------
 * C[m,n] = beta*C + op(A)[m,k] . op(B)[k,n], beta in {0, 1}.
 *   op(A) = A   (A stored [m,k]) when trans_a == 0,
 *           A^T (A stored [k,m]) when trans_a == 1; likewise B.
 * Tensor::matmul (tensor.rs:264-273) is trans_a=0, trans_b=0, beta=0.
 * The Matmul VJP (tensor.rs:424-444) is dA += G.B^T (trans_b=1, beta=1)
 * followed by dB += A^T.G (trans_a=1, beta=1), in that order, because the
 * two pending buffers are the same buffer when A and B are the same node.
 * With beta == 0, C is not read.  k == 0 writes beta*C (tensor.rs:265,421).
 */
int katsu_hip_gemm_f32(const float *a, const float *b, float *c, size_t m, size_t n,
                       size_t k, int trans_a, int trans_b, float beta);
int katsu_hip_gemm_f32_dev(const float *a, const float *b, float *c, size_t m, size_t n,
                           size_t k, int trans_a, int trans_b, float beta, void *stream);

/* The whole Matmul VJP on device buffers (Op::backward Matmul arm,
 * tensor.rs:418-445), for C[m,n] = A[m,k] . B[k,n] with upstream gradient
 * G[m,n]:
 *   da[m,k] = beta_a*da + G . B^T     then     db[k,n] = beta_b*db + A^T . G
 * A NULL da or db skips that product (the parent needs no gradient).  When
 * da and db overlap (A and B the same node) this is exactly
 * katsu_hip_gemm_f32_dev(G, B, da, m, k, n, 0, 1, beta_a) followed by
 * katsu_hip_gemm_f32_dev(A, G, db, k, n, m, 1, 0, beta_b).  Otherwise the
 * two products may run as one launch, whose k-sums can be added in another
 * (fixed) order than those two calls': within the same f32 bound, and the
 * same bits on every call. */
int katsu_hip_matmul_vjp_f32_dev(const float *a, const float *b, const float *g, float *da,
                                 float *db, size_t m, size_t k, size_t n, float beta_a,
                                 float beta_b, void *stream);

/* ---- S3: convolution forward --------------------------------------------
 * y[n,k,oh,ow] = sum over valid (c,r,s) of x[n,c,oy*stride+r-pad,
 * ox*stride+s-pad] * w[k,c,r,s]  (Conv2D::forward, conv2d.rs:95-115;
 * cross-correlation, padded taps contribute nothing).  y is overwritten. */
int katsu_hip_conv2d_fwd_f32(const float *x, const float *w, float *y,
                             const katsu_conv_geom *g);
int katsu_hip_conv2d_fwd_f32_dev(const float *x, const float *w, float *y,
                                 const katsu_conv_geom *g, void *stream);

/* ---- S4: convolution backward (backward_buffers, conv2d.rs:269-292) -----
 * dx = beta*dx + d(sum(gy*y))/dx:   dx[x] += gy[y] * w[w] over the visit.
 * beta = 0 reproduces the fresh buffer of conv2d.rs:284; beta = 1 adds into
 * an engine's pending buffer (tensor.rs:383-390). */
int katsu_hip_conv2d_bwd_data_f32(const float *gy, const float *w, float *dx,
                                  const katsu_conv_geom *g, float beta);
int katsu_hip_conv2d_bwd_data_f32_dev(const float *gy, const float *w, float *dx,
                                      const katsu_conv_geom *g, float beta, void *stream);

/* dw = beta*dw + sum over the visit of gy[y] * x[x]  (conv2d.rs:289).
 * The reduction over n*oh*ow is split across workgroups and reduced in a
 * fixed order, so results are deterministic run to run.
 * The _dev form needs `workspace` of katsu_hip_conv2d_bwd_filter_workspace
 * bytes (device memory, 256-byte aligned); pass NULL to use a library-owned
 * buffer, which is allocated (hipMalloc) on first need and kept. */
int katsu_hip_conv2d_bwd_filter_workspace(const katsu_conv_geom *g, size_t *bytes);
int katsu_hip_conv2d_bwd_filter_f32(const float *x, const float *gy, float *dw,
                                    const katsu_conv_geom *g, float beta);
int katsu_hip_conv2d_bwd_filter_f32_dev(const float *x, const float *gy, float *dw,
                                        const katsu_conv_geom *g, float beta,
                                        void *workspace, size_t workspace_bytes,
                                        void *stream);

/* Both passes of backward_buffers (conv2d.rs:265-292) in one call:
 * dx = beta*dx + dX and dw = beta*dw + dW, as the two calls above make them
 * (same results, same determinism).  When both passes take their direct
 * gfx950 kernels they share one launch, so dW work fills the GPU while the
 * last dX tiles finish.  dx and dw may be the same buffer (an engine's
 * pending buffer when input and weights are one node, so equal sizes): it
 * then receives beta*buf + dX + dW, dX added first, as the reference's adds
 * are ordered (tensor.rs:383-390).  Buffers that overlap without being the
 * same are rejected with KATSU_E_INVALID.  The _dev form takes the
 * workspace of katsu_hip_conv2d_bwd_filter_workspace (or NULL, as above),
 * which covers this call as well as the filter gradient alone. */
int katsu_hip_conv2d_bwd_f32(const float *x, const float *w, const float *gy, float *dx,
                             float *dw, const katsu_conv_geom *g, float beta);
int katsu_hip_conv2d_bwd_f32_dev(const float *x, const float *w, const float *gy, float *dx,
                                 float *dw, const katsu_conv_geom *g, float beta,
                                 void *workspace, size_t workspace_bytes, void *stream);

/* The one-call backward above with no allocation of any kind: no hipMalloc,
 * hipFree or allocating library routine, on any call.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).  The dW
 * split partials live in a static device array of
 * katsu_hip_noalloc_scratch_bytes() bytes (40 MiB), one copy per GPU, held
 * until the process ends; its address on a device is looked up on the first
 * call there.  Same kernels, plans and results as
 * katsu_hip_conv2d_bwd_f32_dev; a geometry whose partials would not fit
 * returns KATSU_E_SCRATCH before any launch (no plan of this library needs
 * more than 37.7 MB).  Every call on a GPU shares that GPU's array, so calls
 * that overlap in time on one GPU (two streams, or two threads) race: the
 * caller orders them. */
int katsu_hip_conv2d_bwd_f32_dev_noalloc(const float *x, const float *w, const float *gy,
                                         float *dx, float *dw, const katsu_conv_geom *g,
                                         float beta, void *stream);
size_t katsu_hip_noalloc_scratch_bytes(void);

/* Number of device allocations (hipMalloc) this library has made since it
 * was loaded: its scratch and staging buffers and the katsu_hip_malloc pool.
 * No counterpart in the reference; it lets a caller that cannot allocate
 * check that a code path allocated nothing (the count does not change). */
uint64_t katsu_hip_device_allocations(void);

/* ---- Device residency and the engine's elementwise work -----------------
 * For callers that keep tensor data on the GPU between calls (a device
 * mirror per immutable node, tensor.rs:96-107), accumulate adjoints in
 * device pending buffers (tensor.rs:327-360) and run the elementwise ops,
 * sum and their VJPs there (tensor.rs:217-247, 392-417).  No reference
 * function corresponds to the buffer calls: the reference has no device.
 *
 * katsu_hip_stream: the library's stream (initialising the library).
 * katsu_hip_malloc/free: device memory from a caching pool; a freed block is
 * reused by later allocations in stream order, so callers that use other
 * streams synchronise before freeing.  All blocks are released by
 * katsu_hip_shutdown.
 * katsu_hip_upload/download: count floats host->device / device->host;
 * both return after the copy completes. */
void *katsu_hip_stream(void);
int katsu_hip_malloc(void **ptr, size_t bytes);
int katsu_hip_free(void *ptr);
int katsu_hip_upload(void *dst, const float *src, size_t count, void *stream);
int katsu_hip_download(float *dst, const void *src, size_t count, void *stream);
int katsu_hip_sync(void *stream);

/* c = beta*c + (a + b) and c = beta*c + a*b over n floats, beta in {0, 1}:
 * Tensor::add / Tensor::mul (tensor.rs:217-240) with beta 0; Mul's VJP
 * pending[a] += g*b (tensor.rs:398-409) with beta 1.  Bit-identical to the
 * reference's loops. */
int katsu_hip_add_f32_dev(const float *a, const float *b, float *c, size_t n, float beta,
                          void *stream);
int katsu_hip_mul_f32_dev(const float *a, const float *b, float *c, size_t n, float beta,
                          void *stream);
/* y = beta*y + x (Add's VJP, tensor.rs:392-397; publishing pending into an
 * existing gradient, tensor.rs:349-357; beta = 0 copies into a buffer the
 * caller knows is still zero).  Bit-identical. */
int katsu_hip_accumulate_f32_dev(const float *x, float *y, size_t n, float beta, void *stream);
/* x = value (fresh zero buffers, tensor.rs:120-125 and 328-331). */
int katsu_hip_fill_f32_dev(float *x, size_t n, float value, void *stream);
/* y = beta*y + s[0] with s on the device (Sum's VJP, tensor.rs:410-417). */
int katsu_hip_add_scalar_f32_dev(const float *s, float *y, size_t n, float beta, void *stream);
/* out[0] = beta*out[0] + sum(x) (Tensor::sum, tensor.rs:242-247).  A fixed
 * tree, identical run to run; it differs from the reference's sequential
 * fold within the f32 summation bound. */
int katsu_hip_sum_f32_dev(const float *x, size_t n, float *out, float beta, void *stream);
/* The stem workload's pooling chain (config 5): out[r] = sum_c y[r][c] / cols,
 * and its VJP dy[r][c] = beta*dy[r][c] + scale*g[r]. */
int katsu_hip_mean_rows_f32_dev(const float *y, size_t rows, size_t cols, float *out,
                                void *stream);
int katsu_hip_broadcast_rows_f32_dev(const float *g, size_t rows, size_t cols, float scale,
                                     float *dy, float beta, void *stream);

/* Grad-CAM over an activation map and its gradient (the raw material
 * get_activation_map provides, conv2d.rs:140-148; the method the reference
 * outlines in docs/conv2d.md, "O que falta para Grad-CAM"), NCHW [n][c][hw]:
 *   alpha[n][c] = mean over hw of grad[n][c][.]
 *   cam[n][p]   = max(0, sum_c alpha[n][c] * act[n][c][p])
 *   then each image's map divided by its maximum (all-zero maps stay zero).
 * cam holds n*hw floats.  No counterpart in the reference's code. */
int katsu_hip_gradcam_f32_dev(const float *act, const float *grad, size_t n, size_t c,
                              size_t hw, float *cam, void *stream);

/* Grad-CAM's last step, resizing each map to the original image
 * (docs/conv2d.md, "O que falta para Grad-CAM": "redimensionar para a imagem
 * original"): n maps [ih][iw] -> dst [n][oh][ow], bilinear with half-pixel
 * centres.  Output row oy samples source row
 * sy = max(0, (oy + 0.5) * ih/oh - 0.5) and blends rows floor(sy) and
 * floor(sy) + 1 (clamped to ih - 1) with weights 1 - f and f,
 * f = sy - floor(sy); columns likewise.  Each blend is rounded as
 * (1 - f)*a + f*b (no fused multiply-add); a neighbour of weight exactly 0 is
 * left out, so NaN or Inf reaches only the outputs that use that pixel.
 * Equal sizes copy every value as it is, non-finite ones included.
 * ih*iw and oh*ow must each be <= 2^31 - 1.  No counterpart in the
 * reference's code. */
int katsu_hip_resize_bilinear_f32_dev(const float *src, size_t n, size_t ih, size_t iw,
                                      size_t oh, size_t ow, float *dst, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* KATSU_HIP_H */
