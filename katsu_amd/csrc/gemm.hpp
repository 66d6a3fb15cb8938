// gemm.hpp -- the fp32 MFMA GEMM of the matmul seams (tensor.rs:264-273 and
// the VJP, tensor.rs:424-444) for aligned problems: C = beta*C + op(A) op(B)
// with M, N, K multiples of 4 and 16-byte aligned row-major operands.
//
// Block tile BM x BN x BK (BK a multiple of 16), four waves in a 2 x 2 grid, each wave FM x
// FN fragments of 16 x 16 (v_mfma_f32_16x16x4_f32).  Every global load and
// LDS access is 16 bytes wide:
//   * within a 16-deep k block, step s of lane group g (lanes 16g..16g+15)
//     takes k = 4g + s (any bijection works if A and B agree), so an
//     operand stored k-contiguous in LDS ([i][k]) gives one lane its four
//     steps in one ds_read_b128;
//   * an operand stored i-contiguous ([k][i]) is read FM floats at a time
//     across the fragments: fragment a's MFMA row m is tile row FM*m + a;
// and each operand keeps its global orientation in LDS, so staging never
// transposes.  Split-K writes fixed partial slices that the caller reduces
// in a fixed order (dw_split_reduce), so results are run-to-run identical.
#pragma once

#include "direct.hpp"

namespace katsu {

struct GemmArgs {
    const float *a, *b;
    float *c;            // C, or the partial slices when split_stride != 0
    int M, N, K;
    int lda, ldb, ldc;   // row strides of A, B as stored, and of the output
    float beta;          // applied when writing C directly
    int tiles_m, tiles_n, splits, kchunk;  // kchunk: k range of one split (multiple of 16)
    int64_t split_stride;                  // floats between partial slices, or 0
    uint32_t a_bytes, b_bytes;
    int gm;  // register-direct GEMM: tile rows per group of consecutive tiles (divides tiles_m)
};

template <int BM, int BN, int BK_, bool TA, bool TB>
struct GemmGeo {
    static constexpr int BK = BK_;
    static_assert(BK % 16 == 0, "whole 16-deep k blocks");
    // A: TA = 0 stored [i][k] (pitch BK + 4: 16-byte rows, the 8 lanes of an
    //    LDS cycle on distinct banks); TA = 1 stored [k][i] (pitch BM + 4).
    static constexpr int PA = TA ? BM + 4 : BK + 4;
    static constexpr int SA = TA ? BK * PA : BM * PA;
    static constexpr int PB = TB ? BK + 4 : BN + 4;
    static constexpr int SB = TB ? BN * PB : BK * PB;
    static constexpr int STAGE = SA + SB;
    static constexpr size_t kBytes = 2 * (size_t)STAGE * sizeof(float);
};

template <int N>
struct FloatN;
template <>
struct FloatN<1> { using T = float; };
template <>
struct FloatN<2> { using T = float2; };
template <>
struct FloatN<4> { using T = floatx4; };

template <int N>
__device__ __forceinline__ float lane_of(const typename FloatN<N>::T &v, int i) {
    if constexpr (N == 1) return v;
    else if constexpr (N == 2) return i == 0 ? v.x : v.y;
    else return v[i];
}

// WG wave groups of four waves share a block tile: group g takes the tile's
// k-tiles g, g + WG, ... through LDS stages of its own, and the groups' sums
// are added in group order at the end.  Two groups keep two waves on every
// SIMD when the grid has only about one block per CU.
// Block `bid` of the `nb` blocks of problem g (gemm_kernel, or one of the
// two problems of gemm_vjp_kernel).
template <int BM, int BN, int BK_, bool TA, bool TB, int WG>
__device__ __forceinline__ void gemm_block(const GemmArgs &g, int bid, int nb) {
    using Geo = GemmGeo<BM, BN, BK_, TA, TB>;
    static_assert(WG == 1 || WG == 2, "one or two wave groups");
    constexpr int BK = Geo::BK;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 16, FN = WN / 16;
    static_assert(WG == 1 || FM * FN * 4 * 256 <= 2 * WG * Geo::STAGE,
                  "the group hand-off fits in the stages");
    static_assert(FM == 1 || FM == 2 || FM == 4, "FM");
    static_assert(FN == 1 || FN == 2 || FN == 4, "FN");
    constexpr int A4 = BM * BK / 4 / 256;  // float4 loads per thread per tile
    constexpr int B4 = BN * BK / 4 / 256;
    static_assert(A4 >= 1 && B4 >= 1, "tile too small for 256 threads");

    extern __shared__ float smem_all[];
    const int tid = threadIdx.x & 255, grp = threadIdx.x >> 8;
    const int lane = tid & 63, wave = tid >> 6;
    const int wi0 = (wave >> 1) * WM, wj0 = (wave & 1) * WN;
    const int l16 = lane & 15, lg = lane >> 4;
    float *smem = smem_all + grp * 2 * Geo::STAGE;

    const int t = xcd_swizzle(bid, nb);
    const int split = t / (g.tiles_m * g.tiles_n);
    const int tile = t - split * (g.tiles_m * g.tiles_n);
    const int i0 = (tile % g.tiles_m) * BM, j0 = (tile / g.tiles_m) * BN;
    const int kb = split * g.kchunk;
    const int ke = min(kb + g.kchunk, g.K);

    const __amdgpu_buffer_rsrc_t ra = buf_rsrc(g.a, g.a_bytes);
    const __amdgpu_buffer_rsrc_t rb = buf_rsrc(g.b, g.b_bytes);
    floatx4 va[A4], vb[B4];

    // Global float4 of the tile at k0: A (i, k) is a[i*lda + k] (TA = 0) or
    // a[k*lda + i] (TA = 1); B (k, j) is b[k*ldb + j] (TB = 0) or b[j*ldb + k].
    auto load = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < A4; ++q) {
            const int f = q * 256 + tid;
            int off;
            if (!TA) {
                const int i = f / (BK / 4), c = f % (BK / 4);
                const int gi = i0 + i, gk = k0 + 4 * c;
                off = (gi < g.M && gk < ke) ? (gi * g.lda + gk) * 4 : kOOB;
            } else {
                const int k = f / (BM / 4), c = f % (BM / 4);
                const int gk = k0 + k, gi = i0 + 4 * c;
                off = (gk < ke && gi < g.M) ? (gk * g.lda + gi) * 4 : kOOB;
            }
            va[q] = buf_load4(ra, off);
        }
#pragma unroll
        for (int q = 0; q < B4; ++q) {
            const int f = q * 256 + tid;
            int off;
            if (!TB) {
                const int k = f / (BN / 4), c = f % (BN / 4);
                const int gk = k0 + k, gj = j0 + 4 * c;
                off = (gk < ke && gj < g.N) ? (gk * g.ldb + gj) * 4 : kOOB;
            } else {
                const int j = f / (BK / 4), c = f % (BK / 4);
                const int gj = j0 + j, gk = k0 + 4 * c;
                off = (gj < g.N && gk < ke) ? (gj * g.ldb + gk) * 4 : kOOB;
            }
            vb[q] = buf_load4(rb, off);
        }
    };
    auto store = [&](float *st) __attribute__((always_inline)) {
        float *sa = st, *sb = st + Geo::SA;
#pragma unroll
        for (int q = 0; q < A4; ++q) {
            const int f = q * 256 + tid;
            float *d = !TA ? sa + (f / (BK / 4)) * Geo::PA + 4 * (f % (BK / 4))
                           : sa + (f / (BM / 4)) * Geo::PA + 4 * (f % (BM / 4));
            *reinterpret_cast<floatx4 *>(d) = va[q];
        }
#pragma unroll
        for (int q = 0; q < B4; ++q) {
            const int f = q * 256 + tid;
            float *d = !TB ? sb + (f / (BN / 4)) * Geo::PB + 4 * (f % (BN / 4))
                           : sb + (f / (BK / 4)) * Geo::PB + 4 * (f % (BK / 4));
            *reinterpret_cast<floatx4 *>(d) = vb[q];
        }
    };

    floatx4 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};

    // The fragments of one 16-deep k block: step s of lane group lg is
    // k = 16*kq + 4*lg + s.
    struct Frag {
        float a[4][FM], b[4][FN];
    };
    auto read = [&](const float *st, int kq, Frag &fr) __attribute__((always_inline)) {
        const float *sa = st, *sb = st + Geo::SA;
        if (!TA) {
#pragma unroll
            for (int a = 0; a < FM; ++a) {
                const floatx4 v = *reinterpret_cast<const floatx4 *>(
                    sa + (wi0 + 16 * a + l16) * Geo::PA + 16 * kq + 4 * lg);
#pragma unroll
                for (int s = 0; s < 4; ++s) fr.a[s][a] = v[s];
            }
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const auto v = *reinterpret_cast<const typename FloatN<FM>::T *>(
                    sa + (16 * kq + 4 * lg + s) * Geo::PA + wi0 + FM * l16);
#pragma unroll
                for (int a = 0; a < FM; ++a) fr.a[s][a] = lane_of<FM>(v, a);
            }
        }
        if (TB) {
#pragma unroll
            for (int b = 0; b < FN; ++b) {
                const floatx4 v = *reinterpret_cast<const floatx4 *>(
                    sb + (wj0 + 16 * b + l16) * Geo::PB + 16 * kq + 4 * lg);
#pragma unroll
                for (int s = 0; s < 4; ++s) fr.b[s][b] = v[s];
            }
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const auto v = *reinterpret_cast<const typename FloatN<FN>::T *>(
                    sb + (16 * kq + 4 * lg + s) * Geo::PB + wj0 + FN * l16);
#pragma unroll
                for (int b = 0; b < FN; ++b) fr.b[s][b] = lane_of<FN>(v, b);
            }
        }
    };
    auto mma = [&](const Frag &fr) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int a = 0; a < FM; ++a)
#pragma unroll
                for (int b = 0; b < FN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(fr.a[s][a], fr.b[s][b],
                                                                     acc[a][b], 0, 0, 0);
    };
    // LDS reads per k block (b128 for k-contiguous operands, one FloatN per
    // step otherwise) and MFMAs per k block.
    constexpr int RD = (TA ? 4 : FM) + (TB ? FN : 4);
    constexpr int MF = 4 * FM * FN;
    // The BK-deep tile of a stage, software-pipelined: the fragments of k
    // block kq+1 are read while kq's MFMAs run, so a wave alone on its SIMD
    // (one block per CU) still keeps the matrix pipe busy.
    auto compute = [&](const float *st) __attribute__((always_inline)) {
        constexpr int NKQ = BK / 16;
        Frag f0, f1;
        read(st, 0, f0);
        asm volatile("" ::: "memory");
#pragma unroll
        for (int kq = 0; kq < NKQ; kq += 2) {
            if (kq + 1 < NKQ) read(st, kq + 1, f1);
            mma(f0);
            order_reads_then_mfma<RD, MF>();
            if (kq + 1 >= NKQ) break;
            if (kq + 2 < NKQ) read(st, kq + 2, f0);
            mma(f1);
            order_reads_then_mfma<RD, MF>();
        }
    };

    // Rounds of WG k-tiles; every group runs every round (a k-tile past the
    // end loads as zeros), so the block's barriers stay matched.
    const int nrounds = kb < ke ? (int)((ke - kb + WG * BK - 1) / (WG * BK)) : 0;
    auto kof = [&](int r) { return kb + (r * WG + grp) * BK; };
    if (nrounds > 0) {
        float *st0 = smem, *st1 = smem + Geo::STAGE;
        load(kof(0));
        store(st0);
        __syncthreads();
        for (int r = 0; r < nrounds; r += 2) {
            const bool m1 = r + 1 < nrounds, m2 = r + 2 < nrounds;
            if (m1) load(kof(r + 1));
            compute(st0);
            if (m1) store(st1);
            __syncthreads();
            if (!m1) break;
            if (m2) load(kof(r + 2));
            compute(st1);
            if (m2) store(st0);
            __syncthreads();
        }
    }
    if constexpr (WG == 2) {
        // Group 1 hands its sums to group 0 through LDS (the stages are
        // free after the last barrier): value idx of thread tid at idx*256 + tid.
        float *red = smem_all;
        if (grp == 1) {
#pragma unroll
            for (int a = 0; a < FM; ++a)
#pragma unroll
                for (int b = 0; b < FN; ++b)
#pragma unroll
                    for (int v = 0; v < 4; ++v) red[((a * FN + b) * 4 + v) * 256 + tid] = acc[a][b][v];
        }
        __syncthreads();
        if (grp == 1) return;
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int b = 0; b < FN; ++b)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[a][b][v] += red[((a * FN + b) * 4 + v) * 256 + tid];
    }

    // Epilogue: fragment (a, b), register v is row m = 4*lg + v, column n = l16.
    float *out = g.split_stride ? g.c + (int64_t)split * g.split_stride : g.c;
    const bool direct = g.split_stride == 0;
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int m = 4 * lg + v;
            const int gi = i0 + wi0 + (TA ? FM * m + a : 16 * a + m);
            if (gi >= g.M) continue;
            float *row = out + (int64_t)gi * g.ldc;
            if (!TB && FN == 4) {
                const int gj = j0 + wj0 + 4 * l16;
                if (gj < g.N) {
                    floatx4 r = floatx4{acc[a][0][v], acc[a][1][v], acc[a][2][v], acc[a][3][v]};
                    floatx4 *d = reinterpret_cast<floatx4 *>(row + gj);
                    if (direct && g.beta != 0.f) r += *d;
                    *d = r;
                }
            } else {
#pragma unroll
                for (int b = 0; b < FN; ++b) {
                    const int gj = j0 + wj0 + (TB ? 16 * b + l16 : FN * l16 + b);
                    if (gj < g.N) {
                        float *p = row + gj;
                        *p = (direct && g.beta != 0.f) ? *p + acc[a][b][v] : acc[a][b][v];
                    }
                }
            }
        }
}

// ---------------------------------------------------------------------------
// Register-direct GEMM (gemm_rd_*): a 64 x 64 block tile whose KS waves each
// take 1/KS of K, read both operands straight from memory into MFMA operand
// registers (no LDS stage, no barrier in the k-loop) D k-blocks of 16 ahead,
// and add their sums through LDS once, in wave order, at the end (K is
// KS * NKB * 16, the whole k-loop unrolled).  For a
// problem with about one 64 x 64 tile per CU (1024^3) this keeps every SIMD
// on one wave's MFMAs without the per-k-tile barriers of the staged kernel.
//
// Operand registers per k-block of 16 (step s of lane group g is
// k = kb + 4g + s, as in gemm_block):
//   A, TA = 0 ([i][k]): fragment a row m is i0 + 16a + m; one 16-byte load
//      per fragment gives the lane its four steps.
//   A, TA = 1 ([k][i]): fragment a row m is i0 + 4m + a; one 16-byte load per
//      step gives the lane its value in all four fragments.
//   B likewise: TB = 1 ([j][k]) column n of fragment b is j0 + 16b + n, one
//      load per fragment; TB = 0 ([k][j]) column n is j0 + 4n + b, one load
//      per step.
// So a k-block is eight 16-byte loads and 64 MFMAs per wave.
template <bool TA, bool TB, int KS, int NKB, int D>
__device__ __forceinline__ void gemm_rd_block(const GemmArgs &g, int bid, int nb) {
    constexpr int T = 64;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, g4 = lane >> 4;
    const int tile = xcd_swizzle(bid, nb);
    // Tiles in groups of gm tile rows, row fastest within a group: the
    // consecutive tiles one XCD takes cover a patch gm rows tall, so its L2
    // holds fewer operand panels (gm = tiles_m is plain column order).
    const int gsz = g.gm * g.tiles_n, grp = tile / gsz, gi = tile - grp * gsz;
    const int i0 = (grp * g.gm + gi % g.gm) * T, j0 = (gi / g.gm) * T;
    const int kb0 = w * NKB * 16;  // K = KS * NKB * 16 (host-checked)

    const __amdgpu_buffer_rsrc_t ra = buf_rsrc(g.a, g.a_bytes);
    const __amdgpu_buffer_rsrc_t rb = buf_rsrc(g.b, g.b_bytes);
    // Lane parts of the byte offsets (kOOB outside the matrix) and the
    // uniform part per k-block (soffset).  Every in-range lane's address
    // stays inside its operand, whatever soffset's range checking.
    int va[4], vb[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (!TA) {
            const int i = i0 + 16 * q + l16;
            va[q] = i < g.M ? (i * g.lda + 4 * g4) * 4 : kOOB;
        } else {
            const int i = i0 + 4 * l16;
            va[q] = i < g.M ? ((4 * g4 + q) * g.lda + i) * 4 : kOOB;
        }
        if (TB) {
            const int j = j0 + 16 * q + l16;
            vb[q] = j < g.N ? (j * g.ldb + 4 * g4) * 4 : kOOB;
        } else {
            const int j = j0 + 4 * l16;
            vb[q] = j < g.N ? ((4 * g4 + q) * g.ldb + j) * 4 : kOOB;
        }
    }
    // Byte advance of one k-block: along k within a row (k-contiguous
    // operand) or 16 rows (otherwise).
    const int sa = TA ? 16 * g.lda * 4 : 64, sbk = TB ? 64 : 16 * g.ldb * 4;
    const int a_k0 = TA ? kb0 * g.lda * 4 : kb0 * 4, b_k0 = TB ? kb0 * 4 : kb0 * g.ldb * 4;

    // fr[slot][0][q]: A load q, fr[slot][1][q]: B load q.
    floatx4 fr[D][2][4];
    auto fetch = [&](int slot, int kblk) __attribute__((always_inline)) {
        const int oa = a_k0 + kblk * sa, ob = b_k0 + kblk * sbk;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            fr[slot][0][q] = __builtin_bit_cast(
                floatx4, __builtin_amdgcn_raw_buffer_load_b128(ra, va[q], oa, 0));
#pragma unroll
        for (int q = 0; q < 4; ++q)
            fr[slot][1][q] = __builtin_bit_cast(
                floatx4, __builtin_amdgcn_raw_buffer_load_b128(rb, vb[q], ob, 0));
    };
    floatx4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};

    // The whole k-loop unrolled (NKB blocks): the ring of D blocks in flight
    // is then plain data flow, and each block waits only for its own loads.
#pragma unroll
    for (int p = 0; p < D && p < NKB; ++p) fetch(p, p);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
        floatx4 cur[2][4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            cur[0][q] = fr[kb % D][0][q];
            cur[1][q] = fr[kb % D][1][q];
        }
        const bool refill = kb + D < NKB;
        if (refill) fetch(kb % D, kb + D);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const float av = TA ? cur[0][s][a] : cur[0][a][s];
                    const float bv = TB ? cur[1][b][s] : cur[1][s][b];
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[a][b], 0, 0, 0);
                }
        if (refill) __builtin_amdgcn_sched_group_barrier(0x020, 8, 0);  // the refill
        __builtin_amdgcn_sched_group_barrier(0x008, 64, 0);             // then the MFMAs
        // Nothing crosses a block boundary: the scheduler would otherwise
        // sink each refill to the block that uses it.
        __builtin_amdgcn_sched_barrier(0);
    }

    // Row and column of fragment (a, b), register v, this lane.
    auto row_of = [&](int a, int v) { const int m = 4 * g4 + v; return TA ? i0 + 4 * m + a : i0 + 16 * a + m; };
    auto col_of = [&](int b) { return TB ? j0 + 16 * b + l16 : j0 + 4 * l16 + b; };
    auto put = [&](int a, int v, const float *val) __attribute__((always_inline)) {
        const int i = row_of(a, v);
        if (i >= g.M) return;
        float *row = g.c + (int64_t)i * g.ldc;
        if (!TB) {
            const int j = j0 + 4 * l16;
            if (j >= g.N) return;
            floatx4 r = floatx4{val[0], val[1], val[2], val[3]};
            floatx4 *d = reinterpret_cast<floatx4 *>(row + j);
            if (g.beta != 0.f) r += *d;
            *d = r;
        } else {
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int j = col_of(b);
                if (j < g.N) row[j] = g.beta != 0.f ? row[j] + val[b] : val[b];
            }
        }
    };
    if constexpr (KS == 1) {
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float val[4] = {acc[a][0][v], acc[a][1][v], acc[a][2][v], acc[a][3][v]};
                put(a, v, val);
            }
    } else {
        // The waves' sums through LDS: value idx = (a*4 + v)*4 + b of wave p
        // at part[p][idx*64 + lane]; wave w then adds, in wave order, the
        // (a, v) groups [w*16/KS, (w+1)*16/KS) and stores them.
        extern __shared__ float part[];
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    part[(w * 64 + (a * 4 + v) * 4 + b) * 64 + lane] = acc[a][b][v];
        __syncthreads();
        constexpr int GPW = 16 / KS;  // (a, v) groups per wave
#pragma unroll
        for (int e = 0; e < GPW; ++e) {
            const int av = w * GPW + e, a = av >> 2, v = av & 3;
            float val[4];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                float t = part[(av * 4 + b) * 64 + lane];
#pragma unroll
                for (int p = 1; p < KS; ++p) t += part[(p * 64 + av * 4 + b) * 64 + lane];
                val[b] = t;
            }
            put(a, v, val);
        }
    }
}

template <bool TA, bool TB, int KS, int NKB, int D, int OCC>
__global__ void __launch_bounds__(64 * KS, OCC) gemm_rd_kernel(const GemmArgs g) {
    gemm_rd_block<TA, TB, KS, NKB, D>(g, blockIdx.x, gridDim.x);
}

// One 64 x 64 tile of a register-direct problem, as gemm_rd_block lays it
// out: its operand resources, the lane parts of its operand offsets and
// their per-k-block advance.
template <bool TA, bool TB, int NKB>
struct RdTile {
    __amdgpu_buffer_rsrc_t ra, rb;
    int va[4], vb[4];
    int sa, sbk, a_k0, b_k0, i0, j0;

    __device__ __forceinline__ void init(const GemmArgs &g, int tile, int w, int lane) {
        const int l16 = lane & 15, g4 = lane >> 4;
        const int gsz = g.gm * g.tiles_n, grp = tile / gsz, gi = tile - grp * gsz;
        i0 = (grp * g.gm + gi % g.gm) * 64;
        j0 = (gi / g.gm) * 64;
        const int kb0 = w * NKB * 16;
        ra = buf_rsrc(g.a, g.a_bytes);
        rb = buf_rsrc(g.b, g.b_bytes);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (!TA) {
                const int i = i0 + 16 * q + l16;
                va[q] = i < g.M ? (i * g.lda + 4 * g4) * 4 : kOOB;
            } else {
                const int i = i0 + 4 * l16;
                va[q] = i < g.M ? ((4 * g4 + q) * g.lda + i) * 4 : kOOB;
            }
            if (TB) {
                const int j = j0 + 16 * q + l16;
                vb[q] = j < g.N ? (j * g.ldb + 4 * g4) * 4 : kOOB;
            } else {
                const int j = j0 + 4 * l16;
                vb[q] = j < g.N ? ((4 * g4 + q) * g.ldb + j) * 4 : kOOB;
            }
        }
        sa = TA ? 16 * g.lda * 4 : 64;
        sbk = TB ? 64 : 16 * g.ldb * 4;
        a_k0 = TA ? kb0 * g.lda * 4 : kb0 * 4;
        b_k0 = TB ? kb0 * 4 : kb0 * g.ldb * 4;
    }
    // The eight 16-byte loads of k-block kblk: dst[0][q] A, dst[1][q] B.
    __device__ __forceinline__ void fetch(floatx4 (&dst)[2][4], int kblk) const {
        const int oa = a_k0 + kblk * sa, ob = b_k0 + kblk * sbk;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            dst[0][q] = __builtin_bit_cast(
                floatx4, __builtin_amdgcn_raw_buffer_load_b128(ra, va[q], oa, 0));
#pragma unroll
        for (int q = 0; q < 4; ++q)
            dst[1][q] = __builtin_bit_cast(
                floatx4, __builtin_amdgcn_raw_buffer_load_b128(rb, vb[q], ob, 0));
    }
};

// The 64 MFMAs of one k-block (gemm_rd_block's order).
template <bool TA, bool TB>
__device__ __forceinline__ void rd_mma(floatx4 (&acc)[4][4], const floatx4 (&cur)[2][4]) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const float av = TA ? cur[0][s][a] : cur[0][a][s];
                const float bv = TB ? cur[1][b][s] : cur[1][s][b];
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[a][b], 0, 0, 0);
            }
}

// The KS waves' sums added through LDS in wave order and stored, as at the
// end of gemm_rd_block (KS > 1).
template <bool TA, bool TB, int KS>
__device__ __forceinline__ void rd_store(const GemmArgs &g, const floatx4 (&acc)[4][4], int i0,
                                         int j0, int w, int lane, float *part) {
    const int l16 = lane & 15, g4 = lane >> 4;
    auto put = [&](int a, int v, const float *val) __attribute__((always_inline)) {
        const int m = 4 * g4 + v;
        const int i = TA ? i0 + 4 * m + a : i0 + 16 * a + m;
        if (i >= g.M) return;
        float *row = g.c + (int64_t)i * g.ldc;
        if (!TB) {
            const int j = j0 + 4 * l16;
            if (j >= g.N) return;
            floatx4 r = floatx4{val[0], val[1], val[2], val[3]};
            floatx4 *d = reinterpret_cast<floatx4 *>(row + j);
            if (g.beta != 0.f) r += *d;
            *d = r;
        } else {
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int j = j0 + 16 * b + l16;
                if (j < g.N) row[j] = g.beta != 0.f ? row[j] + val[b] : val[b];
            }
        }
    };
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                part[(w * 64 + (a * 4 + v) * 4 + b) * 64 + lane] = acc[a][b][v];
    __syncthreads();
    constexpr int GPW = 16 / KS;
#pragma unroll
    for (int e = 0; e < GPW; ++e) {
        const int av = w * GPW + e, a = av >> 2, v = av & 3;
        float val[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            float t = part[(av * 4 + b) * 64 + lane];
#pragma unroll
            for (int p = 1; p < KS; ++p) t += part[(p * 64 + av * 4 + b) * 64 + lane];
            val[b] = t;
        }
        put(a, v, val);
    }
}

// The matmul VJP's dA (NT, nt) and dB (TN, tn) tiles of the same index in
// one block, one after the other: the loads of dB's first D k-blocks are
// issued during dA's last D k-blocks (the ring of loads in flight runs on
// from one product into the next), so the second tile starts without a
// load round trip, and dA's store epilogue overlaps dB's first loads.  Each
// tile's loads, MFMAs and wave-order sum are those of gemm_rd_block, so the
// bits are those of the two products computed apart.  Both problems have
// the same tile grid (nb tiles).
template <int KS, int NKB, int D>
__device__ __forceinline__ void gemm_rd_pair_block(const GemmArgs &nt, const GemmArgs &tn, int bid,
                                                   int nb) {
    static_assert(KS > 1, "the waves' sums go through LDS");
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tile = xcd_swizzle(bid, nb);
    extern __shared__ float part[];
    RdTile<false, true, NKB> t0;
    RdTile<true, false, NKB> t1;
    t0.init(nt, tile, w, lane);
    t1.init(tn, tile, w, lane);

    floatx4 fr[D][2][4];
    floatx4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < D && p < NKB; ++p) t0.fetch(fr[p], p);
    // dA: k-block kb sits in slot kb % D; the refill of its slot is block
    // kb + D of dA, or past dA's end, block kb + D - NKB of dB.
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
        floatx4 cur[2][4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            cur[0][q] = fr[kb % D][0][q];
            cur[1][q] = fr[kb % D][1][q];
        }
        if (kb + D < NKB)
            t0.fetch(fr[kb % D], kb + D);
        else if (kb + D - NKB < NKB)
            t1.fetch(fr[kb % D], kb + D - NKB);
        rd_mma<false, true>(acc, cur);
        __builtin_amdgcn_sched_group_barrier(0x020, 8, 0);   // the refill
        __builtin_amdgcn_sched_group_barrier(0x008, 64, 0);  // then the MFMAs
        __builtin_amdgcn_sched_barrier(0);
    }
    rd_store<false, true, KS>(nt, acc, t0.i0, t0.j0, w, lane, part);
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};
    // dB: k-block kb sits in slot (NKB + kb) % D.
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
        constexpr int kOff = NKB % D;
        const int slot = (kOff + kb) % D;
        floatx4 cur[2][4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            cur[0][q] = fr[slot][0][q];
            cur[1][q] = fr[slot][1][q];
        }
        const bool refill = kb + D < NKB;
        if (refill) t1.fetch(fr[slot], kb + D);
        rd_mma<true, false>(acc, cur);
        if (refill) __builtin_amdgcn_sched_group_barrier(0x020, 8, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 64, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
    // dA's sums in LDS may still be read by a wave that is behind.
    __syncthreads();
    rd_store<true, false, KS>(tn, acc, t1.i0, t1.j0, w, lane, part);
}

template <int KS, int NKB, int D>
__global__ void __launch_bounds__(64 * KS, 1)
    gemm_rd_vjp_pair_kernel(const GemmArgs nt, const GemmArgs tn) {
    gemm_rd_pair_block<KS, NKB, D>(nt, tn, blockIdx.x, gridDim.x);
}

// The matmul VJP's dA (NT) and dB (TN) in one register-direct launch (see
// gemm_vjp_kernel for the block split).
template <int KS, int NKB, int D, int OCC>
__global__ void __launch_bounds__(64 * KS, OCC)
    gemm_rd_vjp_kernel(const GemmArgs nt, const GemmArgs tn, int nb0) {
    if ((int)blockIdx.x < nb0)
        gemm_rd_block<false, true, KS, NKB, D>(nt, blockIdx.x, nb0);
    else
        gemm_rd_block<true, false, KS, NKB, D>(tn, blockIdx.x - nb0, gridDim.x - nb0);
}

template <int BM, int BN, int BK_, bool TA, bool TB, int WG>
__global__ void __launch_bounds__(256 * WG, 2 / WG) gemm_kernel(const GemmArgs g) {
    gemm_block<BM, BN, BK_, TA, TB, WG>(g, blockIdx.x, gridDim.x);
}

// The matmul VJP's two products in one launch (tensor.rs:424-444): blocks
// [0, nb0) compute dA = beta*dA + G B^T (NT), the rest dB = beta*dB + A^T G
// (TN).  The host uses it only when dA and dB do not overlap, so the two
// results are those of the two launches in the reference's order.  nb0 is a
// multiple of 8, so each problem's blocks keep their XCD placement.
template <int BM, int BN, int BK_, int WG>
__global__ void __launch_bounds__(256 * WG, 2 / WG)
    gemm_vjp_kernel(const GemmArgs nt, const GemmArgs tn, int nb0) {
    if ((int)blockIdx.x < nb0)
        gemm_block<BM, BN, BK_, false, true, WG>(nt, blockIdx.x, nb0);
    else
        gemm_block<BM, BN, BK_, true, false, WG>(tn, blockIdx.x - nb0, gridDim.x - nb0);
}

}  // namespace katsu
