/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_mx.hip -- MXFP4 matrix kernels for gfx950.
 *
 * mx_gemm: grouped "weights x activations" on the bf16 matrix cores, weights read
 * straight out of packed MXFP4. Replaces the arithmetic of the reference's
 * k3_matmul_mxfp4 (src/core/k3_ops.c:1380-1785) for every shape the MoE path uses.
 *
 *   One wave owns MT row tiles of 16 weight rows and NT token tiles of 16 activation
 *   rows and walks K in steps of 256 elements (8 MX blocks). In a step, lane l (row
 *   r = l%16 of each tile, lane group g = l/16) loads 32 contiguous bytes = two whole MX
 *   blocks (8s+2g, 8s+2g+1) of its row with two 16-byte loads, plus the two scale
 *   bytes. Four lanes of a group therefore read 128 contiguous bytes of one row and a
 *   wave instruction touches 16 full rows' worth of one cache line each.
 *
 *   The 64 codes a lane holds are expanded in registers by v_cvt_scalef32_pk_bf16_fp4,
 *   which writes E2M1 * 2^(s-127) as bf16. That is exact for every scale byte 0..254
 *   (a 3-bit mantissa times a power of two; bf16 has fp32's exponent range and keeps
 *   subnormals here), so the weights enter the MFMA exactly; a block whose scale byte is
 *   255 has its codes zeroed, contributing nothing as in the reference.
 *
 *   v_mfma_f32_16x16x32_bf16 sums over 32 k-slots: lane group g supplies slots 8g..8g+7.
 *   Because the contraction is a sum, which activation element a slot carries is free as
 *   long as A and B agree; here slot i of group g in sub-step (kb, p) is element
 *   (8s+2g+kb)*32 + 8p + i, i.e. each lane feeds a whole block of its own row across the
 *   eight sub-steps, so no lane ever needs bytes another lane loaded.
 *
 *   Activations are fp32 in the reference. They arrive split into bf16 hi + lo
 *   (x = hi + lo + r, |r| <= 2^-17|x|) and each sub-step issues one MFMA per term, so the
 *   products are those of a 16-bit-mantissa activation against the exact weight and the
 *   accumulation is fp32: far inside max|err| <= 1e-4 ||ref||inf. With nsplit == 1 the
 *   activation is rounded to bf16 once (the prefill precision mode).
 *
 *   kw waves of one workgroup may split one item's K range; their fp32 partials are
 *   summed through LDS in wave order, so the result is deterministic for a given launch
 *   shape.
 *
 * Modes:
 *   PLAIN  one matrix, activation rows 0..ntok-1, y[tok][row].
 *   GATEUP expert jobs from the gather; tiles 0..MT/2-1 are gate rows, MT/2.. the same
 *          rows of up; the activation (SiLU or SiTU) is applied in registers and written
 *          as its own bf16 split, [assignment][inter], ready to be the next B operand.
 *   DOWN   expert jobs; activation rows are assignments; contrib[assignment][hidden].
 */
#include "k3_common.h"
#include "k3_select.h"

#include <type_traits>
#include <utility>
#include "k3k.h"

namespace {

/* f(std::integral_constant<int, s>{}) for s = 0 .. N-1, unrolled at compile time (register
 * slots of a load ring must be indexed by constants) */
template <typename F, int... S>
__device__ __forceinline__ void k3_static_for_impl(F &&f, std::integer_sequence<int, S...>)
{
    (f(std::integral_constant<int, S>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void k3_static_for(F &&f)
{
    k3_static_for_impl(f, std::make_integer_sequence<int, N>{});
}

struct ExpertQDev {
    const uint8_t *p1, *s1, *p3, *s3, *p2, *s2;
};

__device__ __forceinline__ uint4 ld16(const uint8_t *p)
{
    return k3_ldg16(p);
}

template <int MODE, int MT, int NT, int NS, int DEPTH, int MAXW>
__global__ __launch_bounds__(64 * MAXW) void mx_gemm_kernel(K3kMxArgs a, int kw)
{
    constexpr int RT = (MODE == K3K_MX_GATEUP) ? MT / 2 : MT;   /* output row tiles */
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int K = a.K, nblk = K >> 5, nsteps = (nblk + 3) >> 2;
    const int rows = a.rows;
    const size_t rstride = (size_t)K >> 1;                 /* packed bytes per row */
    const int n_rb = (rows + 16 * RT - 1) / (16 * RT);
    const int ptok = NT * 16;

    int n_items;
    if (MODE == K3K_MX_PLAIN) n_items = n_rb * ((a.ntok + ptok - 1) / ptok);
    else n_items = (*a.n_passes) * n_rb;

    /* This wave's share of the K steps (each step: 4 MX blocks = 128 elements). */
    const int s0 = (wv * nsteps) / kw, s1 = ((wv + 1) * nsteps) / kw;

    __shared__ k3_f32x4 red[MAXW - 1][MT * NT][64];

    for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
        const int rb = item % n_rb, pass = item / n_rb;
        int tok0, tok1, off = 0;
        const uint8_t *pa[MT];
        const uint8_t *sa[MT];
        if (MODE == K3K_MX_PLAIN) {
            tok0 = pass * ptok;
            tok1 = min(tok0 + ptok, a.ntok);
            for (int m = 0; m < MT; m++) { pa[m] = a.packed; sa[m] = a.scales; }
        } else {
            const int j = a.pass_job[pass];
            const int e = a.job_expert[j];
            off = a.job_off[j];
            tok0 = a.pass_tp[pass] * ptok;
            tok1 = min(tok0 + ptok, a.job_cnt[j]);
            const ExpertQDev q = reinterpret_cast<const ExpertQDev *>(a.bank)[e];
            for (int m = 0; m < MT; m++) {
                if (MODE == K3K_MX_GATEUP) {
                    pa[m] = m < RT ? q.p1 : q.p3;
                    sa[m] = m < RT ? q.s1 : q.s3;
                } else {
                    pa[m] = q.p2;
                    sa[m] = q.s2;
                }
            }
        }
        /* Row base pointers for this lane (rows past the end re-read the last row; their
         * results are discarded). */
        for (int m = 0; m < MT; m++) {
            const int mt = (MODE == K3K_MX_GATEUP) ? (m % RT) : m;
            const int r = min(rb * 16 * RT + 16 * mt + r16, rows - 1);
            pa[m] += (size_t)r * rstride;
            sa[m] += (size_t)r * nblk;
        }

        /* This lane's activation rows (column r16 of each token tile). */
        const uint16_t *xh[NT];
        const uint16_t *xl[NT];
        bool tv[NT];
        for (int nt = 0; nt < NT; nt++) {
            const int ti = tok0 + nt * 16 + r16;
            tv[nt] = ti < tok1;
            int xr = 0;
            if (tv[nt]) {
                if (MODE == K3K_MX_PLAIN) xr = ti;
                else if (MODE == K3K_MX_GATEUP) xr = a.perm[off + ti] / a.topk;
                else xr = a.perm[off + ti];
            }
            xh[nt] = a.xhi + (size_t)xr * K;
            xl[nt] = NS == 2 ? a.xlo + (size_t)xr * K : nullptr;
        }

        k3_f32x4 acc[MT][NT];
        for (int m = 0; m < MT; m++)
            for (int nt = 0; nt < NT; nt++) acc[m][nt] = k3_f32x4{0.f, 0.f, 0.f, 0.f};

        for (int s = s0; s < s1; s += DEPTH) {
            /* Issue every load of DEPTH steps before the first MFMA. */
            uint4 q[DEPTH][MT];
            uint32_t sc[DEPTH][MT];
            uint4 bh[DEPTH][NT][4];
            uint4 bl[DEPTH][NT][4];
#pragma unroll
            for (int d = 0; d < DEPTH; d++) {
                const int blk0 = 4 * (s + d) + g;
                const bool v = (s + d < s1) && blk0 < nblk;
                const int blk = v ? blk0 : 0;     /* masked lanes address block 0 */
#pragma unroll
                for (int m = 0; m < MT; m++) {
                    q[d][m] = v ? ld16(pa[m] + (size_t)blk * 16) : make_uint4(0, 0, 0, 0);
                    sc[d][m] = v ? (uint32_t)((k3_g_u8 *)sa[m])[blk] : 127u;
                }
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    const bool ok = v && tv[nt];
#pragma unroll
                    for (int p = 0; p < 4; p++)
                        bh[d][nt][p] = ok ? k3_ldg16(xh[nt] + (size_t)blk * 32 + 8 * p) : make_uint4(0, 0, 0, 0);
                    if (NS == 2) {
#pragma unroll
                        for (int p = 0; p < 4; p++)
                            bl[d][nt][p] = ok ? k3_ldg16(xl[nt] + (size_t)blk * 32 + 8 * p) : make_uint4(0, 0, 0, 0);
                    }
                }
            }
#pragma unroll
            for (int d = 0; d < DEPTH; d++) {
#pragma unroll
                for (int m = 0; m < MT; m++)
                    if (sc[d][m] == 255u) {          /* NaN byte: the block contributes 0 */
                        q[d][m] = make_uint4(0, 0, 0, 0);
                        sc[d][m] = 127u;             /* finite operand: 0 * 2^0, not 0 * inf */
                    }
#pragma unroll
                for (int p = 0; p < 4; p++) {
#pragma unroll
                    for (int m = 0; m < MT; m++) {
                        const uint32_t codes = p == 0 ? q[d][m].x : p == 1 ? q[d][m].y
                                             : p == 2 ? q[d][m].z : q[d][m].w;
                        const k3_bf16x8 av = k3_dequant8_bf16(codes, k3_e8m0_operand(sc[d][m]));
#pragma unroll
                        for (int nt = 0; nt < NT; nt++) {
                            acc[m][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                av, k3_as_bf16x8(bh[d][nt][p]), acc[m][nt], 0, 0, 0);
                            if (NS == 2)
                                acc[m][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                    av, k3_as_bf16x8(bl[d][nt][p]), acc[m][nt], 0, 0, 0);
                        }
                    }
                }
            }
        }

        /* K-split reduction across the workgroup's waves, in wave order. */
        if (kw > 1) {
            if (wv > 0)
                for (int m = 0; m < MT; m++)
                    for (int nt = 0; nt < NT; nt++) red[wv - 1][m * NT + nt][lane] = acc[m][nt];
            __syncthreads();
            if (wv == 0)
                for (int w = 1; w < kw; w++)
                    for (int m = 0; m < MT; m++)
                        for (int nt = 0; nt < NT; nt++) acc[m][nt] += red[w - 1][m * NT + nt][lane];
        }

        if (wv == 0) {
            /* C layout: lane holds token column r16, weight rows 4g..4g+3 of the tile. */
            for (int nt = 0; nt < NT; nt++) {
                if (!tv[nt]) continue;
                const int ti = tok0 + nt * 16 + r16;
                const int orow = (MODE == K3K_MX_PLAIN) ? ti : a.perm[off + ti];
                for (int m = 0; m < RT; m++) {
                    const int base = rb * 16 * RT + 16 * m + 4 * g;
                    if (MODE == K3K_MX_GATEUP) {
                        uint16_t hi[4], lo[4];
                        for (int jj = 0; jj < 4; jj++) {
                            const float v = k3_act_pair(acc[m][nt][jj], acc[m + RT][nt][jj],
                                                        a.act, a.b1, a.b2);
                            k3_split2(v, hi[jj], lo[jj]);
                        }
                        uint16_t *oh = a.ahi + (size_t)orow * rows;
                        uint16_t *ol = a.alo ? a.alo + (size_t)orow * rows : nullptr;
                        for (int jj = 0; jj < 4; jj++)
                            if (base + jj < rows) {
                                oh[base + jj] = hi[jj];
                                if (ol) ol[base + jj] = lo[jj];
                            }
                    } else {
                        float *o = (MODE == K3K_MX_PLAIN) ? a.y + (size_t)orow * a.ldy
                                                          : a.out + (size_t)orow * rows;
                        for (int jj = 0; jj < 4; jj++)
                            if (base + jj < rows) o[base + jj] = acc[m][nt][jj];
                    }
                }
            }
        }
        if (kw > 1) __syncthreads();
    }
}

template <int MODE, int MT, int NT, int NS, int DEPTH, int MAXW>
int launch_mx(const K3kMxArgs *a, int kw, int grid, hipStream_t st)
{
    if (kw < 1 || kw > MAXW) return k3k_fail("mx_gemm waves per item", hipErrorInvalidValue);
    hipLaunchKernelGGL((mx_gemm_kernel<MODE, MT, NT, NS, DEPTH, MAXW>), dim3(grid), dim3(64 * kw),
                       0, st, *a, kw);
    K3K_LAUNCH_CHECK("mx_gemm launch");
    return 0;
}

/* ---- PLAIN, one or two tokens ---------------------------------------------------------
 * y = W x for ntok <= 2 fp32 token rows; one workgroup per 16-row tile, its waves splitting
 * K. Each wave issues the activation loads first (they return from the cache while the
 * weights stream), then every weight and scale load of its K share; the workgroup stages
 * the activations into LDS as bf16 terms (k3_split2: hi, and lo when NS == 2), so no
 * separate split pass runs. B operand lanes of token columns >= ntok, and of columns past
 * K, are masked to zero without branches (a branch there serialises every LDS read). The
 * waves' partial sums are added in wave order.
 *
 * stage_x: the ntok rows [ntok][K] are contiguous, so float4 i holds elements 4i..4i+3 of
 * the flattened rows and lands at hi[4i], lo[ntok*K + 4i]. */
template <int NS, int XPT>
__device__ __forceinline__ void gemv_stage_x(uint16_t *xs, const float4 (&xv)[XPT], int tid,
                                             int nthr, int nq, int ntok, int K)
{
#pragma unroll
    for (int j = 0; j < XPT; j++) {
        const int i = tid + j * nthr;
        if (i < nq) {
            const float4 v = xv[j];
            uint16_t h[4], l[4];
            k3_split2(v.x, h[0], l[0]);
            k3_split2(v.y, h[1], l[1]);
            k3_split2(v.z, h[2], l[2]);
            k3_split2(v.w, h[3], l[3]);
            *reinterpret_cast<uint2 *>(&xs[4 * i]) =
                make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
            if (NS == 2)
                *reinterpret_cast<uint2 *>(&xs[(size_t)ntok * K + 4 * i]) =
                    make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
        }
    }
}

/* One step (4 MX blocks) of one lane: codes of block blk of its row, scale byte ss. */
template <int NS>
__device__ __forceinline__ void gemv_step(k3_f32x4 (&acc)[2], uint4 qq, uint32_t ss,
                                          const uint16_t *xh, const uint16_t *xl, uint32_t bm)
{
    if (ss == 255u) {                                       /* NaN byte: the block is 0 */
        qq = make_uint4(0, 0, 0, 0);
        ss = 127u;
    }
    const float so = k3_e8m0_operand(ss);
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const uint32_t codes = p == 0 ? qq.x : p == 1 ? qq.y : p == 2 ? qq.z : qq.w;
        const k3_bf16x8 av = k3_dequant8_bf16(codes, so);
        uint4 bh = *reinterpret_cast<const uint4 *>(xh + 8 * p);
        bh.x &= bm; bh.y &= bm; bh.z &= bm; bh.w &= bm;
        acc[p & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, k3_as_bf16x8(bh), acc[p & 1], 0, 0, 0);
        if (NS == 2) {
            uint4 bl = *reinterpret_cast<const uint4 *>(xl + 8 * p);
            bl.x &= bm; bl.y &= bm; bl.z &= bm; bl.w &= bm;
            acc[p & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, k3_as_bf16x8(bl), acc[p & 1], 0, 0, 0);
        }
    }
}

/* The waves' sums in wave order (LDS reused after the products), stored by wave 0. */
__device__ __forceinline__ void gemv_finish(uint16_t *xs, k3_f32x4 acc, int wv, int kw, int lane,
                                            int r16, int g, int ntok, int tile, int rows,
                                            float *y, int ldy)
{
    k3_f32x4 *red = reinterpret_cast<k3_f32x4 *>(xs);
    __syncthreads();
    red[wv * 64 + lane] = acc;
    __syncthreads();
    if (wv == 0) {
        k3_f32x4 part[16];
#pragma unroll
        for (int w = 0; w < 16; w++) part[w] = w < kw ? red[w * 64 + lane] : k3_f32x4{0.f, 0.f, 0.f, 0.f};
        k3_f32x4 sum = part[0];
#pragma unroll
        for (int w = 1; w < 16; w++) sum += part[w];
        if (r16 < ntok) {
            float *o = y + (size_t)r16 * ldy;
            const int base = tile * 16 + 4 * g;
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
                if (base + jj < rows) o[base + jj] = sum[jj];
        }
    }
}

/* mx_gemv_chunk_kernel: K % 512 == 0, one 512-column chunk per wave (kw = K / 512 <= 16),
 * one or two tokens; a workgroup per 16-row tile. The latency of the few loads a lane makes
 * is the whole cost, so nothing else may wait behind them:
 *  - each wave loads only its own chunk of the activations (lane L: columns 8L .. 8L+7 of
 *    each token) first, then its weights (blocks 4i+g, i = 0..3, of its row, and the row's
 *    16 scale bytes of the chunk in one 16-byte load), splits the activations into bf16
 *    terms in a wave-private LDS region and reads its B operands back from there: LDS
 *    operations of one wave complete in order, so no workgroup barrier precedes the
 *    products;
 *  - the activation terms of all tokens share each MFMA (B column j = token j / NS, term
 *    j % NS; the other columns read a zero block), and the four k-slices of a block
 *    accumulate into four independent sums;
 *  - the waves' sums meet through LDS behind one barrier, and 16 ntok threads add them in
 *    wave order. */
template <int NS>
__global__ __launch_bounds__(1024) void mx_gemv_chunk_kernel(K3kMxArgs a, int kw)
{
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];   /* wave w: [ntok NS + 1][512] */
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int K = a.K, nblk = K >> 5, rows = a.rows, ntok = a.ntok;
    const int ncol = ntok * NS;                              /* B columns holding terms */
    const int tile = blockIdx.x;
    float4 xv[2][2];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int h = 0; h < 2; h++)
            xv[t][h] = t < ntok ? *reinterpret_cast<const float4 *>(a.xf32 + (size_t)t * K + wv * 512 + 8 * lane + 4 * h)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
    uint4 q[4];
    const int row = min(tile * 16 + r16, rows - 1);         /* rows past the end: discarded */
    const k3_rsrc rp = k3_make_rsrc(a.packed, (uint32_t)rows * (uint32_t)(K >> 1));
    const k3_rsrc rs = k3_make_rsrc(a.scales, (uint32_t)rows * (uint32_t)nblk);
    const uint32_t pb = (uint32_t)row * (uint32_t)(K >> 1) + (uint32_t)wv * 256u;
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = k3_bload16(rp, pb + (uint32_t)(4 * i + g) * 16u);
    const uint4 sv = k3_bload16(rs, (uint32_t)row * (uint32_t)nblk + (uint32_t)wv * 16u);
    uint16_t *wx = xs + (size_t)wv * (ncol + 1) * 512;       /* column j: wx + 512 j; zeros: wx + 512 ncol */
#pragma unroll
    for (int t = 0; t < 2; t++) {
        if (t >= ntok) break;
        uint16_t h[8], l[8];
        const float f[8] = {xv[t][0].x, xv[t][0].y, xv[t][0].z, xv[t][0].w,
                            xv[t][1].x, xv[t][1].y, xv[t][1].z, xv[t][1].w};
#pragma unroll
        for (int e = 0; e < 8; e++) k3_split2(f[e], h[e], l[e]);
        *reinterpret_cast<uint4 *>(wx + (t * NS) * 512 + 8 * lane) =
            make_uint4(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16),
                       h[4] | ((uint32_t)h[5] << 16), h[6] | ((uint32_t)h[7] << 16));
        if (NS == 2)
            *reinterpret_cast<uint4 *>(wx + (t * NS + 1) * 512 + 8 * lane) =
                make_uint4(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16),
                           l[4] | ((uint32_t)l[5] << 16), l[6] | ((uint32_t)l[7] << 16));
    }
    *reinterpret_cast<uint4 *>(wx + ncol * 512 + 8 * lane) = make_uint4(0, 0, 0, 0);
    __builtin_amdgcn_wave_barrier();
    const uint16_t *bcol = wx + min(r16, ncol) * 512;
    const uint32_t scw[4] = {sv.x, sv.y, sv.z, sv.w};
    k3_f32x4 acc[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int blk = 4 * i + g;                          /* MX block of the chunk */
        uint32_t ss = (scw[i] >> (8 * g)) & 0xffu;
        uint4 qq = q[i];
        if (ss == 255u) {                                   /* NaN byte: the block is 0 */
            qq = make_uint4(0, 0, 0, 0);
            ss = 127u;
        }
        const float so = k3_e8m0_operand(ss);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint32_t codes = p == 0 ? qq.x : p == 1 ? qq.y : p == 2 ? qq.z : qq.w;
            const uint4 bv = *reinterpret_cast<const uint4 *>(bcol + blk * 32 + 8 * p);
            acc[p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k3_dequant8_bf16(codes, so), k3_as_bf16x8(bv), acc[p], 0, 0, 0);
        }
    }
    /* lane (g, r16): rows 4g..4g+3 of column r16; a token's value is its columns' sum */
    k3_f32x4 v = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    if (NS == 2) {
        k3_f32x4 nx;
#pragma unroll
        for (int jj = 0; jj < 4; jj++) nx[jj] = __shfl_down(v[jj], 1, 16);
        v += nx;
    }
    float *red = reinterpret_cast<float *>(xs + (size_t)kw * (ncol + 1) * 512);   /* [kw][ntok][16] */
    if (r16 < ncol && r16 % NS == 0)
        *reinterpret_cast<float4 *>(&red[(wv * ntok + r16 / NS) * 16 + 4 * g]) = make_float4(v[0], v[1], v[2], v[3]);
    __syncthreads();
    if (tid < ntok * 16) {
        const int t = tid >> 4, rr = tid & 15;
        float sum = red[t * 16 + rr];
        for (int w = 1; w < kw; w++) sum += red[(w * ntok + t) * 16 + rr];
        if (tile * 16 + rr < rows) a.y[(size_t)t * a.ldy + tile * 16 + rr] = sum;
    }
}

/* mx_gemv_pair_kernel: mx_gemv_chunk_kernel on 8-row tiles, for matrices with fewer than
 * one 16-row tile per CU (K % 1024 == 0, kw = K / 1024 <= 8 waves): twice the workgroups,
 * each lane loading what it loads there. Wave w takes chunks 2w and 2w + 1 of the tile's
 * 8 rows in one MFMA sequence: A rows 0-7 hold chunk 2w, rows 8-15 chunk 2w + 1, against
 * B columns 0.. (chunk 2w's terms) and 8.. (chunk 2w + 1's). Each chunk's product is the
 * chunk kernel's MFMA sequence at the same k positions, and the chunks' sums are added in
 * chunk order, so y is the chunk kernel's, bit for bit. */
template <int NS>
__global__ __launch_bounds__(512) void mx_gemv_pair_kernel(K3kMxArgs a, int kw)
{
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];   /* chunk c: [ntok NS + 1][512] */
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4, h = r16 >> 3, j8 = r16 & 7;
    const int K = a.K, nblk = K >> 5, rows = a.rows, ntok = a.ntok;
    const int ncol = ntok * NS, nch = 2 * kw;
    const int tile = blockIdx.x;
    /* lane L stages columns 8L .. 8L+7 of both chunks for each token */
    float4 xv[2][2][2];
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int hh = 0; hh < 2; hh++)
                xv[c][t][hh] = t < ntok ? *reinterpret_cast<const float4 *>(a.xf32 + (size_t)t * K + (2 * wv + c) * 512 +
                                                                             8 * lane + 4 * hh)
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
    /* lane (g, r16): row j8 of the tile, chunk 2w + h */
    uint4 q[4];
    const int row = min(tile * 8 + j8, rows - 1);           /* rows past the end: discarded */
    const int ch = 2 * wv + h;
    const k3_rsrc rp = k3_make_rsrc(a.packed, (uint32_t)rows * (uint32_t)(K >> 1));
    const k3_rsrc rs = k3_make_rsrc(a.scales, (uint32_t)rows * (uint32_t)nblk);
    const uint32_t pb = (uint32_t)row * (uint32_t)(K >> 1) + (uint32_t)ch * 256u;
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = k3_bload16(rp, pb + (uint32_t)(4 * i + g) * 16u);
    const uint4 sv = k3_bload16(rs, (uint32_t)row * (uint32_t)nblk + (uint32_t)ch * 16u);
#pragma unroll
    for (int c = 0; c < 2; c++) {
        uint16_t *wx = xs + (size_t)(2 * wv + c) * (ncol + 1) * 512;   /* column j: wx + 512 j; zeros: wx + 512 ncol */
#pragma unroll
        for (int t = 0; t < 2; t++) {
            if (t >= ntok) break;
            uint16_t hb[8], lb[8];
            const float f[8] = {xv[c][t][0].x, xv[c][t][0].y, xv[c][t][0].z, xv[c][t][0].w,
                                xv[c][t][1].x, xv[c][t][1].y, xv[c][t][1].z, xv[c][t][1].w};
#pragma unroll
            for (int e = 0; e < 8; e++) k3_split2(f[e], hb[e], lb[e]);
            *reinterpret_cast<uint4 *>(wx + (t * NS) * 512 + 8 * lane) =
                make_uint4(hb[0] | ((uint32_t)hb[1] << 16), hb[2] | ((uint32_t)hb[3] << 16),
                           hb[4] | ((uint32_t)hb[5] << 16), hb[6] | ((uint32_t)hb[7] << 16));
            if (NS == 2)
                *reinterpret_cast<uint4 *>(wx + (t * NS + 1) * 512 + 8 * lane) =
                    make_uint4(lb[0] | ((uint32_t)lb[1] << 16), lb[2] | ((uint32_t)lb[3] << 16),
                               lb[4] | ((uint32_t)lb[5] << 16), lb[6] | ((uint32_t)lb[7] << 16));
        }
        *reinterpret_cast<uint4 *>(wx + ncol * 512 + 8 * lane) = make_uint4(0, 0, 0, 0);
    }
    __builtin_amdgcn_wave_barrier();
    /* B column r16: column j8 of chunk 2w + h (zeros past its terms) */
    const uint16_t *bcol = xs + (size_t)(2 * wv + h) * (ncol + 1) * 512 + min(j8, ncol) * 512;
    const uint32_t scw[4] = {sv.x, sv.y, sv.z, sv.w};
    k3_f32x4 acc[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int blk = 4 * i + g;                          /* MX block of the chunk */
        uint32_t ss = (scw[i] >> (8 * g)) & 0xffu;
        uint4 qq = q[i];
        if (ss == 255u) {                                   /* NaN byte: the block is 0 */
            qq = make_uint4(0, 0, 0, 0);
            ss = 127u;
        }
        const float so = k3_e8m0_operand(ss);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint32_t codes = p == 0 ? qq.x : p == 1 ? qq.y : p == 2 ? qq.z : qq.w;
            const uint4 bv = *reinterpret_cast<const uint4 *>(bcol + blk * 32 + 8 * p);
            acc[p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k3_dequant8_bf16(codes, so), k3_as_bf16x8(bv), acc[p], 0, 0, 0);
        }
    }
    /* lane (g, r16): rows 4g..4g+3 of column r16; chunk 2w's rows are 0-7 in columns 0-7,
     * chunk 2w + 1's rows 8-15 in columns 8-15; a token's value is its columns' sum */
    k3_f32x4 v = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    if (NS == 2) {
        k3_f32x4 nx;
#pragma unroll
        for (int jj = 0; jj < 4; jj++) nx[jj] = __shfl_down(v[jj], 1, 16);
        v += nx;
    }
    float *red = reinterpret_cast<float *>(xs + (size_t)nch * (ncol + 1) * 512);   /* [nch][ntok][8] */
    if ((g >> 1) == h && j8 < ncol && j8 % NS == 0)
        *reinterpret_cast<float4 *>(&red[(ch * ntok + j8 / NS) * 8 + 4 * (g & 1)]) = make_float4(v[0], v[1], v[2], v[3]);
    __syncthreads();
    if (tid < ntok * 8) {
        const int t = tid >> 3, rr = tid & 7;
        float sum = red[t * 8 + rr];
        for (int c = 1; c < nch; c++) sum += red[(c * ntok + t) * 8 + rr];
        if (tile * 8 + rr < rows) a.y[(size_t)t * a.ldy + tile * 8 + rr] = sum;
    }
}

/* mx_gemv_small_kernel: any K % 32 == 0 (row-major), runs of at most SMAX steps per wave
 * (kw <= 16). A lane loads block 4s+g of its row and that block's scale byte; lanes past
 * the wave's run or past K take the offset 2^31, beyond the buffer's size (< 2^31), where a
 * buffer load returns zero. */
template <int NS, int SMAX>
__global__ __launch_bounds__(1024) void mx_gemv_small_kernel(K3kMxArgs a, int kw)
{
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
    constexpr int XPT = 8;
    const int tid = threadIdx.x, lane = tid & 63, nthr = blockDim.x;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int K = a.K, nblk = K >> 5, nsteps = (nblk + 3) >> 2, rows = a.rows, ntok = a.ntok;
    const int tile = blockIdx.x;
    const int s0 = (wv * nsteps) / kw, s1 = ((wv + 1) * nsteps) / kw;
    const int nq = ntok * (K >> 2);
    float4 xv[XPT];
#pragma unroll
    for (int j = 0; j < XPT; j++) {
        const int i = tid + j * nthr;
        xv[j] = i < nq ? *reinterpret_cast<const float4 *>(a.xf32 + 4 * (size_t)i) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const int row = min(tile * 16 + r16, rows - 1);
    const k3_rsrc rp = k3_make_rsrc(a.packed, (uint32_t)rows * (uint32_t)(K >> 1));
    const k3_rsrc rs = k3_make_rsrc(a.scales, (uint32_t)rows * (uint32_t)nblk);
    const uint32_t pbase = (uint32_t)row * (uint32_t)(K >> 1), sbase = (uint32_t)row * (uint32_t)nblk;
    uint4 q[SMAX];
    uint32_t sc[SMAX];
#pragma unroll
    for (int i = 0; i < SMAX; i++) {
        const int blk = 4 * (s0 + i) + g;
        const bool v = s0 + i < s1 && blk < nblk;
        q[i] = k3_bload16(rp, v ? pbase + (uint32_t)blk * 16u : 0x80000000u);
        sc[i] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rs, v ? sbase + (uint32_t)blk : 0x80000000u, 0, 0);
    }
    gemv_stage_x<NS>(xs, xv, tid, nthr, nq, ntok, K);
    __syncthreads();
    const int xr = r16 < ntok ? r16 : 0;
    k3_f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int i = 0; i < SMAX; i++) {
        const int blk0 = 4 * (s0 + i) + g;
        const bool kv = s0 + i < s1 && blk0 < nblk;          /* columns past K contribute 0 */
        const int blk = kv ? blk0 : nblk - 1;
        const uint32_t bm = (r16 < ntok && kv) ? ~0u : 0u;
        gemv_step<NS>(acc, q[i], sc[i], &xs[(size_t)xr * K + blk * 32],
                      &xs[(size_t)(ntok + xr) * K + blk * 32], bm);
    }
    gemv_finish(xs, acc[0] + acc[1], wv, kw, lane, r16, g, ntok, tile, a.rows, a.y, a.ldy);
}

/* ---- decode of a few assignments ------------------------------------------------------
 * mx_decode_kernel: GATEUP / DOWN when the batch has at most 16 assignments (T * topk),
 * straight from the router's idx, without the gather. Item = (assignment a, TPW tiles of
 * 16 rows), one workgroup each; its TPW * ks waves (ks = blockDim / (64 TPW)): wave w takes
 * tile w % TPW and the K share w / TPW of the ks equal shares of 512-column chunks, and
 * streams it with two chunks of weights in flight. (4 tiles x 2 shares when the
 * assignments fill the chip; 1 tile x up to 16 shares for one or two assignments.) The
 * workgroup stages the activations once (GATEUP: token a / topk from fp32, split
 * in-kernel; DOWN: assignment a's bf16 terms) plus a 1 KB block of zeros: lanes of token
 * columns > 0 read the zeros, so the B operands need no masking. The K shares are added
 * in order, then GATEUP writes act(gate, up) of assignment a as bf16 terms and DOWN writes
 * contrib[a]. A dropped expert (NULL weights) is skipped; the combine leaves it out.
 * DOWN's block 0 stores the number of dropped assignments in *a.drops. SEL (gate/up of a
 * few tokens): the workgroup first selects its token's experts from the router's scored
 * records (select_rounds), so no separate selection kernel runs. Two activation
 * terms share one MFMA: column 0 is the hi term, column 1 the lo term, added at the end. */
template <int MODE, int NS, int LAYOUT, int TPW, bool SEL = false, bool SPLIT = false, int DEPTH = 2>
__global__ __launch_bounds__(TPW == 4 ? 512 : 1024) void mx_decode_kernel(K3kMxArgs a)
{
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];   /* [NS][K], zeros[512] */
    /* SPLIT (GATEUP, one tile per workgroup): a workgroup takes gate or up of its tile and
     * writes the fp32 sum to a.gu; otherwise gate + up, or down */
    static_assert(!SPLIT || (MODE == K3K_MX_GATEUP && TPW == 1 && !SEL), "split gate/up");
    constexpr int NM = MODE == K3K_MX_GATEUP && !SPLIT ? 2 : 1;
    /* activation pieces per thread: K <= 8192, the host keeps 64 TPW ks XPT >= 2048 */
    constexpr int XPT = TPW == 4 ? 4 : 8;
    constexpr int WPOL = LAYOUT == 1 ? K3_LD_NT : K3_LD_DEFAULT;
    const int tid = threadIdx.x, lane = tid & 63, nthr = blockDim.x;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int KS = nthr / (64 * TPW);
    const int r16 = lane & 15, g = lane >> 4;
    const int K = a.K, nblk = K >> 5, rows = a.rows, ntile = (rows + 15) >> 4, nchunk = K >> 9;
    const int ngrp = (ntile + TPW - 1) / TPW;
    const int bx = SPLIT ? (int)blockIdx.x >> 1 : (int)blockIdx.x;
    const int which = SPLIT ? (int)blockIdx.x & 1 : 0;      /* SPLIT: 0 gate, 1 up */
    const int asg = bx / ngrp, tg = bx % ngrp;
    const int tw = tg * TPW + wv % TPW, ks = wv / TPW;
    const int tile = min(tw, ntile - 1);                    /* past the last tile: discarded */
    const int c0 = ks * nchunk / KS, c1 = (ks + 1) * nchunk / KS;
    const ExpertQDev *bank = reinterpret_cast<const ExpertQDev *>(a.bank);
    auto present = [&](int e) {
        if (e < 0 || e >= a.n_experts) return false;
        const ExpertQDev b = bank[e];
        return b.p1 && b.s1 && b.p3 && b.s3 && b.p2 && b.s2;
    };
    /* the dropped assignments, counted by DOWN's block 0 (the slots are final by then) */
    if (MODE == K3K_MX_DOWN && a.drops) {
        if (blockIdx.x == 0 && tid == 0) {
            int nd = 0;
            for (int i = 0; i < a.n_assign; i++) {
                const int e = a.idx[i];
                nd += e >= 0 && e < a.n_experts && !present(e);
            }
            *a.drops = nd;
        }
    }
    /* activation loads first: they return while the selection runs and the weights stream */
    float4 xv[XPT];
    uint4 hv[XPT];
    const int nq = MODE == K3K_MX_GATEUP ? K >> 2 : NS * (K >> 3);
#pragma unroll
    for (int j = 0; j < XPT; j++) {
        const int i = tid + j * nthr;
        if (MODE == K3K_MX_GATEUP)
            xv[j] = i < nq ? *reinterpret_cast<const float4 *>(a.xf32 + (size_t)(asg / a.topk) * K + 4 * i)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
        else
            hv[j] = i < nq ? *reinterpret_cast<const uint4 *>((i < (K >> 3) ? a.xhi : a.xlo) + (size_t)asg * K +
                                                                8 * (i % (K >> 3)))
                           : make_uint4(0, 0, 0, 0);
    }
    int eix;
    if constexpr (SEL) {
        /* the token's experts: the router's selection from router_small's scored records.
         * The workgroups of slot j need only the j + 1 largest keys (the selection's first
         * j + 1 picks do not depend on the later ones; an uncertified logit is recomputed
         * when it could reach those), so slot 0 starts its weight stream after one
         * extraction per level instead of topk; the first workgroup of the token's last
         * slot selects all topk and writes idx / wt */
        __shared__ SelSmem<8> ssm;
        __shared__ int sel_id[64];
        const int t = asg / a.topk, j = asg % a.topk;
        const bool writer = j == a.topk - 1 && tg == 0;
        ExcTable exc;
        exc.pairs = a.exc.pairs;
        exc.index = a.exc.index;
        exc.bits = a.exc.bits;
        exc.kmin = a.exc.kmin;
        exc.kmax = a.exc.kmax;
        exc.base = a.exc.base;
        exc.mmin = a.exc.mmin;
        exc.mwords = a.exc.mwords;
        exc.n = a.exc.n;
        const float4 *pre = reinterpret_cast<const float4 *>(a.pre);
        for (int e = tid; e < 64 * 8; e += nthr)
            select_put_record(ssm, e, e < a.n_experts ? pre[(size_t)t * a.n_experts + e] : make_float4(0.f, 0.f, 0.f, 0.f),
                              e < a.n_experts ? (a.rbias ? a.rbias[e] : 0.0f) : -INFINITY);
        __syncthreads();
        int nre;
        const uint64_t mysel = select_rounds<8>(ssm, a.xf32 + (size_t)t * K, a.rw, a.rbias, K, a.n_experts,
                                                j + 1, exc, nre);
        if (wv == 0) {
            int id;
            float w;
            select_weight<8>(ssm, mysel, j + 1, a.renorm, a.rscale, id, w);   /* w: writer only */
            if (lane <= j) {
                sel_id[lane] = id >= 0 ? id : 0;            /* none left: expert 0, weight 0 */
                if (writer) {
                    a.idx_out[(size_t)t * a.topk + lane] = id >= 0 ? id : 0;
                    a.wt_out[(size_t)t * a.topk + lane] = w;
                }
            }
            if (writer && lane == 0 && a.nrecomp) a.nrecomp[t] = nre;
        }
        __syncthreads();
        eix = sel_id[j];
    } else {
        eix = a.idx[asg];
    }
    ExpertQDev q = {};
    if (eix >= 0 && eix < a.n_experts) q = bank[eix];
    const uint8_t *pm[NM], *sm[NM];
    if (SPLIT) {
        pm[0] = which ? q.p3 : q.p1; sm[0] = which ? q.s3 : q.s1;
    } else if (MODE == K3K_MX_GATEUP) {
        pm[0] = q.p1; sm[0] = q.s1;
        pm[NM - 1] = q.p3; sm[NM - 1] = q.s3;
    } else {
        pm[0] = q.p2; sm[0] = q.s2;
    }
    if (!(q.p1 && q.s1 && q.p3 && q.s3 && q.p2 && q.s2)) return;   /* dropped or out of range */
    const uint32_t prow = LAYOUT == 1 ? k3_tile_prows(rows) : (uint32_t)rows;
    k3_rsrc rp[NM], rs[NM];
#pragma unroll
    for (int m = 0; m < NM; m++) {
        rp[m] = k3_make_rsrc(pm[m], prow * (uint32_t)(K >> 1));
        rs[m] = k3_make_rsrc(sm[m], prow * (uint32_t)nblk);
    }
    const int row = min(tile * 16 + r16, rows - 1);
    /* chunk c of this wave's tile: LAYOUT 1, four contiguous 1 KB loads and one scale
     * dword (byte i = step i); LAYOUT 0, blocks 4i+g of the lane's row and the row's 16
     * scale bytes (dword i, byte g = step i) */
    uint4 qa[DEPTH][NM][4];
    uint4 sq[DEPTH][NM];
    /* Chunks past the wave's last are loaded too, at an offset beyond every buffer (2^31):
     * they return zeros and move no data. With no load under a branch, every wait counts
     * exactly the loads issued after the one it waits for, so chunks c + 1 .. c + DEPTH - 1
     * stay in flight while chunk c is multiplied. */
    constexpr uint32_t OOB = 0x80000000u;
    auto load = [&](int c, auto slot) {
        constexpr int S = decltype(slot)::value;
        const bool in = c < c1;
#pragma unroll
        for (int m = 0; m < NM; m++) {
            if (LAYOUT == 1) {
                const uint32_t tc = k3_tile_idx(tile, c, nchunk);
#pragma unroll
                for (int i = 0; i < 4; i++)
                    qa[S][m][i] = k3_bload16<WPOL>(rp[m], in ? tc * 4096u + (uint32_t)i * 1024u + (uint32_t)lane * 16u : OOB);
                sq[S][m].x = k3_bload4<WPOL>(rs[m], in ? tc * 256u + (uint32_t)lane * 4u : OOB);
            } else {
                const uint32_t pb = (uint32_t)row * (uint32_t)(K >> 1) + (uint32_t)c * 256u;
#pragma unroll
                for (int i = 0; i < 4; i++) qa[S][m][i] = k3_bload16<WPOL>(rp[m], in ? pb + (uint32_t)(4 * i + g) * 16u : OOB);
                sq[S][m] = k3_bload16<WPOL>(rs[m], in ? (uint32_t)row * (uint32_t)nblk + (uint32_t)c * 16u : OOB);
            }
        }
    };
    /* issued in the loop's order (slot 0, 1, ...): the waits at the loop head take the worse
     * of the two ways in, so a reordered prologue would make them wait for later slots too */
    k3_static_for<DEPTH>([&](auto sl) {
        load(c0 + decltype(sl)::value, sl);
        __builtin_amdgcn_sched_barrier(0);
    });
    for (int i = tid; i < 64; i += nthr)
        reinterpret_cast<uint4 *>(&xs[(size_t)NS * K])[i] = make_uint4(0, 0, 0, 0);
    if (MODE == K3K_MX_GATEUP) {
        gemv_stage_x<NS>(xs, xv, tid, nthr, nq, 1, K);
    } else {
#pragma unroll
        for (int j = 0; j < XPT; j++) {
            const int i = tid + j * nthr;
            if (i < nq) *reinterpret_cast<uint4 *>(&xs[8 * i]) = hv[j];    /* hi then lo */
        }
    }
    __syncthreads();
    k3_f32x4 acc[NM][2];
#pragma unroll
    for (int m = 0; m < NM; m++) acc[m][0] = acc[m][1] = k3_f32x4{0.f, 0.f, 0.f, 0.f};
    auto comp = [&](int c, auto slot) {
        constexpr int S = decltype(slot)::value;
        /* column 0: the hi term, column 1 (two terms): the lo term, the rest: zeros */
        const uint16_t *hb = r16 == 0            ? &xs[c * 512 + g * 32]
                             : (NS == 2 && r16 == 1) ? &xs[(size_t)K + c * 512 + g * 32]
                                                     : &xs[(size_t)NS * K + g * 32];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint4 qm[NM];
            float so[NM];
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const uint32_t sw = LAYOUT == 1 ? sq[S][m].x >> (8 * i)
                                  : (i == 0 ? sq[S][m].x : i == 1 ? sq[S][m].y : i == 2 ? sq[S][m].z : sq[S][m].w) >> (8 * g);
                uint32_t ss = sw & 0xffu;
                qm[m] = qa[S][m][i];
                /* NaN byte: the block is 0 (a tiled bank stores such a block as zero codes
                 * with scale 127 already) */
                if (LAYOUT == 0 && ss == 255u) {
                    qm[m] = make_uint4(0, 0, 0, 0);
                    ss = 127u;
                }
                so[m] = k3_e8m0_operand(ss);
            }
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const uint4 bh = *reinterpret_cast<const uint4 *>(hb + 128 * i + 8 * p);
#pragma unroll
                for (int m = 0; m < NM; m++) {
                    const uint32_t codes = p == 0 ? qm[m].x : p == 1 ? qm[m].y : p == 2 ? qm[m].z : qm[m].w;
                    const k3_bf16x8 av = k3_dequant8_bf16(codes, so[m]);
                    acc[m][p & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, k3_as_bf16x8(bh), acc[m][p & 1], 0, 0, 0);
                }
            }
        }
    };
    int c = c0;
    for (; c + DEPTH - 1 < c1; c += DEPTH)
        k3_static_for<DEPTH>([&](auto sl) {
            comp(c + decltype(sl)::value, sl);
            load(c + decltype(sl)::value + DEPTH, sl);
        });
    k3_static_for<DEPTH - 1>([&](auto sl) {
        if (c + decltype(sl)::value < c1) comp(c + decltype(sl)::value, sl);
    });
    /* K shares in order: share 0 adds those of shares 1.. (LDS reused after the products);
     * then column 0 (hi) + column 1 (lo) */
    k3_f32x4 *red = reinterpret_cast<k3_f32x4 *>(xs);
    if (KS > 1) {
        __syncthreads();
        if (ks > 0)
#pragma unroll
            for (int m = 0; m < NM; m++)
                red[(((ks - 1) * TPW + wv % TPW) * NM + m) * 64 + lane] = acc[m][0] + acc[m][1];
        __syncthreads();
    }
    k3_f32x4 own[NM], nxt[NM];                      /* this lane's column, and lane + 1's */
#pragma unroll
    for (int m = 0; m < NM; m++) {
        own[m] = acc[m][0] + acc[m][1];
#pragma unroll
        for (int jj = 0; jj < 4; jj++) nxt[m][jj] = __shfl_down(own[m][jj], 1, 16);
    }
    if (ks == 0 && r16 == 0 && tw < ntile) {
        k3_f32x4 sum[NM];
#pragma unroll
        for (int m = 0; m < NM; m++) {
            sum[m] = own[m];
            for (int k2 = 1; k2 < KS; k2++) sum[m] += red[(((k2 - 1) * TPW + wv % TPW) * NM + m) * 64 + lane];
            if (NS == 2) {
                k3_f32x4 lo = nxt[m];
                for (int k2 = 1; k2 < KS; k2++) lo += red[(((k2 - 1) * TPW + wv % TPW) * NM + m) * 64 + lane + 1];
                sum[m] += lo;
            }
        }
        const int base = tw * 16 + 4 * g;
        if (SPLIT) {
            float *o = a.gu + ((size_t)asg * 2 + which) * rows;
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
                if (base + jj < rows) o[base + jj] = sum[0][jj];
        } else if (MODE == K3K_MX_GATEUP) {
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
                if (base + jj < rows) {
                    uint16_t hi, lo;
                    k3_split2(k3_act_pair(sum[0][jj], sum[NM - 1][jj], a.act, a.b1, a.b2), hi, lo);
                    a.ahi[(size_t)asg * rows + base + jj] = hi;
                    if (NS == 2) a.alo[(size_t)asg * rows + base + jj] = lo;
                }
        } else {
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
                if (base + jj < rows) a.out[(size_t)asg * rows + base + jj] = sum[0][jj];
        }
    }
}

/* mx_decode_combine_kernel: DOWN and the weighted combine of the decode path in one
 * kernel. A workgroup takes one (token t, 16-row tile) and all of the token's topk slots:
 * wave w = (slot j = w % topk, K share ks = w / topk) streams the tile's rows of slot j's
 * down matrix over its share of the 512-column chunks, like mx_decode_kernel with one tile
 * per wave. The slots' activation terms are staged in LDS once per workgroup. Then the
 * shares of a slot are added in share order (the sums mx_decode_kernel writes to contrib)
 * and out[t][row] = 0 + sum_j wt[t][j] * slot j's sum, j ascending, over the slots whose
 * expert is in range and present in the bank -- the combine's rule and order
 * (k3_ops.c:641-642). An absent slot's wave reads through an empty descriptor (zeros) and
 * its sum is left out. Two activation terms share one MFMA (columns 0 and 1), each term's
 * shares are added in order, then hi + lo. */
template <int NS, int LAYOUT, bool GU = false, int DEPTH = 2>
__global__ __launch_bounds__(1024) void mx_decode_combine_kernel(K3kMxArgs a)
{
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];   /* [topk][NS][K], zeros[512] */
    __shared__ float red[16 * 2 * 16];                              /* [slot, share][term][16 rows] */
    __shared__ int vsh[16];
    __shared__ float wsh[16];
    constexpr int WPOL = LAYOUT == 1 ? K3_LD_NT : K3_LD_DEFAULT;
    const int tid = threadIdx.x, lane = tid & 63, nthr = blockDim.x;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int topk = a.topk, KS = nthr / (64 * topk);
    const int j = wv % topk, ks = wv / topk;
    const int r16 = lane & 15, g = lane >> 4;
    const int K = a.K, nblk = K >> 5, rows = a.rows, ntile = (rows + 15) >> 4, nchunk = K >> 9;
    const int t = blockIdx.x / ntile, tile = blockIdx.x % ntile;
    const int c0 = ks * nchunk / KS, c1 = (ks + 1) * nchunk / KS;
    const ExpertQDev *bank = reinterpret_cast<const ExpertQDev *>(a.bank);
    if (a.drops && blockIdx.x == 0 && tid == 0) {          /* dropped assignments */
        int nd = 0;
        for (int i = 0; i < a.n_assign; i++) {
            const int e = a.idx[i];
            if (e >= 0 && e < a.n_experts) {
                const ExpertQDev b = bank[e];
                nd += !(b.p1 && b.s1 && b.p3 && b.s3 && b.p2 && b.s2);
            }
        }
        *a.drops = nd;
    }
    const int eix = a.idx[t * topk + j];
    const float wj = a.wt[t * topk + j];                    /* in flight with the rest */
    ExpertQDev q = {};
    if (eix >= 0 && eix < a.n_experts) q = bank[eix];
    const bool valid = q.p1 && q.s1 && q.p3 && q.s3 && q.p2 && q.s2;
    const uint32_t prow = LAYOUT == 1 ? k3_tile_prows(rows) : (uint32_t)rows;
    const k3_rsrc rp = k3_make_rsrc(q.p2, valid ? prow * (uint32_t)(K >> 1) : 0u);
    const k3_rsrc rs = k3_make_rsrc(q.s2, valid ? prow * (uint32_t)nblk : 0u);
    const int row = min(tile * 16 + r16, rows - 1);
    uint4 qa[DEPTH][4];
    uint4 sq[DEPTH];
    /* chunks past the wave's last load zeros from beyond the buffer, so no load sits under
     * a branch and the waits count exactly (as in mx_decode_kernel) */
    constexpr uint32_t OOB = 0x80000000u;
    auto load = [&](int c, auto slot) {
        constexpr int S = decltype(slot)::value;
        const bool in = c < c1;
        if (LAYOUT == 1) {
            const uint32_t tc = k3_tile_idx(tile, c, nchunk);
#pragma unroll
            for (int i = 0; i < 4; i++)
                qa[S][i] = k3_bload16<WPOL>(rp, in ? tc * 4096u + (uint32_t)i * 1024u + (uint32_t)lane * 16u : OOB);
            sq[S].x = k3_bload4<WPOL>(rs, in ? tc * 256u + (uint32_t)lane * 4u : OOB);
        } else {
            const uint32_t pb = (uint32_t)row * (uint32_t)(K >> 1) + (uint32_t)c * 256u;
#pragma unroll
            for (int i = 0; i < 4; i++) qa[S][i] = k3_bload16<WPOL>(rp, in ? pb + (uint32_t)(4 * i + g) * 16u : OOB);
            sq[S] = k3_bload16<WPOL>(rs, in ? (uint32_t)row * (uint32_t)nblk + (uint32_t)c * 16u : OOB);
        }
    };
    /* GU: the first pieces of the gate and up sums are requested before the weights, so
     * that waiting for them (loads complete in order) leaves the weight loads in flight */
    const k3_rsrc rg = k3_make_rsrc(a.gu, GU ? (uint32_t)a.n_assign * 2u * (uint32_t)K * 4u : 0u);
    const uint32_t gb = ((uint32_t)(t * topk + j) * 2u * (uint32_t)K + (uint32_t)c0 * 512u) * 4u;
    const uint32_t ub = gb + (uint32_t)K * 4u;
    uint4 gv0[2][2], uv0[2][2];
    auto load_gu = [&](int i0, uint4 (&gv)[2][2], uint4 (&uv)[2][2]) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const uint32_t o = (uint32_t)(i0 + lane + 64 * u) * 32u;
            gv[u][0] = k3_bload16(rg, gb + o);
            gv[u][1] = k3_bload16(rg, gb + o + 16u);
            uv[u][0] = k3_bload16(rg, ub + o);
            uv[u][1] = k3_bload16(rg, ub + o + 16u);
        }
    };
    if constexpr (GU) load_gu(0, gv0, uv0);
    __builtin_amdgcn_sched_barrier(0);
    k3_static_for<DEPTH>([&](auto sl) {                     /* in the loop's order */
        load(c0 + decltype(sl)::value, sl);
        __builtin_amdgcn_sched_barrier(0);
    });
    /* this wave's slot and columns of the activation terms into [slot][term][K] (the waves
     * of one slot stage disjoint column ranges), and the row of zeros (every wave writes the
     * same zeros): no workgroup barrier before the products */
    if constexpr (GU) {
        /* from the gate and up sums (fp32): act(gate, up) and its bf16 terms, as the gate/up
         * kernel's epilogue forms them; a piece is 8 columns */
        const int nq = (c1 - c0) * 64;
        for (int i0 = 0; i0 < nq; i0 += 128) {
            uint4 gv[2][2], uv[2][2];
            if (i0 == 0) {
#pragma unroll
                for (int u = 0; u < 2; u++)
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        gv[u][h] = gv0[u][h];
                        uv[u][h] = uv0[u][h];
                    }
            } else {
                load_gu(i0, gv, uv);
            }
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int i = i0 + lane + 64 * u;
                if (i >= nq) continue;
                const float gf[8] = {__uint_as_float(gv[u][0].x), __uint_as_float(gv[u][0].y), __uint_as_float(gv[u][0].z),
                                     __uint_as_float(gv[u][0].w), __uint_as_float(gv[u][1].x), __uint_as_float(gv[u][1].y),
                                     __uint_as_float(gv[u][1].z), __uint_as_float(gv[u][1].w)};
                const float uf[8] = {__uint_as_float(uv[u][0].x), __uint_as_float(uv[u][0].y), __uint_as_float(uv[u][0].z),
                                     __uint_as_float(uv[u][0].w), __uint_as_float(uv[u][1].x), __uint_as_float(uv[u][1].y),
                                     __uint_as_float(uv[u][1].z), __uint_as_float(uv[u][1].w)};
                uint32_t hw[4], lw[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    uint16_t h0, l0, h1, l1;
                    k3_split2(k3_act_pair(gf[2 * e], uf[2 * e], a.act, a.b1, a.b2), h0, l0);
                    k3_split2(k3_act_pair(gf[2 * e + 1], uf[2 * e + 1], a.act, a.b1, a.b2), h1, l1);
                    hw[e] = h0 | ((uint32_t)h1 << 16);
                    lw[e] = l0 | ((uint32_t)l1 << 16);
                }
                *reinterpret_cast<uint4 *>(&xs[((size_t)j * NS) * K + c0 * 512 + 8 * i]) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
                if (NS == 2)
                    *reinterpret_cast<uint4 *>(&xs[((size_t)j * NS + 1) * K + c0 * 512 + 8 * i]) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
            }
        }
        reinterpret_cast<uint4 *>(&xs[(size_t)topk * NS * K])[lane] = make_uint4(0, 0, 0, 0);
    } else {
        const int nq = (c1 - c0) * 64;                      /* 16-byte pieces per term */
        const uint32_t bytes = (uint32_t)a.n_assign * (uint32_t)K * 2u;
        const uint32_t src = (uint32_t)(t * topk + j) * (uint32_t)K + (uint32_t)c0 * 512u;
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const k3_rsrc rx = k3_make_rsrc(s == 0 ? a.xhi : a.xlo, bytes);
            for (int i0 = 0; i0 < nq; i0 += 256) {
                uint4 v[4];
#pragma unroll
                for (int u = 0; u < 4; u++) v[u] = k3_bload16(rx, (src + 8u * (uint32_t)(i0 + lane + 64 * u)) * 2u);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int i = i0 + lane + 64 * u;
                    if (i < nq)
                        *reinterpret_cast<uint4 *>(&xs[((size_t)j * NS + s) * K + c0 * 512 + 8 * i]) = v[u];
                }
            }
        }
        reinterpret_cast<uint4 *>(&xs[(size_t)topk * NS * K])[lane] = make_uint4(0, 0, 0, 0);
    }
    if (ks == 0 && lane == 0) {
        vsh[j] = valid ? 1 : 0;
        wsh[j] = wj;
    }
    __builtin_amdgcn_wave_barrier();
    k3_f32x4 acc[2] = {k3_f32x4{0.f, 0.f, 0.f, 0.f}, k3_f32x4{0.f, 0.f, 0.f, 0.f}};
    const uint16_t *zb = &xs[(size_t)topk * NS * K + g * 32];
    auto comp = [&](int c, auto slot) {
        constexpr int S = decltype(slot)::value;
        /* column 0: the hi term, column 1 (two terms): the lo term, the rest: zeros */
        const uint16_t *hb = r16 == 0              ? &xs[(size_t)j * NS * K + c * 512 + g * 32]
                             : (NS == 2 && r16 == 1) ? &xs[((size_t)j * NS + 1) * K + c * 512 + g * 32]
                                                     : zb;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t sw = LAYOUT == 1 ? sq[S].x >> (8 * i)
                              : (i == 0 ? sq[S].x : i == 1 ? sq[S].y : i == 2 ? sq[S].z : sq[S].w) >> (8 * g);
            uint32_t ss = sw & 0xffu;
            uint4 qm = qa[S][i];
            /* NaN byte: the block is 0 (tiled: stored as zero codes, scale 127) */
            if (LAYOUT == 0 && ss == 255u) {
                qm = make_uint4(0, 0, 0, 0);
                ss = 127u;
            }
            const float so = k3_e8m0_operand(ss);
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const uint4 bh = *reinterpret_cast<const uint4 *>(hb + 128 * i + 8 * p);
                const uint32_t codes = p == 0 ? qm.x : p == 1 ? qm.y : p == 2 ? qm.z : qm.w;
                const k3_bf16x8 av = k3_dequant8_bf16(codes, so);
                acc[p & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, k3_as_bf16x8(bh), acc[p & 1], 0, 0, 0);
            }
        }
    };
    int c = c0;
    for (; c + DEPTH - 1 < c1; c += DEPTH)
        k3_static_for<DEPTH>([&](auto sl) {
            comp(c + decltype(sl)::value, sl);
            load(c + decltype(sl)::value + DEPTH, sl);
        });
    k3_static_for<DEPTH - 1>([&](auto sl) {
        if (c + decltype(sl)::value < c1) comp(c + decltype(sl)::value, sl);
    });
    /* lanes of token column 0 (hi) and 1 (lo) hold the tile's 16 rows, four each */
    if (r16 < NS) {
        const k3_f32x4 sum = acc[0] + acc[1];
#pragma unroll
        for (int jj = 0; jj < 4; jj++) red[((j * KS + ks) * 2 + r16) * 16 + 4 * g + jj] = sum[jj];
    }
    __syncthreads();
    if (tid < 16 && tile * 16 + tid < rows) {
        float o = 0.0f;
        for (int jj = 0; jj < topk; jj++) {
            if (!vsh[jj]) continue;
            /* each term's shares in order, then hi + lo */
            float d = red[((jj * KS) * 2) * 16 + tid];
            for (int k2 = 1; k2 < KS; k2++) d += red[((jj * KS + k2) * 2) * 16 + tid];
            if (NS == 2) {
                float l = red[((jj * KS) * 2 + 1) * 16 + tid];
                for (int k2 = 1; k2 < KS; k2++) l += red[((jj * KS + k2) * 2 + 1) * 16 + tid];
                d += l;
            }
            o = __fadd_rn(o, __fmul_rn(wsh[jj], d));
        }
        a.out[(size_t)t * rows + tile * 16 + tid] = o;
    }
}

/* ---- expert jobs, LDS-staged activations ---------------------------------------------
 * mx_moe_kernel: the GATEUP / DOWN modes in passes of up to PT tokens, K % 512 == 0.
 *
 * A workgroup of NW waves takes one item = (pass, row block); the waves own consecutive
 * row tiles (MT tiles of 16 rows each) and walk K in chunks of 512 elements (16 MX
 * blocks = 4 steps of 128). K order inside a chunk: at step d, lane group g (lanes
 * 16g..16g+15) holds MX block 4d+g of its row (the MFMA's K permutation is free as long
 * as A and B agree). Weights come in one of two layouts:
 *   LAYOUT 0, row-major (the reference's): per step a lane loads its block's 16 bytes
 *     (a wave: 16 rows x 64 contiguous bytes), per chunk one 16-byte load of the row's
 *     16 scale bytes, of which it uses one per step;
 *   LAYOUT 1, tiled (mx_tile_kernel, k3_tile_idx): the bytes of a 16-row tile's chunk
 *     stored in lane order, so a wave's load is 1 KB contiguous and a lane's four scale
 *     bytes of the chunk are one 4-byte load; the four tiles of a group lie side by side
 *     chunk after chunk.
 * The pass's activation rows (hi, lo) for the chunk are staged once in LDS by the whole
 * workgroup (double buffered), one wave-uniform row-half per wave instruction and only for
 * the pass's real tokens; B lanes of token columns past the pass read a row of zeros.
 * While chunk c is multiplied, the weight/scale loads and the activation loads of chunk
 * c+1 are in flight (activations issued first, so waiting for them leaves the weight
 * loads outstanding).
 * Passes of up to 8 tokens with two activation terms put both terms in one MFMA column
 * block (PACK): column t is token t's hi term, column 8 + t its lo term, so each weight
 * fragment takes one MFMA instead of two; the epilogue adds column 8 + t to column t.
 */
template <int MODE, int MT, int NS, int PT, int NB, int NW, int WPE, int LAYOUT, int DEPTH>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WPE, 8)))
void mx_moe_kernel(K3kMxArgs a)
{
    static_assert(PT <= 16 * NB, "a pass fits the MFMA column blocks");
    constexpr bool PACK = NS == 2 && PT <= 8 && NB == 1;     /* hi and lo in one column block */
    constexpr int RT = (MODE == K3K_MX_GATEUP) ? MT / 2 : MT;
    constexpr int KC = 512, SPC = 4, LDT = KC + 8;           /* LDS row: 16-byte pad */
    /* tiled MXFP4 weights are streamed once per pass and non-temporal; row-major ones keep
     * the default policy (a 128-byte line is consumed by two steps' loads) */
    constexpr int WPOL = LAYOUT == 1 ? K3_LD_NT : K3_LD_DEFAULT;
    constexpr int NRH = PT * NS;                             /* staged row-halves per chunk */
    constexpr int PPW = (NRH + NW - 1) / NW;                 /* row-halves per wave */
    /* row PT of each buffer/half stays zero: the B operand of absent token columns */
    __shared__ __attribute__((aligned(16))) uint16_t bsh[2][NS][PT + 1][LDT];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int K = a.K, nblk = K >> 5, nchunk = nblk >> 4;
    const int rows = a.rows;
    const uint32_t rstride = (uint32_t)K >> 1;
    const int rpw = 16 * RT, rpg = NW * rpw;
    const int n_rb = (rows + rpg - 1) / rpg;
    const int n_items = (*a.n_passes) * n_rb;
    /* requires K % 512 == 0: the host routes other K to mx_gemm_kernel */

    /* the stamps pointer waits in LDS: held in registers through the loop it would spill */
    __shared__ unsigned long long *stamp_sh;
    if (tid == 0) {
        stamp_sh = a.stamps;
        if (a.stamps) k3_stamp_begin(a.stamps);
    }
    for (int i = tid; i < 2 * NS * LDT / 8; i += 64 * NW) {
        const int bh = i / (LDT / 8), o = i % (LDT / 8);
        *reinterpret_cast<uint4 *>(&bsh[bh / NS][bh % NS][PT][o * 8]) = make_uint4(0, 0, 0, 0);
    }

    for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
        const int rb = item % n_rb, pass = item / n_rb;
        const int j = a.pass_job[pass];
        const int e = a.job_expert[j];
        const int off = a.job_off[j];
        const int tok0 = a.pass_tp[pass] * PT;
        const int ntok = min(PT, a.job_cnt[j] - tok0);
        const ExpertQDev q = reinterpret_cast<const ExpertQDev *>(a.bank)[e];
        /* one buffer descriptor per matrix (wave-uniform); per-lane byte offsets */
        const uint32_t prow = LAYOUT == 1 ? k3_tile_prows(rows) : (uint32_t)rows;
        const uint32_t pbytes = prow * rstride;
        const uint32_t sbytes = prow * nblk;
        k3_rsrc rp0, rp1, rs0, rs1;
        if (MODE == K3K_MX_GATEUP) {
            rp0 = k3_make_rsrc(q.p1, pbytes); rs0 = k3_make_rsrc(q.s1, sbytes);
            rp1 = k3_make_rsrc(q.p3, pbytes); rs1 = k3_make_rsrc(q.s3, sbytes);
        } else {
            rp0 = rp1 = k3_make_rsrc(q.p2, pbytes);
            rs0 = rs1 = k3_make_rsrc(q.s2, sbytes);
        }
        uint32_t poff[MT], soff[MT];
        const int ntile = (rows + 15) >> 4;
#pragma unroll
        for (int m = 0; m < MT; m++) {
            const int mt = (MODE == K3K_MX_GATEUP) ? (m % RT) : m;
            if (LAYOUT == 0) {
                const int r = min(rb * rpg + wv * rpw + 16 * mt + r16, rows - 1);
                poff[m] = (uint32_t)r * rstride + (uint32_t)g * 16u;
                soff[m] = (uint32_t)r * (uint32_t)nblk;
            } else {
                const int t = min((rb * rpg + wv * rpw) / 16 + mt, ntile - 1);
                poff[m] = k3_tile_idx(t, 0, nchunk) * 4096u + (uint32_t)lane * 16u;
                soff[m] = k3_tile_idx(t, 0, nchunk) * 256u + (uint32_t)lane * 4u;
            }
        }
        /* staging: wave wv copies row-halves wv, wv+NW, ...; lane = 16-byte piece */
        const uint32_t xbytes = (uint32_t)a.n_xrows * (uint32_t)K * 2u;
        const k3_rsrc rxh = k3_make_rsrc(a.xhi, xbytes);
        const k3_rsrc rxl = k3_make_rsrc(NS == 2 ? a.xlo : a.xhi, xbytes);
        /* every staging load is issued (rows past the pass read the pass's first token; only
         * their LDS stores are skipped), so that the waits count exactly the loads issued
         * after the one they wait for */
        uint32_t gsrc[PPW];
#pragma unroll
        for (int i = 0; i < PPW; i++) {
            const int rh = wv + NW * i, p = rh / NS;
            const int ar = a.perm[off + tok0 + (rh < NRH && p < ntok ? p : 0)];
            const int xr = (MODE == K3K_MX_GATEUP) ? ar / a.topk : ar;
            gsrc[i] = ((uint32_t)xr * (uint32_t)K + (uint32_t)lane * 8u) * 2u;
        }
        /* B operand rows: token column nb*16 + r16 of the pass, or the zero row; PACK: token
         * r16 % 8 of term r16 / 8 */
        int brow[NB];
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            const int tk = PACK ? (r16 & 7) : nb * 16 + r16;
            brow[nb] = tk < ntok ? tk : PT;
        }
        const int bterm = PACK ? (r16 >> 3) : 0;

        k3_f32x4 acc[MT][NB];
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
            for (int nb = 0; nb < NB; nb++) acc[m][nb] = k3_f32x4{0.f, 0.f, 0.f, 0.f};

        /* Weights in registers, DEPTH chunks ahead: qa[slot][d] holds step d of a chunk.
         * DEPTH 1: step d of chunk c+1 is loaded into qa[0][d] right after step d of chunk
         * c has consumed it. DEPTH 2: chunks alternate between two slots and step d of
         * chunk c+2 is loaded into chunk c's slot. Scales follow one chunk behind. */
        constexpr int NSLOT = DEPTH == 2 ? 2 : 1;
        constexpr int SQN = MT * (LAYOUT == 0 ? 4 : 1);
        uint4 qa[NSLOT][SPC][MT];
        uint32_t sq[SQN], sqn[SQN], sqnn[SQN];
        uint4 bst[PPW];

        /* Loads past the last chunk are issued too, at an offset beyond the buffer (2^31:
         * every operand is smaller): they return zeros and move no data. */
        constexpr uint32_t OOB = 0x80000000u;
        auto load_b = [&](int c) {
            const uint32_t co = (uint32_t)c * KC * 2u;
#pragma unroll
            for (int i = 0; i < PPW; i++) {
                const int rh = wv + NW * i;
                bst[i] = k3_bload16(rh % NS ? rxl : rxh, c < nchunk ? gsrc[i] + co : OOB);
            }
        };
        auto store_b = [&](int buf) {
#pragma unroll
            for (int i = 0; i < PPW; i++) {
                const int rh = wv + NW * i;
                if (rh < NRH && rh / NS < ntok)
                    *reinterpret_cast<uint4 *>(&bsh[buf][rh % NS][rh / NS][lane * 8]) = bst[i];
            }
        };
        auto load_step = [&](int c, int d, auto slot) {
            constexpr int S = decltype(slot)::value;
            const uint32_t bo = LAYOUT == 0 ? (uint32_t)c * 256u + (uint32_t)d * 64u
                                            : (uint32_t)c * K3_TILE_CSTRIDE + (uint32_t)d * 1024u;
#pragma unroll
            for (int m = 0; m < MT; m++)
                qa[S][d][m] = k3_bload16<WPOL>(m < RT || MODE != K3K_MX_GATEUP ? rp0 : rp1,
                                               c < nchunk ? poff[m] + bo : OOB);
        };
        auto load_scales = [&](int c, uint32_t *ss) {
#pragma unroll
            for (int m = 0; m < MT; m++) {
                const k3_rsrc rs = m < RT || MODE != K3K_MX_GATEUP ? rs0 : rs1;
                if (LAYOUT == 0) {
                    const uint4 v = k3_bload16<WPOL>(rs, c < nchunk ? soff[m] + (uint32_t)c * 16u : OOB);
                    ss[4 * m] = v.x; ss[4 * m + 1] = v.y; ss[4 * m + 2] = v.z; ss[4 * m + 3] = v.w;
                } else {
                    ss[m] = k3_bload4<WPOL>(rs, c < nchunk ? soff[m] + (uint32_t)c * K3_TILE_SCSTRIDE : OOB);
                }
            }
        };

        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, NSLOT - 1>;
        load_b(0);
        load_scales(0, sq);
#pragma unroll
        for (int d = 0; d < SPC; d++) load_step(0, d, I0{});
        if (DEPTH == 2) {
            load_scales(1, sqn);
#pragma unroll
            for (int d = 0; d < SPC; d++) load_step(1, d, I1{});
        }
        store_b(0);
        __syncthreads();
        auto chunk = [&](int c, auto slot) {
            constexpr int S = decltype(slot)::value;
            const int buf = c & 1;
            const bool more = c + 1 < nchunk;
            /* Every prefetch is issued (past the end: zeros, no data moved), so that the waits
             * count exactly the loads issued after the one they wait for. For decode passes
             * the barrier keeps the compiler from sinking the staging loads down to their LDS
             * stores, which would wait for them (and every older load) on the spot; larger
             * passes would hold too many registers for the staging across the chunk. */
            load_b(c + 1);
            load_scales(c + DEPTH, DEPTH == 2 ? sqnn : sqn);
            if constexpr (PT <= 8) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int d = 0; d < SPC; d++) {
                /* B operand: token columns (or the zero row), block 4d+g of the chunk */
                uint4 bh[NB][4], bl[NB][4];
#pragma unroll
                for (int nb = 0; nb < NB; nb++) {
                    const uint4 *bp = reinterpret_cast<const uint4 *>(&bsh[buf][bterm][brow[nb]][(4 * d + g) * 32]);
                    const uint4 *bq = reinterpret_cast<const uint4 *>(&bsh[buf][NS - 1][brow[nb]][(4 * d + g) * 32]);
#pragma unroll
                    for (int pp = 0; pp < 4; pp++) {
                        bh[nb][pp] = bp[pp];
                        if (NS == 2 && !PACK) bl[nb][pp] = bq[pp];
                    }
                }
                uint4 qq[MT];
                float so[MT];
#pragma unroll
                for (int m = 0; m < MT; m++) {
                    const uint32_t sraw = LAYOUT == 0 ? (sq[4 * m + d] >> (8 * g)) & 0xFFu
                                                      : (sq[m] >> (8 * d)) & 0xFFu;
                    /* NaN byte: the block is 0 (a tiled bank stores it as zeros, scale 127) */
                    const bool nanb = LAYOUT == 0 && sraw == 255u;
                    const uint32_t keep = nanb ? 0u : ~0u;       /* a mask, not a branch */
                    qq[m] = qa[S][d][m];
                    qq[m].x &= keep;
                    qq[m].y &= keep;
                    qq[m].z &= keep;
                    qq[m].w &= keep;
                    so[m] = k3_e8m0_operand(nanb ? 127u : sraw);
                }
#pragma unroll
                for (int m = 0; m < MT; m++)
#pragma unroll
                    for (int pp = 0; pp < 4; pp++) {
                        const uint32_t codes = pp == 0 ? qq[m].x : pp == 1 ? qq[m].y : pp == 2 ? qq[m].z : qq[m].w;
                        const k3_bf16x8 av = k3_dequant8_bf16(codes, so[m]);
#pragma unroll
                        for (int nb = 0; nb < NB; nb++) {
                            acc[m][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, k3_as_bf16x8(bh[nb][pp]), acc[m][nb], 0, 0, 0);
                            if (NS == 2 && !PACK)
                                acc[m][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, k3_as_bf16x8(bl[nb][pp]), acc[m][nb], 0, 0, 0);
                        }
                    }
                load_step(c + DEPTH, d, slot);
            }
            if (more) store_b(buf ^ 1);
#pragma unroll
            for (int m = 0; m < SQN; m++) {
                sq[m] = sqn[m];
                if (DEPTH == 2) sqn[m] = sqnn[m];
            }
            __syncthreads();
        };
        for (int c = 0; c < nchunk; c += NSLOT) {
            chunk(c, I0{});
            if (NSLOT == 2 && c + 1 < nchunk) chunk(c + 1, I1{});
        }

        /* epilogue: lane holds token column nb*16 + r16, rows 4g..4g+3 of each tile; PACK:
         * column t gains column 8 + t (hi + lo) */
        if (PACK) {
#pragma unroll
            for (int m = 0; m < MT; m++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++) acc[m][0][jj] += __shfl_down(acc[m][0][jj], 8, 16);
        }
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            const int tk = nb * 16 + r16;
            if (tk >= ntok || (PACK && r16 >= 8)) continue;
            const int orow = a.perm[off + tok0 + tk];
            for (int m = 0; m < RT; m++) {
                const int base = rb * rpg + wv * rpw + 16 * m + 4 * g;
                if (MODE == K3K_MX_GATEUP) {
                    uint16_t hi[4], lo[4];
                    for (int jj = 0; jj < 4; jj++) {
                        const float v = k3_act_pair(acc[m][nb][jj], acc[m + RT][nb][jj], a.act, a.b1, a.b2);
                        k3_split2(v, hi[jj], lo[jj]);
                    }
                    uint16_t *oh = a.ahi + (size_t)orow * rows;
                    uint16_t *ol = a.alo ? a.alo + (size_t)orow * rows : nullptr;
                    for (int jj = 0; jj < 4; jj++)
                        if (base + jj < rows) {
                            oh[base + jj] = hi[jj];
                            if (ol) ol[base + jj] = lo[jj];
                        }
                } else {
                    float *o = a.out + (size_t)orow * rows;
                    if (base + 3 < rows && (rows & 3) == 0) {
                        *reinterpret_cast<float4 *>(o + base) =
                            make_float4(acc[m][nb][0], acc[m][nb][1], acc[m][nb][2], acc[m][nb][3]);
                    } else {
                        for (int jj = 0; jj < 4; jj++)
                            if (base + jj < rows) o[base + jj] = acc[m][nb][jj];
                    }
                }
            }
        }
    }
    if (tid == 0) {
        unsigned long long *sp = stamp_sh;
        if (sp) k3_stamp_end(sp);
    }
}

template <int MODE, int MT, int NS, int PT, int NW, int WPE, int LAYOUT, int DEPTH = 1, int NB = 1>
int launch_moe(const K3kMxArgs *a, int grid, hipStream_t st)
{
    K3kMxArgs b = *a;
    b.stamps = k3k_stamps_take(MODE == K3K_MX_GATEUP ? 1 : 2, grid);
    hipLaunchKernelGGL((mx_moe_kernel<MODE, MT, NS, PT, NB, NW, WPE, LAYOUT, DEPTH>), dim3(grid), dim3(64 * NW),
                       0, st, b);
    K3K_LAUNCH_CHECK("mx_moe launch");
    return 0;
}

/* ---- prefill: large token passes, one-term activations --------------------------------
 * mx_prefill_kernel: GATEUP / DOWN for passes of up to 16*NB tokens with the activations
 * as single bf16 terms (the prefill precision), weights in the tiled MXFP4 layout. An item
 * is (pass, row block); a wave owns MT tiles of 16 weight rows and all the pass's tokens,
 * so every dequantized weight fragment feeds NB MFMAs and each weight byte is read once per
 * pass. K is staged 128 * SPC columns at a time: the pass's activations for a stage are
 * copied into LDS by the buffer unit (buffer_load ... lds: no registers, no LDS store
 * instructions), double-buffered with one barrier per stage, and shared by the NW waves.
 *
 * LDS layout of a stage buffer: 16-byte slots, token p's column piece o (8 bf16) at slot
 * p * (PR + 1) + o: rows padded by one slot, so the 16 tokens of a fragment read start 4
 * banks apart and cover all 64 banks. A DMA instruction fills 64 consecutive slots (lane L
 * the L-th), so each lane loads the piece that its slot holds (a padding slot loads its
 * row's first piece again).
 *
 * The inner loop is software-pipelined over sub-steps u of 32 columns with no branches:
 * while the MT x NB MFMAs of sub-step u issue, the wave dequantizes sub-step u+1's weights
 * (v_cvt_scalef32_pk_bf16_fp4, exact) into a second set of A fragments and reads u+1's B
 * fragments from LDS into the registers that u's MFMAs of the same token block have just
 * consumed; the issue order is pinned with scheduling-group barriers. Weights are loaded
 * two stages ahead into alternating register slots, each step's registers reloaded as soon
 * as its last sub-step is dequantized.
 *
 * All addresses are in bounds by construction: a wave's weight tiles are clamped to the
 * last tile of the matrix, and prefetches past the last stage re-read it (GATEUP) or read
 * at an offset past the end of their buffer (DOWN: zeros, no data moved).
 * Token blocks of a pass past its last token are computed on whatever their LDS rows hold
 * (those rows load a valid token's activations): an output column of an MFMA depends only
 * on its own B row, and those columns are never stored. Weight loads keep the default
 * cache policy: an expert with several passes re-reads its weights, and the caches then
 * serve part of them. */
__device__ __forceinline__ uint4 k3_bload16s(k3_rsrc r, uint32_t voff, uint32_t soff)
{
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ uint32_t k3_bload4s(k3_rsrc r, uint32_t voff, uint32_t soff)
{
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}

template <int MODE, int MT, int NB, int SPC, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 8)))
void mx_prefill_kernel(K3kMxArgs a)
{
    constexpr int KC = 128 * SPC, PT = 16 * NB, PR = KC / 8;
    constexpr int RT = (MODE == K3K_MX_GATEUP) ? MT / 2 : MT;
    constexpr int PRP = PR + 1;                               /* slots per token row */
    constexpr int DPW = (PT * PRP + 64 * NW - 1) / (64 * NW); /* DMA instructions per wave */
    constexpr int NSL = DPW * 64 * NW;                        /* 16-byte slots per stage */
    constexpr int NU = 4 * SPC;                               /* 32-column sub-steps per stage */
    /* s_waitcnt operand: vmcnt <= one stage's weight and scale loads (MT (SPC + 1)), the
     * other counters unconstrained (gfx9 encoding: vmcnt 3:0 and 15:14, expcnt 6:4,
     * lgkmcnt 11:8) */
    constexpr int NLD = MT * (SPC + 1);
    static_assert(NLD < 64, "vmcnt field");
    constexpr int WAIT_STAGE = (NLD & 15) | (7 << 4) | (15 << 8) | ((NLD >> 4) << 14);
    constexpr int WAIT_STAGE_LDS = (NLD & 15) | (7 << 4) | ((NLD >> 4) << 14);   /* and lgkmcnt 0 */
    __shared__ __attribute__((aligned(1024))) uint4 bs0[NSL];
    __shared__ __attribute__((aligned(1024))) uint4 bs1[NSL];
    __shared__ int orow_sh[PT];                               /* the pass's output rows */

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int K = a.K, nblk = K >> 5, nstage = K / KC, nchunk = K >> 9;
    const int rows = a.rows;
    const uint32_t rstride = (uint32_t)K >> 1;
    const int rpw = 16 * RT, rpg = NW * rpw;
    const int n_rb = (rows + rpg - 1) / rpg;
    /* Workgroups go to the XCDs in turn (workgroup b to XCD b % 8). Group x of workgroups
     * (b % nx == x) takes the passes [P x / nx, P (x + 1) / nx) -- an expert's passes are
     * consecutive -- with the row block innermost, so the workgroups of one pass run at
     * about the same time on one XCD and fetch its activations (and the passes of one
     * expert its weights) into that XCD's L2 once. */
    const int npass = *a.n_passes;
    const int nx = min((int)gridDim.x, K3_NXCD);
    const int xg = blockIdx.x % nx, li = blockIdx.x / nx;
    const int nlw = ((int)gridDim.x - 1 - xg) / nx + 1;
    const int pbeg = (int)((long)npass * xg / nx), pend = (int)((long)npass * (xg + 1) / nx);
    const int n_items = (pend - pbeg) * n_rb;
    /* lane's B fragment slot: token r16 (+16 per block), piece 16 (u / 4) + 4 g + u % 4 of
     * the stage (the 8 columns matching the weight codes it holds) */
    const int lrd = r16 * PRP + 4 * g;
    const uint32_t lvoff = (uint32_t)lane * 16u, lsoff = (uint32_t)lane * 4u;
    /* Prefetches past the last stage are issued too, so that every wait counts exactly the
     * loads issued after the one it waits for: DOWN's at a per-lane offset of 2^31, beyond
     * every buffer (zeros, no data moved); GATEUP's re-read the last stage, because the
     * offset select would cost it registers it does not have. The wave-uniform part of
     * each address stays clamped inside the buffer. */
    constexpr uint32_t OOB = 0x80000000u;
    /* the stamps pointer waits in LDS: held in registers through the loop it would spill */
    __shared__ unsigned long long *stamp_sh;
    if (tid == 0) {
        stamp_sh = a.stamps;
        if (a.stamps) k3_stamp_begin(a.stamps);
    }

    /* The group's next item: with a.queue, the next number of the group's counter (zero at
     * launch), so that the workgroups that finish early take more items (fixed shares had
     * left the median workgroup idle the last 9-10 % of the kernel: items of 16 to 56
     * stages, 13 or 14 of them per workgroup); else the fixed share item, item + nlw, ... */
    /* (the counter's address waits in LDS: held in registers through the loop it would
     * spill, as the stamps pointer would) */
    const bool queued = a.queue != nullptr;
    __shared__ int item_sh;
    __shared__ int *queue_sh;
    if (tid == 0) queue_sh = queued ? a.queue + xg : nullptr;
    auto next_item = [&](int cur) -> int {
        if (!queued) return cur < 0 ? li : cur + nlw;
        if (tid == 0) item_sh = __hip_atomic_fetch_add(queue_sh, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        return __builtin_amdgcn_readfirstlane(item_sh);
    };

    for (int item = next_item(-1); item < n_items; item = next_item(item)) {
        const int rb = item % n_rb, pass = pbeg + item / n_rb;
        const int j = a.pass_job[pass];
        const int e = a.job_expert[j];
        const int off = a.job_off[j];
        const int tok0 = a.pass_tp[pass] * PT;
        const int ntok = __builtin_amdgcn_readfirstlane(min(PT, a.job_cnt[j] - tok0));
        const ExpertQDev q = reinterpret_cast<const ExpertQDev *>(a.bank)[e];
        const uint32_t prow = k3_tile_prows(rows);
        const uint32_t pbytes = prow * rstride;
        const uint32_t sbytes = prow * nblk;
        k3_rsrc rp0, rp1, rs0, rs1;
        if (MODE == K3K_MX_GATEUP) {
            rp0 = k3_make_rsrc(q.p1, pbytes); rs0 = k3_make_rsrc(q.s1, sbytes);
            rp1 = k3_make_rsrc(q.p3, pbytes); rs1 = k3_make_rsrc(q.s3, sbytes);
        } else {
            rp0 = rp1 = k3_make_rsrc(q.p2, pbytes);
            rs0 = rs1 = k3_make_rsrc(q.s2, sbytes);
        }
        /* the wave's tiles (wave-uniform byte offsets), clamped to the last tile */
        uint32_t ptile[MT], stile[MT];
        const int ntile = (rows + 15) >> 4;
#pragma unroll
        for (int m = 0; m < MT; m++) {
            const int mt = (MODE == K3K_MX_GATEUP) ? (m % RT) : m;
            const int t = min((rb * rpg + wv * rpw) / 16 + mt, ntile - 1);
            ptile[m] = k3_tile_idx(t, 0, nchunk) * 4096u;
            stile[m] = k3_tile_idx(t, 0, nchunk) * 256u;
        }
        /* DMA sources: instruction i of this wave fills slots 64 (wv + NW i) + lane */
        const uint32_t xbytes = (uint32_t)a.n_xrows * (uint32_t)K * 2u;
        const k3_rsrc rx = k3_make_rsrc(a.xhi, xbytes);
        uint32_t gsrc[DPW];
#pragma unroll
        for (int i = 0; i < DPW; i++) {
            const int s = 64 * (wv + NW * i) + lane, p = s / PRP, o = (s % PRP) % PR;
            const int ar = a.perm[off + tok0 + (p < ntok ? p : 0)];
            const int xr = (MODE == K3K_MX_GATEUP) ? ar / a.topk : ar;
            gsrc[i] = ((uint32_t)xr * (uint32_t)K + (uint32_t)o * 8u) * 2u;
        }

        k3_f32x4 acc[MT][NB];
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
            for (int nb = 0; nb < NB; nb++) acc[m][nb] = k3_f32x4{0.f, 0.f, 0.f, 0.f};

        uint4 qa[2][SPC][MT];                 /* weights of two stages (register slots) */
        uint32_t ss[2][MT];                   /* scale dwords of the two stages, by slot */
        k3_bf16x8 avc[MT], avn[MT];           /* A fragments: sub-step u and u + 1 */
        uint4 bv[NB];                         /* B fragments of the current sub-step */
        auto load_step = [&](int c, int d, auto slot) {
            constexpr int S = decltype(slot)::value;
            /* the 128-column step s of the tile: chunk s / 4, step s % 4 */
            const uint32_t s = (uint32_t)min(c * SPC + d, nstage * SPC - 1);
            const uint32_t bo = (s >> 2) * K3_TILE_CSTRIDE + (s & 3u) * 1024u;
            const uint32_t vo = (MODE == K3K_MX_GATEUP || c < nstage) ? lvoff : OOB;
#pragma unroll
            for (int m = 0; m < MT; m++)
                qa[S][d][m] = k3_bload16s(m < RT || MODE != K3K_MX_GATEUP ? rp0 : rp1, vo, ptile[m] + bo);
        };
        /* the scale dword (4 steps' bytes) of stage c's 512-column chunk into a register slot
         * (c clamped: past the end re-reads the last stage) */
        auto load_scales = [&](int c, auto slot) {
            constexpr int S = decltype(slot)::value;
            const uint32_t so = (uint32_t)(min(c, nstage - 1) * SPC >> 2) * K3_TILE_SCSTRIDE;
            const uint32_t vo = (MODE == K3K_MX_GATEUP || c < nstage) ? lsoff : OOB;
#pragma unroll
            for (int m = 0; m < MT; m++)
                ss[S][m] = k3_bload4s(m < RT || MODE != K3K_MX_GATEUP ? rs0 : rs1, vo, stile[m] + so);
        };
        auto lds_b = [&](auto bufsel, int nb, int u) -> uint4 {
            constexpr int B = decltype(bufsel)::value;
            return (B ? bs1 : bs0)[lrd + nb * 16 * PRP + 16 * (u >> 2) + (u & 3)];
        };
        /* dequantize sub-step u of a register slot; the scale of step c SPC + u / 4 */
        auto deq = [&](const uint4 (&qs)[SPC][MT], const uint32_t *sw, int c, int u, k3_bf16x8 *dst) {
#pragma unroll
            for (int m = 0; m < MT; m++) {
                /* a NaN-scale block is stored as zero codes with scale 127 in the tiled bank */
                const uint32_t sraw = (sw[m] >> (8 * ((c * SPC + (u >> 2)) & 3))) & 0xFFu;
                const uint4 qv = qs[u >> 2][m];
                const uint32_t codes = (u & 3) == 0 ? qv.x : (u & 3) == 1 ? qv.y : (u & 3) == 2 ? qv.z : qv.w;
                dst[m] = k3_dequant8_bf16(codes, k3_e8m0_operand(sraw));
            }
        };

        using P0 = std::integral_constant<int, 0>;
        using P1 = std::integral_constant<int, 1>;
        /* The K loop for passes of NBU token blocks (the blocks past the pass's last token
         * are not computed). */
        auto run = [&](auto nbu_c) {
            constexpr int NBU = decltype(nbu_c)::value;
            constexpr int DPU = (NBU * 16 * PRP + 64 * NW - 1) / (64 * NW);   /* DMA per wave */
            /* stage c's activations (the NBU blocks) into stage buffer B; c clamped: past
             * the end re-reads the last stage */
            auto dma_b = [&](int c, auto bufsel) {
                constexpr int B = decltype(bufsel)::value;
                const uint32_t so = (uint32_t)min(c, nstage - 1) * KC * 2u;
#pragma unroll
                for (int i = 0; i < DPU; i++)
                    k3_dma16(rx, (B ? bs1 : bs0) + 64 * (wv + NW * i), (MODE == K3K_MX_GATEUP || c < nstage) ? gsrc[i] : OOB, so);
            };
            /* Every prefetch is issued unconditionally, so that the wait for a stage's
             * weights counts exactly the loads issued after them instead of draining the
             * queue; the stage count is even. The previous item's last DMA (zeros) has
             * landed and every wave is past its reads before stages 0 and 1 are fetched. */
            /* the output rows of the pass's tokens, loaded under the wait below and kept in
             * LDS once every wave is past the previous item's epilogue, so that this item's
             * epilogue stores wait for nothing */
            const int prow = tid < ntok ? a.perm[off + tok0 + tid] : 0;
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (tid < PT) orow_sh[tid] = prow;
            dma_b(0, P0{});
            dma_b(1, P1{});
            load_scales(0, P0{});
#pragma unroll
            for (int d = 0; d < SPC; d++) load_step(0, d, P0{});
            load_scales(1, P1{});
#pragma unroll
            for (int d = 0; d < SPC; d++) load_step(1, d, P1{});
            deq(qa[0], ss[0], 0, 0, avc);
            __builtin_amdgcn_s_waitcnt(WAIT_STAGE);       /* everything but stage 1's loads */
            __syncthreads();
#pragma unroll
            for (int nb = 0; nb < NBU; nb++) bv[nb] = lds_b(P0{}, nb, 0);

            auto stage = [&](int c, auto slot) {
                constexpr int S = decltype(slot)::value;
                using SN = std::integral_constant<int, S ^ 1>;
#pragma unroll
                for (int u = 0; u < NU; u++) {
                    if (u == NU - 1) {
                        /* This wave's reads of buffer S are in registers and stage c + 1's
                         * activations (DMA issued a stage ago, before this stage's weight
                         * and scale loads) have landed; after the barrier both hold for
                         * every wave: buffer S takes stage c + 2, and the last sub-step's
                         * MFMAs overlap the first reads of stage c + 1. */
                        __builtin_amdgcn_s_waitcnt(WAIT_STAGE_LDS);
                        __syncthreads();
                        dma_b(c + 2, slot);
                    }
                    if (u + 1 < NU) deq(qa[S], ss[S], c, u + 1, avn);
                    else deq(qa[S ^ 1], ss[S ^ 1], c + 1, 0, avn);
#pragma unroll
                    for (int nb = 0; nb < NBU; nb++) {
#pragma unroll
                        for (int m = 0; m < MT; m++)
                            acc[m][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(avc[m], k3_as_bf16x8(bv[nb]), acc[m][nb], 0, 0, 0);
                        if (u + 1 < NU) bv[nb] = lds_b(slot, nb, u + 1);
                        else bv[nb] = lds_b(SN{}, nb, 0);
                    }
                    /* step u / 4's last sub-step is dequantized: its registers take stage
                     * c + 2, and after the stage's last step its scale dwords too */
                    if ((u & 3) == 2) load_step(c + 2, u >> 2, slot);
                    if (u == NU - 2) load_scales(c + 2, slot);
#pragma unroll
                    for (int m = 0; m < MT; m++) avc[m] = avn[m];
                    /* issue order of the sub-step: each token block's MT MFMAs interleaved
                     * with the next sub-step's dequantization, then that block's next B read */
#pragma unroll
                    for (int nb = 0; nb < NBU; nb++) {
#pragma unroll
                        for (int m = 0; m < MT; m++) {
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);      /* MFMA */
                            __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);      /* VALU */
                        }
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);          /* DS read */
                        if ((u & 3) == 2 && nb < MT) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0); /* VMEM */
                        if (u == NU - 2 && nb + MT >= NBU) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            };
            for (int c = 0; c < nstage; c += 2) {
                stage(c, P0{});
                stage(c + 1, P1{});
            }
        };
        switch ((ntok + 15) >> 4) {
            case 1: if (NB >= 1) run(std::integral_constant<int, (NB >= 1 ? 1 : NB)>{}); break;
            case 2: if (NB >= 2) run(std::integral_constant<int, (NB >= 2 ? 2 : NB)>{}); break;
            case 3: if (NB >= 3) run(std::integral_constant<int, (NB >= 3 ? 3 : NB)>{}); break;
            case 4: if (NB >= 4) run(std::integral_constant<int, (NB >= 4 ? 4 : NB)>{}); break;
            case 5: if (NB >= 5) run(std::integral_constant<int, (NB >= 5 ? 5 : NB)>{}); break;
            default: run(std::integral_constant<int, NB>{}); break;
        }

#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            const int tk = nb * 16 + r16;
            if (tk >= ntok) continue;
            const int orow = orow_sh[tk];
            for (int m = 0; m < RT; m++) {
                const int base = rb * rpg + wv * rpw + 16 * m + 4 * g;
                if (MODE == K3K_MX_GATEUP) {
                    /* the activation is rounded to bf16: its fast form suffices */
                    uint16_t h[4];
#pragma unroll
                    for (int jj = 0; jj < 4; jj++)
                        h[jj] = k3_bf16_rne(k3_act_pair_fast(acc[m][nb][jj], acc[m + RT][nb][jj], a.act, a.b1, a.b2));
                    uint16_t *oh = a.ahi + (size_t)orow * rows + base;
                    if (base + 3 < rows && (rows & 3) == 0) {
                        *reinterpret_cast<uint2 *>(oh) = make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
                    } else {
                        for (int jj = 0; jj < 4; jj++)
                            if (base + jj < rows) oh[jj] = h[jj];
                    }
                    __builtin_amdgcn_sched_barrier(0);
                } else {
                    float *o = a.out + (size_t)orow * rows;
                    if (base + 3 < rows && (rows & 3) == 0) {
                        *reinterpret_cast<float4 *>(o + base) =
                            make_float4(acc[m][nb][0], acc[m][nb][1], acc[m][nb][2], acc[m][nb][3]);
                    } else {
                        for (int jj = 0; jj < 4; jj++)
                            if (base + jj < rows) o[base + jj] = acc[m][nb][jj];
                    }
                }
            }
        }
    }
    if (tid == 0) {
        unsigned long long *sp = stamp_sh;
        if (sp) k3_stamp_end(sp);
    }
}

template <int MODE, int MT, int NB, int SPC, int NW>
int launch_prefill(const K3kMxArgs *a, int grid, hipStream_t st)
{
    K3kMxArgs b = *a;
    b.stamps = k3k_stamps_take(MODE == K3K_MX_GATEUP ? 3 : 4, grid);
    hipLaunchKernelGGL((mx_prefill_kernel<MODE, MT, NB, SPC, NW>), dim3(grid), dim3(64 * NW), 0, st, b);
    K3K_LAUNCH_CHECK("mx_prefill launch");
    return 0;
}

/* ---- generic vector-unit GEMV: any even K, group <= 64, fp32 arithmetic ---------- */
/* One wave per row; lane-strided elements, weight = E2M1 * 2^(s-127) in fp32 (exact),
 * fp32 fma accumulation, butterfly reduction. */
__global__ __launch_bounds__(256) void mx_gemv_valu_kernel(float *y, const float *x,
                                                           const uint8_t *packed,
                                                           const uint8_t *scales, int in,
                                                           int rows, int group)
{
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int ngrp = (in + group - 1) / group;
    const uint8_t *pr = packed + (size_t)r * (in / 2);
    const uint8_t *sr = scales + (size_t)r * ngrp;
    float acc = 0.0f;
    for (int i = lane; i < in; i += 64) {
        const uint32_t sb = sr[i / group];
        if (sb == 255u) continue;
        const uint32_t b = pr[i >> 1];
        const uint32_t code = (i & 1) ? (b >> 4) : (b & 15u);
        acc = fmaf(k3_e2m1_value(code) * k3_e8m0_value(sb), x[i], acc);
    }
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (lane == 0) y[r] = acc;
}

__global__ void mx_dequant_kernel(float *out, const uint8_t *packed, const uint8_t *scales,
                                  int rows, int pcols, int group)
{
    const int width = pcols * 2, ngrp = (width + group - 1) / group;
    const size_t n = (size_t)rows * width;
    for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < n;
         t += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(t / width), i = (int)(t % width);
        const uint32_t b = packed[(size_t)r * pcols + (i >> 1)];
        const uint32_t code = (i & 1) ? (b >> 4) : (b & 15u);
        out[t] = k3_e2m1_value(code) * k3_e8m0_value(scales[(size_t)r * ngrp + i / group]);
    }
}

/* Row-major MXFP4 -> the tiled layout read by the LAYOUT 1 kernels. For row tile t (16
 * rows), K chunk c (16 blocks of 32), i = k3_tile_idx(t, c) and lane l = 16g + r (r = row
 * in tile):
 *   codes:  tpacked[(i*4 + d)*1024 + 16l ..+16] = block 4d+g of row 16t+r
 *   scales: tscales[i*256 + 4l + d]             = scale of that block
 * A block whose scale byte is 255 (NaN, zero in the reference) is stored as zero codes with
 * scale byte 127, which contributes the same zero. Rows past `rows` (up to the next
 * multiple of 64) are zero codes with scale byte 0. */
__global__ void mx_tile_kernel(uint8_t *tpacked, uint8_t *tscales, const uint8_t *packed,
                               const uint8_t *scales, int rows, int K)
{
    const int nchunk = K / 512, nblk = K / 32, ntile = (int)(k3_tile_prows(rows) / 16);
    const size_t n = (size_t)ntile * nchunk * 64;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const int l = (int)(i & 63);
        const size_t tc = i >> 6;                          /* t*nchunk + c */
        const int c = (int)(tc % nchunk), t = (int)(tc / nchunk);
        const int r = l & 15, g = l >> 4, row = 16 * t + r;
        uint32_t sw = 0;
        for (int d = 0; d < 4; d++) {
            const int blk = c * 16 + 4 * d + g;
            uint4 v = make_uint4(0, 0, 0, 0);
            uint32_t sb = 0;
            if (row < rows) {
                v = *reinterpret_cast<const uint4 *>(packed + (size_t)row * (K / 2) + (size_t)blk * 16);
                sb = scales[(size_t)row * nblk + blk];
            }
            /* NaN scale: the block contributes 0. Stored as zero codes with scale 2^0, so
             * the kernels that read this layout need no test for it. */
            if (sb == 255u) {
                v = make_uint4(0, 0, 0, 0);
                sb = 127u;
            }
            *reinterpret_cast<uint4 *>(tpacked + (((size_t)k3_tile_idx(t, c, nchunk) * 4 + d) * 1024) + (size_t)l * 16) = v;
            sw |= sb << (8 * d);
        }
        *reinterpret_cast<uint32_t *>(tscales + (size_t)k3_tile_idx(t, c, nchunk) * 256 + (size_t)l * 4) = sw;
    }
}

}  // namespace

extern "C" int k3k_mx_gemm(int mode, const K3kMxArgs *a, void *stream)
{
    hipStream_t st = (hipStream_t)stream;
    if (a->K <= 0 || (a->K & 31) || a->rows <= 0) return k3k_fail("mx_gemm shape", hipErrorInvalidValue);
    const int cus = k3k_cu_count();
    const int nsteps = (a->K / 32 + 3) / 4;
    if (mode == K3K_MX_PLAIN) {
        if (a->ntok <= 0) return 0;
        if (a->xf32) {
            /* one or two fp32 tokens, activations staged in LDS: waves of one 512-column
             * chunk when K allows, else up to 16 waves of <= 8 steps */
            if (!k3k_mx_small_ok(a->ntok, a->K, a->nsplit, a->rows, a->xf32))
                return k3k_fail("mx_gemm: fp32 activations need ntok <= 2 and a small K",
                                hipErrorInvalidValue);
            const bool chunked = a->K % 512 == 0 && a->K <= 16 * 512;
            const int kw = chunked ? a->K / 512 : (nsteps + 7) / 8;
            size_t lds = (size_t)a->nsplit * a->ntok * a->K * 2;
            if (lds < (size_t)kw * 1024) lds = (size_t)kw * 1024;
            /* chunked: per wave ntok nsplit + 1 columns of 512 bf16, then the sums */
            if (chunked) lds = (size_t)kw * (a->ntok * a->nsplit + 1) * 1024 + (size_t)kw * a->ntok * 64;
            /* fewer 16-row tiles than CUs: 8-row tiles, two chunks per wave */
            const bool pair = chunked && a->K % 1024 == 0 && (a->rows + 15) / 16 < cus;
            const int grid = pair ? (a->rows + 7) / 8 : (a->rows + 15) / 16;
            void (*kern)(K3kMxArgs, int);
            if (pair)
                kern = a->nsplit == 2 ? mx_gemv_pair_kernel<2> : mx_gemv_pair_kernel<1>;
            else if (chunked)
                kern = a->nsplit == 2 ? mx_gemv_chunk_kernel<2> : mx_gemv_chunk_kernel<1>;
            else
                kern = a->nsplit == 2 ? mx_gemv_small_kernel<2, 8> : mx_gemv_small_kernel<1, 8>;
            const int wpb = pair ? kw / 2 : kw;             /* waves per workgroup */
            hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * wpb), lds, st, *a, wpb);
            K3K_LAUNCH_CHECK("mx_gemv_small launch");
            return 0;
        }
        /* One matrix: items of 16 rows; K split over up to 16 waves of a workgroup so that
         * about 2k waves each issue their whole K share (<= 4 steps) at once. */
        const int items = ((a->rows + 15) / 16) * ((a->ntok + 15) / 16);
        int kw = (nsteps + 3) / 4;
        if (kw > 16) kw = 16;
        const int grid = items < cus * 8 ? items : cus * 8;
        if (a->nsplit == 2) return launch_mx<K3K_MX_PLAIN, 1, 1, 2, 2, 16>(a, kw, grid, st);
        return launch_mx<K3K_MX_PLAIN, 1, 1, 1, 2, 16>(a, kw, grid, st);
    }
    if (a->pass_tok == 48 || a->pass_tok == 96) {
        /* large prefill batches on a tiled bank: 48-token passes (K staged 256 columns at a
         * time) or 96-token passes (128 columns at a time, so the pass fits in LDS twice
         * per CU); weights two stages ahead; each dequantized weight fragment feeds 3 or 6
         * MFMA column blocks */
        if (a->K % 512 || a->nsplit != 1 || a->layout != 1)
            return k3k_fail("mx_moe: 48/96-token passes need K % 512 == 0, bf16 activations and "
                            "a tiled bank", hipErrorInvalidValue);
        const bool gu = mode == K3K_MX_GATEUP;
        /* 8 waves per workgroup (one workgroup per CU at two waves per SIMD): twice the rows
         * per staged copy of the pass's activations of 4 waves, half the activation reads */
        const int rpg = gu ? 256 : 512;
        const long items = (long)a->max_passes * ((a->rows + rpg - 1) / rpg);
        const int grid = (int)(items < (long)cus ? (items > 0 ? items : 1) : (long)cus);
        if (a->pass_tok == 96)
            return gu ? launch_prefill<K3K_MX_GATEUP, 4, 6, 1, 8>(a, grid, st)
                      : launch_prefill<K3K_MX_DOWN, 4, 6, 1, 8>(a, grid, st);
        return gu ? launch_prefill<K3K_MX_GATEUP, 4, 3, 2, 8>(a, grid, st)
                  : launch_prefill<K3K_MX_DOWN, 4, 3, 2, 8>(a, grid, st);
    }
    if (a->pass_tok == 32) {
        /* prefill: 32-token passes, two MFMA column blocks per weight fragment, activations
         * as one bf16 term (the bf16-MFMA prefill precision) */
        if (a->K % 512 || a->nsplit != 1)
            return k3k_fail("mx_moe: 32-token passes need K % 512 == 0 and bf16 activations",
                            hipErrorInvalidValue);
        const bool gu = mode == K3K_MX_GATEUP;
        const int rpg = gu ? 128 : 256;
        const long items = (long)a->max_passes * ((a->rows + rpg - 1) / rpg);
        const int grid = (int)(items < (long)cus * 4 ? (items > 0 ? items : 1) : (long)cus * 4);
        const bool tiled = a->layout == 1;
        if (gu)
            return tiled ? launch_moe<K3K_MX_GATEUP, 4, 1, 32, 4, 2, 1, 1, 2>(a, grid, st)
                         : launch_moe<K3K_MX_GATEUP, 4, 1, 32, 4, 2, 0, 1, 2>(a, grid, st);
        return tiled ? launch_moe<K3K_MX_DOWN, 4, 1, 32, 4, 2, 1, 1, 2>(a, grid, st)
                     : launch_moe<K3K_MX_DOWN, 4, 1, 32, 4, 2, 0, 1, 2>(a, grid, st);
    }
    if (a->pass_tok == 8) {
        /* LDS-staged expert kernel: K % 512 == 0. Items are 4 waves x MT tiles of 16 rows;
         * when there are too few of them to fill the chip (decode at batch 1-4), halve the
         * tiles per wave so that twice as many workgroups stream weights, and (gate/up, 14
         * chunks of K) keep two chunks of weights in flight per wave. */
        if (a->K % 512) return k3k_fail("mx_moe: K % 512 != 0", hipErrorInvalidValue);
        const bool gu = mode == K3K_MX_GATEUP;
        const long items4 = (long)a->max_passes * ((a->rows + (gu ? 127 : 255)) / (gu ? 128 : 256));
        const bool small = items4 < 2L * cus;
        const int rpg = gu ? (small ? 64 : 128) : (small ? 128 : 256);
        const long items = (long)a->max_passes * ((a->rows + rpg - 1) / rpg);
        const int grid = (int)(items < (long)cus * 4 ? (items > 0 ? items : 1) : (long)cus * 4);
        const bool tiled = a->layout == 1;
        const bool ns2 = a->nsplit == 2;
#define K3_MOE_LAUNCH(MODE, MT, D)                                                           \
    return tiled ? (ns2 ? launch_moe<MODE, MT, 2, 8, 4, 2, 1, D>(a, grid, st)                \
                        : launch_moe<MODE, MT, 1, 8, 4, 2, 1, D>(a, grid, st))               \
                 : (ns2 ? launch_moe<MODE, MT, 2, 8, 4, 2, 0, D>(a, grid, st)                \
                        : launch_moe<MODE, MT, 1, 8, 4, 2, 0, D>(a, grid, st))
        if (gu) {
            if (small) K3_MOE_LAUNCH(K3K_MX_GATEUP, 2, 2);
            K3_MOE_LAUNCH(K3K_MX_GATEUP, 4, 1);
        }
        if (small) K3_MOE_LAUNCH(K3K_MX_DOWN, 2, 1);
        K3_MOE_LAUNCH(K3K_MX_DOWN, 4, 1);
#undef K3_MOE_LAUNCH
    }
    if (a->pass_tok != 16 || a->layout != 0)
        return k3k_fail("mx_gemm: expert passes of 16 tokens need the row-major layout",
                        hipErrorInvalidValue);
    /* Expert jobs: 16 output rows per item (GATEUP: 16 gate + the same 16 up rows). */
    const int n_rb = mode == K3K_MX_GATEUP ? (a->rows + 15) / 16 : (a->rows + 31) / 32;
    const long items = (long)a->max_passes * n_rb;
    int kw = 1;
    while (kw < 8 && items * kw < (long)cus * 8 && nsteps / (2 * kw) >= 4) kw *= 2;
    long grid = items < (long)cus * 16 / kw ? items : (long)cus * 16 / kw;
    if (grid < 1) grid = 1;
    if (mode == K3K_MX_GATEUP) {
        if (a->nsplit == 2) return launch_mx<K3K_MX_GATEUP, 2, 1, 2, 2, 8>(a, kw, (int)grid, st);
        return launch_mx<K3K_MX_GATEUP, 2, 1, 1, 2, 8>(a, kw, (int)grid, st);
    }
    if (a->nsplit == 2) return launch_mx<K3K_MX_DOWN, 2, 1, 2, 2, 8>(a, kw, (int)grid, st);
    return launch_mx<K3K_MX_DOWN, 2, 1, 1, 2, 8>(a, kw, (int)grid, st);
}

extern "C" int k3k_mx_decode(int mode, const K3kMxArgs *a, void *stream)
{
    if (a->n_assign <= 0) return 0;
    if (a->K % 512 || a->K > 16 * 512 || a->n_assign > 16 || a->layout > 1 ||
        (mode == K3K_MX_GATEUP && (uintptr_t)a->xf32 % 16) ||
        (size_t)k3_tile_prows(a->rows) * (a->K / 2) >= 0x80000000u)
        return k3k_fail("mx_decode: shape", hipErrorInvalidValue);
    /* 4 tiles per workgroup, K over 2 waves per tile, when that gives >= 256 workgroups;
     * otherwise (one or two assignments) 1 tile per workgroup, K over up to 16 waves
     * (at least 4, which the activation staging needs) */
    const int ntile = (a->rows + 15) / 16, nchunk = a->K / 512;
    const bool wide = (long)a->n_assign * ((ntile + 3) / 4) >= 256 || nchunk < 4;
    /* gate and up in workgroups of their own, sums to a.gu (one tile per workgroup) */
    const bool split = mode == K3K_MX_GATEUP && a->gu && !a->sel;
    if (split && wide) return k3k_fail("mx_decode: split gate/up needs few assignments", hipErrorInvalidValue);
    const int nm = mode == K3K_MX_GATEUP && !split ? 2 : 1;
    const int tpw = wide ? 4 : 1;
    const int ks = wide ? 2 : (nchunk < 16 ? nchunk : 16);
    size_t lds = (size_t)a->nsplit * a->K * 2 + 1024;
    if (lds < (size_t)(ks - 1) * tpw * nm * 1024) lds = (size_t)(ks - 1) * tpw * nm * 1024;
    const int grid = a->n_assign * ((ntile + tpw - 1) / tpw) * (split ? 2 : 1);
    void (*kern)(K3kMxArgs);
    const bool ns2 = a->nsplit == 2, tiled = a->layout == 1;
#define K3_DEC(MODE, TPW)                                                                          \
    kern = tiled ? (ns2 ? mx_decode_kernel<MODE, 2, 1, TPW> : mx_decode_kernel<MODE, 1, 1, TPW>)     \
                 : (ns2 ? mx_decode_kernel<MODE, 2, 0, TPW> : mx_decode_kernel<MODE, 1, 0, TPW>)
#define K3_DEC_SEL(TPW)                                                                            \
    kern = tiled ? (ns2 ? mx_decode_kernel<K3K_MX_GATEUP, 2, 1, TPW, true>                           \
                        : mx_decode_kernel<K3K_MX_GATEUP, 1, 1, TPW, true>)                          \
                 : (ns2 ? mx_decode_kernel<K3K_MX_GATEUP, 2, 0, TPW, true>                           \
                        : mx_decode_kernel<K3K_MX_GATEUP, 1, 0, TPW, true>)
    if (mode == K3K_MX_GATEUP && a->sel) {
        if (!a->pre || !a->rw || !a->idx_out || !a->wt_out || a->n_experts > 512 || a->topk > 64 ||
            a->n_assign % a->topk)
            return k3k_fail("mx_decode: selection arguments", hipErrorInvalidValue);
        if (wide) K3_DEC_SEL(4);
        else K3_DEC_SEL(1);
    } else if (split) {
        kern = tiled ? (ns2 ? mx_decode_kernel<K3K_MX_GATEUP, 2, 1, 1, false, true>
                            : mx_decode_kernel<K3K_MX_GATEUP, 1, 1, 1, false, true>)
                     : (ns2 ? mx_decode_kernel<K3K_MX_GATEUP, 2, 0, 1, false, true>
                            : mx_decode_kernel<K3K_MX_GATEUP, 1, 0, 1, false, true>);
    } else if (mode == K3K_MX_GATEUP) {
        if (wide) K3_DEC(K3K_MX_GATEUP, 4);
        else K3_DEC(K3K_MX_GATEUP, 1);
    } else {
        if (wide) K3_DEC(K3K_MX_DOWN, 4);
        else K3_DEC(K3K_MX_DOWN, 1);
    }
#undef K3_DEC
#undef K3_DEC_SEL
    hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * tpw * ks), lds, (hipStream_t)stream, *a);
    K3K_LAUNCH_CHECK("mx_decode launch");
    return 0;
}

/* dynamic LDS of mx_decode_combine_kernel: all of the CU's 160 KB but its 4 KB of static arrays */
#define K3_DC_LDS_MAX (160 * 1024 - 4096)

/* The fused kernel is used where it is faster than mx_decode_kernel DOWN + the combine
 * kernel and the slots' activation terms of one token fit in its LDS: one or two
 * assignments (7168 x 2048: 18.3 against 20.3 us for one expert's FFN), and one token of
 * up to eight slots with one K share per slot (eight waves), so that two workgroups fit a
 * CU and every tile's workgroup is resident at once. */
static int dc_shares(int topk, int K)
{
    const int nchunk = K / 512;
    int ks = (topk <= 2 ? 16 : 8) / topk;
    if (ks < 1) ks = 1;
    return ks > nchunk ? nchunk : ks;
}

extern "C" int k3k_mx_decode_combine_ok(int n_assign, int topk, int nsplit, int K, int rows)
{
    const long ntile = (rows + 15) / 16;
    const bool wide = (long)n_assign * ((ntile + 3) / 4) >= 256 || K / 512 < 4;
    const bool one_token = n_assign == topk && topk <= 8 && K / 512 >= 1;
    return (!wide || one_token) && topk >= 1 && topk <= 16 &&
           (size_t)topk * nsplit * K * 2 + 1024 <= K3_DC_LDS_MAX;
}

extern "C" int k3k_mx_decode_split_ok(int n_assign, int topk, int nsplit, int K, int rows, int K_down,
                                      int rows_down)
{
    const long ntile = (rows + 15) / 16;
    const bool wide = (long)n_assign * ((ntile + 3) / 4) >= 256 || K / 512 < 4;
    return !wide && k3k_mx_decode_combine_ok(n_assign, topk, nsplit, K_down, rows_down);
}

extern "C" int k3k_mx_decode_combine(const K3kMxArgs *a, void *stream)
{
    if (a->n_assign <= 0) return 0;
    if (a->K % 512 || a->K > 16 * 512 || a->n_assign > 16 || a->layout > 1 || a->topk < 1 ||
        a->n_assign % a->topk || !a->wt ||
        (size_t)k3_tile_prows(a->rows) * (a->K / 2) >= 0x80000000u)
        return k3k_fail("mx_decode_combine: shape", hipErrorInvalidValue);
    /* waves: topk slots x K shares, at most 16 (at most 8 from three slots) */
    const int ks = dc_shares(a->topk, a->K);
    const int T = a->n_assign / a->topk, ntile = (a->rows + 15) / 16;
    if ((size_t)a->topk * a->nsplit * a->K * 2 + 1024 > K3_DC_LDS_MAX)
        return k3k_fail("mx_decode_combine: LDS", hipErrorInvalidValue);
    const size_t lds = (size_t)a->topk * a->nsplit * a->K * 2 + 1024;
    void (*kern)(K3kMxArgs);
    const bool ns2 = a->nsplit == 2, tiled = a->layout == 1;
    if (a->gu)      /* activations from the gate and up sums */
        kern = tiled ? (ns2 ? mx_decode_combine_kernel<2, 1, true> : mx_decode_combine_kernel<1, 1, true>)
                     : (ns2 ? mx_decode_combine_kernel<2, 0, true> : mx_decode_combine_kernel<1, 0, true>);
    else
        kern = tiled ? (ns2 ? mx_decode_combine_kernel<2, 1> : mx_decode_combine_kernel<1, 1>)
                     : (ns2 ? mx_decode_combine_kernel<2, 0> : mx_decode_combine_kernel<1, 0>);
    static bool attr = false;
    if (!attr) {
        const void *ks8[8] = {reinterpret_cast<const void *>(mx_decode_combine_kernel<2, 1>),
                              reinterpret_cast<const void *>(mx_decode_combine_kernel<1, 1>),
                              reinterpret_cast<const void *>(mx_decode_combine_kernel<2, 0>),
                              reinterpret_cast<const void *>(mx_decode_combine_kernel<1, 0>),
                              reinterpret_cast<const void *>(mx_decode_combine_kernel<2, 1, true>),
                              reinterpret_cast<const void *>(mx_decode_combine_kernel<1, 1, true>),
                              reinterpret_cast<const void *>(mx_decode_combine_kernel<2, 0, true>),
                              reinterpret_cast<const void *>(mx_decode_combine_kernel<1, 0, true>)};
        for (int i = 0; i < 8; i++) {
            const hipError_t e = hipFuncSetAttribute(ks8[i], hipFuncAttributeMaxDynamicSharedMemorySize, K3_DC_LDS_MAX);
            if (e != hipSuccess) return k3k_fail("mx_decode_combine: LDS attribute", e);
        }
        attr = true;
    }
    hipLaunchKernelGGL(kern, dim3(T * ntile), dim3(64 * a->topk * ks), lds, (hipStream_t)stream, *a);
    K3K_LAUNCH_CHECK("mx_decode_combine launch");
    return 0;
}

extern "C" int k3k_mx_tile(uint8_t *tpacked, uint8_t *tscales, const uint8_t *packed,
                           const uint8_t *scales, int rows, int K, void *stream)
{
    if (rows <= 0) return 0;
    if (K <= 0 || K % 512) return k3k_fail("mx_tile: K % 512 != 0", hipErrorInvalidValue);
    const size_t n = (size_t)(k3_tile_prows(rows) / 16) * (K / 512) * 64;
    const size_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(mx_tile_kernel, dim3(blocks < 16384 ? (unsigned)blocks : 16384u), dim3(256),
                       0, (hipStream_t)stream, tpacked, tscales, packed, scales, rows, K);
    K3K_LAUNCH_CHECK("mx_tile launch");
    return 0;
}

extern "C" int k3k_mx_gemv_valu(float *y, const float *x, const uint8_t *packed,
                                const uint8_t *scales, int in, int rows, int group, void *stream)
{
    if (rows <= 0) return 0;
    hipLaunchKernelGGL(mx_gemv_valu_kernel, dim3((rows + 3) / 4), dim3(256), 0,
                       (hipStream_t)stream, y, x, packed, scales, in, rows, group);
    K3K_LAUNCH_CHECK("mx_gemv_valu launch");
    return 0;
}

extern "C" int k3k_mx_dequant(float *out, const uint8_t *packed, const uint8_t *scales, int rows,
                              int pcols, int group, void *stream)
{
    const size_t n = (size_t)rows * pcols * 2;
    if (n == 0) return 0;
    const size_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(mx_dequant_kernel, dim3(blocks < 65536 ? (unsigned)blocks : 65536u),
                       dim3(256), 0, (hipStream_t)stream, out, packed, scales, rows, pcols, group);
    K3K_LAUNCH_CHECK("mx_dequant launch");
    return 0;
}
