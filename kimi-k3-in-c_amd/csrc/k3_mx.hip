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
#include "k3k.h"

namespace {

struct ExpertQDev {
    const uint8_t *p1, *s1, *p3, *s3, *p2, *s2;
};

__device__ __forceinline__ uint4 ld16(const uint8_t *p)
{
    return *reinterpret_cast<const uint4 *>(p);
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
                    sc[d][m] = v ? (uint32_t)sa[m][blk] : 127u;
                }
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    const bool ok = v && tv[nt];
                    const uint4 *ph = reinterpret_cast<const uint4 *>(xh[nt] + (size_t)blk * 32);
#pragma unroll
                    for (int p = 0; p < 4; p++) bh[d][nt][p] = ok ? ph[p] : make_uint4(0, 0, 0, 0);
                    if (NS == 2) {
                        const uint4 *pl = reinterpret_cast<const uint4 *>(xl[nt] + (size_t)blk * 32);
#pragma unroll
                        for (int p = 0; p < 4; p++) bl[d][nt][p] = ok ? pl[p] : make_uint4(0, 0, 0, 0);
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

}  // namespace

extern "C" int k3k_mx_gemm(int mode, const K3kMxArgs *a, void *stream)
{
    hipStream_t st = (hipStream_t)stream;
    if (a->K <= 0 || (a->K & 31) || a->rows <= 0) return k3k_fail("mx_gemm shape", hipErrorInvalidValue);
    const int cus = k3k_cu_count();
    const int nsteps = (a->K / 32 + 3) / 4;
    if (mode == K3K_MX_PLAIN) {
        if (a->ntok <= 0) return 0;
        /* One matrix: items of 16 rows; K split over up to 16 waves of a workgroup so that
         * about 2k waves each issue their whole K share (<= 4 steps) at once. */
        const int items = ((a->rows + 15) / 16) * ((a->ntok + 15) / 16);
        int kw = (nsteps + 3) / 4;
        if (kw > 16) kw = 16;
        const int grid = items < cus * 8 ? items : cus * 8;
        if (a->nsplit == 2) return launch_mx<K3K_MX_PLAIN, 1, 1, 2, 2, 16>(a, kw, grid, st);
        return launch_mx<K3K_MX_PLAIN, 1, 1, 1, 2, 16>(a, kw, grid, st);
    }
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
