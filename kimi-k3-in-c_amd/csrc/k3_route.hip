/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_route.hip -- the routing side of the MoE layer on gfx950: activation split, the
 * sigmoid top-k router, the expert-major gather, the weighted combine, and the small
 * elementwise kernels (activation, RMSNorm).
 */
#include "k3_common.h"
#include "k3_expf.h"
#include "k3_select.h"
#include "k3k.h"

#include <string.h>

namespace {

struct ExpertQDev {
    const uint8_t *p1, *s1, *p3, *s3, *p2, *s2;
};

__device__ __forceinline__ bool expert_present(const void *bank, int e)
{
    /* all six pointers tested without short-circuit, so they load together */
    const ExpertQDev q = reinterpret_cast<const ExpertQDev *>(bank)[e];
    return (q.p1 != nullptr) & (q.s1 != nullptr) & (q.p3 != nullptr) & (q.s3 != nullptr) &
           (q.p2 != nullptr) & (q.s2 != nullptr);
}

/* ---- fp32 -> bf16 hi/lo ----------------------------------------------------------- */
/* four elements per float4: 16-byte loads, 8-byte stores (n % 4 == 0, 16-byte aligned x).
 * A thread takes SPLIT_U float4s a grid stride apart and requests them all before it
 * converts any, so each lane keeps SPLIT_U loads in flight (with one, a full chip of
 * waves keeps too few bytes in flight to cover the memory latency). */
constexpr int SPLIT_U = 4;
__device__ __forceinline__ void split4_store(uint2 *hi, uint2 *lo, size_t i, float4 v)
{
    uint16_t h[4], l[4];
    k3_split2(v.x, h[0], l[0]);
    k3_split2(v.y, h[1], l[1]);
    k3_split2(v.z, h[2], l[2]);
    k3_split2(v.w, h[3], l[3]);
    hi[i] = make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
    if (lo) lo[i] = make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
}

__global__ void split4_kernel(uint2 *hi, uint2 *lo, const float4 *x, size_t n4)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + (SPLIT_U - 1) * stride < n4; i += SPLIT_U * stride) {
        float4 v[SPLIT_U];
#pragma unroll
        for (int u = 0; u < SPLIT_U; u++) v[u] = x[i + u * stride];
#pragma unroll
        for (int u = 0; u < SPLIT_U; u++) split4_store(hi, lo, i + u * stride, v[u]);
    }
    for (; i < n4; i += stride) split4_store(hi, lo, i, x[i]);
}

__global__ void split_kernel(uint16_t *hi, uint16_t *lo, const float *x, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        uint16_t h, l;
        k3_split2(x[i], h, l);
        hi[i] = h;
        if (lo) lo[i] = l;
    }
}

/* ---- router scores ------------------------------------------------------------------
 * logit[t][e] = the reference's own fp64 chain: acc = 0; for k ascending: acc += (double)
 * W[e][k] * (double)x[t][k] (k3_ops.c:446-450), score = 1/(1+expf(-(float)acc)) with the
 * host libm's expf (k3_ops.c:451) and choice = score + bias (k3_ops.c:452). The exact
 * score (router_score), the reference's chain (chain_block) and the selection
 * (select_rounds) are in k3_select.h, shared with the decode kernels. */

/* ---- router logits, certified ---------------------------------------------------------
 * The reference's logit is one sequential fp64 chain per (token, expert):
 *   a_0 = 0, a_{i+1} = fl(a_i + w_i x_i), i ascending, logit = (float)a_n
 * (k3_ops.c:446-451; the product of two floats is exact in fp64, so fma(w, x, a) rounds
 * like the separate multiply and add). Run literally, that is a 7168-step dependent chain
 * per logit. Instead:
 *
 * 1. The partial kernels compute, per K chunk k of C_k columns, the chunk's own sum P_k
 *    (from 0, its products added in any order with at most 32 roundings per 32-column
 *    sub-block) and R_k, an upper bound on the sum of |r_i| over the intermediate values
 *    r_i that are rounded: per sub-block, 32 * (|r at its start| + ||w||_1 * ||x||_inf of
 *    the sub-block).
 * 2. router_final_kernel sums S = P_0 + P_1 + ... in k order and bounds |S - a_n|: with
 *    u = 2^-53 and Q_k the prefix before chunk k, the reference's chain errs from the
 *    exact sum by at most u * sum_i |a_i| <= u * sum_k (C_k |Q_k| + R_k), this
 *    computation by at most u * sum_k (R_k + |Q_{k+1}|); B = 1.01 u sum_k (C_k |Q_k| +
 *    2 R_k + |Q_{k+1}|) + 4u|S| covers both and the second-order terms. If every value in
 *    [S - B, S + B] rounds to the same float, that float is the reference's logit.
 * 3. Logits that are not certified and could matter -- the expert is selected (its weight
 *    must be exact) or its choice could reach the selection -- are recomputed with the
 *    reference's chain itself, and the selection is redone until no such logit is left.
 */

/* A computed bound rb with relative error below rel - 1 as a float that is no smaller
 * than the true bound: scaled up, converted, scaled by one more float rounding; the floor
 * 2^-120 covers the absolute (subnormal) rounding errors that escape the relative form. */
__device__ __forceinline__ float bound_up(double rb, double rel)
{
    return (float)(rb * rel) * (1.0f + 0x1p-20f) + 0x1p-120f;
}

constexpr int RP_KS = 32, RP_SUB = 32;     /* chunk granule and bound sub-block, columns */

/* Partials of more than four tokens on the fp64 matrix cores. v_mfma_f64_16x16x4f64 adds
 * to each element of a 16 x 16 block four exact products (fp32 operands widened to fp64
 * multiply exactly) with at most four round-to-nearest additions, so a chunk's value is
 * again a sum of its products with at most 32 roundings per 32-column sub-block, each of
 * an intermediate bounded by |r at the sub-block's start| + ||w||_1 ||x||_inf of the
 * sub-block: R_k keeps the form above. (Measured on gfx950: the instruction adds the four
 * products to the accumulator one after another in k order, each addition rounded to
 * nearest even; the bound needs only their count.) The order of the products inside a
 * sub-block is free (both operands take the same permutation): lane group q = l / 16
 * takes columns 8q .. 8q + 7, so a lane's operands of a sub-block are two 16-byte LDS
 * reads.
 *
 * Tokens are the rows of the blocks (A operand, row i at lane i + 16 q), experts the
 * columns (B operand), so element (i, j) sits at lane j + 16 (i % 4), register i / 4 and
 * 16 lanes store 16 consecutive experts of one token. A wave computes MT x ME blocks
 * (16 MT tokens x 16 ME experts), the 4 waves of a workgroup 2 x 2 of those. W and x are
 * staged in LDS as fp32 (rows padded to 36 floats: the 16-byte reads of 8 consecutive
 * lanes fall on distinct banks), double buffered, with the sub-block norms. The bound is
 * accumulated in fp32, rounded up at the end by its relative error ((nsub + 4) 2^-24).
 *
 * The sub-blocks are loaded two ahead into a ring of two register slots. With BUF (rows
 * a multiple of 4 floats, 16-byte aligned, W and x under 2 GiB) every load is a buffer
 * load with no branch around it (rows and columns past the tile's read at an offset beyond
 * the buffer: zeros), so each wait counts exactly the loads issued after the ones it waits
 * for and sub-block sc + 2 stays in flight while sc is multiplied and sc + 1 stored.
 *
 * On gfx950 the fp64 MFMA and the vector instructions of the waves of a SIMD do not
 * overlap (measured: each fp32 FMA between two v_mfma_f64_16x16x4f64 adds 1-2 ns to the
 * SIMD's time), so the kernel's time is about the MFMAs' plus the vector work's plus the
 * latency the waves cannot hide. */
constexpr int RM_LD = 36;

/* v combined with the value of the lane DPP control CTRL names (quad_perm, row_half_mirror:
 * each names a lane of the same group of eight) */
template <int CTRL>
__device__ __forceinline__ float dpp8_f32(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
/* sum / maximum over each aligned group of 8 lanes, in every lane of the group: pairs
 * (quad_perm [1,0,3,2]), quads ([2,3,0,1]), then the two quads (row_half_mirror), so lane
 * 8g + i holds ((v0 + v1) + (v2 + v3)) + ((v4 + v5) + (v6 + v7)) of its group, the order of
 * an xor-1, 2, 4 butterfly */
__device__ __forceinline__ float group8_sum(float v)
{
    v += dpp8_f32<0xB1>(v);
    v += dpp8_f32<0x4E>(v);
    return v + dpp8_f32<0x141>(v);
}
__device__ __forceinline__ float group8_max(float v)
{
    v = fmaxf(v, dpp8_f32<0xB1>(v));
    v = fmaxf(v, dpp8_f32<0x4E>(v));
    return fmaxf(v, dpp8_f32<0x141>(v));
}

template <int MT, int ME, bool BUF>
__global__ __launch_bounds__(256) void router_partial_mfma_kernel(double *part, float *rbound,
                                                                  const float *x, int T,
                                                                  const float *W, int hidden,
                                                                  int n_experts, int chunk, int vec,
                                                                  int deal, int *ctr, int *idx_reset,
                                                                  int n_reset)
{
    /* the final kernel's arrival counter starts every launch at zero, and the idx it gathers
     * at -1 (its gathering workgroup waits for each entry to be set) */
    if (ctr && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0) {
        if (threadIdx.x == 0) *ctr = 0;
        for (int i = threadIdx.x; i < n_reset; i += blockDim.x) idx_reset[i] = -1;
    }
    typedef double d4 __attribute__((ext_vector_type(4)));
    constexpr int TB = 32 * MT, EB = 32 * ME;           /* workgroup tile: tokens, experts */
    constexpr int NWP = EB / 32, NXP = TB / 32;         /* float4 pieces per thread: W, x */
    __shared__ __attribute__((aligned(16))) float ws[2][EB * RM_LD];
    __shared__ __attribute__((aligned(16))) float xs[2][TB * RM_LD];
    __shared__ float wn[2][EB];                          /* sum |w| over the sub-block */
    __shared__ float xn[2][TB];                          /* max |x| over the sub-block */
    const int tid = threadIdx.x, l = tid & 63, wv = tid >> 6;
    const int wt = wv >> 1, we = wv & 1;                 /* the wave's block of the tile */
    /* A one-dimensional grid dealt to the XCDs (workgroup b runs on XCD b % 8), so that
     * each W and x piece is fetched into one XCD's L2 once instead of once per token tile /
     * expert tile:
     *   deal 1 (a chunk count that is a multiple of 8): the workgroups of one chunk run on
     *     one XCD;
     *   deal 2: the (chunk, token tile) pairs, chunk-major, in eight contiguous ranges, one
     *     per XCD; an XCD walks its pairs in order, the expert tiles of a pair one after
     *     another (they share the pair's x piece), the token tiles of a chunk one after
     *     another (they share the chunk's W pieces). */
    int bx = blockIdx.x, by = blockIdx.y, ks = blockIdx.z;
    if (deal) {
        const int nee = (n_experts + EB - 1) / EB, ntt = (T + TB - 1) / TB;
        const int nks = (hidden + chunk - 1) / chunk;
        const int i = blockIdx.x / K3_NXCD, xcd = blockIdx.x % K3_NXCD;
        if (deal == 1) {
            const int g = nee * ntt;
            ks = xcd + K3_NXCD * (i / g);
            if (ks >= nks) return;
            bx = (i % g) % nee;
            by = (i % g) / nee;
        } else {
            const int per = (nks * ntt + K3_NXCD - 1) / K3_NXCD, pi = i / nee;
            const int pr = xcd * per + pi;
            if (pi >= per || pr >= nks * ntt) return;
            ks = pr / ntt;
            by = pr % ntt;
            bx = i % nee;
        }
    }
    const int e0 = bx * EB, t0 = by * TB;
    const int kb0 = ks * chunk, kb1 = min(hidden, kb0 + chunk);
    const int nsub = (kb1 - kb0 + RP_KS - 1) / RP_KS;
    const float *Wt = W + (size_t)e0 * hidden, *xt = x + (size_t)t0 * hidden;
    float4 wst[2][NWP], xst[2][NXP];                    /* the ring: two sub-blocks */
    k3_rsrc rsw, rsx;
    if constexpr (BUF) {
        rsw = k3_make_rsrc(W, (uint32_t)((size_t)n_experts * hidden * 4));
        rsx = k3_make_rsrc(x, (uint32_t)((size_t)T * hidden * 4));
    }
    auto fetch = [&](const float *base, int rows_valid, int r, int k) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < rows_valid) {
            const float *src = base + (size_t)r * hidden + k;
            if (vec && k + 3 < kb1) v = *reinterpret_cast<const float4 *>(src);
            else {
                v.x = k < kb1 ? src[0] : 0.f;
                v.y = k + 1 < kb1 ? src[1] : 0.f;
                v.z = k + 2 < kb1 ? src[2] : 0.f;
                v.w = k + 3 < kb1 ? src[3] : 0.f;
            }
        }
        return v;
    };
    /* rows of a multiple of 4 floats: a piece is wholly inside or past kb1 */
    auto fetch_buf = [&](k3_rsrc rs, int row0, int rows_valid, int r, int k) {
        const bool in = r < rows_valid && k < kb1;
        const uint32_t off = in ? (uint32_t)(((size_t)(row0 + r) * hidden + k) * 4) : 0x80000000u;
        return __builtin_bit_cast(float4, k3_bload16(rs, off));
    };
    /* piece p = tid + 256 i: row p / 8, columns 4 (p % 8) .. + 3 */
    auto load = [&](int sc, auto slot) {
        constexpr int S = decltype(slot)::value;
        const int k0 = kb0 + sc * RP_KS + (tid & 7) * 4;
#pragma unroll
        for (int i = 0; i < NWP; i++)
            wst[S][i] = BUF ? fetch_buf(rsw, e0, n_experts - e0, (tid + 256 * i) >> 3, k0)
                            : fetch(Wt, n_experts - e0, (tid + 256 * i) >> 3, k0);
#pragma unroll
        for (int i = 0; i < NXP; i++)
            xst[S][i] = BUF ? fetch_buf(rsx, t0, T - t0, (tid + 256 * i) >> 3, k0)
                            : fetch(xt, T - t0, (tid + 256 * i) >> 3, k0);
    };
    auto store = [&](int buf, auto slot) {
        constexpr int S = decltype(slot)::value;
        const int c = (tid & 7) * 4;
#pragma unroll
        for (int i = 0; i < NWP; i++) {
            const int r = (tid + 256 * i) >> 3;
            *reinterpret_cast<float4 *>(&ws[buf][r * RM_LD + c]) = wst[S][i];
            const float a = group8_sum(fabsf(wst[S][i].x) + fabsf(wst[S][i].y) + fabsf(wst[S][i].z) +
                                       fabsf(wst[S][i].w));
            if ((tid & 7) == 0) wn[buf][r] = a;
        }
#pragma unroll
        for (int i = 0; i < NXP; i++) {
            const int r = (tid + 256 * i) >> 3;
            *reinterpret_cast<float4 *>(&xs[buf][r * RM_LD + c]) = xst[S][i];
            const float m = group8_max(fmaxf(fmaxf(fabsf(xst[S][i].x), fabsf(xst[S][i].y)),
                                             fmaxf(fabsf(xst[S][i].z), fabsf(xst[S][i].w))));
            if ((tid & 7) == 0) xn[buf][r] = m;
        }
    };
    using R0 = std::integral_constant<int, 0>;
    using R1 = std::integral_constant<int, 1>;

    const int q = l >> 4, r16 = l & 15;
    const int trow = wt * 16 * MT, erow = we * 16 * ME;  /* the wave's first token / expert */
    d4 acc[MT][ME];
    float rb[MT][ME][4];
#pragma unroll
    for (int a = 0; a < MT; a++)
#pragma unroll
        for (int b = 0; b < ME; b++) {
            acc[a][b] = d4{0.0, 0.0, 0.0, 0.0};
#pragma unroll
            for (int r = 0; r < 4; r++) rb[a][b][r] = 0.0f;
        }

    load(0, R0{});
    load(1, R1{});
    store(0, R0{});
    __syncthreads();
    /* sub-block sc: its ring slot (sc & 1) is free once it is in LDS, so sc + 2 loads into
     * it; then sc is multiplied out of LDS buffer sc & 1 and sc + 1 stored into the other */
    auto step = [&](int sc, auto slot) {
        constexpr int S = decltype(slot)::value;
        const int buf = S;
        load(sc + 2, slot);
        /* bound term of this sub-block from the chains' values at its start: element
         * (i, j) of block (a, b) is token trow + 16 a + 4 r + q, expert erow + 16 b + r16 */
        {
            float xr[MT][4], we_[ME];
#pragma unroll
            for (int a = 0; a < MT; a++)
#pragma unroll
                for (int r = 0; r < 4; r++) xr[a][r] = xn[buf][trow + 16 * a + 4 * r + q];
#pragma unroll
            for (int b = 0; b < ME; b++) we_[b] = wn[buf][erow + 16 * b + r16];
#pragma unroll
            for (int a = 0; a < MT; a++)
#pragma unroll
                for (int b = 0; b < ME; b++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        rb[a][b][r] = fmaf((float)RP_SUB, (float)fabs(acc[a][b][r]) + we_[b] * xr[a][r],
                                           rb[a][b][r]);
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float4 xa[MT], wb[ME];
#pragma unroll
            for (int a = 0; a < MT; a++)
                xa[a] = *reinterpret_cast<const float4 *>(&xs[buf][(trow + 16 * a + r16) * RM_LD + 8 * q + 4 * h]);
#pragma unroll
            for (int b = 0; b < ME; b++)
                wb[b] = *reinterpret_cast<const float4 *>(&ws[buf][(erow + 16 * b + r16) * RM_LD + 8 * q + 4 * h]);
#pragma unroll
            for (int s = 0; s < 4; s++) {
                double av[MT], bv[ME];
#pragma unroll
                for (int a = 0; a < MT; a++) av[a] = (double)(s == 0 ? xa[a].x : s == 1 ? xa[a].y : s == 2 ? xa[a].z : xa[a].w);
#pragma unroll
                for (int b = 0; b < ME; b++) bv[b] = (double)(s == 0 ? wb[b].x : s == 1 ? wb[b].y : s == 2 ? wb[b].z : wb[b].w);
#pragma unroll
                for (int a = 0; a < MT; a++)
#pragma unroll
                    for (int b = 0; b < ME; b++)
                        acc[a][b] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[a], bv[b], acc[a][b], 0, 0, 0);
            }
        }
        /* past the chunk the slot holds zeros (BUF) and the buffer is not read again */
        store(buf ^ 1, std::integral_constant<int, S ^ 1>{});
        __syncthreads();
    };
    /* whole pairs in the loop, so that no load or store sits under a branch there */
    int sc = 0;
    for (; sc + 1 < nsub; sc += 2) {
        step(sc, R0{});
        step(sc + 1, R1{});
    }
    if (sc < nsub) step(sc, R0{});
    /* relative error of the fp32 bound: (nsub + 4) roundings of 2^-24, the float sums of
     * |w| at most 2^-18 */
    const double up = 1.0 + 0x1p-17 + (double)(nsub + 4) * 0x1p-24;
#pragma unroll
    for (int a = 0; a < MT; a++)
#pragma unroll
        for (int b = 0; b < ME; b++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t = t0 + trow + 16 * a + 4 * r + q, e = e0 + erow + 16 * b + r16;
                if (e < n_experts && t < T) {
                    const size_t o = ((size_t)ks * T + t) * n_experts + e;
                    part[o] = acc[a][b][r];
                    rbound[o] = bound_up((double)rb[a][b][r], up);
                }
            }
}

/* The partials of a few tokens (T <= RS_T): one lane per (expert, chunk of RS_CH
 * columns) runs the chunk's chain for every token. The lane issues all of its W row
 * segment's loads at once (32 x 16 bytes) so that one memory latency covers the chunk;
 * the tokens' chunk is staged in LDS as fp64 (read as broadcasts) with the per-sub-block
 * maxima of |x|. The bound R_k per chain uses the lane's own sums of |w| over each
 * 32-column sub-block. */
constexpr int RS_T = 4, RS_CH = 128;

template <int NT>
__global__ __launch_bounds__(256) void router_partial_small_kernel(double *part, float *rbound,
                                                                   const float *x, int T,
                                                                   const float *W, int hidden,
                                                                   int n_experts, int vec)
{
    __shared__ double xsh[NT][RS_CH];
    __shared__ double xmx[NT][RS_CH / 32];
    const int ks = blockIdx.y;
    const int e = blockIdx.x * 256 + threadIdx.x;
    const int kb0 = ks * RS_CH, len = min(RS_CH, hidden - kb0);
    const float *wr = W + (size_t)min(e, n_experts - 1) * hidden + kb0;
    /* one token: the whole segment in registers, issued before the staging so that the
     * two latencies overlap; more tokens: one sub-block at a time */
    constexpr int WQ = NT == 1 ? RS_CH / 4 : 8;
    float4 wv[WQ];
    auto fetch = [&](int q0) {
#pragma unroll
        for (int q = 0; q < WQ; q++) {
            const int k = 4 * (q0 + q);
            if (vec && len == RS_CH) wv[q] = *reinterpret_cast<const float4 *>(wr + k);
            else
                wv[q] = make_float4(k < len ? wr[k] : 0.f, k + 1 < len ? wr[k + 1] : 0.f,
                                    k + 2 < len ? wr[k + 2] : 0.f, k + 3 < len ? wr[k + 3] : 0.f);
        }
    };
    if (NT == 1) fetch(0);
    /* stage the tokens' chunk; 32 consecutive threads reduce one sub-block's max |x| */
    for (int i0 = 0; i0 < NT * RS_CH; i0 += 256) {
        const int i = i0 + threadIdx.x;
        const int t = i / RS_CH, k = i % RS_CH;
        double v = 0.0;
        if (i < NT * RS_CH) {
            v = (t < T && k < len) ? (double)x[(size_t)t * hidden + kb0 + k] : 0.0;
            xsh[t][k] = v;
        }
        double m = fabs(v);
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) m = fmax(m, __shfl_xor(m, o, 64));
        if (i < NT * RS_CH && (k & 31) == 0) xmx[t][k >> 5] = m;
    }
    __syncthreads();
    if (e >= n_experts) return;
    double acc[NT], rb[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) { acc[t] = 0.0; rb[t] = 0.0; }
    auto subblock = [&](int sb, int qb) {
        float wn = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const float4 v = wv[qb + q];
            wn += fabsf(v.x) + fabsf(v.y) + fabsf(v.z) + fabsf(v.w);
        }
#pragma unroll
        for (int t = 0; t < NT; t++)
            rb[t] = fma(32.0, fabs(acc[t]) + (double)wn * xmx[t][sb], rb[t]);
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const float4 v = wv[qb + q];
            const int k = sb * 32 + 4 * q;
#pragma unroll
            for (int t = 0; t < NT; t++) {
                acc[t] = fma((double)v.x, xsh[t][k], acc[t]);
                acc[t] = fma((double)v.y, xsh[t][k + 1], acc[t]);
                acc[t] = fma((double)v.z, xsh[t][k + 2], acc[t]);
                acc[t] = fma((double)v.w, xsh[t][k + 3], acc[t]);
            }
        }
    };
    if (NT == 1) {
#pragma unroll
        for (int sb = 0; sb < RS_CH / 32; sb++) subblock(sb, sb * 8);
    } else {
#pragma unroll 1
        for (int sb = 0; sb < RS_CH / 32; sb++) {
            fetch(sb * 8);
            subblock(sb, 0);
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++)
        if (t < T) {
            const size_t o = ((size_t)ks * T + t) * n_experts + e;
            part[o] = acc[t];
            rbound[o] = bound_up(rb[t], 1.0 + 0x1p-17);
        }
}

/* The float next to finite f towards +inf (up) or -inf (down). */
__device__ __forceinline__ float next_float(float f, bool up)
{
    if (f == 0.0f) return up ? 0x1p-149f : -0x1p-149f;
    const uint32_t b = __float_as_uint(f);
    const bool away = (f > 0.0f) == up;                       /* magnitude grows */
    return __uint_as_float(away ? b + 1u : b - 1u);
}

/* Midpoints between f and its float neighbours; a double in (lo, hi) rounds to f. */
__device__ __forceinline__ void round_interval(float f, double &lo, double &hi)
{
    const float dn = next_float(f, false), up = next_float(f, true);
    lo = isinf(dn) ? -0x1.ffffffp+127 : 0.5 * ((double)f + (double)dn);
    hi = isinf(up) ? 0x1.ffffffp+127 : 0.5 * ((double)f + (double)up);
}

/* The certification of a logit from its chunk sums (S = Q, the sum of P_k in k order, and
 * bs, the sum of C_k |Q_k| + 2 R_k + |Q_{k+1}|): with u = 2^-53, B = 1.01 u bs + 4u|S|
 * bounds |S - a_n| (the reference's chain), so the logit (float)a_n is one of the floats
 * from (float)(S - B) to (float)(S + B) (rounding is monotone). The score is certain (ok)
 * when that range is one float, or two neighbouring floats whose scores are equal (the
 * choice, score + bias, is then certain too); otherwise scmax is the score of the largest
 * float the logit can be. Non-finite sums come from inf/NaN inputs and propagate alike in
 * any order (ok). fword = exc_word((float)Q, exc), loaded by the caller. */
struct Certified {
    float sc, scmax;
    bool ok;
};

__device__ __forceinline__ Certified certify_score(double Q, double bs, const ExcTable &exc,
                                                   uint32_t fword)
{
    const float f = (float)Q;
    Certified r;
    r.sc = router_score_w(f, fword, exc);
    r.scmax = r.sc;
    r.ok = true;
    if (fabs(Q) <= 0x1.fffffffffffffp+1023) {
        const double B = 1.01 * 0x1p-53 * bs + 4.0 * 0x1p-53 * fabs(Q) + 0x1p-1060;
        double mlo, mhi;
        round_interval(f, mlo, mhi);
        if (!((Q - B > mlo) && (Q + B < mhi))) {
            const float lo = (float)(Q - B), hi = (float)(Q + B);
            const bool finite = fabsf(lo) <= 0x1.fffffep+127f && fabsf(hi) <= 0x1.fffffep+127f;
            if (finite && (lo == hi || next_float(lo, true) == hi)) {
                const float slo = router_score(lo, exc), shi = router_score(hi, exc);
                if (slo == shi) {
                    r.sc = slo;
                    r.scmax = slo;
                } else {
                    r.ok = false;
                    r.scmax = fmaxf(slo, shi);
                }
            } else {
                r.ok = false;
                r.scmax = router_score(fabsf(hi) <= 0x1.fffffep+127f ? next_float(hi, true) : hi, exc);
            }
        }
    }
    return r;
}

/* Router logits of a few tokens (T <= RS_T, hidden <= 64 * RS_CH), certified and scored in
 * one kernel: a workgroup per expert, lane k of every wave owns 128-column chunk k, and wave
 * w its 32-column sub-block w.
 * - Loads cover full 128-byte lines: lane l loads columns 4(l % 8).. of sub-block w of chunks
 *   l / 8 + 8j (j < 8), for W and for each token, and the wave's LDS buffer turns that into
 *   one sub-block per lane (a chunk's 16-byte group q at group (q + k) mod 8, so the lanes'
 *   16-byte reads fall on distinct banks). Every load is a buffer load with no branch
 *   around it (past the end, or a masked offset, reads 0), all issued at once.
 * - A chunk's value: each of its four sub-blocks is a chain of its own from 0 (one per wave
 *   and token), then J = ((c0 + c1) + c2) + c3. Its rounded intermediates are the chains'
 *   partial sums, each at most ||w||_1 ||x||_inf of the sub-block (times 1 + 32u), and the
 *   joins, each at most |J before it| + that norm; the reference's own partial sums over
 *   the chunk are bounded alike. So R_k = sum over sub-blocks of 34 (|J before it| +
 *   ||w||_1 ||x||_inf) bounds both uses of R_k in the certification (34 >= 33 (1 + 32u) for
 *   the rounded terms, >= 32 for the reference's).
 * - Wave t then finishes token t: lane k joins chunk k; every lane runs the chunks' sum in
 *   k order (Q_{k+1} = Q_k + P_k, the rounding the bound describes) on broadcast LDS reads
 *   and keeps its own Q_k, Q_{k+1}; lane k forms C_k |Q_k| + 2 R_k + |Q_{k+1}|, the wave
 *   adds those (any order: bs only bounds); lane 0 certifies (certify_score), its
 *   exception-bitmap word requested before the ordered sum for the sum in any order (the
 *   two round to the same float but for rare ties, which load it again), and stores pre[t][e] =
 *   {score, score of the upper end, uncertified ? 1 : 0, 0}. */
template <bool VEC>
__device__ __forceinline__ float4 rs_load4(k3_rsrc r, uint32_t col)
{
    if (VEC) return __builtin_bit_cast(float4, k3_bload16(r, 4u * col));
    return make_float4(__uint_as_float(k3_bload4(r, 4u * col)), __uint_as_float(k3_bload4(r, 4u * col + 4u)),
                       __uint_as_float(k3_bload4(r, 4u * col + 8u)), __uint_as_float(k3_bload4(r, 4u * col + 12u)));
}

/* a + (a of the lane DPP control CTRL names; 0 in rows outside RM) */
template <int CTRL, int RM>
__device__ __forceinline__ double dpp_add_f64(double a)
{
    const uint64_t b = __builtin_bit_cast(uint64_t, a);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, RM, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, RM, 0xf, false);
    return a + __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

/* Sum of a double over the wave by DPP, returned in every lane: pairs, quads, row halves,
 * rows, then rows 0-1 / 2-3 (row_bcast15) and 0-3 (row_bcast31) into lane 63. */
__device__ __forceinline__ double wave_sum_f64(double v)
{
    v = dpp_add_f64<0xB1, 0xf>(v);      /* quad_perm [1,0,3,2] */
    v = dpp_add_f64<0x4E, 0xf>(v);      /* quad_perm [2,3,0,1] */
    v = dpp_add_f64<0x141, 0xf>(v);     /* row_half_mirror */
    v = dpp_add_f64<0x140, 0xf>(v);     /* row_mirror */
    v = dpp_add_f64<0x142, 0xa>(v);     /* row_bcast15 */
    v = dpp_add_f64<0x143, 0xc>(v);     /* row_bcast31 */
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), 63);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

template <int NT, bool VEC>
__global__ __launch_bounds__(256) void router_small_kernel(float4 *pre, const float *x, int T,
                                                           const float *W, int hidden,
                                                           int n_experts, ExcTable exc)
{
    __shared__ __attribute__((aligned(16))) float tr[4][64 * 32];  /* per wave: 64 chunks x 32 */
    __shared__ __attribute__((aligned(16))) double csh[NT][4][64];  /* chain value per sub-block */
    __shared__ float xmsh[NT][4][64];                               /* ||x||_inf per sub-block */
    __shared__ float wnsh[4][64];                                   /* ||w||_1 per sub-block */
    __shared__ __attribute__((aligned(16))) double jsh[NT][64];     /* chunk values P_k */
    const int tid = threadIdx.x, lane = tid & 63, sb = tid >> 6;
    const int e = blockIdx.x;
    const int ks = (hidden + RS_CH - 1) / RS_CH;
    const k3_rsrc wr = k3_make_rsrc(W + (size_t)e * hidden, 4u * (uint32_t)hidden);
    const k3_rsrc xr = k3_make_rsrc(x, 4u * (uint32_t)(T * hidden));
    /* loads j: chunk l / 8 + 8j, columns 4(l % 8)..4(l % 8) + 3 of sub-block sb */
    const int lq = lane & 7, lk = lane >> 3;
    float4 wl[8], xl[NT][8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int col = (lk + 8 * j) * RS_CH + sb * 32 + 4 * lq;
        wl[j] = rs_load4<VEC>(wr, (uint32_t)col);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            /* token t's columns col.. (zero past the row or past T: an offset past the end) */
            const uint32_t o = (uint32_t)(t * hidden + col);
            if (VEC) {
                xl[t][j] = __builtin_bit_cast(float4, k3_bload16(xr, t < T && col < hidden ? 4u * o : 0xfffffff0u));
            } else {
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; i++)
                    v[i] = __uint_as_float(k3_bload4(xr, t < T && col + i < hidden ? 4u * (o + i) : 0xfffffff0u));
                xl[t][j] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    }
    /* through the wave's buffer: a row of 32 per chunk, group q of chunk k at (q + k) mod 8 */
    float *wb = tr[sb];
    auto transpose = [&](const float4 (&in)[8], float4 (&out)[8]) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int k = lk + 8 * j;
            *reinterpret_cast<float4 *>(&wb[k * 32 + 4 * ((lq + k) & 7)]) = in[j];
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int q = 0; q < 8; q++) out[q] = *reinterpret_cast<const float4 *>(&wb[lane * 32 + 4 * ((q + lane) & 7)]);
        __builtin_amdgcn_wave_barrier();
    };
    float4 wq[8];
    transpose(wl, wq);
    {
        /* ||w||_1 as a pairwise sum: relative error under 2^-21 */
        float s4[8];
#pragma unroll
        for (int q = 0; q < 8; q++) s4[q] = (fabsf(wq[q].x) + fabsf(wq[q].y)) + (fabsf(wq[q].z) + fabsf(wq[q].w));
        wnsh[sb][lane] = ((s4[0] + s4[1]) + (s4[2] + s4[3])) + ((s4[4] + s4[5]) + (s4[6] + s4[7]));
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        if (t >= T) break;
        float4 xq[8];
        transpose(xl[t], xq);
        float m[8];
#pragma unroll
        for (int q = 0; q < 8; q++)
            m[q] = fmaxf(fmaxf(fabsf(xq[q].x), fabsf(xq[q].y)), fmaxf(fabsf(xq[q].z), fabsf(xq[q].w)));
        xmsh[t][sb][lane] = fmaxf(fmaxf(fmaxf(m[0], m[1]), fmaxf(m[2], m[3])), fmaxf(fmaxf(m[4], m[5]), fmaxf(m[6], m[7])));
        double a = 0.0;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            a = fma((double)wq[q].x, (double)xq[q].x, a);
            a = fma((double)wq[q].y, (double)xq[q].y, a);
            a = fma((double)wq[q].z, (double)xq[q].z, a);
            a = fma((double)wq[q].w, (double)xq[q].w, a);
        }
        csh[t][sb][lane] = a;
    }
    __syncthreads();
    const int t = sb;                               /* wave t finishes token t */
    if (t >= T) return;
    /* lane k: chunk k's value and R_k (lanes past the last chunk hold zeros) */
    double J = csh[t][0][lane];
    double rb = 34.0 * ((double)wnsh[0][lane] * (double)xmsh[t][0][lane]);
#pragma unroll
    for (int s = 1; s < 4; s++) {
        rb = fma(34.0, fabs(J) + (double)wnsh[s][lane] * (double)xmsh[t][s][lane], rb);
        J += csh[t][s][lane];
    }
    /* rounded up: the float sums of |w| carry at most a 2^-18 relative error */
    const double R = (double)bound_up(rb, 1.0 + 0x1p-17);
    jsh[t][lane] = J;
    /* the exception-bitmap word of the sum in any order, requested now: the ordered sum
     * below rounds to the same float (same bits) but for rare ties, which load it again */
    const double Sa = wave_sum_f64(J);
    const uint32_t fwa = exc_word((float)Sa, exc);
    __builtin_amdgcn_wave_barrier();
    /* the sum in k order in every lane (broadcast reads); lane k keeps Q_k and Q_{k+1} */
    double pk[64];
#pragma unroll
    for (int k = 0; k < 64; k += 2) {
        const double2 v = *reinterpret_cast<const double2 *>(&jsh[t][k]);
        pk[k] = v.x;
        pk[k + 1] = v.y;
    }
    double q = 0.0, q0 = 0.0, q1 = 0.0;
#pragma unroll
    for (int k = 0; k < 64; k++) {
        if (k == lane) q0 = q;
        if (k < ks) q += pk[k];
        if (k == lane) q1 = q;
    }
    const double S = q;
    const uint32_t fw = __float_as_uint((float)S) == __float_as_uint((float)Sa) ? fwa : exc_word((float)S, exc);
    const double ck = (double)min(RS_CH, hidden - min(lane, ks - 1) * RS_CH);
    const double term = lane < ks ? fma(ck, fabs(q0), fma(2.0, R, fabs(q1))) : 0.0;
    const double bs = wave_sum_f64(term);
    if (lane == 0) {
        const Certified cs = certify_score(S, bs, exc, fw);
        pre[(size_t)t * n_experts + e] = make_float4(cs.sc, cs.scmax, cs.ok ? 0.0f : 1.0f, 0.0f);
    }
}

/* router_final_kernel: up to RF_MAXE experts, RF_MAXW waves; RF_KB chunk partials per load batch. */
constexpr int RF_MAXE = 2048, RF_MAXW = 16, RF_KB = 32;

/* The expert-major gather's operands (gather_block). ctr: the arrival counter of the
 * router's final kernel when that kernel runs the gather itself. */
struct GatherDev {
    int *offsets, *perm, *job_expert, *job_off, *job_cnt, *pass_job, *pass_tp, *pass_job2, *pass_tp2;
    int *counts;
    const int *idx;
    const void *bank;
    int N, n_experts, pass_tok, pass_tok2;
    int *ctr;
};
template <bool COH>
__device__ void gather_block(const GatherDev &g);

/* One workgroup per token: every thread certifies and scores SL experts (tid + nthr i) --
 * from router_small_kernel's scored records (PRE) or from the chunk partials, summed in
 * k order and certified here (certify_score) -- into LDS; then select_rounds (wave 0
 * selects, the workgroup recomputes what matters) and select_weight; renormalise and
 * scale (k3_ops.c:459-475). nrecomp[t] (optional) counts recomputes. KB: chunk partials
 * loaded per batch. */
template <int SL, int SW, int KB, bool PRE, bool GATHER = false>
__global__ __launch_bounds__(KB > 32 ? 512 : 1024) void router_final_kernel(int *idx, float *wt, int *nrecomp,
                                                            const double *part,
                                                            const float *rbound, int ksplit,
                                                            int chunk, const float *x,
                                                            const float *W, const float *bias,
                                                            int T, int hidden, int n_experts,
                                                            int topk, int renorm,
                                                            float routed_scale, ExcTable exc,
                                                            GatherDev g)
{
    __shared__ SelSmem<SW> sm;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nthr = blockDim.x;
    const int t = blockIdx.x;
#pragma unroll
    for (int i = 0; i < SL; i++) {
        const int e = tid + nthr * i;
        if (e >= 64 * SW) break;
        if (e >= n_experts) {
            select_put_record(sm, e, make_float4(0.f, 0.f, 0.f, 0.f), -INFINITY);
        } else if (PRE) {
            /* scored by router_small_kernel */
            select_put_record(sm, e, reinterpret_cast<const float4 *>(part)[(size_t)t * n_experts + e],
                              bias ? bias[e] : 0.0f);
        } else {
            double Q = 0.0, bs = 0.0;
            for (int k0 = 0; k0 < ksplit; k0 += KB) {
                /* one batch of chunk loads in flight together */
                double pv[KB];
                float rv[KB];
#pragma unroll
                for (int kk = 0; kk < KB; kk++) {
                    const int k = min(k0 + kk, ksplit - 1);
                    const size_t o = ((size_t)k * T + t) * n_experts + e;
                    pv[kk] = part[o];
                    rv[kk] = rbound[o];
                }
#pragma unroll
                for (int kk = 0; kk < KB; kk++) {
                    const int k = k0 + kk;
                    if (k < ksplit) {
                        const int ck = min(chunk, hidden - k * chunk);
                        bs += (double)ck * fabs(Q) + 2.0 * (double)rv[kk];
                        Q += pv[kk];
                        bs += fabs(Q);
                    }
                }
            }
            const Certified cs = certify_score(Q, bs, exc, exc_word((float)Q, exc));
            select_put_record(sm, e, make_float4(cs.sc, cs.scmax, cs.ok ? 0.0f : 1.0f, 0.0f),
                              bias ? bias[e] : 0.0f);
        }
    }
    __syncthreads();
    int nre;
    const uint64_t mysel = select_rounds<SW>(sm, x + (size_t)t * hidden, W, bias, hidden, n_experts, topk, exc, nre);
    if (wv == 0) {
        int id;
        float w;
        select_weight<SW>(sm, mysel, topk, renorm, routed_scale, id, w);
        if (lane < topk) {
            if (GATHER)   /* written through to where every XCD's gather reads it */
                __hip_atomic_store(idx + (size_t)t * topk + lane, id >= 0 ? id : 0, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            else
                idx[(size_t)t * topk + lane] = id >= 0 ? id : 0;
            wt[(size_t)t * topk + lane] = w;
        }
        if (nrecomp && lane == 0) nrecomp[t] = nre;
    }
    if constexpr (GATHER) {
        /* The workgroup that finishes last runs the gather over every token's idx. Each
         * workgroup's idx stores (agent-scope atomics, written through to where every XCD
         * reads) are acknowledged (vmcnt 0) before it counts itself in on an agent-scope
         * counter. The partial kernel, a launch earlier on the stream, set every idx to -1
         * and the counter to zero, so those stores happen-before this launch: an agent-scope
         * load of an idx returns -1 or this launch's value, and the gather reads each until
         * it is set (in practice at once: the stores were acknowledged before the count). No
         * release fence (an L2 write-back) is needed. The last workgroup leaves the counter
         * at zero. */
        __shared__ int s_last;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0)
            s_last = __hip_atomic_fetch_add(g.ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     (int)gridDim.x - 1;
        __syncthreads();
        if (s_last) {
            gather_block<true>(g);
            if (tid == 0) __hip_atomic_store(g.ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

/* ---- expert-major gather -----------------------------------------------------------
 * One workgroup of 1024 threads. Counting sort by expert, stable in assignment order.
 * Counts by LDS atomics; the scans of (count, jobs, passes) over experts by wave shuffles
 * plus one pass over the 16 wave totals. Placement in chunks of 1024 assignments: each
 * wave ranks its lanes among equal experts with ballots; up to 1024 experts, per-wave
 * expert counts (16-bit, in LDS) give every lane the count of its expert in earlier
 * waves, so a chunk costs three barriers; past 1024 experts the waves commit one after
 * another. */
constexpr int G_MAXE = 4096, G_WCNT_E = 1024;

/* inclusive scan over a wave, then over the workgroup's 16 wave totals */
/* Exclusive scans of NV values at once over a 1024-thread workgroup (one pair of barriers
 * for all of them): x[i] becomes the sum of v[i] over the lower threads, tot[i] the total. */
template <int NV>
__device__ __forceinline__ void block_scan_excl_n(int (&x)[NV], int (*wtotn)[NV], int lane, int wv,
                                                  int (&tot)[NV])
{
    int v[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) v[i] = x[i];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1)
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int y = __shfl_up(x[i], o, 64);
            if (lane >= o) x[i] += y;
        }
    if (lane == 63)
#pragma unroll
        for (int i = 0; i < NV; i++) wtotn[wv][i] = x[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NV; i++) {
        int base = 0;
        tot[i] = 0;
        for (int w = 0; w < 16; w++) {
            const int tw = wtotn[w][i];
            if (w < wv) base += tw;
            tot[i] += tw;
        }
        x[i] = base + x[i] - v[i];
    }
    __syncthreads();
}

/* From per-expert counts cnt[] (LDS): offsets[], fill[] (= offsets, in LDS), the jobs,
 * the passes and counts[0..3], as the gather's header describes. With pass_tok2 > 0 the
 * experts holding more than pass_tok assignments get passes of pass_tok2 in the second
 * list instead. Called by all 1024 threads; ends with a barrier. */
__device__ void gather_plan(const int *cnt, int *fill, int (*wtot5)[5], int *offsets, int *job_expert,
                            int *job_off, int *job_cnt, int *pass_job, int *pass_tp,
                            int *pass_job2, int *pass_tp2, int *counts, int n_experts,
                            const unsigned char *pres, int pass_tok, int pass_tok2)
{
    auto big = [&](int c) { return pass_tok2 > 0 && c > pass_tok; };
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    /* per-thread sums over a contiguous expert range, then workgroup scans */
    const int per = (n_experts + 1023) / 1024;
    const int ea = tid * per, eb = min(n_experts, ea + per);
    int local = 0, ljobs = 0, lpass = 0, lpass2 = 0, ldrop = 0;
    for (int e = ea; e < eb; e++) {
        local += cnt[e];
        if (cnt[e] > 0) {
            if (pres[e]) {
                ljobs++;
                if (big(cnt[e])) lpass2 += (cnt[e] + pass_tok2 - 1) / pass_tok2;
                else lpass += (cnt[e] + pass_tok - 1) / pass_tok;
            } else {
                ldrop += cnt[e];
            }
        }
    }
    int sv[5] = {local, ljobs, lpass, lpass2, ldrop}, tot[5];
    block_scan_excl_n<5>(sv, wtot5, lane, wv, tot);
    int run = sv[0], jrun = sv[1], prun = sv[2], prun2 = sv[3];
    const int tot_a = tot[0], tot_b = tot[1], tot_c = tot[2], tot_e = tot[3], tot_d = tot[4];
    for (int e = ea; e < eb; e++) {
        offsets[e] = run;
        fill[e] = run;
        if (cnt[e] > 0 && pres[e]) {
            job_expert[jrun] = e;
            job_off[jrun] = run;
            job_cnt[jrun] = cnt[e];
            if (big(cnt[e])) {
                const int np = (cnt[e] + pass_tok2 - 1) / pass_tok2;
                for (int p = 0; p < np; p++) {
                    pass_job2[prun2 + p] = jrun;
                    pass_tp2[prun2 + p] = p;
                }
                prun2 += np;
            } else {
                const int np = (cnt[e] + pass_tok - 1) / pass_tok;
                for (int p = 0; p < np; p++) {
                    pass_job[prun + p] = jrun;
                    pass_tp[prun + p] = p;
                }
                prun += np;
            }
            jrun++;
        }
        run += cnt[e];
    }
    if (tid == 0) {
        offsets[n_experts] = tot_a;
        counts[0] = tot_b;
        counts[1] = tot_c;
        counts[2] = tot_d;
        counts[3] = tot_e;
    }
    if (tid >= 4 && tid < 4 + K3K_QUEUE_INTS) counts[tid] = 0;    /* the work-item counters */
    __syncthreads();
}

/* The one-workgroup gather (1024 threads); COH: idx was written during this launch by other
 * workgroups (agent-scope stores) over the -1 the previous launch left, so it is read with
 * agent-scope loads, each until it is set. */
template <bool COH>
__device__ void gather_block(const GatherDev &g)
{
    int *offsets = g.offsets, *perm = g.perm;
    const int N = g.N, n_experts = g.n_experts;
    auto idx_at = [&](int a) {
        if (!COH) return g.idx[a];
        int v = __hip_atomic_load(const_cast<int *>(g.idx) + a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        /* -1 until this launch's store is visible (bounded: a value never stored reads as no
         * expert after about 2^20 polls) */
        for (int spin = 0; v < 0 && spin < (1 << 20); spin++) {
            __builtin_amdgcn_s_sleep(1);
            v = __hip_atomic_load(const_cast<int *>(g.idx) + a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return v;
    };
    __shared__ int cnt[G_MAXE];
    __shared__ int fill[G_MAXE];
    __shared__ int wtot5[16][5];
    __shared__ unsigned char pres[G_MAXE];
    __shared__ unsigned short wcnt[16][G_WCNT_E];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    /* A thread's first two assignments' experts are loaded once, together with the bank
     * entries' presence, and serve both the counting and the placement (a batch of more
     * than 2048 assignments reads the rest again where it needs them). */
    const int ev0 = tid < N ? idx_at(tid) : -1;
    const int ev1 = tid + 1024 < N ? idx_at(tid + 1024) : -1;
    for (int e = tid; e < n_experts; e += 1024) {
        cnt[e] = 0;
        pres[e] = expert_present(g.bank, e) ? 1 : 0;
    }
    __syncthreads();
    for (int a = tid; a < N; a += 1024) {
        const int e = a == tid ? ev0 : a == tid + 1024 ? ev1 : idx_at(a);
        if (e >= 0 && e < n_experts) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    gather_plan(cnt, fill, wtot5, offsets, g.job_expert, g.job_off, g.job_cnt, g.pass_job, g.pass_tp,
                g.pass_job2, g.pass_tp2, g.counts, n_experts, pres, g.pass_tok, g.pass_tok2);

    /* stable placement */
    const bool wide = n_experts > G_WCNT_E;
    for (int c0 = 0; c0 < N; c0 += 1024) {
        const int a = c0 + tid;
        const int e = c0 == 0 ? ev0 : c0 == 1024 ? ev1 : a < N ? idx_at(a) : -1;
        const bool ok = e >= 0 && e < n_experts;
        /* rank among earlier lanes of this wave with the same expert */
        uint64_t pending = __ballot(ok);
        int rank = 0;
        uint64_t mine = 0;
        while (pending) {
            const int leader = __ffsll((unsigned long long)pending) - 1;
            const int el = __shfl(e, leader, 64);
            const uint64_t m = __ballot(ok && e == el);
            if (ok && e == el) {
                mine = m;
                rank = __popcll(m & ((1ull << lane) - 1ull));
            }
            pending &= ~m;
        }
        const int m = __popcll(mine);
        if (!wide) {
            for (int i = tid; i < 16 * n_experts; i += 1024) wcnt[i / n_experts][i % n_experts] = 0;
            __syncthreads();
            if (ok && rank == 0) wcnt[wv][e] = (unsigned short)m;
            __syncthreads();
            if (ok) {
                int base = fill[e];
                for (int w = 0; w < wv; w++) base += wcnt[w][e];
                perm[base + rank] = a;
            }
            __syncthreads();
            for (int x = tid; x < n_experts; x += 1024) {
                int add = 0;
                for (int w = 0; w < 16; w++) add += wcnt[w][x];
                fill[x] += add;
            }
            __syncthreads();
        } else {
            for (int w = 0; w < 16; w++) {
                if (wv == w && ok) perm[fill[e] + rank] = a;
                __syncthreads();
                if (wv == w && ok && rank == m - 1) fill[e] += m;
                __syncthreads();
            }
        }
    }
}

__global__ __launch_bounds__(1024) void gather_kernel(GatherDev g)
{
    gather_block<false>(g);
}

/* The same gather over many workgroups, for large batches (more than GM_MIN assignments,
 * at most G_WCNT_E experts): chunks of GM_C assignments.
 *  1. gather_hist_kernel: chunk c's count of expert e -> hist[c * n_experts + e].
 *  2. gather_scan_kernel (one workgroup): per-expert totals, then gather_plan; hist becomes
 *     the position in perm of chunk c's first assignment of expert e.
 *  3. gather_place_kernel: each chunk ranks its assignments stably (ballots inside a wave,
 *     per-wave counts across waves) from those positions.
 * perm comes out identical to the one-workgroup kernel's. */
constexpr int GM_C = 512, GM_MIN = 2048;

__global__ __launch_bounds__(GM_C) void gather_hist_kernel(int *hist, const int *idx, int N,
                                                           int n_experts, int nchunk)
{
    __shared__ int cnt[G_WCNT_E];
    const int c = blockIdx.x, tid = threadIdx.x;
    for (int e = tid; e < n_experts; e += GM_C) cnt[e] = 0;
    __syncthreads();
    const int a = c * GM_C + tid;
    if (a < N) {
        const int e = idx[a];
        if (e >= 0 && e < n_experts) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    for (int e = tid; e < n_experts; e += GM_C) hist[(size_t)c * n_experts + e] = cnt[e];
}

__global__ __launch_bounds__(1024) void gather_scan_kernel(int *hist, int *offsets, int *job_expert,
                                                           int *job_off, int *job_cnt, int *pass_job,
                                                           int *pass_tp, int *pass_job2,
                                                           int *pass_tp2, int *counts, int n_experts,
                                                           int nchunk, const void *bank, int pass_tok,
                                                           int pass_tok2)
{
    __shared__ int cnt[G_WCNT_E];
    __shared__ int fill[G_WCNT_E];
    __shared__ int wtot5[16][5];
    __shared__ unsigned char pres[G_WCNT_E];
    const int tid = threadIdx.x;
    /* a thread per expert; its chunk counts are a strided column (coalesced across the
     * threads), read 16 at a time so that the loads overlap */
    for (int e = tid; e < n_experts; e += 1024) {
        const bool pr = expert_present(bank, e);
        int t = 0;
#pragma unroll 16
        for (int c = 0; c < nchunk; c++) t += hist[(size_t)c * n_experts + e];
        cnt[e] = t;
        pres[e] = pr ? 1 : 0;
    }
    __syncthreads();
    gather_plan(cnt, fill, wtot5, offsets, job_expert, job_off, job_cnt, pass_job, pass_tp,
                pass_job2, pass_tp2, counts, n_experts, pres, pass_tok, pass_tok2);
    for (int e = tid; e < n_experts; e += 1024) {
        int run = fill[e];
#pragma unroll 16
        for (int c = 0; c < nchunk; c++) {
            const int v = hist[(size_t)c * n_experts + e];
            hist[(size_t)c * n_experts + e] = run;
            run += v;
        }
    }
}

__global__ __launch_bounds__(GM_C) void gather_place_kernel(int *perm, const int *hist,
                                                            const int *idx, int N, int n_experts,
                                                            int nchunk)
{
    constexpr int NWV = GM_C / 64;
    __shared__ unsigned short wcnt[NWV][G_WCNT_E];
    const int c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    for (int i = tid; i < NWV * n_experts; i += GM_C) wcnt[i / n_experts][i % n_experts] = 0;
    const int a = c * GM_C + tid;
    const int e = a < N ? idx[a] : -1;
    const bool ok = e >= 0 && e < n_experts;
    /* rank among earlier lanes of this wave with the same expert */
    uint64_t pending = __ballot(ok);
    int rank = 0;
    uint64_t mine = 0;
    while (pending) {
        const int leader = __ffsll((unsigned long long)pending) - 1;
        const int el = __shfl(e, leader, 64);
        const uint64_t m = __ballot(ok && e == el);
        if (ok && e == el) {
            mine = m;
            rank = __popcll(m & ((1ull << lane) - 1ull));
        }
        pending &= ~m;
    }
    __syncthreads();
    if (ok && rank == 0) wcnt[wv][e] = (unsigned short)__popcll(mine);
    __syncthreads();
    if (ok) {
        int base = hist[(size_t)c * n_experts + e];
        for (int w = 0; w < wv; w++) base += wcnt[w][e];
        perm[base + rank] = a;
    }
}

/* ---- combine: out[t] = 0 + sum_j wt[t][j] * contrib[t*topk + j], j ascending -------
 * A slot contributes nothing when its expert index is out of range or its bank entry is
 * absent. Every slot's row is loaded (it is valid memory either way) and the sum selects,
 * so that all topk loads are in flight together; the first JB slots' rows are loaded
 * before the slots' validity (idx, then the bank entry) is known, so the two chains of
 * loads overlap. */
template <bool VEC>
__global__ __launch_bounds__(256) void combine_kernel(float *out, const float *contrib,
                                                     const float *wt, const int *idx,
                                                     const void *bank, int n_experts, int T,
                                                     int topk, int E)
{
    constexpr int JB = 8;
    __shared__ float wsl[K3_MAX_TOPK_DEV];
    __shared__ int vsl[K3_MAX_TOPK_DEV];
    const int t = blockIdx.y;
    const int i = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    const bool active = i < E;
    const float *c0 = contrib + (size_t)t * topk * E + (active ? i : 0);
    float cv[JB][4];
    auto load = [&](int j0) {
#pragma unroll
        for (int jj = 0; jj < JB; jj++) {
            const int j = min(j0 + jj, topk - 1);
            const float *c = c0 + (size_t)j * E;
            if (VEC) {
                /* unconditional: c0 points at column 0 for threads past the row; the rows are
                 * read once (non-temporal) */
                const k3_f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const k3_f32x4 *>(c));
                cv[jj][0] = v[0]; cv[jj][1] = v[1]; cv[jj][2] = v[2]; cv[jj][3] = v[3];
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++) cv[jj][q] = i + q < E ? c[q] : 0.0f;
            }
        }
    };
    /* the slot's expert and weight first, then the rows, then the bank entry */
    int e = -1;
    float ws = 0.0f;
    if (threadIdx.x < topk) {
        e = idx[t * topk + threadIdx.x];
        ws = wt[t * topk + threadIdx.x];
    }
    load(0);
    if (threadIdx.x < topk) {
        vsl[threadIdx.x] = e >= 0 && e < n_experts && (!bank || expert_present(bank, e));
        wsl[threadIdx.x] = ws;
    }
    __syncthreads();
    if (!active) return;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j0 = 0; j0 < topk; j0 += JB) {
        if (j0 > 0) load(j0);
#pragma unroll
        for (int jj = 0; jj < JB; jj++) {
            const int j = j0 + jj;
            if (j < topk && vsl[j]) {
                const float w = wsl[j];
#pragma unroll
                for (int q = 0; q < 4; q++) acc[q] = __fadd_rn(acc[q], __fmul_rn(w, cv[jj][q]));
            }
        }
    }
    float *o = out + (size_t)t * E + i;
    if (VEC) *reinterpret_cast<float4 *>(o) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    else
        for (int q = 0; q < 4; q++)
            if (i + q < E) o[q] = acc[q];
}

/* ---- elementwise --------------------------------------------------------------------- */
__global__ void act_split_kernel(uint16_t *hi, uint16_t *lo, const float *gu, int n, int rows, int act,
                                 float b1, float b2)
{
    const size_t total = (size_t)n * rows;
    for (size_t k = (size_t)blockIdx.x * blockDim.x + threadIdx.x; k < total;
         k += (size_t)gridDim.x * blockDim.x) {
        const size_t r = k / n, i = k % n;
        const float *x = gu + r * 2 * (size_t)n;
        uint16_t h, l;
        k3_split2(k3_act_pair(x[i], x[n + i], act, b1, b2), h, l);
        hi[k] = h;
        if (lo) lo[k] = l;
    }
}

__global__ void act_kernel(float *y, const float *gu, int n, int rows, int act, float b1, float b2)
{
    const size_t total = (size_t)n * rows;
    for (size_t k = (size_t)blockIdx.x * blockDim.x + threadIdx.x; k < total;
         k += (size_t)gridDim.x * blockDim.x) {
        const size_t r = k / n, i = k % n;
        const float *x = gu + r * 2 * (size_t)n;
        y[k] = k3_act_pair(x[i], x[n + i], act, b1, b2);
    }
}

/* k3_ops.c:94-102: fp64 sum of squares, inv = (float)(1/sqrt(ss/n + eps)),
 * y = (w * x) * inv. One workgroup per row. */
__global__ __launch_bounds__(256) void rmsnorm_kernel(float *y, const float *x, const float *w,
                                                      int n, float eps)
{
    __shared__ double part[256];
    const float *xr = x + (size_t)blockIdx.x * n;
    float *yr = y + (size_t)blockIdx.x * n;
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) ss = fma((double)xr[i], (double)xr[i], ss);
    part[threadIdx.x] = ss;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) part[threadIdx.x] += part[threadIdx.x + s];
        __syncthreads();
    }
    const float inv = (float)(1.0 / sqrt(part[0] / (double)n + (double)eps));
    for (int i = threadIdx.x; i < n; i += 256) yr[i] = __fmul_rn(__fmul_rn(w[i], xr[i]), inv);
}

/* The same for rows of at most 256 EPT elements: each thread loads its EPT elements (and
 * weights) once into registers, the fp64 squares are summed per thread, across the wave by
 * butterfly and across the four waves in order, then the row is written from the registers.
 * A short row is one load latency and one barrier instead of a loop and a barrier tree. */
template <int EPT>
__global__ __launch_bounds__(256) void rmsnorm_reg_kernel(float *y, const float *x, const float *w,
                                                          int n, float eps)
{
    __shared__ double wsum[4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float *xr = x + (size_t)blockIdx.x * n;
    float *yr = y + (size_t)blockIdx.x * n;
    float xv[EPT], wvv[EPT];
#pragma unroll
    for (int k = 0; k < EPT; k++) {
        const int i = tid + 256 * k;
        xv[k] = i < n ? xr[i] : 0.0f;
        wvv[k] = i < n ? w[i] : 0.0f;
    }
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < EPT; k++) ss = fma((double)xv[k], (double)xv[k], ss);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if (lane == 0) wsum[wv] = ss;
    __syncthreads();
    const double tot = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    const float inv = (float)(1.0 / sqrt(tot / (double)n + (double)eps));
#pragma unroll
    for (int k = 0; k < EPT; k++) {
        const int i = tid + 256 * k;
        if (i < n) yr[i] = __fmul_rn(__fmul_rn(wvv[k], xv[k]), inv);
    }
}

__global__ void axpy_kernel(float *out, const float *add, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = __fadd_rn(out[i], add[i]);
}

__global__ void scale_kernel(float *out, const float *in, float s, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = __fmul_rn(in[i], s);
}

unsigned grid1d(size_t n, unsigned bs)
{
    size_t b = (n + bs - 1) / bs;
    if (b < 1) b = 1;
    if (b > 8192) b = 8192;
    return (unsigned)b;
}

}  // namespace

extern "C" int k3k_split_bf16(uint16_t *hi, uint16_t *lo, const float *x, size_t n, void *stream)
{
    if (!n) return 0;
    const bool v4 = n % 4 == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)hi % 8) == 0 &&
                    ((uintptr_t)lo % 8) == 0;
    if (v4)
        /* SPLIT_U float4s per thread from 2^21 float4s on (4096 x 7168: 73 -> 62 us); below
         * that one per thread, the grid's full width (512 x 7168: 7.0 against 7.9 us) */
        hipLaunchKernelGGL(split4_kernel,
                           dim3(n / 4 >= ((size_t)1 << 21) ? grid1d((n / 4 + SPLIT_U - 1) / SPLIT_U, 256)
                                                           : grid1d(n / 4, 256)),
                           dim3(256), 0, (hipStream_t)stream,
                           reinterpret_cast<uint2 *>(hi), reinterpret_cast<uint2 *>(lo),
                           reinterpret_cast<const float4 *>(x), n / 4);
    else
        hipLaunchKernelGGL(split_kernel, dim3(grid1d(n, 256)), dim3(256), 0, (hipStream_t)stream, hi,
                           lo, x, n);
    K3K_LAUNCH_CHECK("split launch");
    return 0;
}

/* Matrix-core partials: a workgroup covers RM_TB tokens x RM_EB experts (one 16 x 32
 * block per wave). */
constexpr int RM_TB = 32, RM_EB = 64;

extern "C" int k3k_router_chunk(int T, int hidden, int n_experts)
{
    if (T <= RS_T) return RS_CH;          /* one lane per (expert, 128-column chunk) */
    const long tiles = (long)((n_experts + RM_EB - 1) / RM_EB) * ((T + RM_TB - 1) / RM_TB);
    const long cus = k3k_cu_count() > 0 ? k3k_cu_count() : 1;
    /* Few tiles (small batches): a chunk count that is a multiple of the XCD count, so that
     * each chunk's workgroups run on one XCD and fetch its W and x pieces once
     * (router_partial_mfma_kernel's grouped grid), about 1.5 workgroups per CU, chunks of at
     * least 224 columns */
    if (tiles * K3_NXCD <= cus) {
        long ks = ((3 * cus) / 2 + tiles - 1) / tiles;
        ks = (ks + K3_NXCD - 1) / K3_NXCD * K3_NXCD;
        while (ks > K3_NXCD && hidden / ks < 224) ks -= K3_NXCD;
        const long chunk = ((hidden + ks - 1) / ks + RP_KS - 1) / RP_KS * RP_KS;
        if (chunk >= 224 && ((hidden + chunk - 1) / chunk) % K3_NXCD == 0) return (int)chunk;
    }
    /* chunks a multiple of 32 columns and at least 256; among those, the split whose
     * busiest CU has the least work (workgroups per CU x columns per workgroup), the most
     * workgroups among equals (a shorter tail) up to 12 per CU (more partials to sum) */
    long kmax = (hidden + 255) / 256;
    if (kmax < 1) kmax = 1;
    long best_chunk = 0, best_load = -1;
    for (long ks = 1; ks <= kmax; ks++) {
        long chunk = (hidden + ks - 1) / ks;
        chunk = (chunk + RP_KS - 1) / RP_KS * RP_KS;
        const long n = (hidden + chunk - 1) / chunk;
        const long per_cu = (tiles * n + cus - 1) / cus;
        if (best_load >= 0 && per_cu > 12) break;
        const long load = per_cu * chunk;
        if (best_load < 0 || load <= best_load) { best_load = load; best_chunk = chunk; }
    }
    return (int)best_chunk;
}

/* Up to RS_T tokens and 64 chunks of RS_CH columns: router_small_kernel certifies and
 * scores the logits itself, and the final kernel starts from its records. */
static bool router_small_mode(int T, int hidden)
{
    return T <= RS_T && (hidden + RS_CH - 1) / RS_CH <= 64;
}

extern "C" int k3k_router_small(int T, int hidden)
{
    return router_small_mode(T, hidden) ? 1 : 0;
}

static ExcTable exc_view(const K3kExc *exc)
{
    ExcTable e;
    memset(&e, 0, sizeof e);
    if (exc) {
        e.pairs = exc->pairs;
        e.index = exc->index;
        e.bits = exc->bits;
        e.kmin = exc->kmin;
        e.kmax = exc->kmax;
        e.base = exc->base;
        e.mmin = exc->mmin;
        e.mwords = exc->mwords;
        e.n = exc->n;
    }
    return e;
}

extern "C" int k3k_router_partial(double *part, float *rbound, const float *x, int T,
                                  const float *W, int hidden, int n_experts, int chunk,
                                  int *ctr, int *idx, int n_idx, const K3kExc *exc, void *stream)
{
    if (ctr && n_idx > 0 && !idx) return k3k_fail("router_partial: idx to reset", hipErrorInvalidValue);
    if (!ctr) n_idx = 0;
    if (T <= 0 || n_experts <= 0) return 0;
    if (chunk <= 0 || chunk % RP_KS) return k3k_fail("router_partial: chunk", hipErrorInvalidValue);
    const int ks = (hidden + chunk - 1) / chunk;
    const int vec = (hidden % 4 == 0) && ((((uintptr_t)x) | ((uintptr_t)W)) % 16 == 0);
    hipStream_t st = (hipStream_t)stream;
    if (router_small_mode(T, hidden)) {
        if (chunk != RS_CH) return k3k_fail("router_partial: chunk", hipErrorInvalidValue);
        const size_t lds = 0;
        const ExcTable e = exc_view(exc);
        float4 *pre = reinterpret_cast<float4 *>(part);
        const dim3 grid(n_experts);
        if (T == 1 && vec)
            hipLaunchKernelGGL((router_small_kernel<1, true>), grid, dim3(256), lds, st, pre, x, T, W,
                               hidden, n_experts, e);
        else if (T == 1)
            hipLaunchKernelGGL((router_small_kernel<1, false>), grid, dim3(256), lds, st, pre, x, T, W,
                               hidden, n_experts, e);
        else if (vec)
            hipLaunchKernelGGL((router_small_kernel<RS_T, true>), grid, dim3(256), lds, st, pre, x, T,
                               W, hidden, n_experts, e);
        else
            hipLaunchKernelGGL((router_small_kernel<RS_T, false>), grid, dim3(256), lds, st, pre, x, T,
                               W, hidden, n_experts, e);
    } else if (T <= RS_T) {
        if (chunk != RS_CH) return k3k_fail("router_partial: chunk", hipErrorInvalidValue);
        dim3 grid((n_experts + 255) / 256, ks);
        if (T == 1)
            hipLaunchKernelGGL(router_partial_small_kernel<1>, grid, dim3(256), 0, st, part, rbound,
                               x, T, W, hidden, n_experts, vec);
        else
            hipLaunchKernelGGL(router_partial_small_kernel<RS_T>, grid, dim3(256), 0, st, part,
                               rbound, x, T, W, hidden, n_experts, vec);
    } else {
        static_assert(RM_TB == 32 * 1 && RM_EB == 32 * 2, "tile of router_partial_mfma_kernel<1, 2>");
        const int nee = (n_experts + RM_EB - 1) / RM_EB, ntt = (T + RM_TB - 1) / RM_TB;
        /* dealt to the XCDs: whole chunks when their count is a multiple of the XCD count,
         * else ranges of (chunk, token tile) pairs */
        const int deal = ks % K3_NXCD == 0 ? 1 : 2;
        const int per = (ks * ntt + K3_NXCD - 1) / K3_NXCD;
        const dim3 grid = deal == 1 ? dim3((unsigned)(nee * ntt * ks)) : dim3((unsigned)(K3_NXCD * per * nee));
        const bool buf = vec && (size_t)n_experts * hidden * 4 < 0x80000000u &&
                         (size_t)T * hidden * 4 < 0x80000000u;
        if (buf)
            hipLaunchKernelGGL((router_partial_mfma_kernel<1, 2, true>), grid, dim3(256), 0, st, part,
                               rbound, x, T, W, hidden, n_experts, chunk, vec, deal, ctr, idx, n_idx);
        else
            hipLaunchKernelGGL((router_partial_mfma_kernel<1, 2, false>), grid, dim3(256), 0, st, part,
                               rbound, x, T, W, hidden, n_experts, chunk, vec, deal, ctr, idx, n_idx);
    }
    K3K_LAUNCH_CHECK("router_partial launch");
    return 0;
}

extern "C" int k3k_router_gathers(int T, int hidden, int n_experts, int topk)
{
    (void)hidden;
    return T > RS_T && n_experts <= RF_MAXE && topk <= 64 && k3k_gather_scratch(T, topk, n_experts) == 0;
}

static GatherDev gather_dev(const K3kGatherArgs *g, const int *idx, int N, int n_experts)
{
    GatherDev d;
    memset(&d, 0, sizeof d);
    if (g) {
        d.offsets = g->offsets;
        d.perm = g->perm;
        d.job_expert = g->job_expert;
        d.job_off = g->job_off;
        d.job_cnt = g->job_cnt;
        d.pass_job = g->pass_job;
        d.pass_tp = g->pass_tp;
        d.pass_job2 = g->pass_job2;
        d.pass_tp2 = g->pass_tp2;
        d.counts = g->counts;
        d.bank = g->bank;
        d.pass_tok = g->pass_tok;
        d.pass_tok2 = g->pass_tok2;
        d.ctr = g->ctr;
    }
    d.idx = idx;
    d.N = N;
    d.n_experts = n_experts;
    return d;
}

extern "C" int k3k_router_final(int *idx, float *wt, int *nrecomp, const double *part,
                                const float *rbound, int chunk, const float *x, const float *W,
                                const float *bias, int T, int hidden, int n_experts, int topk,
                                int renorm, float routed_scale, const K3kExc *exc,
                                const K3kGatherArgs *gather, void *stream)
{
    if (T <= 0) return 0;
    if (n_experts > RF_MAXE || topk > 64)
        return k3k_fail("router_final: n_experts or topk too large", hipErrorInvalidValue);
    const ExcTable e = exc_view(exc);
    const int ks = (hidden + chunk - 1) / chunk;
    int nw = (n_experts + 63) / 64;
    if (nw > RF_MAXW) nw = RF_MAXW;
    hipStream_t st = (hipStream_t)stream;
    const bool pre = router_small_mode(T, hidden);
    const GatherDev gd = gather_dev(gather, idx, T * topk, n_experts);
    if (gather) {
        /* the selection, then the gather in the workgroup that finishes last (1024 threads) */
        if (!k3k_router_gathers(T, hidden, n_experts, topk) || !gather->ctr || n_experts > G_MAXE ||
            (gather->pass_tok2 > 0 && (!gather->pass_job2 || !gather->pass_tp2)))
            return k3k_fail("router_final: the gather cannot run here", hipErrorInvalidValue);
#define K3_RFG(SL, SW, KB)                                                                           \
    hipLaunchKernelGGL((router_final_kernel<SL, SW, KB, false, true>), dim3(T), dim3(1024), 0, st, idx, wt, \
                       nrecomp, part, rbound, ks, chunk, x, W, bias, T, hidden, n_experts, topk, renorm, \
                       routed_scale, e, gd)
        if (n_experts <= 512 && ks <= 16) K3_RFG(1, 8, 16);
        else if (n_experts <= 512) K3_RFG(1, 8, RF_KB);
        else if (n_experts <= 1024) K3_RFG(1, 16, RF_KB);
        else K3_RFG(2, 32, RF_KB);
#undef K3_RFG
        K3K_LAUNCH_CHECK("router_final launch");
        return 0;
    }
    /* scored records (a few tokens) or the chunk partials: a lane per expert (two past
     * 1024), all of a lane's partials in one load batch when they are at most 32 -- up to 512
     * experts the batch is sized to the chunk count (2, 4, 8 or 16: no repeated loads, fewer
     * registers, more workgroups per CU) -- or 64 for up to 64 tokens and 512 experts (more
     * registers, fewer waves per CU: only while the tokens do not fill the chip). The
     * selection is two-level when the expert groups fit (select_rounds), else wave 0 selects
     * over SW keys per lane: 8 up to 512 experts, 16 up to 1024, else 32 (each pick rescans
     * the picking lane's SW keys). */
#define K3_RF(SL, SW, KB, PRE, NT)                                                                  \
    hipLaunchKernelGGL((router_final_kernel<SL, SW, KB, PRE>), dim3(T), dim3(NT), 0, st, idx, wt, nrecomp, \
                       part, rbound, ks, chunk, x, W, bias, T, hidden, n_experts, topk, renorm,        \
                       routed_scale, e, gd)
    if (pre && n_experts <= 512) K3_RF(1, 8, RF_KB, true, 64 * nw);
    else if (pre && n_experts <= 1024) K3_RF(1, 16, RF_KB, true, 64 * nw);
    else if (pre) K3_RF(2, 32, RF_KB, true, 64 * nw);
    else if (n_experts <= 512 && ks <= 2) K3_RF(1, 8, 2, false, 64 * nw);
    else if (n_experts <= 512 && ks <= 4) K3_RF(1, 8, 4, false, 64 * nw);
    else if (n_experts <= 512 && ks <= 8) K3_RF(1, 8, 8, false, 64 * nw);
    else if (n_experts <= 512 && ks <= 16) K3_RF(1, 8, 16, false, 64 * nw);
    else if (n_experts <= 512 && ks > 32 && ks <= 64 && T <= 64) K3_RF(1, 8, 64, false, 64 * nw);
    else if (n_experts <= 512) K3_RF(1, 8, RF_KB, false, 64 * nw);
    else if (n_experts <= 64 * RF_MAXW) K3_RF(1, 16, RF_KB, false, 64 * nw);
    else K3_RF(2, 32, RF_KB, false, 64 * nw);
#undef K3_RF
    K3K_LAUNCH_CHECK("router_final launch");
    return 0;
}

extern "C" int k3k_gather(int *offsets, int *perm, int *job_expert, int *job_off, int *job_cnt,
                          int *pass_job, int *pass_tp, int *pass_job2, int *pass_tp2, int *counts,
                          int *hist, const int *idx, int T, int topk, int n_experts,
                          const void *bank, int pass_tok, int pass_tok2, void *stream)
{
    if (n_experts > G_MAXE) return k3k_fail("gather: too many experts", hipErrorInvalidValue);
    if (pass_tok2 > 0 && (!pass_job2 || !pass_tp2))
        return k3k_fail("gather: second pass list missing", hipErrorInvalidValue);
    hipStream_t st = (hipStream_t)stream;
    const int N = T * topk;
    const size_t need = k3k_gather_scratch(T, topk, n_experts);
    if (need && hist) {
        const int nchunk = (N + GM_C - 1) / GM_C;
        hipLaunchKernelGGL(gather_hist_kernel, dim3(nchunk), dim3(GM_C), 0, st, hist, idx, N,
                           n_experts, nchunk);
        hipLaunchKernelGGL(gather_scan_kernel, dim3(1), dim3(1024), 0, st, hist, offsets, job_expert,
                           job_off, job_cnt, pass_job, pass_tp, pass_job2, pass_tp2, counts,
                           n_experts, nchunk, bank, pass_tok, pass_tok2);
        hipLaunchKernelGGL(gather_place_kernel, dim3(nchunk), dim3(GM_C), 0, st, perm, hist, idx, N,
                           n_experts, nchunk);
    } else {
        const K3kGatherArgs ga = {offsets, perm, job_expert, job_off, job_cnt, pass_job, pass_tp,
                                  pass_job2, pass_tp2, counts, bank, topk, pass_tok, pass_tok2, NULL};
        hipLaunchKernelGGL(gather_kernel, dim3(1), dim3(1024), 0, st, gather_dev(&ga, idx, N, n_experts));
    }
    K3K_LAUNCH_CHECK("gather launch");
    return 0;
}

extern "C" size_t k3k_gather_scratch(int T, int topk, int n_experts)
{
    const long N = (long)T * topk;
    if (N <= GM_MIN || n_experts > G_WCNT_E) return 0;
    return (size_t)((N + GM_C - 1) / GM_C) * (size_t)n_experts;
}

extern "C" int k3k_combine(float *out, const float *contrib, const float *wt, const int *idx,
                           const void *bank, int n_experts, int T, int topk, int E, void *stream)
{
    if (T <= 0) return 0;
    if (topk > K3_MAX_TOPK_DEV) return k3k_fail("combine: topk too large", hipErrorInvalidValue);
    const int vec = (E % 4 == 0) && ((((uintptr_t)out) | ((uintptr_t)contrib)) % 16 == 0);
    dim3 grid(((E + 3) / 4 + 255) / 256, T);
    if (vec)
        hipLaunchKernelGGL(combine_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, out, contrib,
                           wt, idx, bank, n_experts, T, topk, E);
    else
        hipLaunchKernelGGL(combine_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, out, contrib,
                           wt, idx, bank, n_experts, T, topk, E);
    K3K_LAUNCH_CHECK("combine launch");
    return 0;
}

extern "C" int k3k_act_split(uint16_t *hi, uint16_t *lo, const float *gu, int n, int rows, int act,
                             float b1, float b2, void *stream)
{
    const size_t total = (size_t)n * rows;
    if (!total) return 0;
    hipLaunchKernelGGL(act_split_kernel, dim3(grid1d(total, 256)), dim3(256), 0, (hipStream_t)stream, hi, lo,
                       gu, n, rows, act, b1, b2);
    K3K_LAUNCH_CHECK("act_split launch");
    return 0;
}

extern "C" int k3k_act(float *y, const float *gu, int n, int rows, int act, float b1, float b2,
                       void *stream)
{
    const size_t total = (size_t)n * rows;
    if (!total) return 0;
    hipLaunchKernelGGL(act_kernel, dim3(grid1d(total, 256)), dim3(256), 0, (hipStream_t)stream, y,
                       gu, n, rows, act, b1, b2);
    K3K_LAUNCH_CHECK("act launch");
    return 0;
}

extern "C" int k3k_rmsnorm(float *y, const float *x, const float *w, int n, int rows, float eps,
                           void *stream)
{
    if (rows <= 0) return 0;
    if (n <= 256 * 16)
        hipLaunchKernelGGL(rmsnorm_reg_kernel<16>, dim3(rows), dim3(256), 0, (hipStream_t)stream, y, x, w,
                           n, eps);
    else if (n <= 256 * 32)
        hipLaunchKernelGGL(rmsnorm_reg_kernel<32>, dim3(rows), dim3(256), 0, (hipStream_t)stream, y, x, w,
                           n, eps);
    else
        hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, y, x, w, n,
                           eps);
    K3K_LAUNCH_CHECK("rmsnorm launch");
    return 0;
}

extern "C" int k3k_axpy_rows(float *out, const float *add, size_t n, void *stream)
{
    if (!n) return 0;
    hipLaunchKernelGGL(axpy_kernel, dim3(grid1d(n, 256)), dim3(256), 0, (hipStream_t)stream, out,
                       add, n);
    K3K_LAUNCH_CHECK("axpy launch");
    return 0;
}

extern "C" int k3k_scale(float *out, const float *in, float s, size_t n, void *stream)
{
    if (!n) return 0;
    hipLaunchKernelGGL(scale_kernel, dim3(grid1d(n, 256)), dim3(256), 0, (hipStream_t)stream, out,
                       in, s, n);
    K3K_LAUNCH_CHECK("scale launch");
    return 0;
}
