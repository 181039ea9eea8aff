/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_route.hip -- the routing side of the MoE layer on gfx950: activation split, the
 * sigmoid top-k router, the expert-major gather, the weighted combine, and the small
 * elementwise kernels (activation, RMSNorm).
 */
#include "k3_common.h"
#include "k3_expf.h"
#include "k3k.h"

#include <string.h>

namespace {

struct ExpertQDev {
    const uint8_t *p1, *s1, *p3, *s3, *p2, *s2;
};

__device__ __forceinline__ bool expert_present(const void *bank, int e)
{
    const ExpertQDev q = reinterpret_cast<const ExpertQDev *>(bank)[e];
    return q.p1 && q.s1 && q.p3 && q.s3 && q.p2 && q.s2;
}

/* ---- fp32 -> bf16 hi/lo ----------------------------------------------------------- */
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
 * W[e][k] * (double)x[t][k] (k3_ops.c:446-450). A product of two floats is exact in fp64,
 * so fma(w, x, acc) rounds exactly like the separate multiply and add; one lane runs one
 * (token, expert) chain in the reference's order, so the logit is bit-identical to the
 * reference's by construction. Then score = 1/(1+expf(-(float)acc)) with the host libm's
 * expf (k3_ops.c:451) and choice = score + bias (k3_ops.c:452).
 *
 * A workgroup covers EB experts x TB tokens (EB*TB = 256 lanes): EB = 4, TB = 64 (a wave
 * is 64 tokens of one expert) when there are many tokens, EB = 64, TB = 4 (a wave is 64
 * experts of one token) when there are few. K walks in chunks of RC columns; W and x of the
 * chunk are staged in LDS (double buffered) and each lane reads its W row and x row 4
 * columns at a time. */

struct ExcTable {
    const uint32_t *pairs;      /* sorted (key bits of v, libm expf(v) bits) */
    const uint32_t *index;      /* index[b] = first pair with (key >> 12) - base >= b */
    const uint32_t *bits;       /* membership bitmap over |key| in [mmin, mmax], per sign */
    uint32_t kmin, kmax, base, mmin, mwords;
    int n;
};

/* libm-exact score 1/(1+expf(v)), v = -logit: the deterministic correctly rounded
 * candidate, replaced where the host libm's expf differs (exception table built at build
 * time from that libm). One bitmap load decides membership; only members search their
 * bucket (key >> 12, at most 17 pairs). */
__device__ __forceinline__ float router_score(float logit, const ExcTable &x)
{
    const float v = -logit;
    float E = k3_expf_det(v);
    const uint32_t key = __float_as_uint(v);
    const uint32_t mag = key & 0x7fffffffu;
    if (x.n > 0 && mag >= x.mmin) {
        const uint32_t bi = mag - x.mmin, w = bi >> 5;
        if (w < x.mwords && ((x.bits[(key >> 31) * x.mwords + w] >> (bi & 31)) & 1u)) {
            const uint32_t bkt = (key >> 12) - x.base;
            int lo = (int)x.index[bkt], hi = (int)x.index[bkt + 1];
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (x.pairs[2 * mid] < key) lo = mid + 1;
                else hi = mid;
            }
            if (lo < x.n && x.pairs[2 * lo] == key) E = __uint_as_float(x.pairs[2 * lo + 1]);
        }
    }
    return 1.0f / (1.0f + E);
}

/* ---- router logits, certified ---------------------------------------------------------
 * The reference's logit is one sequential fp64 chain per (token, expert):
 *   a_0 = 0, a_{i+1} = fl(a_i + w_i x_i), i ascending, logit = (float)a_n
 * (k3_ops.c:446-451; the product of two floats is exact in fp64, so fma(w, x, a) rounds
 * like the separate multiply and add). Run literally, that is a 7168-step dependent chain
 * per logit. Instead:
 *
 * 1. router_partial_kernel computes, per K chunk k of C_k columns, the chunk's own chain
 *    P_k (from 0, ascending) and R_k, an upper bound on the sum of |r_i| over the chunk's
 *    intermediate values r_i: per 32-column sub-block, 32 * (|r at its start| + ||w||_1 *
 *    ||x||_inf of the sub-block).
 * 2. router_final_kernel sums S = P_0 + P_1 + ... in k order and bounds |S - a_n|: with
 *    u = 2^-53 and Q_k the prefix before chunk k, the reference's chain errs from the
 *    exact sum by at most u * sum_i |a_i| <= u * sum_k (C_k |Q_k| + R_k), this
 *    computation by at most u * sum_k (R_k + |Q_{k+1}|); B = 1.01 u sum_k (C_k |Q_k| +
 *    2 R_k + |Q_{k+1}|) + 4u|S| covers both and the second-order terms. If every value in
 *    [S - B, S + B] rounds to the same float, that float is the reference's logit.
 * 3. Logits that are not certified and could matter -- the expert is selected (its weight
 *    must be exact) or its choice could reach the selection -- are recomputed with the
 *    reference's chain itself, and the selection is redone until no such logit is left.
 *
 * The partial kernel: a workgroup computes 32 experts x 64 tokens over one chunk, a thread
 * 2 experts x 4 tokens. W and x are staged in LDS 32 columns at a time (double buffered),
 * widened to fp64 once while staging (the conversion costs four times an fp64 fma), with
 * the sub-block norms; the threads' LDS reads are mostly broadcasts. */
constexpr int RP_E = 32, RP_T = 64, RP_KS = 32, RP_SUB = 32, RP_LD = RP_KS + 2;

__global__ __launch_bounds__(256) void router_partial_kernel(double *part, float *rbound,
                                                             const float *x, int T, const float *W,
                                                             int hidden, int n_experts, int chunk,
                                                             int vec)
{
    __shared__ __attribute__((aligned(16))) double ws[2][RP_E][RP_LD];
    __shared__ __attribute__((aligned(16))) double xs[2][RP_T][RP_LD];
    __shared__ float wn[2][RP_E];                    /* sum |w| over the sub-block */
    __shared__ float xn[2][RP_T];                    /* max |x| over the sub-block */
    const int tid = threadIdx.x;
    const int eg = tid & 15, tg = tid >> 4;          /* experts 2eg, 2eg+1; tokens 4tg.. */
    const int e0 = blockIdx.x * RP_E, t0 = blockIdx.y * RP_T, ks = blockIdx.z;
    const int kb0 = ks * chunk, kb1 = min(hidden, kb0 + chunk);
    const int nsub = (kb1 - kb0 + RP_KS - 1) / RP_KS;
    const float *Wt = W + (size_t)e0 * hidden, *xt = x + (size_t)t0 * hidden;
    /* staging: W 32 rows x 8 float4 = 256 pieces (1 per thread), x 64 x 8 = 512 (2) */
    float4 wst, xst[2];
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
    auto load = [&](int sc) {
        const int k0 = kb0 + sc * RP_KS;
        wst = fetch(Wt, n_experts - e0, tid >> 3, k0 + (tid & 7) * 4);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int pc = tid + 256 * i;
            xst[i] = fetch(xt, T - t0, pc >> 3, k0 + (pc & 7) * 4);
        }
    };
    auto put = [&](double *dst, float4 v) {
        reinterpret_cast<double2 *>(dst)[0] = make_double2((double)v.x, (double)v.y);
        reinterpret_cast<double2 *>(dst)[1] = make_double2((double)v.z, (double)v.w);
    };
    auto store = [&](int buf) {
        /* 8 consecutive threads hold one row's 32 columns */
        {
            const int r = tid >> 3, c = (tid & 7) * 4;
            put(&ws[buf][r][c], wst);
            float a = fabsf(wst.x) + fabsf(wst.y) + fabsf(wst.z) + fabsf(wst.w);
            a += __shfl_xor(a, 1, 64);
            a += __shfl_xor(a, 2, 64);
            a += __shfl_xor(a, 4, 64);
            if ((tid & 7) == 0) wn[buf][r] = a;
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int pc = tid + 256 * i, r = pc >> 3, c = (pc & 7) * 4;
            put(&xs[buf][r][c], xst[i]);
            float m = fmaxf(fmaxf(fabsf(xst[i].x), fabsf(xst[i].y)), fmaxf(fabsf(xst[i].z), fabsf(xst[i].w)));
            m = fmaxf(m, __shfl_xor(m, 1, 64));
            m = fmaxf(m, __shfl_xor(m, 2, 64));
            m = fmaxf(m, __shfl_xor(m, 4, 64));
            if ((pc & 7) == 0) xn[buf][r] = m;
        }
    };

    double acc[2][4], rb[2][4];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) { acc[a][b] = 0.0; rb[a][b] = 0.0; }

    load(0);
    store(0);
    __syncthreads();
    for (int sc = 0; sc < nsub; sc++) {
        const int buf = sc & 1;
        if (sc + 1 < nsub) load(sc + 1);
        /* bound term of this sub-block, from the chains' values at its start */
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const double an = (double)wn[buf][2 * eg + a] * (double)xn[buf][4 * tg + b];
                rb[a][b] = fma((double)RP_SUB, fabs(acc[a][b]) + an, rb[a][b]);
            }
#pragma unroll 4
        for (int k = 0; k < RP_KS; k += 2) {
            const double2 w0 = *reinterpret_cast<const double2 *>(&ws[buf][2 * eg][k]);
            const double2 w1 = *reinterpret_cast<const double2 *>(&ws[buf][2 * eg + 1][k]);
            double2 xv[4];
#pragma unroll
            for (int b = 0; b < 4; b++) xv[b] = *reinterpret_cast<const double2 *>(&xs[buf][4 * tg + b][k]);
#pragma unroll
            for (int b = 0; b < 4; b++) {
                acc[0][b] = fma(w0.x, xv[b].x, acc[0][b]);
                acc[1][b] = fma(w1.x, xv[b].x, acc[1][b]);
            }
#pragma unroll
            for (int b = 0; b < 4; b++) {
                acc[0][b] = fma(w0.y, xv[b].y, acc[0][b]);
                acc[1][b] = fma(w1.y, xv[b].y, acc[1][b]);
            }
        }
        if (sc + 1 < nsub) store(buf ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int e = e0 + 2 * eg + a, t = t0 + 4 * tg + b;
            if (e < n_experts && t < T) {
                const size_t o = ((size_t)ks * T + t) * n_experts + e;
                part[o] = acc[a][b];
                /* rounded up: the float sums of |w| carry at most a 2^-18 relative error */
                rbound[o] = (float)(rb[a][b] * (1.0 + 0x1p-17)) * (1.0f + 0x1p-20f);
            }
        }
}

/* The same partials for a few tokens (T <= RS_T): one lane per (expert, chunk) runs the
 * chunk's chain for every token; the lane streams its W row segment itself (float4), the
 * tokens' chunk is staged in LDS as fp64 and read as broadcasts. The bound R_k per chain
 * uses the lane's own running sum of |w| over each 32-column sub-block. */
constexpr int RS_T = 4;

template <int NT>
__global__ __launch_bounds__(256) void router_partial_small_kernel(double *part, float *rbound,
                                                                   const float *x, int T,
                                                                   const float *W, int hidden,
                                                                   int n_experts, int chunk,
                                                                   int vec)
{
    extern __shared__ double xsh[];                  /* [NT][chunk] */
    const int ks = blockIdx.y;
    const int e = blockIdx.x * 256 + threadIdx.x;
    const int kb0 = ks * chunk, kb1 = min(hidden, kb0 + chunk);
    const int len = kb1 - kb0;
    for (int i = threadIdx.x; i < NT * chunk; i += 256) {
        const int t = i / chunk, k = i % chunk;
        xsh[i] = (t < T && k < len) ? (double)x[(size_t)t * hidden + kb0 + k] : 0.0;
    }
    __syncthreads();
    if (e >= n_experts) return;
    /* sub-block maxima of |x| per token */
    const float *wr = W + (size_t)e * hidden + kb0;
    double acc[NT], rb[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) { acc[t] = 0.0; rb[t] = 0.0; }
    for (int s0 = 0; s0 < len; s0 += 32) {
        const int sl = min(32, len - s0);
        float wv[32];
        if (vec && sl == 32) {
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const float4 v = *reinterpret_cast<const float4 *>(wr + s0 + 4 * q);
                wv[4 * q] = v.x; wv[4 * q + 1] = v.y; wv[4 * q + 2] = v.z; wv[4 * q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int q = 0; q < 32; q++) wv[q] = q < sl ? wr[s0 + q] : 0.0f;
        }
        float wn = 0.0f;
#pragma unroll
        for (int q = 0; q < 32; q++) wn += fabsf(wv[q]);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            double xm = 0.0;
#pragma unroll
            for (int q = 0; q < 32; q++) xm = fmax(xm, fabs(xsh[t * chunk + s0 + min(q, sl - 1)]));
            rb[t] = fma(32.0, fabs(acc[t]) + (double)wn * xm, rb[t]);
        }
#pragma unroll
        for (int q = 0; q < 32; q++) {
            const double wd = (double)wv[q];
#pragma unroll
            for (int t = 0; t < NT; t++)
                if (q < sl) acc[t] = fma(wd, xsh[t * chunk + s0 + q], acc[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++)
        if (t < T) {
            const size_t o = ((size_t)ks * T + t) * n_experts + e;
            part[o] = acc[t];
            rbound[o] = (float)(rb[t] * (1.0 + 0x1p-17)) * (1.0f + 0x1p-20f);
        }
}

/* The reference's own chain for one logit (the fallback of the certification). */
__device__ __forceinline__ double router_chain(const float *w, const float *x, int hidden)
{
    double acc = 0.0;
    int k = 0;
    for (; k + 8 <= hidden; k += 8) {
        float wv[8], xv[8];
#pragma unroll
        for (int j = 0; j < 8; j++) { wv[j] = w[k + j]; xv[j] = x[k + j]; }
#pragma unroll
        for (int j = 0; j < 8; j++) acc = fma((double)wv[j], (double)xv[j], acc);
    }
    for (; k < hidden; k++) acc = fma((double)w[k], (double)x[k], acc);
    return acc;
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

/* One workgroup per token, one lane per expert (SL experts per lane past 1024): certify
 * the logit, score, then topk rounds of the reference's rule -- largest choice, lowest
 * index among equals, strictly above -inf, none left: idx 0, weight 0 (k3_ops.c:459-467)
 * -- with a wave argmax and one barrier per round; recompute what matters and repeat;
 * renormalise and scale (k3_ops.c:469-475). nrecomp[t] (optional) counts recomputes. */
constexpr int RF_MAXE = 2048, RF_MAXW = 16, RF_KB = 32;

template <int SL>
__global__ __launch_bounds__(1024) void router_final_kernel(int *idx, float *wt, int *nrecomp,
                                                            const double *part,
                                                            const float *rbound, int ksplit,
                                                            int chunk, const float *x,
                                                            const float *W, const float *bias,
                                                            int T, int hidden, int n_experts,
                                                            int topk, int renorm,
                                                            float routed_scale, ExcTable exc)
{
    __shared__ float rbv[2][RF_MAXW];
    __shared__ int rbi[2][RF_MAXW];
    __shared__ float selw[64];
    __shared__ int selid[64];
    __shared__ int nre_sh;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, nw = blockDim.x >> 6;
    const int nthr = blockDim.x;
    const int t = blockIdx.x;
    if (tid == 0) nre_sh = 0;
    float c[SL], cmax[SL], sc[SL];
    bool unc[SL];
#pragma unroll
    for (int i = 0; i < SL; i++) {
        const int e = tid + nthr * i;
        c[i] = -INFINITY;
        cmax[i] = -INFINITY;
        sc[i] = 0.0f;
        unc[i] = false;
        if (e < n_experts) {
            double Q = 0.0, bs = 0.0;
            for (int k0 = 0; k0 < ksplit; k0 += RF_KB) {
                /* one batch of chunk loads in flight together */
                double pv[RF_KB];
                float rv[RF_KB];
#pragma unroll
                for (int kk = 0; kk < RF_KB; kk++) {
                    const int k = min(k0 + kk, ksplit - 1);
                    const size_t o = ((size_t)k * T + t) * n_experts + e;
                    pv[kk] = part[o];
                    rv[kk] = rbound[o];
                }
#pragma unroll
                for (int kk = 0; kk < RF_KB; kk++) {
                    const int k = k0 + kk;
                    if (k < ksplit) {
                        const int ck = min(chunk, hidden - k * chunk);
                        bs += (double)ck * fabs(Q) + 2.0 * (double)rv[kk];
                        Q += pv[kk];
                        bs += fabs(Q);
                    }
                }
            }
            const float f = (float)Q;
            /* non-finite sums come from inf/NaN inputs and propagate alike in any order */
            bool ok = true;
            float fhi = f;
            if (fabs(Q) <= 0x1.fffffffffffffp+1023) {
                const double B = 1.01 * 0x1p-53 * bs + 4.0 * 0x1p-53 * fabs(Q) + 0x1p-1060;
                double mlo, mhi;
                round_interval(f, mlo, mhi);
                ok = (Q - B > mlo) && (Q + B < mhi);
                if (!ok) {
                    const float hb = (float)(Q + B);
                    fhi = fabsf(hb) <= 0x1.fffffep+127f ? next_float(hb, true) : hb;
                }
            }
            sc[i] = router_score(f, exc);
            const float bb = bias ? bias[e] : 0.0f;
            c[i] = sc[i] + bb;
            cmax[i] = c[i];
            if (!ok) {
                unc[i] = true;
                cmax[i] = router_score(fhi, exc) + bb;      /* choice is monotone in logit */
            }
        }
    }
    __syncthreads();
    for (int round = 0; round <= n_experts; round++) {
        float cc[SL];
        bool sel[SL];
#pragma unroll
        for (int i = 0; i < SL; i++) { cc[i] = c[i]; sel[i] = false; }
        float ckth = -INFINITY;
        int nsel = 0;
        for (int j = 0; j < topk; j++) {
            float bv = -INFINITY;
            int bi = -1;
#pragma unroll
            for (int i = 0; i < SL; i++)
                if (cc[i] > bv) { bv = cc[i]; bi = tid + nthr * i; }
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const float ov = __shfl_xor(bv, o, 64);
                const int oi = __shfl_xor(bi, o, 64);
                if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
            }
            if (lane == 0) { rbv[j & 1][wv] = bv; rbi[j & 1][wv] = bi; }
            __syncthreads();
            bv = -INFINITY;
            bi = -1;
            for (int w = 0; w < nw; w++) {
                const float ov = rbv[j & 1][w];
                const int oi = rbi[j & 1][w];
                if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
            }
            if (bi >= 0) {
                nsel++;
                ckth = bv;
#pragma unroll
                for (int i = 0; i < SL; i++)
                    if (bi == tid + nthr * i) {
                        cc[i] = -INFINITY;
                        sel[i] = true;
                        selw[j] = sc[i];
                        selid[j] = bi;
                    }
            } else if (tid == 0) {
                selw[j] = 0.0f;
                selid[j] = 0;
            }
        }
        /* uncertified logits that matter: selected, or able to reach the selection */
        bool need_any = false;
        bool need[SL];
#pragma unroll
        for (int i = 0; i < SL; i++) {
            need[i] = unc[i] && (sel[i] || nsel < topk || cmax[i] >= ckth);
            need_any |= need[i];
        }
        if (!__syncthreads_or(need_any)) break;
#pragma unroll
        for (int i = 0; i < SL; i++)
            if (need[i]) {
                const int e = tid + nthr * i;
                const double a = router_chain(W + (size_t)e * hidden, x + (size_t)t * hidden, hidden);
                sc[i] = router_score((float)a, exc);
                c[i] = sc[i] + (bias ? bias[e] : 0.0f);
                cmax[i] = c[i];
                unc[i] = false;
                atomicAdd(&nre_sh, 1);
            }
        __syncthreads();
    }
    __syncthreads();
    if (wv == 0) {
        float w = lane < topk ? selw[lane] : 0.0f;
        if (renorm && topk > 1) {
            double s = 0.0;
            for (int j = 0; j < topk; j++) s += (double)__shfl(w, j, 64);   /* j ascending */
            const float inv = (float)(1.0 / (s + 1e-20));
            w = w * inv;
        }
        if (lane < topk) {
            idx[(size_t)t * topk + lane] = selid[lane];
            wt[(size_t)t * topk + lane] = w * routed_scale;
        }
        if (nrecomp && lane == 0) nrecomp[t] = nre_sh;
    }
}

/* ---- expert-major gather -----------------------------------------------------------
 * One workgroup of 1024 threads. Counting sort by expert, stable in assignment order:
 * chunks of 1024 assignments are placed in order; inside a chunk each wave ranks its
 * lanes among equal experts with ballots, and waves commit one after another. */
constexpr int G_MAXE = 4096;

__global__ __launch_bounds__(1024) void gather_kernel(int *offsets, int *perm, int *job_expert,
                                                      int *job_off, int *job_cnt, int *pass_job,
                                                      int *pass_tp, int *counts, const int *idx,
                                                      int N, int n_experts, const void *bank,
                                                      int pass_tok)
{
    __shared__ int cnt[G_MAXE];
    __shared__ int fill[G_MAXE];
    __shared__ int wsum[32];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    for (int e = tid; e < n_experts; e += 1024) cnt[e] = 0;
    __syncthreads();
    for (int a = tid; a < N; a += 1024) {
        const int e = idx[a];
        if (e >= 0 && e < n_experts) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();

    /* Exclusive scan of counts -> offsets; per-thread serial over a contiguous range. */
    const int per = (n_experts + 1023) / 1024;
    const int ea = tid * per, eb = min(n_experts, ea + per);
    int local = 0, ljobs = 0, lpass = 0, ldrop = 0;
    for (int e = ea; e < eb; e++) {
        local += cnt[e];
        if (cnt[e] > 0) {
            if (expert_present(bank, e)) {
                ljobs++;
                lpass += (cnt[e] + pass_tok - 1) / pass_tok;
            } else {
                ldrop += cnt[e];
            }
        }
    }
    /* block scans of (local, ljobs, lpass) via shared memory, 3 passes */
    __shared__ int sc_a[1024], sc_b[1024], sc_c[1024];
    sc_a[tid] = local;
    sc_b[tid] = ljobs;
    sc_c[tid] = lpass;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {
        const int va = tid >= o ? sc_a[tid - o] : 0;
        const int vb = tid >= o ? sc_b[tid - o] : 0;
        const int vc = tid >= o ? sc_c[tid - o] : 0;
        __syncthreads();
        sc_a[tid] += va;
        sc_b[tid] += vb;
        sc_c[tid] += vc;
        __syncthreads();
    }
    int run = sc_a[tid] - local, jrun = sc_b[tid] - ljobs, prun = sc_c[tid] - lpass;
    for (int e = ea; e < eb; e++) {
        offsets[e] = run;
        fill[e] = run;
        if (cnt[e] > 0 && expert_present(bank, e)) {
            job_expert[jrun] = e;
            job_off[jrun] = run;
            job_cnt[jrun] = cnt[e];
            const int np = (cnt[e] + pass_tok - 1) / pass_tok;
            for (int p = 0; p < np; p++) {
                pass_job[prun + p] = jrun;
                pass_tp[prun + p] = p;
            }
            prun += np;
            jrun++;
        }
        run += cnt[e];
    }
    if (tid == 1023) {
        offsets[n_experts] = sc_a[1023];
        counts[0] = sc_b[1023];
        counts[1] = sc_c[1023];
    }
    /* dropped assignment total */
    if (lane == 0) wsum[wv] = 0;
    __syncthreads();
    atomicAdd(&wsum[wv], ldrop);
    __syncthreads();
    if (tid == 0) {
        int d = 0;
        for (int w = 0; w < 16; w++) d += wsum[w];
        counts[2] = d;
    }
    __syncthreads();

    /* Stable placement. */
    for (int c0 = 0; c0 < N; c0 += 1024) {
        const int a = c0 + tid;
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
        for (int w = 0; w < 16; w++) {
            if (wv == w && ok) {
                perm[fill[e] + rank] = a;
            }
            __syncthreads();
            if (wv == w && ok && rank == __popcll(mine) - 1) fill[e] += __popcll(mine);
            __syncthreads();
        }
    }
}

/* ---- combine: out[t] = 0 + sum_j wt[t][j] * contrib[t*topk + j], j ascending ------- */
__global__ void combine_kernel(float *out, const float *contrib, const float *wt, const int *idx,
                               const void *bank, int n_experts, int T, int topk, int E)
{
    const int t = blockIdx.y;
    const int i = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (t >= T || i >= E) return;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < topk; j++) {
        const int a = t * topk + j;
        const int e = idx[a];
        if (e < 0 || e >= n_experts) continue;          /* filtered: contributes nothing */
        if (bank && !expert_present(bank, e)) continue; /* dropped: contributes nothing */
        const float w = wt[a];
        const float *c = contrib + (size_t)a * E + i;
        for (int q = 0; q < 4; q++)
            if (i + q < E) acc[q] = __fadd_rn(acc[q], __fmul_rn(w, c[q]));
    }
    for (int q = 0; q < 4; q++)
        if (i + q < E) out[(size_t)t * E + i + q] = acc[q];
}

/* ---- elementwise --------------------------------------------------------------------- */
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
    hipLaunchKernelGGL(split_kernel, dim3(grid1d(n, 256)), dim3(256), 0, (hipStream_t)stream, hi,
                       lo, x, n);
    K3K_LAUNCH_CHECK("split launch");
    return 0;
}

extern "C" int k3k_router_chunk(int T, int hidden, int n_experts)
{
    if (T <= RS_T) {
        /* one lane per (expert, chunk): 256-column chunks, at most 32 of them */
        int chunk = 256;
        while ((hidden + chunk - 1) / chunk > RF_KB) chunk += 256;
        return chunk;
    }
    /* enough workgroups to fill the chip, chunks a multiple of 32 columns */
    const long tiles = (long)((n_experts + RP_E - 1) / RP_E) * ((T + RP_T - 1) / RP_T);
    long ks = (2L * k3k_cu_count() + tiles - 1) / tiles;
    const long kmax = (hidden + 255) / 256;
    if (ks > kmax) ks = kmax;
    if (ks < 1) ks = 1;
    int chunk = (int)((hidden + ks - 1) / ks);
    chunk = (chunk + RP_KS - 1) / RP_KS * RP_KS;
    return chunk;
}

extern "C" int k3k_router_partial(double *part, float *rbound, const float *x, int T,
                                  const float *W, int hidden, int n_experts, int chunk,
                                  void *stream)
{
    if (T <= 0 || n_experts <= 0) return 0;
    if (chunk <= 0 || chunk % RP_KS) return k3k_fail("router_partial: chunk", hipErrorInvalidValue);
    const int ks = (hidden + chunk - 1) / chunk;
    const int vec = (hidden % 4 == 0) && ((((uintptr_t)x) | ((uintptr_t)W)) % 16 == 0);
    hipStream_t st = (hipStream_t)stream;
    if (T <= RS_T) {
        dim3 grid((n_experts + 255) / 256, ks);
        const size_t lds = (size_t)RS_T * chunk * sizeof(double);
        if (T == 1)
            hipLaunchKernelGGL(router_partial_small_kernel<1>, grid, dim3(256), (size_t)chunk * 8, st,
                               part, rbound, x, T, W, hidden, n_experts, chunk, vec);
        else
            hipLaunchKernelGGL(router_partial_small_kernel<RS_T>, grid, dim3(256), lds, st, part,
                               rbound, x, T, W, hidden, n_experts, chunk, vec);
    } else {
        dim3 grid((n_experts + RP_E - 1) / RP_E, (T + RP_T - 1) / RP_T, ks);
        hipLaunchKernelGGL(router_partial_kernel, grid, dim3(256), 0, st, part, rbound, x, T, W,
                           hidden, n_experts, chunk, vec);
    }
    K3K_LAUNCH_CHECK("router_partial launch");
    return 0;
}

extern "C" int k3k_router_final(int *idx, float *wt, int *nrecomp, const double *part,
                                const float *rbound, int chunk, const float *x, const float *W,
                                const float *bias, int T, int hidden, int n_experts, int topk,
                                int renorm, float routed_scale, const K3kExc *exc, void *stream)
{
    if (T <= 0) return 0;
    if (n_experts > RF_MAXE || topk > 64)
        return k3k_fail("router_final: n_experts or topk too large", hipErrorInvalidValue);
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
    const int ks = (hidden + chunk - 1) / chunk;
    int nw = (n_experts + 63) / 64;
    if (nw > RF_MAXW) nw = RF_MAXW;
    hipStream_t st = (hipStream_t)stream;
    if (n_experts <= 64 * RF_MAXW)
        hipLaunchKernelGGL(router_final_kernel<1>, dim3(T), dim3(64 * nw), 0, st, idx, wt, nrecomp,
                           part, rbound, ks, chunk, x, W, bias, T, hidden, n_experts, topk, renorm,
                           routed_scale, e);
    else
        hipLaunchKernelGGL(router_final_kernel<2>, dim3(T), dim3(64 * nw), 0, st, idx, wt, nrecomp,
                           part, rbound, ks, chunk, x, W, bias, T, hidden, n_experts, topk, renorm,
                           routed_scale, e);
    K3K_LAUNCH_CHECK("router_final launch");
    return 0;
}

extern "C" int k3k_gather(int *offsets, int *perm, int *job_expert, int *job_off, int *job_cnt,
                          int *pass_job, int *pass_tp, int *counts, const int *idx, int T,
                          int topk, int n_experts, const void *bank, int pass_tok, void *stream)
{
    if (n_experts > G_MAXE) return k3k_fail("gather: too many experts", hipErrorInvalidValue);
    hipLaunchKernelGGL(gather_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, offsets, perm,
                       job_expert, job_off, job_cnt, pass_job, pass_tp, counts, idx, T * topk,
                       n_experts, bank, pass_tok);
    K3K_LAUNCH_CHECK("gather launch");
    return 0;
}

extern "C" int k3k_combine(float *out, const float *contrib, const float *wt, const int *idx,
                           const void *bank, int n_experts, int T, int topk, int E, void *stream)
{
    if (T <= 0) return 0;
    dim3 grid((E / 4 + 255) / 256 + 1, T);
    hipLaunchKernelGGL(combine_kernel, grid, dim3(256), 0, (hipStream_t)stream, out, contrib, wt,
                       idx, bank, n_experts, T, topk, E);
    K3K_LAUNCH_CHECK("combine launch");
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
