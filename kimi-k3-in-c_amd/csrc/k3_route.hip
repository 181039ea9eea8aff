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

/* The same partials for a few tokens (T <= RS_T): one lane per (expert, chunk of RS_CH
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

/* The certification of a logit from its chunk sums (S = Q, the sum of P_k in k order, and
 * bs, the sum of C_k |Q_k| + 2 R_k + |Q_{k+1}|): with u = 2^-53, B = 1.01 u bs + 4u|S|
 * bounds |S - a_n| (the reference's chain). If every value in [S - B, S + B] rounds to the
 * same float, that float is the logit (ok); otherwise scmax is the score of the largest
 * float the logit can be. Non-finite sums come from inf/NaN inputs and propagate alike in
 * any order (ok). */
struct Certified {
    float sc, scmax;
    bool ok;
};

__device__ __forceinline__ Certified certify_score(double Q, double bs, const ExcTable &exc)
{
    const float f = (float)Q;
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
    Certified r;
    r.sc = router_score(f, exc);
    r.ok = ok;
    r.scmax = ok ? r.sc : router_score(fhi, exc);
    return r;
}

/* Router logits of a few tokens (T <= RS_T, hidden <= 64 * RS_CH), certified and scored in
 * one kernel: a wave per expert, lane k runs the chain of 128-column chunk k for every
 * token (as router_partial_small_kernel), then one lane per token sums the lanes' partials
 * in k order, certifies (certify_score) and stores pre[t][e] = {score, score of the upper
 * end, uncertified ? 1 : 0, 0}.
 * W is read in full 128-byte lines: for 32-column sub-block sb, lane l loads columns
 * 4(l % 8).. of sub-block sb of chunks l / 8 + 8j (j < 8), and a per-wave LDS buffer turns
 * that into one chunk per lane. The tokens are staged once, rows padded to ks * RS_CH.
 * In both LDS layouts a chunk's 16-byte group q sits at group (q + k) mod (its groups), so
 * the lanes' 16-byte reads of their own chunks fall on distinct banks. */
template <int NT>
__global__ __launch_bounds__(256) void router_small_kernel(float4 *pre, const float *x, int T,
                                                           const float *W, int hidden,
                                                           int n_experts, int vec, ExcTable exc)
{
    extern __shared__ __attribute__((aligned(16))) float xsf[];   /* [T][ks * RS_CH] */
    __shared__ __attribute__((aligned(16))) float wsh[4][64 * 32]; /* per wave: 64 chunks x 32 */
    __shared__ double psh[4][NT][64];
    __shared__ float rsh[4][NT][64];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int e = blockIdx.x * 4 + wv;
    const int ks = (hidden + RS_CH - 1) / RS_CH;
    const int kb0 = lane * RS_CH, len = max(0, min(RS_CH, hidden - kb0));
    const float *wr = W + (size_t)min(e, n_experts - 1) * hidden;
    /* W loads: sub-block sb, j: chunk l / 8 + 8j, columns 4(l % 8)..4(l % 8) + 3 */
    float4 wl[4][8];
    const int lq = lane & 7, lk = lane >> 3;
#pragma unroll
    for (int sb = 0; sb < 4; sb++)
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int col = (lk + 8 * j) * RS_CH + sb * 32 + 4 * lq;
            if (vec && col + 3 < hidden)
                wl[sb][j] = *reinterpret_cast<const float4 *>(wr + col);
            else
                wl[sb][j] = make_float4(col < hidden ? wr[col] : 0.f, col + 1 < hidden ? wr[col + 1] : 0.f,
                                        col + 2 < hidden ? wr[col + 2] : 0.f, col + 3 < hidden ? wr[col + 3] : 0.f);
        }
    /* stage the tokens: eight loads per thread in flight, then the stores */
    const int rowp = ks * RS_CH;
    auto slot = [&](int t, int col) {
        const int k = col / RS_CH, j = col % RS_CH;
        return t * rowp + k * RS_CH + ((j + 4 * k) & (RS_CH - 1));
    };
    if (vec) {
        const int nq = T * hidden / 4, rq = hidden / 4;
        for (int i0 = 0; i0 < nq; i0 += 256 * 8) {
            float4 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int i = i0 + tid + 256 * j;
                v[j] = i < nq ? reinterpret_cast<const float4 *>(x)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int i = i0 + tid + 256 * j;
                if (i < nq) *reinterpret_cast<float4 *>(&xsf[slot(i / rq, 4 * (i % rq))]) = v[j];
            }
        }
    } else {
        const int n = T * hidden;
        for (int i0 = 0; i0 < n; i0 += 256 * 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int i = i0 + tid + 256 * j;
                v[j] = i < n ? x[i] : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int i = i0 + tid + 256 * j;
                if (i < n) xsf[slot(i / hidden, i % hidden)] = v[j];
            }
        }
    }
    __syncthreads();
    double acc[NT], rb[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) { acc[t] = 0.0; rb[t] = 0.0; }
    float *wb = wsh[wv];
    const int xk = lane < ks ? kb0 : 0;             /* lanes past the last chunk read chunk 0 */
#pragma unroll
    for (int sb = 0; sb < 4; sb++) {
        /* this sub-block of every chunk through the wave's buffer: chunk k at 32 k, group q
         * of it at (q + k) mod 8 */
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int k = lk + 8 * j;
            *reinterpret_cast<float4 *>(&wb[k * 32 + 4 * ((lq + k) & 7)]) = wl[sb][j];
        }
        __builtin_amdgcn_wave_barrier();
        float4 wq[8];
#pragma unroll
        for (int q = 0; q < 8; q++) wq[q] = *reinterpret_cast<const float4 *>(&wb[lane * 32 + 4 * ((q + lane) & 7)]);
        __builtin_amdgcn_wave_barrier();
        float wn = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; q++)
            wn += fabsf(wq[q].x) + fabsf(wq[q].y) + fabsf(wq[q].z) + fabsf(wq[q].w);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (t >= T) break;
            float xv[32];
            float xm = 0.0f;
#pragma unroll
            for (int j4 = 0; j4 < 8; j4++) {
                const int k = sb * 32 + 4 * j4;
                const float4 v = *reinterpret_cast<const float4 *>(&xsf[t * rowp + xk + ((k + 4 * lane) & (RS_CH - 1))]);
                xv[4 * j4] = k < len ? v.x : 0.0f;
                xv[4 * j4 + 1] = k + 1 < len ? v.y : 0.0f;
                xv[4 * j4 + 2] = k + 2 < len ? v.z : 0.0f;
                xv[4 * j4 + 3] = k + 3 < len ? v.w : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < 32; j++) xm = fmaxf(xm, fabsf(xv[j]));
            rb[t] = fma(32.0, fabs(acc[t]) + (double)wn * (double)xm, rb[t]);
#pragma unroll
            for (int q = 0; q < 8; q++) {
                acc[t] = fma((double)wq[q].x, (double)xv[4 * q], acc[t]);
                acc[t] = fma((double)wq[q].y, (double)xv[4 * q + 1], acc[t]);
                acc[t] = fma((double)wq[q].z, (double)xv[4 * q + 2], acc[t]);
                acc[t] = fma((double)wq[q].w, (double)xv[4 * q + 3], acc[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        psh[wv][t][lane] = acc[t];
        /* rounded up: the float sums of |w| carry at most a 2^-18 relative error */
        rsh[wv][t][lane] = (float)(rb[t] * (1.0 + 0x1p-17)) * (1.0f + 0x1p-20f);
    }
    __syncthreads();
    if (lane < T && e < n_experts) {
        const int t = lane;
        double pv[64];
        float rv[64];
#pragma unroll
        for (int k = 0; k < 64; k++) {
            pv[k] = psh[wv][t][k];
            rv[k] = rsh[wv][t][k];
        }
        /* Q_{k+1} = Q_k + P_k in k order (the rounding the bound describes); bs, the sum of
         * C_k |Q_k| + 2 R_k + |Q_{k+1}|, only bounds and is added in any order (its own
         * relative error, under 2^-45, is far inside the bound's 1% slack) */
        double qk[65];
        qk[0] = 0.0;
#pragma unroll
        for (int k = 0; k < 64; k++) qk[k + 1] = k < ks ? qk[k] + pv[k] : qk[k];
        double term[64];
#pragma unroll
        for (int k = 0; k < 64; k++) {
            const int ck = min(RS_CH, hidden - k * RS_CH);
            term[k] = k < ks ? fma((double)ck, fabs(qk[k]), fma(2.0, (double)rv[k], fabs(qk[k + 1]))) : 0.0;
        }
#pragma unroll
        for (int w = 32; w > 0; w >>= 1)
#pragma unroll
            for (int k = 0; k < w; k++) term[k] += term[k + w];
        const Certified cs = certify_score(qk[64], term[0], exc);
        pre[(size_t)t * n_experts + e] = make_float4(cs.sc, cs.scmax, cs.ok ? 0.0f : 1.0f, 0.0f);
    }
}

/* One workgroup per token, one lane per expert (SL experts per lane past 1024): certify
 * the logit, score, then the reference's rule topk times -- largest choice, lowest index
 * among equals, strictly above -inf, none left: idx 0, weight 0 (k3_ops.c:459-467) -- as
 * topk extractions of a wave maximum (DPP) per wave, then over the waves' candidates in
 * wave 0, one barrier between; recompute what matters and repeat; renormalise and scale
 * (k3_ops.c:469-475). nrecomp[t] (optional) counts recomputes. KB: chunk partials loaded
 * per batch (64 for up to 512 experts, one batch at decode sizes). */
constexpr int RF_MAXE = 2048, RF_MAXW = 16, RF_KB = 32;

/* unsigned order of a non-NaN float that matches its numeric order (-0 as +0) */
__device__ __forceinline__ uint32_t choice_order(float v)
{
    const uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

/* 32-bit max / min of the wave by DPP, the same in every lane: pairs, quads (quad_perm),
 * 8 (row half mirror), 16 (row mirror), then rows 0-1 and 2-3 (row_bcast15 into rows 1,
 * 3) and rows 0-3 (row_bcast31 into rows 2, 3), so lane 63 holds the result. */
/* (rows outside RM read the identity of the operation, so each step is one DPP max/min) */
template <int CTRL, int RM, uint32_t ID>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp((int)ID, (int)v, CTRL, RM, 0xf, false);
}

template <bool MAX>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v)
{
    constexpr uint32_t ID = MAX ? 0u : 0xffffffffu;
    auto op = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
    v = op(v, dpp_u32<0xB1, 0xf, ID>(v));      /* quad_perm [1,0,3,2] */
    v = op(v, dpp_u32<0x4E, 0xf, ID>(v));      /* quad_perm [2,3,0,1] */
    v = op(v, dpp_u32<0x141, 0xf, ID>(v));     /* row_half_mirror */
    v = op(v, dpp_u32<0x140, 0xf, ID>(v));     /* row_mirror */
    v = op(v, dpp_u32<0x142, 0xa, ID>(v));     /* row_bcast15 */
    v = op(v, dpp_u32<0x143, 0xc, ID>(v));     /* row_bcast31 */
    return __builtin_amdgcn_readlane(v, 63);
}

/* Selection key (order-preserving bits of the choice) << 32 | ~expert: the largest key is
 * the largest choice, then the lowest expert. The wave's largest key, in every lane: the
 * largest high word, then the largest low word among the lanes holding it. */
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k)
{
    const uint32_t hi = wave_reduce_u32<true>((uint32_t)(k >> 32));
    const uint32_t lo = wave_reduce_u32<true>((uint32_t)(k >> 32) == hi ? (uint32_t)k : 0u);
    return ((uint64_t)hi << 32) | lo;
}

template <int SL, int KB, bool PRE>
__global__ __launch_bounds__(KB > 32 ? 512 : 1024) void router_final_kernel(int *idx, float *wt, int *nrecomp,
                                                            const double *part,
                                                            const float *rbound, int ksplit,
                                                            int chunk, const float *x,
                                                            const float *W, const float *bias,
                                                            int T, int hidden, int n_experts,
                                                            int topk, int renorm,
                                                            float routed_scale, ExcTable exc)
{
    __shared__ uint64_t candk[RF_MAXW][64];
    __shared__ uint64_t selk[64];
    __shared__ float csh[RF_MAXE], ssh[RF_MAXE];
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
        if (e < n_experts && PRE) {
            /* scored by router_small_kernel: {score, score of the upper end, uncertified} */
            const float4 pr = reinterpret_cast<const float4 *>(part)[(size_t)t * n_experts + e];
            sc[i] = pr.x;
            const float bb = bias ? bias[e] : 0.0f;
            c[i] = sc[i] + bb;
            cmax[i] = c[i];
            if (pr.z != 0.0f) {
                unc[i] = true;
                cmax[i] = pr.y + bb;
            }
        } else if (e < n_experts) {
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
            const Certified cs = certify_score(Q, bs, exc);
            sc[i] = cs.sc;
            const float bb = bias ? bias[e] : 0.0f;
            c[i] = sc[i] + bb;
            cmax[i] = c[i];
            if (!cs.ok) {
                unc[i] = true;
                cmax[i] = cs.scmax + bb;                    /* choice is monotone in logit */
            }
        }
    }
    __syncthreads();
    for (int round = 0; round <= n_experts; round++) {
        /* Selection keys: (order-preserving bits of the choice, ~expert) as one 64-bit
         * integer, so that "larger choice, then lower index" is a plain unsigned max; a
         * choice that is not > -inf (NaN, -inf) is the key 0 and is never selected. */
        uint64_t key[SL];
#pragma unroll
        for (int i = 0; i < SL; i++) {
            const int e = tid + nthr * i;
            csh[min(e, RF_MAXE - 1)] = e < n_experts ? c[i] : 0.0f;
            ssh[min(e, RF_MAXE - 1)] = e < n_experts ? sc[i] : 0.0f;
            key[i] = (e < n_experts && c[i] > -INFINITY)
                         ? ((uint64_t)choice_order(c[i]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)e)
                         : 0ull;
        }
        /* 1. each wave extracts its topk largest keys, largest first (topk rounds of a
         *    wave max; a key taken is zeroed); 2. wave 0 does the same over the waves'
         *    candidates. Keys are distinct (the expert index is part of the key). */
        for (int j = 0; j < topk; j++) {
            uint64_t b = key[0];
#pragma unroll
            for (int i = 1; i < SL; i++) b = b > key[i] ? b : key[i];
            const uint64_t m = wave_max_key(b);
#pragma unroll
            for (int i = 0; i < SL; i++)
                if (key[i] == m) key[i] = 0ull;
            if (lane == 0) candk[wv][j] = m;
        }
        __syncthreads();
        if (wv == 0) {
            const int ncand = nw * topk;
            if (ncand <= 64) {
                uint64_t mk = lane < ncand ? candk[lane / topk][lane % topk] : 0ull;
                for (int j = 0; j < topk; j++) {
                    const uint64_t m = wave_max_key(mk);
                    if (mk == m) mk = 0ull;
                    if (lane == 0) selk[j] = m;
                }
            } else {
                uint64_t mk[RF_MAXW];
#pragma unroll
                for (int q = 0; q < RF_MAXW; q++) {
                    const int ci = lane + 64 * q;
                    mk[q] = ci < ncand ? candk[ci / topk][ci % topk] : 0ull;
                }
                for (int j = 0; j < topk; j++) {
                    uint64_t b = 0ull;
#pragma unroll
                    for (int q = 0; q < RF_MAXW; q++) b = b > mk[q] ? b : mk[q];
                    const uint64_t m = wave_max_key(b);
#pragma unroll
                    for (int q = 0; q < RF_MAXW; q++)
                        if (mk[q] == m) mk[q] = 0ull;
                    if (lane == 0) selk[j] = m;
                }
            }
        }
        __syncthreads();
        bool sel[SL];
#pragma unroll
        for (int i = 0; i < SL; i++) sel[i] = false;
        int nsel = 0;
        float ckth = -INFINITY;
        for (int j = 0; j < topk; j++) {
            const uint64_t kj = selk[j];
            if (kj != 0ull) {
                const int id = (int)(0xffffffffu - (uint32_t)kj);
                nsel++;
                ckth = csh[id];
#pragma unroll
                for (int i = 0; i < SL; i++)
                    if (id == tid + nthr * i) sel[i] = true;
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
        const uint64_t kj = lane < topk ? selk[lane] : 0ull;
        const int id = kj != 0ull ? (int)(0xffffffffu - (uint32_t)kj) : -1;
        float w = id >= 0 ? ssh[id] : 0.0f;
        if (renorm && topk > 1) {
            double s = 0.0;
            for (int j = 0; j < topk; j++) s += (double)__shfl(w, j, 64);   /* j ascending */
            const float inv = (float)(1.0 / (s + 1e-20));
            w = w * inv;
        }
        if (lane < topk) {
            idx[(size_t)t * topk + lane] = id >= 0 ? id : 0;
            wt[(size_t)t * topk + lane] = w * routed_scale;
        }
        if (nrecomp && lane == 0) nrecomp[t] = nre_sh;
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
__device__ __forceinline__ int block_scan_excl(int v, int *wtot, int lane, int wv, int &total)
{
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) wtot[wv] = x;
    __syncthreads();
    int base = 0;
    total = 0;
    for (int w = 0; w < 16; w++) {
        const int tw = wtot[w];
        if (w < wv) base += tw;
        total += tw;
    }
    __syncthreads();
    return base + x - v;
}

__global__ __launch_bounds__(1024) void gather_kernel(int *offsets, int *perm, int *job_expert,
                                                      int *job_off, int *job_cnt, int *pass_job,
                                                      int *pass_tp, int *counts, const int *idx,
                                                      int N, int n_experts, const void *bank,
                                                      int pass_tok)
{
    __shared__ int cnt[G_MAXE];
    __shared__ int fill[G_MAXE];
    __shared__ int wtot[16];
    __shared__ unsigned short wcnt[16][G_WCNT_E];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    for (int e = tid; e < n_experts; e += 1024) cnt[e] = 0;
    __syncthreads();
    for (int a = tid; a < N; a += 1024) {
        const int e = idx[a];
        if (e >= 0 && e < n_experts) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();

    /* per-thread sums over a contiguous expert range, then workgroup scans */
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
    int tot_a, tot_b, tot_c, tot_d;
    int run = block_scan_excl(local, wtot, lane, wv, tot_a);
    int jrun = block_scan_excl(ljobs, wtot, lane, wv, tot_b);
    int prun = block_scan_excl(lpass, wtot, lane, wv, tot_c);
    (void)block_scan_excl(ldrop, wtot, lane, wv, tot_d);
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
    if (tid == 0) {
        offsets[n_experts] = tot_a;
        counts[0] = tot_b;
        counts[1] = tot_c;
        counts[2] = tot_d;
    }
    __syncthreads();

    /* stable placement */
    const bool wide = n_experts > G_WCNT_E;
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

/* ---- combine: out[t] = 0 + sum_j wt[t][j] * contrib[t*topk + j], j ascending -------
 * A slot contributes nothing when its expert index is out of range or its bank entry is
 * absent. Every slot's row is loaded (it is valid memory either way) and the sum selects,
 * so that all topk loads are in flight together. */
__global__ __launch_bounds__(256) void combine_kernel(float *out, const float *contrib,
                                                     const float *wt, const int *idx,
                                                     const void *bank, int n_experts, int T,
                                                     int topk, int E, int vec)
{
    __shared__ float wsl[K3_MAX_TOPK_DEV];
    __shared__ int vsl[K3_MAX_TOPK_DEV];
    const int t = blockIdx.y;
    if (threadIdx.x < topk) {
        const int a = t * topk + threadIdx.x;
        const int e = idx[a];
        const bool ok = e >= 0 && e < n_experts && (!bank || expert_present(bank, e));
        vsl[threadIdx.x] = ok;
        wsl[threadIdx.x] = wt[a];
    }
    __syncthreads();
    const int i = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= E) return;
    const float *c0 = contrib + (size_t)t * topk * E + i;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    constexpr int JB = 8;
    for (int j0 = 0; j0 < topk; j0 += JB) {
        float cv[JB][4];
#pragma unroll
        for (int jj = 0; jj < JB; jj++) {
            const int j = min(j0 + jj, topk - 1);
            const float *c = c0 + (size_t)j * E;
            if (vec) {
                const float4 v = *reinterpret_cast<const float4 *>(c);
                cv[jj][0] = v.x; cv[jj][1] = v.y; cv[jj][2] = v.z; cv[jj][3] = v.w;
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++) cv[jj][q] = i + q < E ? c[q] : 0.0f;
            }
        }
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
    if (vec) *reinterpret_cast<float4 *>(o) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    else
        for (int q = 0; q < 4; q++)
            if (i + q < E) o[q] = acc[q];
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
    if (T <= RS_T) return RS_CH;          /* one lane per (expert, 128-column chunk) */
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

/* Up to RS_T tokens and 64 chunks of RS_CH columns whose staged rows fit in LDS beside
 * the kernel's own 45 KB: router_small_kernel certifies and scores the logits itself, and
 * the final kernel starts from its records. */
constexpr size_t RS_LDS_DYN = 160 * 1024 - 45 * 1024;

static bool router_small_mode(int T, int hidden)
{
    const size_t ks = (size_t)(hidden + RS_CH - 1) / RS_CH;
    return T <= RS_T && ks <= 64 && (size_t)T * ks * RS_CH * 4 <= RS_LDS_DYN;
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
                                  const K3kExc *exc, void *stream)
{
    if (T <= 0 || n_experts <= 0) return 0;
    if (chunk <= 0 || chunk % RP_KS) return k3k_fail("router_partial: chunk", hipErrorInvalidValue);
    const int ks = (hidden + chunk - 1) / chunk;
    const int vec = (hidden % 4 == 0) && ((((uintptr_t)x) | ((uintptr_t)W)) % 16 == 0);
    hipStream_t st = (hipStream_t)stream;
    if (router_small_mode(T, hidden)) {
        if (chunk != RS_CH) return k3k_fail("router_partial: chunk", hipErrorInvalidValue);
        const size_t lds = (size_t)T * ks * RS_CH * 4;
        const ExcTable e = exc_view(exc);
        float4 *pre = reinterpret_cast<float4 *>(part);
        const dim3 grid((n_experts + 3) / 4);
        if (T == 1) {
            hipLaunchKernelGGL(router_small_kernel<1>, grid, dim3(256), lds, st, pre, x, T, W, hidden,
                               n_experts, vec, e);
        } else {
            static bool attr = false;
            if (!attr) {
                (void)hipFuncSetAttribute(reinterpret_cast<const void *>(router_small_kernel<RS_T>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)RS_LDS_DYN);
                attr = true;
            }
            hipLaunchKernelGGL(router_small_kernel<RS_T>, grid, dim3(256), lds, st, pre, x, T, W,
                               hidden, n_experts, vec, e);
        }
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
    const ExcTable e = exc_view(exc);
    const int ks = (hidden + chunk - 1) / chunk;
    int nw = (n_experts + 63) / 64;
    if (nw > RF_MAXW) nw = RF_MAXW;
    hipStream_t st = (hipStream_t)stream;
    /* scored records (a few tokens), else the chunk partials: for up to 64 tokens and 512
     * experts (<= 8 waves) in one batch of up to 64 loads (more registers, fewer waves per
     * CU: only while the tokens do not fill the chip) */
    const bool pre = router_small_mode(T, hidden);
    if (pre && n_experts <= 64 * RF_MAXW)
        hipLaunchKernelGGL((router_final_kernel<1, RF_KB, true>), dim3(T), dim3(64 * nw), 0, st, idx, wt,
                           nrecomp, part, rbound, ks, chunk, x, W, bias, T, hidden, n_experts, topk,
                           renorm, routed_scale, e);
    else if (pre)
        hipLaunchKernelGGL((router_final_kernel<2, RF_KB, true>), dim3(T), dim3(64 * nw), 0, st, idx, wt,
                           nrecomp, part, rbound, ks, chunk, x, W, bias, T, hidden, n_experts, topk,
                           renorm, routed_scale, e);
    else if (n_experts <= 512 && ks <= 64 && T <= 64)
        hipLaunchKernelGGL((router_final_kernel<1, 64, false>), dim3(T), dim3(64 * nw), 0, st, idx, wt,
                           nrecomp, part, rbound, ks, chunk, x, W, bias, T, hidden, n_experts, topk,
                           renorm, routed_scale, e);
    else if (n_experts <= 64 * RF_MAXW)
        hipLaunchKernelGGL((router_final_kernel<1, RF_KB, false>), dim3(T), dim3(64 * nw), 0, st, idx, wt,
                           nrecomp, part, rbound, ks, chunk, x, W, bias, T, hidden, n_experts, topk,
                           renorm, routed_scale, e);
    else
        hipLaunchKernelGGL((router_final_kernel<2, RF_KB, false>), dim3(T), dim3(64 * nw), 0, st, idx, wt,
                           nrecomp, part, rbound, ks, chunk, x, W, bias, T, hidden, n_experts, topk,
                           renorm, routed_scale, e);
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
    if (topk > K3_MAX_TOPK_DEV) return k3k_fail("combine: topk too large", hipErrorInvalidValue);
    const int vec = (E % 4 == 0) && ((((uintptr_t)out) | ((uintptr_t)contrib)) % 16 == 0);
    dim3 grid(((E + 3) / 4 + 255) / 256, T);
    hipLaunchKernelGGL(combine_kernel, grid, dim3(256), 0, (hipStream_t)stream, out, contrib, wt,
                       idx, bank, n_experts, T, topk, E, vec);
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
