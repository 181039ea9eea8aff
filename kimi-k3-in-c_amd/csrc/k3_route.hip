/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_route.hip -- the routing side of the MoE layer on gfx950: activation split, the
 * sigmoid top-k router, the expert-major gather, the weighted combine, and the small
 * elementwise kernels (activation, RMSNorm).
 */
#include "k3_common.h"
#include "k3_expf.h"
#include "k3k.h"

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

/* ---- router logits ------------------------------------------------------------------
 * part[ks][t][e] = sum over the ks-th K chunk of (double)W[e][k] * (double)x[t][k],
 * accumulated with fp64 fma in ascending k. A product of two floats is exact in fp64, so
 * each fma equals the reference's separate multiply and add (k3_ops.c:449-450); only the
 * grouping of the 7168-term sum differs from the reference's single ascending chain.
 * Workgroup tile: 64 experts x 16 tokens; each thread one expert x 4 tokens. */
constexpr int RT_E = 64, RT_T = 16, RT_K = 64;

__global__ __launch_bounds__(256) void router_partial_kernel(double *part, const float *x, int T,
                                                             const float *W, int hidden,
                                                             int n_experts, int ksplit)
{
    __shared__ float ws[RT_E][RT_K + 1];
    __shared__ float xs[RT_T][RT_K];
    const int e0 = blockIdx.x * RT_E, t0 = blockIdx.y * RT_T, ks = blockIdx.z;
    const int kc = (hidden + ksplit - 1) / ksplit;
    const int k0 = ks * kc, k1 = min(hidden, k0 + kc);
    const int tid = threadIdx.x, el = tid & 63, tg = tid >> 6;
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (int kb = k0; kb < k1; kb += RT_K) {
        for (int i = tid; i < RT_E * RT_K; i += 256) {
            const int r = i / RT_K, c = i % RT_K;
            const int e = e0 + r, k = kb + c;
            ws[r][c] = (e < n_experts && k < k1) ? W[(size_t)e * hidden + k] : 0.0f;
        }
        for (int i = tid; i < RT_T * RT_K; i += 256) {
            const int r = i / RT_K, c = i % RT_K;
            const int t = t0 + r, k = kb + c;
            xs[r][c] = (t < T && k < k1) ? x[(size_t)t * hidden + k] : 0.0f;
        }
        __syncthreads();
        const int kn = min(RT_K, k1 - kb);
        for (int k = 0; k < kn; k++) {
            const double w = (double)ws[el][k];
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] = fma(w, (double)xs[tg * 4 + i][k], acc[i]);
        }
        __syncthreads();
    }
    const int e = e0 + el;
    if (e < n_experts)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = t0 + tg * 4 + i;
            if (t < T) part[((size_t)ks * T + t) * n_experts + e] = acc[i];
        }
}

/* libm-exact router score 1/(1+expf(v)) for v = -logit: the deterministic candidate,
 * overridden where host libm's expf gives a different score (table built at build time:
 * sorted (key bits, libm expf bits) pairs, binary searched). */
__device__ __forceinline__ float router_score(float logit, const uint32_t *exc, int n_exc)
{
    const float v = -logit;
    float E = k3_expf_det(v);
    if (n_exc > 0) {
        const uint32_t key = __float_as_uint(v);
        int lo = 0, hi = n_exc;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            const uint32_t k = exc[2 * mid];
            if (k < key) lo = mid + 1;
            else hi = mid;
        }
        if (lo < n_exc && exc[2 * lo] == key) E = __uint_as_float(exc[2 * lo + 1]);
    }
    return 1.0f / (1.0f + E);
}

/* One workgroup per token: logits (partials summed in ascending chunk order, rounded to
 * fp32), score, biased choice, then topk rounds of "largest choice, lowest index among
 * equals, strictly above -inf" exactly as the reference's first-strict-max scan
 * (k3_ops.c:459-467), then renormalisation and scaling (k3_ops.c:469-475). */
constexpr int RF_MAXE = 2048;

__global__ __launch_bounds__(256) void router_final_kernel(int *idx, float *wt, int *nrecomp,
                                                           const double *part, int ksplit,
                                                           const float *bias, int T,
                                                           int n_experts, int topk, int renorm,
                                                           float routed_scale,
                                                           const uint32_t *exc, int n_exc)
{
    __shared__ float score[RF_MAXE];
    __shared__ float choice[RF_MAXE];
    __shared__ float rv[256];
    __shared__ int ri[256];
    __shared__ float wsel[K3_MAX_TOPK_DEV];
    const int t = blockIdx.x, tid = threadIdx.x;
    for (int e = tid; e < n_experts; e += 256) {
        double s = 0.0;
        for (int ks = 0; ks < ksplit; ks++) s += part[((size_t)ks * T + t) * n_experts + e];
        const float sc = router_score((float)s, exc, n_exc);
        score[e] = sc;
        choice[e] = sc + (bias ? bias[e] : 0.0f);
    }
    __syncthreads();
    for (int j = 0; j < topk; j++) {
        float bv = -INFINITY;
        int bi = -1;
        for (int e = tid; e < n_experts; e += 256) {
            const float c = choice[e];
            if (c > bv) { bv = c; bi = e; }           /* ascending e: first strict max */
        }
        rv[tid] = bv;
        ri[tid] = bi;
        __syncthreads();
        for (int s = 128; s > 0; s >>= 1) {
            if (tid < s) {
                const float ov = rv[tid + s];
                const int oi = ri[tid + s];
                /* keep the larger value; among equal values the lower index */
                if (oi >= 0 && (ri[tid] < 0 || ov > rv[tid] || (ov == rv[tid] && oi < ri[tid]))) {
                    rv[tid] = ov;
                    ri[tid] = oi;
                }
            }
            __syncthreads();
        }
        if (tid == 0) {
            const int best = ri[0];
            if (best < 0) {
                idx[(size_t)t * topk + j] = 0;
                wsel[j] = 0.0f;
            } else {
                idx[(size_t)t * topk + j] = best;
                wsel[j] = score[best];
                choice[best] = -INFINITY;
            }
        }
        __syncthreads();
    }
    if (tid == 0) {
        if (renorm && topk > 1) {
            double s = 0.0;
            for (int j = 0; j < topk; j++) s += (double)wsel[j];
            const float inv = (float)(1.0 / (s + 1e-20));
            for (int j = 0; j < topk; j++) wsel[j] = wsel[j] * inv;
        }
        for (int j = 0; j < topk; j++) wt[(size_t)t * topk + j] = wsel[j] * routed_scale;
        if (nrecomp) nrecomp[t] = 0;
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

extern "C" int k3k_router_partial(double *part, const float *x, int T, const float *W, int hidden,
                                  int n_experts, int ksplit, void *stream)
{
    if (T <= 0) return 0;
    dim3 grid((n_experts + RT_E - 1) / RT_E, (T + RT_T - 1) / RT_T, ksplit);
    hipLaunchKernelGGL(router_partial_kernel, grid, dim3(256), 0, (hipStream_t)stream, part, x, T,
                       W, hidden, n_experts, ksplit);
    K3K_LAUNCH_CHECK("router_partial launch");
    return 0;
}

extern "C" int k3k_router_final(int *idx, float *wt, int *nrecomp, const double *part, int ksplit,
                                const float *x, const float *W, const float *bias, int T,
                                int hidden, int n_experts, int topk, int renorm,
                                float routed_scale, const uint32_t *exc, int n_exc, void *stream)
{
    (void)x;
    (void)W;
    (void)hidden;
    if (T <= 0) return 0;
    if (n_experts > RF_MAXE || topk > K3_MAX_TOPK_DEV)
        return k3k_fail("router_final: n_experts or topk too large", hipErrorInvalidValue);
    hipLaunchKernelGGL(router_final_kernel, dim3(T), dim3(256), 0, (hipStream_t)stream, idx, wt,
                       nrecomp, part, ksplit, bias, T, n_experts, topk, renorm, routed_scale, exc,
                       n_exc);
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
