/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_oracle.c -- CPU restatement of the reference's routed-MoE hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see k3_oracle.h). Written for this project from the
 * reference's documented arithmetic; each function names the reference lines whose
 * operation order it reproduces. Build with -ffp-contract=off and without -ffast-math,
 * as the reference requires (Makefile:132-139 of the reference): every fma() below is an
 * explicit single rounding and every other operation rounds on its own.
 */
#include "k3_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int orc_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------ tables ---- */
/* OCP MX E2M1 by 4-bit code, bit 3 the sign (k3_ops.c:1066-1069). Code 8 is -0.0. */
static const float E2M1[16] = {
    0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
    -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f,
};

/* E8M0 byte -> 2^(b-127), with the NaN byte 255 read as 0 (k3_ops.c:1335-1339). The
 * value for b = 0 is the fp32 subnormal 2^-127, exact. */
static float e8m0(unsigned b)
{
    return b == 255u ? 0.0f : ldexpf(1.0f, (int)b - 127);
}

static void fatal(const char *msg, int v)
{
    fprintf(stderr, "k3 oracle: FATAL, %s (%d)\n", msg, v);
    abort();
}

/* ----------------------------------------------------------------- dequant ---- */
/* k3_ops.c:1787-1817: out[r][i] = E2M1[nibble] * 2^(s-127), the low nibble of each byte
 * the even element, scale byte 255 -> 0. Exact: no rounding anywhere. */
void orc_mxfp4_dequant(float *out, const unsigned char *packed, const unsigned char *scales,
                       int rows, int pcols, int group)
{
    const int width = pcols * 2;
    const int ngrp = (width + group - 1) / group;
    for (int r = 0; r < rows; r++) {
        const unsigned char *pr = packed + (size_t)r * pcols;
        const unsigned char *sr = scales + (size_t)r * ngrp;
        float *o = out + (size_t)r * width;
        for (int i = 0; i < width; i++) {
            const unsigned b = pr[i >> 1];
            const unsigned code = (i & 1) ? (b >> 4) : (b & 15u);
            o[i] = E2M1[code] * e8m0(sr[i / group]);
        }
    }
}

/* ------------------------------------------------------------ MXFP4 GEMV ---- */
/* One row on the reference's AVX2 flat-row path (k3_ops.c:1435-1532), taken whenever
 * group is a multiple of 16. The scale is folded into each E2M1 weight in fp32 (exact:
 * a 3-bit mantissa times a power of two), element i of each 16-element chunk feeds
 * double lane i%16 through fma, a chunk whose scale byte is 255 is skipped entirely, and
 * the lanes reduce as q[m] = (l[m]+l[8+m]) + (l[4+m]+l[12+m]), then (q0+q2)+(q1+q3).
 * Remaining elements (in % 16) are fma'd one at a time, scale folded the same way and
 * NOT skipped for byte 255 (their weight is then +-0). */
static double row_flat(const unsigned char *pr, const unsigned char *sr, const double *xd,
                       int in, int group)
{
    double l[16];
    for (int k = 0; k < 16; k++) l[k] = 0.0;
    const int cpg = group >> 4;
    int i = 0, g = 0, c = 0;
    for (; i + 15 < in; i += 16) {
        const unsigned sb = sr[g];
        if (sb != 255u) {
            const float sc = e8m0(sb);
            const unsigned char *pb = pr + (i >> 1);
            double w[16];
            for (int k = 0; k < 8; k++) {
                w[2 * k]     = (double)(E2M1[pb[k] & 15u] * sc);
                w[2 * k + 1] = (double)(E2M1[pb[k] >> 4] * sc);
            }
            for (int k = 0; k < 16; k++) l[k] = fma(w[k], xd[i + k], l[k]);
        }
        if (++c == cpg) { c = 0; g++; }
    }
    double q[4];
    for (int m = 0; m < 4; m++) q[m] = (l[m] + l[8 + m]) + (l[4 + m] + l[12 + m]);
    double acc = (q[0] + q[2]) + (q[1] + q[3]);
    for (; i < in; i++) {
        const unsigned b = pr[i >> 1];
        const unsigned code = (i & 1) ? (b >> 4) : (b & 15u);
        acc = fma((double)(E2M1[code] * e8m0(sr[i / group])), xd[i], acc);
    }
    return acc;
}

/* One row on the reference's AVX2 grouped path (k3_ops.c:1534-1781), taken when group is
 * not a multiple of 16. Per group (skipped when its scale byte is 255): unscaled E2M1
 * weights, 16-element chunks into four 4-lane double accumulators v0..v3 (element k of
 * the chunk into v[k/4] lane k%4), then at most one 8-element chunk into v0, v1, then
 * a[m] = (v0[m]+v2[m]) + (v1[m]+v3[m]), sub = (a0+a1)+(a2+a3), then a scalar fma tail;
 * finally acc += sub * 2^(s-127), the product exact in double. */
static double row_grouped(const unsigned char *pr, const unsigned char *sr, const double *xd,
                          int in, int group)
{
    const int ngrp = (in + group - 1) / group;
    const int gbyte = group / 2;
    double acc = 0.0;
    for (int g = 0; g < ngrp; g++) {
        const unsigned sb = sr[g];
        if (sb == 255u) continue;
        const unsigned char *pb = pr + (size_t)g * gbyte;
        const double *xg = xd + (size_t)g * group;
        int n = in - g * group;
        if (n > group) n = group;
        double v[4][4];
        for (int a = 0; a < 4; a++)
            for (int b = 0; b < 4; b++) v[a][b] = 0.0;
        int i = 0;
        for (; i + 15 < n; i += 16)
            for (int k = 0; k < 16; k++) {
                const unsigned b = pb[(i + k) >> 1];
                const unsigned code = (k & 1) ? (b >> 4) : (b & 15u);
                v[k >> 2][k & 3] = fma((double)E2M1[code], xg[i + k], v[k >> 2][k & 3]);
            }
        for (; i + 7 < n; i += 8)
            for (int k = 0; k < 8; k++) {
                const unsigned b = pb[(i + k) >> 1];
                const unsigned code = (k & 1) ? (b >> 4) : (b & 15u);
                v[k >> 2][k & 3] = fma((double)E2M1[code], xg[i + k], v[k >> 2][k & 3]);
            }
        double a[4];
        for (int m = 0; m < 4; m++) a[m] = (v[0][m] + v[2][m]) + (v[1][m] + v[3][m]);
        double sub = (a[0] + a[1]) + (a[2] + a[3]);
        for (; i < n; i++) {
            const unsigned b = pb[i >> 1];
            sub = fma((double)E2M1[(i & 1) ? (b >> 4) : (b & 15u)], xg[i], sub);
        }
        acc += sub * (double)e8m0(sb);
    }
    return acc;
}

/* k3_ops.c:1380-1785. Preconditions abort exactly where the reference's do (:1383-1401). */
void orc_matmul_mxfp4(float *y, const float *x, const unsigned char *packed,
                      const unsigned char *scales, int in, int rows, int group)
{
    if (in & 1) fatal("k3_matmul_mxfp4 called with odd in", in);
    if (group > 64) fatal("k3_matmul_mxfp4 called with group > 64", group);
    const int pcols = in / 2;
    const int ngrp = (in + group - 1) / group;
    double *xd = (double *)malloc((size_t)(in > 0 ? in : 1) * sizeof(double));
    if (!xd) fatal("oracle allocation", in);
    for (int i = 0; i < in; i++) xd[i] = (double)x[i];
    const int flat = (group & 15) == 0;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (rows > 64)
#endif
    for (int r = 0; r < rows; r++) {
        const unsigned char *pr = packed + (size_t)r * pcols;
        const unsigned char *sr = scales + (size_t)r * ngrp;
        const double acc = flat ? row_flat(pr, sr, xd, in, group)
                                : row_grouped(pr, sr, xd, in, group);
        y[r] = (float)acc;
    }
    free(xd);
}

/* ------------------------------------------------------------- fp32 / bf16 ---- */
/* k3_ops.c:265-291 and 1108-1213: sixteen double accumulators, element i into i%16 via
 * fma, b_m = (a[m]+a[m+4]) + (a[m+8]+a[m+12]), acc = (b0+b1)+(b2+b3), fma tail. The bf16
 * kernel is the same arithmetic on weights widened by a 16-bit shift, so the two agree
 * bit for bit (test_ops.c:798-848 of the reference asserts it). */
static inline float bf16f(uint16_t h)
{
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static double dot16_f32(const float *row, const float *x, int in)
{
    double a[16];
    for (int k = 0; k < 16; k++) a[k] = 0.0;
    int i = 0;
    for (; i + 15 < in; i += 16)
        for (int k = 0; k < 16; k++) a[k] = fma((double)row[i + k], (double)x[i + k], a[k]);
    double b[4];
    for (int m = 0; m < 4; m++) b[m] = (a[m] + a[m + 4]) + (a[m + 8] + a[m + 12]);
    double acc = (b[0] + b[1]) + (b[2] + b[3]);
    for (; i < in; i++) acc = fma((double)row[i], (double)x[i], acc);
    return acc;
}

static double dot16_bf16(const uint16_t *row, const float *x, int in)
{
    double a[16];
    for (int k = 0; k < 16; k++) a[k] = 0.0;
    int i = 0;
    for (; i + 15 < in; i += 16)
        for (int k = 0; k < 16; k++)
            a[k] = fma((double)bf16f(row[i + k]), (double)x[i + k], a[k]);
    double b[4];
    for (int m = 0; m < 4; m++) b[m] = (a[m] + a[m + 4]) + (a[m + 8] + a[m + 12]);
    double acc = (b[0] + b[1]) + (b[2] + b[3]);
    for (; i < in; i++) acc = fma((double)bf16f(row[i]), (double)x[i], acc);
    return acc;
}

void orc_matmul(float *y, const float *x, const float *W, int in, int out)
{
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (out > 64)
#endif
    for (int o = 0; o < out; o++) y[o] = (float)dot16_f32(W + (size_t)o * in, x, in);
}

void orc_matmul_bf16(float *y, const float *x, const uint16_t *W, int in, int out)
{
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (out > 64)
#endif
    for (int o = 0; o < out; o++) y[o] = (float)dot16_bf16(W + (size_t)o * in, x, in);
}

/* ------------------------------------------------------------------ router ---- */
static inline float sigmoid_ref(float v) { return 1.0f / (1.0f + expf(-v)); }

/* k3_ops.c:419-478. Logit = sequential double sum of (double)W*(double)x (a separate
 * multiply and add: -ffp-contract=off), score = 1/(1+expf(-(float)logit)),
 * choice = score + bias. top-k = k rounds of strict first-max over ascending e with the
 * taken entry set to -inf (ties to the lowest index; no candidate -> idx 0, w 0).
 * Weights are the UNBIASED scores, renormalised by (float)(1/(sum_double + 1e-20)) when
 * renorm && topk > 1, then scaled. */
void orc_router(int *idx, float *w, const float *x, const float *W, const float *bias,
                int hidden, int n_experts, int topk, int renorm, float routed_scale)
{
    float *score = (float *)malloc((size_t)n_experts * sizeof(float));
    float *choice = (float *)malloc((size_t)n_experts * sizeof(float));
    if (!score || !choice) fatal("oracle allocation", n_experts);
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (n_experts > 64)
#endif
    for (int e = 0; e < n_experts; e++) {
        const float *row = W + (size_t)e * hidden;
        double acc = 0.0;
        for (int i = 0; i < hidden; i++) {
            const double p = (double)row[i] * (double)x[i];
            acc = acc + p;
        }
        score[e] = sigmoid_ref((float)acc);
        choice[e] = score[e] + (bias ? bias[e] : 0.0f);
    }
    for (int j = 0; j < topk; j++) {
        int best = -1;
        float bv = -INFINITY;
        for (int e = 0; e < n_experts; e++)
            if (choice[e] > bv) { bv = choice[e]; best = e; }
        if (best < 0) { idx[j] = 0; w[j] = 0.0f; continue; }
        idx[j] = best;
        w[j] = score[best];
        choice[best] = -INFINITY;
    }
    if (renorm && topk > 1) {
        double s = 0.0;
        for (int j = 0; j < topk; j++) s += (double)w[j];
        const float inv = (float)(1.0 / (s + 1e-20));
        for (int j = 0; j < topk; j++) w[j] *= inv;
    }
    for (int j = 0; j < topk; j++) w[j] *= routed_scale;
    free(score);
    free(choice);
}

/* -------------------------------------------------------------- activations ---- */
/* k3_ops.c:110-123: a = b1*tanhf(g/b1)*sigmoid(g) (the sigmoid sees the uncapped gate),
 * u = b2*tanhf(up/b2), y = a*u, evaluated left to right in float. */
void orc_situ_glu(float *y, const float *x, int n, float b1, float b2)
{
    for (int i = 0; i < n; i++) {
        const float g = x[i];
        const float a = b1 * tanhf(g / b1) * sigmoid_ref(g);
        const float u = b2 * tanhf(x[n + i] / b2);
        y[i] = a * u;
    }
}

/* SiLU(gate)*up in the reference's own SiLU form, acc*sigmoidf_(acc) (k3_ops.c:160,105):
 * y = (g * sigmoid(g)) * u in float. */
void orc_silu_glu(float *y, const float *x, int n)
{
    for (int i = 0; i < n; i++) {
        const float g = x[i];
        const float a = g * sigmoid_ref(g);
        y[i] = a * x[n + i];
    }
}

/* k3_ops.c:94-102. */
void orc_rmsnorm(float *y, const float *x, const float *w, int n, float eps)
{
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
    const float inv = (float)(1.0 / sqrt(ss / (double)n + (double)eps));
    for (int i = 0; i < n; i++) y[i] = w[i] * x[i] * inv;
}

/* ---------------------------------------------------------------- experts ---- */
static void act_apply(float *y, const float *gu, int n, int act, float b1, float b2)
{
    if (act == ORC_ACT_SILU) orc_silu_glu(y, gu, n);
    else orc_situ_glu(y, gu, n, b1, b2);
}

void orc_expert_ffn(float *out, const float *x, const OrcExpertQ *q, int hidden, int inter,
                    int act, float b1, float b2, float wt)
{
    float *gu = (float *)malloc((size_t)3 * inter * sizeof(float));
    float *dn = (float *)malloc((size_t)hidden * sizeof(float));
    if (!gu || !dn) fatal("oracle allocation", hidden);
    float *a = gu + 2 * inter;
    orc_matmul_mxfp4(gu, x, q->p1, q->s1, hidden, inter, 32);
    orc_matmul_mxfp4(gu + inter, x, q->p3, q->s3, hidden, inter, 32);
    act_apply(a, gu, inter, act, b1, b2);
    orc_matmul_mxfp4(dn, a, q->p2, q->s2, inter, hidden, 32);
    for (int i = 0; i < hidden; i++) out[i] = 0.0f + wt * dn[i];
    free(gu);
    free(dn);
}

/* orc_expert_ffn for n tokens of one expert, expert-major (the reference's prefill order,
 * k3_ops.c:742-794): each matrix is dequantized once (orc_mxfp4_dequant: E2M1 x 2^(s-127)
 * folded in fp32, exact, byte 255 -> 0) and every weight row is dotted against all n
 * tokens while it is in cache, out[t] = down(act(gate x_t, up x_t)) with no combine
 * weight. The dot product is dot16_f32: fp64 fma into 16 lanes by element index mod 16,
 * then the reduction (l[m]+l[8+m])+(l[4+m]+l[12+m]) and (q0+q2)+(q1+q3), the operation
 * order of row_flat (the reference's flat-row path, k3_ops.c:1435-1532); with every scale
 * byte below 255, or finite activations, the products and sums are those of
 * orc_matmul_mxfp4 (a skipped chunk adds nothing, a zero weight adds +-0), so each output
 * equals orc_expert_ffn's. Test helper for full batch sizes: it is the per-token oracle
 * reordered, and the tests check the two against each other. */
#define FM_R 8       /* rows and tokens per cache tile */
#define FM_T 16

void orc_expert_ffn_many(float *out, const float *x, int n, const OrcExpertQ *q, int hidden,
                         int inter, int act, float b1, float b2)
{
    const size_t big = (size_t)hidden * inter;
    float *w = (float *)malloc(big * sizeof(float));
    float *gu = (float *)malloc((size_t)n * 2 * inter * sizeof(float));
    float *a = (float *)malloc((size_t)n * inter * sizeof(float));
    if (!w || !gu || !a) fatal("oracle allocation", n);
    for (int m = 0; m < 2; m++) {
        const unsigned char *pk = m == 0 ? q->p1 : q->p3, *sc = m == 0 ? q->s1 : q->s3;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
        for (int r = 0; r < inter; r++)
            orc_mxfp4_dequant(w + (size_t)r * hidden, pk + (size_t)r * (hidden / 2),
                              sc + (size_t)r * ((hidden + 31) / 32), 1, hidden / 2, 32);
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
        for (int r0 = 0; r0 < inter; r0 += FM_R)
            for (int t0 = 0; t0 < n; t0 += FM_T)          /* a tile of tokens stays in cache */
                for (int r = r0; r < r0 + FM_R && r < inter; r++)
                    for (int t = t0; t < t0 + FM_T && t < n; t++)
                        gu[(size_t)t * 2 * inter + (size_t)m * inter + r] =
                            (float)dot16_f32(w + (size_t)r * hidden, x + (size_t)t * hidden, hidden);
    }
    for (int t = 0; t < n; t++) act_apply(a + (size_t)t * inter, gu + (size_t)t * 2 * inter, inter, act, b1, b2);
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int r = 0; r < hidden; r++)
        orc_mxfp4_dequant(w + (size_t)r * inter, q->p2 + (size_t)r * (inter / 2),
                          q->s2 + (size_t)r * ((inter + 31) / 32), 1, inter / 2, 32);
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int r0 = 0; r0 < hidden; r0 += FM_R)
        for (int t0 = 0; t0 < n; t0 += FM_T)
            for (int r = r0; r < r0 + FM_R && r < hidden; r++)
                for (int t = t0; t < t0 + FM_T && t < n; t++)
                    out[(size_t)t * hidden + r] =
                        (float)dot16_f32(w + (size_t)r * inter, a + (size_t)t * inter, inter);
    free(w);
    free(gu);
    free(a);
}

void orc_moe_routed(float *out, int *idx, float *wt, const float *x, int T,
                    const float *router_w, const float *bias, const OrcExpertQ *bank,
                    int hidden, int inter, int n_experts, int topk, int renorm,
                    float routed_scale, int act, float b1, float b2)
{
    const int E = hidden, I = inter;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) if (T > 1)
#endif
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * E;
        float *ot = out + (size_t)t * E;
        int *it = idx + (size_t)t * topk;
        float *wtt = wt + (size_t)t * topk;
        float *gu = (float *)malloc((size_t)(3 * I + E) * sizeof(float));
        if (!gu) fatal("oracle allocation", E);
        float *a = gu + 2 * I, *dn = a + I;
        orc_router(it, wtt, xt, router_w, bias, E, n_experts, topk, renorm, routed_scale);
        for (int i = 0; i < E; i++) ot[i] = 0.0f;
        for (int j = 0; j < topk; j++) {
            const OrcExpertQ *q = &bank[it[j]];
            orc_matmul_mxfp4(gu, xt, q->p1, q->s1, E, I, 32);
            orc_matmul_mxfp4(gu + I, xt, q->p3, q->s3, E, I, 32);
            act_apply(a, gu, I, act, b1, b2);
            orc_matmul_mxfp4(dn, a, q->p2, q->s2, I, E, 32);
            const float wj = wtt[j];
            for (int i = 0; i < E; i++) ot[i] += wj * dn[i];
        }
        free(gu);
    }
}

void orc_gather(int *offsets, int *perm, const int *idx, int T, int topk, int n_experts)
{
    for (int e = 0; e <= n_experts; e++) offsets[e] = 0;
    for (int a = 0; a < T * topk; a++) offsets[idx[a] + 1]++;
    for (int e = 0; e < n_experts; e++) offsets[e + 1] += offsets[e];
    int *fill = (int *)malloc((size_t)(n_experts > 0 ? n_experts : 1) * sizeof(int));
    if (!fill) fatal("oracle allocation", n_experts);
    for (int e = 0; e < n_experts; e++) fill[e] = offsets[e];
    for (int a = 0; a < T * topk; a++) perm[fill[idx[a]]++] = a;
    free(fill);
}

/* k3_ops.c:556-656 with src == NULL and fp32 weights: route on the full width, project
 * down to the latent, run the selected experts there (k3_matmul + SiTU-GLU), sum them
 * weighted in j order, RMSNorm the aggregate, project up, then add the unweighted shared
 * expert computed on the original input. */
void orc_moe_latent(float *out, const float *x, const OrcMoeW *w, const OrcMoeCfg *c, int T)
{
    const int E = c->hidden, L = c->latent, I = c->inter, SI = c->inter * c->n_shared;
    float *z = (float *)malloc((size_t)(2 * L + 3 * I + L + 3 * SI + E) * sizeof(float));
    int *idx = (int *)malloc((size_t)c->topk * sizeof(int));
    float *wt = (float *)malloc((size_t)c->topk * sizeof(float));
    if (!z || !idx || !wt) fatal("oracle allocation", E);
    float *accL = z + L, *gu = accL + L, *act = gu + 2 * I, *edn = act + I;
    float *sgu = edn + L, *sact = sgu + 2 * SI, *sdn = sact + SI;
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * E;
        float *ot = out + (size_t)t * E;
        orc_router(idx, wt, xt, w->gate, w->bias, E, c->n_experts, c->topk, c->renorm,
                   c->routed_scale);
        orc_matmul(z, xt, w->down, E, L);
        for (int i = 0; i < L; i++) accL[i] = 0.0f;
        for (int j = 0; j < c->topk; j++) {
            const float *e1 = w->w1 + (size_t)idx[j] * I * L;
            const float *e3 = w->w3 + (size_t)idx[j] * I * L;
            const float *e2 = w->w2 + (size_t)idx[j] * L * I;
            orc_matmul(gu, z, e1, L, I);
            orc_matmul(gu + I, z, e3, L, I);
            orc_situ_glu(act, gu, I, c->b1, c->b2);
            orc_matmul(edn, act, e2, I, L);
            const float wj = wt[j];
            for (int i = 0; i < L; i++) accL[i] += wj * edn[i];
        }
        if (c->latent_norm) orc_rmsnorm(accL, accL, w->latent_norm, L, c->rms_eps);
        orc_matmul(ot, accL, w->up, L, E);
        orc_matmul(sgu, xt, w->sh1, E, SI);
        orc_matmul(sgu + SI, xt, w->sh3, E, SI);
        orc_situ_glu(sact, sgu, SI, c->b1, c->b2);
        orc_matmul(sdn, sact, w->sh2, SI, E);
        for (int i = 0; i < E; i++) ot[i] += sdn[i];
    }
    free(z);
    free(idx);
    free(wt);
}

/* ------------------------------------------------- streamed MXFP4 LatentMoE ---- */
/* k3_mmw (include/k3/k3.h:289-295) for the two weight types the MoE tail uses here. */
static void mmw(float *y, const float *x, const void *W, int wdt, int in, int out)
{
    if (wdt == 1) orc_matmul_bf16(y, x, (const uint16_t *)W, in, out);
    else if (wdt == 0) orc_matmul(y, x, (const float *)W, in, out);
    else fatal("orc_moe_q: weight type not restated", wdt);
}

/* One (token, slot) of a streamed expert: gate/up out of MXFP4, SiTU, down
 * (k3_ops.c:628-631 and :788-791, identical arithmetic). */
static void expert_q(float *edn, const float *z, const OrcExpertQ *q, int L, int I,
                     float b1, float b2, float *gu, float *act)
{
    orc_matmul_mxfp4(gu, z, q->p1, q->s1, L, I, 32);
    orc_matmul_mxfp4(gu + I, z, q->p3, q->s3, L, I, 32);
    orc_situ_glu(act, gu, I, b1, b2);
    orc_matmul_mxfp4(edn, act, q->p2, q->s2, I, L, 32);
}

/* The tail shared by both forms (k3_ops.c:646-654 and :813-820): RMSNorm of the
 * aggregate, up-projection, then the shared expert on the original input added
 * unweighted. acc is modified in place. */
static void moe_tail(float *ot, float *acc, const float *xt, const OrcMoeQW *w,
                     const OrcMoeCfg *c, float *sgu, float *sact, float *sdn)
{
    const int E = c->hidden, L = c->latent, SI = c->inter * c->n_shared;
    if (c->latent_norm) orc_rmsnorm(acc, acc, w->latent_norm, L, c->rms_eps);
    mmw(ot, acc, w->up, w->wdt, L, E);
    mmw(sgu, xt, w->sh1, w->wdt, E, SI);
    mmw(sgu + SI, xt, w->sh3, w->wdt, E, SI);
    orc_situ_glu(sact, sgu, SI, c->b1, c->b2);
    mmw(sdn, sact, w->sh2, w->wdt, SI, E);
    for (int i = 0; i < E; i++) ot[i] += sdn[i];
}

typedef struct {
    float *z, *acc, *gu, *act, *edn, *sgu, *sact, *sdn;
} QScr;

static void qscr_alloc(QScr *s, const OrcMoeCfg *c)
{
    const int E = c->hidden, L = c->latent, I = c->inter, SI = c->inter * c->n_shared;
    float *p = (float *)malloc((size_t)(2 * L + 3 * I + L + 3 * SI + E) * sizeof(float));
    if (!p) fatal("oracle allocation", E);
    s->z = p;
    s->acc = s->z + L;
    s->gu = s->acc + L;
    s->act = s->gu + 2 * I;
    s->edn = s->act + I;
    s->sgu = s->edn + L;
    s->sact = s->sgu + 2 * SI;
    s->sdn = s->sact + SI;
}

/* k3_moe (k3_ops.c:556-656) with a streamed source, tokens one after another. idx/wt
 * are topk-wide and reused per token, so they end holding the last token's routing
 * (after the cache-only compaction, whose tail keeps the router's values). */
static void moe_q_tokens(float *out, const float *x, const OrcMoeQW *w, const OrcMoeCfg *c,
                         int T, int *idx, float *wt, long *drops)
{
    const int E = c->hidden, L = c->latent, I = c->inter, K = c->topk;
    OrcExpertSrc *src = w->src;
    QScr s;
    qscr_alloc(&s, c);
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * E;
        float *ot = out + (size_t)t * E;
        orc_router(idx, wt, xt, w->gate, w->bias, E, c->n_experts, K, c->renorm,
                   c->routed_scale);
        int nk = K;
        if (w->cache_only && src->resident) {
            int m = 0;
            float wsum = 0.0f;
            for (int j = 0; j < K; j++)
                if (src->resident(src, w->layer, idx[j], NULL)) {
                    idx[m] = idx[j];
                    wt[m] = wt[j];
                    wsum += wt[j];
                    m++;
                }
            nk = m;
            if (wsum > 0.0f)
                for (int j = 0; j < nk; j++) wt[j] /= wsum;
        }
        mmw(s.z, xt, w->down, w->wdt, E, L);
        for (int i = 0; i < L; i++) s.acc[i] = 0.0f;
        if (!w->cache_only && src->getmany) src->getmany(src, w->layer, idx, nk);
        for (int j = 0; j < nk; j++) {
            OrcExpertQ q;
            const int miss = w->cache_only ? !src->resident(src, w->layer, idx[j], &q)
                                           : (src->get(src, w->layer, idx[j], &q) != 0);
            if (miss) {
                if (!w->cache_only) (*drops)++;
                continue;
            }
            expert_q(s.edn, s.z, &q, L, I, c->b1, c->b2, s.gu, s.act);
            const float wj = wt[j];
            for (int i = 0; i < L; i++) s.acc[i] += wj * s.edn[i];
        }
        moe_tail(ot, s.acc, xt, w, c, s.sgu, s.sact, s.sdn);
    }
    free(s.z);
}

/* moe_prefill_chunk (k3_ops.c:717-825): route and down-project every token of the chunk,
 * list its unique experts in first-seen (t, j) order, fetch each once (a failed fetch is
 * one drop for the chunk and zeroes every slot it would have filled), compute every
 * (token, slot) of that expert into contrib, then per token sum contrib in slot order and
 * finish with the same tail as k3_moe. idx/wt are not written. */
static void moe_q_chunk(float *out, const float *x, const OrcMoeQW *w, const OrcMoeCfg *c,
                        int T, long *drops)
{
    const int E = c->hidden, L = c->latent, I = c->inter, K = c->topk, N = c->n_experts;
    OrcExpertSrc *src = w->src;
    int *ridx = (int *)malloc((size_t)T * K * sizeof(int));
    float *rwt = (float *)malloc((size_t)T * K * sizeof(float));
    float *zz = (float *)malloc((size_t)T * L * sizeof(float));
    float *contrib = (float *)malloc((size_t)T * K * L * sizeof(float));
    int *uniq = (int *)malloc((size_t)T * K * sizeof(int));
    char *seen = (char *)calloc((size_t)N, 1);
    if (!ridx || !rwt || !zz || !contrib || !uniq || !seen) fatal("oracle allocation", T);
    QScr s;
    qscr_alloc(&s, c);
    int nu = 0;
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * E;
        int *it = ridx + (size_t)t * K;
        orc_router(it, rwt + (size_t)t * K, xt, w->gate, w->bias, E, N, K, c->renorm,
                   c->routed_scale);
        mmw(zz + (size_t)t * L, xt, w->down, w->wdt, E, L);
        for (int j = 0; j < K; j++)
            if (it[j] >= 0 && it[j] < N && !seen[it[j]]) {
                seen[it[j]] = 1;
                uniq[nu++] = it[j];
            }
    }
    if (src->getmany) src->getmany(src, w->layer, uniq, nu);
    for (int u = 0; u < nu; u++) {
        const int e = uniq[u];
        OrcExpertQ q;
        const int ok = src->get(src, w->layer, e, &q) == 0;
        if (!ok) (*drops)++;
        for (int t = 0; t < T; t++)
            for (int j = 0; j < K; j++) {
                if (ridx[(size_t)t * K + j] != e) continue;
                float *cb = contrib + ((size_t)t * K + j) * L;
                if (!ok) {
                    memset(cb, 0, (size_t)L * sizeof(float));
                    continue;
                }
                expert_q(cb, zz + (size_t)t * L, &q, L, I, c->b1, c->b2, s.gu, s.act);
            }
    }
    for (int t = 0; t < T; t++) {
        float *acc = zz + (size_t)t * L;
        const float *wtt = rwt + (size_t)t * K;
        for (int i = 0; i < L; i++) acc[i] = 0.0f;
        for (int j = 0; j < K; j++) {
            const float wj = wtt[j];
            const float *cb = contrib + ((size_t)t * K + j) * L;
            for (int i = 0; i < L; i++) acc[i] += wj * cb[i];
        }
        moe_tail(out + (size_t)t * E, acc, x + (size_t)t * E, w, c, s.sgu, s.sact, s.sdn);
    }
    free(ridx);
    free(rwt);
    free(zz);
    free(contrib);
    free(uniq);
    free(seen);
    free(s.z);
}

void orc_moe_q(float *out, const float *x, const OrcMoeQW *w, const OrcMoeCfg *c, int T,
               int *idx, float *wt, int prefill, long *drops)
{
    if (!w->src) fatal("orc_moe_q needs a source", 0);
    /* k3_moe_prefill (k3_ops.c:689-715): the per-token form for T <= 1 or cache-only,
     * else 64-token chunks, a chunk of one token again per token. */
    if (!prefill || T <= 1 || w->cache_only) {
        moe_q_tokens(out, x, w, c, T, idx, wt, drops);
        return;
    }
    for (int t0 = 0; t0 < T; t0 += 64) {
        const int n = T - t0 < 64 ? T - t0 : 64;
        float *o = out + (size_t)t0 * c->hidden;
        const float *xi = x + (size_t)t0 * c->hidden;
        if (n == 1) moe_q_tokens(o, xi, w, c, 1, idx, wt, drops);
        else moe_q_chunk(o, xi, w, c, n, drops);
    }
}

/* ------------------------------------------------------------ bench helpers ---- */
uint64_t orc_fnv1a(const float *v, size_t n)
{
    uint64_t h = 1469598103934665603ull;
    for (size_t k = 0; k < n; k++) {
        uint32_t u;
        memcpy(&u, &v[k], 4);
        for (int t = 0; t < 4; t++) {
            h ^= (u >> (8 * t)) & 0xFFu;
            h *= 1099511628211ull;
        }
    }
    return h;
}

static inline unsigned xs32(unsigned s)
{
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    return s;
}

void orc_fill_f(float *p, size_t n, unsigned s)
{
    for (size_t i = 0; i < n; i++) {
        s = xs32(s);
        p[i] = ((float)(s >> 8) / 8388608.0f - 1.0f) * 0.05f;
    }
}

void orc_fill_b(unsigned char *p, size_t n, unsigned s)
{
    for (size_t i = 0; i < n; i++) {
        s = xs32(s);
        p[i] = (unsigned char)(s >> 13);
    }
}

void orc_fill_bf16(uint16_t *p, size_t n, unsigned s)
{
    for (size_t i = 0; i < n; i++) {
        s = xs32(s);
        const float f = ((float)(s >> 8) / 8388608.0f - 1.0f) * 0.05f;
        uint32_t u;
        memcpy(&u, &f, 4);
        p[i] = (uint16_t)(u >> 16);
    }
}
