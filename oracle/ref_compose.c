/* SPDX-License-Identifier: Apache-2.0 */
/*
 * ref_compose.c -- TEST INFRASTRUCTURE ONLY. Drives the compiled reference (_ref/libk3ref.so,
 * built from the reference's own src/core/k3_ops.c) through the routed-MoE composition the
 * benchmark measures: per token, k3_router, then for each slot j the expert triple
 * k3_matmul_mxfp4 (gate, up), the activation, k3_matmul_mxfp4 (down), and the weighted add
 * accL[i] += wt[j] * edn[i] starting from zero -- the reference's k3_moe routed loop
 * (k3_ops.c:576-643) with z := x. Tokens are processed one after another, each kernel
 * parallel inside (OpenMP), exactly as k3_moe runs them.
 *
 * The reference has no SiLU-GLU expert activation; act == 1 applies (g * s(g)) * u with
 * s(g) = 1/(1 + expf(-g)), the reference's own SiLU form (k3_ops.c:105, 160).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    const unsigned char *p1, *s1, *p3, *s3, *p2, *s2;
} RefExpertQ;

/* Symbols of the compiled reference (include/k3/k3.h:137, 241-243, 565-566). */
void k3_matmul_mxfp4(float *y, const float *x, const unsigned char *packed,
                     const unsigned char *scales, int in, int rows, int group);
void k3_router(int *idx, float *w, const float *x, const float *W, const float *bias,
               int hidden, int n_experts, int topk, int renorm, float routed_scale);
void k3_situ_glu(float *y, const float *x, int n, float b1, float b2);

static void silu_glu(float *y, const float *x, int n)
{
    for (int i = 0; i < n; i++) {
        const float g = x[i];
        const float a = g * (1.0f / (1.0f + expf(-g)));
        y[i] = a * x[n + i];
    }
}

static void expert(float *acc, const float *xt, const RefExpertQ *q, int E, int I, int act,
                   float b1, float b2, float wj, float *gu, float *a, float *dn)
{
    k3_matmul_mxfp4(gu, xt, q->p1, q->s1, E, I, 32);
    k3_matmul_mxfp4(gu + I, xt, q->p3, q->s3, E, I, 32);
    if (act == 1) silu_glu(a, gu, I);
    else k3_situ_glu(a, gu, I, b1, b2);
    k3_matmul_mxfp4(dn, a, q->p2, q->s2, I, E, 32);
    for (int i = 0; i < E; i++) acc[i] += wj * dn[i];
}

int ref_expert_ffn(float *out, const float *x, const RefExpertQ *q, int E, int I, int act,
                   float b1, float b2, float wt)
{
    float *gu = malloc((size_t)(3 * I + E) * sizeof(float));
    if (!gu) return -1;
    for (int i = 0; i < E; i++) out[i] = 0.0f;
    expert(out, x, q, E, I, act, b1, b2, wt, gu, gu + 2 * I, gu + 3 * I);
    free(gu);
    return 0;
}

int ref_moe_routed(float *out, int *idx, float *wt, const float *x, int T, const float *router_w,
                   const float *bias, const RefExpertQ *bank, int E, int I, int n_experts, int topk,
                   int renorm, float routed_scale, int act, float b1, float b2)
{
    float *gu = malloc((size_t)(3 * I + E) * sizeof(float));
    if (!gu) return -1;
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * E;
        float *ot = out + (size_t)t * E;
        int *it = idx + (size_t)t * topk;
        float *wtt = wt + (size_t)t * topk;
        k3_router(it, wtt, xt, router_w, bias, E, n_experts, topk, renorm, routed_scale);
        for (int i = 0; i < E; i++) ot[i] = 0.0f;
        for (int j = 0; j < topk; j++)
            expert(ot, xt, &bank[it[j]], E, I, act, b1, b2, wtt[j], gu, gu + 2 * I, gu + 3 * I);
    }
    free(gu);
    return 0;
}
