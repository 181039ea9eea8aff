/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_oracle.h -- CPU restatement of the kimi-k3-in-c routed-MoE hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is the oracle that the HIP library is compared
 * against. Only tests/, the smoke entry point and the CPU-baseline leg of bench.py load
 * it; the product library never links or calls it.
 *
 * Every function restates, in code written for this project, the arithmetic of the
 * reference C kernel it names (src/core/k3_ops.c of the reference, compiled for x86-64
 * with AVX2 + FMA and -ffp-contract=off, which is the path the reference's own build
 * selects on this class of host). "Restates" means the same operations in the same order
 * with the same rounding, so the outputs are bit-identical to the reference build; the
 * tests in tests/test_oracle.py check exactly that against the compiled reference and
 * the reference's fixtures.
 */
#ifndef K3_ORACLE_H
#define K3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Expert triple as the reference's K3ExpertQ (include/k3/k3.h:323-327). */
typedef struct {
    const unsigned char *p1, *s1;   /* gate */
    const unsigned char *p3, *s3;   /* up   */
    const unsigned char *p2, *s2;   /* down */
} OrcExpertQ;

enum { ORC_ACT_SITU = 0, ORC_ACT_SILU = 1 };

void orc_mxfp4_dequant(float *out, const unsigned char *packed, const unsigned char *scales,
                       int rows, int pcols, int group);
void orc_matmul_mxfp4(float *y, const float *x, const unsigned char *packed,
                      const unsigned char *scales, int in, int rows, int group);
void orc_matmul(float *y, const float *x, const float *W, int in, int out);
void orc_matmul_bf16(float *y, const float *x, const uint16_t *W, int in, int out);
void orc_router(int *idx, float *w, const float *x, const float *W, const float *bias,
                int hidden, int n_experts, int topk, int renorm, float routed_scale);
void orc_situ_glu(float *y, const float *x, int n, float b1, float b2);
void orc_silu_glu(float *y, const float *x, int n);
void orc_rmsnorm(float *y, const float *x, const float *w, int n, float eps);

/* One routed expert at width `hidden`, intermediate `inter`:
 *   out[i] = 0 + wt * down(act(gate x, up x))[i]          (k3_ops.c:628-631, 641-642)   */
void orc_expert_ffn(float *out, const float *x, const OrcExpertQ *q, int hidden, int inter,
                    int act, float b1, float b2, float wt);

/* The same expert for n tokens x[n][hidden], expert-major: out[t] = down(act(gate x_t,
 * up x_t)) (no combine weight), each matrix dequantized once; equal to orc_expert_ffn per
 * token (a reordering of the same operations; tests pin the two together). */
void orc_expert_ffn_many(float *out, const float *x, int n, const OrcExpertQ *q, int hidden,
                         int inter, int act, float b1, float b2);

/* Routed MoE layer over T tokens: k3_moe's routed loop (k3_ops.c:576-643) with z := x
 * and no latent/shared tail. bank[e] addresses expert e. idx/wt are [T][topk]. */
void orc_moe_routed(float *out, int *idx, float *wt, const float *x, int T,
                    const float *router_w, const float *bias, const OrcExpertQ *bank,
                    int hidden, int inter, int n_experts, int topk, int renorm,
                    float routed_scale, int act, float b1, float b2);

/* Expert-major gather of T*topk assignments: experts in ascending id, (t, j) ascending
 * inside one expert, the order moe_prefill_chunk visits them (k3_ops.c:783-794).
 * offsets has n_experts+1 entries; perm[p] = t*topk + j. */
void orc_gather(int *offsets, int *perm, const int *idx, int T, int topk, int n_experts);

/* The reference's full LatentMoE block with a resident fp32 expert bank (k3_ops.c:556-656),
 * for the ops/moe.json fixture. */
typedef struct {
    int hidden, latent, inter, n_experts, topk, n_shared, renorm, latent_norm;
    float routed_scale, rms_eps, b1, b2;
} OrcMoeCfg;
typedef struct {
    const float *gate, *bias, *w1, *w3, *w2, *latent_norm, *down, *up, *sh1, *sh3, *sh2;
} OrcMoeW;
void orc_moe_latent(float *out, const float *x, const OrcMoeW *w, const OrcMoeCfg *c, int T);

/* Expert source with the reference's K3ExpertSrc layout (include/k3/k3.h:332-355), so a
 * caller can hand the same struct to the oracle and to the library under test. */
typedef struct OrcExpertSrc {
    int (*get)(struct OrcExpertSrc *self, int layer, int expert, OrcExpertQ *out);
    int (*getmany)(struct OrcExpertSrc *self, int layer, const int *experts, int n);
    int (*resident)(struct OrcExpertSrc *self, int layer, int expert, OrcExpertQ *out);
    void *ctx;
} OrcExpertSrc;

/* The LatentMoE weights of the streamed form: router, trunk projections and shared
 * expert of weight type wdt (0 fp32, 1 bf16), experts from src. */
typedef struct {
    const float *gate, *bias, *latent_norm;
    const void *down, *up, *sh1, *sh3, *sh2;
    int wdt;
    OrcExpertSrc *src;
    int layer, cache_only;
} OrcMoeQW;

/* k3_moe (prefill 0, k3_ops.c:556-656) or k3_moe_prefill (prefill 1, :689-825) with
 * MXFP4 experts from w->src, calling get / getmany / resident in the reference's order.
 * idx/wt (topk each) are written as the reference writes them; *drops is incremented
 * where the reference increments k3_expert_drops. */
void orc_moe_q(float *out, const float *x, const OrcMoeQW *w, const OrcMoeCfg *c, int T,
               int *idx, float *wt, int prefill, long *drops);

/* FNV-1a over the bytes of a float vector (benchmarks/bench_kernels.c:44-52). */
uint64_t orc_fnv1a(const float *v, size_t n);
/* The reference benchmark's xorshift32 fillers (benchmarks/bench_kernels.c:54-89). */
void orc_fill_f(float *p, size_t n, unsigned seed);
void orc_fill_b(unsigned char *p, size_t n, unsigned seed);
void orc_fill_bf16(uint16_t *p, size_t n, unsigned seed);

int orc_threads(void);

#ifdef __cplusplus
}
#endif
#endif
