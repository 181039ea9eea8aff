/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3.h -- MI355X drop-in for the routed-expert MoE hot path of kimi-k3-in-c.
 *
 * This header is the C ABI of libk3amd.so. The first half re-declares, with the same
 * names, signatures, struct layouts and error behaviour, the subset of the reference's
 * public header (include/k3/k3.h of the reference) that the MoE hot path uses, so that a
 * caller built against the reference links against this library unchanged. Each entry
 * names the reference declaration it replaces. The second half adds entry points the
 * reference does not have (a fused expert FFN, a routed MoE layer, device residency for
 * weights); those carry no ABI constraint from the reference.
 *
 * Semantics shared by every host-pointer entry point below:
 *   - all pointers are HOST pointers, exactly as in the reference; outputs are written in
 *     full before the call returns (the call is synchronous);
 *   - weights are uploaded to HBM for the call unless they were registered with
 *     k3_dev_register(), in which case the resident device copy is used and no PCIe
 *     transfer of the weights happens;
 *   - preconditions the reference aborts on abort here too, with a FATAL message, and a
 *     HIP error (no device, out of memory, kernel fault) also aborts: a void kernel never
 *     returns with its output unwritten (reference src/core/k3_ops.c:37-78);
 *   - every entry point may be called from several host threads at once, as the
 *     reference's kernels may (reference docs/API.md:138-139): the library takes one
 *     process-wide lock per call and runs the calls one after another on its HIP stream,
 *     so concurrent callers are safe and see the same results as sequential ones.
 */
#ifndef K3_AMD_H
#define K3_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------ reference-compatible types ---- */

/* Model configuration; same fields, order and types as the reference's K3Cfg
 * (include/k3/k3.h:73-120). The MoE path reads hidden, rms_eps, n_experts, topk,
 * n_shared, latent, moe_inter, routed_scale, moe_renorm, latent_norm, situ_b1, situ_b2. */
typedef struct {
    int hidden;
    int n_layers;
    int vocab;
    float rms_eps;
    int kda_heads;
    int kda_head_dim;
    int conv_k;
    float gate_lb;
    int n_heads;
    int q_lora;
    int kv_lora;
    int qk_nope;
    int qk_rope;
    int v_head;
    int mla_out_gate;
    int n_experts;
    int topk;
    int n_shared;
    int latent;
    int moe_inter;
    float routed_scale;
    int moe_renorm;
    int latent_norm;
    int first_dense;
    int dense_inter;
    int attn_res_block;
    float situ_b1;
    float situ_b2;
    int n_full_attn;
    int *full_attn;
} K3Cfg;

/* Weight-matrix dtype tags (reference include/k3/k3.h:270). */
enum { K3_WF32 = 0, K3_WBF16 = 1, K3_WI8 = 2 };

/* bf16 -> f32 is a 16-bit left shift (reference include/k3/k3.h:274-279). */
static inline float k3_bf16f(uint16_t h)
{
    union { uint32_t u; float f; } v;
    v.u = (uint32_t)h << 16;
    return v.f;
}

/* One routed expert in packed MXFP4: gate (p1, s1), up (p3, s3), down (p2, s2)
 * (reference include/k3/k3.h:323-327). */
typedef struct {
    const unsigned char *p1, *s1;
    const unsigned char *p3, *s3;
    const unsigned char *p2, *s2;
} K3ExpertQ;

/* Expert source callbacks (reference include/k3/k3.h:332-355). */
typedef struct K3ExpertSrc {
    int (*get)(struct K3ExpertSrc *self, int layer, int expert, K3ExpertQ *out);
    int (*getmany)(struct K3ExpertSrc *self, int layer, const int *experts, int n);
    int (*resident)(struct K3ExpertSrc *self, int layer, int expert, K3ExpertQ *out);
    void *ctx;
} K3ExpertSrc;

/* MoE layer weights (reference include/k3/k3.h:357-380). */
typedef struct {
    const float *gate, *bias;
    const float *w1, *w3, *w2;
    const float *latent_norm;
    const void *down, *up;
    const void *sh1, *sh3, *sh2;
    int wdt;
    struct K3ExpertSrc *src;
    int layer;
    int cache_only;
} K3MoeW;

/* MXFP4 group size and top-k bound (reference include/k3/k3.h:548, 557). */
#define K3_MXFP4_GROUP 32
#define K3_MAX_TOPK 64

/* ------------------------------------------------ reference-compatible calls ---- */

/* y[out] = W[out][in] . x[in], W fp32 row-major.
 * Replaces k3_matmul, reference include/k3/k3.h:168. */
void k3_matmul(float *y, const float *x, const float *W, int in, int out);

/* y = W x with W bf16, widened exactly. Replaces k3_matmul_bf16, reference
 * include/k3/k3.h:281. */
void k3_matmul_bf16(float *y, const float *x, const uint16_t *W, int in, int out);

/* Per-row int8 matmul of the draft model, rows [f32 scale][int8 x in]. Replaces
 * k3_matmul_q8, reference include/k3/k3.h:285 (no exactness contract there or here). */
void k3_matmul_q8(float *y, const float *x, const void *W, int in, int out);

/* Tagged dispatch (reference include/k3/k3.h:289-295). */
static inline void k3_mmw(float *y, const float *x, const void *W, int wdt, int in, int out)
{
    if (wdt == K3_WBF16) k3_matmul_bf16(y, x, (const uint16_t *)W, in, out);
    else if (wdt == K3_WI8) k3_matmul_q8(y, x, W, in, out);
    else k3_matmul(y, x, (const float *)W, in, out);
}

/* out[rows][pcols*2] = E2M1[nibble] * 2^(scale-127), low nibble = even element, scale
 * byte 255 -> 0. Replaces k3_mxfp4_dequant, reference include/k3/k3.h:559-560. */
void k3_mxfp4_dequant(float *out, const unsigned char *packed, const unsigned char *scales,
                      int rows, int pcols, int group);

/* y[rows] = W[rows][in] . x[in], W packed MXFP4 [rows][in/2] with E8M0 scales
 * [rows][ceil(in/group)]. Aborts on odd `in` or group > 64 like the reference; the
 * device path additionally requires group to be even. Replaces k3_matmul_mxfp4,
 * reference include/k3/k3.h:565-566. */
void k3_matmul_mxfp4(float *y, const float *x, const unsigned char *packed,
                     const unsigned char *scales, int in, int rows, int group);

/* Sigmoid router, one token: selection on score+bias, weights from the unbiased scores,
 * renormalised and scaled; idx/w in descending selection order. Replaces k3_router,
 * reference include/k3/k3.h:241-243. n_experts is limited to 2048 (the reference takes any
 * count; Kimi K3 has 896): the selection keeps every expert's scored record in one
 * workgroup's LDS. A larger count aborts with a FATAL message. */
void k3_router(int *idx, float *w, const float *x, const float *W, const float *bias,
               int hidden, int n_experts, int topk, int renorm, float routed_scale);

/* SiTU-GLU over [gate | up] of width 2n. Replaces k3_situ_glu, reference
 * include/k3/k3.h:137. */
void k3_situ_glu(float *y, const float *x, int n, float b1, float b2);

/* y = w * x / sqrt(mean(x^2) + eps). Replaces k3_rmsnorm, reference include/k3/k3.h:130. */
void k3_rmsnorm(float *y, const float *x, const float *w, int n, float eps);

/* Count of routed experts that failed to load (reference include/k3/k3.h:388). */
extern long k3_expert_drops;

/* Scratch floats for k3_moe (reference include/k3/k3.h:382). */
size_t k3_moe_scratch(const K3Cfg *c);

/* Stable LatentMoE block over T tokens (route on the full width, down-project, routed
 * experts in latent space, RMSNorm of the aggregate, up-project, unweighted shared
 * expert). Replaces k3_moe, reference include/k3/k3.h:418-419. */
void k3_moe(float *out, const float *x, const K3MoeW *w, const K3Cfg *c, int T, int *idx,
            float *wt, float *scratch);

/* Expert-major batched form; per-token results identical to k3_moe. Replaces
 * k3_moe_prefill, reference include/k3/k3.h:425-426. */
void k3_moe_prefill(float *out, const float *x, const K3MoeW *w, const K3Cfg *c, int T,
                    int *idx, float *wt, float *scratch);

/* ------------------------------------------------------- entry points added ---- */

/* Expert activation. SiTU-GLU is the reference's (k3_ops.c:110-123); SiLU-GLU is
 * (g * sigmoid(g)) * up in the reference's own SiLU form (k3_ops.c:160, 105). */
enum { K3_ACT_SITU = 0, K3_ACT_SILU = 1 };

/* One routed expert FFN straight out of MXFP4, fused:
 *   out[hidden] = wt * down(act(gate . x, up . x))
 * x is [hidden], q addresses the gate/up [inter][hidden] and down [hidden][inter]
 * packed matrices (group 32). The arithmetic of one iteration of k3_moe's routed loop
 * (reference k3_ops.c:628-631, 641-642) with accL starting at zero. No reference
 * counterpart as a single call. */
void k3_expert_ffn(float *out, const float *x, const K3ExpertQ *q, int hidden, int inter,
                   int act, float b1, float b2, float wt);

/* Routed MoE layer over T tokens, hidden width E, MXFP4 experts of intermediate I:
 *   per token: k3_router on router_w/bias; for j < topk, in j order,
 *   out[t] += wt[t][j] * expert_ffn(idx[t][j], x[t]) starting from zero.
 * This is k3_moe's routed inner loop (reference k3_ops.c:576-643) with z := x, computed
 * expert-major on the device (gather by expert, grouped expert GEMV/GEMM, weighted
 * scatter-add combine in slot order). bank has n_experts entries of host pointers
 * (each may be registered for residency). idx/wt ([T][topk]) receive the routing. An
 * expert whose bank entry has a NULL pointer counts as a failed load: it increments
 * k3_expert_drops, prints EXPERT DROP and contributes zero, as k3_moe does
 * (k3_ops.c:616-626). prec selects the expert matmul precision: 0 = fp32-accurate
 * (activations split into two bf16 terms), 1 = activations rounded to bf16 once. */
void k3_moe_routed(float *out, int *idx, float *wt, const float *x, int T,
                   const float *router_w, const float *bias, const K3ExpertQ *bank,
                   int hidden, int inter, int n_experts, int topk, int renorm,
                   float routed_scale, int act, float b1, float b2, int prec);

/* An expert bank resident in HBM behind the reference's K3ExpertSrc: the device-side
 * counterpart of the reference's host-RAM expert cache (src/cache/k3_cache.h, whose slots
 * become K3ExpertQ pointers at src/cache/k3_cache.c:24-33). k3_devbank_source() returns a
 * K3ExpertSrc to put in K3MoeW.src: its get() means "ensure resident in HBM" and returns
 * DEVICE pointers (a miss fetches the expert's host bytes from `upstream`, any host-pointer
 * K3ExpertSrc, or fails when upstream is NULL), getmany() is the batch form and resident()
 * answers without a transfer. k3_moe / k3_moe_prefill given this source run the experts
 * straight from the slots, with no weight transfer once the experts are resident. Experts
 * are width x inter MXFP4 (gate/up [inter][width], down [width][inter], group 32); `slots`
 * experts fit, least recently used evicted first, never one that the running MoE call has
 * fetched. layout K3_BANK_TILED regroups each matrix once at admission for the expert
 * kernels (widths multiples of 512), K3_BANK_ROWS keeps the reference's byte order.
 * Device pointers from get() stay valid until that slot is evicted. No reference
 * counterpart as a function; the run layout is the reference's (src/io/k3_load.h:3-18). */
enum { K3_BANK_ROWS = 0, K3_BANK_TILED = 1 };
typedef struct K3DevBank K3DevBank;
typedef struct {
    long hits, misses, evictions, failures;
    unsigned long long bytes_uploaded;   /* host-to-device weight bytes so far */
    int resident, slots;
    size_t slot_bytes;
} K3DevBankStats;
K3DevBank *k3_devbank_create(int n_layers, int n_experts, int width, int inter, int slots,
                             int layout, K3ExpertSrc *upstream);
K3ExpertSrc *k3_devbank_source(K3DevBank *bank);
/* Bytes of one expert's on-disk run: 3 * (width*inter/2 + width*inter/32), 17,547,264 for
 * Kimi K3's 3584 x 3072 experts. */
size_t k3_devbank_run_bytes(int width, int inter);
/* Admits (or replaces) expert (layer, expert) from its contiguous run, in the reference's
 * order w1.packed w1.scale w2.packed w2.scale w3.packed w3.scale (gate = w1, down = w2,
 * up = w3). Returns 0, or -1 with k3_dev_last_error(). */
int k3_devbank_put_run(K3DevBank *bank, int layer, int expert, const void *run, size_t bytes);
int k3_devbank_stats(const K3DevBank *bank, K3DevBankStats *st);
void k3_devbank_destroy(K3DevBank *bank);

/* Device residency. Registers [host, host+bytes) as immutable weights: a device copy is
 * made now and every later call that receives a pointer inside the range reads the copy.
 * Returns 0, or -1 on failure (message from k3_dev_last_error). The caller must not
 * modify the host bytes while registered; k3_dev_unregister drops the copy. */
int k3_dev_register(const void *host, size_t bytes);
int k3_dev_unregister(const void *host);
/* Device address of a registered host pointer, or NULL. */
void *k3_dev_lookup(const void *host);
const char *k3_dev_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* K3_AMD_H */
