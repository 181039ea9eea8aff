/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_host.c -- the reference's host-pointer API (include/k3.h) on the MI355X.
 *
 * C99. Every entry point takes host buffers exactly as the reference's does, moves the
 * activations to HBM, resolves weights to their registered device copy (or uploads them
 * for this call), runs the HIP kernels through the k3k ABI / k3_dev entry points on the
 * library's stream, and copies the outputs back before returning. A HIP failure aborts
 * with a FATAL message: these functions return void, and returning with the output
 * unwritten is the failure the reference refuses to allow (src/core/k3_ops.c:37-78).
 *
 * The reference's kernels may be called from several threads at once (its docs/API.md:
 * 138-139). Here every entry point holds one process-wide recursive lock for its whole
 * duration, so concurrent calls run one after another on the library's stream and share
 * its device buffers safely; recursive, because a K3ExpertSrc callback that k3_moe calls
 * may itself be this library's HBM bank.
 */
#define _XOPEN_SOURCE 700
#include "k3.h"
#include "k3_bank.h"
#include "k3_dev.h"
#include "k3k.h"

#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

long k3_expert_drops = 0;

/* ---------------------------------------------------------------- plumbing ---- */
static pthread_mutex_t g_mu;
static pthread_once_t g_mu_once = PTHREAD_ONCE_INIT;

static void mu_init(void)
{
    pthread_mutexattr_t a;
    pthread_mutexattr_init(&a);
    pthread_mutexattr_settype(&a, PTHREAD_MUTEX_RECURSIVE);
    pthread_mutex_init(&g_mu, &a);
    pthread_mutexattr_destroy(&a);
}

void k3h_lock(void)
{
    pthread_once(&g_mu_once, mu_init);
    pthread_mutex_lock(&g_mu);
}

void k3h_unlock(void) { pthread_mutex_unlock(&g_mu); }

static void *g_stream = NULL;
static char g_regerr[256];

void k3h_set_error(const char *fmt, const char *what)
{
    snprintf(g_regerr, sizeof g_regerr, fmt, what);
}

static void fatal(const char *what)
{
    fprintf(stderr,
            "k3: FATAL, %s: %s\n"
            "    Aborting rather than returning with the output unwritten.\n",
            what, k3k_error());
    abort();
}

int k3h_init(void)
{
    if (g_stream) return 0;
    if (k3k_init() || !(g_stream = k3k_stream_create())) {
        k3h_set_error("no usable HIP device: %s", k3k_error());
        return -1;
    }
    return 0;
}

void *k3h_stream(void) { return g_stream; }

static void lib_init(void)
{
    if (k3h_init()) fatal("no usable HIP device");
}

static void check(int rc, const char *what)
{
    if (rc) {
        fprintf(stderr, "k3: FATAL, %s: %s\n", what, rc == -2 ? k3d_error() : k3k_error());
        abort();
    }
}

/* Reusable device buffers, one per role, grown on demand. */
enum { B_X, B_Y, B_P, B_S, B_WS, B_BIAS, B_RW, B_IDX, B_WT, B_ARENA, B_BANK, B_Z, B_ACC,
       B_SGU, B_SDN, B_OUT, B_W2, B_W3, B_T0, B_T1, B_T2, B_XS, B_SACT, B_SSDN, B_SXS, B_FACT,
       B_COUNT };
static void *g_buf[B_COUNT];
static size_t g_cap[B_COUNT];

static void *buf(int slot, size_t bytes)
{
    if (bytes == 0) bytes = 4;
    if (g_cap[slot] < bytes) {
        if (g_buf[slot]) {
            /* every stream: the library stream's side stream may still read it */
            check(k3k_sync(NULL), "synchronize before buffer growth");
            k3k_free(g_buf[slot]);
        }
        size_t cap = bytes + bytes / 4;
        g_buf[slot] = k3k_malloc(cap);
        if (!g_buf[slot]) fatal("device allocation");
        g_cap[slot] = cap;
    }
    return g_buf[slot];
}

static void *upload(int slot, const void *h, size_t bytes)
{
    void *d = buf(slot, bytes);
    check(k3k_h2d(d, h, bytes, g_stream), "host to device copy");
    return d;
}

static void download(void *h, const void *d, size_t bytes)
{
    check(k3k_d2h(h, d, bytes, g_stream), "device to host copy");
    check(k3k_sync(g_stream), "synchronize");
}

/* Pinned staging for copies the host waits for by event, grown on demand. */
static void *g_pin = NULL;
static size_t g_pin_cap = 0;
static void *g_pin_ev = NULL;

static void *pinned(size_t bytes)
{
    if (g_pin_cap < bytes) {
        check(k3k_sync(NULL), "synchronize before staging growth");
        k3k_host_free(g_pin);
        g_pin_cap = bytes + bytes / 4;
        g_pin = k3k_host_alloc(g_pin_cap);
        if (!g_pin) fatal("pinned host allocation");
    }
    if (!g_pin_ev && !(g_pin_ev = k3k_event_create())) fatal("event creation");
    return g_pin;
}

/* ---------------------------------------------------------------- registry ---- */
typedef struct {
    const unsigned char *host;
    size_t bytes;
    void *dev;
} Reg;
static Reg *g_reg = NULL;
static int g_nreg = 0, g_capreg = 0;

static const Reg *reg_find(const void *host)
{
    const unsigned char *h = (const unsigned char *)host;
    for (int i = 0; i < g_nreg; i++)
        if (h >= g_reg[i].host && h < g_reg[i].host + g_reg[i].bytes) return &g_reg[i];
    return NULL;
}

static void *k3_dev_lookup_impl(const void *host)
{
    const Reg *r = host ? reg_find(host) : NULL;
    if (!r) return NULL;
    return (char *)r->dev + ((const unsigned char *)host - r->host);
}

const char *k3_dev_last_error(void) { return g_regerr; }

static int k3_dev_register_impl(const void *host, size_t bytes)
{
    if (!host || !bytes) {
        snprintf(g_regerr, sizeof g_regerr, "k3_dev_register: empty range");
        return -1;
    }
    if (k3h_init()) {
        snprintf(g_regerr, sizeof g_regerr, "k3_dev_register: %s", k3k_error());
        return -1;
    }
    const unsigned char *h = (const unsigned char *)host;
    for (int i = 0; i < g_nreg; i++)
        if (h < g_reg[i].host + g_reg[i].bytes && g_reg[i].host < h + bytes) {
            snprintf(g_regerr, sizeof g_regerr, "k3_dev_register: range overlaps a registered one");
            return -1;
        }
    void *d = k3k_malloc(bytes);
    if (!d || k3k_h2d(d, host, bytes, g_stream) || k3k_sync(g_stream)) {
        snprintf(g_regerr, sizeof g_regerr, "k3_dev_register: %s", k3k_error());
        if (d) k3k_free(d);
        return -1;
    }
    if (g_nreg == g_capreg) {
        int cap = g_capreg ? 2 * g_capreg : 16;
        Reg *n = (Reg *)realloc(g_reg, (size_t)cap * sizeof(Reg));
        if (!n) {
            k3k_free(d);
            snprintf(g_regerr, sizeof g_regerr, "k3_dev_register: out of host memory");
            return -1;
        }
        g_reg = n;
        g_capreg = cap;
    }
    g_reg[g_nreg].host = h;
    g_reg[g_nreg].bytes = bytes;
    g_reg[g_nreg].dev = d;
    g_nreg++;
    return 0;
}

static int k3_dev_unregister_impl(const void *host)
{
    for (int i = 0; i < g_nreg; i++)
        if (g_reg[i].host == (const unsigned char *)host) {
            if (g_stream) k3k_sync(g_stream);
            k3k_free(g_reg[i].dev);
            g_reg[i] = g_reg[g_nreg - 1];
            g_nreg--;
            return 0;
        }
    snprintf(g_regerr, sizeof g_regerr, "k3_dev_unregister: not registered");
    return -1;
}

/* Device view of host weights: the registered copy, else an upload into `slot`. */
static const void *weights(int slot, const void *host, size_t bytes)
{
    void *d = k3_dev_lookup(host);
    if (d) return d;
    return upload(slot, host, bytes);
}

static int aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

/* ------------------------------------------------------------------- GEMVs ---- */
static void k3_matmul_impl(float *y, const float *x, const float *W, int in, int out)
{
    if (out <= 0) return;
    lib_init();
    const float *dw = (const float *)weights(B_P, W, (size_t)in * out * 4);
    const float *dx = (const float *)upload(B_X, x, (size_t)(in > 0 ? in : 1) * 4);
    float *dy = (float *)buf(B_Y, (size_t)out * 4);
    check(k3k_gemv_f32(dy, dx, dw, in, out, 1, out, g_stream), "k3_matmul");
    download(y, dy, (size_t)out * 4);
}

static void k3_matmul_bf16_impl(float *y, const float *x, const uint16_t *W, int in, int out)
{
    if (out <= 0) return;
    lib_init();
    const uint16_t *dw = (const uint16_t *)weights(B_P, W, (size_t)in * out * 2);
    const float *dx = (const float *)upload(B_X, x, (size_t)(in > 0 ? in : 1) * 4);
    float *dy = (float *)buf(B_Y, (size_t)out * 4);
    check(k3k_gemv_bf16(dy, dx, dw, in, out, 1, out, g_stream), "k3_matmul_bf16");
    download(y, dy, (size_t)out * 4);
}

static void k3_matmul_q8_impl(float *y, const float *x, const void *W, int in, int out)
{
    if (out <= 0) return;
    lib_init();
    const void *dw = weights(B_P, W, (size_t)out * (4 + (size_t)in));
    const float *dx = (const float *)upload(B_X, x, (size_t)(in > 0 ? in : 1) * 4);
    float *dy = (float *)buf(B_Y, (size_t)out * 4);
    check(k3k_gemv_q8(dy, dx, dw, in, out, 1, out, g_stream), "k3_matmul_q8");
    download(y, dy, (size_t)out * 4);
}

/* The reference's k3_matmul_mxfp4 refuses an odd `in` and a group above 64 with a FATAL
 * abort (k3_ops.c:1383-1401); callers that rely on that still get it. */
static void mxfp4_preconditions(int in, int group)
{
    if (in & 1) {
        fprintf(stderr,
                "k3: FATAL, k3_matmul_mxfp4 called with in=%d, which is odd.\n"
                "    Two elements share each packed byte, so a row of an odd width has no\n"
                "    whole-byte stride; the matrix cannot be addressed as given.\n",
                in);
        abort();
    }
    if (group > 64 || group <= 0) {
        fprintf(stderr,
                "k3: FATAL, k3_matmul_mxfp4 called with group=%d, outside 1..64.\n"
                "    The MXFP4 format used here scales blocks of at most 64 elements\n"
                "    (32 in every checkpoint); a larger or empty block is rejected.\n",
                group);
        abort();
    }
}

static void k3_matmul_mxfp4_impl(float *y, const float *x, const unsigned char *packed,
                     const unsigned char *scales, int in, int rows, int group)
{
    mxfp4_preconditions(in, group);
    if (rows <= 0) return;
    if (in <= 0) {
        memset(y, 0, (size_t)rows * sizeof(float));
        return;
    }
    lib_init();
    const int ngrp = (in + group - 1) / group;
    const uint8_t *dp = (const uint8_t *)weights(B_P, packed, (size_t)rows * (in / 2));
    const uint8_t *ds = (const uint8_t *)weights(B_S, scales, (size_t)rows * ngrp);
    const float *dx = (const float *)upload(B_X, x, (size_t)in * 4);
    float *dy = (float *)buf(B_Y, (size_t)rows * 4);
    if (group == 32 && in % 32 == 0 && aligned16(dp)) {
        const size_t wsb = k3d_matmul_mxfp4_ws(1, in);
        check(k3d_matmul_mxfp4(dy, dx, 1, dp, ds, in, rows, 0, buf(B_WS, wsb), wsb, g_stream),
              "k3_matmul_mxfp4");
    } else {
        check(k3k_mx_gemv_valu(dy, dx, dp, ds, in, rows, group, g_stream), "k3_matmul_mxfp4");
    }
    download(y, dy, (size_t)rows * 4);
}

static void k3_mxfp4_dequant_impl(float *out, const unsigned char *packed, const unsigned char *scales,
                      int rows, int pcols, int group)
{
    if (rows <= 0 || pcols <= 0) return;
    if (group <= 0) {
        fprintf(stderr, "k3: FATAL, k3_mxfp4_dequant called with group=%d.\n", group);
        abort();
    }
    lib_init();
    const int width = pcols * 2, ngrp = (width + group - 1) / group;
    const uint8_t *dp = (const uint8_t *)weights(B_P, packed, (size_t)rows * pcols);
    const uint8_t *ds = (const uint8_t *)weights(B_S, scales, (size_t)rows * ngrp);
    float *dy = (float *)buf(B_Y, (size_t)rows * width * 4);
    check(k3k_mx_dequant(dy, dp, ds, rows, pcols, group, g_stream), "k3_mxfp4_dequant");
    download(out, dy, (size_t)rows * width * 4);
}

/* ------------------------------------------------------------ router, norms ---- */
static void k3_router_impl(int *idx, float *w, const float *x, const float *W, const float *bias,
               int hidden, int n_experts, int topk, int renorm, float routed_scale)
{
    if (topk <= 0) return;
    if (topk > K3_MAX_TOPK) {
        fprintf(stderr, "k3: FATAL, k3_router called with topk=%d above K3_MAX_TOPK=%d.\n", topk,
                K3_MAX_TOPK);
        abort();
    }
    lib_init();
    const float *dW = (const float *)weights(B_RW, W, (size_t)n_experts * hidden * 4);
    const float *db = bias ? (const float *)weights(B_BIAS, bias, (size_t)n_experts * 4) : NULL;
    const float *dx = (const float *)upload(B_X, x, (size_t)hidden * 4);
    int *di = (int *)buf(B_IDX, (size_t)topk * 4);
    float *dwt = (float *)buf(B_WT, (size_t)topk * 4);
    const size_t wsb = k3d_router_ws(1, hidden, n_experts);
    check(k3d_router(di, dwt, dx, 1, dW, db, hidden, n_experts, topk, renorm, routed_scale,
                     buf(B_WS, wsb), wsb, g_stream),
          "k3_router");
    check(k3k_d2h(idx, di, (size_t)topk * 4, g_stream), "device to host copy");
    download(w, dwt, (size_t)topk * 4);
}

static void k3_situ_glu_impl(float *y, const float *x, int n, float b1, float b2)
{
    if (n <= 0) return;
    lib_init();
    const float *dx = (const float *)upload(B_X, x, (size_t)2 * n * 4);
    float *dy = (float *)buf(B_Y, (size_t)n * 4);
    check(k3k_act(dy, dx, n, 1, K3_ACT_SITU, b1, b2, g_stream), "k3_situ_glu");
    download(y, dy, (size_t)n * 4);
}

static void k3_rmsnorm_impl(float *y, const float *x, const float *w, int n, float eps)
{
    if (n <= 0) return;
    lib_init();
    const float *dx = (const float *)upload(B_X, x, (size_t)n * 4);
    const float *dw = (const float *)weights(B_P, w, (size_t)n * 4);
    float *dy = (float *)buf(B_Y, (size_t)n * 4);
    check(k3k_rmsnorm(dy, dx, dw, n, 1, eps, g_stream), "k3_rmsnorm");
    download(y, dy, (size_t)n * 4);
}

/* -------------------------------------------------------------- expert bank ---- */
typedef struct {
    const unsigned char *p1, *s1, *p3, *s3, *p2, *s2;
} QPtr;

static size_t pk_bytes(int rows, int in) { return (size_t)rows * (in / 2); }
static size_t sc_bytes(int rows, int in) { return (size_t)rows * ((in + 31) / 32); }

/* Device copy of one expert's six tensors: registered pieces are referenced in place;
 * the rest are uploaded into the arena at *arena_off. Packed tensors must be 16-byte
 * aligned on the device for the matrix-core loads; a misaligned registered piece is
 * copied to an aligned arena slot. */
static void resolve_expert(QPtr *d, const K3ExpertQ *h, int hidden, int inter, char *arena,
                           size_t *arena_off)
{
    const void *src[6] = {h->p1, h->s1, h->p3, h->s3, h->p2, h->s2};
    const size_t sz[6] = {pk_bytes(inter, hidden), sc_bytes(inter, hidden),
                          pk_bytes(inter, hidden), sc_bytes(inter, hidden),
                          pk_bytes(hidden, inter), sc_bytes(hidden, inter)};
    const unsigned char *out[6];
    for (int k = 0; k < 6; k++) {
        void *dv = k3_dev_lookup(src[k]);
        if (dv && (k & 1 || aligned16(dv))) {
            out[k] = (const unsigned char *)dv;
            continue;
        }
        const size_t o = (*arena_off + 255u) & ~(size_t)255u;
        if (dv) check(k3k_d2d(arena + o, dv, sz[k], g_stream), "expert copy");
        else check(k3k_h2d(arena + o, src[k], sz[k], g_stream), "expert upload");
        out[k] = (const unsigned char *)(arena + o);
        *arena_off = o + sz[k];
    }
    d->p1 = out[0]; d->s1 = out[1]; d->p3 = out[2];
    d->s3 = out[3]; d->p2 = out[4]; d->s2 = out[5];
}

static size_t expert_upload_bytes(const K3ExpertQ *h, int hidden, int inter)
{
    const void *src[6] = {h->p1, h->s1, h->p3, h->s3, h->p2, h->s2};
    const size_t sz[6] = {pk_bytes(inter, hidden), sc_bytes(inter, hidden),
                          pk_bytes(inter, hidden), sc_bytes(inter, hidden),
                          pk_bytes(hidden, inter), sc_bytes(hidden, inter)};
    size_t n = 0;
    for (int k = 0; k < 6; k++) {
        void *dv = k3_dev_lookup(src[k]);
        if (!dv || (!(k & 1) && !aligned16(dv))) n += ((sz[k] + 255u) & ~(size_t)255u) + 256u;
    }
    return n;
}

static int expert_ok(const K3ExpertQ *q)
{
    return q->p1 && q->s1 && q->p3 && q->s3 && q->p2 && q->s2;
}

/* Fallback for shapes the matrix-core path does not take (hidden or inter not a multiple
 * of 32): per assignment, three vector-unit MXFP4 GEMVs and the activation, then the
 * ordered combine. out_d, idx (host), wt_d, x_d are device/host as named. */
static void experts_generic(float *out_d, const int *idx, const float *wt_d, const int *idx_d,
                            const float *x_d, int T, const QPtr *bank, int hidden, int inter,
                            int n_experts, int topk, int act, float b1, float b2)
{
    const size_t N = (size_t)T * topk;
    float *contrib = (float *)buf(B_T0, N * hidden * 4);
    float *gu = (float *)buf(B_T1, (size_t)2 * inter * 4);
    float *a = (float *)buf(B_T2, (size_t)inter * 4);
    for (int t = 0; t < T; t++)
        for (int j = 0; j < topk; j++) {
            const int e = idx[t * topk + j];
            if (e < 0 || e >= n_experts || !bank[e].p1) continue;
            const QPtr *q = &bank[e];
            const float *xt = x_d + (size_t)t * hidden;
            check(k3k_mx_gemv_valu(gu, xt, q->p1, q->s1, hidden, inter, 32, g_stream), "expert gate");
            check(k3k_mx_gemv_valu(gu + inter, xt, q->p3, q->s3, hidden, inter, 32, g_stream), "expert up");
            check(k3k_act(a, gu, inter, 1, act, b1, b2, g_stream), "expert act");
            check(k3k_mx_gemv_valu(contrib + (size_t)(t * topk + j) * hidden, a, q->p2, q->s2, inter,
                                   hidden, 32, g_stream),
                  "expert down");
        }
    check(k3k_combine(out_d, contrib, wt_d, idx_d, NULL, n_experts, T, topk, hidden, g_stream),
          "combine");
}

/* Runs the expert half for a device bank already resolved into `bank` (host array of
 * device pointers, NULL where absent): out_d[T][hidden] = sum_j wt * expert(x). */
static void run_bank(float *out_d, const int *idx, const int *idx_d, const float *wt_d,
                     const float *x_d, int T, const QPtr *bank, int hidden, int inter,
                     int n_experts, int topk, int act, float b1, float b2, int prec, int layout)
{
    if ((hidden % 32) == 0 && (inter % 32) == 0) {
        void *bank_d = upload(B_BANK, bank, (size_t)n_experts * sizeof(QPtr));
        const size_t wsb = k3d_moe_ws(T, hidden, inter, n_experts, topk, prec);
        check(k3d_moe_experts(out_d, idx_d, wt_d, x_d, T, bank_d, layout, hidden, inter,
                              n_experts, topk, act, b1, b2, prec, buf(B_WS, wsb), wsb, NULL, NULL,
                              NULL, g_stream),
              "moe experts");
    } else {
        experts_generic(out_d, idx, wt_d, idx_d, x_d, T, bank, hidden, inter, n_experts, topk, act,
                        b1, b2);
    }
    check(k3k_sync(g_stream), "synchronize");
}

/* Resolves the experts selected in idx (host) from a host bank and runs them. */
static void run_experts_mxfp4(float *out_d, const int *idx, const int *idx_d, const float *wt_d,
                              const float *x_d, int T, const K3ExpertQ *hbank, int hidden,
                              int inter, int n_experts, int topk, int act, float b1, float b2,
                              int prec)
{
    QPtr *bank = (QPtr *)calloc((size_t)n_experts, sizeof(QPtr));
    unsigned char *sel = (unsigned char *)calloc((size_t)n_experts, 1);
    if (!bank || !sel) {
        fprintf(stderr, "k3: FATAL, host allocation for the expert bank failed.\n");
        abort();
    }
    size_t need = 0;
    for (int a = 0; a < T * topk; a++) {
        const int e = idx[a];
        if (e < 0 || e >= n_experts || sel[e]) continue;
        sel[e] = 1;
        if (expert_ok(&hbank[e])) need += expert_upload_bytes(&hbank[e], hidden, inter);
    }
    char *arena = need ? (char *)buf(B_ARENA, need) : NULL;
    size_t off = 0;
    for (int e = 0; e < n_experts; e++)
        if (sel[e] && expert_ok(&hbank[e])) resolve_expert(&bank[e], &hbank[e], hidden, inter, arena, &off);
    run_bank(out_d, idx, idx_d, wt_d, x_d, T, bank, hidden, inter, n_experts, topk, act, b1, b2, prec,
             K3D_LAYOUT_ROWS);
    free(bank);
    free(sel);
}

static void report_drop(int layer, int expert, const char *what)
{
    k3_expert_drops++;
    fprintf(stderr, "EXPERT DROP: layer %d expert %d failed to load; this %s is CORRUPT\n", layer,
            expert, what);
}

static void k3_expert_ffn_impl(float *out, const float *x, const K3ExpertQ *q, int hidden, int inter, int act,
                   float b1, float b2, float wt)
{
    if (hidden <= 0) return;
    mxfp4_preconditions(hidden, 32);
    mxfp4_preconditions(inter, 32);
    lib_init();
    const int idx0 = 0;
    const float *dx = (const float *)upload(B_X, x, (size_t)hidden * 4);
    const int *di = (const int *)upload(B_IDX, &idx0, 4);
    const float *dw = (const float *)upload(B_WT, &wt, 4);
    float *dy = (float *)buf(B_OUT, (size_t)hidden * 4);
    if (!expert_ok(q)) {
        report_drop(0, 0, "token");
        memset(out, 0, (size_t)hidden * 4);
        return;
    }
    run_experts_mxfp4(dy, &idx0, di, dw, dx, 1, q, hidden, inter, 1, 1, act, b1, b2, 0);
    download(out, dy, (size_t)hidden * 4);
}

static void k3_moe_routed_impl(float *out, int *idx, float *wt, const float *x, int T, const float *router_w,
                   const float *bias, const K3ExpertQ *bank, int hidden, int inter, int n_experts,
                   int topk, int renorm, float routed_scale, int act, float b1, float b2, int prec)
{
    if (T <= 0) return;
    if (topk < 1 || topk > K3_MAX_TOPK) {
        fprintf(stderr, "k3: FATAL, k3_moe_routed called with topk=%d outside 1..%d.\n", topk,
                K3_MAX_TOPK);
        abort();
    }
    mxfp4_preconditions(hidden, 32);
    mxfp4_preconditions(inter, 32);
    lib_init();
    const float *dW = (const float *)weights(B_RW, router_w, (size_t)n_experts * hidden * 4);
    const float *db = bias ? (const float *)weights(B_BIAS, bias, (size_t)n_experts * 4) : NULL;
    const float *dx = (const float *)upload(B_X, x, (size_t)T * hidden * 4);
    int *di = (int *)buf(B_IDX, (size_t)T * topk * 4);
    float *dwt = (float *)buf(B_WT, (size_t)T * topk * 4);
    const size_t wsb = k3d_router_ws(T, hidden, n_experts);
    check(k3d_router(di, dwt, dx, T, dW, db, hidden, n_experts, topk, renorm, routed_scale,
                     buf(B_WS, wsb), wsb, g_stream),
          "k3_moe_routed router");
    check(k3k_d2h(idx, di, (size_t)T * topk * 4, g_stream), "device to host copy");
    download(wt, dwt, (size_t)T * topk * 4);
    for (int a = 0; a < T * topk; a++)
        if (!expert_ok(&bank[idx[a]])) report_drop(0, idx[a], "token");
    float *dy = (float *)buf(B_OUT, (size_t)T * hidden * 4);
    run_experts_mxfp4(dy, idx, di, dwt, dx, T, bank, hidden, inter, n_experts, topk, act, b1, b2,
                      prec);
    download(out, dy, (size_t)T * hidden * 4);
}

/* ------------------------------------------------------------- LatentMoE ---- */
size_t k3_moe_scratch(const K3Cfg *c)
{
    const int SI = c->moe_inter * c->n_shared;
    return (size_t)2 * c->latent + (size_t)3 * c->moe_inter + (size_t)c->latent +
           (size_t)3 * SI + (size_t)c->hidden;
}

static size_t wbytes(int wdt, int in, int out)
{
    if (wdt == K3_WBF16) return (size_t)in * out * 2;
    if (wdt == K3_WI8) return (size_t)out * (4 + (size_t)in);
    return (size_t)in * out * 4;
}

/* y[t*ldy + o] = W x[t] for a tagged weight matrix (k3_mmw, reference k3.h:289-295). Up to
 * four tokens stream the weights through the vector-unit GEMV; more bf16 tokens go to the
 * matrix-core GEMM with the activations split into two bf16 terms (fp32-accurate). */
static void mmw_on(float *y_d, const float *x_d, int ntok, const void *W, int wdt, int in, int out,
                   int ldy, int slot, int xs_slot, void *stream)
{
    const void *dw = weights(slot, W, wbytes(wdt, in, out));
    int rc;
    if (wdt == K3_WBF16 && ntok > 4 && in % 64 == 0 &&
        (unsigned long long)out * in * 2 < 0x80000000ull && (unsigned long long)ntok * in * 2 < 0x80000000ull) {
        uint16_t *xs = (uint16_t *)buf(xs_slot, (size_t)ntok * in * 4);
        uint16_t *xl = xs + (size_t)ntok * in;
        check(k3k_split_bf16(xs, xl, x_d, (size_t)ntok * in, stream), "activation split");
        rc = k3k_dense_gemm(y_d, ldy, 0, (const uint16_t *)dw, xs, xl, out, ntok, in, NULL, 0, stream);
    } else if (wdt == K3_WBF16) rc = k3k_gemv_bf16(y_d, x_d, (const uint16_t *)dw, in, out, ntok, ldy, stream);
    else if (wdt == K3_WI8) rc = k3k_gemv_q8(y_d, x_d, dw, in, out, ntok, ldy, stream);
    else rc = k3k_gemv_f32(y_d, x_d, (const float *)dw, in, out, ntok, ldy, stream);
    check(rc, "k3_mmw");
}

static void mmw_dev(float *y_d, const float *x_d, int ntok, const void *W, int wdt, int in, int out,
                    int ldy, int slot)
{
    mmw_on(y_d, x_d, ntok, W, wdt, in, out, ldy, slot, B_XS, g_stream);
}

/* ---------------------------------------------------- streamed-expert fetching ---- */
#define MOE_DEV_BLOCK 1024    /* tokens per device pass of the experts (bounds contrib) */

/* The experts of one MoE call, fetched through K3ExpertSrc in exactly the order the
 * reference calls it, so a source sees the same get / getmany / resident sequence and the
 * same drops are counted:
 *   k3_moe (k3_ops.c:576-626), per token: the cache-only compaction through resident(),
 *     getmany(idx, nk) unless cache-only, then get() (resident() when cache-only) for
 *     every slot j < nk; a failed get() is one drop for that (token, slot);
 *   moe_prefill_chunk (k3_ops.c:728-781), per 64-token chunk: getmany over the chunk's
 *     unique experts in first-seen (t, j) order, then one get() per unique expert; a
 *     failed get() is one drop for the chunk and empties every slot of the chunk that
 *     selected it (a chunk of one token goes through the per-token form, :710-713).
 * Each expert's bytes go to the device on its first successful fetch of the call (or, from
 * this library's HBM bank, are used where they lie), before the next callback can recycle
 * them. didx is the device copy of the routing: -1 marks a slot that contributes nothing
 * (dropped, filtered by the cache-only routing, or past the kept slots). */
typedef struct {
    const K3MoeW *w;
    int L, I, N, K, T;
    int bank_layout;          /* -1: the source hands out host pointers; else K3_BANK_* */
    QPtr *bank;               /* [N] device pointers of the experts fetched since the last pass */
    char *arena;
    size_t off;
    int *hidx, *didx;
    float *hwt;
    /* the device passes: assignments computed so far, one pass's routing, the device
     * aggregate [T][L], latent activations, routing and weights */
    unsigned char *done;
    int *pidx;
    int passes;
    float *dacc;
    const float *dz;
    int *di;
    float *dwt;
    float b1, b2;
} Fetch;

/* One device pass over the assignments whose experts have been fetched since the last pass
 * and that no earlier pass has computed (every other slot -1: it contributes nothing). The
 * first pass writes the aggregate, later ones add onto it. */
static void run_fetched(Fetch *f)
{
    const int L = f->L, K = f->K, T = f->T;
    const size_t TK = (size_t)T * K;
    int any = 0;
    for (size_t a = 0; a < TK; a++) {
        const int e = f->didx[a];
        const int ready = !f->done[a] && e >= 0 && e < f->N && f->bank[e].p1;
        f->pidx[a] = ready ? e : -1;
        if (ready) {
            f->done[a] = 1;
            any = 1;
        }
    }
    if (!any && f->passes > 0) return;
    float *dst = f->passes == 0 ? f->dacc : (float *)buf(B_SDN, (size_t)T * L * 4);
    check(k3k_h2d(f->di, f->pidx, TK * 4, g_stream), "host to device copy");
    check(k3k_h2d(f->dwt, f->hwt, TK * 4, g_stream), "host to device copy");
    const int layout = f->bank_layout >= 0 ? f->bank_layout : K3D_LAYOUT_ROWS;
    for (int b0 = 0; b0 < T; b0 += MOE_DEV_BLOCK) {
        const int nb = T - b0 < MOE_DEV_BLOCK ? T - b0 : MOE_DEV_BLOCK;
        const size_t o = (size_t)b0 * K;
        run_bank(dst + (size_t)b0 * L, f->pidx + o, f->di + o, f->dwt + o, f->dz + (size_t)b0 * L, nb,
                 f->bank, L, f->I, f->N, K, K3_ACT_SITU, f->b1, f->b2, 0, layout);
    }
    if (f->passes > 0) {
        check(k3k_axpy_rows(f->dacc, dst, (size_t)T * L, g_stream), "aggregate");
        check(k3k_sync(g_stream), "synchronize");
    }
    f->passes++;
}

static int fetch(Fetch *f, int e, int via_resident)
{
    K3ExpertSrc *s = f->w->src;
    K3ExpertQ q;
    memset(&q, 0, sizeof q);
    int miss;
    /* An HBM bank whose slots this call all holds: compute what is fetched, release the
     * slots, then fetch (the reference's cache multiplies each expert before its next get,
     * so it never needs more than topk + 1 slots; k3_cache.c:305) */
    if (!via_resident && f->bank_layout >= 0 && k3_bank_full(s, f->w->layer, e)) {
        run_fetched(f);
        k3_bank_call(s, 0);
        k3_bank_call(s, 1);
        memset(f->bank, 0, (size_t)f->N * sizeof(QPtr));
    }
    if (via_resident) miss = !s->resident || !s->resident(s, f->w->layer, e, &q);
    else miss = s->get(s, f->w->layer, e, &q) != 0;
    /* a source that reports success with a missing tensor is treated as a failed fetch
     * (the reference would dereference the NULL pointer) */
    if (miss || !expert_ok(&q) || e < 0 || e >= f->N) return 0;
    if (!f->bank[e].p1) {
        if (f->bank_layout >= 0) {
            f->bank[e].p1 = q.p1; f->bank[e].s1 = q.s1; f->bank[e].p3 = q.p3;
            f->bank[e].s3 = q.s3; f->bank[e].p2 = q.p2; f->bank[e].s2 = q.s2;
        } else {
            resolve_expert(&f->bank[e], &q, f->L, f->I, f->arena, &f->off);
            check(k3k_sync(g_stream), "synchronize");   /* bytes taken before the next get() */
        }
    }
    return 1;
}

/* k3_moe's per-token form for token t. */
static void fetch_token(Fetch *f, int t)
{
    const K3MoeW *w = f->w;
    const int K = f->K;
    int *it = f->hidx + (size_t)t * K, *dt = f->didx + (size_t)t * K;
    float *wtt = f->hwt + (size_t)t * K;
    int nk = K;
    if (w->cache_only && w->src->resident) {
        int m = 0;
        float wsum = 0.0f;
        for (int j = 0; j < K; j++)
            if (w->src->resident(w->src, w->layer, it[j], NULL)) {
                it[m] = it[j];
                wtt[m] = wtt[j];
                wsum += wtt[j];
                m++;
            }
        nk = m;
        if (wsum > 0.0f)
            for (int j = 0; j < nk; j++) wtt[j] /= wsum;
    }
    if (!w->cache_only && w->src->getmany) w->src->getmany(w->src, w->layer, it, nk);
    for (int j = 0; j < K; j++) dt[j] = -1;
    for (int j = 0; j < nk; j++) {
        if (fetch(f, it[j], w->cache_only)) {
            dt[j] = it[j];
        } else if (!w->cache_only) {
            report_drop(w->layer, it[j], "token");
        }
    }
}

/* moe_prefill_chunk's fetch for the n-token chunk starting at t0. */
static void fetch_chunk(Fetch *f, int t0, int n, int *uniq, unsigned char *seen)
{
    const K3MoeW *w = f->w;
    const int K = f->K;
    const size_t a0 = (size_t)t0 * K, a1 = (size_t)(t0 + n) * K;
    int nu = 0;
    memset(seen, 0, (size_t)f->N);
    for (size_t a = a0; a < a1; a++) {
        const int e = f->hidx[a];
        f->didx[a] = e;
        if (e >= 0 && e < f->N && !seen[e]) {
            seen[e] = 1;
            uniq[nu++] = e;
        }
    }
    if (w->src->getmany) w->src->getmany(w->src, w->layer, uniq, nu);
    for (int u = 0; u < nu; u++) {
        const int e = uniq[u];
        if (fetch(f, e, 0)) continue;
        report_drop(w->layer, e, "chunk");
        for (size_t a = a0; a < a1; a++)
            if (f->hidx[a] == e) f->didx[a] = -1;
    }
}

/* Stable LatentMoE over T tokens (reference k3_ops.c:556-656), batched on the device:
 * route all tokens, down-project, run the selected experts expert-major, sum in slot
 * order, RMSNorm the aggregate, up-project, add the unweighted shared expert. The
 * arithmetic per token is the same in both forms, as in the reference; `batched` selects
 * the fetch order and drop accounting of k3_moe_prefill's expert-major chunks over
 * k3_moe's per-token one. idx/wt receive what the reference leaves there: the last
 * token's routing after a per-token pass, nothing after a batched chunk. */

static void moe_latent(float *out, const float *x, const K3MoeW *w, const K3Cfg *c, int T,
                       int *idx_last, float *wt_last, int batched)
{
    const int E = c->hidden, L = c->latent, I = c->moe_inter, K = c->topk, N = c->n_experts;
    const int SI = I * c->n_shared;
    if (T <= 0) return;
    if (K < 1 || K > K3_MAX_TOPK) {
        fprintf(stderr, "k3: FATAL, k3_moe called with topk=%d outside 1..%d.\n", K, K3_MAX_TOPK);
        abort();
    }
    lib_init();
    const size_t TK = (size_t)T * K;
    int *hidx = (int *)malloc(TK * sizeof(int));
    int *didx = (int *)malloc(TK * sizeof(int));
    float *hwt = (float *)malloc(TK * sizeof(float));
    if (!hidx || !didx || !hwt) {
        fprintf(stderr, "k3: FATAL, host allocation in k3_moe failed.\n");
        abort();
    }
    /* 1. route on the full width */
    const float *dx = (const float *)upload(B_X, x, (size_t)T * E * 4);
    const float *dW = (const float *)weights(B_RW, w->gate, (size_t)N * E * 4);
    const float *db = w->bias ? (const float *)weights(B_BIAS, w->bias, (size_t)N * 4) : NULL;
    int *di = (int *)buf(B_IDX, TK * 4);
    float *dwt = (float *)buf(B_WT, TK * 4);
    {
        const size_t wsb = k3d_router_ws(T, E, N);
        check(k3d_router(di, dwt, dx, T, dW, db, E, N, K, c->moe_renorm, c->routed_scale,
                         buf(B_WS, wsb), wsb, g_stream),
              "k3_moe router");
    }
    /* the routing comes back through pinned memory; the host waits for it alone, while the
     * device goes on with the down-projection */
    {
        char *pin = (char *)pinned(TK * 8);
        check(k3k_d2h(pin, di, TK * 4, g_stream), "device to host copy");
        check(k3k_d2h(pin + TK * 4, dwt, TK * 4, g_stream), "device to host copy");
        check(k3k_event_record(g_pin_ev, g_stream), "event");
    }
    /* 2. down-project into the latent space */
    float *dz = (float *)buf(B_Z, (size_t)T * L * 4);
    mmw_dev(dz, dx, T, w->down, w->wdt, E, L, L, B_P);
    /* 6. (ahead) the shared expert depends on x alone: with its weights resident it runs on
     * the library stream's side stream, forked after the routing and the down-projection
     * (the critical path), beside the routed experts, and joined before its sum is added */
    const size_t wsh = wbytes(w->wdt, E, SI);
    const int shared = SI > 0 && w->sh1 && w->sh3 && w->sh2;
    const int shared_side = shared && k3_dev_lookup(w->sh1) && k3_dev_lookup(w->sh3) &&
                            k3_dev_lookup(w->sh2) && wsh > 0;
    float *sdn = NULL;
    if (shared_side) {
        void *side = NULL;
        check(k3k_fork(g_stream, &side), "fork");
        float *sgu = (float *)buf(B_SGU, (size_t)T * 2 * SI * 4);
        float *sact = (float *)buf(B_SACT, (size_t)T * SI * 4);
        sdn = (float *)buf(B_SSDN, (size_t)T * E * 4);
        mmw_on(sgu, dx, T, w->sh1, w->wdt, E, SI, 2 * SI, B_P, B_SXS, side);
        mmw_on(sgu + SI, dx, T, w->sh3, w->wdt, E, SI, 2 * SI, B_P, B_SXS, side);
        check(k3k_act(sact, sgu, SI, T, K3_ACT_SITU, c->situ_b1, c->situ_b2, side), "shared act");
        mmw_on(sdn, sact, T, w->sh2, w->wdt, SI, E, E, B_P, B_SXS, side);
    }

    check(k3k_event_sync(g_pin_ev), "routing copy");
    memcpy(hidx, g_pin, TK * 4);
    memcpy(hwt, (char *)g_pin + TK * 4, TK * 4);

    /* 3. routed experts, weighted sum in slot order */
    float *dacc = (float *)buf(B_ACC, (size_t)T * L * 4);
    int wrote_last = 0;
    if (w->src) {
        Fetch f;
        memset(&f, 0, sizeof f);
        f.w = w;
        f.L = L;
        f.I = I;
        f.N = N;
        f.K = K;
        f.T = T;
        f.hidx = hidx;
        f.didx = didx;
        f.hwt = hwt;
        f.dacc = dacc;
        f.dz = dz;
        f.di = di;
        f.dwt = dwt;
        f.b1 = c->situ_b1;
        f.b2 = c->situ_b2;
        for (size_t a = 0; a < TK; a++) didx[a] = -1;
        f.bank_layout = k3_bank_layout(w->src, L, I);
        if (f.bank_layout == -2) {
            fprintf(stderr, "k3: FATAL, k3_moe: the HBM expert bank holds experts of another "
                            "shape than latent=%d x moe_inter=%d.\n", L, I);
            abort();
        }
        f.bank = (QPtr *)calloc((size_t)N, sizeof(QPtr));
        f.done = (unsigned char *)calloc(TK, 1);
        f.pidx = (int *)malloc(TK * sizeof(int));
        int *uniq = (int *)malloc(TK * sizeof(int));
        unsigned char *seen = (unsigned char *)calloc((size_t)N, 1);
        if (!f.bank || !f.done || !f.pidx || !uniq || !seen) {
            fprintf(stderr, "k3: FATAL, host allocation in k3_moe failed.\n");
            abort();
        }
        if (f.bank_layout < 0) {
            /* upper bound of the upload arena: every expert the routing names, once */
            int nu = 0;
            for (size_t a = 0; a < TK; a++) {
                const int e = hidx[a];
                if (e >= 0 && e < N && !seen[e]) { seen[e] = 1; nu++; }
            }
            const size_t per_expert = 2 * (pk_bytes(I, L) + sc_bytes(I, L)) + pk_bytes(L, I) +
                                      sc_bytes(L, I) + 6 * 512;
            f.arena = nu ? (char *)buf(B_ARENA, (size_t)nu * per_expert) : NULL;
        }
        k3_bank_call(w->src, 1);
        if (batched) {
            for (int t0 = 0; t0 < T; t0 += 64) {
                const int n = T - t0 < 64 ? T - t0 : 64;
                if (n == 1) {
                    fetch_token(&f, t0);
                    wrote_last = 1;
                } else {
                    fetch_chunk(&f, t0, n, uniq, seen);
                }
            }
        } else {
            for (int t = 0; t < T; t++) fetch_token(&f, t);
            wrote_last = 1;
        }
        /* the assignments not computed yet, on the routing the device uses: kept slots,
         * renormalised weights */
        run_fetched(&f);
        k3_bank_call(w->src, 0);
        free(f.bank);
        free(f.done);
        free(f.pidx);
        free(uniq);
        free(seen);
    } else {
        /* Resident fp32 bank (fixtures only in the reference, k3_ops.c:632-640). */
        const size_t per13 = (size_t)I * L, per2 = (size_t)L * I;
        const float *w1 = (const float *)weights(B_W2, w->w1, per13 * N * 4);
        const float *w3 = (const float *)weights(B_W3, w->w3, per13 * N * 4);
        const float *w2 = (const float *)weights(B_T2, w->w2, per2 * N * 4);
        float *contrib = (float *)buf(B_T0, TK * L * 4);
        float *gu = (float *)buf(B_T1, (size_t)2 * I * 4);
        float *a = (float *)buf(B_FACT, (size_t)I * 4);     /* not B_SGU: the side stream's */
        for (int t = 0; t < T; t++)
            for (int j = 0; j < K; j++) {
                const int e = hidx[t * K + j];
                if (e < 0 || e >= N) continue;
                const float *zt = dz + (size_t)t * L;
                check(k3k_gemv_f32(gu, zt, w1 + (size_t)e * per13, L, I, 1, I, g_stream), "expert w1");
                check(k3k_gemv_f32(gu + I, zt, w3 + (size_t)e * per13, L, I, 1, I, g_stream), "expert w3");
                check(k3k_act(a, gu, I, 1, K3_ACT_SITU, c->situ_b1, c->situ_b2, g_stream), "expert act");
                check(k3k_gemv_f32(contrib + (size_t)(t * K + j) * L, a, w2 + (size_t)e * per2, I, L, 1,
                                   L, g_stream),
                      "expert w2");
            }
        check(k3k_combine(dacc, contrib, dwt, di, NULL, N, T, K, L, g_stream), "combine");
        wrote_last = 1;
    }

    /* 4. RMSNorm of the aggregate, 5. up-project */
    if (c->latent_norm) {
        const float *dn = (const float *)weights(B_T1, w->latent_norm, (size_t)L * 4);
        check(k3k_rmsnorm(dacc, dacc, dn, L, T, c->rms_eps, g_stream), "latent rmsnorm");
    }
    float *dout = (float *)buf(B_OUT, (size_t)T * E * 4);
    mmw_dev(dout, dacc, T, w->up, w->wdt, L, E, E, B_P);

    /* 6. shared expert on the original input, added unweighted */
    if (shared_side) {
        check(k3k_join(g_stream), "join");
        check(k3k_axpy_rows(dout, sdn, (size_t)T * E, g_stream), "shared add");
    } else if (shared) {
        float *sgu = (float *)buf(B_SGU, (size_t)T * 2 * SI * 4);
        float *sact = (float *)buf(B_SACT, (size_t)T * SI * 4);
        sdn = (float *)buf(B_SSDN, (size_t)T * E * 4);
        mmw_dev(sgu, dx, T, w->sh1, w->wdt, E, SI, 2 * SI, B_P);
        mmw_dev(sgu + SI, dx, T, w->sh3, w->wdt, E, SI, 2 * SI, B_P);
        check(k3k_act(sact, sgu, SI, T, K3_ACT_SITU, c->situ_b1, c->situ_b2, g_stream), "shared act");
        mmw_dev(sdn, sact, T, w->sh2, w->wdt, SI, E, E, B_P);
        check(k3k_axpy_rows(dout, sdn, (size_t)T * E, g_stream), "shared add");
    }
    download(out, dout, (size_t)T * E * 4);
    if (wrote_last) {
        if (idx_last) memcpy(idx_last, hidx + (size_t)(T - 1) * K, (size_t)K * sizeof(int));
        if (wt_last) memcpy(wt_last, hwt + (size_t)(T - 1) * K, (size_t)K * sizeof(float));
    }
    free(hidx);
    free(didx);
    free(hwt);
}

void k3_moe(float *out, const float *x, const K3MoeW *w, const K3Cfg *c, int T, int *idx,
            float *wt, float *scratch)
{
    (void)scratch;
    k3h_lock();
    moe_latent(out, x, w, c, T, idx, wt, 0);
    k3h_unlock();
}

void k3_moe_prefill(float *out, const float *x, const K3MoeW *w, const K3Cfg *c, int T, int *idx,
                    float *wt, float *scratch)
{
    (void)scratch;
    /* the reference's conditions for its batched form (k3_ops.c:693-702) */
    const int batched = w->src && T > 1 && !w->cache_only && !getenv("K3_NO_BATCH_PREFILL");
    k3h_lock();
    moe_latent(out, x, w, c, T, idx, wt, batched);
    k3h_unlock();
}

/* ------------------------------------------ locked entry points (see the top) ---- */
void k3_matmul(float *y, const float *x, const float *W, int in, int out)
{
    k3h_lock();
    k3_matmul_impl(y, x, W, in, out);
    k3h_unlock();
}

void k3_matmul_bf16(float *y, const float *x, const uint16_t *W, int in, int out)
{
    k3h_lock();
    k3_matmul_bf16_impl(y, x, W, in, out);
    k3h_unlock();
}

void k3_matmul_q8(float *y, const float *x, const void *W, int in, int out)
{
    k3h_lock();
    k3_matmul_q8_impl(y, x, W, in, out);
    k3h_unlock();
}

void k3_matmul_mxfp4(float *y, const float *x, const unsigned char *packed,
                     const unsigned char *scales, int in, int rows, int group)
{
    k3h_lock();
    k3_matmul_mxfp4_impl(y, x, packed, scales, in, rows, group);
    k3h_unlock();
}

void k3_mxfp4_dequant(float *out, const unsigned char *packed, const unsigned char *scales,
                      int rows, int pcols, int group)
{
    k3h_lock();
    k3_mxfp4_dequant_impl(out, packed, scales, rows, pcols, group);
    k3h_unlock();
}

void k3_router(int *idx, float *w, const float *x, const float *W, const float *bias,
               int hidden, int n_experts, int topk, int renorm, float routed_scale)
{
    k3h_lock();
    k3_router_impl(idx, w, x, W, bias, hidden, n_experts, topk, renorm, routed_scale);
    k3h_unlock();
}

void k3_situ_glu(float *y, const float *x, int n, float b1, float b2)
{
    k3h_lock();
    k3_situ_glu_impl(y, x, n, b1, b2);
    k3h_unlock();
}

void k3_rmsnorm(float *y, const float *x, const float *w, int n, float eps)
{
    k3h_lock();
    k3_rmsnorm_impl(y, x, w, n, eps);
    k3h_unlock();
}

void k3_expert_ffn(float *out, const float *x, const K3ExpertQ *q, int hidden, int inter, int act,
                   float b1, float b2, float wt)
{
    k3h_lock();
    k3_expert_ffn_impl(out, x, q, hidden, inter, act, b1, b2, wt);
    k3h_unlock();
}

void k3_moe_routed(float *out, int *idx, float *wt, const float *x, int T, const float *router_w,
                   const float *bias, const K3ExpertQ *bank, int hidden, int inter, int n_experts,
                   int topk, int renorm, float routed_scale, int act, float b1, float b2, int prec)
{
    k3h_lock();
    k3_moe_routed_impl(out, idx, wt, x, T, router_w, bias, bank, hidden, inter, n_experts, topk,
                       renorm, routed_scale, act, b1, b2, prec);
    k3h_unlock();
}

int k3_dev_register(const void *host, size_t bytes)
{
    k3h_lock();
    int r = k3_dev_register_impl(host, bytes);
    k3h_unlock();
    return r;
}

int k3_dev_unregister(const void *host)
{
    k3h_lock();
    int r = k3_dev_unregister_impl(host);
    k3h_unlock();
    return r;
}

void *k3_dev_lookup(const void *host)
{
    k3h_lock();
    void *r = k3_dev_lookup_impl(host);
    k3h_unlock();
    return r;
}
