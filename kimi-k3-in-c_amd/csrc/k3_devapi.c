/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_devapi.c -- the device-pointer entry points (include/k3_dev.h), in C99 over the
 * kernel ABI (k3k.h). Each call carves its scratch from the caller's workspace with the
 * same layout function that sizes it, so sizing and use cannot drift apart.
 */
#include "k3_dev.h"
#include "k3.h"
#include "k3k.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

extern const int k3_expf_exc_n;
extern const uint32_t k3_expf_exc[];

static __thread char g_msg[512];   /* the last error, per thread */

static int fail(const char *what)
{
    snprintf(g_msg, sizeof g_msg, "%s: %s", what, k3k_error());
    return -1;
}

static int bad(const char *what)
{
    snprintf(g_msg, sizeof g_msg, "%s", what);
    return -2;
}

const char *k3d_error(void) { return g_msg; }

int k3dx_bad(const char *msg) { return bad(msg); }

static int exc_table(const K3kExc **out);

/* Device selection and the one-time uploads (router tables), so that no later entry point
 * allocates or synchronises and the layer can be captured in a graph. */
int k3d_init(void)
{
    if (k3k_init()) return fail("init");
    if (k3k_side_init()) return fail("init: side stream");
    if (k3s_static_setup()) return fail("init: static workspace");
    const K3kExc *e;
    return exc_table(&e);
}
void *k3d_stream_create(void)
{
    if (k3d_init()) return NULL;
    void *s = k3k_stream_create();
    if (!s) fail("k3d_stream_create");
    return s;
}
int k3d_stream_destroy(void *s) { return k3k_stream_destroy(s) ? fail("k3d_stream_destroy") : 0; }
int k3d_graph_begin(void *s) { return k3k_graph_begin(s) ? fail("k3d_graph_begin") : 0; }
int k3d_graph_end(void *s, void **exec) { return k3k_graph_end(s, exec) ? fail("k3d_graph_end") : 0; }
int k3d_graph_launch(void *exec, void *s) { return k3k_graph_launch(exec, s) ? fail("k3d_graph_launch") : 0; }
int k3d_graph_destroy(void *exec) { return k3k_graph_destroy(exec) ? fail("k3d_graph_destroy") : 0; }
void *k3d_malloc(size_t bytes)
{
    if (k3d_init()) return NULL;
    void *p = k3k_malloc(bytes);
    if (!p) fail("k3d_malloc");
    return p;
}
int k3d_free(void *p) { return k3k_free(p) ? fail("k3d_free") : 0; }
int k3d_h2d(void *d, const void *h, size_t n, void *s) { return k3k_h2d(d, h, n, s) ? fail("h2d") : 0; }
int k3d_d2h(void *h, const void *d, size_t n, void *s) { return k3k_d2h(h, d, n, s) ? fail("d2h") : 0; }
int k3d_sync(void *s) { return k3k_sync(s) ? fail("sync") : 0; }

int k3d_prof_begin(int max_marks) { return k3k_prof_enable(max_marks) ? fail("prof_begin") : 0; }
int k3d_prof_end(double *ms, int *count, int n_stages)
{
    return k3k_prof_collect(ms, count, n_stages) ? fail("prof_end") : 0;
}
int k3d_prof_mark(void *stream, int stage) { return k3k_prof_mark(stream, stage) ? fail("prof_mark") : 0; }
int k3d_stamps_begin(void *dbuf, size_t bytes) { return k3k_stamps_enable(dbuf, bytes); }
int k3d_stamps_end(int *kinds, int *grids, int max, int *n) { return k3k_stamps_collect(kinds, grids, max, n); }

/* The libm exception table of the router score and its bucket index, uploaded once per
 * process. */
static K3kExc g_exc;
static int g_exc_ready = 0;

static int exc_table(const K3kExc **out)
{
    if (!g_exc_ready) {
        const int n = k3_expf_exc_n;
        memset(&g_exc, 0, sizeof g_exc);
        if (n > 0) {
            const uint32_t kmin = k3_expf_exc[0], kmax = k3_expf_exc[2 * (n - 1)];
            const uint32_t base = kmin >> 12, nb = (kmax >> 12) - base + 1;
            uint32_t *index = (uint32_t *)malloc((size_t)(nb + 1) * 4);
            if (!index) return bad("router exception index: out of host memory");
            uint32_t i = 0;
            for (uint32_t bk = 0; bk <= nb; bk++) {
                while (i < (uint32_t)n && (k3_expf_exc[2 * i] >> 12) - base < bk) i++;
                index[bk] = i;
            }
            /* membership bitmap over |key| in [mmin, mmax], one word array per sign */
            uint32_t mmin = 0xffffffffu, mmax = 0;
            for (int j = 0; j < n; j++) {
                const uint32_t m = k3_expf_exc[2 * j] & 0x7fffffffu;
                if (m < mmin) mmin = m;
                if (m > mmax) mmax = m;
            }
            const uint32_t mwords = ((mmax - mmin) >> 5) + 1;
            uint32_t *bits = (uint32_t *)calloc((size_t)2 * mwords, 4);
            if (!bits) {
                free(index);
                return bad("router exception bitmap: out of host memory");
            }
            for (int j = 0; j < n; j++) {
                const uint32_t key = k3_expf_exc[2 * j], bi = (key & 0x7fffffffu) - mmin;
                bits[(size_t)(key >> 31) * mwords + (bi >> 5)] |= 1u << (bi & 31);
            }
            uint32_t *dp = (uint32_t *)k3k_malloc((size_t)2 * n * 4);
            uint32_t *di = (uint32_t *)k3k_malloc((size_t)(nb + 1) * 4);
            uint32_t *db = (uint32_t *)k3k_malloc((size_t)2 * mwords * 4);
            int rc = !dp || !di || !db || k3k_h2d(dp, k3_expf_exc, (size_t)2 * n * 4, NULL) ||
                     k3k_h2d(di, index, (size_t)(nb + 1) * 4, NULL) ||
                     k3k_h2d(db, bits, (size_t)2 * mwords * 4, NULL) || k3k_sync(NULL);
            free(index);
            free(bits);
            if (rc) return fail("router exception table upload");
            g_exc.bits = db;
            g_exc.mmin = mmin;
            g_exc.mwords = mwords;
            g_exc.pairs = dp;
            g_exc.index = di;
            g_exc.kmin = kmin;
            g_exc.kmax = kmax;
            g_exc.base = base;
            g_exc.n = n;
        }
        g_exc_ready = 1;
    }
    *out = &g_exc;
    return 0;
}

/* ---- workspace carving ------------------------------------------------------------- */
typedef struct {
    char *base;
    size_t off;
} Carve;

static void *take(Carve *c, size_t bytes)
{
    const size_t o = (c->off + 255u) & ~(size_t)255u;
    c->off = o + (bytes ? bytes : 1);
    return c->base ? (void *)(c->base + o) : NULL;
}

/* ---- MXFP4 GEMV / GEMM --------------------------------------------------------------- */
typedef struct {
    uint16_t *xhi, *xlo;
} MxWs;

static size_t mx_layout(Carve *c, MxWs *w, int ntok, int in)
{
    w->xhi = (uint16_t *)take(c, (size_t)ntok * in * 2);
    w->xlo = (uint16_t *)take(c, (size_t)ntok * in * 2);
    return c->off;
}

size_t k3d_matmul_mxfp4_ws(int ntok, int in)
{
    Carve c = {NULL, 0};
    MxWs w;
    return mx_layout(&c, &w, ntok, in);
}

int k3d_matmul_mxfp4(float *y, const float *x, int ntok, const uint8_t *packed,
                     const uint8_t *scales, int in, int rows, int prec, void *ws, size_t ws_bytes,
                     void *stream)
{
    if (in <= 0 || (in % 32) || rows < 0 || ntok < 0) return bad("k3d_matmul_mxfp4: need in % 32 == 0");
    if (ntok == 0 || rows == 0) return 0;
    if (ws_bytes < k3d_matmul_mxfp4_ws(ntok, in)) return bad("k3d_matmul_mxfp4: workspace too small");
    Carve c = {(char *)ws, 0};
    MxWs w;
    mx_layout(&c, &w, ntok, in);
    K3kMxArgs a;
    memset(&a, 0, sizeof a);
    a.packed = packed;
    a.scales = scales;
    if (k3k_mx_small_ok(ntok, in, prec == 0 ? 2 : 1, rows, x)) {
        a.xf32 = x;                 /* one or two tokens: the kernel splits x itself */
    } else {
        if (k3k_split_bf16(w.xhi, prec == 0 ? w.xlo : NULL, x, (size_t)ntok * in, stream))
            return fail("split");
        a.xhi = w.xhi;
        a.xlo = w.xlo;
    }
    a.y = y;
    a.ntok = ntok;
    a.ldy = rows;
    a.rows = rows;
    a.K = in;
    a.nsplit = prec == 0 ? 2 : 1;
    k3k_prof_mark(stream, K3D_STAGE_BEGIN);
    if (k3k_mx_gemm(K3K_MX_PLAIN, &a, stream)) return fail("mx_gemm");
    k3k_prof_mark(stream, K3D_STAGE_GEMV);
    return 0;
}

int k3d_matmul_f32(float *y, const float *x, int ntok, const float *W, int in, int out, void *stream)
{
    k3k_prof_mark(stream, K3D_STAGE_BEGIN);
    if (k3k_gemv_f32(y, x, W, in, out, ntok, out, stream)) return fail("gemv_f32");
    k3k_prof_mark(stream, K3D_STAGE_GEMV);
    return 0;
}

int k3d_matmul_bf16(float *y, const float *x, int ntok, const uint16_t *W, int in, int out,
                    void *stream)
{
    k3k_prof_mark(stream, K3D_STAGE_BEGIN);
    if (k3k_gemv_bf16(y, x, W, in, out, ntok, out, stream)) return fail("gemv_bf16");
    k3k_prof_mark(stream, K3D_STAGE_GEMV);
    return 0;
}

/* ---- router -------------------------------------------------------------------------- */
typedef struct {
    double *part;
    float *rbound;
    int *nrecomp;
    int *ctr;                   /* the final kernel's arrival counter, when it gathers */
    int chunk;
    void *i8;                   /* scratch of the int8 partials (NULL: the fp64 ones) */
} RtWs;

static size_t router_layout(Carve *c, RtWs *w, int T, int hidden, int n_experts)
{
    const int c8 = k3k_router_i8_chunk(T, hidden, n_experts);
    w->chunk = c8 ? c8 : k3k_router_chunk(T, hidden, n_experts);
    const size_t ks = (size_t)((hidden + w->chunk - 1) / w->chunk);
    /* chunk partials, or (a few tokens) one 16-byte scored record per logit */
    w->part = (double *)take(c, (ks < 2 ? 2 : ks) * T * n_experts * 8);
    w->rbound = (float *)take(c, ks * T * n_experts * 4);
    w->nrecomp = (int *)take(c, (size_t)T * 4);
    w->ctr = (int *)take(c, 4);
    w->i8 = c8 ? take(c, k3k_router_i8_bytes(T, hidden, n_experts, c8)) : NULL;
    return c->off;
}

size_t k3d_router_ws(int T, int hidden, int n_experts)
{
    Carve c = {NULL, 0};
    RtWs w;
    return router_layout(&c, &w, T, hidden, n_experts);
}

/* gather (may be NULL): the router's final kernel also runs the expert-major gather */
static int router_run(int *idx, float *wt, const float *x, int T, const float *W,
                      const float *bias, int hidden, int n_experts, int topk, int renorm,
                      float routed_scale, const RtWs *w, const K3kGatherArgs *gather, void *stream)
{
    const K3kExc *exc;
    int rc = exc_table(&exc);
    if (rc) return rc;
    K3kGatherArgs g;
    if (gather) {
        g = *gather;
        g.ctr = w->ctr;
    }
    /* the int8 partials where they apply (16-byte aligned rows), else the fp64 ones with the
     * same chunks */
    if (w->i8 && !((((uintptr_t)x) | ((uintptr_t)W)) % 16)) {
        if (k3k_router_partial_i8(w->part, w->rbound, w->i8, x, T, W, hidden, n_experts, w->chunk,
                                  gather ? w->ctr : NULL, gather ? idx : NULL, gather ? T * topk : 0,
                                  stream))
            return fail("router_partial_i8");
    } else if (k3k_router_partial(w->part, w->rbound, x, T, W, hidden, n_experts, w->chunk,
                                  gather ? w->ctr : NULL, gather ? idx : NULL, gather ? T * topk : 0,
                                  exc, stream)) {
        return fail("router_partial");
    }
    if (k3k_router_final(idx, wt, w->nrecomp, w->part, w->rbound, w->chunk, x, W, bias, T, hidden,
                         n_experts, topk, renorm, routed_scale, exc, gather ? &g : NULL, stream))
        return fail("router_final");
    return 0;
}

int k3d_router_recomputed(int *h_counts, const void *ws, int T, int hidden, int n_experts)
{
    if (T <= 0) return 0;
    Carve c = {(char *)ws, 0};
    RtWs w;
    router_layout(&c, &w, T, hidden, n_experts);
    if (k3k_d2h(h_counts, w.nrecomp, (size_t)T * 4, NULL) || k3k_sync(NULL)) return fail("router_recomputed");
    return 0;
}

int k3d_router_partials(double *h_part, float *h_rbound, int *h_chunk, size_t cap, const void *ws, int T,
                        int hidden, int n_experts)
{
    if (T <= 4 || k3k_router_small(T, hidden)) return bad("k3d_router_partials: a few tokens are scored whole");
    Carve c = {(char *)ws, 0};
    RtWs w;
    router_layout(&c, &w, T, hidden, n_experts);
    const int ks = (hidden + w.chunk - 1) / w.chunk;
    const size_t n = (size_t)ks * T * n_experts;
    if (n > cap) return bad("k3d_router_partials: cap");
    if (k3k_d2h(h_part, w.part, n * 8, NULL) || k3k_d2h(h_rbound, w.rbound, n * 4, NULL) || k3k_sync(NULL))
        return fail("router_partials");
    *h_chunk = w.chunk;
    return ks;
}

int k3d_router(int *idx, float *wt, const float *x, int T, const float *W, const float *bias,
               int hidden, int n_experts, int topk, int renorm, float routed_scale, void *ws,
               size_t ws_bytes, void *stream)
{
    if (T <= 0) return 0;
    if (topk < 1 || topk > K3_MAX_TOPK) return bad("k3d_router: topk outside 1..64");
    if (n_experts < 1 || n_experts > 2048) return bad("k3d_router: n_experts outside 1..2048");
    if (ws_bytes < k3d_router_ws(T, hidden, n_experts)) return bad("k3d_router: workspace too small");
    Carve c = {(char *)ws, 0};
    RtWs w;
    router_layout(&c, &w, T, hidden, n_experts);
    return router_run(idx, wt, x, T, W, bias, hidden, n_experts, topk, renorm, routed_scale, &w, NULL,
                      stream);
}

/* ---- MoE experts ----------------------------------------------------------------------- */
typedef struct {
    uint16_t *xhi, *xlo, *ahi, *alo;
    int *offsets, *perm, *job_expert, *job_off, *job_cnt, *pass_job, *pass_tp, *counts, *ghist;
    int *pass_job2, *pass_tp2;
    float *contrib;
    float *gu;                  /* decode path: gate and up sums [N][2][inter], or NULL */
    int max_passes, max_passes2;
} MoeWs;

/* Tokens per expert pass. The LDS-staged expert kernels need both matrix widths to be
 * multiples of 512: passes of 8 tokens, or of 32 (two MFMA column blocks) when the
 * activations are single bf16 terms and the batch averages at least 8 tokens per expert
 * (prefill). Other shapes run the register-fed kernel (16, row-major bank only). */
/* One-term (prefill) activations at 8-32 tokens per expert on average on a tiled bank: two
 * pass lists (below). */
static int moe_two_lists(int T, int n_experts, int topk, int prec, int layout)
{
    return prec == 1 && layout == K3D_LAYOUT_TILED && (long)T * topk >= 8L * n_experts &&
           (long)T * topk < 32L * n_experts;
}

/* Tokens per expert pass. 8 for decode (fp32-accurate, weight streaming), 16 when the
 * widths are not multiples of 512; one-term (prefill) activations take, for a tiled bank, 8
 * from 8 tokens per expert on average (with the second list), 48 from 32 and 96 from 64;
 * for a row-major bank 32 from 8. Sizing: a row-major bank's first list has at most N / 32
 * passes beyond one per expert; a tiled bank's at most N / 8 where there is no second list,
 * and one per expert where there is (its experts hold at most 8 assignments). */
static int moe_pass_tok(int T, int hidden, int inter, int n_experts, int topk, int prec, int layout)
{
    if (hidden % 512 || inter % 512) return 16;
    if (prec == 1 && layout == K3D_LAYOUT_TILED && (long)T * topk >= 64L * n_experts) return 96;
    if (prec == 1 && layout == K3D_LAYOUT_TILED && (long)T * topk >= 32L * n_experts) return 48;
    if (moe_two_lists(T, n_experts, topk, prec, layout)) return 8;
    if (prec == 1 && (long)T * topk >= 8L * n_experts) return 32;
    return 8;
}

/* The second pass list: where moe_two_lists holds, the experts holding more than pass_tok
 * (8) assignments -- all but the coldest, and the hot ones of a skewed routing -- take the
 * prefill kernel's 96-token passes, so their weights stream once per 96 tokens, and the
 * rest one 8-token pass each on the streaming kernel. (Config 4, 512 tokens with skewed
 * routing: 309 experts of at most 32 assignments in 32-token passes and 21 hot ones in the
 * second list took 1.47 ms for gate/up + down; 282 experts of at most 8 in 8-token passes
 * and 48 in the second list take 1.40 ms.) */
#define MOE_PASS_TOK2 96
static int moe_pass_tok2(int T, int n_experts, int topk, int prec, int layout)
{
    return moe_two_lists(T, n_experts, topk, prec, layout) ? MOE_PASS_TOK2 : 0;
}

/* The decode path (k3k_mx_decode): at most 16 assignments, widths multiples of 512 up to
 * 8192, the tokens 16-byte aligned. */
static int moe_decode_ok(int T, int hidden, int inter, int topk, const float *x)
{
    return (long)T * topk <= 16 && hidden % 512 == 0 && inter % 512 == 0 && hidden <= 8192 &&
           inter <= 8192 && ((uintptr_t)x % 16) == 0;
}

static size_t moe_layout(Carve *c, MoeWs *w, int T, int hidden, int inter, int n_experts, int topk,
                         int prec)
{
    const size_t N = (size_t)T * topk;
    const int maxjobs = (int)(N < (size_t)n_experts ? N : (size_t)n_experts);
    w->max_passes = maxjobs + (int)(N / (size_t)moe_pass_tok(T, hidden, inter, n_experts, topk, prec,
                                                                K3D_LAYOUT_ROWS)) + 1;
    if (!moe_two_lists(T, n_experts, topk, prec, K3D_LAYOUT_TILED)) {
        const int pt = moe_pass_tok(T, hidden, inter, n_experts, topk, prec, K3D_LAYOUT_TILED);
        const int mp = maxjobs + (int)(N / (size_t)pt) + 1;
        if (mp > w->max_passes) w->max_passes = mp;
    }
    w->xhi = (uint16_t *)take(c, (size_t)T * hidden * 2);
    w->xlo = prec == 0 ? (uint16_t *)take(c, (size_t)T * hidden * 2) : NULL;
    w->ahi = (uint16_t *)take(c, N * inter * 2);
    w->alo = prec == 0 ? (uint16_t *)take(c, N * inter * 2) : NULL;
    w->offsets = (int *)take(c, (size_t)(n_experts + 1) * 4);
    w->perm = (int *)take(c, N * 4);
    w->job_expert = (int *)take(c, (size_t)maxjobs * 4);
    w->job_off = (int *)take(c, (size_t)maxjobs * 4);
    w->job_cnt = (int *)take(c, (size_t)maxjobs * 4);
    w->pass_job = (int *)take(c, (size_t)w->max_passes * 4);
    w->pass_tp = (int *)take(c, (size_t)w->max_passes * 4);
    /* second list (one-term activations): experts of more than 8 assignments, each pass of
     * up to 96 tokens -- at most N / 96 full passes plus one per such expert */
    w->max_passes2 = prec == 1 ? (int)(N / MOE_PASS_TOK2 + N / 9 + 2) : 0;
    w->pass_job2 = prec == 1 ? (int *)take(c, (size_t)w->max_passes2 * 4) : NULL;
    w->pass_tp2 = prec == 1 ? (int *)take(c, (size_t)w->max_passes2 * 4) : NULL;
    w->counts = (int *)take(c, (size_t)(4 + K3K_QUEUE_INTS) * 4);
    {
        const size_t gs = k3k_gather_scratch(T, topk, n_experts);
        w->ghist = gs ? (int *)take(c, gs * 4) : NULL;
    }
    w->contrib = (float *)take(c, N * hidden * 4);
    /* the decode path's gate and up sums, when gate and up take workgroups of their own */
    w->gu = N <= 16 ? (float *)take(c, N * 2 * (size_t)inter * 4) : NULL;
    return c->off;
}

size_t k3d_moe_ws(int T, int hidden, int inter, int n_experts, int topk, int prec)
{
    Carve c = {NULL, 0};
    MoeWs w;
    RtWs r;
    moe_layout(&c, &w, T, hidden, inter, n_experts, topk, prec);
    router_layout(&c, &r, T, hidden, n_experts);
    return c.off;
}

static int moe_check(const char *fn, int hidden, int inter, int n_experts, int topk, int layout)
{
    static char msg[160];
    if (n_experts < 1 || n_experts > 2048) {
        snprintf(msg, sizeof msg, "%s: n_experts outside 1..2048", fn);
        return bad(msg);
    }
    if ((hidden % 32) || (inter % 32)) {
        snprintf(msg, sizeof msg, "%s: hidden and inter must be multiples of 32", fn);
        return bad(msg);
    }
    if (topk < 1 || topk > K3_MAX_TOPK) {
        snprintf(msg, sizeof msg, "%s: topk outside 1..64", fn);
        return bad(msg);
    }
    if (layout != K3D_LAYOUT_ROWS && layout != K3D_LAYOUT_TILED) {
        snprintf(msg, sizeof msg, "%s: unknown bank layout %d", fn, layout);
        return bad(msg);
    }
    if (layout == K3D_LAYOUT_TILED && (hidden % 512 || inter % 512)) {
        snprintf(msg, sizeof msg, "%s: a tiled bank needs hidden and inter multiples of 512", fn);
        return bad(msg);
    }
    return 0;
}

/* The router's selection done inside the decode gate/up kernel (a few tokens): the scored
 * records of k3k_router_partial and what the selection needs; idx / wt are written there. */
typedef struct {
    const void *pre;
    const float *rw, *rbias;
    int renorm;
    float rscale;
    const K3kExc *exc;
    int *nrecomp;
    int *idx;
    float *wt;
} RouterSel;

static int moe_experts_ws(float *out, const int *idx, const float *wt, const float *x, int T,
                          const void *bank, int layout, int hidden, int inter, int n_experts,
                          int topk, int act, float b1, float b2, int prec, const MoeWs *w,
                          int *perm_out, int *offsets_out, int *drops_out, const RouterSel *sel,
                          int x_split, int gathered, void *stream)
{
    int *perm = perm_out ? perm_out : w->perm;
    int *offsets = offsets_out ? offsets_out : w->offsets;
    const int pass_tok = moe_pass_tok(T, hidden, inter, n_experts, topk, prec, layout);
    if (moe_decode_ok(T, hidden, inter, topk, x)) {
        /* a few assignments: one workgroup per (assignment, 16-row tile), straight from idx;
         * the gather runs only when its permutation is asked for */
        if ((perm_out || offsets_out) &&
            k3k_gather(offsets, perm, w->job_expert, w->job_off, w->job_cnt, w->pass_job, w->pass_tp,
                       NULL, NULL, w->counts, w->ghist, idx, T, topk, n_experts, bank, pass_tok, 0,
                       stream))
            return fail("gather");
        k3k_prof_mark(stream, K3D_STAGE_GATHER);
        K3kMxArgs a;
        memset(&a, 0, sizeof a);
        a.bank = bank;
        a.layout = layout;
        a.idx = idx;
        a.n_assign = T * topk;
        a.drops = w->counts + 2;
        a.n_experts = n_experts;
        a.topk = topk;
        a.act = act;
        a.b1 = b1;
        a.b2 = b2;
        a.nsplit = prec == 0 ? 2 : 1;
        a.xf32 = x;
        a.ahi = w->ahi;
        a.alo = w->alo;
        a.rows = inter;
        a.K = hidden;
        if (sel) {
            a.sel = 1;
            a.pre = sel->pre;
            a.rw = sel->rw;
            a.rbias = sel->rbias;
            a.renorm = sel->renorm;
            a.rscale = sel->rscale;
            a.exc = *sel->exc;
            a.idx_out = sel->idx;
            a.wt_out = sel->wt;
            a.nrecomp = sel->nrecomp;
        }
        /* one tile per workgroup (a few assignments): gate and up in workgroups of their own,
         * their fp32 sums taken up by the down + combine kernel */
        if (!sel && w->gu &&
            k3k_mx_decode_split_ok(T * topk, topk, a.nsplit, hidden, inter, inter, hidden))
            a.gu = w->gu;
        if (k3k_mx_decode(K3K_MX_GATEUP, &a, stream)) return fail("mx_decode gateup");
        a.sel = 0;
        k3k_prof_mark(stream, K3D_STAGE_GATEUP);
        a.xhi = w->ahi;
        a.xlo = w->alo;
        a.out = out;
        a.wt = wt;
        a.rows = hidden;
        a.K = inter;
        if (k3k_mx_decode_combine_ok(T * topk, topk, a.nsplit, inter, hidden)) {
            /* down and the combine in one kernel */
            if (k3k_mx_decode_combine(&a, stream)) return fail("mx_decode down+combine");
            k3k_prof_mark(stream, K3D_STAGE_DOWN);
        } else {
            a.out = w->contrib;
            if (k3k_mx_decode(K3K_MX_DOWN, &a, stream)) return fail("mx_decode down");
            k3k_prof_mark(stream, K3D_STAGE_DOWN);
            if (k3k_combine(out, w->contrib, wt, idx, bank, n_experts, T, topk, hidden, stream))
                return fail("combine");
        }
        k3k_prof_mark(stream, K3D_STAGE_COMBINE);
        if (drops_out && k3k_d2d(drops_out, w->counts + 2, 4, stream)) return fail("drops");
        return 0;
    }
    /* (the routed layer runs the split beside its router, on the side stream) */
    if (!x_split && k3k_split_bf16(w->xhi, w->xlo, x, (size_t)T * hidden, stream)) return fail("split");
    const int pass_tok2 = moe_pass_tok2(T, n_experts, topk, prec, layout);
    /* (gathered: the router's final kernel has run the gather) */
    if (!gathered &&
        k3k_gather(offsets, perm, w->job_expert, w->job_off, w->job_cnt, w->pass_job, w->pass_tp,
                   w->pass_job2, w->pass_tp2, w->counts, w->ghist, idx, T, topk, n_experts, bank,
                   pass_tok, pass_tok2, stream))
        return fail("gather");
    k3k_prof_mark(stream, K3D_STAGE_GATHER);
    K3kMxArgs a;
    memset(&a, 0, sizeof a);
    a.bank = bank;
    a.pass_tok = pass_tok;
    a.layout = layout;
    a.job_expert = w->job_expert;
    a.job_off = w->job_off;
    a.job_cnt = w->job_cnt;
    a.pass_job = w->pass_job;
    a.pass_tp = w->pass_tp;
    a.n_passes = w->counts + 1;
    a.perm = perm;
    a.topk = topk;
    a.act = act;
    a.b1 = b1;
    a.b2 = b2;
    a.nsplit = prec == 0 ? 2 : 1;
    a.max_passes = w->max_passes;
    /* gate/up: K = hidden, rows = inter, activations are the tokens */
    a.xhi = w->xhi;
    a.xlo = w->xlo;
    a.ahi = w->ahi;
    a.alo = w->alo;
    a.rows = inter;
    a.K = hidden;
    a.n_xrows = T;
    /* the second pass list: same jobs, the prefill kernel's passes */
    K3kMxArgs a2 = a;
    a2.pass_tok = pass_tok2;
    a2.pass_job = w->pass_job2;
    a2.pass_tp = w->pass_tp2;
    a2.n_passes = w->counts + 3;
    a2.max_passes = w->max_passes2;
    /* the second list's gate/up and down run on a side stream beside the first's */
    void *side = NULL;
    if (pass_tok2 && k3k_fork(stream, &side)) return fail("fork");
    a.queue = w->counts + 4;
    a2.queue = w->counts + 4 + 2 * K3K_NXCD_Q;
    if (k3k_mx_gemm(K3K_MX_GATEUP, &a, stream)) return fail("mx_gemm gateup");
    if (pass_tok2 && k3k_mx_gemm(K3K_MX_GATEUP, &a2, side)) return fail("mx_gemm gateup (96)");
    k3k_prof_mark(stream, K3D_STAGE_GATEUP);
    /* down: K = inter, rows = hidden, activations are the assignments */
    a.xhi = w->ahi;
    a.xlo = w->alo;
    a.out = w->contrib;
    a.rows = hidden;
    a.K = inter;
    a.n_xrows = T * topk;
    a.queue = w->counts + 4 + K3K_NXCD_Q;
    if (k3k_mx_gemm(K3K_MX_DOWN, &a, stream)) return fail("mx_gemm down");
    if (pass_tok2) {
        a2.xhi = a.xhi;
        a2.xlo = a.xlo;
        a2.out = a.out;
        a2.rows = a.rows;
        a2.K = a.K;
        a2.n_xrows = a.n_xrows;
        a2.queue = w->counts + 4 + 3 * K3K_NXCD_Q;
        if (k3k_mx_gemm(K3K_MX_DOWN, &a2, side)) return fail("mx_gemm down (96)");
        if (k3k_join(stream)) return fail("join");
    }
    k3k_prof_mark(stream, K3D_STAGE_DOWN);
    if (k3k_combine(out, w->contrib, wt, idx, bank, n_experts, T, topk, hidden, stream)) return fail("combine");
    k3k_prof_mark(stream, K3D_STAGE_COMBINE);
    if (drops_out && k3k_d2d(drops_out, w->counts + 2, 4, stream)) return fail("drops");
    return 0;
}

int k3d_moe_experts(float *out, const int *idx, const float *wt, const float *x, int T,
                    const void *bank, int layout, int hidden, int inter, int n_experts, int topk,
                    int act, float b1, float b2, int prec, void *ws, size_t ws_bytes,
                    int *perm_out, int *offsets_out, int *drops_out, void *stream)
{
    if (T <= 0) return 0;
    int rc = moe_check("k3d_moe_experts", hidden, inter, n_experts, topk, layout);
    if (rc) return rc;
    if (ws_bytes < k3d_moe_ws(T, hidden, inter, n_experts, topk, prec))
        return bad("k3d_moe_experts: workspace too small");
    Carve c = {(char *)ws, 0};
    MoeWs w;
    moe_layout(&c, &w, T, hidden, inter, n_experts, topk, prec);
    k3k_prof_mark(stream, K3D_STAGE_BEGIN);
    return moe_experts_ws(out, idx, wt, x, T, bank, layout, hidden, inter, n_experts, topk, act,
                          b1, b2, prec, &w, perm_out, offsets_out, drops_out, NULL, 0, 0, stream);
}

int k3d_moe_routed(float *out, int *idx, float *wt, const float *x, int T, const float *router_w,
                   const float *bias, const void *bank, int layout, int hidden, int inter,
                   int n_experts, int topk, int renorm, float routed_scale, int act, float b1,
                   float b2, int prec, void *ws, size_t ws_bytes, int *perm_out, int *offsets_out,
                   int *drops_out, void *stream)
{
    if (T <= 0) return 0;
    int rc = moe_check("k3d_moe_routed", hidden, inter, n_experts, topk, layout);
    if (rc) return rc;
    if (ws_bytes < k3d_moe_ws(T, hidden, inter, n_experts, topk, prec))
        return bad("k3d_moe_routed: workspace too small");
    Carve c = {(char *)ws, 0};
    MoeWs w;
    RtWs r;
    moe_layout(&c, &w, T, hidden, inter, n_experts, topk, prec);
    router_layout(&c, &r, T, hidden, n_experts);
    k3k_prof_mark(stream, K3D_STAGE_BEGIN);
    if (moe_decode_ok(T, hidden, inter, topk, x) && k3k_router_small(T, hidden) && n_experts <= 512 &&
        !perm_out && !offsets_out) {
        /* a few tokens: the scored logits, then the decode gate/up kernel selects the
         * experts itself (no selection kernel) and writes idx / wt */
        const K3kExc *exc;
        rc = exc_table(&exc);
        if (rc) return rc;
        if (k3k_router_partial(r.part, r.rbound, x, T, router_w, hidden, n_experts, r.chunk, NULL,
                               NULL, 0, exc, stream))
            return fail("router_partial");
        k3k_prof_mark(stream, K3D_STAGE_ROUTER);
        const RouterSel sel = {r.part, router_w, bias, renorm, routed_scale, exc, r.nrecomp, idx, wt};
        return moe_experts_ws(out, idx, wt, x, T, bank, layout, hidden, inter, n_experts, topk, act,
                              b1, b2, prec, &w, NULL, NULL, drops_out, &sel, 0, 0, stream);
    }
    /* past the decode path the expert kernels take the tokens' bf16 split. It depends on x
     * alone: for large batches it runs on the side stream beside the router (event fork /
     * join, captured by a graph like the rest); below 2^22 elements it runs first on the
     * stream, because there the fork and join cost more than the split (batch 64: 1.105 ->
     * 1.085 ms per step) */
    const int split = !moe_decode_ok(T, hidden, inter, topk, x);
    const int split_side = split && (size_t)T * hidden >= ((size_t)1 << 22);
    if (split) {
        void *side = stream;
        if (split_side && k3k_fork(stream, &side)) return fail("fork");
        if (k3k_split_bf16(w.xhi, w.xlo, x, (size_t)T * hidden, side)) return fail("split");
    }
    /* the expert-major gather runs in the router's final kernel when it can (a launch and its
     * gap fewer): the last of its workgroups to finish sorts every token's idx */
    const int gathered = split && k3k_router_gathers(T, hidden, n_experts, topk);
    K3kGatherArgs ga;
    if (gathered) {
        const int pass_tok = moe_pass_tok(T, hidden, inter, n_experts, topk, prec, layout);
        ga.offsets = offsets_out ? offsets_out : w.offsets;
        ga.perm = perm_out ? perm_out : w.perm;
        ga.job_expert = w.job_expert;
        ga.job_off = w.job_off;
        ga.job_cnt = w.job_cnt;
        ga.pass_job = w.pass_job;
        ga.pass_tp = w.pass_tp;
        ga.pass_job2 = w.pass_job2;
        ga.pass_tp2 = w.pass_tp2;
        ga.counts = w.counts;
        ga.bank = bank;
        ga.topk = topk;
        ga.pass_tok = pass_tok;
        ga.pass_tok2 = moe_pass_tok2(T, n_experts, topk, prec, layout);
        ga.ctr = r.ctr;
    }
    rc = router_run(idx, wt, x, T, router_w, bias, hidden, n_experts, topk, renorm, routed_scale,
                    &r, gathered ? &ga : NULL, stream);
    if (rc) return rc;
    if (split_side && k3k_join(stream)) return fail("join");
    k3k_prof_mark(stream, K3D_STAGE_ROUTER);
    return moe_experts_ws(out, idx, wt, x, T, bank, layout, hidden, inter, n_experts, topk, act,
                          b1, b2, prec, &w, perm_out, offsets_out, drops_out, NULL, split, gathered,
                          stream);
}

/* ---- tiled expert layout ---------------------------------------------------------------- */
int k3d_mxfp4_tiled_size(int rows, int in, size_t *packed_bytes, size_t *scales_bytes)
{
    if (rows <= 0 || in <= 0 || in % 512) return bad("k3d_mxfp4_tiled_size: need rows > 0 and in % 512 == 0");
    const size_t prow = ((size_t)rows + 63) / 64 * 64;   /* groups of four 16-row tiles */
    if (packed_bytes) *packed_bytes = prow * (size_t)in / 2;
    if (scales_bytes) *scales_bytes = prow * (size_t)in / 32;
    return 0;
}

int k3d_mxfp4_tile(uint8_t *tpacked, uint8_t *tscales, const uint8_t *packed,
                   const uint8_t *scales, int rows, int in, void *stream)
{
    if (rows <= 0 || in <= 0 || in % 512) return bad("k3d_mxfp4_tile: need rows > 0 and in % 512 == 0");
    return k3k_mx_tile(tpacked, tscales, packed, scales, rows, in, stream) ? fail("mx_tile") : 0;
}

/* ---- dense (bf16) shared expert ------------------------------------------------------------
 * Two launches of the dense GEMM kernel (k3_gemm.hip) after the activation split: gate and up
 * in one pass over x with the activation and its bf16 split in the epilogue, then down,
 * written or added onto y (one fp32 add of the finished sum, the reference's
 * `ot[i] += sdn[i]`, k3_ops.c:654). */
typedef struct {
    uint16_t *xhi, *xlo, *ahi, *alo;
    float *part;
    size_t part_bytes;
} ShWs;

static size_t shared_layout(Carve *c, ShWs *w, int T, int hidden, int inter, int prec)
{
    w->xhi = (uint16_t *)take(c, (size_t)T * hidden * 2);
    w->xlo = prec == 0 ? (uint16_t *)take(c, (size_t)T * hidden * 2) : NULL;
    w->ahi = (uint16_t *)take(c, (size_t)T * inter * 2);
    w->alo = prec == 0 ? (uint16_t *)take(c, (size_t)T * inter * 2) : NULL;
    /* the GEMMs' K-slice sums (both GEMMs reuse it, one after the other) */
    const size_t pg = k3k_dense_part_bytes(inter, T, hidden, 1), pd = k3k_dense_part_bytes(hidden, T, inter, 0);
    w->part_bytes = pg > pd ? pg : pd;
    w->part = (float *)take(c, w->part_bytes);
    return c->off;
}

size_t k3d_shared_ws(int T, int hidden, int inter, int prec)
{
    Carve c = {NULL, 0};
    ShWs w;
    return shared_layout(&c, &w, T, hidden, inter, prec);
}

int k3d_shared_expert(float *y, int accumulate, const float *x, int T, const uint16_t *w1,
                      const uint16_t *w3, const uint16_t *w2, int hidden, int inter, int act,
                      float b1, float b2, int prec, void *ws, size_t ws_bytes, void *stream)
{
    if (T <= 0) return 0;
    if (hidden % 64 || inter % 64) return bad("k3d_shared_expert: hidden and inter must be multiples of 64");
    if (!w1 || !w3 || !w2) return bad("k3d_shared_expert: missing weights");
    if (ws_bytes < k3d_shared_ws(T, hidden, inter, prec)) return bad("k3d_shared_expert: workspace too small");
    Carve c = {(char *)ws, 0};
    ShWs w;
    shared_layout(&c, &w, T, hidden, inter, prec);
    if (k3k_split_bf16(w.xhi, w.xlo, x, (size_t)T * hidden, stream)) return fail("split");
    if (k3k_dense_gateup(w.ahi, w.alo, w1, w3, w.xhi, w.xlo, inter, T, hidden, act, b1, b2, w.part,
                         w.part_bytes, stream))
        return fail("shared gate/up");
    if (k3k_dense_gemm(y, hidden, accumulate, w2, w.ahi, w.alo, hidden, T, inter, w.part, w.part_bytes,
                       stream))
        return fail("shared down");
    k3k_prof_mark(stream, K3D_STAGE_SHARED);
    return 0;
}
