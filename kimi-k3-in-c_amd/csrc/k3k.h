/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3k.h -- the thin C ABI between the C99 host layer and the HIP kernels.
 *
 * Every function here launches one kernel (or wraps one HIP runtime call) on the given
 * stream and returns 0 or a negative code; k3k_error() describes the last failure. All
 * pointers are DEVICE pointers unless named h_*. Nothing here allocates, except
 * k3k_malloc itself.
 */
#ifndef K3K_H
#define K3K_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime -------------------------------------------------------------------- */
int k3k_init(void);                 /* select device 0 on first use; 0 = ok */
const char *k3k_error(void);
int k3k_device_count(void);
void *k3k_malloc(size_t bytes);     /* NULL on failure */
int k3k_free(void *p);
int k3k_h2d(void *dst, const void *h_src, size_t bytes, void *stream);
int k3k_d2h(void *h_dst, const void *src, size_t bytes, void *stream);
int k3k_d2d(void *dst, const void *src, size_t bytes, void *stream);
int k3k_zero(void *dst, size_t bytes, void *stream);       /* fill kernel, graph-safe */
int k3k_sync(void *stream);
void *k3k_stream_create(void);
int k3k_stream_destroy(void *stream);
int k3k_cu_count(void);
/* Graph capture of the work enqueued on `stream` (a created stream, not NULL). */
/* k3k_fork: *side = a second stream that first waits for the work queued on stream;
 * k3k_join: stream waits for the work queued on the side stream since. */
/* pinned host memory and events (host-side waits for part of a stream's work) */
void *k3k_host_alloc(size_t bytes);
void k3k_host_free(void *p);
void *k3k_event_create(void);
int k3k_event_record(void *ev, void *stream);
int k3k_event_sync(void *ev);
int k3k_side_init(void);
int k3k_fork(void *stream, void **side);
int k3k_join(void *stream);
int k3k_graph_begin(void *stream);
int k3k_graph_end(void *stream, void **exec);
int k3k_graph_launch(void *exec, void *stream);
int k3k_graph_destroy(void *exec);

/* Stage profiler: while enabled, k3k_prof_mark(stream, stage) records a HIP event on the
 * stream; k3k_prof_collect() waits for the device and sums, per stage, the time from the
 * previous mark on the same stream to that stage's mark. */
int k3k_prof_enable(int max_marks);
int k3k_prof_active(void);
int k3k_prof_mark(void *stream, int stage);
int k3k_prof_collect(double *ms, int *count, int n_stages);

/* ---- activations: fp32 -> bf16 split --------------------------------------------- */
/* hi = bf16_rne(x), lo = bf16_rne(x - hi) (lo may be NULL: one-term rounding). */
int k3k_split_bf16(uint16_t *hi, uint16_t *lo, const float *x, size_t n, void *stream);

/* ---- MXFP4 grouped matmul on MFMA -------------------------------------------------
 * A "job" is one weight matrix W [rows][K] in packed MXFP4 (group 32) applied to a list
 * of activation rows: out[row_of(tok)][r] = sum_k W[r][k] * act[row_of(tok)][k].
 * Jobs come either from the expert gather (mode GATEUP / DOWN) or from a single matrix
 * (mode PLAIN). Activations arrive pre-split as bf16 hi (+ lo when nsplit == 2). */
/* The libm expf exception table on the device: sorted (key, value) bit pairs and a bucket
 * index by key >> 12 over [kmin, kmax] (index[b] = first pair whose (key >> 12) - base >= b),
 * and a membership bitmap so that a miss costs one load. */
typedef struct {
    const uint32_t *pairs, *index;
    const uint32_t *bits;      /* membership bits of |key| - mmin: [2 signs][mwords] words */
    uint32_t kmin, kmax, base, mmin, mwords;
    int n;
} K3kExc;

enum { K3K_MX_PLAIN = 0, K3K_MX_GATEUP = 1, K3K_MX_DOWN = 2 };

typedef struct {
    /* PLAIN: one job. */
    const uint8_t *packed, *scales;     /* [rows][K/2], [rows][K/32] */
    const uint16_t *xhi, *xlo;          /* [ntok][K] */
    const float *xf32;                  /* or fp32 rows [ntok][K], ntok <= 2: split in-kernel */
    float *y;                           /* [ntok][ldy] */
    int ntok, ldy;
    /* GATEUP / DOWN: jobs from the gather. A pass is up to pass_tok tokens of one job:
     * 16 (any K % 32 == 0, row-major bank), 8 (K % 512 == 0, either bank layout), 32
     * (K % 512 == 0, bf16 activations) or 48 / 96 (the same on a tiled bank: the prefill
     * kernel). */
    const void *bank;                   /* device K3ExpertQ[n_experts] */
    int pass_tok;
    int layout;                         /* 0: row-major MXFP4, 1: tiled MXFP4 (k3k_mx_tile) */
    const int *job_expert, *job_off, *job_cnt;
    const int *pass_job, *pass_tp, *n_passes;
    const int *perm;                    /* sorted position -> assignment a = t*topk + j */
    int topk;
    float *out;                         /* DOWN: contrib [T*topk][rows]              */
    uint16_t *ahi, *alo;                /* GATEUP: activation split [T*topk][rows]   */
    int act;                            /* K3_ACT_* */
    float b1, b2;
    /* shape */
    int rows, K, nsplit;
    int n_xrows;                        /* rows of the activation arrays (xhi/xlo) */
    int max_passes;                     /* host-side bound on *n_passes (grid sizing) */
    /* k3k_mx_decode: the router's idx [n_assign] (assignment a = t*topk + j -> expert);
     * GATEUP reads tokens from xf32 and stores the dropped count in *drops; DOWN reads
     * the activation terms xhi/xlo [n_assign][K]. */
    const int *idx;
    int n_assign;
    int *drops;
    int n_experts;                      /* idx outside [0, n_experts): absent */
    const float *wt;                    /* k3k_mx_decode_combine: weights [n_assign] */
    /* k3k_mx_decode GATEUP with sel = 1 (a few tokens, k3k_router_small): the kernel selects
     * the tokens' experts itself from router_small's scored records pre [T][n_experts]
     * (router weights rw [n_experts][K], bias rbias or NULL, renorm, rscale, the exception
     * table exc) and writes idx_out / wt_out [T][topk] and nrecomp [T]; idx is unused. */
    int sel;
    const void *pre;
    const float *rw, *rbias;
    int renorm;
    float rscale;
    K3kExc exc;
    int *idx_out;
    float *wt_out;
    int *nrecomp;
    /* Decode with few assignments (k3k_mx_decode_split_ok): gu [n_assign][2][inter] fp32.
     * k3k_mx_decode GATEUP then gives gate and up workgroups of their own and writes the two
     * fp32 sums there (twice the workgroups: one assignment's 128 tiles leave half the CUs
     * idle otherwise); k3k_mx_decode_combine forms act(gate, up) and its bf16 terms from them
     * while staging (the same functions, the same result). NULL: the activation terms. */
    float *gu;
    /* Per-workgroup stamps of the batched expert kernels (k3k_stamps_take), [grid][3] u64:
     * start and end (s_memrealtime, 100 MHz) and the hardware id (XCC_ID << 32 | HW_ID), or
     * NULL. The launchers fill it in. */
    unsigned long long *stamps;
    /* mx_prefill_kernel: K3K_NXCD_Q work-item counters, zero at launch (k3k_gather zeroes the
     * K3K_QUEUE_INTS after its counts), one per XCD group of workgroups: each workgroup takes
     * its next (pass, row block) from its group's counter instead of a fixed share. NULL:
     * fixed shares. */
    int *queue;
} K3kMxArgs;

/* Per-workgroup stamps (a profiling aid): while enabled, each launch of mx_moe_kernel /
 * mx_prefill_kernel takes the next grid * 3 u64 of the device buffer, in launch order;
 * collect returns the launches' kinds (K3D_STAMP_*) and grids and disables. */
int k3k_stamps_enable(void *dbuf, size_t bytes);
unsigned long long *k3k_stamps_take(int kind, int grid);
int k3k_stamps_collect(int *kinds, int *grids, int max, int *n);

int k3k_mx_gemm(int mode, const K3kMxArgs *a, void *stream);

/* GATEUP / DOWN for at most 16 assignments without the gather: one workgroup per
 * (assignment, 16-row tile), K % 512 == 0 and K <= 8192, row-major or tiled bank. */
int k3k_mx_decode(int mode, const K3kMxArgs *a, void *stream);
/* DOWN and the weighted combine of the decode path in one launch: out [T][rows] =
 * 0 + sum_j wt[t][j] * (slot j's down projection), j ascending, over slots whose expert is
 * in range and present (k3k_combine's rule); activation terms xhi/xlo [n_assign][K]. */
int k3k_mx_decode_combine(const K3kMxArgs *a, void *stream);
/* where k3k_mx_decode_combine is used (faster than the two kernels, LDS fits) */
int k3k_mx_decode_combine_ok(int n_assign, int topk, int nsplit, int K, int rows);
/* where the decode gate/up splits gate and up over workgroups (gu, no in-kernel selection):
 * few enough assignments for one tile per workgroup, and a down + combine launch after it */
int k3k_mx_decode_split_ok(int n_assign, int topk, int nsplit, int K, int rows, int K_down,
                           int rows_down);

/* Whether PLAIN may take fp32 activations (xf32): one or two tokens whose bf16 terms fit in
 * 64 KB of LDS, K <= 16384, x 16-byte aligned, the packed matrix under 2 GiB. */
static inline int k3k_mx_small_ok(int ntok, int K, int nsplit, int rows, const void *x)
{
    const long nsteps = ((long)K / 32 + 3) / 4;
    return ntok >= 1 && ntok <= 2 && K % 32 == 0 && (long)nsplit * ntok * K * 2 <= 65536 &&
           nsteps <= 128 && ((uintptr_t)x % 16) == 0 && (unsigned long long)rows * (K / 2) < 0x80000000ull;
}

/* Row-major MXFP4 matrix [rows][K] (K % 512 == 0) -> the tiled layout of the expert kernel:
 * tpacked [ceil(rows/16)*16][K/2] bytes, tscales [ceil(rows/16)*16][K/32] bytes. */
int k3k_mx_tile(uint8_t *tpacked, uint8_t *tscales, const uint8_t *packed, const uint8_t *scales,
                int rows, int K, void *stream);

/* Generic fp32-exact MXFP4 GEMV on the vector units for any even K and group <= 64
 * (y[rows] = W x, one token). Used where the MFMA path's shape assumptions fail. */
int k3k_mx_gemv_valu(float *y, const float *x, const uint8_t *packed, const uint8_t *scales,
                     int in, int rows, int group, void *stream);
int k3k_mx_dequant(float *out, const uint8_t *packed, const uint8_t *scales, int rows,
                   int pcols, int group, void *stream);

/* ---- dense GEMV (vector units, fp32 accumulation) -------------------------------- */
/* y[t*ldy + o] = W[o][:] . x[t][:] for t < ntok, o < out. */
int k3k_gemv_f32(float *y, const float *x, const float *W, int in, int out, int ntok, int ldy,
                 void *stream);
int k3k_gemv_bf16(float *y, const float *x, const uint16_t *W, int in, int out, int ntok,
                  int ldy, void *stream);
int k3k_gemv_q8(float *y, const float *x, const void *W, int in, int out, int ntok, int ldy,
                void *stream);

/* ---- router ----------------------------------------------------------------------- */
/* Router in two launches. k3k_router_partial: per K chunk of `chunk` columns (a multiple
 * of 32, from k3k_router_chunk), the chunk's fp64 chain part[k][t][e] and a bound
 * rbound[k][t][e] on its intermediate magnitudes. k3k_router_final: the certified logit
 * (the reference's sequential fp64 chain recomputed where the bound cannot decide the
 * fp32 rounding and the logit matters), sigmoid with the host libm's expf, biased
 * first-strict-max top-k, renorm, scale -> idx/wt [T][topk]; nrecomp [T] (may be NULL)
 * receives the number of recomputed logits per token. */
int k3k_router_chunk(int T, int hidden, int n_experts);
/* 1 when k3k_router_partial scores and certifies the logits itself (a few tokens): its
 * part then holds one 16-byte record per logit, which a selecting decode gate/up reads. */
int k3k_router_small(int T, int hidden);
/* The expert-major gather's outputs (k3k_gather) and its pass sizes, for the router's final
 * kernel to run the one-workgroup gather itself in its last workgroup to finish, saving a
 * launch. ctr: one int of scratch, zeroed by k3k_router_partial (its ctr argument) before
 * the final kernel counts its workgroups in. */
typedef struct {
    int *offsets, *perm, *job_expert, *job_off, *job_cnt, *pass_job, *pass_tp, *pass_job2,
        *pass_tp2, *counts;
    const void *bank;
    int topk, pass_tok, pass_tok2;
    int *ctr;
} K3kGatherArgs;
/* 1 when k3k_router_final can run the gather (more than a few tokens, the one-workgroup
 * gather's sizes). */
int k3k_router_gathers(int T, int hidden, int n_experts, int topk);
/* ctr (may be NULL): set to zero, and idx [n_idx] to -1, for a following k3k_router_final
 * that gathers (its gathering workgroup waits for every idx it reads to be set). */
int k3k_router_partial(double *part, float *rbound, const float *x, int T, const float *W,
                       int hidden, int n_experts, int chunk, int *ctr, int *idx, int n_idx,
                       const K3kExc *exc, void *stream);
/* The same partials of many tokens on the int8 matrix cores (k3_route_i8.hip): the chunk
 * for T tokens, or 0 where those kernels do not apply (then k3k_router_partial with
 * k3k_router_chunk's chunk); the scratch they need; the partials (x and W 16-byte aligned,
 * chunk from k3k_router_i8_chunk). */
int k3k_router_i8_chunk(int T, int hidden, int n_experts);
size_t k3k_router_i8_bytes(int T, int hidden, int n_experts, int chunk);
int k3k_router_partial_i8(double *part, float *rbound, void *scratch, const float *x, int T,
                          const float *W, int hidden, int n_experts, int chunk, int *ctr, int *idx,
                          int n_idx, void *stream);
/* gather (may be NULL): also run the gather of idx, as k3k_gather would. */
int k3k_router_final(int *idx, float *wt, int *nrecomp, const double *part, const float *rbound,
                     int chunk, const float *x, const float *W, const float *bias, int T,
                     int hidden, int n_experts, int topk, int renorm, float routed_scale,
                     const K3kExc *exc, const K3kGatherArgs *gather, void *stream);

/* ---- gather / combine -------------------------------------------------------------- */
/* Work-item counters after the gather's four counts (counts[4 ..]): K3K_NXCD_Q per expert-
 * kernel launch, for up to four launches (gate/up and down of both pass lists). */
#define K3K_NXCD_Q 8
#define K3K_QUEUE_INTS (4 * K3K_NXCD_Q)
/* Stable expert-major gather of the T*topk assignments in idx. Outputs:
 *   offsets[n_experts+1]; perm[T*topk]: sorted position -> assignment t*topk+j, experts
 *   ascending and (t, j) ascending inside one expert; jobs = experts with at least one
 *   assignment and a present bank entry, ascending: job_expert/job_off/job_cnt; passes
 *   of up to pass_tok tokens of one job: pass_job/pass_tp; counts[0] = n_jobs,
 *   counts[1] = n_passes, counts[2] = assignments whose bank entry is NULL (dropped).
 *   pass_tok2 > 0: jobs of more than pass_tok assignments are split into passes of up to
 *   pass_tok2 tokens in pass_job2/pass_tp2 instead, counts[3] = their number (else 0).
 *   counts[4 .. 4 + K3K_QUEUE_INTS) are set to zero (the expert kernels' work-item
 *   counters), so counts holds 4 + K3K_QUEUE_INTS ints. */
int k3k_gather(int *offsets, int *perm, int *job_expert, int *job_off, int *job_cnt,
               int *pass_job, int *pass_tp, int *pass_job2, int *pass_tp2, int *counts,
               int *hist, const int *idx, int T, int topk, int n_experts, const void *bank,
               int pass_tok, int pass_tok2, void *stream);
/* Ints of scratch (hist) that lets k3k_gather spread a large batch over many workgroups;
 * 0: one workgroup (hist may be NULL). */
size_t k3k_gather_scratch(int T, int topk, int n_experts);
/* out[t][i] = 0 + sum_j wt[t][j] * contrib[t*topk+j][i], j ascending, skipping
 * assignments whose expert index is outside [0, n_experts) or whose bank entry has a
 * NULL pointer (bank == NULL: every in-range expert is present). */
int k3k_combine(float *out, const float *contrib, const float *wt, const int *idx,
                const void *bank, int n_experts, int T, int topk, int E, void *stream);

/* ---- elementwise -------------------------------------------------------------------- */
int k3k_act(float *y, const float *gu, int n, int rows, int act, float b1, float b2,
            void *stream);
/* act over gu [rows][2n] (gate | up) straight into its bf16 split: hi [rows][n], and lo when
 * not NULL (k3k_split_bf16's rounding of the fp32 value k3k_act would write). */
int k3k_act_split(uint16_t *hi, uint16_t *lo, const float *gu, int n, int rows, int act,
                  float b1, float b2, void *stream);

/* ---- dense bf16 GEMM on the matrix cores (k3_gemm.hip) ------------------------------ */
/* y[t][r] (= or, accumulate, +=) sum_k W[r][k] * (xhi + xlo)[t][k], t < T, r < R, row stride
 * ldy: W bf16 [R][K], activations as bf16 terms [T][K] (xlo NULL: one term), K % 64 == 0,
 * operands under 2 GiB. fp32 accumulation and output. part (16-byte aligned, part_bytes of
 * it; may be NULL) lets the GEMM split K into slices when its tiles cannot fill the chip:
 * slice sums go there and are added in slice order; k3k_dense_part_bytes(R, T, K, 0) bytes
 * allow every split it chooses. */
int k3k_dense_gemm(float *y, int ldy, int accumulate, const uint16_t *W, const uint16_t *xhi,
                   const uint16_t *xlo, int R, int T, int K, float *part, size_t part_bytes,
                   void *stream);
/* The dense SwiGLU's first half: act(W_gate x, W_up x) for rows r < R of both [R][K]
 * matrices, written as bf16 terms ahi (and alo when not NULL) [T][R]; part as above, sized
 * by k3k_dense_part_bytes(R, T, K, 1). */
int k3k_dense_gateup(uint16_t *ahi, uint16_t *alo, const uint16_t *wg, const uint16_t *wu,
                     const uint16_t *xhi, const uint16_t *xlo, int R, int T, int K, int act,
                     float b1, float b2, float *part, size_t part_bytes, void *stream);
size_t k3k_dense_part_bytes(int R, int T, int K, int gateup);
int k3k_rmsnorm(float *y, const float *x, const float *w, int n, int rows, float eps,
                void *stream);
int k3k_axpy_rows(float *out, const float *add, size_t n, void *stream); /* out += add */
int k3k_scale(float *out, const float *in, float s, size_t n, void *stream);

/* ---- the allocation-free workspace (k3_static.hip) --------------------------------- */
/* Looks up, once per device, the device address of the library's static workspace for the
 * current device (called by k3d_init). */
int k3s_static_setup(void);
/* Error text for a k3d_* entry point implemented outside k3_devapi.c; returns -2. */
int k3dx_bad(const char *msg);

#ifdef __cplusplus
}
#endif
#endif
