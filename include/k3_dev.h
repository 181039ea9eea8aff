/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_dev.h -- device-pointer entry points of libk3amd.so.
 *
 * The reference has no device: its kernels take host buffers (include/k3/k3.h). These
 * entry points are the same operations for callers whose activations and weights are
 * already resident in HBM (a serving loop, the benchmark): every pointer is a DEVICE
 * pointer, work is enqueued on the caller's HIP stream (NULL = the null stream) and the
 * call returns without synchronising. None of them allocates: scratch comes from a
 * caller-provided workspace of the size the matching *_ws() function reports. They
 * return 0, or a negative value with a message available from k3d_error() (kept per host
 * thread).
 *
 * Work that runs beside the caller's (the activation split beside the router, the hot
 * experts' passes of a skewed prefill batch) goes to a side stream that belongs to the
 * caller's stream, forked from it and joined back into it by events of its own; so calls
 * from several host threads on different streams, at once, never share a stream or an
 * event, and each gives the result it gives alone. A stream's side stream is made by
 * k3d_stream_create (the null stream's by k3d_init), or by the first call on a stream made
 * elsewhere; at most 256 caller streams at once. Calls that overlap on one stream, or
 * share a workspace, race.
 *
 * Each names the reference function whose arithmetic it performs.
 */
#ifndef K3_DEV_H
#define K3_DEV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Selects the device and uploads the router's tables once; after it, no entry point below
 * allocates or synchronises (except k3d_malloc/free/sync and the copies). */
int k3d_init(void);
const char *k3d_error(void);
void *k3d_malloc(size_t bytes);
int k3d_free(void *p);
int k3d_h2d(void *dst, const void *src, size_t bytes, void *stream);
int k3d_d2h(void *dst, const void *src, size_t bytes, void *stream);
int k3d_sync(void *stream);

/* Streams (default priority) and HIP graphs: k3d_graph_begin/end capture everything the
 * k3d_* calls enqueue on a created stream between them (no allocation or synchronisation
 * happens inside those calls); k3d_graph_launch replays it with one launch. The captured
 * pointers are baked in: replay with the same buffers, new contents. */
void *k3d_stream_create(void);
int k3d_stream_destroy(void *stream);
int k3d_graph_begin(void *stream);
int k3d_graph_end(void *stream, void **exec);
int k3d_graph_launch(void *exec, void *stream);
int k3d_graph_destroy(void *exec);

/* Stage profiler (HIP events). Between k3d_prof_begin and k3d_prof_end, the MoE and GEMV
 * entry points record an event at each stage boundary; k3d_prof_end synchronises and
 * returns, per stage, the summed milliseconds and the number of samples. Stage ids: */
enum { K3D_STAGE_BEGIN = 0, K3D_STAGE_ROUTER = 1, K3D_STAGE_GATHER = 2, K3D_STAGE_GATEUP = 3,
       K3D_STAGE_DOWN = 4, K3D_STAGE_COMBINE = 5, K3D_STAGE_GEMV = 6, K3D_STAGE_SHARED = 7,
       K3D_STAGE_COUNT = 8 };
/* Per-workgroup stamps of the batched expert kernels (mx_moe_kernel, mx_prefill_kernel), a
 * profiling aid beside the stage profiler: between k3d_stamps_begin and k3d_stamps_end, each
 * launch of those kernels writes, for each of its workgroups, three u64 into the device
 * buffer dbuf, launch after launch: the workgroup's start and end on the 100 MHz clock and
 * the hardware id it ran on (XCC id << 32 | the HW_ID register: CU in bits 8-11, shader
 * array 12, shader engine 13-15). Launches that no longer fit are not stamped. k3d_stamps_end
 * gives the kinds (K3D_STAMP_*) and grids of the stamped launches in order (up to max; *n =
 * their number) and stops stamping. Not for graph capture: the buffer region is chosen when a
 * call enqueues its work. */
enum { K3D_STAMP_MOE_GATEUP = 1, K3D_STAMP_MOE_DOWN = 2, K3D_STAMP_PREFILL_GATEUP = 3,
       K3D_STAMP_PREFILL_DOWN = 4 };
int k3d_stamps_begin(void *dbuf, size_t bytes);
int k3d_stamps_end(int *kinds, int *grids, int max, int *n);
int k3d_prof_begin(int max_marks);
int k3d_prof_mark(void *stream, int stage);
int k3d_prof_end(double *ms, int *count, int n_stages);

/* Y[ntok][rows] = X[ntok][in] . W^T, W packed MXFP4 with group 32, in % 32 == 0.
 * prec 0: fp32-accurate (activations split into two bf16 terms), prec 1: activations
 * rounded to bf16. Arithmetic of k3_matmul_mxfp4 (reference k3_ops.c:1380-1785). */
size_t k3d_matmul_mxfp4_ws(int ntok, int in);
int k3d_matmul_mxfp4(float *y, const float *x, int ntok, const uint8_t *packed,
                     const uint8_t *scales, int in, int rows, int prec, void *ws,
                     size_t ws_bytes, void *stream);

/* Y[ntok][out] = X[ntok][in] . W^T for fp32 / bf16 weights (reference k3_ops.c:265-291,
 * 1108-1213). */
int k3d_matmul_f32(float *y, const float *x, int ntok, const float *W, int in, int out,
                   void *stream);
int k3d_matmul_bf16(float *y, const float *x, int ntok, const uint16_t *W, int in, int out,
                    void *stream);

/* Router over T tokens: idx/wt [T][topk] (reference k3_ops.c:419-478, per token).
 * n_experts 1..2048 (the selection holds every expert's record in one workgroup's LDS);
 * more returns an error. */
size_t k3d_router_ws(int T, int hidden, int n_experts);
int k3d_router(int *idx, float *wt, const float *x, int T, const float *W, const float *bias,
               int hidden, int n_experts, int topk, int renorm, float routed_scale, void *ws,
               size_t ws_bytes, void *stream);

/* Device layouts of an expert bank's MXFP4 matrices.
 *   K3D_LAYOUT_ROWS:  the reference's, packed [rows][in/2] + scales [rows][in/32] bytes.
 *   K3D_LAYOUT_TILED: the same bytes regrouped per tile of 16 rows x 512 columns in the
 *     order the expert kernel reads them (k3d_mxfp4_tile), the four tiles of each group of
 *     64 rows side by side chunk after chunk; rows are padded to a multiple of 64, in must
 *     be a multiple of 512. A block with scale byte 255 (NaN; zero in the reference) is
 *     stored as zero codes with scale byte 127. Same arithmetic, results bit-identical to
 *     ROWS; the expert kernel streams it at a higher fraction of HBM bandwidth. */
enum { K3D_LAYOUT_ROWS = 0, K3D_LAYOUT_TILED = 1 };
int k3d_mxfp4_tiled_size(int rows, int in, size_t *packed_bytes, size_t *scales_bytes);
int k3d_mxfp4_tile(uint8_t *tpacked, uint8_t *tscales, const uint8_t *packed,
                   const uint8_t *scales, int rows, int in, void *stream);

/* Diagnostics of the last k3d_router call that used workspace `ws` (after the device has
 * finished it; synchronises): h_counts[t] = number of token t's logits whose fp32 rounding
 * the split fp64 sum could not certify and that were recomputed with the reference's
 * sequential chain. */
int k3d_router_recomputed(int *h_counts, const void *ws, int T, int hidden, int n_experts);
/* The chunk partials of the same call (more than four tokens; synchronises): *h_chunk = the
 * chunk width, h_part / h_rbound [ks][T][n_experts] (ks = ceil(hidden / chunk), at most
 * `cap` entries each) the chunk sums P_k and the bounds R_k, |P_k - exact| <= 2^-53 R_k and
 * R_k >= the sum of |the chunk's exact prefix sums|, that the certification uses. Returns
 * ks, or -1. */
int k3d_router_partials(double *h_part, float *h_rbound, int *h_chunk, size_t cap, const void *ws, int T,
                        int hidden, int n_experts);

/* The routed MoE layer (k3_moe's routed loop, reference k3_ops.c:576-643, with z := x),
 * expert-major. bank is a DEVICE array of n_experts K3ExpertQ (k3.h) whose pointers are
 * device pointers, in the given layout; an entry with a NULL pointer is a dropped expert.
 * hidden and inter: multiples of 32 (ROWS) or of 512 (TILED). perm_out (T*topk) and
 * offsets_out (n_experts+1), when not NULL, receive the gather permutation. *drops_out,
 * when not NULL, receives (after the stream reaches it) the number of dropped
 * assignments; it must be a device int. */
size_t k3d_moe_ws(int T, int hidden, int inter, int n_experts, int topk, int prec);
int k3d_moe_routed(float *out, int *idx, float *wt, const float *x, int T,
                   const float *router_w, const float *bias, const void *bank, int layout,
                   int hidden, int inter, int n_experts, int topk, int renorm, float routed_scale,
                   int act, float b1, float b2, int prec, void *ws, size_t ws_bytes,
                   int *perm_out, int *offsets_out, int *drops_out, void *stream);

/* k3d_moe_routed with no workspace argument and no allocation, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. The scratch lives in a static device array
 * of K3D_STATIC_WS_BYTES (40 MiB) that each GPU holds until the process ends: enough for
 * decode batches of up to 64 tokens at hidden 7168 / inter 2048 / 384 experts / top-8 or
 * at 3584 / 3072 / 896 / top-16 (k3d_moe_ws of the call must not exceed it; larger calls
 * return an error). k3d_init must have run on the device first (it looks the array up and
 * makes the one-time uploads). All calls on one GPU share the array: calls that overlap
 * on one GPU race. Otherwise identical to k3d_moe_routed, results bit for bit. */
#define K3D_STATIC_WS_BYTES ((size_t)40 << 20)
size_t k3d_static_ws_bytes(void);
int k3d_moe_routed_static(float *out, int *idx, float *wt, const float *x, int T,
                          const float *router_w, const float *bias, const void *bank, int layout,
                          int hidden, int inter, int n_experts, int topk, int renorm,
                          float routed_scale, int act, float b1, float b2, int prec, int *perm_out,
                          int *offsets_out, int *drops_out, void *stream);

/* The always-on dense shared expert with bf16 weights, on the matrix cores:
 *   s[t] = W2 . act(W1 x[t], W3 x[t]),  W1, W3 [inter][hidden], W2 [hidden][inter] bf16,
 * y = s (accumulate 0) or y += s (accumulate 1, after the routed sum: the order of the
 * reference's shared tail, k3_ops.c:650-654). The reference computes each product with
 * k3_matmul_bf16 (fp64 accumulation); here fp32 MFMA accumulation in the library's own
 * bf16 GEMM kernels (gate and up in one pass with the activation in the epilogue, then
 * down) with the activations as two bf16 terms (prec 0, max|err| <= 1e-4 ||ref||inf) or
 * one (prec 1, 2e-2 relative). hidden and inter must be multiples of 64. Nothing is
 * allocated and no library is initialised, so the call can be captured in a HIP graph. */
size_t k3d_shared_ws(int T, int hidden, int inter, int prec);
int k3d_shared_expert(float *y, int accumulate, const float *x, int T, const uint16_t *w1,
                      const uint16_t *w3, const uint16_t *w2, int hidden, int inter, int act,
                      float b1, float b2, int prec, void *ws, size_t ws_bytes, void *stream);

/* The expert half of the layer for a routing already in idx/wt (device). Slots whose
 * expert index lies outside [0, n_experts), or whose bank entry has a NULL pointer,
 * contribute nothing; drops_out counts the latter. */
int k3d_moe_experts(float *out, const int *idx, const float *wt, const float *x, int T,
                    const void *bank, int layout, int hidden, int inter, int n_experts, int topk,
                    int act, float b1, float b2, int prec, void *ws, size_t ws_bytes,
                    int *perm_out, int *offsets_out, int *drops_out, void *stream);

#ifdef __cplusplus
}
#endif
#endif
