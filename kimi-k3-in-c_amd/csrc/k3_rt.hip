/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_rt.hip -- HIP runtime wrappers behind the k3k C ABI: device selection, memory,
 * copies, the graph-safe zero fill, streams and the last-error string.
 */
#include "k3_common.h"
#include "k3k.h"

#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* the last error, per thread */
static thread_local char g_err[512];
static int g_ready = 0;
static int g_cus = 0;

extern "C" int k3k_fail(const char *what, hipError_t e)
{
    snprintf(g_err, sizeof g_err, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
    return -1;
}

extern "C" const char *k3k_error(void) { return g_err; }

extern "C" int k3k_device_count(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

extern "C" int k3k_init(void)
{
    if (g_ready) return 0;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        snprintf(g_err, sizeof g_err, "no HIP device available (%s)",
                 e == hipSuccess ? "device count 0" : hipGetErrorString(e));
        return -1;
    }
    int dev = 0;
    e = hipGetDevice(&dev);
    if (e != hipSuccess) return k3k_fail("hipGetDevice", e);
    e = hipDeviceGetAttribute(&g_cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return k3k_fail("hipDeviceGetAttribute", e);
    g_ready = 1;
    return 0;
}

extern "C" int k3k_cu_count(void)
{
    if (!g_ready && k3k_init() != 0) return 256;
    return g_cus > 0 ? g_cus : 256;
}

extern "C" void *k3k_malloc(size_t bytes)
{
    void *p = nullptr;
    if (bytes == 0) bytes = 256;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        k3k_fail("hipMalloc", e);
        return nullptr;
    }
    return p;
}

extern "C" int k3k_free(void *p)
{
    if (!p) return 0;
    hipError_t e = hipFree(p);
    return e == hipSuccess ? 0 : k3k_fail("hipFree", e);
}

extern "C" int k3k_h2d(void *dst, const void *src, size_t bytes, void *stream)
{
    if (!bytes) return 0;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream);
    return e == hipSuccess ? 0 : k3k_fail("hipMemcpyAsync H2D", e);
}

extern "C" int k3k_d2h(void *dst, const void *src, size_t bytes, void *stream)
{
    if (!bytes) return 0;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream);
    return e == hipSuccess ? 0 : k3k_fail("hipMemcpyAsync D2H", e);
}

extern "C" int k3k_d2d(void *dst, const void *src, size_t bytes, void *stream)
{
    if (!bytes) return 0;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream);
    return e == hipSuccess ? 0 : k3k_fail("hipMemcpyAsync D2D", e);
}

namespace {
__global__ void zero_kernel(uint32_t *p, size_t nwords, uint8_t *tail, size_t ntail)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < nwords;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
    if (blockIdx.x == 0 && threadIdx.x < ntail) tail[threadIdx.x] = 0;
}
}  // namespace

/* A fill kernel rather than hipMemsetAsync, so that a caller may capture it in a graph. */
extern "C" int k3k_zero(void *dst, size_t bytes, void *stream)
{
    if (!bytes) return 0;
    const size_t nw = bytes / 4, nt = bytes % 4;
    size_t blocks = (nw + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(zero_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (uint32_t *)dst, nw, (uint8_t *)dst + nw * 4, nt);
    K3K_LAUNCH_CHECK("zero launch");
    return 0;
}

/* Pinned host memory (copies from and to it run asynchronously) and events. */
extern "C" void *k3k_host_alloc(size_t bytes)
{
    void *p = nullptr;
    hipError_t e = hipHostMalloc(&p, bytes ? bytes : 64, hipHostMallocDefault);
    if (e != hipSuccess) {
        k3k_fail("hipHostMalloc", e);
        return nullptr;
    }
    return p;
}

extern "C" void k3k_host_free(void *p)
{
    if (p) (void)hipHostFree(p);
}

extern "C" void *k3k_event_create(void)
{
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) {
        k3k_fail("hipEventCreate", e);
        return nullptr;
    }
    return (void *)ev;
}

extern "C" int k3k_event_record(void *ev, void *stream)
{
    hipError_t e = hipEventRecord((hipEvent_t)ev, (hipStream_t)stream);
    return e == hipSuccess ? 0 : k3k_fail("hipEventRecord", e);
}

extern "C" int k3k_event_sync(void *ev)
{
    hipError_t e = hipEventSynchronize((hipEvent_t)ev);
    return e == hipSuccess ? 0 : k3k_fail("hipEventSynchronize", e);
}

extern "C" int k3k_sync(void *stream)
{
    hipError_t e = stream ? hipStreamSynchronize((hipStream_t)stream) : hipDeviceSynchronize();
    return e == hipSuccess ? 0 : k3k_fail("synchronize", e);
}

/* ---- side streams --------------------------------------------------------------------
 * Work that may run beside the caller's (the activation split beside the router, the hot
 * experts' pass list) goes to a side stream of the caller's stream: one per caller stream,
 * created with the default priority, non-blocking, with its own fork and join events.
 * Work is forked after what is already queued on the caller's stream and joined back into
 * it; both are event waits, so a stream being captured into a graph captures the side work
 * too, and calls that overlap on different caller streams never share a stream or an
 * event. Entries are made by k3k_side_init (the null stream, at initialisation), by
 * k3k_stream_create, or on a caller stream's first fork; k3k_stream_destroy removes its
 * stream's entry. */
#define K3_SIDE_MAX 256
struct K3Side {
    hipStream_t caller, side;
    hipEvent_t fork, join;
};
static K3Side g_side[K3_SIDE_MAX];
static int g_nside = 0;
static pthread_mutex_t g_side_mu = PTHREAD_MUTEX_INITIALIZER;

/* The entry of caller stream s (made if absent), or NULL with the error set. */
static K3Side *side_of(hipStream_t s)
{
    pthread_mutex_lock(&g_side_mu);
    K3Side *r = nullptr;
    for (int i = 0; i < g_nside; i++)
        if (g_side[i].caller == s) {
            r = &g_side[i];
            break;
        }
    if (!r) {
        if (g_nside == K3_SIDE_MAX) {
            k3k_fail("side stream: more than 256 caller streams", hipErrorInvalidValue);
        } else {
            K3Side n = {s, nullptr, nullptr, nullptr};
            hipError_t e = hipStreamCreateWithFlags(&n.side, hipStreamNonBlocking);
            if (e == hipSuccess) e = hipEventCreateWithFlags(&n.fork, hipEventDisableTiming);
            if (e == hipSuccess) e = hipEventCreateWithFlags(&n.join, hipEventDisableTiming);
            if (e == hipSuccess) {
                g_side[g_nside] = n;
                r = &g_side[g_nside++];
            } else {
                k3k_fail("side stream: create", e);
                if (n.join) (void)hipEventDestroy(n.join);
                if (n.fork) (void)hipEventDestroy(n.fork);
                if (n.side) (void)hipStreamDestroy(n.side);
            }
        }
    }
    pthread_mutex_unlock(&g_side_mu);
    return r;
}

extern "C" int k3k_side_init(void)
{
    if (k3k_init()) return -1;
    return side_of(nullptr) ? 0 : -1;
}

extern "C" int k3k_fork(void *stream, void **side)
{
    K3Side *sd = side_of((hipStream_t)stream);
    if (!sd) return -1;
    hipError_t e = hipEventRecord(sd->fork, (hipStream_t)stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(sd->side, sd->fork, 0);
    if (e != hipSuccess) return k3k_fail("fork", e);
    *side = sd->side;
    return 0;
}

extern "C" int k3k_join(void *stream)
{
    K3Side *sd = side_of((hipStream_t)stream);
    if (!sd) return -1;
    hipError_t e = hipEventRecord(sd->join, sd->side);
    if (e == hipSuccess) e = hipStreamWaitEvent((hipStream_t)stream, sd->join, 0);
    return e == hipSuccess ? 0 : k3k_fail("join", e);
}

extern "C" void *k3k_stream_create(void)
{
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) {
        k3k_fail("hipStreamCreate", e);
        return nullptr;
    }
    if (!side_of(s)) {
        (void)hipStreamDestroy(s);
        return nullptr;
    }
    return (void *)s;
}

extern "C" int k3k_stream_destroy(void *stream)
{
    if (!stream) return 0;
    pthread_mutex_lock(&g_side_mu);
    for (int i = 0; i < g_nside; i++)
        if (g_side[i].caller == (hipStream_t)stream) {
            (void)hipStreamSynchronize(g_side[i].side);
            (void)hipEventDestroy(g_side[i].fork);
            (void)hipEventDestroy(g_side[i].join);
            (void)hipStreamDestroy(g_side[i].side);
            g_side[i] = g_side[--g_nside];
            break;
        }
    pthread_mutex_unlock(&g_side_mu);
    hipError_t e = hipStreamDestroy((hipStream_t)stream);
    return e == hipSuccess ? 0 : k3k_fail("hipStreamDestroy", e);
}

/* ---- HIP graphs: capture the work enqueued on a stream once, replay it with one launch */
extern "C" int k3k_graph_begin(void *stream)
{
    if (!stream) return k3k_fail("graph capture needs a created stream", hipErrorInvalidValue);
    hipError_t e = hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal);
    return e == hipSuccess ? 0 : k3k_fail("hipStreamBeginCapture", e);
}

extern "C" int k3k_graph_end(void *stream, void **exec)
{
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture((hipStream_t)stream, &g);
    if (e != hipSuccess) return k3k_fail("hipStreamEndCapture", e);
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return k3k_fail("hipGraphInstantiate", e);
    *exec = (void *)x;
    return 0;
}

extern "C" int k3k_graph_launch(void *exec, void *stream)
{
    hipError_t e = hipGraphLaunch((hipGraphExec_t)exec, (hipStream_t)stream);
    return e == hipSuccess ? 0 : k3k_fail("hipGraphLaunch", e);
}

extern "C" int k3k_graph_destroy(void *exec)
{
    if (!exec) return 0;
    hipError_t e = hipGraphExecDestroy((hipGraphExec_t)exec);
    return e == hipSuccess ? 0 : k3k_fail("hipGraphExecDestroy", e);
}

/* ---- stage profiler ------------------------------------------------------------------ */
namespace {
hipEvent_t *g_ev = nullptr;
int *g_ev_stage = nullptr;
hipStream_t *g_ev_stream = nullptr;
int g_ev_cap = 0, g_ev_n = 0, g_prof_on = 0;
}  // namespace

extern "C" int k3k_prof_enable(int max_marks)
{
    if (max_marks <= 0) {
        g_prof_on = 0;
        return 0;
    }
    if (max_marks > g_ev_cap) {
        for (int i = 0; i < g_ev_cap; i++) (void)hipEventDestroy(g_ev[i]);
        free(g_ev);
        free(g_ev_stage);
        free(g_ev_stream);
        g_ev = (hipEvent_t *)calloc((size_t)max_marks, sizeof(hipEvent_t));
        g_ev_stage = (int *)calloc((size_t)max_marks, sizeof(int));
        g_ev_stream = (hipStream_t *)calloc((size_t)max_marks, sizeof(hipStream_t));
        if (!g_ev || !g_ev_stage || !g_ev_stream) {
            g_ev_cap = 0;
            snprintf(g_err, sizeof g_err, "profiler: out of host memory");
            return -1;
        }
        for (int i = 0; i < max_marks; i++) {
            hipError_t e = hipEventCreate(&g_ev[i]);
            if (e != hipSuccess) {
                g_ev_cap = i;
                return k3k_fail("hipEventCreate", e);
            }
        }
        g_ev_cap = max_marks;
    }
    g_ev_n = 0;
    g_prof_on = 1;
    return 0;
}

extern "C" int k3k_prof_active(void) { return g_prof_on; }

extern "C" int k3k_prof_mark(void *stream, int stage)
{
    if (!g_prof_on || g_ev_n >= g_ev_cap) return 0;
    hipError_t e = hipEventRecord(g_ev[g_ev_n], (hipStream_t)stream);
    if (e != hipSuccess) return k3k_fail("hipEventRecord", e);
    g_ev_stage[g_ev_n] = stage;
    g_ev_stream[g_ev_n] = (hipStream_t)stream;
    g_ev_n++;
    return 0;
}

extern "C" int k3k_prof_collect(double *ms, int *count, int n_stages)
{
    for (int s = 0; s < n_stages; s++) { ms[s] = 0.0; count[s] = 0; }
    for (int i = 0; i < g_ev_n; i++) {
        hipError_t e = hipEventSynchronize(g_ev[i]);
        if (e != hipSuccess) return k3k_fail("hipEventSynchronize", e);
    }
    for (int i = 1; i < g_ev_n; i++) {
        int prev = -1;
        for (int j = i - 1; j >= 0; j--)
            if (g_ev_stream[j] == g_ev_stream[i]) { prev = j; break; }
        const int st = g_ev_stage[i];
        if (prev < 0 || st <= 0 || st >= n_stages) continue;   /* stage 0 opens a sequence */
        float t = 0.0f;
        hipError_t e = hipEventElapsedTime(&t, g_ev[prev], g_ev[i]);
        if (e != hipSuccess) return k3k_fail("hipEventElapsedTime", e);
        ms[st] += t;
        count[st]++;
    }
    g_prof_on = 0;
    g_ev_n = 0;
    return 0;
}

/* ---- per-workgroup stamps of the expert kernels (profiling) -------------------------- */
namespace {
unsigned long long *g_st_buf = nullptr;
size_t g_st_cap = 0, g_st_used = 0;          /* in u64 */
constexpr int K3_ST_MAXL = 4096;
int g_st_kind[K3_ST_MAXL], g_st_grid[K3_ST_MAXL], g_st_n = 0;
}  // namespace

extern "C" int k3k_stamps_enable(void *dbuf, size_t bytes)
{
    g_st_buf = (unsigned long long *)dbuf;
    g_st_cap = dbuf ? bytes / 8 : 0;
    g_st_used = 0;
    g_st_n = 0;
    return 0;
}

extern "C" unsigned long long *k3k_stamps_take(int kind, int grid)
{
    if (!g_st_buf || grid <= 0 || g_st_n >= K3_ST_MAXL || g_st_used + 3 * (size_t)grid > g_st_cap)
        return nullptr;
    unsigned long long *p = g_st_buf + g_st_used;
    g_st_used += 3 * (size_t)grid;
    g_st_kind[g_st_n] = kind;
    g_st_grid[g_st_n] = grid;
    g_st_n++;
    return p;
}

extern "C" int k3k_stamps_collect(int *kinds, int *grids, int max, int *n)
{
    const int m = g_st_n < max ? g_st_n : max;
    for (int i = 0; i < m; i++) {
        if (kinds) kinds[i] = g_st_kind[i];
        if (grids) grids[i] = g_st_grid[i];
    }
    if (n) *n = g_st_n;
    k3k_stamps_enable(nullptr, 0);
    return 0;
}
