/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_static.hip -- the routed MoE layer for callers that cannot allocate.
 *
 * k3d_moe_routed takes its scratch (activation splits, gather arrays, router partials,
 * per-assignment contributions) from a caller workspace. Some callers have none to give
 * and may not call hipMalloc: code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation. k3d_moe_routed_static is the same layer with that
 * scratch in `scratch`, a file-scope __device__ array of K3D_STATIC_WS_BYTES that every
 * GPU the library runs on holds until the process ends.
 *
 * In host code `scratch` names a host-side stand-in, not device memory, so its device
 * address is looked up once per device with hipGetSymbolAddress (k3s_static_setup, called
 * by k3d_init with that device current) and only that address is ever handed to kernels.
 * The array keeps whatever the last call left in it; the layer writes every part of its
 * scratch before reading it, so nothing needs clearing. All calls on one GPU share the
 * array: calls that overlap on one GPU (several streams or host threads at once) race.
 */
#include "k3_common.h"
#include "k3_dev.h"
#include "k3k.h"

#include <pthread.h>
#include <stdio.h>

static __device__ __align__(256) unsigned char scratch[K3D_STATIC_WS_BYTES];

#define K3S_MAX_DEVICES 64
static void *g_scratch_dev[K3S_MAX_DEVICES];   /* device address of `scratch`, per device */
static pthread_mutex_t g_scratch_mu = PTHREAD_MUTEX_INITIALIZER;

extern "C" int k3k_fail(const char *what, hipError_t e);

extern "C" int k3s_static_setup(void)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return k3k_fail("static workspace: hipGetDevice", e);
    if (dev < 0 || dev >= K3S_MAX_DEVICES) return k3k_fail("static workspace: device id", hipErrorInvalidDevice);
    pthread_mutex_lock(&g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e == hipSuccess && p) g_scratch_dev[dev] = p;
    }
    void *got = g_scratch_dev[dev];
    pthread_mutex_unlock(&g_scratch_mu);
    if (!got) return k3k_fail("static workspace: hipGetSymbolAddress", e != hipSuccess ? e : hipErrorInvalidSymbol);
    return 0;
}

extern "C" size_t k3d_static_ws_bytes(void) { return K3D_STATIC_WS_BYTES; }

extern "C" int k3d_moe_routed_static(float *out, int *idx, float *wt, const float *x, int T,
                                     const float *router_w, const float *bias, const void *bank,
                                     int layout, int hidden, int inter, int n_experts, int topk,
                                     int renorm, float routed_scale, int act, float b1, float b2,
                                     int prec, int *perm_out, int *offsets_out, int *drops_out,
                                     void *stream)
{
    if (T <= 0) return 0;
    const size_t need = k3d_moe_ws(T, hidden, inter, n_experts, topk, prec);
    if (need > K3D_STATIC_WS_BYTES) {
        char msg[200];
        snprintf(msg, sizeof msg,
                 "k3d_moe_routed_static: this layer needs %zu bytes of scratch, the static "
                 "workspace holds %zu (use k3d_moe_routed with a workspace)",
                 need, (size_t)K3D_STATIC_WS_BYTES);
        return k3dx_bad(msg);
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= K3S_MAX_DEVICES)
        return k3dx_bad("k3d_moe_routed_static: no current device");
    pthread_mutex_lock(&g_scratch_mu);
    void *ws = g_scratch_dev[dev];
    pthread_mutex_unlock(&g_scratch_mu);
    if (!ws) return k3dx_bad("k3d_moe_routed_static: k3d_init has not run on this device");
    return k3d_moe_routed(out, idx, wt, x, T, router_w, bias, bank, layout, hidden, inter,
                          n_experts, topk, renorm, routed_scale, act, b1, b2, prec, ws,
                          K3D_STATIC_WS_BYTES, perm_out, offsets_out, drops_out, stream);
}
