/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_dense.hip -- dense GEMV on the vector units: fp32, bf16 and per-row int8 weights.
 *
 * Replaces k3_matmul (src/core/k3_ops.c:265-291), k3_matmul_bf16 (:1108-1213) and
 * k3_matmul_q8 (:1221-1289) of the reference for the decode shapes.
 *
 * gemv_rows_kernel (row length a multiple of 8, 16-byte aligned operands): a wave owns RW
 * rows and up to NT tokens; lane l takes the 8-element chunks l, l+64, l+128, ... of every
 * row, and issues the loads of U chunks of all RW rows (and the matching x chunks) before
 * any arithmetic, so a lane keeps U*RW 16-byte weight loads in flight and each x chunk it
 * loads serves RW rows. Per lane the products are accumulated in fp32 in ascending column
 * order, then the wave reduces with a butterfly. The fp32 and bf16 kernels are one
 * template, so on weights that are the same values they perform the same operations in
 * the same order and agree bit for bit (the reference holds the same property between its
 * two kernels, tests/unit/test_ops.c:798-848). Accumulation is fp32 where the reference
 * uses fp64; the difference is far inside max|err| <= 1e-4 ||ref||inf. gemv_kernel, one
 * wave per row, takes the remaining shapes.
 */
#include "k3_common.h"
#include "k3k.h"

namespace {

__device__ __forceinline__ float wval(float w) { return w; }
__device__ __forceinline__ float wval(uint16_t h) { return k3_bf16_to_f32(h); }

template <typename WT>
__device__ __forceinline__ void load8(const WT *p, float *w);
template <>
__device__ __forceinline__ void load8<float>(const float *p, float *w)
{
    const float4 a = reinterpret_cast<const float4 *>(p)[0];
    const float4 b = reinterpret_cast<const float4 *>(p)[1];
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}
template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t *p, float *w)
{
    const uint4 v = *reinterpret_cast<const uint4 *>(p);
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
    for (int k = 0; k < 4; k++) {
        w[2 * k] = __uint_as_float(u[k] << 16);
        w[2 * k + 1] = __uint_as_float(u[k] & 0xFFFF0000u);
    }
}

template <typename WT>
__global__ __launch_bounds__(256) void gemv_kernel(float *y, const float *x, const WT *W, int in,
                                                   int out, int vec, int ldy)
{
    const int lane = threadIdx.x & 63;
    const int o = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int t = blockIdx.y;
    if (o >= out) return;
    const WT *row = W + (size_t)o * in;
    const float *xt = x + (size_t)t * in;
    float acc = 0.0f;
    if (vec) {
        for (int c = lane; c < in / 8; c += 64) {
            float w[8];
            load8<WT>(row + 8 * c, w);
            const float4 xa = reinterpret_cast<const float4 *>(xt + 8 * c)[0];
            const float4 xb = reinterpret_cast<const float4 *>(xt + 8 * c)[1];
            acc = fmaf(w[0], xa.x, acc); acc = fmaf(w[1], xa.y, acc);
            acc = fmaf(w[2], xa.z, acc); acc = fmaf(w[3], xa.w, acc);
            acc = fmaf(w[4], xb.x, acc); acc = fmaf(w[5], xb.y, acc);
            acc = fmaf(w[6], xb.z, acc); acc = fmaf(w[7], xb.w, acc);
        }
    } else {
        for (int c = lane; c < (in + 7) / 8; c += 64)
            for (int k = 0; k < 8; k++) {
                const int i = 8 * c + k;
                if (i < in) acc = fmaf(wval(row[i]), xt[i], acc);
            }
    }
    for (int s = 32; s > 0; s >>= 1) acc += __shfl_xor(acc, s, 64);
    if (lane == 0) y[(size_t)t * ldy + o] = acc;
}

/* Draft-model int8 rows [f32 scale][int8 x in] (reference k3_ops.c:1221-1289): fp32
 * accumulation, scale applied once at the end. No exactness contract, as there. */
__global__ __launch_bounds__(256) void gemv_q8_kernel(float *y, const float *x, const uint8_t *W,
                                                      int in, int out, int ldy)
{
    const int lane = threadIdx.x & 63;
    const int o = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int t = blockIdx.y;
    if (o >= out) return;
    const uint8_t *row = W + (size_t)o * (4 + (size_t)in);
    const float *xt = x + (size_t)t * in;
    float acc = 0.0f;
    for (int i = lane; i < in; i += 64) acc = fmaf((float)(int8_t)row[4 + i], xt[i], acc);
    for (int s = 32; s > 0; s >>= 1) acc += __shfl_xor(acc, s, 64);
    if (lane == 0) {
        uint32_t u = (uint32_t)row[0] | ((uint32_t)row[1] << 8) | ((uint32_t)row[2] << 16) |
                     ((uint32_t)row[3] << 24);
        y[(size_t)t * ldy + o] = acc * __uint_as_float(u);
    }
}


/* Raw 8-element weight chunk: one 16-byte load (bf16) or two (fp32); NT loads bypass the
 * caches' retention (weights streamed once per launch). */
typedef unsigned int k3u32x4 __attribute__((ext_vector_type(4)));
typedef float k3f32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ uint4 ld16(const void *p)
{
    if (NT) {
        const k3u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const k3u32x4 *>(p));
        return make_uint4(v.x, v.y, v.z, v.w);
    }
    return *reinterpret_cast<const uint4 *>(p);
}

template <typename WT> struct Chunk8;
template <> struct Chunk8<uint16_t> {
    uint4 v;
    template <bool NT>
    __device__ __forceinline__ void load(const uint16_t *p) { v = ld16<NT>(p); }
    __device__ __forceinline__ float at(int k) const
    {
        const uint32_t u = k < 2 ? v.x : k < 4 ? v.y : k < 6 ? v.z : v.w;
        return __uint_as_float((k & 1) ? (u & 0xFFFF0000u) : (u << 16));
    }
};
template <> struct Chunk8<float> {
    float4 a, b;
    template <bool NT>
    __device__ __forceinline__ void load(const float *p)
    {
        const uint4 u = ld16<NT>(p), v = ld16<NT>(p + 4);
        a = make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
        b = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
    }
    __device__ __forceinline__ float at(int k) const
    {
        return k == 0 ? a.x : k == 1 ? a.y : k == 2 ? a.z : k == 3 ? a.w
             : k == 4 ? b.x : k == 5 ? b.y : k == 6 ? b.z : b.w;
    }
};

template <typename WT, int RW, int NT, int U, bool NTLOAD>
__global__ __launch_bounds__(256) void gemv_rows_kernel(float *__restrict__ y, const float *__restrict__ x,
                                                        const WT *__restrict__ W, int in, int out,
                                                        int ntok, int ldy)
{
    const int lane = threadIdx.x & 63;
    const int r0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RW;
    if (r0 >= out) return;
    const int t0 = blockIdx.y * NT;
    const int nch = in >> 3;
    const WT *row[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) row[r] = W + (size_t)min(r0 + r, out - 1) * in;
    const float *xt[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) xt[t] = x + (size_t)min(t0 + t, ntok - 1) * in;
    float acc[RW][NT];
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[r][t] = 0.0f;
    for (int cb = lane; cb < nch; cb += 64 * U) {
        Chunk8<WT> w[U][RW];
        float4 xa[U][NT], xb[U][NT];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int c = cb + 64 * u;
            if (c < nch) {
#pragma unroll
                for (int r = 0; r < RW; r++) w[u][r].template load<NTLOAD>(row[r] + 8 * (size_t)c);
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    xa[u][t] = reinterpret_cast<const float4 *>(xt[t] + 8 * (size_t)c)[0];
                    xb[u][t] = reinterpret_cast<const float4 *>(xt[t] + 8 * (size_t)c)[1];
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (cb + 64 * u < nch) {
#pragma unroll
                for (int r = 0; r < RW; r++)
#pragma unroll
                    for (int t = 0; t < NT; t++) {
                        float a = acc[r][t];
                        a = fmaf(w[u][r].at(0), xa[u][t].x, a);
                        a = fmaf(w[u][r].at(1), xa[u][t].y, a);
                        a = fmaf(w[u][r].at(2), xa[u][t].z, a);
                        a = fmaf(w[u][r].at(3), xa[u][t].w, a);
                        a = fmaf(w[u][r].at(4), xb[u][t].x, a);
                        a = fmaf(w[u][r].at(5), xb[u][t].y, a);
                        a = fmaf(w[u][r].at(6), xb[u][t].z, a);
                        a = fmaf(w[u][r].at(7), xb[u][t].w, a);
                        acc[r][t] = a;
                    }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) {
            float a = acc[r][t];
            for (int s = 32; s > 0; s >>= 1) a += __shfl_xor(a, s, 64);
            acc[r][t] = a;
        }
    if (lane == 0) {
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int r = 0; r < RW; r++)
                if (t0 + t < ntok && r0 + r < out) y[(size_t)(t0 + t) * ldy + r0 + r] = acc[r][t];
    }
}

/* Launch shapes of the row kernel, measured at 12288 x 7168 bf16 (one token): 2 rows per
 * wave with 8 chunks of each in flight and non-temporal weight loads stream at 6.4 TB/s
 * (4 rows x 4 chunks with cached loads: 5.6 TB/s). Two tokens keep the shape with 4 chunks
 * in flight; more tokens re-read the weights per group of 4, so those loads stay cached. */
constexpr int GV_RW = 2;

template <typename WT>
int launch_gemv(float *y, const float *x, const WT *W, int in, int out, int ntok, int ldy,
                hipStream_t st)
{
    const unsigned nwg = (unsigned)((out + 4 * GV_RW - 1) / (4 * GV_RW));
    if (ntok == 1) {
        hipLaunchKernelGGL((gemv_rows_kernel<WT, GV_RW, 1, 8, true>), dim3(nwg, 1), dim3(256), 0, st, y,
                           x, W, in, out, ntok, ldy);
    } else if (ntok == 2) {
        hipLaunchKernelGGL((gemv_rows_kernel<WT, GV_RW, 2, 4, true>), dim3(nwg, 1), dim3(256), 0, st, y,
                           x, W, in, out, ntok, ldy);
    } else {
        hipLaunchKernelGGL((gemv_rows_kernel<WT, GV_RW, 4, 2, false>),
                           dim3(nwg, (unsigned)((ntok + 3) / 4)), dim3(256), 0, st, y, x, W, in, out,
                           ntok, ldy);
    }
    return 0;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" int k3k_gemv_f32(float *y, const float *x, const float *W, int in, int out, int ntok,
                            int ldy, void *stream)
{
    if (out <= 0 || ntok <= 0) return 0;
    const int vec = (in % 8 == 0) && aligned16(x) && aligned16(W);
    if (vec && in > 0) launch_gemv<float>(y, x, W, in, out, ntok, ldy, (hipStream_t)stream);
    else hipLaunchKernelGGL(gemv_kernel<float>, dim3((out + 3) / 4, ntok), dim3(256), 0,
                            (hipStream_t)stream, y, x, W, in, out, vec, ldy);
    K3K_LAUNCH_CHECK("gemv_f32 launch");
    return 0;
}

extern "C" int k3k_gemv_bf16(float *y, const float *x, const uint16_t *W, int in, int out,
                             int ntok, int ldy, void *stream)
{
    if (out <= 0 || ntok <= 0) return 0;
    const int vec = (in % 8 == 0) && aligned16(x) && aligned16(W);
    if (vec && in > 0) launch_gemv<uint16_t>(y, x, W, in, out, ntok, ldy, (hipStream_t)stream);
    else hipLaunchKernelGGL(gemv_kernel<uint16_t>, dim3((out + 3) / 4, ntok), dim3(256), 0,
                            (hipStream_t)stream, y, x, W, in, out, vec, ldy);
    K3K_LAUNCH_CHECK("gemv_bf16 launch");
    return 0;
}

extern "C" int k3k_gemv_q8(float *y, const float *x, const void *W, int in, int out, int ntok,
                           int ldy, void *stream)
{
    if (out <= 0 || ntok <= 0) return 0;
    hipLaunchKernelGGL(gemv_q8_kernel, dim3((out + 3) / 4, ntok), dim3(256), 0,
                       (hipStream_t)stream, y, x, (const uint8_t *)W, in, out, ldy);
    K3K_LAUNCH_CHECK("gemv_q8 launch");
    return 0;
}
