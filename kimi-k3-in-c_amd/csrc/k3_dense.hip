/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_dense.hip -- dense GEMV on the vector units: fp32, bf16 and per-row int8 weights.
 *
 * Replaces k3_matmul (src/core/k3_ops.c:265-291), k3_matmul_bf16 (:1108-1213) and
 * k3_matmul_q8 (:1221-1289) of the reference for the decode shapes. One wave per output
 * row; lane l takes the 8-element chunks l, l+64, ... of the row with one 16-byte (bf16)
 * or two 16-byte (fp32) loads, accumulates them in fp32 in ascending order and the wave
 * reduces with a butterfly. The fp32 and bf16 kernels are one template, so on weights
 * that are the same values they perform the same operations in the same order and agree
 * bit for bit (the reference holds the same property between its two kernels,
 * tests/unit/test_ops.c:798-848). Accumulation is fp32 where the reference uses fp64;
 * the difference is far inside max|err| <= 1e-4 ||ref||inf.
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

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" int k3k_gemv_f32(float *y, const float *x, const float *W, int in, int out, int ntok,
                            int ldy, void *stream)
{
    if (out <= 0 || ntok <= 0) return 0;
    const int vec = (in % 8 == 0) && aligned16(x) && aligned16(W);
    hipLaunchKernelGGL(gemv_kernel<float>, dim3((out + 3) / 4, ntok), dim3(256), 0,
                       (hipStream_t)stream, y, x, W, in, out, vec, ldy);
    K3K_LAUNCH_CHECK("gemv_f32 launch");
    return 0;
}

extern "C" int k3k_gemv_bf16(float *y, const float *x, const uint16_t *W, int in, int out,
                             int ntok, int ldy, void *stream)
{
    if (out <= 0 || ntok <= 0) return 0;
    const int vec = (in % 8 == 0) && aligned16(x) && aligned16(W);
    hipLaunchKernelGGL(gemv_kernel<uint16_t>, dim3((out + 3) / 4, ntok), dim3(256), 0,
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
