/* SPDX-License-Identifier: Apache-2.0 */
/* k3_common.h -- device-side helpers shared by the HIP translation units. */
#ifndef K3_COMMON_H
#define K3_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 k3_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 k3_bf16x2 __attribute__((ext_vector_type(2)));
typedef float k3_f32x4 __attribute__((ext_vector_type(4)));
typedef float k3_f32x2 __attribute__((ext_vector_type(2)));

/* Upper bound on top-k, as the reference's K3_MAX_TOPK (include/k3/k3.h:557). */
#define K3_MAX_TOPK_DEV 64

/* XCDs of an MI355X (8 x 32 CUs, an L2 each); the dispatcher hands workgroup b to XCD
 * b % 8. Kernels use it only to group work that shares data; results do not depend on it. */
#define K3_NXCD 8

/* Tiled MXFP4 layout (k3k_mx_tile). Row tiles of 16 rows go in groups of 4 (rows padded to
 * a multiple of 64). A tile's chunk c (512 columns: 4 KB of codes, 256 B of scales) has the
 * index k3_tile_idx(t, c) = (group * nchunk + c) * 4 + t % 4, so inside a group the four
 * tiles' chunk c lie side by side, chunk after chunk: a wave that streams its four tiles a
 * chunk at a time reads 16 KB in one piece. With each tile's chunks together instead, the
 * four loads of a step were 16 KB apart for 2048-column rows and the expert down kernel took
 * 0.367 against 0.358 ms.
 * Codes of tile t, chunk c, step d, lane l: byte k3_tile_idx * 4096 + 1024 d + 16 l (the
 * block 4d + g of row 16t + r, l = 16g + r); its scales: the dword at k3_tile_idx * 256 +
 * 4 l, byte d. Moving to chunk c + 1 adds K3_TILE_CSTRIDE (codes) / K3_TILE_SCSTRIDE. */
#define K3_TILE_ROWS_PAD 64
#define K3_TILE_CSTRIDE (4u * 4096u)
#define K3_TILE_SCSTRIDE (4u * 256u)
__host__ __device__ __forceinline__ uint32_t k3_tile_idx(int t, int c, int nchunk)
{
    return ((uint32_t)(t >> 2) * (uint32_t)nchunk + (uint32_t)c) * 4u + (uint32_t)(t & 3);
}
/* rows of a tiled matrix, padded */
__host__ __device__ __forceinline__ uint32_t k3_tile_prows(int rows)
{
    return ((uint32_t)rows + K3_TILE_ROWS_PAD - 1) / K3_TILE_ROWS_PAD * K3_TILE_ROWS_PAD;
}

/* Record a launch/runtime failure for k3k_error() (defined in k3_rt.hip). */
extern "C" int k3k_fail(const char *what, hipError_t e);
#define K3K_LAUNCH_CHECK(what)                                   \
    do {                                                         \
        hipError_t e_ = hipGetLastError();                       \
        if (e_ != hipSuccess) return k3k_fail(what, e_);         \
    } while (0)

/* fp32 -> bf16 bits, round to nearest even. Infinities stay infinite, NaN stays NaN. */
__device__ __forceinline__ uint16_t k3_bf16_rne(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7F800000u) == 0x7F800000u)                 /* inf or NaN */
        return (uint16_t)((u >> 16) | ((u & 0x007FFFFFu) ? 0x0040u : 0u));
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float k3_bf16_to_f32(uint16_t h)
{
    return __uint_as_float((uint32_t)h << 16);
}

/* Two-term bf16 split: x = hi + lo + r with |r| <= 2^-17 |x|. x - hi is exact in fp32. */
__device__ __forceinline__ void k3_split2(float x, uint16_t &hi, uint16_t &lo)
{
    hi = k3_bf16_rne(x);
    const float h = k3_bf16_to_f32(hi);
    const float d = (__float_as_uint(x) & 0x7F800000u) == 0x7F800000u ? 0.0f : x - h;
    lo = k3_bf16_rne(d);
}

/* E8M0 scale byte as the f32 operand of v_cvt_scalef32_pk_*_fp4. The instruction takes
 * only the exponent field of that operand (checked on gfx950 for every byte 0..254,
 * including 0 -> 2^-127), so the byte goes straight into the exponent bits. Byte 255
 * (NaN by the OCP spec, zero in the reference) is handled by the caller zeroing the
 * block's codes, because no exponent field yields a zero scale. */
__device__ __forceinline__ float k3_e8m0_operand(uint32_t s)
{
    return __uint_as_float(s << 23);
}

/* E8M0 byte to its value for fp32 arithmetic: 2^(s-127), 255 -> 0. s = 0 gives the fp32
 * subnormal 2^-127, which the device keeps (fp32 denormals are not flushed). */
__device__ __forceinline__ float k3_e8m0_value(uint32_t s)
{
    if (s == 255u) return 0.0f;
    if (s == 0u) return __uint_as_float(0x00400000u);
    return __uint_as_float(s << 23);
}

__device__ __forceinline__ float k3_e2m1_value(uint32_t code)
{
    const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    const float m = mag[code & 7u];
    return (code & 8u) ? -m : m;
}

/* Eight E2M1 codes (one dword, low nibble first) scaled by 2^(s-127) into eight bf16
 * lanes, exact for every s in 0..254. */
__device__ __forceinline__ k3_bf16x8 k3_dequant8_bf16(uint32_t codes, float scale_op)
{
    const k3_bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, scale_op, 0);
    const k3_bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, scale_op, 1);
    const k3_bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, scale_op, 2);
    const k3_bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, scale_op, 3);
    k3_bf16x8 r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

/* Loads through explicitly global (address space 1) pointers. Pointers read from memory
 * (the expert table) or carried in a struct argument are generic to the compiler, which
 * would otherwise emit flat loads; a flat load also counts against lgkmcnt, so every wait
 * for an LDS read would drain all outstanding weight loads. */
typedef __attribute__((address_space(1))) const uint4 k3_g_uint4;
typedef __attribute__((address_space(1))) const uint8_t k3_g_u8;
typedef __attribute__((address_space(1))) const uint16_t k3_g_u16;
typedef __attribute__((address_space(1))) const float k3_g_f32;
typedef __attribute__((address_space(1))) const int k3_g_int;

__device__ __forceinline__ uint4 k3_ldg16(const void *p)
{
#if defined(__HIP_DEVICE_COMPILE__)
    k3_g_uint4 *gp = (k3_g_uint4 *)p;
    return make_uint4(gp->x, gp->y, gp->z, gp->w);
#else
    (void)p;
    return make_uint4(0, 0, 0, 0);
#endif
}

/* Buffer loads: a wave-uniform descriptor (base, size in bytes) and a per-lane 32-bit byte
 * offset. They count against vmcnt only, and a load past `bytes` returns zeros. The third
 * descriptor word 0x00020000 is the raw-buffer format of the gfx9 family. */
typedef __amdgpu_buffer_rsrc_t k3_rsrc;

__device__ __forceinline__ k3_rsrc k3_make_rsrc(const void *base, uint32_t bytes)
{
    /* The caller guarantees base and bytes are wave-uniform. Pointers read from memory
     * through a generic pointer (the expert table) are divergent to the compiler, which
     * would then wrap every load in a readfirstlane loop; reading lane 0 here makes the
     * descriptor scalar. */
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    void *ub = (void *)(uintptr_t)(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(ub, 0, __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

/* Cache policy of a load: K3_LD_NT marks data streamed once (expert weights), which moves
 * through the caches without displacing what is reused. */
enum { K3_LD_DEFAULT = 0, K3_LD_NT = 2 };
template <int POL = K3_LD_DEFAULT>
__device__ __forceinline__ uint4 k3_bload16(k3_rsrc r, uint32_t off)
{
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POL));
}
template <int POL = K3_LD_DEFAULT>
__device__ __forceinline__ uint32_t k3_bload4(k3_rsrc r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, POL);
}

/* 16 bytes per lane from a buffer straight into LDS (buffer_load_dwordx4 ... lds): lane L
 * writes lds_row + 16 L, where lds_row is wave-uniform; counts against vmcnt. The builtin
 * exists only for the device pass (in the host pass it would drop the kernel's stub). */
__device__ __forceinline__ void k3_dma16(k3_rsrc r, void *lds_row, uint32_t voff, uint32_t soff)
{
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds_row, 16, voff, soff, 0, 0);
#else
    (void)r; (void)lds_row; (void)voff; (void)soff;
#endif
}

__device__ __forceinline__ k3_bf16x8 k3_as_bf16x8(uint4 v)
{
    return __builtin_bit_cast(k3_bf16x8, v);
}

/* Sigmoid in the reference's form 1/(1+expf(-x)) with the device expf. The router does
 * NOT use this one: it reproduces the host libm expf bit for bit (k3_route.hip). */
__device__ __forceinline__ float k3_sigmoid_dev(float x)
{
    return 1.0f / (1.0f + expf(-x));
}

/* Expert activations on one (gate, up) pair, evaluated in the reference's operation
 * order: SiTU-GLU k3_ops.c:115-121, SiLU-GLU (g*sigmoid(g))*u after k3_ops.c:160. */
__device__ __forceinline__ float k3_act_pair(float g, float u, int act, float b1, float b2)
{
    if (act == 1) {
        const float a = g * k3_sigmoid_dev(g);
        return a * u;
    }
    const float a = b1 * tanhf(g / b1) * k3_sigmoid_dev(g);
    const float v = b2 * tanhf(u / b2);
    return a * v;
}

/* The same activations for the bf16 prefill path, whose result is rounded to bf16: exp
 * through the hardware exp2 (__expf) and tanh(y) = 1 - 2 / (e^(2y) + 1), a relative error
 * near 1e-6 (far below bf16's 2^-8) and few registers. */
__device__ __forceinline__ float k3_act_pair_fast(float g, float u, int act, float b1, float b2)
{
    const float sg = __fdividef(1.0f, 1.0f + __expf(-g));
    if (act == 1) return g * sg * u;
    const float tg = 1.0f - __fdividef(2.0f, __expf(2.0f * (g / b1)) + 1.0f);
    const float tu = 1.0f - __fdividef(2.0f, __expf(2.0f * (u / b2)) + 1.0f);
    return (b1 * tg * sg) * (b2 * tu);
}

/* Per-workgroup stamps (K3kMxArgs.stamps): three u64 at the workgroup's slot, its start
 * and end on the 100 MHz clock and the hardware id (XCC_ID << 32 | HW_ID: CU in bits 8-11,
 * shader array 12, shader engine 13-15). The start is stored when it is taken, so that no
 * register holds it through the kernel. */
__device__ __forceinline__ void k3_stamp_begin(unsigned long long *stamps)
{
    stamps[3 * (size_t)blockIdx.x] = __builtin_amdgcn_s_memrealtime();
}

__device__ __forceinline__ void k3_stamp_end(unsigned long long *stamps)
{
    unsigned long long *p = stamps + 3 * (size_t)blockIdx.x;
    const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
    const unsigned hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);     /* HW_REG_HW_ID */
    const unsigned xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20);   /* HW_REG_XCC_ID */
    p[1] = t1;
    p[2] = ((unsigned long long)xcc << 32) | hw;
}

#endif
