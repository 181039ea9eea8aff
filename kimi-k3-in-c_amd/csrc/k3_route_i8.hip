/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_route_i8.hip -- the router's chunk partials of many tokens on the int8 matrix cores.
 *
 * The router's logit is the reference's sequential fp64 chain over the products w_k x_k
 * (src/core/k3_ops.c:444-453); the final kernel (k3_route.hip, router_final_kernel)
 * certifies a logit from per-chunk partials P_k and bounds R_k with
 *   |P_k - exact chunk sum| <= u R_k   and   R_k >= sum over the chunk's columns i of |p_i|,
 * u = 2^-53, p_i the exact sum of the chunk's products up to column i. The fp64 matrix
 * cores compute P_k at 78.6 TFLOP/s, and on gfx950 their instructions and the vector ones
 * of a SIMD do not overlap; this file computes the same (P_k, R_k) from exact integer
 * products instead (the digit splitting of Ozaki's error-free matrix product, with a
 * certified bound in place of exactness for the digits it leaves out).
 *
 * Digits. A row's values in one chunk (x of a token, W of an expert) are scaled by one power
 * of two 2^s so that the largest magnitude lies in [64, 128): V = v 2^s. Then
 *   V = d_1 + 2^-7 d_2 + ... + 2^-35 d_6 + rho,   d_i = trunc of the remainder times
 *   2^7(i-1), |d_i| <= 127, |rho| < 2^-35,
 * every step exact in fp32 (V itself too, except where it scales down into the subnormal
 * range, a loss of at most 2^-126 the bound adds). A value with |V| >= 2^-12 (within 2^-19
 * of the row's largest) has no bit below 2^-35 and is represented exactly. The digit
 * planes are stored in the order of the matrix instruction's operands: the block of a
 * 16-row tile, a 64-column step and a digit is 1 KB, lane L = r + 16 g holding row r's
 * columns 16 g .. 16 g + 15 of the step (A and B take the same lane and byte order, so the
 * instruction pairs equal columns whatever its own K order).
 *
 * Level sums. v_mfma_i32_16x16x64_i8 adds 64 exact int8 products per element into int32.
 * For W digit i and x digit j the product has weight 2^-7(i+j-2); the products of equal
 * level l = i + j share one int32 accumulator, l = 2 .. RI_LMAX (at most 6 products of at
 * most 127^2 per column each: below 2^31 for chunks up to RI_CMAX = 4096 columns). At the end
 *   M = C_2 + 2^-7 (C_3 + 2^-7 (C_4 + ...))     (Horner in fp64)
 * and P_k = M 2^-(s_w + s_x) (exact). With G_ij = 127 min(n_w,i, n_x,j) 2^-7(i+j-2), where
 * n_i >= sum |d_i| over the row's chunk (sum |V| for i = 1, 127 times the nonzero values
 * after), so G_ij >= the chunk's sum of |d_w,i d_x,j| times its weight, the bound on
 * |P_k - exact|, scaled:
 *   - products left out: the sum of G_ij over i + j > RI_LMAX;
 *   - the remainders: W'.X' - w^.x^ = rho_w.X' + w^.rho_x, at most
 *     sum|rho_w| max|X'| + (max|W'| + 2^-35) sum|rho_x|, with sum|rho| <= the sum of
 *     min(|V|, 2^-35) over the values below 2^-12;
 *   - the Horner roundings: 1.01 u sum_l |t_l| over its partial values t_l.
 * The prefix magnitudes: before every 64-column step m the accumulators give the chunk's
 * prefix P_m to within the levels above 4, the fp32 rounding (3.3 2^-24 of the G_ij of
 * levels 2-4), the left-out products and the remainders: |P_m| <= |C_2 + 2^-7 C_3 +
 * 2^-14 C_4| (fp32) + those. So
 *   sum_i |p_i| <= 64 sum_m |P_m| + 64 sum_{j in chunk} |W'_j X'_j|,
 * the second sum bounded by ||W'||_2 ||X'||_2 of the chunk (Cauchy-Schwarz). R_k =
 * max(that, E_k / u) covers both uses; all of it is zero for a zero row. The row chunk's
 * scale and these sums come from digit_scale_kernel (a wave per row chunk), the digits
 * from digit_split_kernel. A row chunk holding an infinity or a NaN is left to a plain
 * fp64 chain (its non-finite sum propagates alike in any order).
 */
#include "k3_common.h"
#include "k3k.h"

#include <type_traits>

namespace {

constexpr int RI_ND = 6;                 /* digits per operand */
constexpr int RI_LMAX = 10;              /* products of digits i, j with i + j <= RI_LMAX */
constexpr int RI_NL = RI_LMAX - 1;       /* level accumulators, l = 2 .. RI_LMAX */
constexpr int RI_STEP = 64;              /* columns per step: one int8 matrix instruction */
constexpr int RI_TT = 64, RI_TE = 64;    /* workgroup tile: tokens, experts */
constexpr int RI_BLK = 1024;             /* bytes of a (16-row tile, step, digit) block */
constexpr int RI_BAD = 0x7fffffff;       /* scale of a row chunk with a non-finite value */
/* blocks of one stage: RI_TT / 16 token tiles and RI_TE / 16 expert tiles, RI_ND digits */
constexpr int RI_XB = RI_TT / 16 * RI_ND, RI_WB = RI_TE / 16 * RI_ND, RI_SB = RI_XB + RI_WB;

/* What the bound needs of one row's chunk, from digit_scale_kernel: the scale exponent
 * (RI_BAD: a non-finite value), bounds on rho = sum |V - digits|, l2 = ||V||_2,
 * mx = max |V|, and n1 >= sum |d_1|, n2 >= sum |d_i| for every later digit i. */
struct RiRow {
    double rho, l2, mx;
    int s;
    int n1, n2;
};

/* Weights of the products' bound terms by level group (left out: i + j > RI_LMAX; levels
 * 5 .. RI_LMAX; levels 2-4) and by whether i and j are the first digit: sum 127 2^-7(i+j-2)
 * over the group's pairs of that class, so that sum over the group of 127 min(n_w,i, n_x,j)
 * 2^-7(i+j-2) = sum over the classes of the weight times min(n_w, n_x) of the class. */
struct RiGw {
    double c[3][2][2];
};
constexpr RiGw ri_gw()
{
    RiGw g = {};
    for (int i = 1; i <= RI_ND; i++)
        for (int j = 1; j <= RI_ND; j++) {
            double w = 127.0;
            for (int q = 0; q < i + j - 2; q++) w *= 0x1p-7;
            const int grp = i + j > RI_LMAX ? 0 : i + j >= 5 ? 1 : 2;
            g.c[grp][i > 1][j > 1] += w;
        }
    return g;
}

/* ---- digit split ---------------------------------------------------------------------- */
struct RiSplit {
    uint8_t *dx, *dw;                 /* digit blocks of x and of W */
    RiRow *rx, *rw;                   /* [row][ks] */
    const float *x, *W;
    int T, E, ntx, ntw;               /* rows and 16-row tiles (padded) of x and W */
    int hidden, chunk, ks;
};

constexpr int RI_CMAX = 4096;          /* longest chunk: 16 pieces of 4 columns per lane */

/* Four values -> their digits (word p holds digit p + 1 of value c in byte c), in fp32:
 * every digit step is exact, and so is V = v 2^s except where it scales down into the
 * subnormal range (|V| < 2^-126, all digits zero). */
__device__ __forceinline__ void ri_digits4(float4 v, int s, uint32_t (&w)[RI_ND])
{
    float r[4] = {ldexpf(v.x, s), ldexpf(v.y, s), ldexpf(v.z, s), ldexpf(v.w, s)};
#pragma unroll
    for (int p = 0; p < RI_ND; p++) {
        uint32_t word = 0u;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float t = truncf(r[c]);
            word |= ((uint32_t)(int)t & 0xffu) << (8 * c);
            r[c] = (r[c] - t) * (p + 1 < RI_ND ? 128.0f : 1.0f);
        }
        w[p] = word;
    }
}

/* A wave per (row, chunk) of x, then of W, every load of the row's chunk in flight at once:
 * the row's largest magnitude m = f 2^e (f in [0.5, 1)) gives the scale s = 7 - e (a
 * non-finite value RI_BAD), then the record's bounds from the scaled values V, without their
 * digits: a value with |V| >= 2^-12 has no bit below 2^-35 and is exact in six digits, a
 * smaller one leaves at most min(|V|, 2^-35); |d_1| <= |V| and |d_i| <= 127 where V != 0. */
__global__ __launch_bounds__(256) void digit_scale_kernel(RiSplit a)
{
    const int gw = (int)(blockIdx.x * 4 + (threadIdx.x >> 6)), lane = threadIdx.x & 63;
    const int nx = a.T * a.ks;
    if (gw >= nx + a.E * a.ks) return;
    const bool isx = gw < nx;
    const int rc = isx ? gw : gw - nx, row = rc / a.ks, k = rc % a.ks;
    const k3_rsrc rs = k3_make_rsrc((isx ? a.x : a.W) + (size_t)row * a.hidden, (uint32_t)a.hidden * 4u);
    const int k0 = k * a.chunk, k1 = min(a.hidden, k0 + a.chunk);
    constexpr int NP = RI_CMAX / 256;
    /* all loads at once, those past the chunk reading zeros from past the row */
    float4 v[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const int c = k0 + 4 * lane + 256 * i;
        v[i] = __builtin_bit_cast(float4, k3_bload16(rs, c < k1 ? (uint32_t)c * 4u : 0x80000000u));
    }
    float m = 0.0f;
    int bad = 0;
#pragma unroll
    for (int i = 0; i < NP; i++) {
        bad |= (int)!isfinite(v[i].x) | (int)!isfinite(v[i].y) | (int)!isfinite(v[i].z) | (int)!isfinite(v[i].w);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        m = fmaxf(m, __shfl_xor(m, o, 64));
        bad |= __shfl_xor(bad, o, 64);
    }
    int s = 0;
    if (bad) s = RI_BAD;
    else if (m > 0.0f) {
        int ex;
        frexpf(m, &ex);
        s = 7 - ex;
    }
    float rem = 0.0f, sq = 0.0f, mx = 0.0f, l1 = 0.0f;
    int nnz = 0;
    if (!bad) {
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const float vv[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float V = fabsf(ldexpf(vv[c], s));
                sq = fmaf(V, V, sq);
                mx = fmaxf(mx, V);
                l1 += V;
                nnz += V != 0.0f;
                rem += V < 0x1p-12f ? fminf(V, 0x1p-35f) : 0.0f;
            }
        }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        rem += __shfl_xor(rem, o, 64);
        sq += __shfl_xor(sq, o, 64);
        l1 += __shfl_xor(l1, o, 64);
        mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        nnz += __shfl_xor(nnz, o, 64);
    }
    if (lane == 0) {
        RiRow r;
        /* fp32 sums of at most 2^12 non-negative terms (V^2 rounded once more): low by a
         * relative 2^-11 at most; scaled down, a value may have lost up to 2^-126 */
        const double fl = s < 0 ? 0x1p-126 : 0.0;
        r.rho = (double)rem * (1.0 + 0x1p-10) + fl * a.chunk;
        r.l2 = sqrt((double)sq * (1.0 + 0x1p-10)) * (1.0 + 0x1p-30) + fl * 64.0;
        r.mx = (double)mx + fl;
        r.s = s;
        r.n1 = (int)ceil((double)l1 * (1.0 + 0x1p-10) + fl * a.chunk);
        r.n2 = 127 * nnz;
        (isx ? a.rx : a.rw)[rc] = r;
    }
}

constexpr int RI_SPS = 4;                      /* steps per split workgroup (a wave each) */

/* Digits: a workgroup per (16-row tile of x or W, RI_SPS steps), wave w step w, lane
 * L = r + 16 g the values of row r at columns 16 g .. 16 g + 15 of the step, written as
 * the 16-byte slot L of the step's six 1 KB blocks (a wave stores whole blocks). Rows past
 * the matrix, and row chunks with a non-finite value, write zero digits. */
__global__ __launch_bounds__(64 * RI_SPS) void digit_split_kernel(RiSplit a)
{
    const int nsx = a.ks * (a.chunk / RI_STEP) / RI_SPS;      /* step groups per tile */
    const bool isx = (int)blockIdx.x < a.ntx * nsx;
    const int bi = isx ? (int)blockIdx.x : (int)blockIdx.x - a.ntx * nsx;
    const int tile = bi / nsx, sg = bi % nsx;
    const int rows = isx ? a.T : a.E, ntile = isx ? a.ntx : a.ntw;
    const int tid = threadIdx.x, L = tid & 63, r = L & 15, g = L >> 4, wv = tid >> 6;
    const int gst = sg * RI_SPS + wv, nst = a.chunk / RI_STEP, k = gst / nst;
    const int row = tile * 16 + r;
    const int c = gst * RI_STEP + 16 * g;
    /* the values' loads do not wait for the scale (rows past the matrix read zeros) */
    const k3_rsrc rs = k3_make_rsrc(isx ? a.x : a.W, (uint32_t)((size_t)rows * a.hidden * 4));
    const uint32_t off = row < rows ? (uint32_t)(((size_t)row * a.hidden + c) * 4) : 0x80000000u;
    float4 val[4];
#pragma unroll
    for (int q = 0; q < 4; q++) val[q] = __builtin_bit_cast(float4, k3_bload16(rs, off + 16u * q));
    const int s = row < rows ? (isx ? a.rx : a.rw)[(size_t)row * a.ks + k].s : RI_BAD;
    const bool live = s != RI_BAD;
    uint32_t w[4][RI_ND];
#pragma unroll
    for (int q = 0; q < 4; q++) ri_digits4(live ? val[q] : make_float4(0.f, 0.f, 0.f, 0.f), live ? s : 0, w[q]);
    uint4 *blk = reinterpret_cast<uint4 *>((isx ? a.dx : a.dw) + ((size_t)gst * ntile + tile) * (RI_ND * RI_BLK)) + L;
#pragma unroll
    for (int p = 0; p < RI_ND; p++) blk[p * (RI_BLK / 16)] = make_uint4(w[0][p], w[1][p], w[2][p], w[3][p]);
}

/* ---- partials ------------------------------------------------------------------------- */
struct RiArgs {
    double *part;
    float *rbound;
    const uint8_t *xd, *wd;               /* digit blocks of x and W */
    uint32_t xbytes, wbytes;
    const RiRow *rx, *rw;                 /* [row][ks] */
    const float *x, *W;                   /* fp32 rows, for the chains of non-finite chunks */
    int T, E, hidden, chunk, ks;
    int ntx, ntw;                         /* 16-row tiles of the digit blocks (padded) */
    int *ctr, *idx_reset, n_reset;
};

__device__ __forceinline__ float ri_bound_up(double rb)
{
    return (float)(rb * (1.0 + 0x1p-40)) * (1.0f + 0x1p-20f) + 0x1p-120f;
}

/* The pair (W digit i, x digit j) of every product, level by level but with the levels
 * interleaved (round q takes the q-th pair of each level), so that consecutive products go
 * into different accumulators. */
struct RiPair {
    int i, j;
};
constexpr int RI_NP = 33;                /* pairs with i, j <= RI_ND and i + j <= RI_LMAX */
struct RiPairs {
    RiPair p[RI_NP];
};
constexpr RiPairs ri_pairs()
{
    RiPairs r = {};
    int n = 0;
    for (int q = 0; q < RI_ND; q++)
        for (int l = 2; l <= RI_LMAX; l++) {
            /* the q-th pair of level l: i from max(1, l - RI_ND) upwards */
            const int i = (l - RI_ND > 1 ? l - RI_ND : 1) + q, j = l - i;
            if (i <= RI_ND && j >= 1 && n < RI_NP) r.p[n++] = RiPair{i, j};
        }
    return r;
}
static_assert(ri_pairs().p[RI_NP - 1].i > 0, "pair count");

/* A workgroup of 8 waves takes (chunk, 64 tokens, 64 experts); wave w the tokens
 * 32 (w >> 2) .. + 31 (two 16-row tiles) and experts 16 (w & 3) .. + 15. Per 64-column step
 * the stage's 48 digit blocks (4 token tiles and 4 expert tiles, 6 digits each: 48 KB) go
 * into LDS by buffer-load DMA (6 per wave), two steps ahead in a ring of three stages, so a
 * stage has two steps of products to arrive in. The barrier is issued directly: the one the
 * compiler emits would also wait for the DMA of the next step, which is meant to land a step
 * later. Loads past the last step read zeros from past the buffer, so every step waits for
 * exactly its own loads. Workgroups are dealt to the XCDs (workgroup b runs on XCD b % 8) in
 * contiguous ranges of (chunk, token tile) pairs, the expert tiles of a pair together, so a
 * token tile's digits are fetched into one L2 and read there by its expert tiles. */
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void router_partial_i8_kernel(RiArgs a)
{
    typedef int v4i __attribute__((ext_vector_type(4)));
    __shared__ __attribute__((aligned(1024))) uint4 xs0[RI_SB * 64];
    __shared__ __attribute__((aligned(1024))) uint4 xs1[RI_SB * 64];
    __shared__ __attribute__((aligned(1024))) uint4 xs2[RI_SB * 64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wt = wv >> 2, we = wv & 3;
    if (a.ctr && blockIdx.x == 0) {
        /* the final kernel's arrival counter, and the idx its gathering workgroup waits on */
        if (tid == 0) *a.ctr = 0;
        for (int i = tid; i < a.n_reset; i += blockDim.x) a.idx_reset[i] = -1;
    }
    const int ntt = a.ntx / (RI_TT / 16), nte = a.ntw / (RI_TE / 16);
    const int npair = a.ks * ntt, per = (npair + K3_NXCD - 1) / K3_NXCD;
    const int bi = blockIdx.x / K3_NXCD, xcd = blockIdx.x % K3_NXCD;
    const int pi = bi / nte, et = bi % nte, pr = xcd * per + pi;
    if (pi >= per || pr >= npair) return;
    const int k = pr / ntt, tt = pr % ntt;
    const int nst = a.chunk / RI_STEP;
    const k3_rsrc rx = k3_make_rsrc(a.xd, a.xbytes), rw = k3_make_rsrc(a.wd, a.wbytes);
    constexpr uint32_t OOB = 0x80000000u;
    constexpr int NLD = RI_SB / 8;                     /* DMA per wave per step */
    static_assert(RI_SB % 8 == 0 && RI_XB % 8 == 0, "DMA slots: whole rounds of the 8 waves");
    /* step st's stage into slot S: block q = wv + 8 i, a token block (tile q / 6, digit
     * q % 6) for q < RI_XB, else expert block q - RI_XB */
    auto load = [&](int st, auto slot) {
        constexpr int S = decltype(slot)::value;
        uint4 *buf = S == 0 ? xs0 : S == 1 ? xs1 : xs2;
        const bool in = st < nst;
        const size_t gst = (size_t)k * nst + (in ? st : 0);
        const uint32_t xb = (uint32_t)((gst * a.ntx + (size_t)tt * (RI_TT / 16)) * (RI_ND * RI_BLK));
        const uint32_t wb = (uint32_t)((gst * a.ntw + (size_t)et * (RI_TE / 16)) * (RI_ND * RI_BLK));
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            const int q = wv + 8 * i;
            if (i < RI_XB / 8)
                k3_dma16(rx, &buf[q * 64], in ? (uint32_t)(q * RI_BLK + lane * 16) : OOB, in ? xb : 0u);
            else
                k3_dma16(rw, &buf[q * 64], in ? (uint32_t)((q - RI_XB) * RI_BLK + lane * 16) : OOB, in ? wb : 0u);
        }
    };
    v4i acc[RI_NL][2];
#pragma unroll
    for (int l = 0; l < RI_NL; l++) acc[l][0] = acc[l][1] = v4i{0, 0, 0, 0};
    float snap[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    constexpr RiPairs PR = ri_pairs();
    auto step = [&](int st, auto slot) {
        constexpr int S = decltype(slot)::value;
        constexpr int S2 = (S + 2) % 3;
        const uint4 *cur = S == 0 ? xs0 : S == 1 ? xs1 : xs2;
        /* this step's stage is in (the next step's stays in flight); after the barrier every
         * wave's part of it has landed and every wave is past the step that read slot S2 */
        __builtin_amdgcn_s_waitcnt((NLD & 15) | (7 << 4) | (15 << 8) | ((NLD >> 4) << 14));
        __asm__ volatile("s_barrier" ::: "memory");
        load(st + 2, std::integral_constant<int, S2>{});
        v4i xa[RI_ND][2], wb[RI_ND];
#pragma unroll
        for (int p = 0; p < RI_ND; p++) {
#pragma unroll
            for (int h = 0; h < 2; h++)
                xa[p][h] = __builtin_bit_cast(v4i, cur[((2 * wt + h) * RI_ND + p) * 64 + lane]);
            wb[p] = __builtin_bit_cast(v4i, cur[(RI_XB + we * RI_ND + p) * 64 + lane]);
        }
        /* the prefix before this step, from levels 2-4 (written one step ago) */
        if (st > 0) {
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    snap[h][r] += fabsf(fmaf((float)acc[2][h][r], 0x1p-14f,
                                             fmaf((float)acc[1][h][r], 0x1p-7f, (float)acc[0][h][r])));
        }
#pragma unroll
        for (int n = 0; n < RI_NP; n++) {
            const int i = PR.p[n].i, j = PR.p[n].j;
#pragma unroll
            for (int h = 0; h < 2; h++)
                acc[i + j - 2][h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[j - 1][h], wb[i - 1], acc[i + j - 2][h], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    using Z0 = std::integral_constant<int, 0>;
    using Z1 = std::integral_constant<int, 1>;
    using Z2 = std::integral_constant<int, 2>;
    load(0, Z0{});
    load(1, Z1{});
    int st = 0;
    for (; st + 2 < nst; st += 3) {
        step(st, Z0{});
        step(st + 1, Z1{});
        step(st + 2, Z2{});
    }
    if (st < nst) step(st, Z0{});
    if (st + 1 < nst) step(st + 1, Z1{});
    /* the loads past the last step (zeros) land before the workgroup's LDS is released */
    __builtin_amdgcn_s_waitcnt(0);
    /* element (r) of block h: token 32 wt + 16 h + 4 (lane / 16) + r, expert 16 we + lane % 16 */
    const int e = et * RI_TE + 16 * we + (lane & 15);
    if (e >= a.E) return;
    const double C = (double)a.chunk;
    constexpr RiGw GW = ri_gw();
    const RiRow we_ = a.rw[(size_t)e * a.ks + k];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int t = tt * RI_TT + 32 * wt + 16 * h + 4 * (lane >> 4) + r;
            if (t >= a.T) continue;
            const size_t o = ((size_t)k * a.T + t) * a.E + e;
            const RiRow xt = a.rx[(size_t)t * a.ks + k];
            if (xt.s == RI_BAD || we_.s == RI_BAD) {
                /* a non-finite value: the chunk's own fp64 chain, its partial values'
                 * magnitudes as the bound (what it would be for finite values) */
                const int c0 = k * a.chunk, c1 = min(a.hidden, c0 + a.chunk);
                const float *xr = a.x + (size_t)t * a.hidden, *wr = a.W + (size_t)e * a.hidden;
                double s = 0.0, b = 0.0;
                for (int c = c0; c < c1; c++) {
                    s = fma((double)wr[c], (double)xr[c], s);
                    b += fabs(s);
                }
                a.part[o] = s;
                a.rbound[o] = ri_bound_up(b);
                continue;
            }
            double tv = (double)acc[RI_NL - 1][h][r], errc = fabs(tv);
#pragma unroll
            for (int l = RI_NL - 2; l >= 0; l--) {
                tv = fma(tv, 0x1p-7, (double)acc[l][h][r]);
                errc += fabs(tv);
            }
            /* 127 min(n_w,i, n_x,j) >= sum |d_w,i d_x,j| over the chunk, by level group:
             * left out (above RI_LMAX), levels 5 .. RI_LMAX (not in the prefix estimate),
             * levels 2-4 (their fp32 rounding in it) */
            const double m[2][2] = {{(double)min(we_.n1, xt.n1), (double)min(we_.n1, xt.n2)},
                                    {(double)min(we_.n2, xt.n1), (double)min(we_.n2, xt.n2)}};
            double gs[3];
#pragma unroll
            for (int q = 0; q < 3; q++)
                gs[q] = (GW.c[q][0][0] * m[0][0] + GW.c[q][0][1] * m[0][1]) + (GW.c[q][1][0] * m[1][0] + GW.c[q][1][1] * m[1][1]);
            const double om = gs[0], t5 = gs[1], f4 = gs[2];
            const double rho = we_.rho * xt.mx + (we_.mx + 0x1p-35) * xt.rho;
            const double esc = om + rho + 1.01 * 0x1p-53 * errc;
            const double rref = 64.0 * (double)snap[h][r] * (1.0 + 0x1p-15) +
                                C * (t5 + 3.3 * 0x1p-24 * f4 + om + rho) + 64.0 * we_.l2 * xt.l2 * (1.0 + 0x1p-30);
            const int sc = -(we_.s + xt.s);
            a.part[o] = ldexp(tv, sc);
            a.rbound[o] = ri_bound_up(ldexp(fmax(rref, esc * 0x1p53), sc));
        }
}

}  // namespace

/* ---- host side ------------------------------------------------------------------------ */
/* The int8 partials serve batches of at least RI_MIN_T tokens with rows of a multiple of
 * 256 columns; fewer tokens keep the fp64 kernels (at 512 tokens those took 84 us against
 * 100 us for the digits and the int8 partials). */
constexpr int RI_MIN_T = 1024;

static int ri_round(int v, int m) { return (v + m - 1) / m * m; }

extern "C" int k3k_router_i8_chunk(int T, int hidden, int n_experts)
{
    if (T < RI_MIN_T || hidden <= 0 || hidden % RI_STEP || n_experts <= 0) return 0;
    const long tiles = (long)(ri_round(T, RI_TT) / RI_TT) * (ri_round(n_experts, RI_TE) / RI_TE);
    const long cus = k3k_cu_count() > 0 ? k3k_cu_count() : 1;
    /* the fewest chunks (equal, whole step groups of the split) that give every CU two
     * workgroups, at most RI_CMAX columns each (a scale wave holds its row's chunk) */
    if (hidden % (RI_STEP * RI_SPS)) return 0;
    const int ngrp = hidden / (RI_STEP * RI_SPS);
    int ks = 1;
    for (; ks < ngrp; ks++)
        if (ngrp % ks == 0 && tiles * ks >= 2 * cus && hidden / ks <= RI_CMAX) break;
    while (hidden / ks > RI_CMAX || ngrp % ks) ks++;
    const size_t xbytes = (size_t)ri_round(T, RI_TT) * (size_t)hidden * RI_ND;
    const size_t wbytes = (size_t)ri_round(n_experts, RI_TE) * (size_t)hidden * RI_ND;
    if (xbytes >= ((size_t)1 << 31) || wbytes >= ((size_t)1 << 31)) return 0;
    return hidden / ks;
}

static size_t ri_al(size_t n) { return (n + 255) / 256 * 256; }

extern "C" size_t k3k_router_i8_bytes(int T, int hidden, int n_experts, int chunk)
{
    if (chunk <= 0) return 0;
    const size_t ks = (size_t)(hidden / chunk), Tp = ri_round(T, RI_TT), Ep = ri_round(n_experts, RI_TE);
    return ri_al(Tp * hidden * RI_ND) + ri_al(Ep * hidden * RI_ND) + ri_al(Tp * ks * sizeof(RiRow)) +
           ri_al(Ep * ks * sizeof(RiRow));
}

extern "C" int k3k_router_partial_i8(double *part, float *rbound, void *scratch, const float *x, int T,
                                     const float *W, int hidden, int n_experts, int chunk, int *ctr,
                                     int *idx, int n_idx, void *stream)
{
    if (ctr && n_idx > 0 && !idx) return k3k_fail("router_partial_i8: idx to reset", hipErrorInvalidValue);
    if (!ctr) n_idx = 0;
    if (T <= 0 || n_experts <= 0) return 0;
    if (chunk != k3k_router_i8_chunk(T, hidden, n_experts) || !scratch ||
        (((uintptr_t)x) | ((uintptr_t)W)) % 16)
        return k3k_fail("router_partial_i8: shape", hipErrorInvalidValue);
    const int ks = hidden / chunk, Tp = ri_round(T, RI_TT), Ep = ri_round(n_experts, RI_TE);
    char *p = (char *)scratch;
    auto take = [&](size_t n) { char *q = p; p += ri_al(n); return q; };
    uint8_t *xd = (uint8_t *)take((size_t)Tp * hidden * RI_ND);
    uint8_t *wd = (uint8_t *)take((size_t)Ep * hidden * RI_ND);
    RiRow *rx = (RiRow *)take((size_t)Tp * ks * sizeof(RiRow));
    RiRow *rwv = (RiRow *)take((size_t)Ep * ks * sizeof(RiRow));
    hipStream_t st = (hipStream_t)stream;
    const RiSplit sa = {xd, wd, rx, rwv, x, W, T, n_experts, Tp / 16, Ep / 16, hidden, chunk, ks};
    hipLaunchKernelGGL(digit_scale_kernel, dim3((unsigned)(((size_t)(T + n_experts) * ks + 3) / 4)), dim3(256), 0, st,
                       sa);
    K3K_LAUNCH_CHECK("digit scale launch");
    const int nsx = hidden / RI_STEP / RI_SPS;
    hipLaunchKernelGGL(digit_split_kernel, dim3((unsigned)((Tp / 16 + Ep / 16) * nsx)), dim3(64 * RI_SPS), 0, st, sa);
    K3K_LAUNCH_CHECK("digit split launch");
    RiArgs a;
    a.part = part;
    a.rbound = rbound;
    a.xd = xd;
    a.wd = wd;
    a.xbytes = (uint32_t)((size_t)Tp * hidden * RI_ND);
    a.wbytes = (uint32_t)((size_t)Ep * hidden * RI_ND);
    a.rx = rx;
    a.rw = rwv;
    a.x = x;
    a.W = W;
    a.T = T;
    a.E = n_experts;
    a.hidden = hidden;
    a.chunk = chunk;
    a.ks = ks;
    a.ntx = Tp / 16;
    a.ntw = Ep / 16;
    a.ctr = ctr;
    a.idx_reset = idx;
    a.n_reset = n_idx;
    const int npair = ks * (Tp / RI_TT), per = (npair + K3_NXCD - 1) / K3_NXCD;
    const int grid = per * (Ep / RI_TE) * K3_NXCD;
    hipLaunchKernelGGL(router_partial_i8_kernel, dim3(grid), dim3(512), 0, st, a);
    K3K_LAUNCH_CHECK("router partial i8 launch");
    return 0;
}
