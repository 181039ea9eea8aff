/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_gemm.hip -- dense bf16 GEMM on the matrix cores: the always-on shared expert and the
 * trunk projections of many tokens.
 *
 *   Y[t][r] (=, or +=) sum_k W[r][k] * X[t][k]     W bf16 [R][K], X as bf16 terms [T][K]
 *
 * The reference computes these products one token at a time with k3_matmul_bf16 (fp64
 * accumulation, src/core/k3_ops.c:1108-1213); its shared expert is k3_moe's tail
 * (:650-654). Here tokens are batched into a GEMM with fp32 accumulation; activations
 * arrive as one bf16 term (2e-2 bar) or two (hi + lo, x = hi + lo within 2^-17|x|, the
 * 1e-4 ||ref||inf bar), each term one v_mfma_f32_16x16x32_bf16 into the same accumulator.
 *
 * A workgroup of 4 waves (2 x 2) owns a tile of 128 weight rows x BN tokens and walks K 64
 * columns at a time. Each step's A (128 x 64) and B (BN x 64 per term) tiles are loaded
 * from global memory with 16-byte buffer loads (8 consecutive lanes read one row's 128
 * contiguous bytes; rows past R or T read zeros), kept in registers while the MFMAs consume
 * the previous step from LDS, then stored into the other half of a double-buffered LDS
 * (rows padded to 72 elements so the fragment reads of 16 rows spread over the banks); one
 * barrier per step. A wave owns 64 rows x BN/2 tokens: 4 x BN/32 MFMA tiles.
 *
 * GATEUP: the 128 rows are 64 gate rows (W = w_gate) and the same 64 rows of w_up, laid out
 * so that every wave holds 32 gate and the matching 32 up rows; the epilogue applies the
 * activation to each (gate, up) pair in registers and writes it as bf16 term(s) [T][R], the
 * input of the next GEMM. PLAIN writes or accumulates fp32 Y with row stride ldy.
 *
 * Tiles are ordered row block major, token block minor, and dealt to the 8 XCDs in
 * contiguous ranges (workgroup b runs on XCD b % 8), so the token blocks that share a weight
 * row block run on one XCD and read it through one L2.
 */
#include "k3_common.h"
#include "k3k.h"

namespace {

constexpr int DG_KS = 64;             /* K columns per step */
constexpr int DG_LD = DG_KS + 8;      /* LDS row stride in bf16 elements (144 bytes) */
constexpr int DG_BM = 128;            /* weight rows per workgroup */

struct DgArgs {
    const uint16_t *w0, *w1;          /* PLAIN: w0 [R][K]; GATEUP: gate w0, up w1, [R][K] each */
    const uint16_t *xhi, *xlo;        /* [T][K] */
    int R, T, K;
    float *y;                         /* PLAIN output [T][ldy] */
    int ldy, accumulate;
    uint16_t *ahi, *alo;              /* GATEUP output [T][R] (alo may be null) */
    int act;
    float b1, b2;
    int ntr, ntt, per_xcd;            /* row blocks, token blocks, tiles per XCD */
};

template <int MODE, int NS, int BN>
__global__ __launch_bounds__(256) void dense_gemm_kernel(DgArgs a)
{
    constexpr int NJ = BN / 32;                    /* token fragments per wave */
    __shared__ __attribute__((aligned(16))) uint16_t As[2][DG_BM * DG_LD];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][NS][BN * DG_LD];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wv >> 1, wn = wv & 1;
    const int g = lane >> 4, r16 = lane & 15;

    const int xcd = blockIdx.x % K3_NXCD;
    const int tile = xcd * a.per_xcd + (int)blockIdx.x / K3_NXCD;
    if (tile >= a.ntr * a.ntt) return;
    const int rb = tile / a.ntt, tb = tile % a.ntt;
    const int tok0 = tb * BN;
    /* first weight row of this tile in w0 (and w1): GATEUP tiles cover 64 rows of each */
    const int row0 = MODE == K3K_MX_GATEUP ? rb * (DG_BM / 2) : rb * DG_BM;

    const uint32_t Kb = (uint32_t)a.K * 2u;        /* bytes per row */
    const k3_rsrc rw0 = k3_make_rsrc(a.w0, (uint32_t)a.R * Kb);
    const k3_rsrc rw1 = k3_make_rsrc(MODE == K3K_MX_GATEUP ? a.w1 : a.w0, (uint32_t)a.R * Kb);
    const k3_rsrc rxh = k3_make_rsrc(a.xhi, (uint32_t)a.T * Kb);
    const k3_rsrc rxl = k3_make_rsrc(NS == 2 ? a.xlo : a.xhi, (uint32_t)a.T * Kb);

    /* global -> register staging: thread tid loads chunk c = tid + 256 i of a tile, row
     * c / 8, 16-byte column c % 8 */
    constexpr int NA = DG_BM * 8 / 256, NB = BN * 8 / 256;
    uint4 ra[NA], rbh[NB], rbl[NS == 2 ? NB : 1];
    uint32_t aoff[NA], boff[NB];
    /* Rows past R or T get an offset at 2^31, beyond every operand (each is < 2 GiB): the
     * buffer loads return zeros there. Chunk i of thread tid lies in rows 32i..32i+31, so
     * for GATEUP the first half of the chunks are gate rows and the second half up rows. */
    constexpr uint32_t OOB = 0x80000000u;
#pragma unroll
    for (int i = 0; i < NA; i++) {
        const int c = tid + 256 * i, row = c >> 3, col = c & 7;
        const int wrow = MODE == K3K_MX_GATEUP ? row0 + (row & (DG_BM / 2 - 1)) : row0 + row;
        aoff[i] = wrow < a.R ? (uint32_t)wrow * Kb + (uint32_t)col * 16u : OOB;
    }
#pragma unroll
    for (int i = 0; i < NB; i++) {
        const int c = tid + 256 * i, row = c >> 3, col = c & 7;
        const int t = tok0 + row;
        boff[i] = t < a.T ? (uint32_t)t * Kb + (uint32_t)col * 16u : OOB;
    }
    auto gload = [&](int ks) {
        const uint32_t kb = (uint32_t)ks * (DG_KS * 2);
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const uint32_t o = aoff[i] == OOB ? OOB : aoff[i] + kb;
            ra[i] = (MODE == K3K_MX_GATEUP && i >= NA / 2) ? k3_bload16(rw1, o) : k3_bload16(rw0, o);
        }
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const uint32_t o = boff[i] == OOB ? OOB : boff[i] + kb;
            rbh[i] = k3_bload16(rxh, o);
            if (NS == 2) rbl[i] = k3_bload16(rxl, o);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const int c = tid + 256 * i;
            *reinterpret_cast<uint4 *>(&As[buf][(c >> 3) * DG_LD + (c & 7) * 8]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int c = tid + 256 * i;
            *reinterpret_cast<uint4 *>(&Bs[buf][0][(c >> 3) * DG_LD + (c & 7) * 8]) = rbh[i];
            if (NS == 2) *reinterpret_cast<uint4 *>(&Bs[buf][NS - 1][(c >> 3) * DG_LD + (c & 7) * 8]) = rbl[i];
        }
    };

    /* the wave's 4 row fragments inside the 128-row tile */
    int arow[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        arow[i] = MODE == K3K_MX_GATEUP ? (i < 2 ? wm * 32 + 16 * i : DG_BM / 2 + wm * 32 + 16 * (i - 2))
                                        : wm * 64 + 16 * i;
    const int bcol0 = wn * (BN / 2);

    k3_f32x4 acc[4][NJ];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[i][j] = k3_f32x4{0.f, 0.f, 0.f, 0.f};

    const int nks = a.K / DG_KS;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int ks = 0; ks < nks; ks++) {
        const int buf = ks & 1;
        if (ks + 1 < nks) gload(ks + 1);
#pragma unroll
        for (int kk = 0; kk < DG_KS; kk += 32) {
            k3_bf16x8 af[4], bf[NS][NJ];
#pragma unroll
            for (int i = 0; i < 4; i++)
                af[i] = k3_as_bf16x8(*reinterpret_cast<const uint4 *>(&As[buf][(arow[i] + r16) * DG_LD + kk + 8 * g]));
#pragma unroll
            for (int s = 0; s < NS; s++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    bf[s][j] = k3_as_bf16x8(*reinterpret_cast<const uint4 *>(
                        &Bs[buf][s][(bcol0 + 16 * j + r16) * DG_LD + kk + 8 * g]));
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
#pragma unroll
                    for (int s = 0; s < NS; s++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[s][j], acc[i][j], 0, 0, 0);
        }
        if (ks + 1 < nks) lstore(buf ^ 1);
        __syncthreads();
    }

    /* epilogue: lane holds token column r16 and rows 4g..4g+3 of each 16 x 16 tile */
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int t = tok0 + bcol0 + 16 * j + r16;
        if (t >= a.T) continue;
        if (MODE == K3K_MX_GATEUP) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int r = row0 + wm * 32 + 16 * i + 4 * g;
                uint16_t hi[4], lo[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float v = k3_act_pair(acc[i][j][e], acc[i + 2][j][e], a.act, a.b1, a.b2);
                    k3_split2(v, hi[e], lo[e]);
                }
                uint16_t *oh = a.ahi + (size_t)t * a.R + r;
                uint16_t *ol = a.alo ? a.alo + (size_t)t * a.R + r : nullptr;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (r + e < a.R) {
                        oh[e] = hi[e];
                        if (ol) ol[e] = lo[e];
                    }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = row0 + arow[i] + 4 * g;
                float *o = a.y + (size_t)t * a.ldy + r;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (r + e < a.R) o[e] = a.accumulate ? o[e] + acc[i][j][e] : acc[i][j][e];
            }
        }
    }
}

template <int MODE, int NS, int BN>
int launch_dense(DgArgs a, hipStream_t st)
{
    const int rows_per_tile = MODE == K3K_MX_GATEUP ? DG_BM / 2 : DG_BM;
    a.ntr = (a.R + rows_per_tile - 1) / rows_per_tile;
    a.ntt = (a.T + BN - 1) / BN;
    const int tiles = a.ntr * a.ntt;
    a.per_xcd = (tiles + K3_NXCD - 1) / K3_NXCD;
    hipLaunchKernelGGL((dense_gemm_kernel<MODE, NS, BN>), dim3((unsigned)(a.per_xcd * K3_NXCD)), dim3(256),
                       0, st, a);
    K3K_LAUNCH_CHECK("dense gemm launch");
    return 0;
}

/* Token block: 64 tokens while the tiles cannot fill the chip's 256 CUs, else 128. */
template <int MODE, int NS>
int dispatch_dense(const DgArgs &a, hipStream_t st)
{
    const int rows_per_tile = MODE == K3K_MX_GATEUP ? DG_BM / 2 : DG_BM;
    const long tiles128 = (long)((a.R + rows_per_tile - 1) / rows_per_tile) * ((a.T + 127) / 128);
    if (tiles128 >= 512) return launch_dense<MODE, NS, 128>(a, st);
    return launch_dense<MODE, NS, 64>(a, st);
}

}  // namespace

extern "C" int k3k_dense_gemm(float *y, int ldy, int accumulate, const uint16_t *W,
                              const uint16_t *xhi, const uint16_t *xlo, int R, int T, int K,
                              void *stream)
{
    if (R <= 0 || T <= 0) return 0;
    if (K <= 0 || K % DG_KS) return k3k_fail("dense gemm: K must be a multiple of 64", hipErrorInvalidValue);
    if ((unsigned long long)R * K * 2 >= 0x80000000ull || (unsigned long long)T * K * 2 >= 0x80000000ull)
        return k3k_fail("dense gemm: operand of 2 GiB or more", hipErrorInvalidValue);
    DgArgs a = {};
    a.w0 = W;
    a.xhi = xhi;
    a.xlo = xlo;
    a.R = R;
    a.T = T;
    a.K = K;
    a.y = y;
    a.ldy = ldy;
    a.accumulate = accumulate;
    return xlo ? dispatch_dense<K3K_MX_PLAIN, 2>(a, (hipStream_t)stream)
               : dispatch_dense<K3K_MX_PLAIN, 1>(a, (hipStream_t)stream);
}

extern "C" int k3k_dense_gateup(uint16_t *ahi, uint16_t *alo, const uint16_t *wg, const uint16_t *wu,
                                const uint16_t *xhi, const uint16_t *xlo, int R, int T, int K, int act,
                                float b1, float b2, void *stream)
{
    if (R <= 0 || T <= 0) return 0;
    if (K <= 0 || K % DG_KS) return k3k_fail("dense gate/up: K must be a multiple of 64", hipErrorInvalidValue);
    if ((unsigned long long)R * K * 2 >= 0x80000000ull || (unsigned long long)T * K * 2 >= 0x80000000ull)
        return k3k_fail("dense gate/up: operand of 2 GiB or more", hipErrorInvalidValue);
    DgArgs a = {};
    a.w0 = wg;
    a.w1 = wu;
    a.xhi = xhi;
    a.xlo = xlo;
    a.R = R;
    a.T = T;
    a.K = K;
    a.ahi = ahi;
    a.alo = alo;
    a.act = act;
    a.b1 = b1;
    a.b2 = b2;
    return xlo ? dispatch_dense<K3K_MX_GATEUP, 2>(a, (hipStream_t)stream)
               : dispatch_dense<K3K_MX_GATEUP, 1>(a, (hipStream_t)stream);
}
