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
 * A workgroup of 4 waves (2 x 2) owns a tile of 128 weight rows x BN tokens (BN = 128 with
 * one activation term, 64 with two) and walks its K range 64 columns at a time. A wave owns
 * 64 rows x BN/2 tokens, 4 x BN/32 accumulator blocks: per 32 columns it reads 4 weight and
 * BN/32 (per term) activation fragments from LDS for 16 MFMAs, so the LDS delivers what the
 * matrix cores consume. A step's two 32-column halves read their fragments into registers
 * of their own, each half's reads issued under the other half's MFMAs. Each 64-column
 * step's tiles sit in a double-buffered LDS (rows padded to 72 elements: the 16 rows of a
 * fragment read start 36 banks apart, so a 16-lane group's 16-byte reads cover the 64 banks
 * once); one barrier per step. The weight tile A (128 x 64) comes from global memory with
 * 16-byte buffer loads (8 consecutive lanes read one row's 128 contiguous bytes; rows past R
 * read zeros from beyond the buffer) two steps ahead, in a ring of two register slots, and
 * is stored into LDS; the activation tile B (BN x 64 per term) goes into LDS by buffer-load
 * DMA one step ahead.
 *
 * When the tiles cannot give every CU a workgroup, K is split into S slices (at least
 * 256 columns each): slice s writes its fp32 sums to part[s][t][col], and a second kernel
 * adds the slices in order and finishes (the activation, or the write / accumulation of
 * y). Without a partials buffer S is 1 and the GEMM kernel finishes itself.
 *
 * GATEUP: the 128 rows are 64 gate rows (W = w_gate) and the same 64 rows of w_up, laid out
 * so that every wave holds 32 gate and the matching 32 up rows; the activation is applied to
 * each (gate, up) pair and written as bf16 term(s) [T][R], the input of the next GEMM (with
 * slices, part columns 0..R-1 hold gate sums and R..2R-1 up sums). PLAIN writes or
 * accumulates fp32 Y with row stride ldy.
 *
 * Tiles are ordered row block major, token block minor, and dealt to the 8 XCDs in
 * contiguous ranges (workgroup b runs on XCD b % 8), so the token blocks and slices that
 * share a weight row block run on one XCD and read it through one L2.
 */
#include "k3_common.h"
#include "k3k.h"

#include <type_traits>

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
    float *part;                      /* nsl > 1: [nsl][T][ncol] fp32 slice sums */
    int nsl, ncol;                    /* K slices; part columns (R, or 2R for GATEUP) */
    int ntr, ntt, per_xcd;            /* row blocks, token blocks, work items per XCD */
};

template <int MODE, int NS, int BN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 8))) void dense_gemm_kernel(DgArgs a)
{
    constexpr int NJ = BN / 32;                    /* token fragments per wave */
    constexpr int NA = DG_BM * 8 / 256;            /* 16-byte weight chunks per thread */
    /* a step's activation tile in LDS: NS terms of BN rows of DG_LD elements, i.e. 9
     * 16-byte slots per row (8 of data, 1 of padding); NDMA DMA instructions per wave fill
     * it, the slots past the tile taking zeros */
    constexpr int BSLOT = NS * BN * DG_LD / 8, NDMA = (BSLOT + 255) / 256;
    static_assert((BN * DG_LD / 8) % 64 == 0, "a DMA instruction stays inside one term");
    __shared__ __attribute__((aligned(16))) uint16_t As[2][DG_BM * DG_LD];
    /* two arrays rather than one indexed array, so that the compiler can tell a DMA into
     * one stage buffer from reads of the other (and waits for no DMA before those reads) */
    __shared__ __attribute__((aligned(16))) uint16_t Bs0[NDMA * 256 * 8], Bs1[NDMA * 256 * 8];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wv >> 1, wn = wv & 1;
    const int g = lane >> 4, r16 = lane & 15;

    const int xcd = blockIdx.x % K3_NXCD;
    const int item = xcd * a.per_xcd + (int)blockIdx.x / K3_NXCD;
    if (item >= a.ntr * a.ntt * a.nsl) return;
    const int sl = item % a.nsl, tile = item / a.nsl;
    const int rb = tile / a.ntt, tb = tile % a.ntt;
    const int tok0 = tb * BN;
    /* first weight row of this tile in w0 (and w1): GATEUP tiles cover 64 rows of each */
    const int row0 = MODE == K3K_MX_GATEUP ? rb * (DG_BM / 2) : rb * DG_BM;
    const int nks_all = a.K / DG_KS;
    const int ks0 = sl * nks_all / a.nsl, nks = (sl + 1) * nks_all / a.nsl - ks0;

    const uint32_t Kb = (uint32_t)a.K * 2u;        /* bytes per row */
    const k3_rsrc rw0 = k3_make_rsrc(a.w0, (uint32_t)a.R * Kb);
    const k3_rsrc rw1 = k3_make_rsrc(MODE == K3K_MX_GATEUP ? a.w1 : a.w0, (uint32_t)a.R * Kb);
    const k3_rsrc rxh = k3_make_rsrc(a.xhi, (uint32_t)a.T * Kb);
    const k3_rsrc rxl = k3_make_rsrc(NS == 2 ? a.xlo : a.xhi, (uint32_t)a.T * Kb);

    /* Weights: global -> register staging: thread tid loads chunk c = tid + 256 i of the
     * tile, row c / 8, 16-byte column c % 8. Rows past R, and steps past the slice, get an
     * offset at 2^31, beyond every operand (each is < 2 GiB): the buffer loads return zeros
     * there, and no load sits under a branch. Chunk i of thread tid lies in rows
     * 32i..32i+31, so for GATEUP the first half of the chunks are gate rows and the second
     * half up rows. */
    constexpr uint32_t OOB = 0x80000000u;
    uint32_t aoff[NA];
#pragma unroll
    for (int i = 0; i < NA; i++) {
        const int c = tid + 256 * i, row = c >> 3, col = c & 7;
        const int wrow = MODE == K3K_MX_GATEUP ? row0 + (row & (DG_BM / 2 - 1)) : row0 + row;
        aoff[i] = wrow < a.R ? (uint32_t)wrow * Kb + (uint32_t)(ks0 * DG_KS * 2) + (uint32_t)col * 16u : OOB;
    }
    /* Activations: straight into LDS by the buffer unit (buffer_load_dwordx4 ... lds).
     * Instruction i of wave wv fills slots 64 (wv + 4 i) + lane of the stage buffer: term
     * slot / (9 BN), row (slot / 9) % BN, 16-byte column slot % 9 (8: the padding slot).
     * Padding, slots past the tile and rows past T read at OOB (zeros); the step's column
     * offset goes in the scalar offset. */
    uint32_t doff[NDMA];
#pragma unroll
    for (int i = 0; i < NDMA; i++) {
        const int slot = 64 * (wv + 4 * i) + lane, term = slot / (9 * BN);
        const int row = (slot / 9) % BN, col = slot % 9, t = tok0 + row;
        doff[i] = slot < BSLOT && col < 8 && t < a.T && term < NS
                      ? (uint32_t)t * Kb + (uint32_t)(ks0 * DG_KS * 2) + (uint32_t)col * 16u : OOB;
    }
    uint4 ra[2][NA];
    auto gload = [&](int ks, auto slot) {
        constexpr int S = decltype(slot)::value;
        const bool in = ks < nks;
        const uint32_t kb = (uint32_t)ks * (DG_KS * 2);
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const uint32_t o = (aoff[i] == OOB || !in) ? OOB : aoff[i] + kb;
            ra[S][i] = (MODE == K3K_MX_GATEUP && i >= NA / 2) ? k3_bload16(rw1, o) : k3_bload16(rw0, o);
        }
    };
    auto lstore = [&](int buf, auto slot) {
        constexpr int S = decltype(slot)::value;
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const int c = tid + 256 * i;
            *reinterpret_cast<uint4 *>(&As[buf][(c >> 3) * DG_LD + (c & 7) * 8]) = ra[S][i];
        }
    };
    /* step ks's activations into stage buffer buf (past the slice: zeros) */
    auto dma_b = [&](int ks, uint16_t *bs) {
        const bool in = ks < nks;
#pragma unroll
        for (int i = 0; i < NDMA; i++) {
            const k3_rsrc r = (NS == 2 && 64 * (wv + 4 * i) >= 9 * BN) ? rxl : rxh;
            k3_dma16(r, &bs[64 * 8 * (wv + 4 * i)], in ? doff[i] : OOB, (uint32_t)ks * (DG_KS * 2));
        }
    };
    /* s_waitcnt operands: vmcnt at most NA (one step's weight loads; every other counter
     * unconstrained), and at most NDMA */
    constexpr int WAIT_NA = (NA & 15) | (7 << 4) | (15 << 8) | ((NA >> 4) << 14);
    constexpr int WAIT_NDMA = (NDMA & 15) | (7 << 4) | (15 << 8) | ((NDMA >> 4) << 14);

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

    using R0 = std::integral_constant<int, 0>;
    using R1 = std::integral_constant<int, 1>;
    /* A step's two 32-column halves have fragment registers of their own (f0, f1), so that
     * each half's LDS reads are in flight under the other half's MFMAs: half 1's reads
     * issue under half 0's MFMAs, and the next step's half 0 reads (after the barrier that
     * publishes its LDS buffer) under half 1's. */
    k3_bf16x8 f0a[4], f0b[NS][NJ], f1a[4], f1b[NS][NJ];
    auto rfrag = [&](int buf, const uint16_t *bs, int kk, k3_bf16x8 (&af)[4], k3_bf16x8 (&bf)[NS][NJ]) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            af[i] = k3_as_bf16x8(*reinterpret_cast<const uint4 *>(&As[buf][(arow[i] + r16) * DG_LD + kk + 8 * g]));
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
            for (int j = 0; j < NJ; j++)
                bf[s][j] = k3_as_bf16x8(*reinterpret_cast<const uint4 *>(
                    &bs[(s * BN + bcol0 + 16 * j + r16) * DG_LD + kk + 8 * g]));
    };
    auto mma = [&](const k3_bf16x8 (&af)[4], const k3_bf16x8 (&bf)[NS][NJ]) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int s = 0; s < NS; s++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[s][j], acc[i][j], 0, 0, 0);
    };
    /* issue order of a half: its MFMAs, each of the first 4 + NS NJ followed by one of the
     * other half's fragment reads */
    constexpr int NRD = 4 + NS * NJ, NMF = 4 * NJ * NS;
    static_assert(NRD <= NMF, "fragment reads interleave with the MFMAs");
    auto pin = [&]() {
#pragma unroll
        for (int i = 0; i < NRD; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);      /* MFMA */
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);      /* DS read */
        }
        __builtin_amdgcn_sched_group_barrier(0x008, NMF - NRD, 0);
    };
    /* step ks: its weight ring slot (ks & 1) is free once it is in LDS, so ks + 2 loads into
     * it; ks is multiplied out of LDS buffer ks & 1 and ks + 1's weights stored into the
     * other. The activations of ks + 1 (DMA issued a step ago, before ks + 2's weight loads)
     * have landed once at most NA loads are outstanding; after the barrier that holds for
     * every wave, every wave is past its reads of buffer ks & 1, and ks + 2's activations
     * go into it. Past the slice the slots and buffers hold zeros, and the fragments read
     * from them go unused. */
    auto step = [&](int ks, auto slot) {
        constexpr int S = decltype(slot)::value;
        const int buf = S;
        uint16_t *const bcur = S ? Bs1 : Bs0, *const bnxt = S ? Bs0 : Bs1;
        gload(ks + 2, slot);
        /* issued here, ahead of the products (the compiler would otherwise sink them below
         * the next LDS store and wait for step ks + 1 with nothing else in flight) */
        __builtin_amdgcn_sched_barrier(0);
        rfrag(buf, bcur, 32, f1a, f1b);
        mma(f0a, f0b);
        pin();
        __builtin_amdgcn_sched_barrier(0);
        lstore(buf ^ 1, std::integral_constant<int, S ^ 1>{});
        __builtin_amdgcn_s_waitcnt(WAIT_NA);
        __syncthreads();
        dma_b(ks + 2, bcur);
        rfrag(buf ^ 1, bnxt, 0, f0a, f0b);
        mma(f1a, f1b);
        pin();
        __builtin_amdgcn_sched_barrier(0);
    };
    gload(0, R0{});
    gload(1, R1{});
    dma_b(0, Bs0);
    dma_b(1, Bs1);
    lstore(0, R0{});
    __builtin_amdgcn_s_waitcnt(WAIT_NDMA);         /* all but step 1's activations */
    __syncthreads();
    rfrag(0, Bs0, 0, f0a, f0b);
    /* whole pairs in the loop, so that no load or store sits under a branch there */
    int ks = 0;
    for (; ks + 1 < nks; ks += 2) {
        step(ks, R0{});
        step(ks + 1, R1{});
    }
    if (ks < nks) step(ks, R0{});
    /* the last DMAs (zeros past the slice) land before the workgroup's LDS is released */
    __builtin_amdgcn_s_waitcnt(0);

    /* epilogue: lane holds token column r16 and rows 4g..4g+3 of each 16 x 16 tile */
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int t = tok0 + bcol0 + 16 * j + r16;
        if (t >= a.T) continue;
        if (a.nsl > 1) {
            /* this slice's sums, in order of the part columns */
            float *p = a.part + ((size_t)sl * a.T + t) * a.ncol;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int lr = arow[i] + 4 * g;          /* row inside the tile */
                const int col = MODE == K3K_MX_GATEUP
                                    ? (lr < DG_BM / 2 ? row0 + lr : a.R + row0 + lr - DG_BM / 2)
                                    : row0 + lr;
                const int rr = MODE == K3K_MX_GATEUP ? (lr < DG_BM / 2 ? row0 + lr : row0 + lr - DG_BM / 2) : col;
                if (rr + 3 < a.R)
                    *reinterpret_cast<float4 *>(p + col) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
                else
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (rr + e < a.R) p[col + e] = acc[i][j][e];
            }
            continue;
        }
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

/* The slices' sums added in slice order, then the GEMM's finish: GATEUP applies the
 * activation to (gate, up) and writes its bf16 term(s); PLAIN writes or accumulates y. One
 * thread per (token, 4 consecutive rows); R % 4 == 0, y and ldy 16-byte aligned. Every
 * slice's loads are issued before the first sum. */
template <int MODE, int NSL>
__global__ __launch_bounds__(256) void dense_finish_kernel(DgArgs a)
{
    const int n4 = a.R >> 2;
    const size_t total = (size_t)a.T * n4;
    const size_t slice = (size_t)a.T * a.ncol;
    for (size_t k = (size_t)blockIdx.x * blockDim.x + threadIdx.x; k < total; k += (size_t)gridDim.x * blockDim.x) {
        const int t = (int)(k / n4), r = (int)(k % n4) * 4;
        const float *p = a.part + (size_t)t * a.ncol + r;
        k3_f32x4 gs[NSL], us[MODE == K3K_MX_GATEUP ? NSL : 1];
#pragma unroll
        for (int q = 0; q < NSL; q++) {
            gs[q] = __builtin_nontemporal_load(reinterpret_cast<const k3_f32x4 *>(p + q * slice));
            if (MODE == K3K_MX_GATEUP) us[q] = __builtin_nontemporal_load(reinterpret_cast<const k3_f32x4 *>(p + q * slice + a.R));
        }
        k3_f32x4 yv = {0.f, 0.f, 0.f, 0.f};
        float *o = MODE == K3K_MX_GATEUP ? nullptr : a.y + (size_t)t * a.ldy + r;
        if (MODE != K3K_MX_GATEUP && a.accumulate) yv = *reinterpret_cast<const k3_f32x4 *>(o);
        k3_f32x4 s = gs[0], u = MODE == K3K_MX_GATEUP ? us[0] : gs[0];
#pragma unroll
        for (int q = 1; q < NSL; q++) {                /* slice order, one rounding each */
            s += gs[q];
            if (MODE == K3K_MX_GATEUP) u += us[q];
        }
        if (MODE == K3K_MX_GATEUP) {
            const float gv[4] = {s[0], s[1], s[2], s[3]}, uv[4] = {u[0], u[1], u[2], u[3]};
            uint16_t hi[4], lo[4];
#pragma unroll
            for (int e = 0; e < 4; e++) k3_split2(k3_act_pair(gv[e], uv[e], a.act, a.b1, a.b2), hi[e], lo[e]);
            *reinterpret_cast<uint2 *>(a.ahi + (size_t)t * a.R + r) =
                make_uint2(hi[0] | ((uint32_t)hi[1] << 16), hi[2] | ((uint32_t)hi[3] << 16));
            if (a.alo)
                *reinterpret_cast<uint2 *>(a.alo + (size_t)t * a.R + r) =
                    make_uint2(lo[0] | ((uint32_t)lo[1] << 16), lo[2] | ((uint32_t)lo[3] << 16));
        } else {
            if (a.accumulate) s = yv + s;
            *reinterpret_cast<k3_f32x4 *>(o) = s;
        }
    }
}

/* K slices: the fewest that give every CU a workgroup, each slice at least 256 columns (4
 * steps); 1 without a large enough partials buffer or when the output rows are not a
 * multiple of 4. (At 512 tokens, measured, GEMM + slice sums: gate/up 7168 -> 2048, 128
 * tiles, 87 / 47 + 7.5 / 46 + 8.4 / 58 + 13 us at 1 / 2 / 4 / 8 slices; down 2048 -> 7168,
 * 224 tiles, 42 / 30 + 10 / - / 54 + 24 us at 1 / 2 / 8.) */
static int dense_slices(int tiles, int K, int R, int T, int ncol, size_t part_bytes)
{
    if (R % 4) return 1;
    const long want = k3k_cu_count();
    int s = 1;
    while (s < 8 && (long)tiles * s < want && K / DG_KS / (2 * s) >= 4 &&
           (size_t)(2 * s) * T * ncol * 4 <= part_bytes)
        s *= 2;
    return s;
}

template <int MODE, int NS, int BN>
int launch_dense(DgArgs a, size_t part_bytes, hipStream_t st)
{
    const int rows_per_tile = MODE == K3K_MX_GATEUP ? DG_BM / 2 : DG_BM;
    a.ntr = (a.R + rows_per_tile - 1) / rows_per_tile;
    a.ntt = (a.T + BN - 1) / BN;
    const int tiles = a.ntr * a.ntt;
    a.ncol = MODE == K3K_MX_GATEUP ? 2 * a.R : a.R;
    a.nsl = a.part ? dense_slices(tiles, a.K, a.R, a.T, a.ncol, part_bytes) : 1;
    const int items = tiles * a.nsl;
    a.per_xcd = (items + K3_NXCD - 1) / K3_NXCD;
    hipLaunchKernelGGL((dense_gemm_kernel<MODE, NS, BN>), dim3((unsigned)(a.per_xcd * K3_NXCD)), dim3(256),
                       0, st, a);
    K3K_LAUNCH_CHECK("dense gemm launch");
    if (a.nsl > 1) {
        const size_t n = (size_t)a.T * (a.R / 4);
        const size_t blocks = (n + 255) / 256;
        const dim3 grid(blocks < 65536 ? (unsigned)blocks : 65536u);
        if (a.nsl == 2) hipLaunchKernelGGL((dense_finish_kernel<MODE, 2>), grid, dim3(256), 0, st, a);
        else if (a.nsl == 4) hipLaunchKernelGGL((dense_finish_kernel<MODE, 4>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((dense_finish_kernel<MODE, 8>), grid, dim3(256), 0, st, a);
        K3K_LAUNCH_CHECK("dense finish launch");
    }
    return 0;
}

/* Token block: 128 tokens with one activation term, 64 with two (the same registers). */
template <int MODE, int NS>
int dispatch_dense(const DgArgs &a, size_t part_bytes, hipStream_t st)
{
    if constexpr (NS == 1) return launch_dense<MODE, NS, 128>(a, part_bytes, st);
    else return launch_dense<MODE, NS, 64>(a, part_bytes, st);
}

}  // namespace

extern "C" size_t k3k_dense_part_bytes(int R, int T, int K, int gateup)
{
    if (R <= 0 || T <= 0 || K <= 0) return 0;
    return (size_t)8 * T * (gateup ? 2 * (size_t)R : (size_t)R) * 4;
}

extern "C" int k3k_dense_gemm(float *y, int ldy, int accumulate, const uint16_t *W, const uint16_t *xhi,
                              const uint16_t *xlo, int R, int T, int K, float *part, size_t part_bytes,
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
    a.part = ((uintptr_t)part % 16 || ldy % 4 || (uintptr_t)y % 16) ? nullptr : part;
    return xlo ? dispatch_dense<K3K_MX_PLAIN, 2>(a, part_bytes, (hipStream_t)stream)
               : dispatch_dense<K3K_MX_PLAIN, 1>(a, part_bytes, (hipStream_t)stream);
}

extern "C" int k3k_dense_gateup(uint16_t *ahi, uint16_t *alo, const uint16_t *wg, const uint16_t *wu,
                                const uint16_t *xhi, const uint16_t *xlo, int R, int T, int K, int act,
                                float b1, float b2, float *part, size_t part_bytes, void *stream)
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
    a.part = ((uintptr_t)part % 16 || (uintptr_t)ahi % 8 || (alo && (uintptr_t)alo % 8)) ? nullptr : part;
    return xlo ? dispatch_dense<K3K_MX_GATEUP, 2>(a, part_bytes, (hipStream_t)stream)
               : dispatch_dense<K3K_MX_GATEUP, 1>(a, part_bytes, (hipStream_t)stream);
}
