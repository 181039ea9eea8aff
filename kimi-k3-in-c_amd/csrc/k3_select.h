/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_select.h -- the router's device pieces shared by k3_route.hip (the router kernels)
 * and k3_mx.hip (the decode gate/up kernel, which selects a few tokens' experts itself):
 * the host-libm-exact score, the reference's sequential logit chain, and the top-k
 * selection with its recompute rounds.
 */
#ifndef K3_SELECT_H
#define K3_SELECT_H

#include "k3_common.h"
#include "k3_expf.h"

namespace {

struct ExcTable {
    const uint32_t *pairs;      /* sorted (key bits of v, libm expf(v) bits) */
    const uint32_t *index;      /* index[b] = first pair with (key >> 12) - base >= b */
    const uint32_t *bits;       /* membership bitmap over |key| in [mmin, mmax], per sign */
    uint32_t kmin, kmax, base, mmin, mwords;
    int n;
};

/* The word of the exception bitmap that holds v = -logit's magnitude, or 0 outside the
 * bitmap's range. A buffer load with no branch around it (an offset past the end reads 0),
 * so that a caller can issue it early and consume it after other work. */
__device__ __forceinline__ uint32_t exc_word(float logit, const ExcTable &x)
{
    const uint32_t key = __float_as_uint(-logit), mag = key & 0x7fffffffu;
    const uint32_t bi = mag - x.mmin, w = bi >> 5;
    const bool in = x.n > 0 && mag >= x.mmin && w < x.mwords;
    const k3_rsrc r = k3_make_rsrc(x.bits, x.n > 0 ? 8u * x.mwords : 0u);
    return k3_bload4(r, in ? ((key >> 31) * x.mwords + w) * 4u : 0xfffffff0u);
}

/* libm-exact score 1/(1+expf(v)), v = -logit: the deterministic correctly rounded
 * candidate, replaced where the host libm's expf differs (exception table built at build
 * time from that libm). The bitmap word (exc_word) decides membership; only members search
 * their bucket (key >> 12, at most 17 pairs). */
__device__ __forceinline__ float router_score_w(float logit, uint32_t word, const ExcTable &x)
{
    const float v = -logit;
    float E = k3_expf_det(v);
    const uint32_t key = __float_as_uint(v);
    const uint32_t mag = key & 0x7fffffffu;
    if (x.n > 0 && mag >= x.mmin && ((word >> ((mag - x.mmin) & 31)) & 1u)) {
        const uint32_t bkt = (key >> 12) - x.base;
        int lo = (int)x.index[bkt], hi = (int)x.index[bkt + 1];
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (x.pairs[2 * mid] < key) lo = mid + 1;
            else hi = mid;
        }
        if (lo < x.n && x.pairs[2 * lo] == key) E = __uint_as_float(x.pairs[2 * lo + 1]);
    }
    return 1.0f / (1.0f + E);
}

__device__ __forceinline__ float router_score(float logit, const ExcTable &x)
{
    return router_score_w(logit, exc_word(logit, x), x);
}

/* The reference's own chain for one logit (the fallback of the certification), computed
 * by a whole workgroup: acc = 0; for k ascending: acc = fma(w_k, x_k, acc). The chain is one dependent fp64 add per column, so one thread runs it
 * (thread 0), adding the exact products w_k x_k (a product of two floats is exact in
 * fp64, so acc + w_k x_k rounds like fma(w_k, x_k, acc)) that the other waves write into
 * an LDS ring of two RF_BLK-column blocks one block ahead. Every thread of the workgroup
 * calls it; the result is valid in thread 0. */
constexpr int RF_BLK = 512, RF_LIST = 64;

__device__ double chain_block(double (*ring)[RF_BLK], const float *w, const float *x, int hidden)
{
    const int tid = threadIdx.x, nthr = blockDim.x;
    const bool many = nthr > 64;                 /* producers: waves 1.., else every lane */
    const int p0 = many ? tid - 64 : tid, np = many ? nthr - 64 : nthr;
    const int nb = (hidden + RF_BLK - 1) / RF_BLK;
    auto produce = [&](int b) {
        if (p0 < 0) return;
        double *dst = ring[b & 1];
        for (int i = p0; i < RF_BLK; i += np) {
            const int k = b * RF_BLK + i;
            dst[i] = k < hidden ? (double)w[k] * (double)x[k] : 0.0;
        }
    };
    double acc = 0.0;
    produce(0);
    __syncthreads();
    for (int b = 0; b < nb; b++) {
        if (b + 1 < nb) produce(b + 1);
        if (tid == 0) {
            const double2 *p2 = reinterpret_cast<const double2 *>(ring[b & 1]);
            const int n = min(RF_BLK, hidden - b * RF_BLK);
            int i = 0;
            for (; i + 8 <= n; i += 8) {
                const double2 a0 = p2[i / 2], a1 = p2[i / 2 + 1], a2 = p2[i / 2 + 2], a3 = p2[i / 2 + 3];
                acc += a0.x;
                acc += a0.y;
                acc += a1.x;
                acc += a1.y;
                acc += a2.x;
                acc += a2.y;
                acc += a3.x;
                acc += a3.y;
            }
            for (; i < n; i++) acc += ring[b & 1][i];
        }
        __syncthreads();
    }
    return acc;
}

/* unsigned order of a non-NaN float that matches its numeric order (-0 as +0) */
__device__ __forceinline__ uint32_t choice_order(float v)
{
    const uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

/* 32-bit max / min of the wave by DPP, the same in every lane: pairs, quads (quad_perm),
 * 8 (row half mirror), 16 (row mirror), then rows 0-1 and 2-3 (row_bcast15 into rows 1,
 * 3) and rows 0-3 (row_bcast31 into rows 2, 3), so lane 63 holds the result. */
/* (rows outside RM read the identity of the operation, so each step is one DPP max/min) */
template <int CTRL, int RM, uint32_t ID>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp((int)ID, (int)v, CTRL, RM, 0xf, false);
}

template <bool MAX>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v)
{
    constexpr uint32_t ID = MAX ? 0u : 0xffffffffu;
    auto op = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
    v = op(v, dpp_u32<0xB1, 0xf, ID>(v));      /* quad_perm [1,0,3,2] */
    v = op(v, dpp_u32<0x4E, 0xf, ID>(v));      /* quad_perm [2,3,0,1] */
    v = op(v, dpp_u32<0x141, 0xf, ID>(v));     /* row_half_mirror */
    v = op(v, dpp_u32<0x140, 0xf, ID>(v));     /* row_mirror */
    v = op(v, dpp_u32<0x142, 0xa, ID>(v));     /* row_bcast15 */
    v = op(v, dpp_u32<0x143, 0xc, ID>(v));     /* row_bcast31 */
    return __builtin_amdgcn_readlane(v, 63);
}

/* Selection key (order-preserving bits of the choice) << 32 | ~expert: the largest key is
 * the largest choice, then the lowest expert. */
/* The wave's largest key, in every lane: the largest high word (choice), then -- only when
 * several lanes hold it -- the largest low word among them; otherwise the one lane holding
 * the largest choice gives its key. */
__device__ __forceinline__ uint64_t wave_max_key_fast(uint64_t k)
{
    const uint32_t hi = wave_reduce_u32<true>((uint32_t)(k >> 32));
    const uint64_t at = __ballot((uint32_t)(k >> 32) == hi);
    uint32_t lo;
    if (__popcll(at) == 1)
        lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, (int)(__ffsll((unsigned long long)at) - 1));
    else
        lo = wave_reduce_u32<true>((uint32_t)(k >> 32) == hi ? (uint32_t)k : 0u);
    return ((uint64_t)hi << 32) | lo;
}

/* The choice a selection key carries (choice_order inverted; -0 comes back as +0). */
__device__ __forceinline__ float key_choice(uint64_t key)
{
    const uint32_t h = (uint32_t)(key >> 32);
    return __uint_as_float((h & 0x80000000u) ? (h & 0x7fffffffu) : ~h);
}

/* The workgroup's scored experts of one token (written before select_rounds; updated by
 * its recomputes) and the recompute scratch. */
template <int SW>
struct SelSmem {
    float c[64 * SW], cmax[64 * SW], sc[64 * SW];   /* choice, its upper end, score */
    int unc[64 * SW];                              /* 1: logit uncertified */
    int nlist;
    int list[RF_LIST];
    double res[RF_LIST];
    __attribute__((aligned(16))) double prod[2][RF_BLK];
    uint64_t cand[256];                            /* two-level selection: the waves' keys */
    uint64_t last;                                 /* its k-th key and count */
    int nsel;
    int wcnt[16];                                  /* listed experts per wave */
};

/* The reference's rule topk times (largest choice, lowest index among equals, strictly
 * above -inf, none left: idx 0, weight 0; k3_ops.c:459-467) over the scored experts in sm.
 * Keys are unique (the expert's index in the low word), so the selection is the topk
 * largest keys in order, however they are found:
 *  - two levels, when the ng = ceil(n_experts / 64) groups of 64 experts fit the
 *    workgroup's waves and ng * topk <= 256: wave g takes the topk largest keys of group g
 *    (one key per lane, each extraction one wave maximum, wave_max_key_fast), then wave 0
 *    the topk largest of those ng * topk candidates (one to four per lane: a lane holds
 *    candidates l + 64 i and the largest of them, and after each pick the lane that held
 *    it takes its next);
 *  - else wave 0 alone: lane l holds the keys of experts l + 64 i (SW of them) and the
 *    largest of its keys; after each extraction the lane that held it drops the key and
 *    takes its next largest.
 * Lane j of wave 0 keeps the j-th selected key. Uncertified logits that matter (selected,
 * i.e. a key at least the last selected one, or able to reach the selection) are listed in
 * expert order by ballots, recomputed by the whole workgroup with the reference's chain
 * (chain_block) and rescored, and the selection is redone until none is left. Called by
 * every thread after sm is written and a barrier; returns the selected key in lanes
 * 0..topk-1 of wave 0 (0: none), and the number of recomputes in nre. */
template <int SW>
__device__ uint64_t select_rounds(SelSmem<SW> &sm, const float *x, const float *W,
                                  const float *bias, int hidden, int n_experts, int topk,
                                  const ExcTable &exc, int &nre)
{
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, nw = (int)blockDim.x >> 6;
    const int ng = (n_experts + 63) >> 6;
    const bool two = ng <= nw && ng <= SW && ng * topk <= 256;
    const int nc = ng * topk;                       /* level-2 candidates, one to four per lane */
    auto key_of = [&](int e) {
        const float c = sm.c[e];
        return (e < n_experts && c > -INFINITY) ? ((uint64_t)choice_order(c) << 32) | (uint64_t)(0xffffffffu - (uint32_t)e)
                                                : 0ull;
    };
    nre = 0;
    uint64_t mysel = 0ull;
    for (int round = 0; round <= n_experts; round++) {
        if (two) {
            /* level 1: group wv's topk largest keys (0 once none is left) */
            if (wv < ng) {
                uint64_t k = key_of(64 * wv + lane);
                for (int j = 0; j < topk; j++) {
                    const uint64_t m = wave_max_key_fast(k);
                    if (lane == 0) sm.cand[wv * topk + j] = m;
                    if (k == m) k = 0ull;
                }
            }
            __syncthreads();
            /* level 2: the topk largest candidates */
            if (wv == 0 && nc <= 64) {
                uint64_t k = lane < nc ? sm.cand[lane] : 0ull;
                int nsel = 0;
                uint64_t last = 0ull;
                mysel = 0ull;
                for (int j = 0; j < topk; j++) {
                    const uint64_t m = wave_max_key_fast(k);
                    if (m == 0ull) break;           /* no finite choice left */
                    nsel++;
                    last = m;
                    if (lane == j) mysel = m;
                    if (k == m) k = 0ull;
                }
                if (lane == 0) {
                    sm.nsel = nsel;
                    sm.last = last;
                }
            } else if (wv == 0) {
                /* more than 64 candidates: lane l holds candidates l + 64 i and the largest of
                 * them; after each pick the lane that held it drops it and takes its next */
                uint64_t ck[4], head = 0ull;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    ck[i] = lane + 64 * i < nc ? sm.cand[lane + 64 * i] : 0ull;
                    head = head > ck[i] ? head : ck[i];
                }
                int nsel = 0;
                uint64_t last = 0ull;
                mysel = 0ull;
                for (int j = 0; j < topk; j++) {
                    const uint64_t m = wave_max_key_fast(head);
                    if (m == 0ull) break;           /* no finite choice left */
                    nsel++;
                    last = m;
                    if (lane == j) mysel = m;
                    if (head == m) {
                        uint64_t h2 = 0ull;
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            if (ck[i] == m) ck[i] = 0ull;
                            h2 = h2 > ck[i] ? h2 : ck[i];
                        }
                        head = h2;
                    }
                }
                if (lane == 0) {
                    sm.nsel = nsel;
                    sm.last = last;
                }
            }
            __syncthreads();
            /* every wave lists its group's uncertified logits that matter, in expert order */
            const int nsel = sm.nsel;
            const uint64_t last = sm.last;
            const float ckth = nsel > 0 ? key_choice(last) : -INFINITY;
            bool need = false;
            if (wv < ng) {
                const int e = 64 * wv + lane;
                need = e < n_experts && sm.unc[e] && (nsel < topk || key_of(e) >= last || sm.cmax[e] >= ckth);
            }
            const uint64_t bm = __ballot(need);
            if (lane == 0) sm.wcnt[wv] = __popcll(bm);
            __syncthreads();
            int base = 0, total = 0;
            for (int w = 0; w < nw; w++) {
                const int cw = sm.wcnt[w];
                if (w < wv) base += cw;
                total += cw;
            }
            const int slot = base + __popcll(bm & ((1ull << lane) - 1ull));
            if (need && slot < RF_LIST) sm.list[slot] = 64 * wv + lane;
            if (tid == 0) sm.nlist = min(total, RF_LIST);
        } else if (wv == 0) {
            uint64_t key[SW];
            uint64_t head = 0ull;
#pragma unroll
            for (int i = 0; i < SW; i++) {
                const int e = lane + 64 * i;
                const float c = sm.c[e];
                key[i] = (e < n_experts && c > -INFINITY)
                             ? ((uint64_t)choice_order(c) << 32) | (uint64_t)(0xffffffffu - (uint32_t)e)
                             : 0ull;
                head = head > key[i] ? head : key[i];
            }
            uint32_t taken = 0u;                    /* bit i: key i was selected */
            int nsel = 0;
            uint64_t last = 0ull;
            mysel = 0ull;
            for (int j = 0; j < topk; j++) {
                const uint64_t m = wave_max_key_fast(head);
                if (m == 0ull) break;               /* no finite choice left */
                nsel++;
                last = m;
                if (lane == j) mysel = m;
                if (head == m) {
                    uint64_t h2 = 0ull;
#pragma unroll
                    for (int i = 0; i < SW; i++) {
                        if (key[i] == m) {
                            key[i] = 0ull;
                            taken |= 1u << i;
                        }
                        h2 = h2 > key[i] ? h2 : key[i];
                    }
                    head = h2;
                }
            }
            const float ckth = nsel > 0 ? key_choice(last) : -INFINITY;
            /* uncertified logits that matter, listed in ballot order (up to RF_LIST; the
             * rest wait for the next round) */
            int base = 0;
#pragma unroll
            for (int i = 0; i < SW; i++) {
                const int e = lane + 64 * i;
                const bool need = e < n_experts && sm.unc[e] &&
                                  (((taken >> i) & 1u) || nsel < topk || sm.cmax[e] >= ckth);
                const uint64_t m = __ballot(need);
                const int slot = base + __popcll(m & ((1ull << lane) - 1ull));
                if (need && slot < RF_LIST) sm.list[slot] = e;
                base += __popcll(m);
            }
            if (lane == 0) sm.nlist = min(base, RF_LIST);
        }
        __syncthreads();
        const int nl = sm.nlist;
        if (nl == 0) break;
        for (int j = 0; j < nl; j++) {
            const double a = chain_block(sm.prod, W + (size_t)sm.list[j] * hidden, x, hidden);
            if (tid == 0) sm.res[j] = a;
        }
        __syncthreads();
        if (tid < nl) {
            const int e = sm.list[tid];
            const float sc = router_score((float)sm.res[tid], exc);
            const float c = sc + (bias ? bias[e] : 0.0f);
            sm.c[e] = c;
            sm.cmax[e] = c;
            sm.sc[e] = sc;
            sm.unc[e] = 0;
        }
        nre += nl;
        __syncthreads();
    }
    return mysel;
}

/* Wave 0, after select_rounds: lane j's expert (-1: none) and its weight -- the unbiased
 * score, renormalised by (float)(1/(sum_j double + 1e-20)) in j order when renorm and
 * topk > 1, times routed_scale (k3_ops.c:469-475); 0 for none. */
template <int SW>
__device__ __forceinline__ void select_weight(const SelSmem<SW> &sm, uint64_t mysel, int topk,
                                              int renorm, float routed_scale, int &id, float &wt)
{
    const int lane = threadIdx.x & 63;
    id = mysel != 0ull ? (int)(0xffffffffu - (uint32_t)mysel) : -1;
    float w = (lane < topk && id >= 0) ? sm.sc[id] : 0.0f;
    if (renorm && topk > 1) {
        double s = 0.0;
        for (int j = 0; j < topk; j++)                      /* j ascending */
            s += (double)__uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(w), j));
        const float inv = (float)(1.0 / (s + 1e-20));
        w = w * inv;
    }
    wt = w * routed_scale;
}

/* The scored record of router_small_kernel for one expert: {score, score of the upper
 * end of its logit's interval, uncertified ? 1 : 0, 0}; choice = score + bias. */
template <int SW>
__device__ __forceinline__ void select_put_record(SelSmem<SW> &sm, int e, float4 pr, float bb)
{
    sm.sc[e] = pr.x;
    sm.c[e] = pr.x + bb;
    const bool unc = pr.z != 0.0f;
    sm.cmax[e] = unc ? pr.y + bb : pr.x + bb;           /* choice is monotone in logit */
    sm.unc[e] = unc ? 1 : 0;
}

}  // namespace

#endif
