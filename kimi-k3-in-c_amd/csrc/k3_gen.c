/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_gen.c -- the synthetic-input generator shared by the benchmark, the tests and the
 * fixture script. The reference has no Gaussian or Zipf generator (its bench uses a
 * xorshift32 uniform, benchmarks/bench_kernels.c:54-89), so this defines one.
 *
 * Counter-based: element i of stream `seed` is a function of (seed, i) alone, so any
 * slice of any tensor (one expert of a 384-expert bank, say) can be regenerated on its
 * own, in parallel, and bit-identically on every host running the same libm.
 *
 *   u64(seed, i)   splitmix64's output for state seed + (i+1)*0x9E3779B97F4A7C15
 *                  (Steele, Lea, Flood, "Fast splittable pseudorandom number generators",
 *                  OOPSLA 2014; the finaliser constants of Vigna's splitmix64.c)
 *   bytes          byte i = byte (i mod 8) of u64(seed, i / 8), little-endian
 *   E8M0 in [lo,hi] lo + floor(hi32(u64) * (hi-lo+1) / 2^32)
 *   normal         Box-Muller in double: u1 = (top53(u64(seed,2k)) + 1) 2^-53,
 *                  u2 = top53(u64(seed,2k+1)) 2^-53, r = sqrt(-2 ln u1),
 *                  z(2k) = r cos(2 pi u2), z(2k+1) = r sin(2 pi u2);
 *                  value = (float)(mean + sigma z)
 */
#include "k3_gen.h"

#include <math.h>
#include <string.h>

static inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t k3g_u64(uint64_t seed, uint64_t i)
{
    return mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ull);
}

void k3g_bytes(uint8_t *p, size_t n, uint64_t seed)
{
    const size_t words = n / 8;
#pragma omp parallel for schedule(static) if (n > (1u << 20))
    for (size_t w = 0; w < words; w++) {
        const uint64_t v = k3g_u64(seed, w);
        memcpy(p + 8 * w, &v, 8);   /* little-endian host: byte k = bits 8k..8k+7 */
    }
    if (n % 8) {
        const uint64_t v = k3g_u64(seed, words);
        for (size_t k = 0; k < n % 8; k++) p[8 * words + k] = (uint8_t)(v >> (8 * k));
    }
}

void k3g_e8m0(uint8_t *p, size_t n, uint64_t seed, int lo, int hi)
{
    const uint64_t span = (uint64_t)(hi - lo + 1);
#pragma omp parallel for schedule(static) if (n > (1u << 20))
    for (size_t i = 0; i < n; i++)
        p[i] = (uint8_t)(lo + (int)(((k3g_u64(seed, i) >> 32) * span) >> 32));
}

void k3g_normal(float *p, size_t n, uint64_t seed, double mean, double sigma)
{
    const size_t pairs = (n + 1) / 2;
#pragma omp parallel for schedule(static) if (n > (1u << 16))
    for (size_t k = 0; k < pairs; k++) {
        const double u1 = (double)((k3g_u64(seed, 2 * k) >> 11) + 1) * 0x1p-53;
        const double u2 = (double)(k3g_u64(seed, 2 * k + 1) >> 11) * 0x1p-53;
        const double r = sqrt(-2.0 * log(u1));
        const double th = 6.283185307179586 * u2;
        p[2 * k] = (float)(mean + sigma * (r * cos(th)));
        if (2 * k + 1 < n) p[2 * k + 1] = (float)(mean + sigma * (r * sin(th)));
    }
}

void k3g_bf16_normal(uint16_t *p, size_t n, uint64_t seed, double mean, double sigma)
{
    const size_t pairs = (n + 1) / 2;
#pragma omp parallel for schedule(static) if (n > (1u << 16))
    for (size_t k = 0; k < pairs; k++) {
        const double u1 = (double)((k3g_u64(seed, 2 * k) >> 11) + 1) * 0x1p-53;
        const double u2 = (double)(k3g_u64(seed, 2 * k + 1) >> 11) * 0x1p-53;
        const double r = sqrt(-2.0 * log(u1));
        const double th = 6.283185307179586 * u2;
        for (int h = 0; h < 2 && 2 * k + h < n; h++) {
            const float f = (float)(mean + sigma * (r * (h ? sin(th) : cos(th))));
            uint32_t u;
            memcpy(&u, &f, 4);
            /* round to nearest even; the values are finite by construction */
            u += 0x7FFFu + ((u >> 16) & 1u);
            p[2 * k + h] = (uint16_t)(u >> 16);
        }
    }
}

/* Stream ids of one expert's six tensors: p1 s1 p3 s3 p2 s2 (gate, up, down). */
uint64_t k3g_expert_seed(uint64_t seed, int expert, int tensor)
{
    return k3g_u64(seed, (uint64_t)expert * 8u + (uint64_t)tensor);
}

void k3g_mxfp4_expert(uint8_t *p1, uint8_t *s1, uint8_t *p3, uint8_t *s3, uint8_t *p2,
                      uint8_t *s2, int hidden, int inter, uint64_t seed, int expert,
                      int e8m0_lo, int e8m0_hi)
{
    const size_t pk = (size_t)hidden * inter / 2, sc = (size_t)hidden * inter / 32;
    k3g_bytes(p1, pk, k3g_expert_seed(seed, expert, 0));
    k3g_e8m0(s1, sc, k3g_expert_seed(seed, expert, 1), e8m0_lo, e8m0_hi);
    k3g_bytes(p3, pk, k3g_expert_seed(seed, expert, 2));
    k3g_e8m0(s3, sc, k3g_expert_seed(seed, expert, 3), e8m0_lo, e8m0_hi);
    k3g_bytes(p2, pk, k3g_expert_seed(seed, expert, 4));
    k3g_e8m0(s2, sc, k3g_expert_seed(seed, expert, 5), e8m0_lo, e8m0_hi);
}
