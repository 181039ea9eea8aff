/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_gen.h -- deterministic synthetic inputs (benchmark and tests). No counterpart in
 * the reference, whose bench uses a xorshift32 uniform only
 * (benchmarks/bench_kernels.c:54-89). See k3_gen.c for the exact definition.
 */
#ifndef K3_GEN_H
#define K3_GEN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

uint64_t k3g_u64(uint64_t seed, uint64_t i);
void k3g_bytes(uint8_t *p, size_t n, uint64_t seed);
void k3g_e8m0(uint8_t *p, size_t n, uint64_t seed, int lo, int hi);
void k3g_normal(float *p, size_t n, uint64_t seed, double mean, double sigma);
void k3g_bf16_normal(uint16_t *p, size_t n, uint64_t seed, double mean, double sigma);
uint64_t k3g_expert_seed(uint64_t seed, int expert, int tensor);
/* One expert: gate/up [inter][hidden] and down [hidden][inter] in MXFP4 (group 32), codes
 * uniform bytes, E8M0 uniform in [e8m0_lo, e8m0_hi]. */
void k3g_mxfp4_expert(uint8_t *p1, uint8_t *s1, uint8_t *p3, uint8_t *s3, uint8_t *p2,
                      uint8_t *s2, int hidden, int inter, uint64_t seed, int expert,
                      int e8m0_lo, int e8m0_hi);

#ifdef __cplusplus
}
#endif
#endif
