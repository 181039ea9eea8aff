/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_expf.h -- a deterministic expf candidate, bit-identical on the host and the device.
 *
 * The reference router computes score = 1/(1 + expf(-logit)) with the host libm expf
 * (src/core/k3_ops.c:451). That expf is not correctly rounded (about 1.7e5 of the 2.2e9
 * floats in [-104, 89] differ from the correctly rounded value on glibc 2.35), so a
 * device that wants the same scores cannot simply be accurate: it must reproduce libm.
 *
 * The approach: this function is evaluated with the same IEEE binary64 operations, in
 * the same order, with no contraction, on both sides, so its result is identical on the
 * host and on gfx950. At build time a host program walks every float in [-104, 89],
 * compares (float)k3_exp_det(x) with libm's expf(x) and records the inputs where the
 * router score 1/(1+E) would differ; the device consults that table. Everything else
 * agrees by construction.
 *
 * Method: Cody-Waite range reduction x = n ln2 + r (ln2 split as in fdlibm's e_exp.c,
 * ln2_hi with its low 21 bits zero), |r| <= ln2/2, exp(r) by its Taylor series to degree
 * 13 (truncation < 5e-18 relative) in Horner form with fused multiply-adds, then an exact
 * scaling by 2^n built from the exponent bits.
 */
#ifndef K3_EXPF_H
#define K3_EXPF_H

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define K3_HD __host__ __device__
#else
#define K3_HD
#include <math.h>
#endif

static K3_HD inline double k3_exp_det(double x)
{
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
    const double inv_ln2 = 0x1.71547652b82fep+0;
    const double ln2_hi = 0x1.62e42fee00000p-1;
    const double ln2_lo = 0x1.a39ef35793c76p-33;
    const double shifter = 0x1.8p52;
    const double t = x * inv_ln2;
    const double u = t + shifter;
    const double n = u - shifter;
    double r = fma(-n, ln2_hi, x);
    r = fma(-n, ln2_lo, r);
    double p = 0x1.6124613a86d09p-33;          /* 1/13! */
    p = fma(p, r, 0x1.1eed8eff8d898p-29);      /* 1/12! */
    p = fma(p, r, 0x1.ae64567f544e4p-26);      /* 1/11! */
    p = fma(p, r, 0x1.27e4fb7789f5cp-22);      /* 1/10! */
    p = fma(p, r, 0x1.71de3a556c734p-19);      /* 1/9!  */
    p = fma(p, r, 0x1.a01a01a01a01ap-16);      /* 1/8!  */
    p = fma(p, r, 0x1.a01a01a01a01ap-13);      /* 1/7!  */
    p = fma(p, r, 0x1.6c16c16c16c17p-10);      /* 1/6!  */
    p = fma(p, r, 0x1.1111111111111p-7);       /* 1/5!  */
    p = fma(p, r, 0x1.5555555555555p-5);       /* 1/4!  */
    p = fma(p, r, 0x1.5555555555555p-3);       /* 1/3!  */
    p = fma(p, r, 0x1.0000000000000p-1);       /* 1/2!  */
    p = fma(p, r, 1.0);
    p = fma(p, r, 1.0);
    const int64_t ni = (int64_t)n;
    const uint64_t bits = (uint64_t)(ni + 1023) << 52;
    double sc;
    memcpy(&sc, &bits, 8);
    return p * sc;
}

/* expf candidate for float inputs in [-104, 89]; outside, the libm results are 0 / inf
 * and are returned directly. */
static K3_HD inline float k3_expf_det(float x)
{
    if (x < -104.0f) return 0.0f;
    if (x > 89.0f) return (float)(1.0 / 0.0);
    return (float)k3_exp_det((double)x);
}

#endif
