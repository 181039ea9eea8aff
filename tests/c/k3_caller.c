/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_caller.c -- a plain C99 caller of libk3amd.so, compiled against include/k3.h only.
 *
 * It makes the two calls the reference's kernel benchmark makes (benchmarks/
 * bench_kernels.c:102-145 of the reference): k3_matmul_bf16 on the KDA q-projection shape
 * (12288 x 7168) and k3_matmul_mxfp4 on an expert matrix (3072 x 3584, every scale 2^0),
 * with the inputs that benchmark generates (a xorshift32 stream: float values
 * ((s >> 8) / 2^23 - 1) * 0.05, bytes s >> 13, bf16 as the top half of such a float;
 * seeds 12345 / 999 and 777 / 4242), so its outputs can be checked against the reference's
 * own. Each call runs twice: once on host weights (uploaded for the call) and once after
 * k3_dev_register made them resident. Outputs go to the file named by argv[1]:
 * y_bf16[12288], y_bf16_resident[12288], y_mx[3072], y_mx_resident[3072] (fp32).
 */
#define _POSIX_C_SOURCE 199309L
#include "k3.h"

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static unsigned next(unsigned s)
{
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    return s;
}

static float unit(unsigned s) { return ((float)(s >> 8) / 8388608.0f - 1.0f) * 0.05f; }

static double now(void)
{
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec + 1e-9 * t.tv_nsec;
}

int main(int argc, char **argv)
{
    if (argc < 2) {
        fprintf(stderr, "usage: %s OUT.bin\n", argv[0]);
        return 2;
    }
    FILE *f = fopen(argv[1], "wb");
    if (!f) return 2;

    /* bf16 GEMV, 7168 -> 12288 */
    const int in = 7168, out = 12288;
    uint16_t *W = malloc((size_t)in * out * sizeof *W);
    float *x = malloc((size_t)in * sizeof *x), *y = malloc((size_t)out * sizeof *y);
    if (!W || !x || !y) return 3;
    unsigned s = 12345u;
    for (size_t i = 0; i < (size_t)in * out; i++) {
        s = next(s);
        const float v = unit(s);
        uint32_t u;
        memcpy(&u, &v, 4);
        W[i] = (uint16_t)(u >> 16);
    }
    s = 999u;
    for (int i = 0; i < in; i++) x[i] = unit(s = next(s));
    k3_matmul_bf16(y, x, W, in, out);
    fwrite(y, sizeof *y, (size_t)out, f);
    if (k3_dev_register(W, (size_t)in * out * sizeof *W) != 0) {
        fprintf(stderr, "k3_dev_register: %s\n", k3_dev_last_error());
        return 4;
    }
    k3_matmul_bf16(y, x, W, in, out);
    double t0 = now();
    for (int r = 0; r < 20; r++) k3_matmul_bf16(y, x, W, in, out);
    printf("k3_matmul_bf16 %d x %d, resident weights: %.1f us per call (host buffers in/out)\n",
           out, in, (now() - t0) / 20 * 1e6);
    fwrite(y, sizeof *y, (size_t)out, f);
    k3_dev_unregister(W);

    /* MXFP4 GEMV, 3584 -> 3072 */
    const int min = 3584, rows = 3072;
    unsigned char *pk = malloc((size_t)rows * min / 2), *sc = malloc((size_t)rows * min / 32);
    float *xm = malloc((size_t)min * sizeof *xm), *ym = malloc((size_t)rows * sizeof *ym);
    if (!pk || !sc || !xm || !ym) return 3;
    s = 777u;
    for (size_t i = 0; i < (size_t)rows * min / 2; i++) pk[i] = (unsigned char)((s = next(s)) >> 13);
    memset(sc, 127, (size_t)rows * min / 32);
    s = 4242u;
    for (int i = 0; i < min; i++) xm[i] = unit(s = next(s));
    k3_matmul_mxfp4(ym, xm, pk, sc, min, rows, K3_MXFP4_GROUP);
    fwrite(ym, sizeof *ym, (size_t)rows, f);
    if (k3_dev_register(pk, (size_t)rows * min / 2) || k3_dev_register(sc, (size_t)rows * min / 32)) {
        fprintf(stderr, "k3_dev_register: %s\n", k3_dev_last_error());
        return 4;
    }
    k3_matmul_mxfp4(ym, xm, pk, sc, min, rows, K3_MXFP4_GROUP);
    t0 = now();
    for (int r = 0; r < 20; r++) k3_matmul_mxfp4(ym, xm, pk, sc, min, rows, K3_MXFP4_GROUP);
    printf("k3_matmul_mxfp4 %d x %d, resident weights: %.1f us per call (host buffers in/out)\n",
           rows, min, (now() - t0) / 20 * 1e6);
    fwrite(ym, sizeof *ym, (size_t)rows, f);
    k3_dev_unregister(pk);
    k3_dev_unregister(sc);
    printf("k3_expert_drops = %ld\n", k3_expert_drops);
    fclose(f);
    free(W); free(x); free(y); free(pk); free(sc); free(xm); free(ym);
    return 0;
}
