/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_blas.hip -- the one plain library GEMM of the library: the dense bf16 shared expert's
 * products, y[t][r] = beta * y[t][r] + sum_k W[r][k] * x[t][k] (W bf16 [R][K], x bf16 [T][K],
 * fp32 accumulation and output), through rocBLAS gemm_ex. Host code only.
 *
 * One rocBLAS handle per process, created on first use; its stream is set per call and the
 * two are held together under a mutex, so calls from several threads serialise here.
 * Atomics are disallowed on the handle, so results do not depend on the run.
 */
#include "k3_common.h"
#include "k3k.h"

#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <mutex>

namespace {
std::mutex g_blas_mu;
rocblas_handle g_blas = nullptr;
}  // namespace

extern "C" int k3k_gemm_bf16_nt(float *y, int ldy, const uint16_t *W, const uint16_t *x, int R,
                                int T, int K, float beta, void *stream)
{
    if (R <= 0 || T <= 0) return 0;
    if (K <= 0 || ldy < R) return k3k_fail("gemm_bf16: shape", hipErrorInvalidValue);
    std::lock_guard<std::mutex> lock(g_blas_mu);
    if (!g_blas) {
        if (rocblas_create_handle(&g_blas) != rocblas_status_success) {
            g_blas = nullptr;
            return k3k_fail("gemm_bf16: rocblas_create_handle", hipErrorNotInitialized);
        }
        rocblas_set_atomics_mode(g_blas, rocblas_atomics_not_allowed);
    }
    if (rocblas_set_stream(g_blas, (hipStream_t)stream) != rocblas_status_success)
        return k3k_fail("gemm_bf16: rocblas_set_stream", hipErrorInvalidValue);
    const float alpha = 1.0f;
    /* column-major view: y (R x T, ld ldy) = W^T (W: K x R, ld K) * x (K x T, ld K) */
    const rocblas_status s =
        rocblas_gemm_ex(g_blas, rocblas_operation_transpose, rocblas_operation_none, R, T, K, &alpha, W,
                        rocblas_datatype_bf16_r, K, x, rocblas_datatype_bf16_r, K, &beta, y,
                        rocblas_datatype_f32_r, ldy, y, rocblas_datatype_f32_r, ldy,
                        rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
    if (s != rocblas_status_success) return k3k_fail("gemm_bf16: rocblas_gemm_ex", hipErrorLaunchFailure);
    return 0;
}
