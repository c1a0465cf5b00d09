/*
 * Micro-kernel type gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt (W4A8), variant mfma_gfx950.
 *
 * A is qai8dx: int8 [m, k] row-major with per-row asymmetric quantization (scale_a[m],
 * zero_point_a[m]). B is qsi4cxt: int4 [n, k] stored as [n, k/2] bytes, two nibbles per byte
 * (low nibble = even k), value = nibble - 8, per-channel f32 scale_b[n]. bias f32 [n] and C
 * f32 [m, n] are optional. D is f32 [m, n]. k must be even.
 *
 * Per output (reference tqt_kernel_gemm_i8_i4_4x1vl_rvv.h:77-419):
 *   acc = sum_k a*b - zero_point_a[m] * sum_k b                       (int32)
 *   f = (float)acc; f = f * scale_a[m]; f = f * scale_b[n]; f += C; f += bias   (no FMA)
 *   D = fmin(fmax(f, clamp_min), clamp_max)
 *
 * Drop-in for src/gemm/gemm_i8_i4/gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt/
 * tqt_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_4x1vl_rvv.h:41-87. ldb is counted in int4
 * elements (= k for a dense matrix), as in the reference.
 */
#ifndef TQT_GEMM_1XNBIAS_CLAMP_F32_QAI8DX_QSI4CXT_MFMA_GFX950_H
#define TQT_GEMM_1XNBIAS_CLAMP_F32_QAI8DX_QSI4CXT_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference ..._4x1vl_rvv.h:41 / :43 */
size_t tqt_get_m_step_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(void);
size_t tqt_get_n_step_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(void);
/* reference ..._4x1vl_rvv.h:46: (m_idx * lda + k_idx) bytes */
size_t tqt_get_a_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(size_t m_idx,
                                                                          size_t k_idx,
                                                                          size_t lda);
/* reference ..._4x1vl_rvv.h:51: n_idx * (ldb / 2) + k_idx / 2 bytes (k_idx even) */
size_t tqt_get_b_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(size_t n_idx,
                                                                          size_t k_idx,
                                                                          size_t ldb);
/* reference ..._4x1vl_rvv.h:54: (m_idx * ldc + n_idx) * 4 bytes */
size_t tqt_get_c_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(size_t m_idx,
                                                                          size_t n_idx,
                                                                          size_t ldc);
/* reference ..._4x1vl_rvv.h:57: n_idx * 4 bytes */
size_t tqt_get_bias_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(size_t n_idx);
/* reference ..._4x1vl_rvv.h:59: (m_idx * ldd + n_idx) * 4 bytes */
size_t tqt_get_d_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(size_t m_idx,
                                                                          size_t n_idx,
                                                                          size_t ldd);
/* reference ..._4x1vl_rvv.h:62: m * n * 4 bytes */
size_t tqt_get_d_size_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(size_t m, size_t n);

/* reference ..._4x1vl_rvv.h:84-87 */
void tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    float clamp_min, float clamp_max, const struct tqt_qai8dx_qsi4cx_params *params);

/* Stream-ordered form (no counterpart in the reference). */
void tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    float clamp_min, float clamp_max, const struct tqt_qai8dx_qsi4cx_params *params,
    void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
