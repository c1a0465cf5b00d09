/*
 * Micro-kernel type gemm_1xnbias_clamp_f32_f16_qsi4c2t, variant mfma_gfx950.
 *
 * Computes D = clamp(C + A * dequant(B) + bias) with A f16 [m, k], B int4 [n, k/2] bytes
 * (nibble 2j = k 2j, value q - 8), block scales scale_b [n, ldsb] f16 (one per bl k), and C,
 * bias, the clamp bounds and D in f32. The result is the f32 value of the reference test's
 * oracle for this type, reference_gemm_quantized_weight_mixed<float16_t, float>
 * (test/common/reference_gemm.cpp:132-179): products exact in f32, f32 accumulation, C, bias
 * and clamp in f32, no rounding to f16 (the RVV kernel instead accumulates in f16, which its
 * test accepts within 1.0).
 *
 * Drop-in for src/gemm/gemm_f16_i4/gemm_1xnbias_clamp_f32_f16_qsi4c2t/tqt_gemm_1xnbias_clamp_f32_f16_qsi4c2t_8x2vl_rvv.h
 * (the line of each declaration is given below). Every tensor pointer is device-
 * accessible; the runs return with their output written; the _async forms (no
 * counterpart in the reference) enqueue on a hipStream_t instead. Params structs and
 * scalars stay on the host.
 */
#ifndef TQT_GEMM_1XNBIAS_CLAMP_F32_F16_QSI4C2T_MFMA_GFX950_H
#define TQT_GEMM_1XNBIAS_CLAMP_F32_F16_QSI4C2T_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference :26 */
size_t tqt_get_m_step_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(void);
/* reference :28 */
size_t tqt_get_n_step_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(void);
/* reference :31 */
size_t tqt_get_a_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(
    size_t m_idx, size_t k_idx, size_t lda, size_t bl);
/* reference :36 */
size_t tqt_get_b_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb, size_t bl);
/* reference :40 */
size_t tqt_get_scale_b_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(
    size_t n_idx, size_t b_idx, size_t ldsb);
/* reference :44 */
size_t tqt_get_c_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc);
/* reference :47 */
size_t tqt_get_bias_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(size_t n_idx);
/* reference :49 */
size_t tqt_get_d_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd);
/* reference :52 */
size_t tqt_get_d_size_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(size_t m, size_t n);
/* reference :77 */
void tqt_run_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(
    size_t m, size_t n, size_t k, size_t bl, const void *A, size_t lda, size_t k_idx_a,
    const void *B, size_t ldb, size_t k_idx_b, const void *scale_b, size_t ldsb, const void *C,
    size_t ldc, void *D, size_t ldd, const void *bias, float clamp_min, float clamp_max);
/* stream-ordered form */
void tqt_run_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950_async(
    size_t m, size_t n, size_t k, size_t bl, const void *A, size_t lda, size_t k_idx_a,
    const void *B, size_t ldb, size_t k_idx_b, const void *scale_b, size_t ldsb, const void *C,
    size_t ldc, void *D, size_t ldd, const void *bias, float clamp_min, float clamp_max,
    void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
