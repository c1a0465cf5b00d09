/*
 * Micro-kernel type gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt, variant mfma_gfx950.
 *
 * Computes D = clamp(f32 epilogue(A * (B - 8))) exactly as gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt
 * does (zero-point correction, RNE conversion, * scale_a[m], * scale_b[n], + C, + bias, max,
 * min; every step rounded, no fused multiply-add), with C, bias and D in bf16: C and bias are
 * widened exactly to f32, the bf16 clamp bounds are widened to f32, and the result is rounded
 * once to bf16 (nearest even; a NaN is stored as the canonical quiet NaN 0x7fc0), as the
 * reference epilogue tqt_kernel_gemm_i8_i4_4x1vl_rvv.h:428-628 does.
 *
 * Drop-in for src/gemm/gemm_i8_i4/gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt/tqt_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_4x1vl_rvv.h
 * (the line of each declaration is given below). Every tensor pointer is device-
 * accessible; the runs return with their output written; the _async forms (no
 * counterpart in the reference) enqueue on a hipStream_t instead. Params structs and
 * scalars stay on the host.
 */
#ifndef TQT_GEMM_1XNBIAS_CLAMP_BF16_QAI8DX_QSI4CXT_MFMA_GFX950_H
#define TQT_GEMM_1XNBIAS_CLAMP_BF16_QAI8DX_QSI4CXT_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference :41 */
size_t tqt_get_m_step_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950(void);
/* reference :43 */
size_t tqt_get_n_step_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950(void);
/* reference :46 */
size_t tqt_get_a_offset_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950(
    size_t m_idx, size_t k_idx, size_t lda);
/* reference :51 */
size_t tqt_get_b_offset_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb);
/* reference :54 */
size_t tqt_get_c_offset_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc);
/* reference :57 */
size_t tqt_get_bias_offset_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950(size_t n_idx);
/* reference :59 */
size_t tqt_get_d_offset_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd);
/* reference :62 */
size_t tqt_get_d_size_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950(size_t m, size_t n);
/* reference :84 */
void tqt_run_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    bfloat16_t clamp_min, bfloat16_t clamp_max, const struct tqt_qai8dx_qsi4cx_params *params);
/* stream-ordered form */
void tqt_run_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    bfloat16_t clamp_min, bfloat16_t clamp_max, const struct tqt_qai8dx_qsi4cx_params *params,
    void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
