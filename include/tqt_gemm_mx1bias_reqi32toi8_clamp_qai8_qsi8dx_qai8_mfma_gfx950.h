/*
 * Micro-kernel type gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8, variant mfma_gfx950.
 *
 * Computes D = clamp(requantize(C + A * B + bias)) with A int8 [m, k] (weights, symmetric,
 * per-row scale_a[m] or one scale when quant_channel_a == 1), B int8 [k, n] row-major
 * (activations, scalar scale_b; zero_point_b folded into the bias by the caller), C int32
 * [m, n] (optional), bias int32 [m] (Mx1: one per row), D int8 [m, n]: per row the multiplier of
 * scale_a[i] * scale_b / scale_d (tqt_quantize_multiplier, shift = -shift - 1), then the
 * requantization and clamp of gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt.
 *
 * Drop-in for src/gemm/gemm_i8_i8/gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8/tqt_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_4x1vl_rvv.h
 * (the line of each declaration is given below). Every tensor pointer is device-
 * accessible; the runs return with their output written; the _async forms (no
 * counterpart in the reference) enqueue on a hipStream_t instead. Params structs and
 * scalars stay on the host.
 */
#ifndef TQT_GEMM_MX1BIAS_REQI32TOI8_CLAMP_QAI8_QSI8DX_QAI8_MFMA_GFX950_H
#define TQT_GEMM_MX1BIAS_REQI32TOI8_CLAMP_QAI8_QSI8DX_QAI8_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference :36 */
size_t tqt_get_m_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(void);
/* reference :43 */
size_t tqt_get_n_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(void);
/* reference :52 */
size_t tqt_get_a_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m_idx, size_t k_idx, size_t lda);
/* reference :63 */
size_t tqt_get_b_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb);
/* reference :74 */
size_t tqt_get_c_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc);
/* reference :83 */
size_t tqt_get_bias_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m_idx);
/* reference :92 */
size_t tqt_get_d_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd);
/* reference :102 */
size_t tqt_get_d_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m, size_t n);
/* reference :129 */
void tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qsi8dx_qai8_params *params);
/* stream-ordered form */
void tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qsi8dx_qai8_params *params,
    void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
