/*
 * Micro-kernel type gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt, variant mfma_gfx950.
 *
 * Computes D = clamp(requantize(C + A * B^T + bias)) with A int8 [m, k] row-major, B int8
 * [n, k] row-major ("t": the transposed weight), bias int32 [n] (1xN broadcast, optional),
 * C int32 [m, n] (optional) and D int8 [m, n].
 *
 * Requantization per column j (reference tqt_kernel_gemm_i8_i8_4x1vl_rvv.h:334-408 and
 * tqt_utils_i8_i8.h:16-132):
 *   (mult_j, e_j) = quantize_multiplier((double)scale_a * (double)scale_b[q(j)] / (double)scale_d)
 *   shift_j = -e_j - 1,  q(j) = quant_channel_b == 1 ? 0 : j
 *   y = floor((int64)acc * mult_j / 2^32); y >>= (shift_j & 31); y += zero_point_d (int32 wrap)
 *   D = min(max(saturate_int8(y), clamp_min), clamp_max)
 * zero_point_a is not read (callers fold it into bias).
 *
 * Drop-in for src/gemm/gemm_i8_i8/gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt/
 * tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_4x1vl_rvv.h:36-132. params->scale_b
 * must be device-accessible; the multipliers are derived on the device with the same double
 * arithmetic, so nothing is allocated and no device-to-host copy happens.
 */
#ifndef TQT_GEMM_1XNBIAS_REQI32TOI8_CLAMP_QAI8_QAI8_QSI8CXT_MFMA_GFX950_H
#define TQT_GEMM_1XNBIAS_REQI32TOI8_CLAMP_QAI8_QAI8_QSI8CXT_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference ..._4x1vl_rvv.h:36 / :43 */
size_t tqt_get_m_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(void);
size_t tqt_get_n_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(void);
/* reference ..._4x1vl_rvv.h:52: (m_idx * lda + k_idx) bytes */
size_t tqt_get_a_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t m_idx,
                                                                                    size_t k_idx,
                                                                                    size_t lda);
/* reference ..._4x1vl_rvv.h:63: (n_idx * ldb + k_idx) bytes */
size_t tqt_get_b_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t n_idx,
                                                                                    size_t k_idx,
                                                                                    size_t ldb);
/* reference ..._4x1vl_rvv.h:74: (m_idx * ldc + n_idx) * 4 bytes */
size_t tqt_get_c_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t m_idx,
                                                                                    size_t n_idx,
                                                                                    size_t ldc);
/* reference ..._4x1vl_rvv.h:83: n_idx * 4 bytes */
size_t tqt_get_bias_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t n_idx);
/* reference ..._4x1vl_rvv.h:92: (m_idx * ldd + n_idx) bytes */
size_t tqt_get_d_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t m_idx,
                                                                                    size_t n_idx,
                                                                                    size_t ldd);
/* reference ..._4x1vl_rvv.h:102: m * n bytes */
size_t tqt_get_d_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t m,
                                                                                  size_t n);

/* reference ..._4x1vl_rvv.h:129-132 */
void tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qai8_qsi8cx_params *params);

/* Stream-ordered form (no counterpart in the reference): enqueues on `stream` (hipStream_t)
 * and returns without waiting. */
void tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qai8_qsi8cx_params *params,
    void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
