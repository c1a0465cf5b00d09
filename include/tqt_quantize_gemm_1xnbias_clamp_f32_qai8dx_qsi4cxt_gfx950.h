/*
 * The fused W4A8 decode step: dynamic per-row qai8dx quantization of f32 activations followed by
 * gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt on them, in one launch.
 *
 * No counterpart in the reference library: it stands for the two calls a decode loop makes, the
 * reference's test-side activation quantization (quantize_a_per_row_asym,
 * test/gemm/test_gemm_i8_i4_rvv.cpp:40-77, here tqt_run_quantize_qai8dx_f32_gfx950) and the
 * W4A8 run (…qai8dx_qsi4cxt_4x1vl_rvv.cpp:157-198, here
 * tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950), and its results are bit-identical
 * to those two calls:
 *   1. A [m, lda] f32 is quantized row by row into A_q [m, lda_q] int8, scale_a [m] and
 *      zero_point_a [m], exactly as tqt_run_quantize_qai8dx_f32_gfx950 writes them;
 *   2. D [m, ldd] = the W4A8 GEMV of A_q against B ([n, ldb / 2] bytes of int4 pairs) with the
 *      params {scale_a, zero_point_a, scale_b}, C, bias and the clamp bounds, as
 *      tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950 computes it with m_idx = n_idx = 0
 *      and k_idx = 0.
 * With m = 1 and k = 2048 or 4096 (16-byte aligned A and B, 4-byte aligned A_q, ldb / 2 a
 * multiple of 16) both run in one kernel: every workgroup quantizes the row while its weight
 * loads are in flight; otherwise the two launches run back to back on the stream.
 *
 * All arrays are device pointers; A_q, scale_a and zero_point_a are outputs. The plain form
 * returns with the outputs written; the _async form enqueues on `stream` (a hipStream_t, NULL =
 * the default stream).
 */
#ifndef TQT_QUANTIZE_GEMM_1XNBIAS_CLAMP_F32_QAI8DX_QSI4CXT_GFX950_H
#define TQT_QUANTIZE_GEMM_1XNBIAS_CLAMP_F32_QAI8DX_QSI4CXT_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

void tqt_run_quantize_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_gfx950(
    size_t m, size_t n, size_t k, const float *A, size_t lda, int8_t *A_q, size_t lda_q,
    float *scale_a, int32_t *zero_point_a, const void *B, size_t ldb, const void *C, size_t ldc,
    void *D, size_t ldd, const void *bias, float clamp_min, float clamp_max,
    const float *scale_b);

void tqt_run_quantize_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_gfx950_async(
    size_t m, size_t n, size_t k, const float *A, size_t lda, int8_t *A_q, size_t lda_q,
    float *scale_a, int32_t *zero_point_a, const void *B, size_t ldb, const void *C, size_t ldc,
    void *D, size_t ldd, const void *bias, float clamp_min, float clamp_max,
    const float *scale_b, void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
