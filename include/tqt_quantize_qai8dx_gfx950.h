/*
 * Dynamic per-row asymmetric int8 quantization of f32 activations into the qai8dx operand of
 * gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt (and its packed sibling): the step before the W4A8
 * GEMV of a decode loop, run on the GPU so the activations never leave HBM.
 *
 * No counterpart in the reference library: the reference has this step only as test-side code,
 * quantize_a_per_row_asym (test/gemm/test_gemm_i8_i4_rvv.cpp:40-77, with quantize_i8 from
 * test/common/test_common.h:232-240). The results are bit-identical to it:
 *   fmax = max(0, max_k A[r, k]), fmin = min(0, min_k A[r, k]), s = (fmax - fmin) / 255
 *   s == 0:  scale_a[r] = 1, zero_point_a[r] = 0, A_q[r, :] = 0
 *   else:    zero_point_a[r] = clamp(nearbyint(-128 - fmin / s), -128, 127), scale_a[r] = s,
 *            A_q[r, k] = clamp(nearbyint(A[r, k] / s) + zero_point_a[r], -128, 127)
 * (float arithmetic, correctly rounded divisions, round-half-even nearbyint, no fused
 * multiply-add).
 *
 * A [m, lda] f32, A_q [m, lda_q] int8, scale_a [m] f32 and zero_point_a [m] int32 are device
 * pointers; lda, lda_q >= k. The plain form returns with the outputs written; the _async form
 * enqueues on `stream` (a hipStream_t, NULL = the default stream).
 */
#ifndef TQT_QUANTIZE_QAI8DX_GFX950_H
#define TQT_QUANTIZE_QAI8DX_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

void tqt_run_quantize_qai8dx_f32_gfx950(size_t m, size_t k, const float *A, size_t lda,
                                        int8_t *A_q, size_t lda_q, float *scale_a,
                                        int32_t *zero_point_a);

void tqt_run_quantize_qai8dx_f32_gfx950_async(size_t m, size_t k, const float *A, size_t lda,
                                              int8_t *A_q, size_t lda_q, float *scale_a,
                                              int32_t *zero_point_a, void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
