/*
 * Micro-kernel type gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt, variant mfma_gfx950.
 *
 * Computes D = clamp(f(sum_k int16(A - zero_point_a[m]) * B)) with A int8 [m, k] quantized
 * per row (scale_a[m], zero_point_a[m]), B int8 [n, k] quantized per channel (scale_b[n],
 * symmetric), as tqt_kernel_gemm_qai8dx_qsi8cx_4x1vl_rvv.h defines it, bit for bit:
 * acc is the int32 (wrap-around) sum; f = f32(acc) * (scale_b[n] * scale_a[m]),
 * + bias[n] (f32; +0 when bias is NULL), then max with clamp_min and min with clamp_max in the
 * RISC-V sense (a NaN operand yields the other one, -0 orders below +0). Every step is one
 * rounded f32 operation (dequant_fp32, :145-215).
 * C is not an input (the reference ignores it; pass NULL). The kernels compute the sum as
 * sum A * B - zero_point_a[m] * sum B; for a zero point outside [-32640, 32640], where
 * A - zero_point_a[m] leaves 16 bits, the affected outputs are summed term by term with the
 * reference's 16-bit difference.
 *
 * Drop-in for src/gemm/gemm_i8_i8/gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt/tqt_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_4x1vl_rvv.h
 * (the line of each declaration is given below). Every tensor pointer is device-
 * accessible; the runs return with their output written; the _async forms (no
 * counterpart in the reference) enqueue on a hipStream_t instead. Params structs and
 * scalars stay on the host.
 */
#ifndef TQT_GEMM_1XNBIAS_CLAMP_F32_QAI8DX_QSI8CXT_MFMA_GFX950_H
#define TQT_GEMM_1XNBIAS_CLAMP_F32_QAI8DX_QSI8CXT_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference :36 */
size_t tqt_get_m_step_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(void);
/* reference :43 */
size_t tqt_get_n_step_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(void);
/* reference :52 */
size_t tqt_get_a_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(
    size_t m_idx, size_t k_idx, size_t lda);
/* reference :65 */
size_t tqt_get_b_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb);
/* reference :75 */
size_t tqt_get_c_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc);
/* reference :83 */
size_t tqt_get_bias_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(size_t n_idx);
/* reference :92 */
size_t tqt_get_d_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd);
/* reference :101 */
size_t tqt_get_d_size_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(size_t m, size_t n);
/* reference :130 */
void tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    float clamp_min, float clamp_max, const struct tqt_qai8dxp_qsi8cxp_params *params);
/* stream-ordered form */
void tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    float clamp_min, float clamp_max, const struct tqt_qai8dxp_qsi8cxp_params *params,
    void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
