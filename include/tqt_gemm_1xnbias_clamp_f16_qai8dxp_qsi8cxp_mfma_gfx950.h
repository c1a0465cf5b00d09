/*
 * Micro-kernel type gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp, variant mfma_gfx950.
 *
 * Computes D = clamp(f(sum_k int16(A - zero_point_a[m]) * B)) with A int8 [m, k] quantized
 * per row (scale_a[m], zero_point_a[m]), B int8 [n, k] quantized per channel (scale_b[n],
 * symmetric), as tqt_kernel_gemm_qai8dx_qsi8cx_4x1vl_rvv.h defines it, bit for bit:
 * acc is the int32 (wrap-around) sum; the f32 product f32(acc) * (scale_b[n] * scale_a[m]) is
 * rounded to f16, the f16 bias[n] (+0 when bias is NULL) is added in f16 (one rounding), then
 * max / min with the f16 bounds in the RISC-V sense; a NaN is stored as 0x7e00
 * (dequant_fp16, :217-330).
 * C is not an input (the reference ignores it; pass NULL). The kernels compute the sum as
 * sum A * B - zero_point_a[m] * sum B; for a zero point outside [-32640, 32640], where
 * A - zero_point_a[m] leaves 16 bits, the affected outputs are summed term by term with the
 * reference's 16-bit difference.
 * A and B are pre-packed by this type's packers (the qai8_qai8p_qsi8cxp layout).
 *
 * Packed layout (this build's; the reference's is its own [m/MR, k, MR] / [n/vl, k, vl]):
 * rows (m of A, n of B) form panels of m_step / n_step rows. Panel p holds rows
 * [p*step, p*step + w), w = min(step, rows - p*step), and starts at element p*step*ld_packed,
 * moved back by k_idx*(step - w) elements when a panel after the first is narrower (the
 * reference's tail rule, tqt_gemm_pack_rvv.h:314-318). Inside a panel each row is cut into
 * 16-byte chunks stored chunk-major: chunk c of local row r at byte 16*c*w + r*cw,
 * cw = min(16, row bytes - 16*c). A chunk is one MFMA lane fragment (16 k bytes, or
 * 32 int4 values); the kernels load one chunk of 8 or more consecutive rows per group of
 * consecutive lanes, whole cache lines.
 * The packed_offset getters keep the reference's formula (idx*ld + k_idx*min(actual, step))
 * elements; it addresses element (idx, k_idx) of a full-K packing when k_idx is a whole number
 * of chunks, and the start of a k_idx sub-buffer packed with that k_idx in any case. Packed
 * sizes equal the unpacked ones.
 *
 * Drop-in for src/gemm/gemm_i8_i8/gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp/tqt_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_4x1vl_rvv.h
 * (the line of each declaration is given below). Every pointer, source and packed
 * buffers included, is device-accessible; the packers run on the GPU and, like the runs,
 * return with their output written; the _async forms (no counterpart in the reference)
 * enqueue on a hipStream_t instead. Params structs and scalars stay on the host.
 */
#ifndef TQT_GEMM_1XNBIAS_CLAMP_F16_QAI8DXP_QSI8CXP_MFMA_GFX950_H
#define TQT_GEMM_1XNBIAS_CLAMP_F16_QAI8DXP_QSI8CXP_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference :36 */
size_t tqt_get_m_step_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950(void);
/* reference :43 */
size_t tqt_get_n_step_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950(void);
/* reference :55 */
size_t tqt_get_a_packed_offset_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950(
    size_t m_idx, size_t k_idx, size_t lda, size_t actual_m);
/* reference :70 */
size_t tqt_get_b_packed_offset_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb, size_t actual_n);
/* reference :82 */
size_t tqt_get_c_offset_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc);
/* reference :90 */
size_t tqt_get_bias_offset_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950(size_t n_idx);
/* reference :99 */
size_t tqt_get_d_offset_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd);
/* reference :108 */
size_t tqt_get_d_size_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950(size_t m, size_t n);
/* reference :116 */
size_t tqt_get_a_packed_size_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950(size_t m, size_t k);
/* reference :124 */
size_t tqt_get_b_packed_size_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950(size_t n, size_t k);
/* reference :135 */
void tqt_run_a_pack_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950(
    size_t m, size_t k, size_t lda, size_t lda_packed, size_t k_idx, const void *A, void *A_packed);
/* stream-ordered form */
void tqt_run_a_pack_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950_async(
    size_t m, size_t k, size_t lda, size_t lda_packed, size_t k_idx, const void *A, void *A_packed,
    void *stream);
/* reference :149 */
void tqt_run_b_pack_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed);
/* stream-ordered form */
void tqt_run_b_pack_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950_async(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed,
    void *stream);
/* reference :163 */
void tqt_run_bt_pack_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed);
/* stream-ordered form */
void tqt_run_bt_pack_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950_async(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed,
    void *stream);
/* reference :194 */
void tqt_run_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, float16_t clamp_min, float16_t clamp_max,
    const struct tqt_qai8dxp_qsi8cxp_params *params);
/* stream-ordered form */
void tqt_run_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, float16_t clamp_min, float16_t clamp_max,
    const struct tqt_qai8dxp_qsi8cxp_params *params, void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
