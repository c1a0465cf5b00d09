/*
 * Micro-kernel type gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p, variant mfma_gfx950.
 *
 * Computes D = clamp(requantize(C + A * B + bias)) with A int8 [m, k] (weights, symmetric,
 * per-row scale_a[m] or one scale when quant_channel_a == 1), B int8 [k, n] row-major
 * (activations, scalar scale_b; zero_point_b folded into the bias by the caller), C int32
 * [m, n] (optional), bias int32 [m] (Mx1: one per row), D int8 [m, n]: per row the multiplier of
 * scale_a[i] * scale_b / scale_d (tqt_quantize_multiplier, shift = -shift - 1), then the
 * requantization and clamp of gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt.
 * A and B are pre-packed (A from [m, k] by run_a_pack; B from [k, n] by run_b_pack or from
 * [n, k] by run_bt_pack), in the layout of gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp.
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
 * Drop-in for src/gemm/gemm_i8_i8/gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p/tqt_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_4x1vl_rvv.h
 * (the line of each declaration is given below). Every pointer, source and packed
 * buffers included, is device-accessible; the packers run on the GPU and, like the runs,
 * return with their output written; the _async forms (no counterpart in the reference)
 * enqueue on a hipStream_t instead. Params structs and scalars stay on the host.
 */
#ifndef TQT_GEMM_MX1BIAS_REQI32TOI8_CLAMP_QAI8_QSI8DXP_QAI8P_MFMA_GFX950_H
#define TQT_GEMM_MX1BIAS_REQI32TOI8_CLAMP_QAI8_QSI8DXP_QAI8P_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference :36 */
size_t tqt_get_m_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(void);
/* reference :43 */
size_t tqt_get_n_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(void);
/* reference :53 */
size_t tqt_get_a_packed_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(
    size_t m_idx, size_t k_idx, size_t lda, size_t actual_m);
/* reference :64 */
size_t tqt_get_b_packed_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb, size_t actual_n);
/* reference :74 */
size_t tqt_get_c_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc);
/* reference :83 */
size_t tqt_get_bias_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(
    size_t m_idx);
/* reference :92 */
size_t tqt_get_d_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd);
/* reference :102 */
size_t tqt_get_d_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(
    size_t m, size_t n);
/* reference :111 */
size_t tqt_get_a_packed_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(
    size_t m, size_t k);
/* reference :120 */
size_t tqt_get_b_packed_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(
    size_t n, size_t k);
/* reference :132 */
void tqt_run_a_pack_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(
    size_t m, size_t k, size_t lda, size_t lda_packed, size_t k_idx, const void *A, void *A_packed);
/* stream-ordered form */
void tqt_run_a_pack_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950_async(
    size_t m, size_t k, size_t lda, size_t lda_packed, size_t k_idx, const void *A, void *A_packed,
    void *stream);
/* reference :144 */
void tqt_run_b_pack_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed);
/* stream-ordered form */
void tqt_run_b_pack_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950_async(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed,
    void *stream);
/* reference :156 */
void tqt_run_bt_pack_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed);
/* stream-ordered form */
void tqt_run_bt_pack_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950_async(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed,
    void *stream);
/* reference :184 */
void tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const struct tqt_qai8_qsi8dx_qai8_params *params);
/* stream-ordered form */
void tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const struct tqt_qai8_qsi8dx_qai8_params *params, void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
