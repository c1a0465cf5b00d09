/*
 * Micro-kernel type convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp, variant mfma_gfx950.
 *
 * Explicit-im2col convolution, channel-last, packed: run_a_im2colpack writes im2col(activation)
 * of one group (the [M, K] matrix of convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt) straight
 * into the packed A layout of gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp (leading
 * dimension lda_packed, the packers' k_idx tail rule); run_bt_pack packs the weights [N, K];
 * run_conv is that GEMM. The geometry getters are that GEMM's.
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
 * Drop-in for src/conv/conv_i8_i8/convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp/tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_4x1vl_rvv.h
 * (the line of each declaration is given below). Every pointer, source and packed
 * buffers included, is device-accessible; the packers run on the GPU and, like the runs,
 * return with their output written; the _async forms (no counterpart in the reference)
 * enqueue on a hipStream_t instead. Params structs and scalars stay on the host.
 */
#ifndef TQT_CONVCL_1XNBIAS_REQI32TOI8_CLAMP_QAI8_QAI8P_QSI8CXP_MFMA_GFX950_H
#define TQT_CONVCL_1XNBIAS_REQI32TOI8_CLAMP_QAI8_QAI8P_QSI8CXP_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference :31 */
size_t tqt_get_m_step_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(void);
/* reference :38 */
size_t tqt_get_n_step_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(void);
/* reference :48 */
size_t tqt_get_a_im2colpack_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t m_idx, size_t k_idx, size_t lda, size_t actual_m);
/* reference :59 */
size_t tqt_get_b_packed_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb, size_t actual_n);
/* reference :69 */
size_t tqt_get_c_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc);
/* reference :78 */
size_t tqt_get_bias_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t n_idx);
/* reference :88 */
size_t tqt_get_d_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd);
/* reference :98 */
size_t tqt_get_d_size_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t m, size_t n);
/* reference :107 */
size_t tqt_get_a_im2colpack_size_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t m, size_t k);
/* reference :116 */
size_t tqt_get_b_packed_size_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t n, size_t k);
/* reference :128 */
void tqt_run_bt_pack_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed);
/* stream-ordered form */
void tqt_run_bt_pack_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed,
    void *stream);
/* reference :139 */
void tqt_run_a_im2colpack_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t group_idx, const void *activation, size_t lda_packed, size_t k_idx, void *A_packed,
    const tqt_conv_params *params);
/* stream-ordered form */
void tqt_run_a_im2colpack_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(
    size_t group_idx, const void *activation, size_t lda_packed, size_t k_idx, void *A_packed,
    const tqt_conv_params *params, void *stream);
/* reference :169 */
void tqt_run_conv_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const struct tqt_qai8_qai8_qsi8cx_params *params);
/* stream-ordered form */
void tqt_run_conv_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const struct tqt_qai8_qai8_qsi8cx_params *params, void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
