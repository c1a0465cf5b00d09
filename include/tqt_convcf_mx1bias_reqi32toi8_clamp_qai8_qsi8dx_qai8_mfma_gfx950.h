/*
 * Micro-kernel type convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8, variant mfma_gfx950.
 *
 * Explicit-im2col convolution, channel-first: run_im2col writes im2col(activation) of one
 * group (NCDHW input) as the row-major int8 matrix B [K, N] (K = IC_per_group*KD*KH*KW in
 * (ic, kd, kh, kw) order, N = OD*OH*OW output pixels, zeros for padding taps; reference
 * src/common/tqt_conv.h:51-119), and run_conv is gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8
 * with the weights as A [OC_per_group, K]: D [OC_per_group, N] int8 (channel-first output).
 *
 * Drop-in for src/conv/conv_i8_i8/convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8/tqt_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_4x1vl_rvv.h
 * (the line of each declaration is given below). Every tensor pointer is device-
 * accessible; the runs return with their output written; the _async forms (no
 * counterpart in the reference) enqueue on a hipStream_t instead. Params structs and
 * scalars stay on the host.
 */
#ifndef TQT_CONVCF_MX1BIAS_REQI32TOI8_CLAMP_QAI8_QSI8DX_QAI8_MFMA_GFX950_H
#define TQT_CONVCF_MX1BIAS_REQI32TOI8_CLAMP_QAI8_QSI8DX_QAI8_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference :33 */
size_t tqt_get_m_step_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(void);
/* reference :40 */
size_t tqt_get_n_step_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(void);
/* reference :49 */
size_t tqt_get_a_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m_idx, size_t k_idx, size_t lda);
/* reference :60 */
size_t tqt_get_c_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc);
/* reference :69 */
size_t tqt_get_bias_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m_idx);
/* reference :78 */
size_t tqt_get_d_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd);
/* reference :88 */
size_t tqt_get_d_size_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m, size_t n);
/* reference :97 */
size_t tqt_get_b_im2col_size_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t k, size_t n);
/* reference :107 */
size_t tqt_get_b_im2col_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb_im2col);
/* reference :118 */
void tqt_run_im2col_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t group_idx, const void *activation, void *im2col_buf, const tqt_conv_params *params);
/* stream-ordered form */
void tqt_run_im2col_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950_async(
    size_t group_idx, const void *activation, void *im2col_buf, const tqt_conv_params *params,
    void *stream);
/* reference :149 */
void tqt_run_conv_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qsi8dx_qai8_params *params);
/* stream-ordered form */
void tqt_run_conv_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qsi8dx_qai8_params *params,
    void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
