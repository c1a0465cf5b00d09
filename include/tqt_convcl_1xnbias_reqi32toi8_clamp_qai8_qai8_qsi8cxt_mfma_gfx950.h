/*
 * Micro-kernel type convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt, variant mfma_gfx950.
 *
 * Explicit-im2col convolution, channel-last: run_im2col writes im2col(activation) of one group
 * as the row-major int8 matrix A [M, K] (M = OD*OH*OW output pixels, K = KD*KH*KW*IC_per_group
 * in (kd, kh, kw, ic) order, zeros for padding taps; reference src/common/tqt_conv.h:131-202),
 * and run_conv is gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt on it with the weights
 * B [N, K] (N = OC_per_group): D [M, N] int8. The geometry getters are that GEMM's.
 *
 * Drop-in for src/conv/conv_i8_i8/convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt/tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_4x1vl_rvv.h
 * (the line of each declaration is given below). Every tensor pointer is device-
 * accessible; the runs return with their output written; the _async forms (no
 * counterpart in the reference) enqueue on a hipStream_t instead. Params structs and
 * scalars stay on the host.
 */
#ifndef TQT_CONVCL_1XNBIAS_REQI32TOI8_CLAMP_QAI8_QAI8_QSI8CXT_MFMA_GFX950_H
#define TQT_CONVCL_1XNBIAS_REQI32TOI8_CLAMP_QAI8_QAI8_QSI8CXT_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference :34 */
size_t tqt_get_m_step_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(void);
/* reference :41 */
size_t tqt_get_n_step_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(void);
/* reference :50 */
size_t tqt_get_b_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb);
/* reference :61 */
size_t tqt_get_c_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc);
/* reference :70 */
size_t tqt_get_bias_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t n_idx);
/* reference :80 */
size_t tqt_get_d_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd);
/* reference :90 */
size_t tqt_get_d_size_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m, size_t n);
/* reference :99 */
size_t tqt_get_a_im2col_size_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m, size_t k);
/* reference :109 */
size_t tqt_get_a_im2col_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m_idx, size_t k_idx, size_t lda_im2col);
/* reference :124 */
void tqt_run_im2col_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t group_idx, const void *activation, void *im2col_buf, const tqt_conv_params *params);
/* stream-ordered form */
void tqt_run_im2col_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950_async(
    size_t group_idx, const void *activation, void *im2col_buf, const tqt_conv_params *params,
    void *stream);
/* reference :154 */
void tqt_run_conv_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qai8_qsi8cx_params *params);
/* stream-ordered form */
void tqt_run_conv_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qai8_qsi8cx_params *params,
    void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
