/*
 * Micro-kernel type igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8, variant mfma_gfx950.
 *
 * Implicit-GEMM convolution, channel-first: D [m, pixels] int8 = the mx1bias GEMM of the
 * weights A [m = OC_per_group, K] (K = IC_per_group*KD*KH*KW in (ic, kd, kh, kw) order) with the
 * channel-first im2col of one group of the NCDHW input, gathered on the fly, for the output
 * pixels [n_idx, n_idx + n); row i of D is written at D + i * ldd + n_idx. C is not read (the
 * reference ignores it). The requantization is the per-row one of
 * gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8.
 *
 * Drop-in for src/conv/igemm_i8_i8/igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8/tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_1vlx4_rvv.h
 * (the line of each declaration is given below). Every tensor pointer is device-
 * accessible; the runs return with their output written; the _async forms (no
 * counterpart in the reference) enqueue on a hipStream_t instead. Params structs and
 * scalars stay on the host.
 */
#ifndef TQT_IGEMMCF_MX1BIAS_REQI32TOI8_CLAMP_QAI8_QSI8DX_QAI8_MFMA_GFX950_H
#define TQT_IGEMMCF_MX1BIAS_REQI32TOI8_CLAMP_QAI8_QSI8DX_QAI8_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference :39 */
size_t tqt_get_m_step_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(void);
/* reference :44 */
size_t tqt_get_n_step_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(void);
/* reference :53 */
size_t tqt_get_a_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m_idx, size_t k_idx, size_t lda);
/* reference :64 */
size_t tqt_get_c_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc);
/* reference :73 */
size_t tqt_get_bias_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m_idx);
/* reference :83 */
size_t tqt_get_d_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd);
/* reference :93 */
size_t tqt_get_d_size_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m, size_t n);
/* reference :121 */
void tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *input, size_t group_idx, size_t n_idx, size_t k_idx_b,
    const void *A, size_t lda, size_t k_idx_a, const void *C, size_t ldc, void *D, size_t ldd,
    const void *bias, int8_t clamp_min, int8_t clamp_max, const tqt_conv_params *conv_params,
    const struct tqt_qai8_qsi8dx_qai8_params *quant_params);
/* stream-ordered form */
void tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *input, size_t group_idx, size_t n_idx, size_t k_idx_b,
    const void *A, size_t lda, size_t k_idx_a, const void *C, size_t ldc, void *D, size_t ldd,
    const void *bias, int8_t clamp_min, int8_t clamp_max, const tqt_conv_params *conv_params,
    const struct tqt_qai8_qsi8dx_qai8_params *quant_params, void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
