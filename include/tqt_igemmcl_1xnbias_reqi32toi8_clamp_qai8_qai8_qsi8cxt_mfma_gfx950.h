/*
 * Micro-kernel type igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt (int8 implicit-GEMM
 * convolution, channels-last), variant mfma_gfx950.
 *
 * input is NDHWC int8 [ID, IH, IW, IC] (one image, or a batch folded into the depth
 * dimension). B is the weight [OC_per_group, K] int8 with K ordered (kd, kh, kw, ic) as in
 * the reference's tqt_im2col_cl (src/common/tqt_conv.h:131-202). Output pixel p of this call
 * is global pixel m_idx + p, written to D + (m_idx + p) * ldd (D is addressed absolutely by
 * m_idx, as in the reference). Out-of-bounds taps contribute int8 0. The epilogue is the
 * W8A8 requantization (bias, requantize, saturate, clamp). C, ldc, k, k_idx_a and k_idx_b
 * are ignored, as in the reference.
 *
 * Drop-in for src/conv/igemm_i8_i8/igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt/
 * tqt_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_4x1vl_rvv.h (functions at the .cpp
 * :26-71 and :194-286). There is no get_a_offset, as in the reference.
 */
#ifndef TQT_IGEMMCL_1XNBIAS_REQI32TOI8_CLAMP_QAI8_QAI8_QSI8CXT_MFMA_GFX950_H
#define TQT_IGEMMCL_1XNBIAS_REQI32TOI8_CLAMP_QAI8_QAI8_QSI8CXT_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference ..._4x1vl_rvv.cpp:26 / :31 */
size_t tqt_get_m_step_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(void);
size_t tqt_get_n_step_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(void);
/* reference ..._4x1vl_rvv.cpp:36: (n_idx * ldb + k_idx) bytes */
size_t tqt_get_b_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb);
/* reference ..._4x1vl_rvv.cpp:44: (m_idx * ldc + n_idx) * 4 bytes */
size_t tqt_get_c_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc);
/* reference ..._4x1vl_rvv.cpp:52: n_idx * 4 bytes */
size_t tqt_get_bias_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t n_idx);
/* reference ..._4x1vl_rvv.cpp:59: (m_idx * ldd + n_idx) bytes */
size_t tqt_get_d_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd);
/* reference ..._4x1vl_rvv.cpp:67: m * n bytes */
size_t tqt_get_d_size_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t m,
                                                                                    size_t n);

/* reference ..._4x1vl_rvv.cpp:194-198 */
void tqt_run_igemm_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *input, size_t group_idx, size_t m_idx,
    size_t k_idx_a, const void *B, size_t ldb, size_t k_idx_b, const void *C, size_t ldc,
    void *D, size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const tqt_conv_params *conv_params, const struct tqt_qai8_qai8_qsi8cx_params *quant_params);

/* Stream-ordered form (no counterpart in the reference). */
void tqt_run_igemm_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *input, size_t group_idx, size_t m_idx,
    size_t k_idx_a, const void *B, size_t ldb, size_t k_idx_b, const void *C, size_t ldc,
    void *D, size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const tqt_conv_params *conv_params, const struct tqt_qai8_qai8_qsi8cx_params *quant_params,
    void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
