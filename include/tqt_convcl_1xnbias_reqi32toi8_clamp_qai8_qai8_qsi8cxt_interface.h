/*
 * Interface of micro-kernel type convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt: function-pointer types and the ukernel
 * struct that every variant of this type fills. Same names, member order and signatures
 * as the reference's src/conv/conv_i8_i8/convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt/tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_interface.h:27-70,
 * so a caller that binds a variant through this struct can bind the gfx950 variant
 * (tqt_*_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950) unchanged.
 */
#ifndef TQT_CONVCL_1XNBIAS_REQI32TOI8_CLAMP_QAI8_QAI8_QSI8CXT_INTERFACE_H
#define TQT_CONVCL_1XNBIAS_REQI32TOI8_CLAMP_QAI8_QAI8_QSI8CXT_INTERFACE_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef size_t (*tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_m_step_func_t)(void);
typedef size_t (*tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_n_step_func_t)(void);
typedef size_t (*tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_b_offset_func_t)(
    size_t n_idx, size_t k_idx, size_t ldb);
typedef size_t (*tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_c_offset_func_t)(
    size_t m_idx, size_t n_idx, size_t ldc);
typedef size_t (*tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_bias_offset_func_t)(
    size_t n_idx);
typedef size_t (*tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_d_offset_func_t)(
    size_t m_idx, size_t n_idx, size_t ldd);
typedef size_t (*tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_d_size_func_t)(
    size_t m, size_t n);
typedef size_t (*tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_a_im2col_size_func_t)(
    size_t m, size_t k);
typedef size_t (*tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_a_im2col_offset_func_t)(
    size_t m_idx, size_t k_idx, size_t lda_im2col);
typedef void (*tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_run_im2col_func_t)(
    size_t group_idx, const void *activation, void *im2col_buf, const tqt_conv_params *params);
typedef void (*tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_run_conv_func_t)(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qai8_qsi8cx_params *params);

struct tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_ukernel
{
    tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_m_step_func_t get_m_step;
    tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_n_step_func_t get_n_step;
    tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_b_offset_func_t get_b_offset;
    tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_c_offset_func_t get_c_offset;
    tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_bias_offset_func_t get_bias_offset;
    tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_d_offset_func_t get_d_offset;
    tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_d_size_func_t get_d_size;
    tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_a_im2col_size_func_t get_a_im2col_size;
    tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_get_a_im2col_offset_func_t get_a_im2col_offset;
    tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_run_im2col_func_t run_im2col;
    tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_run_conv_func_t run_conv;
};

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
