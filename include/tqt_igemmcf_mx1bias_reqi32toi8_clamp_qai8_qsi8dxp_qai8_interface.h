/*
 * Interface of micro-kernel type igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8: function-pointer types and the ukernel
 * struct that every variant of this type fills. Same names, member order and signatures
 * as the reference's src/conv/igemm_i8_i8/igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8/tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_interface.h:34-76,
 * so a caller that binds a variant through this struct can bind the gfx950 variant
 * (tqt_*_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950) unchanged.
 */
#ifndef TQT_IGEMMCF_MX1BIAS_REQI32TOI8_CLAMP_QAI8_QSI8DXP_QAI8_INTERFACE_H
#define TQT_IGEMMCF_MX1BIAS_REQI32TOI8_CLAMP_QAI8_QSI8DXP_QAI8_INTERFACE_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef size_t (*tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_m_step_func_t)(void);
typedef size_t (*tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_n_step_func_t)(void);
typedef size_t (*tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_a_packed_offset_func_t)(
    size_t m_idx, size_t k_idx, size_t lda, size_t actual_m);
typedef size_t (*tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_c_offset_func_t)(
    size_t m_idx, size_t n_idx, size_t ldc);
typedef size_t (*tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_bias_offset_func_t)(
    size_t m_idx);
typedef size_t (*tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_d_offset_func_t)(
    size_t m_idx, size_t n_idx, size_t ldd);
typedef size_t (*tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_d_size_func_t)(
    size_t m, size_t n);
typedef size_t (*tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_a_packed_size_func_t)(
    size_t m, size_t k);
typedef void (*tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_run_a_pack_func_t)(
    size_t m, size_t k, size_t ldw, size_t ldw_packed, size_t k_idx, const void *weight,
    void *weight_packed);
typedef void (*tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_run_igemm_func_t)(
    size_t m, size_t n, size_t k, const void *input, size_t group_idx, size_t n_idx, size_t k_idx_b,
    const void *A_packed, size_t lda, size_t k_idx_a, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const tqt_conv_params *conv_params, const struct tqt_qai8_qsi8dx_qai8_params *quant_params);

struct tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_ukernel
{
    tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_m_step_func_t get_m_step;
    tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_n_step_func_t get_n_step;
    tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_a_packed_offset_func_t get_a_packed_offset;
    tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_c_offset_func_t get_c_offset;
    tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_bias_offset_func_t get_bias_offset;
    tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_d_offset_func_t get_d_offset;
    tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_d_size_func_t get_d_size;
    tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_get_a_packed_size_func_t get_a_packed_size;
    tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_run_a_pack_func_t run_a_pack;
    tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_run_igemm_func_t run_igemm;
};

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
