/*
 * Interface of micro-kernel type gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp: function-pointer types and the ukernel
 * struct that every variant of this type fills. Same names, member order and signatures
 * as the reference's src/gemm/gemm_i8_i8/gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp/tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_interface.h:23-66,
 * so a caller that binds a variant through this struct can bind the gfx950 variant
 * (tqt_*_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950) unchanged.
 */
#ifndef TQT_GEMM_1XNBIAS_REQI32TOI8_CLAMP_QAI8_QAI8_QSI8CXP_INTERFACE_H
#define TQT_GEMM_1XNBIAS_REQI32TOI8_CLAMP_QAI8_QAI8_QSI8CXP_INTERFACE_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef size_t (*tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_m_step_func_t)(void);
typedef size_t (*tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_n_step_func_t)(void);
typedef size_t (*tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_a_offset_func_t)(
    size_t m_idx, size_t k_idx, size_t lda);
typedef size_t (*tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_b_packed_offset_func_t)(
    size_t n_idx, size_t k_idx, size_t ldb, size_t actual_n);
typedef size_t (*tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_c_offset_func_t)(
    size_t m_idx, size_t n_idx, size_t ldc);
typedef size_t (*tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_bias_offset_func_t)(size_t n_idx);
typedef size_t (*tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_d_offset_func_t)(
    size_t m_idx, size_t n_idx, size_t ldd);
typedef size_t (*tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_d_size_func_t)(size_t m, size_t n);
typedef size_t (*tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_b_packed_size_func_t)(
    size_t n, size_t k);
typedef void (*tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_run_b_pack_func_t)(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed);
typedef void (*tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_run_bt_pack_func_t)(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed);
typedef void (*tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_run_gemm_func_t)(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B_packed,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qai8_qsi8cx_params *params);

struct tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_ukernel
{
    tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_m_step_func_t get_m_step;
    tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_n_step_func_t get_n_step;
    tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_a_offset_func_t get_a_offset;
    tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_b_packed_offset_func_t get_b_packed_offset;
    tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_c_offset_func_t get_c_offset;
    tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_bias_offset_func_t get_bias_offset;
    tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_d_offset_func_t get_d_offset;
    tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_d_size_func_t get_d_size;
    tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_get_b_packed_size_func_t get_b_packed_size;
    tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_run_b_pack_func_t run_b_pack;
    tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_run_bt_pack_func_t run_bt_pack;
    tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_run_gemm_func_t run_gemm;
};

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
