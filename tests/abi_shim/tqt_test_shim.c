/*
 * Test-side C caller of the library. It plays the part of a framework that binds the gfx950
 * variants through the reference-shaped interface structs (tqt_*_interface.h) and calls them
 * with C argument types, including _Float16 by value, which Python's ctypes cannot pass.
 * Assigning each variant to its interface struct member is the compile-time check that every
 * signature matches the interface exactly.
 */
#include <stdint.h>
#include <string.h>

#include "tqt_gemm_1xnbias_clamp_f16_f16_qsi4c2t_interface.h"
#include "tqt_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_interface.h"
#include "tqt_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_interface.h"
#include "tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950.h"
#include "tqt_gemm_clamp_i32_i8_i8_interface.h"
#include "tqt_gemm_clamp_i32_i8_i8_mfma_gfx950.h"
#include "tqt_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_interface.h"
#include "tqt_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950.h"
#include "tqt_gemm_clamp_i32_i8p_i8p_interface.h"
#include "tqt_gemm_clamp_i32_i8p_i8p_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_interface.h"
#include "tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_interface.h"
#include "tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_interface.h"
#include "tqt_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_interface.h"
#include "tqt_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950.h"
#include "tqt_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_interface.h"
#include "tqt_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_interface.h"
#include "tqt_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950.h"
#include "tqt_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_interface.h"
#include "tqt_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950.h"
#include "tqt_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_interface.h"
#include "tqt_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950.h"
#include "tqt_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_interface.h"
#include "tqt_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950.h"
#include "tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_interface.h"
#include "tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950.h"
#include "tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_interface.h"
#include "tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950.h"
#include "tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_interface.h"
#include "tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950.h"
#include "tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_interface.h"
#include "tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_interface.h"
#include "tqt_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_interface.h"
#include "tqt_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_interface.h"
#include "tqt_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_interface.h"
#include "tqt_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f32_f16_qsi4c2t_interface.h"
#include "tqt_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_interface.h"
#include "tqt_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt_interface.h"
#include "tqt_gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_interface.h"
#include "tqt_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_interface.h"
#include "tqt_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_interface.h"
#include "tqt_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950.h"

static const struct tqt_gemm_clamp_i32_i8_i8_ukernel k_clamp = {
    tqt_get_m_step_gemm_clamp_i32_i8_i8_mfma_gfx950,
    tqt_get_n_step_gemm_clamp_i32_i8_i8_mfma_gfx950,
    tqt_get_a_offset_gemm_clamp_i32_i8_i8_mfma_gfx950,
    tqt_get_b_offset_gemm_clamp_i32_i8_i8_mfma_gfx950,
    tqt_get_c_offset_gemm_clamp_i32_i8_i8_mfma_gfx950,
    tqt_get_d_offset_gemm_clamp_i32_i8_i8_mfma_gfx950,
    tqt_get_d_size_gemm_clamp_i32_i8_i8_mfma_gfx950,
    tqt_run_gemm_clamp_i32_i8_i8_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_ukernel k_w8a8 = {
    tqt_get_m_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_a_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_b_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_ukernel k_w4a8 = {
    tqt_get_m_step_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_a_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_b_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_clamp_f16_f16_qsi4c2t_ukernel k_w4a16 = {
    tqt_get_m_step_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950,
    tqt_get_a_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950,
    tqt_get_b_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950,
    tqt_get_scale_b_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950,
    tqt_run_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950,
};

static const struct tqt_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_ukernel k_igemm = {
    tqt_get_m_step_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_n_step_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_b_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_c_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_bias_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_d_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_d_size_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_run_igemm_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
};

static const struct tqt_gemm_clamp_i32_i8p_i8p_ukernel k_clampp = {
    tqt_get_m_step_gemm_clamp_i32_i8p_i8p_mfma_gfx950,
    tqt_get_n_step_gemm_clamp_i32_i8p_i8p_mfma_gfx950,
    tqt_get_a_packed_offset_gemm_clamp_i32_i8p_i8p_mfma_gfx950,
    tqt_get_b_packed_offset_gemm_clamp_i32_i8p_i8p_mfma_gfx950,
    tqt_get_c_offset_gemm_clamp_i32_i8p_i8p_mfma_gfx950,
    tqt_get_d_offset_gemm_clamp_i32_i8p_i8p_mfma_gfx950,
    tqt_get_d_size_gemm_clamp_i32_i8p_i8p_mfma_gfx950,
    tqt_get_a_packed_size_gemm_clamp_i32_i8p_i8p_mfma_gfx950,
    tqt_get_b_packed_size_gemm_clamp_i32_i8p_i8p_mfma_gfx950,
    tqt_run_a_pack_gemm_clamp_i32_i8p_i8p_mfma_gfx950,
    tqt_run_b_pack_gemm_clamp_i32_i8p_i8p_mfma_gfx950,
    tqt_run_bt_pack_gemm_clamp_i32_i8p_i8p_mfma_gfx950,
    tqt_run_gemm_clamp_i32_i8p_i8p_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_ukernel k_w8a8pb = {
    tqt_get_m_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_get_a_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_get_b_packed_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_get_b_packed_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_run_b_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_run_bt_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_ukernel k_w8a8p = {
    tqt_get_m_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_a_packed_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_b_packed_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_a_packed_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_b_packed_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_run_a_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_run_b_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_run_bt_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_ukernel k_w4a8p = {
    tqt_get_m_step_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_a_packed_offset_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_b_packed_offset_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_a_packed_size_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_b_packed_size_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_run_a_pack_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_run_bt_pack_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_run_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_ukernel k_w4a16p = {
    tqt_get_m_step_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_a_packed_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_b_packed_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_scale_b_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_a_packed_size_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_b_packed_size_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950,
    tqt_run_a_pack_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950,
    tqt_run_bt_pack_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950,
    tqt_run_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950,
};

static const struct tqt_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_ukernel k_igemmp = {
    tqt_get_m_step_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_get_n_step_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_get_b_packed_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_get_c_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_get_bias_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_get_d_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_get_d_size_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_get_b_packed_size_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_run_bt_pack_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
    tqt_run_igemm_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt_ukernel k_w4a8_f16 = {
    tqt_get_m_step_gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_a_offset_gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_b_offset_gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_run_gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_ukernel k_w4a8p_f16 = {
    tqt_get_m_step_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_a_packed_offset_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_b_packed_offset_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_a_packed_size_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_b_packed_size_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_run_a_pack_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_run_bt_pack_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_run_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_ukernel k_w4a8_bf16 = {
    tqt_get_m_step_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_a_offset_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_b_offset_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950,
    tqt_run_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_ukernel k_w4a8p_bf16 = {
    tqt_get_m_step_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_a_packed_offset_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_b_packed_offset_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_a_packed_size_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_get_b_packed_size_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_run_a_pack_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_run_bt_pack_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950,
    tqt_run_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_clamp_f32_f16_qsi4c2t_ukernel k_w4a16f = {
    tqt_get_m_step_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950,
    tqt_get_a_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950,
    tqt_get_b_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950,
    tqt_get_scale_b_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950,
    tqt_run_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_ukernel k_w4a16fp = {
    tqt_get_m_step_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_a_packed_offset_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_b_packed_offset_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_scale_b_offset_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_a_packed_size_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950,
    tqt_get_b_packed_size_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950,
    tqt_run_a_pack_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950,
    tqt_run_bt_pack_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950,
    tqt_run_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_ukernel k_w8dyn = {
    tqt_get_m_step_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_get_a_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_get_b_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_ukernel k_w8dynp = {
    tqt_get_m_step_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_a_packed_offset_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_b_packed_offset_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_a_packed_size_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_b_packed_size_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_run_a_pack_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_run_b_pack_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_run_bt_pack_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_run_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_ukernel k_w8dynh = {
    tqt_get_m_step_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_get_a_offset_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_get_b_offset_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950,
    tqt_run_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950,
};

static const struct tqt_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_ukernel k_w8dynhp = {
    tqt_get_m_step_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_n_step_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_a_packed_offset_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_b_packed_offset_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_c_offset_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_bias_offset_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_d_offset_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_d_size_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_a_packed_size_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_get_b_packed_size_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_run_a_pack_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_run_b_pack_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_run_bt_pack_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950,
    tqt_run_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950,
};

static const struct tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_ukernel k_convcl = {
    tqt_get_m_step_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_n_step_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_b_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_c_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_bias_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_d_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_d_size_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_a_im2col_size_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_get_a_im2col_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_run_im2col_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
    tqt_run_conv_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950,
};

static const struct tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_ukernel k_convclp = {
    tqt_get_m_step_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_n_step_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_a_im2colpack_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_b_packed_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_c_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_bias_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_d_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_d_size_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_a_im2colpack_size_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_get_b_packed_size_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_run_bt_pack_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_run_a_im2colpack_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
    tqt_run_conv_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950,
};

static const struct tqt_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_ukernel k_mx1 = {
    tqt_get_m_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_n_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_a_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_b_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_c_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_bias_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_d_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_d_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
};

static const struct tqt_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_ukernel k_mx1p = {
    tqt_get_m_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_n_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_a_packed_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_b_packed_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_c_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_bias_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_d_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_d_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_a_packed_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_b_packed_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_run_a_pack_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_run_b_pack_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_run_bt_pack_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
};

static const struct tqt_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_ukernel k_convcf = {
    tqt_get_m_step_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_n_step_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_a_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_c_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_bias_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_d_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_d_size_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_b_im2col_size_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_b_im2col_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_run_im2col_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_run_conv_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
};

static const struct tqt_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_ukernel k_convcfp = {
    tqt_get_m_step_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_n_step_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_a_packed_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_b_im2colpack_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_c_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_bias_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_d_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_d_size_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_a_packed_size_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_get_b_im2colpack_size_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_run_a_pack_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_run_b_im2colpack_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
    tqt_run_conv_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950,
};

static const struct tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_ukernel k_igemmcf = {
    tqt_get_m_step_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_n_step_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_a_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_c_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_bias_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_d_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_get_d_size_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
    tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950,
};

static const struct tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_ukernel k_igemmcfp = {
    tqt_get_m_step_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950,
    tqt_get_n_step_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950,
    tqt_get_a_packed_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950,
    tqt_get_c_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950,
    tqt_get_bias_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950,
    tqt_get_d_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950,
    tqt_get_d_size_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950,
    tqt_get_a_packed_size_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950,
    tqt_run_a_pack_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950,
    tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950,
};

/* m_step and n_step of each kernel type read through its interface struct:
 * out[2*t], out[2*t+1] for t = clamp, w8a8, w4a8, w4a16, igemmcl, then the packed types
 * clamp_i32_i8p_i8p, qai8_qai8_qsi8cxp, qai8_qai8p_qsi8cxp, qai8dxp_qsi4cxp, f16p_qsi4c2p,
 * igemmcl qsi8cxp, then the W4A8 output siblings f16 qsi4cxt, f16 qsi4cxp, bf16 qsi4cxt,
 * bf16 qsi4cxp, then the W4A16 f32-output siblings qsi4c2t, qsi4c2p, then the qai8dx x qsi8cx
 * types f32 qsi8cxt, f32 qsi8cxp, f16 qsi8cxt, f16 qsi8cxp, then convcl qsi8cxt, qsi8cxp, then the
 * channel-first gemm_mx1bias, its packed form, convcf, convcf packed, igemmcf, igemmcf packed. */
void tqts_steps_via_interfaces(size_t out[58])
{
    out[0] = k_clamp.get_m_step();
    out[1] = k_clamp.get_n_step();
    out[2] = k_w8a8.get_m_step();
    out[3] = k_w8a8.get_n_step();
    out[4] = k_w4a8.get_m_step();
    out[5] = k_w4a8.get_n_step();
    out[6] = k_w4a16.get_m_step();
    out[7] = k_w4a16.get_n_step();
    out[8] = k_igemm.get_m_step();
    out[9] = k_igemm.get_n_step();
    out[10] = k_clampp.get_m_step();
    out[11] = k_clampp.get_n_step();
    out[12] = k_w8a8pb.get_m_step();
    out[13] = k_w8a8pb.get_n_step();
    out[14] = k_w8a8p.get_m_step();
    out[15] = k_w8a8p.get_n_step();
    out[16] = k_w4a8p.get_m_step();
    out[17] = k_w4a8p.get_n_step();
    out[18] = k_w4a16p.get_m_step();
    out[19] = k_w4a16p.get_n_step();
    out[20] = k_igemmp.get_m_step();
    out[21] = k_igemmp.get_n_step();
    out[22] = k_w4a8_f16.get_m_step();
    out[23] = k_w4a8_f16.get_n_step();
    out[24] = k_w4a8p_f16.get_m_step();
    out[25] = k_w4a8p_f16.get_n_step();
    out[26] = k_w4a8_bf16.get_m_step();
    out[27] = k_w4a8_bf16.get_n_step();
    out[28] = k_w4a8p_bf16.get_m_step();
    out[29] = k_w4a8p_bf16.get_n_step();
    out[30] = k_w4a16f.get_m_step();
    out[31] = k_w4a16f.get_n_step();
    out[32] = k_w4a16fp.get_m_step();
    out[33] = k_w4a16fp.get_n_step();
    out[34] = k_w8dyn.get_m_step();
    out[35] = k_w8dyn.get_n_step();
    out[36] = k_w8dynp.get_m_step();
    out[37] = k_w8dynp.get_n_step();
    out[38] = k_w8dynh.get_m_step();
    out[39] = k_w8dynh.get_n_step();
    out[40] = k_w8dynhp.get_m_step();
    out[41] = k_w8dynhp.get_n_step();
    out[42] = k_convcl.get_m_step();
    out[43] = k_convcl.get_n_step();
    out[44] = k_convclp.get_m_step();
    out[45] = k_convclp.get_n_step();
    out[46] = k_mx1.get_m_step();
    out[47] = k_mx1.get_n_step();
    out[48] = k_mx1p.get_m_step();
    out[49] = k_mx1p.get_n_step();
    out[50] = k_convcf.get_m_step();
    out[51] = k_convcf.get_n_step();
    out[52] = k_convcfp.get_m_step();
    out[53] = k_convcfp.get_n_step();
    out[54] = k_igemmcf.get_m_step();
    out[55] = k_igemmcf.get_n_step();
    out[56] = k_igemmcfp.get_m_step();
    out[57] = k_igemmcfp.get_n_step();
}

/* W4A16 run through the interface struct with _Float16 clamps given as binary16 bits. */
void tqts_run_w4a16(size_t m, size_t n, size_t k, size_t bl, const void *A, size_t lda,
                    const void *B, size_t ldb, const void *scale_b, size_t ldsb, const void *C,
                    size_t ldc, void *D, size_t ldd, const void *bias, uint16_t cmin_bits,
                    uint16_t cmax_bits)
{
    float16_t cmin, cmax;
    memcpy(&cmin, &cmin_bits, 2);
    memcpy(&cmax, &cmax_bits, 2);
    k_w4a16.run_gemm(m, n, k, bl, A, lda, 0, B, ldb, 0, scale_b, ldsb, C, ldc, D, ldd, bias, cmin,
                     cmax);
}

/* Stream-ordered W4A16 for timing. */
void tqts_run_w4a16_async(size_t m, size_t n, size_t k, size_t bl, const void *A, size_t lda,
                          const void *B, size_t ldb, const void *scale_b, size_t ldsb,
                          const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
                          uint16_t cmin_bits, uint16_t cmax_bits, void *stream)
{
    float16_t cmin, cmax;
    memcpy(&cmin, &cmin_bits, 2);
    memcpy(&cmax, &cmax_bits, 2);
    tqt_run_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950_async(m, n, k, bl, A, lda, 0, B, ldb, 0,
                                                                 scale_b, ldsb, C, ldc, D, ldd,
                                                                 bias, cmin, cmax, stream);
}

/* The other four kernel types through their interface structs (synchronous run). */
void tqts_run_clamp(size_t m, size_t n, size_t k, const void *A, size_t lda, const void *B,
                    size_t ldb, const void *C, size_t ldc, void *D, size_t ldd, int32_t cmin,
                    int32_t cmax)
{
    k_clamp.run_gemm(m, n, k, A, lda, 0, B, ldb, 0, C, ldc, D, ldd, cmin, cmax);
}

void tqts_run_w8a8(size_t m, size_t n, size_t k, const void *A, size_t lda, const void *B,
                   size_t ldb, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
                   int8_t cmin, int8_t cmax, const struct tqt_qai8_qai8_qsi8cx_params *params)
{
    k_w8a8.run_gemm(m, n, k, A, lda, 0, B, ldb, 0, C, ldc, D, ldd, bias, cmin, cmax, params);
}

void tqts_run_w4a8(size_t m, size_t n, size_t k, const void *A, size_t lda, const void *B,
                   size_t ldb, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
                   float cmin, float cmax, const struct tqt_qai8dx_qsi4cx_params *params)
{
    k_w4a8.run_gemm(m, n, k, A, lda, 0, B, ldb, 0, C, ldc, D, ldd, bias, cmin, cmax, params);
}

void tqts_run_igemmcl(size_t m, size_t n, const void *input, size_t group_idx, size_t m_idx,
                      const void *B, size_t ldb, void *D, size_t ldd, const void *bias,
                      int8_t cmin, int8_t cmax, const tqt_conv_params *conv,
                      const struct tqt_qai8_qai8_qsi8cx_params *params)
{
    k_igemm.run_igemm(m, n, 0, input, group_idx, m_idx, 0, B, ldb, 0, NULL, 0, D, ldd, bias, cmin,
                      cmax, conv, params);
}

/* Packed W4A16 run (A and B packed by this library's packers) with _Float16 clamps given as
 * binary16 bits: through the interface struct, or stream-ordered when stream != NULL. */
void tqts_run_w4a16p(size_t m, size_t n, size_t k, size_t bl, const void *A_packed, size_t lda,
                     size_t k_idx_a, const void *B_packed, size_t ldb, size_t k_idx_b,
                     const void *scale_b, size_t ldsb, const void *C, size_t ldc, void *D,
                     size_t ldd, const void *bias, uint16_t cmin_bits, uint16_t cmax_bits,
                     void *stream)
{
    float16_t cmin, cmax;
    memcpy(&cmin, &cmin_bits, 2);
    memcpy(&cmax, &cmax_bits, 2);
    if (stream) {
        tqt_run_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950_async(
            m, n, k, bl, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, scale_b, ldsb, C, ldc, D,
            ldd, bias, cmin, cmax, stream);
    } else {
        k_w4a16p.run_gemm(m, n, k, bl, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, scale_b,
                          ldsb, C, ldc, D, ldd, bias, cmin, cmax);
    }
}

/* W4A8 with a 16-bit D (f16 when bf16 == 0, else bf16), the plain (qsi4cxt) or packed (qsi4cxp)
 * type, clamp bounds given as their 16-bit patterns: through the interface struct, or
 * stream-ordered when stream != NULL. */
void tqts_run_w4a8h(int bf16, int packed, size_t m, size_t n, size_t k, const void *A,
                    size_t lda, size_t k_idx_a, const void *B, size_t ldb, size_t k_idx_b,
                    const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
                    uint16_t cmin_bits, uint16_t cmax_bits,
                    const struct tqt_qai8dx_qsi4cx_params *params, void *stream)
{
    if (bf16) {
        bfloat16_t cmin, cmax;
        memcpy(&cmin, &cmin_bits, 2);
        memcpy(&cmax, &cmax_bits, 2);
        if (packed && stream) {
            tqt_run_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950_async(
                m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias, cmin, cmax,
                params, stream);
        } else if (packed) {
            k_w4a8p_bf16.run_gemm(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias,
                                  cmin, cmax, params);
        } else if (stream) {
            tqt_run_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950_async(
                m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias, cmin, cmax,
                params, stream);
        } else {
            k_w4a8_bf16.run_gemm(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias,
                                 cmin, cmax, params);
        }
        return;
    }
    float16_t cmin, cmax;
    memcpy(&cmin, &cmin_bits, 2);
    memcpy(&cmax, &cmax_bits, 2);
    if (packed && stream) {
        tqt_run_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950_async(
            m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias, cmin, cmax, params,
            stream);
    } else if (packed) {
        k_w4a8p_f16.run_gemm(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias, cmin,
                             cmax, params);
    } else if (stream) {
        tqt_run_gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt_mfma_gfx950_async(
            m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias, cmin, cmax, params,
            stream);
    } else {
        k_w4a8_f16.run_gemm(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias, cmin,
                            cmax, params);
    }
}

/* W4A16 with f32 C, bias and D through the interface struct of the plain (qsi4c2t) or packed
 * (qsi4c2p) f32-output type. */
void tqts_run_w4a16f(int packed, size_t m, size_t n, size_t k, size_t bl, const void *A,
                     size_t lda, size_t k_idx_a, const void *B, size_t ldb, size_t k_idx_b,
                     const void *scale_b, size_t ldsb, const void *C, size_t ldc, void *D,
                     size_t ldd, const void *bias, float cmin, float cmax)
{
    if (packed) {
        k_w4a16fp.run_gemm(m, n, k, bl, A, lda, k_idx_a, B, ldb, k_idx_b, scale_b, ldsb, C, ldc, D,
                           ldd, bias, cmin, cmax);
    } else {
        k_w4a16f.run_gemm(m, n, k, bl, A, lda, k_idx_a, B, ldb, k_idx_b, scale_b, ldsb, C, ldc, D,
                          ldd, bias, cmin, cmax);
    }
}

/* qai8dx x qsi8cx with f32 D (clamp bounds as floats) or f16 D (bounds as binary16 bits),
 * plain or packed, through the interface struct; stream-ordered when stream != NULL. */
void tqts_run_w8dyn(int f16, int packed, size_t m, size_t n, size_t k, const void *A, size_t lda,
                    size_t k_idx_a, const void *B, size_t ldb, size_t k_idx_b, void *D,
                    size_t ldd, const void *bias, float cmin, float cmax, uint16_t cmin_bits,
                    uint16_t cmax_bits, const struct tqt_qai8dxp_qsi8cxp_params *params,
                    void *stream)
{
    if (!f16) {
        if (stream) {
            if (packed) {
                tqt_run_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950_async(
                    m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, NULL, 0, D, ldd, bias, cmin, cmax,
                    params, stream);
            } else {
                tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950_async(
                    m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, NULL, 0, D, ldd, bias, cmin, cmax,
                    params, stream);
            }
        } else if (packed) {
            k_w8dynp.run_gemm(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, NULL, 0, D, ldd, bias,
                              cmin, cmax, params);
        } else {
            k_w8dyn.run_gemm(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, NULL, 0, D, ldd, bias, cmin,
                             cmax, params);
        }
        return;
    }
    float16_t hmin, hmax;
    memcpy(&hmin, &cmin_bits, 2);
    memcpy(&hmax, &cmax_bits, 2);
    if (stream) {
        if (packed) {
            tqt_run_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950_async(
                m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, NULL, 0, D, ldd, bias, hmin, hmax,
                params, stream);
        } else {
            tqt_run_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950_async(
                m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, NULL, 0, D, ldd, bias, hmin, hmax,
                params, stream);
        }
    } else if (packed) {
        k_w8dynhp.run_gemm(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, NULL, 0, D, ldd, bias, hmin,
                           hmax, params);
    } else {
        k_w8dynh.run_gemm(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, NULL, 0, D, ldd, bias, hmin,
                          hmax, params);
    }
}

/* convcl through its interface structs: im2col (plain) or fused im2col + pack (packed) of one
 * group, then the convolution GEMM. */
void tqts_run_convcl(int packed, size_t group_idx, const void *activation, void *A_buf,
                     const tqt_conv_params *conv, size_t m, size_t n, size_t k, const void *B,
                     void *D, const void *bias, int8_t cmin, int8_t cmax,
                     const struct tqt_qai8_qai8_qsi8cx_params *params)
{
    if (packed) {
        k_convclp.run_a_im2colpack(group_idx, activation, k, 0, A_buf, conv);
        k_convclp.run_conv(m, n, k, A_buf, k, 0, B, k, 0, NULL, 0, D, n, bias, cmin, cmax, params);
    } else {
        k_convcl.run_im2col(group_idx, activation, A_buf, conv);
        k_convcl.run_conv(m, n, k, A_buf, k, 0, B, k, 0, NULL, 0, D, n, bias, cmin, cmax, params);
    }
}

/* convcf through its interface structs: channel-first im2col [K, N] (plain) or the fused
 * im2col + pack of B and the packing of the weights (packed), then the convolution GEMM. */
void tqts_run_convcf(int packed, size_t group_idx, const void *activation, void *B_buf,
                     const tqt_conv_params *conv, size_t m, size_t n, size_t k, const void *W,
                     void *W_buf, void *D, const void *bias, int8_t cmin, int8_t cmax,
                     const struct tqt_qai8_qsi8dx_qai8_params *params)
{
    if (packed) {
        k_convcfp.run_a_pack(m, k, k, k, 0, W, W_buf);
        k_convcfp.run_b_im2colpack(group_idx, activation, k, 0, B_buf, conv);
        k_convcfp.run_conv(m, n, k, W_buf, k, 0, B_buf, k, 0, NULL, 0, D, n, bias, cmin, cmax,
                           params);
    } else {
        k_convcf.run_im2col(group_idx, activation, B_buf, conv);
        k_convcf.run_conv(m, n, k, W, k, 0, B_buf, n, 0, NULL, 0, D, n, bias, cmin, cmax, params);
    }
}

/* igemmcf through its interface struct (the packed form packs the weights into W_buf first). */
void tqts_run_igemmcf(int packed, size_t m, size_t n, size_t k, const void *input,
                      size_t group_idx, size_t n_idx, const void *W, void *W_buf, void *D,
                      size_t ldd, const void *bias, int8_t cmin, int8_t cmax,
                      const tqt_conv_params *conv,
                      const struct tqt_qai8_qsi8dx_qai8_params *params)
{
    if (packed) {
        k_igemmcfp.run_a_pack(m, k, k, k, 0, W, W_buf);
        k_igemmcfp.run_igemm(m, n, k, input, group_idx, n_idx, 0, W_buf, k, 0, NULL, 0, D, ldd,
                             bias, cmin, cmax, conv, params);
    } else {
        k_igemmcf.run_igemm(m, n, k, input, group_idx, n_idx, 0, W, k, 0, NULL, 0, D, ldd, bias,
                            cmin, cmax, conv, params);
    }
}
