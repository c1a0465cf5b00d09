/*
 * Micro-kernel type igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8, variant mfma_gfx950.
 *
 * Implicit-GEMM convolution, channel-first: D [m, pixels] int8 = the mx1bias GEMM of the
 * weights A [m = OC_per_group, K] (K = IC_per_group*KD*KH*KW in (ic, kd, kh, kw) order) with the
 * channel-first im2col of one group of the NCDHW input, gathered on the fly, for the output
 * pixels [n_idx, n_idx + n); row i of D is written at D + i * ldd + n_idx. C is not read (the
 * reference ignores it). The requantization is the per-row one of
 * gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8.
 * The weights are pre-packed by run_a_pack (the A layout of
 * gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp).
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
 * Drop-in for src/conv/igemm_i8_i8/igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8/tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_1vlx4_rvv.h
 * (the line of each declaration is given below). Every pointer, source and packed
 * buffers included, is device-accessible; the packers run on the GPU and, like the runs,
 * return with their output written; the _async forms (no counterpart in the reference)
 * enqueue on a hipStream_t instead. Params structs and scalars stay on the host.
 */
#ifndef TQT_IGEMMCF_MX1BIAS_REQI32TOI8_CLAMP_QAI8_QSI8DXP_QAI8_MFMA_GFX950_H
#define TQT_IGEMMCF_MX1BIAS_REQI32TOI8_CLAMP_QAI8_QSI8DXP_QAI8_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference :34 */
size_t tqt_get_m_step_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(void);
/* reference :35 */
size_t tqt_get_n_step_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(void);
/* reference :37 */
size_t tqt_get_a_packed_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(
    size_t m_idx, size_t k_idx, size_t lda, size_t actual_m);
/* reference :39 */
size_t tqt_get_c_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc);
/* reference :42 */
size_t tqt_get_bias_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(
    size_t m_idx);
/* reference :44 */
size_t tqt_get_d_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd);
/* reference :47 */
size_t tqt_get_d_size_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(
    size_t m, size_t n);
/* reference :49 */
size_t tqt_get_a_packed_size_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(
    size_t m, size_t k);
/* reference :53 */
void tqt_run_a_pack_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(
    size_t m, size_t k, size_t ldw, size_t ldw_packed, size_t k_idx, const void *weight,
    void *weight_packed);
/* stream-ordered form */
void tqt_run_a_pack_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950_async(
    size_t m, size_t k, size_t ldw, size_t ldw_packed, size_t k_idx, const void *weight,
    void *weight_packed, void *stream);
/* reference :78 */
void tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *input, size_t group_idx, size_t n_idx, size_t k_idx_b,
    const void *A_packed, size_t lda, size_t k_idx_a, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const tqt_conv_params *conv_params, const struct tqt_qai8_qsi8dx_qai8_params *quant_params);
/* stream-ordered form */
void tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *input, size_t group_idx, size_t n_idx, size_t k_idx_b,
    const void *A_packed, size_t lda, size_t k_idx_a, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const tqt_conv_params *conv_params, const struct tqt_qai8_qsi8dx_qai8_params *quant_params,
    void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
