/*
 * Micro-kernel type gemm_1xnbias_clamp_f16_f16p_qsi4c2p, variant mfma_gfx950.
 *
 * Computes D = clamp(C + A * dequant(B) + bias) as gemm_1xnbias_clamp_f16_f16_qsi4c2t does
 * (block scales scale_b [n, ldsb] f16, one per bl k; f16 D), with A pre-packed f16 and B
 * pre-packed int4 ([n, k/2] bytes; ldb and k_idx count int4 elements). scale_b is not packed.
 * B's packed rows are additionally fragment-ordered: inside every whole 64-byte group (four
 * 32-k blocks) of a row the 16-byte chunk c holds 4-byte slice c of each of the four blocks,
 * the operand lane group c of the f16 MFMA takes, so the kernel reads it without a shuffle.
 *
 * Packed layout (this build's; the reference's is its own [m/MR, k, MR] / [n/vl, k, vl]):
 * rows (m of A, n of B) form panels of m_step / n_step rows. Panel p holds rows
 * [p*step, p*step + w), w = min(step, rows - p*step), and starts at element p*step*ld_packed,
 * moved back by k_idx*(step - w) elements when a panel after the first is narrower (the
 * reference's tail rule, tqt_gemm_pack_rvv.h:314-318). Inside a panel each row is cut into
 * 16-byte chunks stored chunk-major: chunk c of local row r at byte 16*c*w + r*cw,
 * cw = min(16, row bytes - 16*c). A chunk is one MFMA lane fragment (8 f16 values or
 * 32 int4 values); 16 channels x 16 bytes make one lane group's contiguous load.
 * The packed_offset getters keep the reference's formula (idx*ld + k_idx*min(actual, step))
 * elements; it addresses element (idx, k_idx) of a full-K packing when k_idx is a whole number
 * of chunks, and the start of a k_idx sub-buffer packed with that k_idx in any case. Packed
 * sizes equal the unpacked ones.
 *
 * Drop-in for src/gemm/gemm_f16_i4/gemm_1xnbias_clamp_f16_f16p_qsi4c2p/tqt_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_8x2vl_rvv.h
 * (the line of each declaration is given below). Every pointer, source and packed
 * buffers included, is device-accessible; the packers run on the GPU and, like the runs,
 * return with their output written; the _async forms (no counterpart in the reference)
 * enqueue on a hipStream_t instead. Params structs and scalars stay on the host.
 */
#ifndef TQT_GEMM_1XNBIAS_CLAMP_F16_F16P_QSI4C2P_MFMA_GFX950_H
#define TQT_GEMM_1XNBIAS_CLAMP_F16_F16P_QSI4C2P_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference :24 */
size_t tqt_get_m_step_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(void);
/* reference :26 */
size_t tqt_get_n_step_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(void);
/* reference :29 */
size_t tqt_get_a_packed_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(
    size_t m_idx, size_t k_idx, size_t lda, size_t actual_m);
/* reference :36 */
size_t tqt_get_b_packed_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb, size_t actual_n);
/* reference :42 */
size_t tqt_get_scale_b_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(
    size_t n_idx, size_t b_idx, size_t ldsb);
/* reference :46 */
size_t tqt_get_c_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc);
/* reference :49 */
size_t tqt_get_bias_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(size_t n_idx);
/* reference :51 */
size_t tqt_get_d_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd);
/* reference :54 */
size_t tqt_get_d_size_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(size_t m, size_t n);
/* reference :57 */
size_t tqt_get_a_packed_size_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(size_t m, size_t k);
/* reference :60 */
size_t tqt_get_b_packed_size_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(size_t n, size_t k);
/* reference :64 */
void tqt_run_a_pack_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(
    size_t m, size_t k, size_t lda, size_t lda_packed, size_t k_idx, const void *A, void *A_packed);
/* stream-ordered form */
void tqt_run_a_pack_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950_async(
    size_t m, size_t k, size_t lda, size_t lda_packed, size_t k_idx, const void *A, void *A_packed,
    void *stream);
/* reference :70 */
void tqt_run_bt_pack_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed);
/* stream-ordered form */
void tqt_run_bt_pack_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950_async(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed,
    void *stream);
/* reference :97 */
void tqt_run_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(
    size_t m, size_t n, size_t k, size_t bl, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *scale_b, size_t ldsb,
    const void *C, size_t ldc, void *D, size_t ldd, const void *bias, float16_t clamp_min,
    float16_t clamp_max);
/* stream-ordered form */
void tqt_run_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950_async(
    size_t m, size_t n, size_t k, size_t bl, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *scale_b, size_t ldsb,
    const void *C, size_t ldc, void *D, size_t ldd, const void *bias, float16_t clamp_min,
    float16_t clamp_max, void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
