/*
 * Micro-kernel type gemm_1xnbias_clamp_f16_f16_qsi4c2t (W4A16), variant mfma_gfx950.
 *
 * A f16 [m, k] row-major. B int4 [n, k] stored as [n, k/2] bytes (low nibble = even k,
 * value = nibble - 8) with one f16 scale per (n, block of bl consecutive k): scale_b [n, ldsb].
 * C f16 [m, n] and bias f16 [n] are optional. D f16 [m, n]. k % bl == 0, bl even >= 2.
 *
 * Numerics: every product a * (q - 8) * s is formed exactly and accumulated in f32; C, bias
 * and the clamp are applied in f32 and the result is rounded once to f16 (round to nearest
 * even). This is the f32-accumulating semantics of the reference's own test oracle
 * (test/common/reference_gemm.cpp:132-179); the RVV kernel instead rounds each dequantized
 * weight to f16 and accumulates in f16 (tqt_kernel_gemm_f16_i4_8x2vl_rvv.h:220-231, 365-478),
 * which the reference test accepts within 1.0 absolute of that oracle.
 *
 * Drop-in for src/gemm/gemm_f16_i4/gemm_1xnbias_clamp_f16_f16_qsi4c2t/
 * tqt_gemm_1xnbias_clamp_f16_f16_qsi4c2t_8x2vl_rvv.h (get_* and run at :24-78 of the header,
 * offsets at tqt_gemm_1xnbias_clamp_f16_f16_qsi4c2t_8x2vl_rvv.cpp:25-86).
 */
#ifndef TQT_GEMM_1XNBIAS_CLAMP_F16_F16_QSI4C2T_MFMA_GFX950_H
#define TQT_GEMM_1XNBIAS_CLAMP_F16_F16_QSI4C2T_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference ..._8x2vl_rvv.cpp:25 / :30 */
size_t tqt_get_m_step_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(void);
size_t tqt_get_n_step_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(void);
/* reference ..._8x2vl_rvv.cpp:35: (m_idx * lda + k_idx) * 2 bytes */
size_t tqt_get_a_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(size_t m_idx,
                                                                       size_t k_idx, size_t lda,
                                                                       size_t bl);
/* reference ..._8x2vl_rvv.cpp:44: n_idx * (ldb / 2) + k_idx / 2 bytes */
size_t tqt_get_b_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(size_t n_idx,
                                                                       size_t k_idx, size_t ldb,
                                                                       size_t bl);
/* reference ..._8x2vl_rvv.cpp:53: (n_idx * ldsb + b_idx) * 2 bytes */
size_t tqt_get_scale_b_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(size_t n_idx,
                                                                             size_t b_idx,
                                                                             size_t ldsb);
/* reference ..._8x2vl_rvv.cpp:61: (m_idx * ldc + n_idx) * 2 bytes */
size_t tqt_get_c_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(size_t m_idx,
                                                                       size_t n_idx, size_t ldc);
/* reference ..._8x2vl_rvv.cpp:69: n_idx * 2 bytes */
size_t tqt_get_bias_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(size_t n_idx);
/* reference ..._8x2vl_rvv.cpp:75: (m_idx * ldd + n_idx) * 2 bytes */
size_t tqt_get_d_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(size_t m_idx,
                                                                       size_t n_idx, size_t ldd);
/* reference ..._8x2vl_rvv.cpp:83: m * n * 2 bytes */
size_t tqt_get_d_size_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(size_t m, size_t n);

/* reference header ..._8x2vl_rvv.h:75-78 (cpp :183-186) */
void tqt_run_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(
    size_t m, size_t n, size_t k, size_t bl, const void *A, size_t lda, size_t k_idx_a,
    const void *B, size_t ldb, size_t k_idx_b, const void *scale_b, size_t ldsb, const void *C,
    size_t ldc, void *D, size_t ldd, const void *bias, float16_t clamp_min, float16_t clamp_max);

/* Stream-ordered form (no counterpart in the reference). */
void tqt_run_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950_async(
    size_t m, size_t n, size_t k, size_t bl, const void *A, size_t lda, size_t k_idx_a,
    const void *B, size_t ldb, size_t k_idx_b, const void *scale_b, size_t ldsb, const void *C,
    size_t ldc, void *D, size_t ldd, const void *bias, float16_t clamp_min, float16_t clamp_max,
    void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
