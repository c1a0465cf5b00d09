/*
 * Micro-kernel type gemm_clamp_i32_i8_i8, variant mfma_gfx950.
 *
 * Computes D = clamp(C + A * B, clamp_min, clamp_max) with A int8 [m, k] row-major,
 * B int8 [k, n] row-major, C int32 [m, n] (optional, NULL allowed) and D int32 [m, n].
 * The clamp applies max(clamp_min) first, then min(clamp_max).
 *
 * Drop-in for the reference variant declared at
 *   src/gemm/gemm_i8_i8/gemm_clamp_i32_i8_i8/tqt_gemm_clamp_i32_i8_i8_4x1vl_rvv.h:29-108
 * with the same argument lists, offsets in bytes, and the same interface struct
 * (tqt_gemm_clamp_i32_i8_i8_interface.h). m_step/n_step report the gfx950 macro-tile; run
 * accepts any m, n, k and any (m_idx, n_idx) sub-tile, like the reference.
 * All pointers are device-accessible (see tqt_gfx950_common.h). run returns with D written.
 */
#ifndef TQT_GEMM_CLAMP_I32_I8_I8_MFMA_GFX950_H
#define TQT_GEMM_CLAMP_I32_I8_I8_MFMA_GFX950_H

#include "tqt_gfx950_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference ..._4x1vl_rvv.h:29 (m_step) / :36 (n_step) */
size_t tqt_get_m_step_gemm_clamp_i32_i8_i8_mfma_gfx950(void);
size_t tqt_get_n_step_gemm_clamp_i32_i8_i8_mfma_gfx950(void);
/* reference ..._4x1vl_rvv.h:45: (m_idx * lda + k_idx) bytes */
size_t tqt_get_a_offset_gemm_clamp_i32_i8_i8_mfma_gfx950(size_t m_idx, size_t k_idx, size_t lda);
/* reference ..._4x1vl_rvv.h:54: (k_idx * ldb + n_idx) bytes */
size_t tqt_get_b_offset_gemm_clamp_i32_i8_i8_mfma_gfx950(size_t n_idx, size_t k_idx, size_t ldb);
/* reference ..._4x1vl_rvv.h:63: (m_idx * ldc + n_idx) * 4 bytes */
size_t tqt_get_c_offset_gemm_clamp_i32_i8_i8_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldc);
/* reference ..._4x1vl_rvv.h:72: (m_idx * ldd + n_idx) * 4 bytes */
size_t tqt_get_d_offset_gemm_clamp_i32_i8_i8_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldd);
/* reference ..._4x1vl_rvv.h:80: m * n * 4 bytes */
size_t tqt_get_d_size_gemm_clamp_i32_i8_i8_mfma_gfx950(size_t m, size_t n);

/* reference ..._4x1vl_rvv.h:105-108 (k_idx_a / k_idx_b are unused, as in the reference) */
void tqt_run_gemm_clamp_i32_i8_i8_mfma_gfx950(size_t m, size_t n, size_t k, const void *A,
                                              size_t lda, size_t k_idx_a, const void *B,
                                              size_t ldb, size_t k_idx_b, const void *C,
                                              size_t ldc, void *D, size_t ldd, int32_t clamp_min,
                                              int32_t clamp_max);

/* Stream-ordered form (no counterpart in the reference): same arguments plus a hipStream_t
 * passed as void*; enqueues the work and returns without waiting. */
void tqt_run_gemm_clamp_i32_i8_i8_mfma_gfx950_async(size_t m, size_t n, size_t k, const void *A,
                                                    size_t lda, size_t k_idx_a, const void *B,
                                                    size_t ldb, size_t k_idx_b, const void *C,
                                                    size_t ldc, void *D, size_t ldd,
                                                    int32_t clamp_min, int32_t clamp_max,
                                                    void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif
