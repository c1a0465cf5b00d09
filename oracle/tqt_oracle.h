/*
 * TEST INFRASTRUCTURE ONLY. CPU restatement of the reference TORQ-Tile semantics for the five
 * kernel types this library implements on gfx950. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only as the checker (or as the timed CPU
 * baseline); the product library never calls it.
 *
 * Every function cites the reference file:line it restates. Plain C99, no half-precision
 * type: f16 values travel as their IEEE binary16 bit patterns (uint16_t).
 */
#ifndef TQT_ORACLE_H
#define TQT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Threads used by the tile loops (OpenMP over m_step x n_step output tiles, the reference's
 * intended threading model, README.md:245-249). 1 = scalar single thread. */
void tqto_set_threads(int n);
int tqto_get_threads(void);

/* IEEE binary16 <-> binary32, round to nearest even on the narrowing side. */
float tqto_f16_to_f32(uint16_t h);
uint16_t tqto_f32_to_f16(float f);

/* bfloat16 <-> binary32: widening is exact; narrowing rounds to nearest even and gives the
 * canonical quiet NaN 0x7fc0 for a NaN (RISC-V vfncvtbf16.f.f.w under the default rounding). */
float tqto_bf16_to_f32(uint16_t b);
uint16_t tqto_f32_to_bf16(float f);

/* src/gemm/gemm_i8_i8/tqt_utils_i8_i8.h:98-132 (+ integer_from_exp :16-91) */
void tqto_quantize_multiplier(double x, int32_t *mult, int32_t *shift);

/* One output of the requantization epilogue, tqt_kernel_gemm_i8_i8_4x1vl_rvv.h:334-408
 * (vmulh, vsra by shift & 31, vadd zp, vnclip x2) then clamp_i8 :231-259.
 * `shift` is the stored shift (= -e - 1, as the run functions store it). */
int8_t tqto_requant_one(int32_t acc, int32_t mult, int32_t shift, int32_t zp, int8_t cmin,
                        int8_t cmax);

/* gemm_clamp_i32_i8_i8 (…/gemm_clamp_i32_i8_i8_4x1vl_rvv.cpp:71-146). B is [k, n]. */
void tqto_gemm_clamp_i32_i8_i8(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                               const int8_t *B, size_t ldb, const int32_t *C, size_t ldc,
                               int32_t *D, size_t ldd, int32_t cmin, int32_t cmax);

/* gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt (…qsi8cxt_4x1vl_rvv.cpp:86-198). B is [n, k].
 * The param struct is passed field by field; scale_b has n entries (1 if quant_channel_b==1). */
void tqto_gemm_qai8_qai8_qsi8cxt(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                                 const int8_t *B, size_t ldb, const int32_t *C, size_t ldc,
                                 int8_t *D, size_t ldd, const int32_t *bias, int8_t cmin,
                                 int8_t cmax, float scale_a, const float *scale_b,
                                 int32_t quant_channel_b, float scale_d, int32_t zero_point_d);

/* The int32 accumulator of the W8A8 path before requantization (C + A.B^T + bias). */
void tqto_gemm_qsi8cxt_acc(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                           const int8_t *B, size_t ldb, const int32_t *C, size_t ldc,
                           const int32_t *bias, int32_t *acc, size_t ldacc);

/* gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt (…qai8dx_qsi4cxt_4x1vl_rvv.cpp:81-198 and
 * tqt_kernel_gemm_i8_i4_4x1vl_rvv.h:77-419). B bytes [n, ldb/2]. */
void tqto_gemm_qai8dx_qsi4cxt_f32(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                                  const uint8_t *B, size_t ldb, const float *C, size_t ldc,
                                  float *D, size_t ldd, const float *bias, float cmin, float cmax,
                                  const float *scale_a, const int32_t *zero_point_a,
                                  const float *scale_b);

/* The f16 / bf16 output siblings gemm_1xnbias_clamp_{f16,bf16}_qai8dx_qsi4cxt
 * (…_4x1vl_rvv.cpp gemm_kernel, epilogue tqt_kernel_gemm_i8_i4_4x1vl_rvv.h:428-628): the f32
 * epilogue above with C and bias widened from the output type, the clamp bounds widened to f32,
 * then one RNE narrowing (a NaN becomes the canonical quiet NaN 0x7e00 / 0x7fc0, as RISC-V
 * conversions give). C, D, bias and the clamps are raw 16-bit patterns; out_bf16 selects bf16. */
void tqto_gemm_qai8dx_qsi4cxt_h16(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                                  const uint8_t *B, size_t ldb, const uint16_t *C, size_t ldc,
                                  uint16_t *D, size_t ldd, const uint16_t *bias, uint16_t cmin,
                                  uint16_t cmax, const float *scale_a,
                                  const int32_t *zero_point_a, const float *scale_b,
                                  int out_bf16);

/* W4A16 with f32 accumulation: the reference test oracle reference_gemm_quantized_weight_mixed
 * (test/common/reference_gemm.cpp:132-179) for TA = TD = f16, evaluated without FMA
 * contraction. A, scale_b, C, bias, D and the clamps are f16 bit patterns. */
void tqto_gemm_f16_qsi4c2t_f32acc(size_t m, size_t n, size_t k, size_t bl, const uint16_t *A,
                                  size_t lda, const uint8_t *B, size_t ldb,
                                  const uint16_t *scale_b, size_t ldsb, const uint16_t *C,
                                  size_t ldc, uint16_t *D, size_t ldd, const uint16_t *bias,
                                  uint16_t cmin, uint16_t cmax);

/* W4A16 with f32 C, bias, clamp bounds and D (test/common/reference_gemm.cpp:132-179 with
 * TA = float16_t, TD = float): the same k loop, no rounding to f16 anywhere. */
void tqto_gemm_f16_qsi4c2t_f32out(size_t m, size_t n, size_t k, size_t bl, const uint16_t *A,
                                  size_t lda, const uint8_t *B, size_t ldb,
                                  const uint16_t *scale_b, size_t ldsb, const float *C, size_t ldc,
                                  float *D, size_t ldd, const float *bias, float cmin, float cmax);

/* binary16 addition rounded once (nearest even), on bit patterns. */
uint16_t tqto_f16_add(uint16_t a, uint16_t b);

/* W8A8 with per-row dynamically quantized A (scale_a[m], zero_point_a[m]) and per-channel
 * symmetric B [n, k] (scale_b[n]), f32 or f16 D (tqt_kernel_gemm_qai8dx_qsi8cx_4x1vl_rvv.h:
 * vwmacc_zp :95-140, dequant_fp32 :145-215, dequant_fp16 :217-330). C is not an input (the
 * reference ignores it). */
void tqto_gemm_qai8dx_qsi8cxt_f32(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                                  const int8_t *B, size_t ldb, float *D, size_t ldd,
                                  const float *bias, float cmin, float cmax,
                                  const float *scale_a, const int32_t *zero_point_a,
                                  const float *scale_b);
void tqto_gemm_qai8dx_qsi8cxt_f16(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                                  const int8_t *B, size_t ldb, uint16_t *D, size_t ldd,
                                  const uint16_t *bias, uint16_t cmin, uint16_t cmax,
                                  const float *scale_a, const int32_t *zero_point_a,
                                  const float *scale_b);

/* W4A16 with the RVV kernel's own numerics (tqt_kernel_gemm_f16_i4_8x2vl_rvv.h:99-717):
 * f16-rounded dequantized weight, sequential f16 FMA over k, f16 bias add, f16 clamp. */
void tqto_gemm_f16_qsi4c2t_rvv(size_t m, size_t n, size_t k, size_t bl, const uint16_t *A,
                               size_t lda, const uint8_t *B, size_t ldb, const uint16_t *scale_b,
                               size_t ldsb, const uint16_t *C, size_t ldc, uint16_t *D,
                               size_t ldd, const uint16_t *bias, uint16_t cmin, uint16_t cmax);

/* Convolution geometry, field-for-field the reference's tqt_conv_params (tqt_conv.h:20-31). */
struct tqto_conv_params
{
    size_t input_shape[3];
    size_t output_shape[3];
    size_t kernel_shape[3];
    size_t stride[3];
    size_t dilation[3];
    size_t pad[3];
    size_t input_channel;
    size_t output_channel;
    size_t groups;
};

/* tqt_im2col_cl<int8_t> (src/common/tqt_conv.h:131-202): [OD*OH*OW, KD*KH*KW*ICpg]. */
void tqto_im2col_cl_i8(size_t group_idx, const int8_t *input, int8_t *col,
                       const struct tqto_conv_params *p);

/* igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt
 * (…igemmcl…qsi8cxt_4x1vl_rvv.cpp:81-286): pixels m_idx .. m_idx+m-1, D addressed absolutely. */
/* Channel-first im2col (src/common/tqt_conv.h:51-119): [ICg*KD*KH*KW, OD*OH*OW] row-major. */
void tqto_im2col_cf_i8(size_t group_idx, const int8_t *input, int8_t *col,
                       const struct tqto_conv_params *p);

/* gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8: A [m, k] per-row scaled weights, B [k, n],
 * C int32 [m, n] (optional), bias int32 [m], per-row requantization, int8 D [m, n]. */
void tqto_gemm_mx1bias_qsi8dx(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                              const int8_t *B, size_t ldb, const int32_t *C, size_t ldc,
                              int8_t *D, size_t ldd, const int32_t *bias, int8_t cmin,
                              int8_t cmax, const float *scale_a, int32_t quant_channel_a,
                              float scale_b, float scale_d, int32_t zp_d);

/* igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8: the mx1bias GEMM on output-pixel columns
 * [n_idx, n_idx + n) of the channel-first im2col of one group. */
void tqto_igemmcf_qsi8dx(size_t m, size_t n, const int8_t *input, size_t group_idx,
                         size_t n_idx, const int8_t *A, size_t lda, int8_t *D, size_t ldd,
                         const int32_t *bias, int8_t cmin, int8_t cmax,
                         const struct tqto_conv_params *p, const float *scale_a,
                         int32_t quant_channel_a, float scale_b, float scale_d, int32_t zp_d);

void tqto_igemmcl_qsi8cxt(size_t m, size_t n, const int8_t *input, size_t group_idx,
                          size_t m_idx, const int8_t *B, size_t ldb, int8_t *D, size_t ldd,
                          const int32_t *bias, int8_t cmin, int8_t cmax,
                          const struct tqto_conv_params *p, float scale_a, const float *scale_b,
                          int32_t quant_channel_b, float scale_d, int32_t zero_point_d);

/* ---- caller-side input preparation used by the reference tests ---- */

/* test/common/test_common.h:232-240 */
int8_t tqto_quantize_i8(float val, float scale, int32_t zp);
/* test/common/test_common.h:268-277 */
int32_t tqto_quantize_bias_i32(float val, float input_scale);
/* test/common/test_common.h:280-290: fused[ch] = bias[ch] - zp * sum(data[ch*cs .. +cs-1]) */
void tqto_fuse_zp_to_bias(int32_t *fused, const int32_t *bias, const int8_t *data, int32_t zp,
                          size_t channels, size_t channel_size);
/* test/common/quantized_gemm_test_runner.h:37-63 */
void tqto_compute_asym_quant_params_i8(const float *data, size_t size, float *scale,
                                       int32_t *zp);
/* test/common/quantized_gemm_test_runner.h:67-86 */
void tqto_compute_sym_quant_params_i8(const float *data, size_t size, float *scale);
/* test/gemm/test_gemm_i8_i4_rvv.cpp:40-77 */
void tqto_quantize_a_per_row_asym(const float *A, size_t m, size_t k, int8_t *A_i8,
                                  float *scale_a, int32_t *zp_a);
/* test/common/quantize_utils.h:34-72 (src and scale are f16 bit patterns) */
void tqto_quantize_fp16_to_int4(size_t n, size_t k, size_t bl, const uint16_t *src,
                                uint8_t *dst, uint16_t *scale, size_t ld_scale);

#ifdef __cplusplus
}
#endif

#endif
