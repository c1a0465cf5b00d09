// TEST INFRASTRUCTURE ONLY. C-linkage entry points onto the reference's own portable
// test-side code, which oracle/Makefile compiles from where it lies under the reference tree
// (test/common/reference_gemm.cpp, reference_conv.cpp, data_generator.cpp) together with the
// header-only helpers included below. Nothing here re-implements reference behaviour: each
// function forwards to the reference symbol named in its comment. Used only to pin the CPU
// restatement in oracle/tqt_oracle.c and to write the golden fixtures under tests/golden/.
#include <cstddef>
#include <cstdint>

#include "src/common/tqt_common.h"
#include "src/common/tqt_conv.h"
#include "src/gemm/gemm_i8_i8/tqt_utils_i8_i8.h"
#include "test/common/data_generator.h"
#include "test/common/quantize_utils.h"
#include "test/common/reference_conv.h"
#include "test/common/reference_gemm.h"
#include "test/common/test_common.h"

using namespace torq_tile::test;

extern "C" {

// src/gemm/gemm_i8_i8/tqt_utils_i8_i8.h:98-132
void tqtr_quantize_multiplier(double x, int32_t *mult, int32_t *shift)
{
    tqt_quantize_multiplier(x, mult, shift);
}

// test/common/reference_gemm.cpp:92-126 (b_layout 0 = [k, n] row-major, 1 = [n, k])
void tqtr_reference_gemm_i32_i8(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                                const int8_t *B, size_t ldb, int b_transposed, const int32_t *C,
                                size_t ldc, int32_t *D, size_t ldd, int32_t cmin, int32_t cmax)
{
    reference_gemm_i32_i8(m, n, k, A, lda, B, ldb,
                          b_transposed ? BLayout::kTransposed : BLayout::kRowMajor, C, ldc, D, ldd,
                          cmin, cmax);
}

// test/common/reference_gemm.cpp:17-67, TA = TD = float, 1xN bias
void tqtr_reference_gemm_f32(size_t m, size_t n, size_t k, const float *A, size_t lda,
                             const float *B, size_t ldb, int b_transposed, const float *C,
                             size_t ldc, float *D, size_t ldd, const float *bias, float cmin,
                             float cmax)
{
    reference_gemm<float, float>(m, n, k, A, lda, B, ldb,
                                 b_transposed ? BLayout::kTransposed : BLayout::kRowMajor, C, ldc,
                                 D, ldd, bias, bias ? BiasMode::k1xN : BiasMode::kNone, cmin,
                                 cmax);
}

// test/common/reference_gemm.cpp:131-179, TA = TD = float16_t (values as binary16 bits)
void tqtr_reference_gemm_qw_mixed_f16(size_t m, size_t n, size_t k, size_t bl,
                                      const uint16_t *A, size_t lda, const uint8_t *B, size_t ldb,
                                      const uint16_t *scale_b, size_t ldsb, const uint16_t *C,
                                      size_t ldc, uint16_t *D, size_t ldd, const uint16_t *bias,
                                      uint16_t cmin_bits, uint16_t cmax_bits)
{
    float16_t cmin, cmax;
    static_assert(sizeof(float16_t) == 2, "binary16");
    __builtin_memcpy(&cmin, &cmin_bits, 2);
    __builtin_memcpy(&cmax, &cmax_bits, 2);
    reference_gemm_quantized_weight_mixed<float16_t, float16_t>(
        m, n, k, bl, reinterpret_cast<const float16_t *>(A), lda, B, ldb,
        reinterpret_cast<const float16_t *>(scale_b), ldsb,
        reinterpret_cast<const float16_t *>(C), ldc, reinterpret_cast<float16_t *>(D), ldd,
        reinterpret_cast<const float16_t *>(bias), bias ? BiasMode::k1xN : BiasMode::kNone, cmin,
        cmax);
}

// test/common/reference_gemm.cpp:131-179, TA = float16_t, TD = float (A, scale_b as binary16
// bits)
void tqtr_reference_gemm_qw_mixed_f16_f32(size_t m, size_t n, size_t k, size_t bl,
                                          const uint16_t *A, size_t lda, const uint8_t *B,
                                          size_t ldb, const uint16_t *scale_b, size_t ldsb,
                                          const float *C, size_t ldc, float *D, size_t ldd,
                                          const float *bias, float cmin, float cmax)
{
    reference_gemm_quantized_weight_mixed<float16_t, float>(
        m, n, k, bl, reinterpret_cast<const float16_t *>(A), lda, B, ldb,
        reinterpret_cast<const float16_t *>(scale_b), ldsb, C, ldc, D, ldd, bias,
        bias ? BiasMode::k1xN : BiasMode::kNone, cmin, cmax);
}

// test/common/reference_conv.cpp:17-127, T = float, channel-last
void tqtr_reference_conv_cl_f32(size_t group_idx, const float *activation, const float *weight,
                                const float *bias, float *output, const tqt_conv_params *params,
                                float cmin, float cmax)
{
    reference_conv<float>(group_idx, activation, weight, bias, output, params,
                          ConvLayout::kChannelLast, cmin, cmax);
}

// src/common/tqt_conv.h:131-202
void tqtr_im2col_cl_i8(size_t group_idx, const int8_t *activation, int8_t *col,
                       const tqt_conv_params *params)
{
    tqt_im2col_cl<int8_t>(group_idx, activation, col, params);
}

// src/common/tqt_conv.h:51-119
void tqtr_im2col_cf_i8(size_t group_idx, const int8_t *activation, int8_t *col,
                       const tqt_conv_params *params)
{
    tqt_im2col_cf<int8_t>(group_idx, activation, col, params);
}

// test/common/data_generator.{h,cpp}: UniformRandomGenerator<T>(low, high, seed).fill_matrix
void tqtr_fill_uniform_f32(float low, float high, uint32_t seed, float *data, size_t rows,
                           size_t cols)
{
    UniformRandomGenerator<float> g(low, high, seed);
    g.fill_matrix(data, rows, cols);
}

void tqtr_fill_uniform_f16(float low, float high, uint32_t seed, uint16_t *data, size_t rows,
                           size_t cols)
{
    UniformRandomGenerator<float16_t> g(low, high, seed);
    g.fill_matrix(reinterpret_cast<float16_t *>(data), rows, cols);
}

void tqtr_fill_uniform_i8(int8_t low, int8_t high, uint32_t seed, int8_t *data, size_t rows,
                          size_t cols)
{
    UniformRandomGenerator<int8_t> g(low, high, seed);
    g.fill_matrix(data, rows, cols);
}

void tqtr_fill_uniform_i32(int32_t low, int32_t high, uint32_t seed, int32_t *data, size_t rows,
                           size_t cols)
{
    UniformRandomGenerator<int32_t> g(low, high, seed);
    g.fill_matrix(data, rows, cols);
}

// test/common/test_common.h:232-240
int8_t tqtr_quantize_i8(float val, float scale, int32_t zp)
{
    return quantize_i8(val, scale, zp);
}

// test/common/test_common.h:268-277
int32_t tqtr_quantize_bias_i32(float val, float input_scale)
{
    return quantize_bias_i32(val, input_scale);
}

// test/common/test_common.h:280-290
void tqtr_fuse_zp_to_bias(int32_t *fused, const int32_t *bias, const int8_t *data, int32_t zp,
                          size_t channels, size_t channel_size)
{
    fuse_zp_to_bias(fused, bias, data, zp, channels, channel_size);
}

// test/common/quantize_utils.h:34-72
void tqtr_quantize_fp16_to_int4(size_t n, size_t k, size_t bl, const uint16_t *src, uint8_t *dst,
                                uint16_t *scale, size_t ld_scale)
{
    quantize_fp16_to_int4(n, k, bl, reinterpret_cast<const float16_t *>(src), dst,
                          reinterpret_cast<float16_t *>(scale), ld_scale);
}

}  // extern "C"
