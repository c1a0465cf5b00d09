/*
 * Shared types of the gfx950 (MI355X) TORQ-Tile quantized micro-kernel library.
 *
 * The parameter structs below keep the reference's field order and types so that a caller
 * built against the reference headers passes the same bytes:
 *   - struct tqt_qai8_qai8_qsi8cx_params  : reference src/gemm/gemm_i8_i8/tqt_params_i8_i8.h:16-24
 *   - struct tqt_qai8dx_qsi4cx_params     : reference src/gemm/gemm_i8_i4/tqt_params_i8_i4.h:23-28
 *   - struct tqt_qai8dxp_qsi8cxp_params   : reference src/gemm/gemm_i8_i8/tqt_params_i8_i8.h:45-50
 *   - struct tqt_qai8_qsi8dx_qai8_params  : reference src/gemm/gemm_i8_i8/tqt_params_i8_i8.h:28-36
 *   - struct tqt_conv_params              : reference src/common/tqt_conv.h:20-31
 *   - float16_t, bfloat16_t               : reference src/common/tqt_common.h:27-28
 *
 * Memory contract of every tqt_run_* in this library: A, B, C, D, bias, and the arrays the
 * param structs point to (scale_a, zero_point_a, scale_b) are device-accessible pointers
 * (hipMalloc, hipMallocManaged or host-pinned-and-mapped memory). The param structs
 * themselves and all scalars are read on the host and copied into kernel arguments.
 *
 * Error convention (reference src/common/tqt_common.h:61-119): the run functions return
 * void. A NULL params pointer makes run_* return without touching D (as the reference does).
 * Violated preconditions and HIP launch failures print "file:line message" to stderr and
 * abort the process, which is what TQT_ERROR does in the reference's debug build.
 */
#ifndef TQT_GFX950_COMMON_H
#define TQT_GFX950_COMMON_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef TQT_FLOAT16_T_DEFINED
#define TQT_FLOAT16_T_DEFINED
typedef _Float16 float16_t;
#endif

/* reference src/common/tqt_common.h:27 */
#ifndef TQT_BFLOAT16_T_DEFINED
#define TQT_BFLOAT16_T_DEFINED
typedef __bf16 bfloat16_t;
#endif

/* Quantization parameters for qai8 (A) x qsi8cx (B) -> qai8 (D).
 * zero_point_a is not read by the kernels: callers fold it into the int32 bias
 * (reference test/common/test_common.h:280-290). */
struct tqt_qai8_qai8_qsi8cx_params
{
    float scale_a;
    int32_t zero_point_a;
    float *scale_b;
    int32_t quant_channel_b;
    float scale_d;
    int32_t zero_point_d;
};

/* Quantization parameters for qai8dx (A, per-row asymmetric) x qsi4cx (B, per-channel
 * symmetric int4) -> float D. scale_a/zero_point_a have m entries, scale_b has n entries. */
struct tqt_qai8dx_qsi4cx_params
{
    const float *scale_a;
    const int32_t *zero_point_a;
    const float *scale_b;
};

/* Quantization parameters for qai8dx (A, per-row asymmetric int8) x qsi8cx (B, per-channel
 * symmetric int8) -> f32 / f16 D, plain and packed. scale_a/zero_point_a have m entries,
 * scale_b has n entries. */
struct tqt_qai8dxp_qsi8cxp_params
{
    float *scale_a;
    int32_t *zero_point_a;
    float *scale_b;
};

/* Quantization parameters for qsi8dx (A = weights, per-row symmetric int8) x qai8 (B =
 * activations, per-tensor asymmetric) -> qai8 D with an Mx1 (per-row) bias. scale_a has m
 * entries (or 1 when quant_channel_a == 1). zero_point_b is not read by the kernels: callers fold
 * it into the int32 bias. */
struct tqt_qai8_qsi8dx_qai8_params
{
    float *scale_a;
    int32_t quant_channel_a;
    float scale_b;
    int32_t zero_point_b;
    float scale_d;
    int32_t zero_point_d;
};

/* 3D convolution geometry (1D/2D set the higher dims to 1). The batch of an NDHWC input
 * can ride in the depth dimension (kernel_d = 1, stride_d = 1, pad_d = 0). */
struct tqt_conv_params
{
    size_t input_shape[3];  /* {input_d, input_h, input_w} */
    size_t output_shape[3]; /* {output_d, output_h, output_w} (caller pre-computes) */
    size_t kernel_shape[3]; /* {kernel_d, kernel_h, kernel_w} */
    size_t stride[3];       /* {stride_d, stride_h, stride_w} */
    size_t dilation[3];     /* {dilation_d, dilation_h, dilation_w} */
    size_t pad[3];          /* {pad_d, pad_h, pad_w} */
    size_t input_channel;
    size_t output_channel;
    size_t groups;
};
typedef struct tqt_conv_params tqt_conv_params;

/* Library identification: returns the offload target the device code was built for
 * ("gfx950"). Has no counterpart in the reference (which is a source-only library). */
const char *tqt_gfx950_target(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* TQT_GFX950_COMMON_H */
