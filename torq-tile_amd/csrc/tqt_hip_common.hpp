// Shared host/device helpers of the gfx950 TORQ-Tile library: error reporting, fragment
// types, the requantization multiplier and epilogue, and launch plumbing.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "tqt_gfx950_common.h"

// ---------------------------------------------------------------------------------------------
// Error convention (reference src/common/tqt_common.h:76-81, TQT_ERROR in a debug build):
// print "file:line message" to stderr and abort.
// ---------------------------------------------------------------------------------------------
#define TQT_FAIL(msg)                                                       \
    do {                                                                    \
        fflush(stdout);                                                     \
        fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, (msg));           \
        abort();                                                            \
    } while (0)

#define TQT_REQUIRE(cond, msg)    \
    do {                          \
        if (!(cond)) {            \
            TQT_FAIL(msg);        \
        }                         \
    } while (0)

#define TQT_HIP_CHECK(expr)                                                             \
    do {                                                                                \
        hipError_t tqt_err_ = (expr);                                                   \
        if (tqt_err_ != hipSuccess) {                                                   \
            fflush(stdout);                                                             \
            fprintf(stderr, "%s:%d HIP error %s: %s\n", __FILE__, __LINE__, #expr,      \
                    hipGetErrorString(tqt_err_));                                       \
            abort();                                                                    \
        }                                                                               \
    } while (0)

namespace tqt {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

inline bool aligned16(const void *p)
{
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

inline hipStream_t as_stream(void *s)
{
    return reinterpret_cast<hipStream_t>(s);
}

// Launch-error check after every kernel launch; the synchronous entry points also wait.
inline void check_launch(const char *where)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fflush(stdout);
        fprintf(stderr, "%s: kernel launch failed: %s\n", where, hipGetErrorString(e));
        abort();
    }
}

inline void finish_sync(hipStream_t stream, const char *where)
{
    check_launch(where);
    hipError_t e = hipStreamSynchronize(stream);
    if (e != hipSuccess) {
        fflush(stdout);
        fprintf(stderr, "%s: kernel execution failed: %s\n", where, hipGetErrorString(e));
        abort();
    }
}

// ---------------------------------------------------------------------------------------------
// Requantization multiplier, evaluated on the device from the same double bits the reference
// uses on the host (reference src/gemm/gemm_i8_i8/tqt_utils_i8_i8.h:16-132): the Q31 fraction
// is the top 30 mantissa bits of x plus the implicit bit, rounded up when the 22 dropped bits
// exceed one half; the exponent follows frexp's [0.5, 1) convention. The run functions then
// store shift = -exponent - 1 (…qsi8cxt_4x1vl_rvv.cpp:158-176).
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ void quantize_multiplier_dev(double x, int32_t &mult, int32_t &shift)
{
    if (x == 0.0) {
        mult = 0;
        shift = 0;
        return;
    }
    const uint64_t u = static_cast<uint64_t>(__double_as_longlong(x));
    const uint64_t sign_mask = 0x8000000000000000ull;
    int64_t q;
    int32_t e;
    if ((u & ~sign_mask) == 0) {
        e = 0;
        q = 0;
    } else {
        const uint32_t exponent_part = static_cast<uint32_t>((u & 0x7ff0000000000000ull) >> 52);
        if (exponent_part == 0x7ffu) {
            e = 0x7fffffff;
            if (u & 0x000fffffffc00000ull) {
                q = 0;
            } else {
                q = (u & sign_mask) ? static_cast<int64_t>(0x8000000000000000ull)
                                    : static_cast<int64_t>(0x7fffffffffffffffll);
            }
        } else {
            e = static_cast<int32_t>(exponent_part - 1023u) + 1;
            q = 0x40000000ll + static_cast<int64_t>((u & 0x000fffffffc00000ull) >> 22);
            if ((u & 0x003fffffull) > 0x00200000ull) {
                q += 1;
            }
            if (u & sign_mask) {
                q = -q;
            }
        }
    }
    if (q == (1ll << 31)) {
        q /= 2;
        e += 1;
    }
    if (e < -31) {
        e = 0;
        q = 0;
    }
    mult = static_cast<int32_t>(q);
    shift = -e - 1;
}

// Column multiplier exactly as the run functions compute it: double(scale_a) * double(scale_b)
// / double(scale_d), column 0 reused for every column when quant_channel_b == 1.
__device__ __forceinline__ void column_multiplier_dev(float scale_a, const float *scale_b,
                                                      int32_t quant_channel_b, float scale_d,
                                                      int col, int32_t &mult, int32_t &shift)
{
    const int src = (quant_channel_b == 1) ? 0 : col;
    const double real = static_cast<double>(scale_a) * static_cast<double>(scale_b[src]) /
                        static_cast<double>(scale_d);
    quantize_multiplier_dev(real, mult, shift);
}

// One output of the requantization epilogue (reference tqt_kernel_gemm_i8_i8_4x1vl_rvv.h:
// requantize_1xn :334-408 = vmulh, vsra by shift & 31, vadd zp, vnclip to i16 then i8;
// clamp_i8 :231-259 = vmax then vmin).
__device__ __forceinline__ int8_t requant_dev(int32_t acc, int32_t mult, int32_t shift,
                                              int32_t zp, int32_t cmin, int32_t cmax)
{
    int32_t y = __mulhi(acc, mult);  // high 32 bits of the signed 64-bit product
    y = y >> (shift & 31);
    y = static_cast<int32_t>(static_cast<uint32_t>(y) + static_cast<uint32_t>(zp));
    y = y < -128 ? -128 : (y > 127 ? 127 : y);
    y = y < cmin ? cmin : y;
    y = y > cmax ? cmax : y;
    return static_cast<int8_t>(y);
}

}  // namespace tqt
