// Dynamic per-row asymmetric int8 quantization of f32 activations (the qai8dx operand of the
// W4A8 kernels) on gfx950: the step before the W4A8 GEMV in a decode loop. The reference has it
// only as test-side code (test/gemm/test_gemm_i8_i4_rvv.cpp:40-77, quantize_i8 from
// test/common/test_common.h:232-240); this is its GPU form, bit-exact:
//   fmax = max(0, max_k x), fmin = min(0, min_k x), s = (fmax - fmin) / 255
//   s == 0: scale 1, zero point 0, every q = 0
//   else zp = clamp(rne(-128 - fmin / s), -128, 127), q = clamp(rne(x / s) + zp, -128, 127)
// with correctly rounded divisions and no fused multiply-add (the library is built with
// -ffp-contract=off). min and max are exact, so their reduction order does not matter.
//
// One workgroup of 256 threads per row: a min/max pass over the row (float4 loads when the row
// is 16-byte aligned), a wave-then-workgroup reduction, then a second pass that quantizes (the
// row is re-read from cache) and writes 4 bytes per thread and step.
#include "tqt_hip_common.hpp"
#include "tqt_quantize_qai8dx_gfx950.h"

#include <cfloat>

namespace tqt {
namespace {

constexpr int kQThreads = 256;
constexpr int kQCache = 4;  // float4 per thread kept in registers (rows of k <= 4096)

__device__ __forceinline__ int8_t quantize_one(float x, float s, float zpf)
{
    return qai8dx_quantize(x, s, zpf);
}

__global__ __launch_bounds__(kQThreads) void quantize_qai8dx_kernel(
    int k, const float *A, long long lda, int8_t *Q, long long ldq, float *scale_a,
    int32_t *zp_a, bool vec)
{
    __shared__ float s_min[kQThreads / 64], s_max[kQThreads / 64];
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const float *x = A + static_cast<long long>(row) * lda;
    int8_t *q = Q + static_cast<long long>(row) * ldq;

    float lo = FLT_MAX, hi = -FLT_MAX;
    const int k4 = vec ? k / 4 : 0;
    // Rows of up to kQCache * kQThreads float4 stay in registers between the min/max pass and
    // the quantizing pass (all of their loads in flight at once, no second read of the row).
    const bool cached = k4 > 0 && k4 <= kQCache * kQThreads;  // k4 > 0: vec and x[0..3] valid
    f32x4 cache[kQCache];
    if (cached) {
#pragma unroll
        for (int c = 0; c < kQCache; ++c) {
            const int i = tid + c * kQThreads;
            cache[c] = reinterpret_cast<const f32x4 *>(x)[i < k4 ? i : 0];
        }
#pragma unroll
        for (int c = 0; c < kQCache; ++c) {
            if (tid + c * kQThreads < k4) {
                const f32x4 v = cache[c];
                lo = fminf(lo, fminf(fminf(v[0], v[1]), fminf(v[2], v[3])));
                hi = fmaxf(hi, fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
            }
        }
    } else {
        for (int i = tid; i < k4; i += kQThreads) {
            const f32x4 v = reinterpret_cast<const f32x4 *>(x)[i];
            lo = fminf(lo, fminf(fminf(v[0], v[1]), fminf(v[2], v[3])));
            hi = fmaxf(hi, fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
        }
    }
    for (int i = 4 * k4 + tid; i < k; i += kQThreads) {
        lo = fminf(lo, x[i]);
        hi = fmaxf(hi, x[i]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        lo = fminf(lo, __shfl_xor(lo, off));
        hi = fmaxf(hi, __shfl_xor(hi, off));
    }
    if ((tid & 63) == 0) {
        s_min[tid >> 6] = lo;
        s_max[tid >> 6] = hi;
    }
    __syncthreads();
    lo = s_min[0];
    hi = s_max[0];
#pragma unroll
    for (int w = 1; w < kQThreads / 64; ++w) {
        lo = fminf(lo, s_min[w]);
        hi = fmaxf(hi, s_max[w]);
    }
    float s;
    int32_t zp;
    if (!qai8dx_row_params(lo, hi, s, zp)) {
        if (tid == 0) {
            scale_a[row] = 1.0f;
            zp_a[row] = 0;
        }
        for (int i = tid; i < k; i += kQThreads) {
            q[i] = 0;
        }
        return;
    }
    if (tid == 0) {
        scale_a[row] = s;
        zp_a[row] = zp;
    }
    const float zpf = static_cast<float>(zp);
    if (cached) {
#pragma unroll
        for (int c = 0; c < kQCache; ++c) {
            const int i = tid + c * kQThreads;
            if (i < k4) {
                const f32x4 v = cache[c];
                const uint32_t b0 = static_cast<uint8_t>(quantize_one(v[0], s, zpf));
                const uint32_t b1 = static_cast<uint8_t>(quantize_one(v[1], s, zpf));
                const uint32_t b2 = static_cast<uint8_t>(quantize_one(v[2], s, zpf));
                const uint32_t b3 = static_cast<uint8_t>(quantize_one(v[3], s, zpf));
                reinterpret_cast<uint32_t *>(q)[i] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
            }
        }
    }
    for (int i = cached ? k4 : tid; i < k4; i += kQThreads) {
        const f32x4 v = reinterpret_cast<const f32x4 *>(x)[i];
        const uint32_t b0 = static_cast<uint8_t>(quantize_one(v[0], s, zpf));
        const uint32_t b1 = static_cast<uint8_t>(quantize_one(v[1], s, zpf));
        const uint32_t b2 = static_cast<uint8_t>(quantize_one(v[2], s, zpf));
        const uint32_t b3 = static_cast<uint8_t>(quantize_one(v[3], s, zpf));
        reinterpret_cast<uint32_t *>(q)[i] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
    }
    for (int i = 4 * k4 + tid; i < k; i += kQThreads) {
        q[i] = quantize_one(x[i], s, zpf);
    }
}

}  // namespace
}  // namespace tqt

using namespace tqt;

extern "C" {

void tqt_run_quantize_qai8dx_f32_gfx950_async(size_t m, size_t k, const float *A, size_t lda,
                                              int8_t *A_q, size_t lda_q, float *scale_a,
                                              int32_t *zero_point_a, void *stream)
{
    if (m == 0) {
        return;
    }
    TQT_REQUIRE(m < (1u << 31) && k < (1u << 31), "dimension exceeds 2^31-1");
    TQT_REQUIRE(scale_a != nullptr && zero_point_a != nullptr, "scale_a / zero_point_a == NULL");
    TQT_REQUIRE((A != nullptr && A_q != nullptr) || k == 0, "A / A_q == NULL");
    TQT_REQUIRE(lda >= k && lda_q >= k, "lda or lda_q < k");
    // float4 loads and 4-byte stores when every row starts aligned for them
    const bool vec = aligned16(A) && lda % 4 == 0 && (reinterpret_cast<uintptr_t>(A_q) & 3) == 0 &&
                     lda_q % 4 == 0;
    hipLaunchKernelGGL(quantize_qai8dx_kernel, dim3(static_cast<unsigned>(m)), dim3(kQThreads), 0,
                       as_stream(stream), static_cast<int>(k), A, static_cast<long long>(lda),
                       A_q, static_cast<long long>(lda_q), scale_a, zero_point_a, vec);
    check_launch("tqt_run_quantize_qai8dx_f32_gfx950");
}

void tqt_run_quantize_qai8dx_f32_gfx950(size_t m, size_t k, const float *A, size_t lda,
                                        int8_t *A_q, size_t lda_q, float *scale_a,
                                        int32_t *zero_point_a)
{
    if (m == 0) {
        return;
    }
    tqt_run_quantize_qai8dx_f32_gfx950_async(m, k, A, lda, A_q, lda_q, scale_a, zero_point_a,
                                             nullptr);
    finish_sync(nullptr, "tqt_run_quantize_qai8dx_f32_gfx950");
}

}  // extern "C"
