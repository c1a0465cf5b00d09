// gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt (W4A8) on gfx950.
//
// Fast path (decode-shaped, any m in chunks of 15 rows): one workgroup of 4 wave64s owns a
// 16-channel weight tile (16 rows of B, contiguous [16, k/2] bytes) for one chunk of up to 15
// activation rows. Each wave streams a quarter of k: one 128-bit load per lane covers 32
// nibbles (k values) of one channel. Nibbles are split with two bit operations into unsigned
// bytes q in [0, 15] and fed to v_mfma_i32_16x16x64_i8 as the B operand; the activation rows
// are the A operand, byte-permuted into the same (even k, odd k) order. Two terms fold the
// -8 zero point of the weights and the per-channel weight sum into the same MFMAs:
//   * an extra MFMA per step with a constant B operand of -8 adds -8 * sum_k a to every
//     column, so the accumulator holds sum_k a * (q - 8) exactly;
//   * activation row `rows` (the first unused row of the 16-row A operand) is all ones, so
//     that accumulator row holds sum_k (q - 8), the rsum_b of the reference.
// The four waves' int32 partials are summed through LDS and the reference's f32 epilogue
// (zero-point correction, two scale multiplies, C, bias, clamp; no FMA) runs per output.
#include "tqt_hip_common.hpp"
#include "tqt_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950.h"

namespace tqt {
namespace {

constexpr int kRowsPerChunk = 15;  // activation rows per workgroup (row 15 is the ones row)
constexpr int kNTile = 16;         // weight channels per workgroup
constexpr int kStepK = 128;        // k values per wave step (4 lane groups x 32 nibbles)
constexpr int kBatch = 8;          // steps whose loads are issued together

struct W4A8Args
{
    int M, N, K;
    const int8_t *A;
    long long lda;
    const uint8_t *B;
    long long bstride;  // bytes between weight rows (= ldb / 2)
    const float *C;
    long long ldc;
    float *D;
    long long ldd;
    const float *bias;
    float cmin, cmax;
    const float *scale_a;
    const int32_t *zp_a;
    const float *scale_b;
};

__device__ __forceinline__ float epilogue_f32(const W4A8Args &a, int gm, int gn, int32_t acc,
                                              int32_t rsum)
{
    // tqt_kernel_gemm_i8_i4_4x1vl_rvv.h:234-419: zp correction (int32), RNE convert, two
    // separate multiplies, C then bias (separate adds), vfmax then vfmin.
    const int32_t v = static_cast<int32_t>(static_cast<uint32_t>(acc) -
                                           static_cast<uint32_t>(a.zp_a[gm]) *
                                               static_cast<uint32_t>(rsum));
    float f = __int2float_rn(v);
    f = __fmul_rn(f, a.scale_a[gm]);
    f = __fmul_rn(f, a.scale_b[gn]);
    if (a.C) {
        f = __fadd_rn(f, a.C[static_cast<long long>(gm) * a.ldc + gn]);
    }
    if (a.bias) {
        f = __fadd_rn(f, a.bias[gn]);
    }
    f = fmaxf(f, a.cmin);
    f = fminf(f, a.cmax);
    return f;
}

__global__ __launch_bounds__(256) void w4a8_mfma_kernel(W4A8Args a)
{
    __shared__ int32_t s_part[4][16][16];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n0 = blockIdx.x * kNTile;
    const int m0 = blockIdx.y * kRowsPerChunk;
    const int rows = min(kRowsPerChunk, a.M - m0);

    const int fr = lane & 15;  // A-operand row (activation) / B-operand column (channel)
    const int fg = lane >> 4;  // k group within the 64-k MFMA step

    // This lane's weight row and activation row.
    const bool w_ok = (n0 + fr) < a.N;
    const uint8_t *wrow = a.B + static_cast<long long>(w_ok ? n0 + fr : 0) * a.bstride + fg * 16;
    const bool a_real = fr < rows;
    const bool a_ones = fr == rows;
    const int8_t *arow = a.A + static_cast<long long>(a_real ? m0 + fr : 0) * a.lda + fg * 32;

    const int nsteps = a.K / kStepK;
    const int per_wave = (nsteps + 3) / 4;
    const int s_begin = wave * per_wave;
    const int s_end = min(nsteps, s_begin + per_wave);

    const i32x4 neg8 = i32x4{static_cast<int32_t>(0xf8f8f8f8u), static_cast<int32_t>(0xf8f8f8f8u),
                             static_cast<int32_t>(0xf8f8f8f8u), static_cast<int32_t>(0xf8f8f8f8u)};
    const i32x4 ones = i32x4{0x01010101, 0x01010101, 0x01010101, 0x01010101};
    i32x4 acc = i32x4{0, 0, 0, 0};

    for (int sb = s_begin; sb < s_end; sb += kBatch) {
        u32x4 wv[kBatch];
        i32x4 av0[kBatch], av1[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int s = sb + i;
            if (s < s_end && w_ok) {
                wv[i] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4 *>(wrow + static_cast<long long>(s) * (kStepK / 2)));
            } else {
                wv[i] = u32x4{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
            }
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int s = sb + i;
            if (s < s_end && a_real) {
                const int8_t *p = arow + static_cast<long long>(s) * kStepK;
                av0[i] = *reinterpret_cast<const i32x4 *>(p);
                av1[i] = *reinterpret_cast<const i32x4 *>(p + 16);
            } else if (a_ones) {
                av0[i] = ones;
                av1[i] = ones;
            } else {
                av0[i] = i32x4{0, 0, 0, 0};
                av1[i] = i32x4{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            if (sb + i >= s_end) {
                break;
            }
            // Weight nibbles -> unsigned bytes: lo = even k, hi = odd k of each byte.
            i32x4 q0, q1;
            q0[0] = static_cast<int32_t>(wv[i][0] & 0x0f0f0f0fu);
            q0[1] = static_cast<int32_t>((wv[i][0] >> 4) & 0x0f0f0f0fu);
            q0[2] = static_cast<int32_t>(wv[i][1] & 0x0f0f0f0fu);
            q0[3] = static_cast<int32_t>((wv[i][1] >> 4) & 0x0f0f0f0fu);
            q1[0] = static_cast<int32_t>(wv[i][2] & 0x0f0f0f0fu);
            q1[1] = static_cast<int32_t>((wv[i][2] >> 4) & 0x0f0f0f0fu);
            q1[2] = static_cast<int32_t>(wv[i][3] & 0x0f0f0f0fu);
            q1[3] = static_cast<int32_t>((wv[i][3] >> 4) & 0x0f0f0f0fu);
            // Activations in the same order: (even bytes, odd bytes) of each 8-byte run.
            i32x4 x0, x1;
            const uint32_t a0 = static_cast<uint32_t>(av0[i][0]), a1 = static_cast<uint32_t>(av0[i][1]);
            const uint32_t a2 = static_cast<uint32_t>(av0[i][2]), a3 = static_cast<uint32_t>(av0[i][3]);
            const uint32_t a4 = static_cast<uint32_t>(av1[i][0]), a5 = static_cast<uint32_t>(av1[i][1]);
            const uint32_t a6 = static_cast<uint32_t>(av1[i][2]), a7 = static_cast<uint32_t>(av1[i][3]);
            x0[0] = static_cast<int32_t>(__builtin_amdgcn_perm(a1, a0, 0x06040200u));
            x0[1] = static_cast<int32_t>(__builtin_amdgcn_perm(a1, a0, 0x07050301u));
            x0[2] = static_cast<int32_t>(__builtin_amdgcn_perm(a3, a2, 0x06040200u));
            x0[3] = static_cast<int32_t>(__builtin_amdgcn_perm(a3, a2, 0x07050301u));
            x1[0] = static_cast<int32_t>(__builtin_amdgcn_perm(a5, a4, 0x06040200u));
            x1[1] = static_cast<int32_t>(__builtin_amdgcn_perm(a5, a4, 0x07050301u));
            x1[2] = static_cast<int32_t>(__builtin_amdgcn_perm(a7, a6, 0x06040200u));
            x1[3] = static_cast<int32_t>(__builtin_amdgcn_perm(a7, a6, 0x07050301u));
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, q0, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, neg8, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, q1, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, neg8, acc, 0, 0, 0);
        }
    }

    // lane holds rows 4*fg + r, column fr of the 16x16 partial
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        s_part[wave][4 * fg + r][fr] = acc[r];
    }
    __syncthreads();
    const int orow = tid >> 4;
    const int ocol = tid & 15;
    const int32_t total = static_cast<int32_t>(
        static_cast<uint32_t>(s_part[0][orow][ocol]) + static_cast<uint32_t>(s_part[1][orow][ocol]) +
        static_cast<uint32_t>(s_part[2][orow][ocol]) + static_cast<uint32_t>(s_part[3][orow][ocol]));
    __syncthreads();
    s_part[0][orow][ocol] = total;
    __syncthreads();
    const int gm = m0 + orow;
    const int gn = n0 + ocol;
    if (orow < rows && gn < a.N) {
        const int32_t rsum = s_part[0][rows][ocol];
        a.D[static_cast<long long>(gm) * a.ldd + gn] = epilogue_f32(a, gm, gn, total, rsum);
    }
}

// Generic path: one thread per output, any alignment, any even k.
__global__ __launch_bounds__(256) void w4a8_generic_kernel(W4A8Args a)
{
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<long long>(a.M) * a.N) {
        return;
    }
    const int gm = static_cast<int>(idx / a.N);
    const int gn = static_cast<int>(idx - static_cast<long long>(gm) * a.N);
    const int8_t *arow = a.A + static_cast<long long>(gm) * a.lda;
    const uint8_t *brow = a.B + static_cast<long long>(gn) * a.bstride;
    uint32_t acc = 0, rsum = 0;
    for (int k = 0; k < a.K; k += 2) {
        const uint8_t byte = brow[k >> 1];
        const int32_t lo = static_cast<int32_t>(byte & 0xf) - 8;
        const int32_t hi = static_cast<int32_t>(byte >> 4) - 8;
        rsum += static_cast<uint32_t>(lo + hi);
        acc += static_cast<uint32_t>(static_cast<int32_t>(arow[k]) * lo);
        acc += static_cast<uint32_t>(static_cast<int32_t>(arow[k + 1]) * hi);
    }
    a.D[static_cast<long long>(gm) * a.ldd + gn] =
        epilogue_f32(a, gm, gn, static_cast<int32_t>(acc), static_cast<int32_t>(rsum));
}

}  // namespace
}  // namespace tqt

using namespace tqt;

extern "C" {

static const size_t kW4A8MStep = 16;
static const size_t kW4A8NStep = 16;

size_t tqt_get_m_step_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(void)
{
    return kW4A8MStep;
}
size_t tqt_get_n_step_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(void)
{
    return kW4A8NStep;
}
size_t tqt_get_a_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(size_t m_idx,
                                                                          size_t k_idx, size_t lda)
{
    TQT_REQUIRE(m_idx % kW4A8MStep == 0, "m_idx % m_step == 0");
    return (m_idx * lda + k_idx) * sizeof(int8_t);
}
size_t tqt_get_b_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(size_t n_idx,
                                                                          size_t k_idx, size_t ldb)
{
    TQT_REQUIRE(n_idx % kW4A8NStep == 0, "n_idx % n_step == 0");
    TQT_REQUIRE(k_idx % 2 == 0, "k_idx % 2 == 0");
    return n_idx * (ldb / 2) + k_idx / 2;
}
size_t tqt_get_c_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(size_t m_idx,
                                                                          size_t n_idx, size_t ldc)
{
    TQT_REQUIRE(m_idx % kW4A8MStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kW4A8NStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldc + n_idx) * sizeof(float);
}
size_t tqt_get_bias_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(size_t n_idx)
{
    TQT_REQUIRE(n_idx % kW4A8NStep == 0, "n_idx % n_step == 0");
    return n_idx * sizeof(float);
}
size_t tqt_get_d_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(size_t m_idx,
                                                                          size_t n_idx, size_t ldd)
{
    TQT_REQUIRE(m_idx % kW4A8MStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kW4A8NStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldd + n_idx) * sizeof(float);
}
size_t tqt_get_d_size_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(size_t m, size_t n)
{
    return m * n * sizeof(float);
}

void tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    float clamp_min, float clamp_max, const struct tqt_qai8dx_qsi4cx_params *params, void *stream)
{
    (void)k_idx_a;
    (void)k_idx_b;
    if (!params) {
        return;  // reference …qai8dx_qsi4cxt_4x1vl_rvv.cpp:165-167
    }
    if (m == 0 || n == 0) {
        return;
    }
    TQT_REQUIRE(k % 2 == 0, "k % 2 == 0");
    TQT_REQUIRE(m < (1u << 31) && n < (1u << 31) && k < (1u << 31), "dimension exceeds 2^31-1");
    TQT_REQUIRE(params->scale_a && params->zero_point_a && params->scale_b,
                "params arrays must be non-NULL");
    TQT_REQUIRE((A != nullptr && B != nullptr) || k == 0, "A/B == NULL");
    TQT_REQUIRE(D != nullptr, "D == NULL");
    W4A8Args a = {};
    a.M = static_cast<int>(m);
    a.N = static_cast<int>(n);
    a.K = static_cast<int>(k);
    a.A = static_cast<const int8_t *>(A);
    a.lda = static_cast<long long>(lda);
    a.B = static_cast<const uint8_t *>(B);
    a.bstride = static_cast<long long>(ldb / 2);
    a.C = static_cast<const float *>(C);
    a.ldc = static_cast<long long>(ldc);
    a.D = static_cast<float *>(D);
    a.ldd = static_cast<long long>(ldd);
    a.bias = static_cast<const float *>(bias);
    a.cmin = clamp_min;
    a.cmax = clamp_max;
    a.scale_a = params->scale_a;
    a.zp_a = params->zero_point_a;
    a.scale_b = params->scale_b;
    hipStream_t s = as_stream(stream);
    const bool fast = (k % kStepK == 0) && (lda % 16 == 0) && ((ldb / 2) % 16 == 0) &&
                      aligned16(A) && aligned16(B);
    if (fast) {
        const unsigned gx = static_cast<unsigned>((n + kNTile - 1) / kNTile);
        const unsigned long long gy = (m + kRowsPerChunk - 1) / kRowsPerChunk;
        TQT_REQUIRE(gy < 65536, "m too large for the decode path");
        hipLaunchKernelGGL(w4a8_mfma_kernel, dim3(gx, static_cast<unsigned>(gy)), dim3(256), 0, s,
                           a);
    } else {
        const long long total = static_cast<long long>(m) * static_cast<long long>(n);
        const long long blocks = (total + 255) / 256;
        TQT_REQUIRE(blocks < (1ll << 31), "grid too large");
        hipLaunchKernelGGL(w4a8_generic_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                           s, a);
    }
    check_launch("tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    float clamp_min, float clamp_max, const struct tqt_qai8dx_qsi4cx_params *params)
{
    if (!params) {
        return;
    }
    tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950_async(
        m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias, clamp_min, clamp_max,
        params, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950");
}

}  // extern "C"
