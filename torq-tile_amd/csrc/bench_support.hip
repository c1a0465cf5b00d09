// Measurement support for bench.py: libtqt_bench_support.so. Not part of the product C ABI
// (nothing in include/ declares these symbols); the product library never calls it.
//
//  * tqtb_read_floor_async: one launch that streams `nbytes` from HBM with 16-byte loads and
//    writes nothing (a sink word only when an impossible checksum comes up). Timed over rotating
//    copies of the same size as a kernel's operands, it is the single-launch read floor of this
//    GPU: what any one launch reading those bytes can reach, launch ramp and drain included.
//    bench.py also uses it over a buffer of twice the Infinity Cache to evict the operands from
//    the caches before a timed region without leaving dirty lines behind.
//  * tqtb_stream_floor_async: the W8A8 stream kernel's load schedule alone (the same grid,
//    tile order, LDS-DMA load roles, four-slot ring, per-stage waits and barriers; no MFMA, no
//    epilogue): the per-CU L2 -> LDS stream floor of that kernel's shape, on cold operands or,
//    with `resident`, with every workgroup reading the first tile's rows (L2-resident).
//  * tqtb_empty_async: an empty kernel launched with a given grid, block and LDS size (the
//    headline kernels' shapes): the launch cost of that shape.
//  * tqtb_run_w4a16*_async: the W4A16 entry points take their clamp bounds as _Float16 by
//    value, which ctypes cannot pass (x86-64 passes them in SSE registers); these forward the
//    bounds given as their 16-bit patterns.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "tqt_hip_common.hpp"

#include "tqt_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950.h"

namespace {

constexpr int kFloorThreads = 256;
constexpr uint32_t kImpossible = 0x9e3779b9u;
typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));

// Workgroup b reads the U * 4 KiB block starting at b * U * 4 KiB: load u of wave w covers the
// 1 KiB at (u * 4 + w) KiB of the block (64 lanes x 16 bytes, whole cache lines), and all U loads
// are issued before any is used, as the GEMV kernels issue theirs. Indices past the end are
// clamped to the last vector (in range; its bytes are then read twice).
template <int U>
__global__ __launch_bounds__(kFloorThreads) void read_floor_kernel(const v4u32 *__restrict__ src,
                                                                    size_t n16, uint32_t *sink)
{
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const size_t base = static_cast<size_t>(blockIdx.x) * U * kFloorThreads;
    v4u32 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        size_t i = base + static_cast<size_t>(u * 4 + wave) * 64 + lane;
        i = i < n16 ? i : n16 - 1;
        v[u] = __builtin_nontemporal_load(&src[i]);
    }
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == kImpossible) {
        sink[blockIdx.x] = acc;
    }
}

template <int U>
int launch_floor(const void *src, size_t nbytes, void *sink, size_t sink_words, hipStream_t s)
{
    const size_t n16 = nbytes / 16;
    const size_t blocks = (n16 + static_cast<size_t>(U) * kFloorThreads - 1) /
                          (static_cast<size_t>(U) * kFloorThreads);
    if (blocks == 0 || blocks > sink_words || blocks >= (1u << 31)) {
        return -1;
    }
    hipLaunchKernelGGL((read_floor_kernel<U>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kFloorThreads), 0, s, static_cast<const v4u32 *>(src), n16,
                       static_cast<uint32_t *>(sink));
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---- stream floor: the W8A8 stream kernel's loads alone (BM 64 x 128 tiles, k in 128-byte
// stages, 8 waves, each issuing 1 A and 2 B blocks of 8 rows x 128 bytes per stage) ----
constexpr int kSfBM = 64;
constexpr int kSfBN = 128;
constexpr int kSfSK = 128;
constexpr int kSfWaves = 8;
constexpr int kSfStages = 4;
constexpr int kSfA = kSfBM / (8 * kSfWaves);  // A blocks per wave per stage
constexpr int kSfB = kSfBN / (8 * kSfWaves);  // B blocks per wave per stage
constexpr int kSfPer = kSfA + kSfB;
constexpr int kSfSlot = (kSfBM + kSfBN) * kSfSK;
constexpr int kSfLds = kSfStages * kSfSlot;

__host__ __device__ constexpr int sf_waitcnt(int vm)
{
    return (vm & 15) | (7 << 4) | (15 << 8) | ((vm >> 4) << 14);  // vmcnt only
}

__global__ __launch_bounds__(kSfWaves * 64) void stream_floor_kernel(
    const int8_t *A, const int8_t *B, int M, int N, int K, int tiles_m, int tiles, int per_xcd,
    int resident, uint32_t *sink)
{
    __shared__ __attribute__((aligned(16))) int8_t ring[kSfStages][kSfSlot];
    const int t = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (t >= tiles) {
        return;
    }
    const int m0 = resident ? 0 : (t % tiles_m) * kSfBM;
    const int n0 = resident ? 0 : (t / tiles_m) * kSfBN;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int8_t *a_row[kSfA];
    const int8_t *b_row[kSfB];
    for (int j = 0; j < kSfA; ++j) {
        const int r = 8 * (wave * kSfA + j) + (lane >> 3);
        const int chunk = (lane & 7) ^ ((r >> 1) & 7);
        a_row[j] = A + static_cast<long long>(min(m0 + r, M - 1)) * K + chunk * 16;
    }
    for (int j = 0; j < kSfB; ++j) {
        const int r = 8 * (wave * kSfB + j) + (lane >> 3);
        const int chunk = (lane & 7) ^ ((r >> 1) & 7);
        b_row[j] = B + static_cast<long long>(min(n0 + r, N - 1)) * K + chunk * 16;
    }
    auto issue = [&](int st, int8_t *slot) {
        const int k0 = st * kSfSK;
        for (int j = 0; j < kSfA; ++j) {
            tqt::dma_lds16(a_row[j] + k0, slot + (wave * kSfA + j) * 1024);
        }
        for (int j = 0; j < kSfB; ++j) {
            tqt::dma_lds16(b_row[j] + k0, slot + kSfBM * kSfSK + (wave * kSfB + j) * 1024);
        }
    };
    const int nst = K / kSfSK;
    for (int i = 0; i < kSfStages - 1 && i < nst; ++i) {
        issue(i, ring[i]);
    }
    for (int st = 0; st < nst; ++st) {
        const int ahead = min(kSfStages - 2, nst - 1 - st);
        if (ahead >= 2) {
            __builtin_amdgcn_s_waitcnt(sf_waitcnt(2 * kSfPer));
        } else if (ahead == 1) {
            __builtin_amdgcn_s_waitcnt(sf_waitcnt(kSfPer));
        } else {
            __builtin_amdgcn_s_waitcnt(sf_waitcnt(0));
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (st + kSfStages - 1 < nst) {
            issue(st + kSfStages - 1, ring[(st + kSfStages - 1) % kSfStages]);
        }
    }
    __builtin_amdgcn_s_waitcnt(sf_waitcnt(0));
    asm volatile("" ::: "memory");
    // one LDS word per lane read back, so the stream has a consumer; written only on an
    // impossible value
    const uint32_t v = *reinterpret_cast<const uint32_t *>(&ring[(nst - 1) % kSfStages][4 * threadIdx.x]);
    if (v == kImpossible && lane == 0) {
        sink[blockIdx.x] = v;
    }
}

__global__ __launch_bounds__(1024) void empty_kernel(uint32_t *sink)
{
    extern __shared__ uint32_t dyn[];
    if (sink == nullptr) {
        dyn[threadIdx.x] = 0;  // never: the launch carries its LDS size only
    }
}

inline float16_t half_from_bits(uint16_t bits)
{
    float16_t h;
    memcpy(&h, &bits, 2);
    return h;
}

}  // namespace

extern "C" {

// Reads nbytes (a multiple of 16, 16-byte aligned src, at least 16) in one launch on `stream`:
// `loads` (1, 2, 4, 8 or 16) 16-byte loads per lane, workgroups of 256 threads each reading
// loads * 4 KiB contiguous. `sink` must hold sink_words words (one per workgroup). Returns 0, or
// -1 on a bad argument or launch error.
int tqtb_read_floor_async(const void *src, size_t nbytes, void *sink, size_t sink_words,
                          int loads, void *stream)
{
    if (src == nullptr || sink == nullptr || nbytes < 16 || (nbytes & 15) != 0 ||
        (reinterpret_cast<uintptr_t>(src) & 15) != 0) {
        return -1;
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    switch (loads) {
    case 1: return launch_floor<1>(src, nbytes, sink, sink_words, s);
    case 2: return launch_floor<2>(src, nbytes, sink, sink_words, s);
    case 4: return launch_floor<4>(src, nbytes, sink, sink_words, s);
    case 8: return launch_floor<8>(src, nbytes, sink, sink_words, s);
    case 16: return launch_floor<16>(src, nbytes, sink, sink_words, s);
    default: return -1;
    }
}

// The W8A8 stream kernel's load schedule over A [M, K] and B [N, K] (M % 64 == 0, N % 128 == 0,
// K % 128 == 0, 16-byte aligned rows): one launch on `stream`. resident != 0: every workgroup
// reads the first tile's 64 + 128 rows. `sink` must hold one word per workgroup (8 * ceil(tiles
// / 8)). Returns 0, or -1 on a bad argument or launch error.
int tqtb_stream_floor_async(const void *A, const void *B, int M, int N, int K, int resident,
                            void *sink, size_t sink_words, void *stream)
{
    if (!A || !B || !sink || M <= 0 || N <= 0 || K <= 0 || M % kSfBM || N % kSfBN ||
        K % kSfSK || (reinterpret_cast<uintptr_t>(A) & 15) || (reinterpret_cast<uintptr_t>(B) & 15)) {
        return -1;
    }
    const int tiles_m = M / kSfBM;
    const int tiles = tiles_m * (N / kSfBN);
    const int per_xcd = (tiles + 7) / 8;
    if (static_cast<size_t>(8 * per_xcd) > sink_words) {
        return -1;
    }
    hipLaunchKernelGGL(stream_floor_kernel, dim3(8 * per_xcd), dim3(kSfWaves * 64), 0,
                       static_cast<hipStream_t>(stream), static_cast<const int8_t *>(A),
                       static_cast<const int8_t *>(B), M, N, K, tiles_m, tiles, per_xcd, resident,
                       static_cast<uint32_t *>(sink));
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// An empty kernel with `blocks` workgroups of `threads` threads (a multiple of 64, at most 1024)
// and `lds_bytes` of LDS.
int tqtb_empty_async(int blocks, int threads, int lds_bytes, void *sink, void *stream)
{
    if (blocks <= 0 || threads <= 0 || threads > 1024 || threads % 64 != 0 || lds_bytes < 0 ||
        lds_bytes > 160 * 1024 || sink == nullptr) {
        return -1;
    }
    hipLaunchKernelGGL(empty_kernel, dim3(blocks), dim3(threads), lds_bytes,
                       static_cast<hipStream_t>(stream), static_cast<uint32_t *>(sink));
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// LDS bytes of the stream kernel's ring (for tqtb_empty_async).
int tqtb_stream_lds_bytes(void)
{
    return kSfLds;
}

void tqtb_run_w4a16_async(size_t m, size_t n, size_t k, size_t bl, const void *A, size_t lda,
                          const void *B, size_t ldb, const void *scale_b, size_t ldsb,
                          const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
                          uint16_t cmin_bits, uint16_t cmax_bits, void *stream)
{
    tqt_run_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950_async(
        m, n, k, bl, A, lda, 0, B, ldb, 0, scale_b, ldsb, C, ldc, D, ldd, bias,
        half_from_bits(cmin_bits), half_from_bits(cmax_bits), stream);
}

void tqtb_run_w4a16p_async(size_t m, size_t n, size_t k, size_t bl, const void *A_packed,
                           size_t lda, const void *B_packed, size_t ldb, const void *scale_b,
                           size_t ldsb, const void *C, size_t ldc, void *D, size_t ldd,
                           const void *bias, uint16_t cmin_bits, uint16_t cmax_bits, void *stream)
{
    tqt_run_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950_async(
        m, n, k, bl, A_packed, lda, 0, B_packed, ldb, 0, scale_b, ldsb, C, ldc, D, ldd, bias,
        half_from_bits(cmin_bits), half_from_bits(cmax_bits), stream);
}

}  // extern "C"
