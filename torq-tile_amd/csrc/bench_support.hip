// Measurement support for bench.py: libtqt_bench_support.so. Not part of the product C ABI
// (nothing in include/ declares these symbols); the product library never calls it.
//
//  * tqtb_read_floor_async: one launch that streams `nbytes` from HBM with 16-byte loads and
//    writes nothing (a sink word only when an impossible checksum comes up). Timed over rotating
//    copies of the same size as a kernel's operands, it is the single-launch read floor of this
//    GPU: what any one launch reading those bytes can reach, launch ramp and drain included.
//    bench.py also uses it over a buffer of twice the Infinity Cache to evict the operands from
//    the caches before a timed region without leaving dirty lines behind.
//  * tqtb_run_w4a16*_async: the W4A16 entry points take their clamp bounds as _Float16 by
//    value, which ctypes cannot pass (x86-64 passes them in SSE registers); these forward the
//    bounds given as their 16-bit patterns.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

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
