// gemm_1xnbias_clamp_f16_f16_qsi4c2t (W4A16, block-quantized int4 weights) on gfx950.
//
// Two MFMA kernels share the math below: w4a16_chunk_kernel (k % 512 == 0: 16 waves per CU walk
// k in 512-wide chunks streamed through a shared LDS ring; see its own comment) and
// w4a16_mfma_kernel (any other k % 128 == 0, k <= 4096). In w4a16_mfma_kernel a workgroup of
// 8 wave64s owns a strip of
// 16-channel weight tiles for one group of 32 activation rows. Wave w owns a fixed slice of k
// (a run of 32-wide scale blocks) and keeps its slice of A (32 rows, f16) in registers for the
// whole strip, so A is read from memory once per workgroup. For each 16-channel tile:
//   * each lane loads 16 contiguous weight bytes (one whole 32-k block of one channel) per
//     128-bit load; a 4x4 lane-group transpose with v_permlane32_swap/v_permlane16_swap gives
//     each lane group its 8-k slice of four consecutive blocks, the MFMA B-operand layout;
//   * nibbles become f16 (q - 8) exactly: (nib | 0x6400) is the f16 value 1024 + q, and a
//     packed f16 subtract of 1032 leaves q - 8;
//   * v_mfma_f32_16x16x32_f16 contracts one scale block (all products exact in f32), and the
//     block's f32 partial is scaled by the f32 value of its f16 scale and accumulated;
//   * the eight waves' f32 partials are summed through LDS; C, bias and the clamp are applied
//     in f32 and the result is stored once: rounded to f16 for the f16 types, as is for the
//     f32-output types (gemm_1xnbias_clamp_f32_f16_qsi4c2t and its packed sibling, whose C and
//     bias are f32 too).
// A generic one-thread-per-output kernel covers every other shape with the reference test
// oracle's exact operation order (reference test/common/reference_gemm.cpp:132-179).
#include <type_traits>

#include "tqt_hip_common.hpp"
#include "tqt_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950.h"

namespace tqt {
namespace {

constexpr int kWaves = 8;
constexpr int kMaxGroupsPerWave = 4;  // 4-block groups (128 k each) per wave -> k <= 4096
constexpr int kMRows = 32;            // activation rows per workgroup (two 16-row MFMA tiles)
constexpr int kNTile = 16;

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// s_waitcnt immediate waiting for vmcnt <= vm only (gfx9: vmcnt[3:0] | expcnt[6:4] |
// lgkmcnt[11:8] | vmcnt[5:4] << 14; expcnt and lgkmcnt at their maximum: no wait).
__host__ __device__ constexpr int waitcnt_vm0(int vm)
{
    return (vm & 15) | (7 << 4) | (15 << 8) | ((vm >> 4) << 14);
}

struct W4A16Args
{
    int M, N, K;
    int ntiles;  // 16-channel tiles
    const _Float16 *A;
    long long lda;
    const uint8_t *B;
    long long bstride;  // bytes between weight rows
    const _Float16 *scale_b;
    long long ldsb;
    const void *C;  // f16 or f32 (the output type)
    long long ldc;
    void *D;
    long long ldd;
    const void *bias;
    float cmin, cmax;
    int bl;
    PackDesc pa, pb;  // packed A / B of the p-variant (read when the kernel's PK bit is set)
};

// Row pointer (bytes) and k multiplier of activation row `row`: f16 element k of the row is at
// row pointer + 2 * k * mul for k a multiple of 8 (one 16-byte chunk).
template <int PK>
__device__ __forceinline__ const uint8_t *a_row_ptr(const W4A16Args &a, int row, int &mul)
{
    const uint8_t *base = reinterpret_cast<const uint8_t *>(a.A);
    if constexpr ((PK & PK_A) != 0) {
        return base + pack_row_fixed<kPackW4A16MStep>(a.pa, row, mul);
    } else {
        mul = 1;
        return base + static_cast<long long>(row) * a.lda * 2;
    }
}

// Weight row pointer and k multiplier of channel n: byte kb (a multiple of 16) is at pointer +
// kb * mul.
template <int PK>
__device__ __forceinline__ const uint8_t *b_row_ptr(const W4A16Args &a, int n, int &mul)
{
    if constexpr ((PK & PK_B) != 0) {
        return a.B + pack_row_fixed<kPackW4A16NStep>(a.pb, n, mul);
    } else {
        mul = 1;
        return a.B + static_cast<long long>(n) * a.bstride;
    }
}

// 4x4 transpose of 32-bit values across the four 16-lane groups: on entry p[j] of lane group
// g holds element (g, j); on exit p[j] of lane group g holds element (j, g).
__device__ __forceinline__ void transpose_lane_groups(uint32_t p[4])
{
    auto s02 = __builtin_amdgcn_permlane32_swap(p[0], p[2], false, false);
    auto s13 = __builtin_amdgcn_permlane32_swap(p[1], p[3], false, false);
    // p0 = [x00 x10 x02 x12], p2 = [x20 x30 x22 x32], p1 = [x01 x11 x03 x13], p3 = [x21 x31 x23 x33]
    auto t01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
    auto t23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
    p[0] = t01[0];
    p[1] = t01[1];
    p[2] = t23[0];
    p[3] = t23[1];
}

// 8 nibbles (k = 0..7 of this lane's slice, nibble i at bits 4i) -> 8 exact f16 values q - 8,
// in slot order k = 0, 4, 1, 5, 2, 6, 3, 7.
__device__ __forceinline__ f16x8 unpack_q8(uint32_t x)
{
    const f16x2 bias = f16x2{static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    uint32_t d[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        d[j] = ((x >> (4 * j)) & 0x000f000fu) | 0x64006400u;
    }
    f16x8 out;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f16x2 h = __builtin_bit_cast(f16x2, d[j]) + bias;
        out[2 * j] = h[0];
        out[2 * j + 1] = h[1];
    }
    return out;
}

// 8 consecutive f16 activations k = 0..7 -> slot order k = 0, 4, 1, 5, 2, 6, 3, 7.
__device__ __forceinline__ f16x8 permute_a(u32x4 v)
{
    u32x4 o;
    o[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
    o[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
    o[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
    o[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
    return __builtin_bit_cast(f16x8, o);
}

template <int PK, int OUT>
__global__ __launch_bounds__(512) void w4a16_mfma_kernel(W4A16Args a)
{
    __shared__ float s_part[2][kWaves][kMRows][kNTile];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int fr = lane & 15;
    const int fg = lane >> 4;
    const int mg0 = blockIdx.y * kMRows;

    // Strip of 16-channel tiles for this workgroup.
    const int t_begin = static_cast<int>((static_cast<long long>(blockIdx.x) * a.ntiles) / gridDim.x);
    const int t_end = static_cast<int>((static_cast<long long>(blockIdx.x + 1) * a.ntiles) / gridDim.x);

    // k slice of this wave, in 4-block groups of 128 k.
    const int ngroups = a.K / 128;
    const int gpw = (ngroups + kWaves - 1) / kWaves;
    const int g_begin = min(ngroups, wave * gpw);
    const int g_cnt = min(ngroups, g_begin + gpw) - g_begin;

    // A operand for every block of the slice and both 16-row tiles. Unconditional loads from
    // clamped addresses keep them all in flight together; unused ones are zeroed afterwards.
    u32x4 ra[kMaxGroupsPerWave * 4][2];
#pragma unroll
    for (int j = 0; j < kMaxGroupsPerWave * 4; ++j) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const int row = min(mg0 + mt * 16 + fr, a.M - 1);
            const int jj = min(j, max(g_cnt * 4 - 1, 0));
            const int k = min((g_begin * 4 + jj) * 32, max(a.K - 32, 0)) + fg * 8;
            int mul;
            const uint8_t *arow = a_row_ptr<PK>(a, row, mul);
            ra[j][mt] = *reinterpret_cast<const u32x4 *>(arow + 2ll * k * mul);
        }
    }
    f16x8 fa[kMaxGroupsPerWave * 4][2];
#pragma unroll
    for (int j = 0; j < kMaxGroupsPerWave * 4; ++j) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const bool ok = j < g_cnt * 4 && mg0 + mt * 16 + fr < a.M;
            const u32x4 z = u32x4{0u, 0u, 0u, 0u};
            fa[j][mt] = permute_a(ok ? ra[j][mt] : z);
        }
    }

    u32x4 wcur[kMaxGroupsPerWave], wnext[kMaxGroupsPerWave];
    uint64_t scur[kMaxGroupsPerWave], snext[kMaxGroupsPerWave];

    auto load_tile = [&](int t, u32x4 (&w)[kMaxGroupsPerWave], uint64_t (&s)[kMaxGroupsPerWave]) {
        const int n = t * kNTile + fr;
        const bool ok = (t < t_end) && (n < a.N);
        int wmul;
        const uint8_t *wrow = b_row_ptr<PK>(a, ok ? n : 0, wmul);
        const _Float16 *srow = a.scale_b + static_cast<long long>(ok ? n : 0) * a.ldsb;
#pragma unroll
        for (int q = 0; q < kMaxGroupsPerWave; ++q) {
            if (ok && q < g_cnt) {
                const int grp = g_begin + q;
                w[q] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4 *>(wrow + static_cast<long long>(grp * 64 + fg * 16) * wmul));
                s[q] = *reinterpret_cast<const uint64_t *>(srow + grp * 4);
            } else {
                w[q] = u32x4{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
                s[q] = 0;
            }
        }
    };

    load_tile(t_begin, wcur, scur);
    int buf = 0;
    for (int t = t_begin; t < t_end; ++t) {
        load_tile(t + 1, wnext, snext);

        f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int q = 0; q < kMaxGroupsPerWave; ++q) {
            if (q < g_cnt) {
                uint32_t p[4] = {wcur[q][0], wcur[q][1], wcur[q][2], wcur[q][3]};
                if constexpr ((PK & PK_B) == 0) {
                    transpose_lane_groups(p);  // packed weights are stored transposed already
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f16x8 wb = unpack_q8(p[j]);
                    const uint16_t sbits = static_cast<uint16_t>(scur[q] >> (16 * j));
                    const float sf = static_cast<float>(__builtin_bit_cast(_Float16, sbits));
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt) {
                        const f32x4 part = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            fa[q * 4 + j][mt], wb, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            acc[mt][r] = __builtin_fmaf(part[r], sf, acc[mt][r]);
                        }
                    }
                }
            }
        }
        // partial of this wave: rows 16*mt + 4*fg + r, column fr
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s_part[buf][wave][mt * 16 + 4 * fg + r][fr] = acc[mt][r];
            }
        }
        __syncthreads();
        {
            const int orow = tid >> 4;  // 0..31
            const int ocol = tid & 15;
            const int gm = mg0 + orow;
            const int gn = t * kNTile + ocol;
            if (gm < a.M && gn < a.N) {
                float v = 0.f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    v += s_part[buf][w][orow][ocol];
                }
                if (a.C) {
                    v += load_out<OUT>(a.C, static_cast<long long>(gm) * a.ldc + gn);
                }
                if (a.bias) {
                    v += load_out<OUT>(a.bias, gn);
                }
                v = fmaxf(v, a.cmin);
                v = fminf(v, a.cmax);
                store_out<OUT>(a.D, static_cast<long long>(gm) * a.ldd + gn, v);
            }
        }
        buf ^= 1;
#pragma unroll
        for (int q = 0; q < kMaxGroupsPerWave; ++q) {
            wcur[q] = wnext[q];
            scur[q] = snext[q];
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Chunk-stream kernel (bl == 32, k % 512 == 0): one workgroup of 16 wave64s per CU owns up to
// four consecutive 16-channel tiles for one group of 32 activation rows and walks k in chunks of
// 512 (sixteen 32-k scale blocks). A chunk -- the 32 rows' 512 activations (32 KiB of f16), the
// tiles' 256 weight bytes per channel (16 KiB) and their 16 scales per channel (2 KiB) -- lands
// in one slot of a three-slot LDS ring by direct global -> LDS loads, two chunks ahead of the one
// being computed, so the whole CU computes behind one stream. Every wave loads two KiB of each
// chunk's activations and a quarter of one tile's weights; waves 0 and 1 also load the scales.
// Wave w computes scale block w of every chunk for all the tiles, so each activation byte is
// read from LDS once and its fragment (permuted once) serves four tiles: per block and tile one
// weight dword per lane (its 8-k slice of the block for one channel), the exact nibble -> f16
// q - 8 decode, two v_mfma_f32_16x16x32_f16 (rows 0-15, 16-31) and the block's f32 partials
// times the block's f16 scale accumulated in f32 -- the per-block scaling of the reference
// test's oracle. At the end the sixteen block partials of each output are added in f64 in block
// order (a fixed order: the result does not depend on timing) and rounded to f32 once; then C,
// bias (both read before the loop), clamp, store.
// LDS layout of a slot (bank-conflict-free reads):
//   activations: row r's 16-byte chunk c (k 8c .. 8c + 7 of the chunk) at slot r * 64 + (c ^ (r & 15)),
//     packed activations chunk-major (chunk c of row r at slot c * 32 + r, as in the panel);
//   plain weights: channel ch of tile t at t * 4096 + ch * 256, block b's 16 bytes at slot b ^ ch;
//   packed weights: the tile's 4 KiB of the chunk as they lie in the panel (16-byte chunk s of
//     row r at (16 s + r) * 16; chunk s holds dword s & 3 of blocks 4 (s >> 2) .. + 3);
//   scales: channel ch's 8 f16 of blocks 8h .. 8h + 7 at h * 1024 + ch * 16.
// Loads are inline asm (no compiler-placed waits, see dma_lds16); the loop waits for its own
// loads with an explicit vmcnt and meets the other waves at one barrier per chunk, after which
// the slot everyone finished in the previous chunk is refilled.
// ---------------------------------------------------------------------------------------------
constexpr int kCsWaves = 16;                         // wave64s per workgroup
constexpr int kCsTiles = 4;                          // tiles per workgroup at most
constexpr int kCsK = 512;                            // k per chunk
constexpr int kCsBlocks = kCsK / 32;                 // scale blocks per chunk (one per wave)
constexpr int kCsA = kMRows * kCsK * 2;              // activation bytes per chunk (32 KiB)
constexpr int kCsW = kCsTiles * kNTile * (kCsK / 2); // weight bytes per chunk (16 KiB)
constexpr int kCsS = kCsTiles * kNTile * kCsBlocks * 2;  // scale bytes per chunk (2 KiB)
constexpr int kCsSlot = kCsA + kCsW + kCsS;
constexpr int kCsRing = 3;                           // ring slots (chunks in flight + 1)

// 8 nibbles (k = 0..7 of one block slice, nibble i at bits 4i) -> 8 exact f16 values q - 8 in
// permute_a's slot order k = 0, 4, 1, 5, 2, 6, 3, 7. Nibbles 0, 4 (2, 6) keep their place and
// become 1024 + q; nibbles 1, 5 (3, 7) stay at bits 4-7 / 20-23 and become 1024 + 16 q, which
// one exact fma scales back (h / 16 - 72 = q - 8).
__device__ __forceinline__ f16x8 unpack_q8_lds(uint32_t x, uint32_t magic)
{
    const f16x2 bias = f16x2{static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    const f16x2 sixteenth = f16x2{static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
    const f16x2 bias16 = f16x2{static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
    const uint32_t y = x >> 8;
    const f16x2 h0 = __builtin_bit_cast(f16x2, (x & 0x000f000fu) | (magic & ~0x000f000fu)) + bias;
    const f16x2 h1 = __builtin_elementwise_fma(
        __builtin_bit_cast(f16x2, (x & 0x00f000f0u) | (magic & ~0x00f000f0u)), sixteenth, bias16);
    const f16x2 h2 = __builtin_bit_cast(f16x2, (y & 0x000f000fu) | (magic & ~0x000f000fu)) + bias;
    const f16x2 h3 = __builtin_elementwise_fma(
        __builtin_bit_cast(f16x2, (y & 0x00f000f0u) | (magic & ~0x00f000f0u)), sixteenth, bias16);
    return f16x8{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
}

// s_waitcnt until at most n (wave-uniform, 0 .. 23) of the wave's vector memory operations are
// pending (vmcnt counts loads, LDS-DMA loads and stores in issue order).
__device__ __forceinline__ void wait_vm_upto(int n)
{
    switch (n) {
#define TQT_VM_CASE(v)                                                                             \
    case v: __builtin_amdgcn_s_waitcnt(waitcnt_vm0(v)); break;
        TQT_VM_CASE(0) TQT_VM_CASE(1) TQT_VM_CASE(2) TQT_VM_CASE(3) TQT_VM_CASE(4) TQT_VM_CASE(5)
        TQT_VM_CASE(6) TQT_VM_CASE(7) TQT_VM_CASE(8) TQT_VM_CASE(9) TQT_VM_CASE(10) TQT_VM_CASE(11)
        TQT_VM_CASE(12) TQT_VM_CASE(13) TQT_VM_CASE(14) TQT_VM_CASE(15) TQT_VM_CASE(16)
        TQT_VM_CASE(17) TQT_VM_CASE(18) TQT_VM_CASE(19) TQT_VM_CASE(20) TQT_VM_CASE(21)
        TQT_VM_CASE(22)
#undef TQT_VM_CASE
    default: __builtin_amdgcn_s_waitcnt(waitcnt_vm0(23)); break;
    }
    asm volatile("" ::: "memory");
}

template <int PK, int OUT, int NS>
__global__ __launch_bounds__(1024) void w4a16_chunk_kernel(W4A16Args a, int nwg)
{
    static_assert(NS >= 2 && 4 * (NS - 1) <= 23, "ring depth");
    static_assert(kCsWaves == kCsBlocks && kCsA == 2 * kCsWaves * 1024 &&
                      kCsW == kCsWaves * 1024 && kCsS == 2 * 1024, "load roles");
    static_assert(NS * kCsSlot >= kCsBlocks * kCsTiles * kMRows * kNTile * 4,
                  "partials fit the ring");
    __shared__ __attribute__((aligned(16))) int8_t s_ring[NS][kCsSlot];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int fr = lane & 15;
    const int fg = lane >> 4;
    const int mg0 = blockIdx.y * kMRows;
    const int t_begin = static_cast<int>((static_cast<long long>(blockIdx.x) * a.ntiles) / nwg);
    const int t_end = static_cast<int>((static_cast<long long>(blockIdx.x + 1) * a.ntiles) / nwg);
    const int ntl = t_end - t_begin;  // 1 .. kCsTiles
    const int nch = a.K / kCsK;

    // This thread's outputs (local tile t = tid / 256, rows u / 16 and u / 16 + 16, column
    // u % 16): bias and C read now, ahead of every ring load, so the epilogue waits for nothing.
    const int et = tid >> 8;
    const int erow = (tid >> 4) & 15;
    const int gn = (t_begin + et) * kNTile + (tid & 15);
    const bool out_col = et < ntl && gn < a.N;
    // Read as raw bits from clamped addresses with no branch, so that no conversion, and no
    // wait for these loads, stands before the ring loads; an absent operand reads the first
    // activation instead (never used).
    const int gn_ld = min(gn, a.N - 1);
    const void *dummy = a.A;
    const uint32_t e_bias = load_out_bits<OUT>(a.bias ? a.bias : dummy, a.bias ? gn_ld : 0);
    uint32_t e_c[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const int gm = min(mg0 + mt * 16 + erow, a.M - 1);  // rows past m are not stored
        e_c[mt] = load_out_bits<OUT>(a.C ? a.C : dummy,
                                     a.C ? static_cast<long long>(gm) * a.ldc + gn_ld : 0);
    }

    // Load roles. Activations, two KiB per wave: plain rows 2w, 2w + 1 (lane i takes the row's
    // chunk i ^ (r & 15)); packed panels chunk-major, so chunks 4w .. 4w + 3 of all 32 rows
    // (lane i of load h takes chunk 4w + 2h + i / 32 of row i % 32: one contiguous KiB). Rows
    // past m read row m - 1 (their outputs are not stored).
    const uint8_t *a_src[2];
    long long a_step;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        int amul;
        if constexpr ((PK & PK_A) != 0) {
            const int r = lane & 31;
            const int ck = 4 * wave + 2 * h + (lane >> 5);
            a_src[h] = a_row_ptr<PK>(a, min(mg0 + r, a.M - 1), amul) +
                       static_cast<long long>(ck * 16) * amul;
        } else {
            const int r = 2 * wave + h;
            a_src[h] = a_row_ptr<PK>(a, min(mg0 + r, a.M - 1), amul) +
                       static_cast<long long>((lane ^ (r & 15)) * 16) * amul;
        }
        a_step = 1024ll * amul;  // bytes per chunk (the same for both loads)
    }
    // Weights: quarter p = w & 3 of tile w >> 2. A workgroup with fewer than four tiles loads
    // its last tile again in place of the missing ones, so every wave issues the same loads for
    // every chunk (and computes four tiles; the missing tiles' outputs are not stored).
    const uint8_t *w_src;
    long long w_step;
    {
        const int t = t_begin + min(wave >> 2, ntl - 1);
        const int p = wave & 3;
        int wmul;
        if constexpr ((PK & PK_B) != 0) {
            // packed chunk 4p + i / 16 of row i % 16: one contiguous KiB of a whole panel
            const uint8_t *rb = b_row_ptr<PK>(a, min(t * kNTile + fr, a.N - 1), wmul);
            w_src = rb + static_cast<long long>(16 * (4 * p + (lane >> 4))) * wmul;
            w_step = 256ll * wmul;
        } else {
            // channel ch = 4p + i / 16, block (i % 16) ^ ch: four whole 256-byte row pieces
            const int ch = 4 * p + (lane >> 4);
            const uint8_t *rb = b_row_ptr<PK>(a, min(t * kNTile + ch, a.N - 1), wmul);
            w_src = rb + 16 * ((lane & 15) ^ ch);
            w_step = 256;
        }
    }
    // Scales: waves 0 and 1, lane i -> channel i % 16 of tile i / 16, blocks 8w .. 8w + 7.
    const _Float16 *s_src = a.scale_b;
    if (wave < 2) {
        const int t = min(t_begin + (lane >> 4), t_end - 1);
        s_src = a.scale_b + static_cast<long long>(min(t * kNTile + fr, a.N - 1)) * a.ldsb +
                8 * wave;
    }
    const bool s_role = wave < 2;

    auto issue = [&](int c, int sl) {
        int8_t *base = &s_ring[sl][0];
        dma_lds16(reinterpret_cast<const int8_t *>(a_src[0] + c * a_step), base + wave * 2048);
        dma_lds16(reinterpret_cast<const int8_t *>(a_src[1] + c * a_step),
                  base + wave * 2048 + 1024);
        dma_lds16(reinterpret_cast<const int8_t *>(w_src + c * w_step), base + kCsA + wave * 1024);
        if (s_role) {
            dma_lds16(reinterpret_cast<const int8_t *>(s_src + kCsBlocks * c),
                      base + kCsA + kCsW + wave * 1024);
        }
    };

    // Compute role: block b = w of every chunk, every tile of the workgroup.
    const int b = wave;
    // rows 0-15 and 16-31 of chunk 4b + fg (plain: row-major, swizzled; packed: chunk-major)
    const int a_off0 = (PK & PK_A) != 0 ? ((4 * b + fg) * 32 + fr) * 16
                                        : (fr * 64 + ((4 * b + fg) ^ fr)) * 16;
    const int a_off1 = a_off0 + ((PK & PK_A) != 0 ? 16 * 16 : 16 * 64 * 16);
    int w_off[kCsTiles], s_off[kCsTiles];
#pragma unroll
    for (int t = 0; t < kCsTiles; ++t) {
        if constexpr ((PK & PK_B) != 0) {
            w_off[t] = kCsA + t * 4096 + ((4 * (b >> 2) + fg) * 16 + fr) * 16 + 4 * (b & 3);
        } else {
            w_off[t] = kCsA + t * 4096 + fr * 256 + ((b ^ fr) * 16) + 4 * fg;
        }
        s_off[t] = kCsA + kCsW + (b >> 3) * 1024 + (t * kNTile + fr) * 16 + (b & 7) * 2;
    }
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));

    f32x4 acc[kCsTiles][2];
#pragma unroll
    for (int t = 0; t < kCsTiles; ++t) {
        acc[t][0] = f32x4{0.f, 0.f, 0.f, 0.f};
        acc[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int npro = min(NS - 1, nch);
    for (int c = 0; c < npro; ++c) {
        issue(c, c);
    }
#pragma unroll 1
    for (int c = 0; c < nch; ++c) {
        // this wave's loads of chunk c are in (later chunks may still be in flight), and every
        // wave's reads of chunk c - 1 are done: meet, then refill chunk c - 1's slot
        // (loads per chunk: 3, and 4 for the scale loaders; 0 pending after the last chunk)
        const int ahead = min(NS - 2, nch - 1 - c);
        if (ahead == 0) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm0(0));
        } else if (s_role) {
            wait_vm_upto(4 * ahead);
        } else {
            wait_vm_upto(3 * ahead);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (c + NS - 1 < nch) {
            issue(c + NS - 1, (c + NS - 1) % NS);
        }
        const int8_t *slot = &s_ring[c % NS][0];
        const f16x8 fa0 = permute_a(*reinterpret_cast<const u32x4 *>(slot + a_off0));
        const f16x8 fa1 = permute_a(*reinterpret_cast<const u32x4 *>(slot + a_off1));
        uint32_t wd[kCsTiles];
        uint16_t sb[kCsTiles];
#pragma unroll
        for (int t = 0; t < kCsTiles; ++t) {
            wd[t] = *reinterpret_cast<const uint32_t *>(slot + w_off[t]);
            sb[t] = *reinterpret_cast<const uint16_t *>(slot + s_off[t]);
        }
#pragma unroll
        for (int t = 0; t < kCsTiles; ++t) {
            const float sf = static_cast<float>(__builtin_bit_cast(_Float16, sb[t]));
            const f16x8 wq = unpack_q8_lds(wd[t], magic);
            const f32x4 p0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                fa0, wq, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            const f32x4 p1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                fa1, wq, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                acc[t][0][r] = __builtin_fmaf(p0[r], sf, acc[t][0][r]);
                acc[t][1][r] = __builtin_fmaf(p1[r], sf, acc[t][1][r]);
            }
        }
    }

    // Partials of block b for local tile t: output (mt, r) of lane L at
    // ((b * kCsTiles + t) * 8 + 4 mt + r) * 64 + L (consecutive lanes, consecutive words).
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    float *part = reinterpret_cast<float *>(&s_ring[0][0]);
#pragma unroll
    for (int t = 0; t < kCsTiles; ++t) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                part[((b * kCsTiles + t) * 8 + 4 * mt + r) * 64 + lane] = acc[t][mt][r];
            }
        }
    }
    __syncthreads();

    if (out_col) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const int gm = mg0 + mt * 16 + erow;
            if (gm < a.M) {
                const int idx = (4 * mt + (erow & 3)) * 64 + (erow >> 2) * 16 + (tid & 15);
                double s = 0.0;
#pragma unroll
                for (int bb = 0; bb < kCsBlocks; ++bb) {
                    s += static_cast<double>(part[(bb * kCsTiles + et) * 8 * 64 + idx]);
                }
                float v = static_cast<float>(s);
                if (a.C) {
                    v += out_from_bits<OUT>(e_c[mt]);
                }
                if (a.bias) {
                    v += out_from_bits<OUT>(e_bias);
                }
                v = fmaxf(v, a.cmin);
                v = fminf(v, a.cmax);
                store_out<OUT>(a.D, static_cast<long long>(gm) * a.ldd + gn, v);
            }
        }
    }
}

// Generic path: the reference test oracle's operation order, one thread per output
// (acc = C; acc += a * (f32(q - 8) * f32(s)) in k order without FMA; acc += bias; clamp).
template <int PK, int OUT>
__global__ __launch_bounds__(256) void w4a16_generic_kernel(W4A16Args a)
{
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<long long>(a.M) * a.N) {
        return;
    }
    const int gm = static_cast<int>(idx / a.N);
    const int gn = static_cast<int>(idx - static_cast<long long>(gm) * a.N);
    float acc = 0.f;
    if (a.C) {
        acc = load_out<OUT>(a.C, static_cast<long long>(gm) * a.ldc + gn);
    }
    const _Float16 *arow = a.A + static_cast<long long>(gm) * a.lda;
    const uint8_t *brow = a.B + static_cast<long long>(gn) * a.bstride;
    const _Float16 *srow = a.scale_b + static_cast<long long>(gn) * a.ldsb;
    // packed operands: the run functions describe an unpacked one with step 0 (row-major)
    const PackRow ra = pack_row_info(a.pa, gm);
    const PackRow rb = pack_row_info(a.pb, gn);
    for (int p = 0; p < a.K; ++p) {
        const uint8_t byte =
            (PK & PK_B) ? a.B[pack_row_byte(rb, w4a16_frag_pos(p >> 1, rb.kbytes))] : brow[p >> 1];
        const int q = (p & 1) ? (byte >> 4) - 8 : (byte & 0xf) - 8;
        const float s = static_cast<float>(srow[p / a.bl]);
        const float bd = __fmul_rn(static_cast<float>(q), s);
        const _Float16 av =
            (PK & PK_A) ? *reinterpret_cast<const _Float16 *>(
                              reinterpret_cast<const uint8_t *>(a.A) + pack_row_byte(ra, 2ll * p))
                        : arow[p];
        acc = __fadd_rn(acc, __fmul_rn(static_cast<float>(av), bd));
    }
    if (a.bias) {
        acc = __fadd_rn(acc, load_out<OUT>(a.bias, gn));
    }
    acc = (acc < a.cmin) ? a.cmin : acc;
    acc = (a.cmax < acc) ? a.cmax : acc;
    store_out<OUT>(a.D, static_cast<long long>(gm) * a.ldd + gn, acc);
}

int device_cu_count()
{
    int dev = 0;
    TQT_HIP_CHECK(hipGetDevice(&dev));
    int cus = 0;
    TQT_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    return cus > 0 ? cus : 1;
}

// Shared body of the W4A16 runs. OUT: OUT_F16 (C, bias, D f16) or OUT_F32 (C, bias, D f32);
// the clamp bounds arrive widened to f32. `packed`: A (f16 rows) and B (int4 rows,
// fragment-ordered) are in the packed layout; k_idx_a / k_idx_b apply the packers' tail rule.
template <int OUT>
void w4a16_run(size_t m, size_t n, size_t k, size_t bl, const void *A, size_t lda,
               size_t k_idx_a, const void *B, size_t ldb, size_t k_idx_b, const void *scale_b,
               size_t ldsb, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
               float clamp_min, float clamp_max, bool packed, hipStream_t s, const char *where)
{
    if (m == 0 || n == 0) {
        return;
    }
    // reference …qsi4c2t_8x2vl_rvv.h:59 / .cpp:38-40: bl even and >= 2, k % bl == 0
    TQT_REQUIRE(bl >= 2 && bl % 2 == 0, "bl >= 2 && bl % 2 == 0");
    TQT_REQUIRE(k % bl == 0, "k % bl == 0");
    TQT_REQUIRE(m < (1u << 31) && n < (1u << 31) && k < (1u << 31), "dimension exceeds 2^31-1");
    TQT_REQUIRE((A && B && scale_b) || k == 0, "A/B/scale_b == NULL");
    TQT_REQUIRE(D != nullptr, "D == NULL");
    W4A16Args a = {};
    a.M = static_cast<int>(m);
    a.N = static_cast<int>(n);
    a.K = static_cast<int>(k);
    a.ntiles = static_cast<int>((n + kNTile - 1) / kNTile);
    a.A = static_cast<const _Float16 *>(A);
    a.lda = static_cast<long long>(lda);
    a.B = static_cast<const uint8_t *>(B);
    a.bstride = static_cast<long long>(ldb / 2);
    a.scale_b = static_cast<const _Float16 *>(scale_b);
    a.ldsb = static_cast<long long>(ldsb);
    a.C = C;
    a.ldc = static_cast<long long>(ldc);
    a.D = D;
    a.ldd = static_cast<long long>(ldd);
    a.bias = bias;
    a.cmin = clamp_min;
    a.cmax = clamp_max;
    a.bl = static_cast<int>(bl);
    bool layout_fast;
    if (packed) {
        TQT_REQUIRE(lda >= k && ldb >= k && ldb % 2 == 0 && k_idx_b % 2 == 0,
                    "packed W4A16 needs lda, ldb >= k and even ldb, k_idx_b");
        a.pa = make_pack(kPackW4A16MStep, kPackW4A16Chunk, m, 2 * lda, 2 * k, 2 * k_idx_a);
        a.pb = make_pack(kPackW4A16NStep, kPackW4A16Chunk, n, ldb / 2, k / 2, k_idx_b / 2);
        // every 16-byte chunk of a packed row starts 16-byte aligned
        layout_fast = ((2 * k_idx_a) % 16 == 0) && ((k_idx_b / 2) % 16 == 0);
    } else {
        a.pa = make_pack(0, kPackW4A16Chunk, m, 2 * lda, 2 * k, 0);
        a.pb = make_pack(0, kPackW4A16Chunk, n, ldb / 2, k / 2, 0);
        layout_fast = lda % 8 == 0 && (ldb / 2) % 16 == 0;
    }
    const bool fast = bl == 32 && k % 128 == 0 && k <= 128u * kWaves * kMaxGroupsPerWave &&
                      layout_fast && ldsb % 4 == 0 && aligned16(A) && aligned16(B) &&
                      (reinterpret_cast<uintptr_t>(scale_b) & 7u) == 0;
    // bl 32 and k % 512 == 0: the chunk-stream kernel
    const bool chunk = bl == 32 && k % kCsK == 0 && k >= kCsK && layout_fast && ldsb % 8 == 0 &&
                       aligned16(A) && aligned16(B) && aligned16(scale_b);
    if (chunk) {
        const int cus = device_cu_count();  // the current device, per call (no cached state)
        const long long need = (a.ntiles + kCsTiles - 1) / kCsTiles;
        const long long nwg = need > cus ? need : (a.ntiles < cus ? a.ntiles : cus);
        const unsigned long long gy = (m + kMRows - 1) / kMRows;
        TQT_REQUIRE(gy < 65536 && nwg < (1ll << 31), "grid too large");
        const dim3 grid(static_cast<unsigned>(nwg), static_cast<unsigned>(gy));
        const int nw = static_cast<int>(nwg);
        if (packed) {
            hipLaunchKernelGGL((w4a16_chunk_kernel<PK_AB, OUT, kCsRing>), grid, dim3(1024), 0, s,
                               a, nw);
        } else {
            hipLaunchKernelGGL((w4a16_chunk_kernel<PK_NONE, OUT, kCsRing>), grid, dim3(1024), 0,
                               s, a, nw);
        }
    } else if (fast) {
        const int cus = device_cu_count();  // the current device, per call (no cached state)
        const int gx = a.ntiles < cus ? a.ntiles : cus;
        const unsigned long long gy = (m + kMRows - 1) / kMRows;
        TQT_REQUIRE(gy < 65536, "m too large");
        const dim3 grid(gx, static_cast<unsigned>(gy));
        if (packed) {
            hipLaunchKernelGGL((w4a16_mfma_kernel<PK_AB, OUT>), grid, dim3(512), 0, s, a);
        } else {
            hipLaunchKernelGGL((w4a16_mfma_kernel<PK_NONE, OUT>), grid, dim3(512), 0, s, a);
        }
    } else {
        const long long total = static_cast<long long>(m) * static_cast<long long>(n);
        const long long blocks = (total + 255) / 256;
        TQT_REQUIRE(blocks < (1ll << 31), "grid too large");
        const dim3 grid(static_cast<unsigned>(blocks));
        if (packed) {
            hipLaunchKernelGGL((w4a16_generic_kernel<PK_AB, OUT>), grid, dim3(256), 0, s, a);
        } else {
            hipLaunchKernelGGL((w4a16_generic_kernel<PK_NONE, OUT>), grid, dim3(256), 0, s, a);
        }
    }
    check_launch(where);
}

}  // namespace
}  // namespace tqt

using namespace tqt;

extern "C" {

// Steps set only a caller's tile stride and the getters' alignment check (the run accepts any m
// and n), so they are launch-sized: 32 rows by 16384 channels.
static const size_t kW4A16MStep = 32;
static const size_t kW4A16NStep = 16384;

size_t tqt_get_m_step_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(void)
{
    return kW4A16MStep;
}
size_t tqt_get_n_step_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(void)
{
    return kW4A16NStep;
}
size_t tqt_get_a_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(size_t m_idx, size_t k_idx,
                                                                       size_t lda, size_t bl)
{
    TQT_REQUIRE(m_idx % kW4A16MStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(bl >= 2 && bl % 2 == 0, "bl >= 2 && bl % 2 == 0");
    TQT_REQUIRE(k_idx % bl == 0, "k_idx % bl == 0");
    return (m_idx * lda + k_idx) * sizeof(float16_t);
}
size_t tqt_get_b_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(size_t n_idx, size_t k_idx,
                                                                       size_t ldb, size_t bl)
{
    TQT_REQUIRE(n_idx % kW4A16NStep == 0, "n_idx % n_step == 0");
    TQT_REQUIRE(bl >= 2 && bl % 2 == 0, "bl >= 2 && bl % 2 == 0");
    TQT_REQUIRE(k_idx % bl == 0, "k_idx % bl == 0");
    return n_idx * (ldb / 2) + k_idx / 2;
}
size_t tqt_get_scale_b_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(size_t n_idx,
                                                                             size_t b_idx,
                                                                             size_t ldsb)
{
    TQT_REQUIRE(n_idx % kW4A16NStep == 0, "n_idx % n_step == 0");
    return (n_idx * ldsb + b_idx) * sizeof(float16_t);
}
size_t tqt_get_c_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(size_t m_idx, size_t n_idx,
                                                                       size_t ldc)
{
    TQT_REQUIRE(m_idx % kW4A16MStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kW4A16NStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldc + n_idx) * sizeof(float16_t);
}
size_t tqt_get_bias_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(size_t n_idx)
{
    TQT_REQUIRE(n_idx % kW4A16NStep == 0, "n_idx % n_step == 0");
    return n_idx * sizeof(float16_t);
}
size_t tqt_get_d_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(size_t m_idx, size_t n_idx,
                                                                       size_t ldd)
{
    TQT_REQUIRE(m_idx % kW4A16MStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kW4A16NStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldd + n_idx) * sizeof(float16_t);
}
size_t tqt_get_d_size_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(size_t m, size_t n)
{
    return m * n * sizeof(float16_t);
}

void tqt_run_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950_async(
    size_t m, size_t n, size_t k, size_t bl, const void *A, size_t lda, size_t k_idx_a,
    const void *B, size_t ldb, size_t k_idx_b, const void *scale_b, size_t ldsb, const void *C,
    size_t ldc, void *D, size_t ldd, const void *bias, float16_t clamp_min, float16_t clamp_max,
    void *stream)
{
    w4a16_run<OUT_F16>(m, n, k, bl, A, lda, k_idx_a, B, ldb, k_idx_b, scale_b, ldsb, C, ldc, D,
                       ldd, bias, static_cast<float>(clamp_min), static_cast<float>(clamp_max),
                       false, as_stream(stream),
              "tqt_run_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(
    size_t m, size_t n, size_t k, size_t bl, const void *A, size_t lda, size_t k_idx_a,
    const void *B, size_t ldb, size_t k_idx_b, const void *scale_b, size_t ldsb, const void *C,
    size_t ldc, void *D, size_t ldd, const void *bias, float16_t clamp_min, float16_t clamp_max)
{
    if (m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950_async(
        m, n, k, bl, A, lda, k_idx_a, B, ldb, k_idx_b, scale_b, ldsb, C, ldc, D, ldd, bias,
        clamp_min, clamp_max, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950");
}

// gemm_1xnbias_clamp_f16_f16p_qsi4c2p (reference …f16p_qsi4c2p_8x2vl_rvv.cpp:121-230; geometry
// getters and packers in packing.hip).
void tqt_run_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950_async(
    size_t m, size_t n, size_t k, size_t bl, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *scale_b, size_t ldsb,
    const void *C, size_t ldc, void *D, size_t ldd, const void *bias, float16_t clamp_min,
    float16_t clamp_max, void *stream)
{
    w4a16_run<OUT_F16>(m, n, k, bl, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, scale_b, ldsb,
                       C, ldc, D, ldd, bias, static_cast<float>(clamp_min),
                       static_cast<float>(clamp_max), true, as_stream(stream),
              "tqt_run_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(
    size_t m, size_t n, size_t k, size_t bl, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *scale_b, size_t ldsb,
    const void *C, size_t ldc, void *D, size_t ldd, const void *bias, float16_t clamp_min,
    float16_t clamp_max)
{
    if (m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950_async(
        m, n, k, bl, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, scale_b, ldsb, C, ldc, D, ldd,
        bias, clamp_min, clamp_max, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950");
}

// gemm_1xnbias_clamp_f32_f16_qsi4c2t (reference …f32_f16_qsi4c2t_8x2vl_rvv.cpp): the W4A16
// kernels with f32 C, bias, clamp bounds and D. The result is the f32 value of the reference
// test's oracle for this type (reference_gemm_quantized_weight_mixed<float16_t, float>), never
// rounded to f16.
size_t tqt_get_m_step_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(void)
{
    return kW4A16MStep;
}
size_t tqt_get_n_step_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(void)
{
    return kW4A16NStep;
}
size_t tqt_get_a_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(size_t m_idx, size_t k_idx,
                                                                       size_t lda, size_t bl)
{
    return tqt_get_a_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(m_idx, k_idx, lda, bl);
}
size_t tqt_get_b_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(size_t n_idx, size_t k_idx,
                                                                       size_t ldb, size_t bl)
{
    return tqt_get_b_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(n_idx, k_idx, ldb, bl);
}
size_t tqt_get_scale_b_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(size_t n_idx,
                                                                             size_t b_idx,
                                                                             size_t ldsb)
{
    return tqt_get_scale_b_offset_gemm_1xnbias_clamp_f16_f16_qsi4c2t_mfma_gfx950(n_idx, b_idx,
                                                                                 ldsb);
}
size_t tqt_get_c_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(size_t m_idx, size_t n_idx,
                                                                       size_t ldc)
{
    TQT_REQUIRE(m_idx % kW4A16MStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kW4A16NStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldc + n_idx) * sizeof(float);
}
size_t tqt_get_bias_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(size_t n_idx)
{
    TQT_REQUIRE(n_idx % kW4A16NStep == 0, "n_idx % n_step == 0");
    return n_idx * sizeof(float);
}
size_t tqt_get_d_offset_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(size_t m_idx, size_t n_idx,
                                                                       size_t ldd)
{
    TQT_REQUIRE(m_idx % kW4A16MStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kW4A16NStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldd + n_idx) * sizeof(float);
}
size_t tqt_get_d_size_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(size_t m, size_t n)
{
    return m * n * sizeof(float);
}

void tqt_run_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950_async(
    size_t m, size_t n, size_t k, size_t bl, const void *A, size_t lda, size_t k_idx_a,
    const void *B, size_t ldb, size_t k_idx_b, const void *scale_b, size_t ldsb, const void *C,
    size_t ldc, void *D, size_t ldd, const void *bias, float clamp_min, float clamp_max,
    void *stream)
{
    w4a16_run<OUT_F32>(m, n, k, bl, A, lda, k_idx_a, B, ldb, k_idx_b, scale_b, ldsb, C, ldc, D,
                       ldd, bias, clamp_min, clamp_max, false, as_stream(stream),
                       "tqt_run_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950(
    size_t m, size_t n, size_t k, size_t bl, const void *A, size_t lda, size_t k_idx_a,
    const void *B, size_t ldb, size_t k_idx_b, const void *scale_b, size_t ldsb, const void *C,
    size_t ldc, void *D, size_t ldd, const void *bias, float clamp_min, float clamp_max)
{
    if (m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950_async(
        m, n, k, bl, A, lda, k_idx_a, B, ldb, k_idx_b, scale_b, ldsb, C, ldc, D, ldd, bias,
        clamp_min, clamp_max, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_1xnbias_clamp_f32_f16_qsi4c2t_mfma_gfx950");
}

// gemm_1xnbias_clamp_f32_f16p_qsi4c2p (reference …f32_f16p_qsi4c2p_8x2vl_rvv.cpp; geometry
// getters and packers in packing.hip).
void tqt_run_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950_async(
    size_t m, size_t n, size_t k, size_t bl, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *scale_b, size_t ldsb,
    const void *C, size_t ldc, void *D, size_t ldd, const void *bias, float clamp_min,
    float clamp_max, void *stream)
{
    w4a16_run<OUT_F32>(m, n, k, bl, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, scale_b, ldsb,
                       C, ldc, D, ldd, bias, clamp_min, clamp_max, true, as_stream(stream),
                       "tqt_run_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950(
    size_t m, size_t n, size_t k, size_t bl, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *scale_b, size_t ldsb,
    const void *C, size_t ldc, void *D, size_t ldd, const void *bias, float clamp_min,
    float clamp_max)
{
    if (m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950_async(
        m, n, k, bl, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, scale_b, ldsb, C, ldc, D, ldd,
        bias, clamp_min, clamp_max, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950");
}

}  // extern "C"
