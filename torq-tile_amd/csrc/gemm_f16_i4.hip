// gemm_1xnbias_clamp_f16_f16_qsi4c2t (W4A16, block-quantized int4 weights) on gfx950.
//
// Three MFMA kernels share the math below: w4a16_lds_kernel (k 2048 and 4096: 16 waves per CU,
// weights streamed through per-wave LDS rings, no per-tile meeting of the waves; see its own
// comment), w4a16_regs_kernel (k 3072: whole CUs, at most four tiles each, two tiles in flight)
// and w4a16_mfma_kernel (any other k % 128 == 0, k <= 4096). In w4a16_mfma_kernel a workgroup of
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

// A slice of a strip kernel's wave: 2 * BPW 16-byte loads per lane covering 32 rows x BPW 32-k
// blocks. Plain A is loaded in whole cache lines -- load j = 2 * jp + rh of row tile mt gives lane
// L row mt * 16 + rh * 8 + L / 8, 16-byte chunk L % 8 of block pair jp -- because 16 rows x 64 B
// per instruction (the MFMA layout) runs at well under half the rate when every row is a separate
// line. Packed A is loaded straight in the MFMA layout (lane (r, g): row mt * 16 + r, chunk g of
// block j), which its chunk-major panels already make whole lines. Rows past m read row m - 1.
template <int BPW, int PK>
__device__ __forceinline__ const uint8_t *a_slice_addr(const W4A16Args &a, int mg0, int wave,
                                                       int lane, int j, int mt)
{
    int row, k;
    if constexpr ((PK & PK_A) != 0) {
        row = mg0 + mt * 16 + (lane & 15);
        k = (wave * BPW + j) * 32 + (lane >> 4) * 8;
    } else {
        row = mg0 + mt * 16 + (j & 1) * 8 + (lane >> 3);
        k = (wave * BPW + (j & ~1)) * 32 + (lane & 7) * 8;
    }
    int mul;
    const uint8_t *arow = a_row_ptr<PK>(a, min(row, a.M - 1), mul);
    return arow + 2ll * k * mul;
}

// The slice as a_slice_addr loaded it -> MFMA A fragments (k in permute_a's slot order). Plain A
// passes through `stage`, 2 KiB of LDS private to the wave: per (jp, mt) 16 rows x 128 B written
// as loaded (chunk c of row r at 16-byte slot c ^ (r & 7): conflict-free both ways) and read back
// as block 2 jp + jj, lane (r, g) taking chunk 4 jj + g of row r. Blocks [J0, J1) only (even
// bounds).
template <int BPW, int PK, int J0 = 0, int J1 = BPW>
__device__ __forceinline__ void a_slice_to_mfma(const u32x4 (&ra)[BPW][2], f16x8 (&fa)[BPW][2],
                                                int8_t *stage, int lane)
{
    static_assert(J0 % 2 == 0 && J1 % 2 == 0 && 0 <= J0 && J0 < J1 && J1 <= BPW, "block range");
    if constexpr ((PK & PK_A) != 0) {
#pragma unroll
        for (int j = J0; j < J1; ++j) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                fa[j][mt] = permute_a(ra[j][mt]);
            }
        }
    } else {
        const int wr = lane >> 3;
        const int wc = lane & 7;
        const int fr = lane & 15;
        const int fg = lane >> 4;
#pragma unroll
        for (int jp = J0 / 2; jp < J1 / 2; ++jp) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
                for (int rh = 0; rh < 2; ++rh) {
                    const int r = rh * 8 + wr;
                    *reinterpret_cast<u32x4 *>(stage + r * 128 + ((wc ^ (r & 7)) << 4)) =
                        ra[2 * jp + rh][mt];
                }
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const u32x4 v = *reinterpret_cast<const u32x4 *>(
                        stage + fr * 128 + (((4 * jj + fg) ^ (fr & 7)) << 4));
                    fa[2 * jp + jj][mt] = permute_a(v);
                }
            }
        }
    }
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
// Strip kernel (bl == 32, k 3072 here; any n): one workgroup of NW wave64s per CU owns up to four
// consecutive 16-channel tiles for one group of 32 activation rows. It loads its A slice once
// (into registers, wave w owning k-blocks [w * BPW, (w + 1) * BPW)) and streams the tiles'
// weights and scales from global memory straight into registers, 16 bytes per lane (one 32-k
// block of one channel); a 4x4 lane-group transpose gives each lane its 8-k slice of four
// consecutive blocks. NW = 8 at k 3072: two waves per SIMD, two tiles in flight (k 2048 and 4096
// take the LDS-staged kernel below: 19.3 us at the bench's k 4096 against 20.7 for this kernel
// with 16 waves, 22.4 with 8). Per tile the math is the one of w4a16_mfma_kernel above; the
// waves' f32 partials meet in LDS. The register sets rotate by unrolling, since a register copy
// would wait for the load still filling it.
// ---------------------------------------------------------------------------------------------
constexpr int kStripTiles = 4;
constexpr int kStripMaxK = 4096;

// 8 nibbles (k = 0..7 of one block slice, nibble i at bits 4i) -> 8 exact f16 values q - 8 in
// slot order k = 0, 4, 1, 5, 2, 6, 3, 7 (the order permute_a gives the activations).
// `magic` is 0x64006400 held in an SGPR, so each insert is one v_bfi_b32.
__device__ __forceinline__ f16x8 unpack_q8_sgpr(uint32_t x, uint32_t magic)
{
    const f16x2 bias = f16x2{static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    f16x8 out;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t d = ((x >> (4 * j)) & 0x000f000fu) | (magic & ~0x000f000fu);
        const f16x2 h = __builtin_bit_cast(f16x2, d) + bias;
        out[2 * j] = h[0];
        out[2 * j + 1] = h[1];
    }
    return out;
}

template <int K, int PK, int OUT, int NW>
__global__ __launch_bounds__(NW * 64) void w4a16_regs_kernel(W4A16Args a, int nwg)
{
    constexpr int BPW = K / (32 * NW);  // 32-k blocks per wave
    constexpr int NG = BPW / 4;         // 4-block groups per wave
    static_assert(BPW % 4 == 0 && BPW >= 4 && K <= kStripMaxK, "strip kernel k");
    __shared__ float s_part[NW * kMRows * kNTile];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int fr = lane & 15;
    const int fg = lane >> 4;
    const int mg0 = blockIdx.y * kMRows;

    const int t_begin = static_cast<int>((static_cast<long long>(blockIdx.x) * a.ntiles) / nwg);
    const int t_end = static_cast<int>((static_cast<long long>(blockIdx.x + 1) * a.ntiles) / nwg);
    const int ntl = t_end - t_begin;  // 1 .. kStripTiles

    // A slice of this wave (unconditional loads: all in flight together).
    u32x4 ra[BPW][2];
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            ra[j][mt] = *reinterpret_cast<const u32x4 *>(
                a_slice_addr<BPW, PK>(a, mg0, wave, lane, j, mt));
        }
    }

    struct TileRegs
    {
        u32x4 w[NG];
        uint64_t s[NG];
    };
    // Tile tl (clamped to the strip, so every call loads: a repeat hits the cache).
    auto load = [&](int tl, TileRegs &r) {
        const int t = t_begin + min(tl, ntl - 1);
        const int n = min(t * kNTile + fr, a.N - 1);
        int wmul;
        const uint8_t *wrow = b_row_ptr<PK>(a, n, wmul);
        const _Float16 *srow = a.scale_b + static_cast<long long>(n) * a.ldsb;
#pragma unroll
        for (int q = 0; q < NG; ++q) {
            const int b0 = wave * BPW + 4 * q;
            r.w[q] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4 *>(wrow + static_cast<long long>((b0 + fg) * 16) * wmul));
            r.s[q] = *reinterpret_cast<const uint64_t *>(srow + b0);
        }
    };
    // register sets in rotation: three (two tiles' loads in flight while one is computed) at
    // 8 waves; two at 16 waves, where four waves per SIMD hide the latency instead
    constexpr int kAhead = NW >= 16 ? 1 : 2;
    TileRegs r0, r1, r2;
    load(0, r0);
    if constexpr (kAhead == 2) {
        load(1, r1);
    }

    // Rows past m hold a copy of row m - 1: they only reach output rows that are not stored.
    // The wave's own partials area of s_part stages its A (no other wave touches it).
    f16x8 fa[BPW][2];
    a_slice_to_mfma<BPW, PK>(ra, fa, reinterpret_cast<int8_t *>(&s_part[wave * kMRows * kNTile]),
                             lane);
    uint32_t magic;
    asm volatile("s_mov_b32 %0, 0x64006400" : "=s"(magic));

    auto tile = [&](int tl, const TileRegs &cur, TileRegs &nxt) {
        load(tl + kAhead, nxt);
        f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int q = 0; q < NG; ++q) {
            uint32_t p[4] = {cur.w[q][0], cur.w[q][1], cur.w[q][2], cur.w[q][3]};
            if constexpr ((PK & PK_B) == 0) {
                transpose_lane_groups(p);  // packed weights are stored transposed already
            }
            // 8 waves: all four blocks' MFMAs first, then their scale FMAs (latency hidden in
            // the wave); 16 waves: block by block (fewer registers; other waves hide it)
            constexpr int JB = NW >= 16 ? 1 : 4;
#pragma unroll
            for (int j0 = 0; j0 < 4; j0 += JB) {
                f32x4 part[JB][2];
#pragma unroll
                for (int jj = 0; jj < JB; ++jj) {
                    const f16x8 wq = unpack_q8_sgpr(p[j0 + jj], magic);
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt) {
                        part[jj][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            fa[4 * q + j0 + jj][mt], wq, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    }
                }
#pragma unroll
                for (int jj = 0; jj < JB; ++jj) {
                    const uint16_t sbits = static_cast<uint16_t>(cur.s[q] >> (16 * (j0 + jj)));
                    const float sf = static_cast<float>(__builtin_bit_cast(_Float16, sbits));
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            acc[mt][r] = __builtin_fmaf(part[jj][mt][r], sf, acc[mt][r]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s_part[(wave * kMRows + mt * 16 + 4 * fg + r) * kNTile + fr] = acc[mt][r];
            }
        }
        __syncthreads();
        const int orow = tid >> 4;
        const int ocol = tid & 15;
        const int gm = mg0 + orow;
        const int gn = (t_begin + tl) * kNTile + ocol;
        if (orow < kMRows && gm < a.M && gn < a.N) {
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                v += s_part[(w * kMRows + orow) * kNTile + ocol];
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
        __syncthreads();  // s_part is rewritten by the next tile
    };
    if constexpr (kAhead == 2) {
        tile(0, r0, r2);
        if (ntl > 1) {
            tile(1, r1, r0);
        }
        if (ntl > 2) {
            tile(2, r2, r1);
        }
        if (ntl > 3) {
            tile(3, r0, r2);
        }
    } else {
        tile(0, r0, r1);
        if (ntl > 1) {
            tile(1, r1, r0);
        }
        if (ntl > 2) {
            tile(2, r0, r1);
        }
        if (ntl > 3) {
            tile(3, r1, r0);
        }
    }
}

// One C / bias element loaded by asm (no compiler-placed wait; the caller waits with s_waitcnt and
// ties the register with an empty asm): 32 bits for f32 outputs, the 16-bit pattern otherwise.
template <int OUT>
__device__ __forceinline__ uint32_t load_out_bits_async(const void *p, long long i)
{
    uint32_t v;
    if constexpr (OUT == OUT_F32) {
        asm volatile("global_load_dword %0, %1, off"
                     : "=v"(v)
                     : "v"(static_cast<const float *>(p) + i)
                     : "memory");
    } else {
        asm volatile("global_load_ushort %0, %1, off"
                     : "=v"(v)
                     : "v"(static_cast<const uint16_t *>(p) + i)
                     : "memory");
    }
    return v;
}

template <int OUT>
__device__ __forceinline__ float out_bits_to_f32(uint32_t v)
{
    if constexpr (OUT == OUT_F32) {
        return __builtin_bit_cast(float, v);
    } else if constexpr (OUT == OUT_F16) {
        return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v)));
    } else {
        return bf16_bits_to_f32(static_cast<uint16_t>(v));
    }
}

// ---------------------------------------------------------------------------------------------
// LDS-staged strip kernel (bl == 32, k 2048 or 4096): the strip kernel's math with the weight
// stream moved off the registers. One workgroup of 16 wave64s per CU owns up to four consecutive
// 16-channel tiles for one group of 32 activation rows; wave w keeps its k-slice of A (BPW 32-k
// blocks) in registers and streams that same k-slice of every tile -- 16 channels x BPW blocks of
// weights, 16 x BPW f16 scales -- into a three-slot LDS ring of its own with direct global -> LDS
// loads, three tiles ahead. No wave reads another wave's ring, so a wave starts a tile as soon as
// its own loads of it have landed and refills the slot as soon as it has read it.
// What bounds it: every CU takes in all of A (256 KiB at k 4096) besides its tiles, and the CU
// serves its waves' requests about group by group (four waves at a time), so the four wave
// groups get their A slices microseconds apart. No wave therefore waits for another: each adds
// its partials of a tile into that tile's f64 sums in LDS (ds_add_f64; the sum of 16 f32
// partials is exact in f64, so the order of arrival does not change it) and counts itself in,
// and goes on to its next tile; wave t finishes tile t (the f32 rounding of the sums, C, bias,
// clamp, store) once all 16 have counted in. Waves 0-3 get their A first and finish their own
// tiles first, so those epilogues overlap the slower waves' math. Every wave requests the first
// half of its A, tile 0, the second half, then its next tiles.
// Plain weights: one load instruction takes 8 channels x 128 B (whole lines), lane i fetching
// block (i & 7) ^ (c & 7) of channel c = i / 8, so block b of channel c lies at 16-byte slot
// b ^ (c & 7) of the channel's 128 bytes and a wave's ds_read_b128 of one block for 16 channels
// hits distinct slots; a whole packed panel's k-slice is contiguous (2 KiB) and is copied as it
// lies. Per tile: the strip kernel's decode, v_mfma_f32_16x16x32_f16 per block and scale FMA.
// ---------------------------------------------------------------------------------------------

// unpack_q8_sgpr with one shift instead of three: nibbles 1, 3 (5, 7) are inserted at bits 4-7
// (20-23), giving 1024 + 16 q, and scaled back by an exact fma (h / 16 - 72 = q - 8).
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

template <int K, int PK, int OUT>
__global__ __launch_bounds__(1024) void w4a16_lds_kernel(W4A16Args a, int nwg)
{
    constexpr int NW = 16;
    constexpr int BPW = K / (32 * NW);        // 32-k blocks per wave (8 or 4)
    constexpr int NG = BPW / 4;               // 4-block groups per wave
    constexpr int HB = BPW / 2;               // blocks per half of the A slice
    constexpr int CB = BPW * 16;              // weight bytes of one channel's k-slice
    constexpr int WSLOT = kNTile * CB;        // weight bytes per wave per tile
    constexpr int SSLOT = 256;                // scale bytes per wave per tile (one dword load)
    constexpr int SLOT = WSLOT + SSLOT;
    constexpr int NSLOT = 3;
    constexpr int NDW = WSLOT / 1024 + 1;     // loads per wave per tile
    constexpr int OUTS = kMRows * kNTile;     // outputs per tile
    static_assert(K == 2048 || K == 4096, "LDS strip kernel k");
    static_assert(kPackW4A16NStep == kNTile, "a packed weight panel is one tile");
    static_assert(kMRows == 32 && kNTile == 16 && OUTS == 8 * 64, "8 outputs per lane per tile");
    static_assert(kStripTiles * kNTile == 64, "one bias per lane of wave 0");
    static_assert(NSLOT * NDW + BPW <= 23, "wait counts");
    __shared__ __attribute__((aligned(16))) int8_t s_ring[NW][NSLOT][SLOT];
    // A staging area of each wave (2 KiB, private)
    __shared__ __attribute__((aligned(16))) int8_t s_stage[NW][2048];
    // per tile of the strip: the 16 waves' partials summed in f64 (output (mt, r) of lane L at
    // (4 mt + r) 64 + L: consecutive lanes, consecutive words) and how many waves added theirs
    __shared__ __attribute__((aligned(16))) double s_acc[kStripTiles][OUTS];
    __shared__ uint32_t s_arrived[kStripTiles];
    __shared__ float s_bias[kStripTiles * kNTile];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int fr = lane & 15;
    const int fg = lane >> 4;
    const int mg0 = blockIdx.y * kMRows;

    const int t_begin = static_cast<int>((static_cast<long long>(blockIdx.x) * a.ntiles) / nwg);
    const int t_end = static_cast<int>((static_cast<long long>(blockIdx.x + 1) * a.ntiles) / nwg);
    const int ntl = t_end - t_begin;  // 1 .. kStripTiles
    const int npro = min(ntl, NSLOT);

    // Zero the tiles' sums and arrival counts before any wave can add to them. The meeting comes
    // before any load is issued: placed after them it would wait for the last wave's last issue,
    // which the CU's address unit delays by microseconds while it takes every wave's loads.
#pragma unroll
    for (int i = tid; i < kStripTiles * OUTS; i += NW * 64) {
        (&s_acc[0][0])[i] = 0.0;
    }
    if (tid < kStripTiles) {
        s_arrived[tid] = 0u;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    // A slice of this wave, loaded by asm so that the compiler adds no wait for it: the waits
    // below count these loads with the ring's (all of them in issue order).
    u32x4 ra[BPW][2];
    auto load_a = [&](int j) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            asm volatile("global_load_dwordx4 %0, %1, off"
                         : "=v"(ra[j][mt])
                         : "v"(a_slice_addr<BPW, PK>(a, mg0, wave, lane, j, mt))
                         : "memory");
        }
    };
#pragma unroll
    for (int j = 0; j < HB; ++j) {
        load_a(j);
    }
    // The bias of every tile's 16 channels, loaded by wave 0 with A for the same reason as A (a
    // compiler-placed wait for a load issued later would drain the whole ring; C, when given, is
    // read that way in the epilogue, at that cost) and parked in LDS.
    uint32_t rb = 0;
    if (wave == 0 && a.bias) {
        const int gn = (t_begin + (lane >> 4)) * kNTile + (lane & 15);
        if ((lane >> 4) < ntl && gn < a.N) {
            rb = load_out_bits_async<OUT>(a.bias, gn);
        }
    }

    // Tiles whose weights are one whole packed panel (16 channels); a narrower last panel is
    // gathered channel by channel like plain rows, into the plain slot layout.
    auto packed_tile = [&](int t) { return (PK & PK_B) != 0 && (t + 1) * kNTile <= a.N; };
    // This wave's k-slice of tile tl into its slot sl: NDW loads.
    auto issue = [&](int tl, int sl) {
        const int t = t_begin + tl;
        int8_t *slot = &s_ring[wave][sl][0];
#pragma unroll
        for (int h = 0; h < WSLOT / 1024; ++h) {
            const uint8_t *src;
            if (packed_tile(t)) {
                int wmul;
                src = b_row_ptr<PK>(a, t * kNTile, wmul) + wave * (kNTile * CB) + h * 1024 +
                      lane * 16;
            } else {
                int c, b;
                if constexpr (BPW == 8) {
                    c = 8 * h + (lane >> 3);
                    b = (lane & 7) ^ (c & 7);
                } else {
                    c = lane >> 2;
                    b = (lane & 3) ^ (c & 3);
                }
                const int n = min(t * kNTile + c, a.N - 1);
                int wmul;
                src = b_row_ptr<PK>(a, n, wmul) + static_cast<long long>(wave * BPW + b) * 16 * wmul;
            }
            dma_lds16(reinterpret_cast<const int8_t *>(src), slot + h * 1024);
        }
        // scales: channel c's BPW f16 at c * 2 BPW (lanes past the 16 channels repeat them)
        constexpr int LPC = BPW / 2;  // lanes (dwords) per channel
        const int c = (lane / LPC) & 15;
        const int n = min(t * kNTile + c, a.N - 1);
        dma_lds4(a.scale_b + static_cast<long long>(n) * a.ldsb + wave * BPW + (lane % LPC) * 2,
                 slot + WSLOT);
    };

    // the first half of A, tile 0, the second half, then the next tiles: tile 0's first blocks
    // compute while the second half lands
    issue(0, 0);
#pragma unroll
    for (int j = HB; j < BPW; ++j) {
        load_a(j);
    }
    for (int i = 1; i < npro; ++i) {
        issue(i, i);
    }
    // In flight, oldest first: A[0, HB) + bias, tile 0 (NDW), A[HB, BPW) (BPW loads), tiles
    // 1 .. npro - 1. First half of A in:
    wait_vm_upto(npro * NDW + BPW);
#pragma unroll
    for (int j = 0; j < HB; ++j) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            asm volatile("" : "+v"(ra[j][mt]));
        }
    }
    asm volatile("" : "+v"(rb));
    if (wave == 0) {
        // read by the wave that finishes a tile, which counts itself in after wave 0 did
        s_bias[lane] = out_bits_to_f32<OUT>(rb);
    }
    // Rows past m hold a copy of row m - 1: they only reach output rows that are not stored.
    // The empty asm keeps the fragments as computed (no re-permutation inside the tile loop).
    int8_t *stage = &s_stage[wave][0];
    f16x8 fa[BPW][2];
    a_slice_to_mfma<BPW, PK, 0, HB>(ra, fa, stage, lane);
#pragma unroll
    for (int j = 0; j < HB; ++j) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            asm volatile("" : "+v"(fa[j][mt]));
        }
    }
    // the second half, once it is in (tile 0 only)
    auto second_half = [&]() {
        wait_vm_upto((npro - 1) * NDW);
#pragma unroll
        for (int j = HB; j < BPW; ++j) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                asm volatile("" : "+v"(ra[j][mt]));
            }
        }
        a_slice_to_mfma<BPW, PK, HB, BPW>(ra, fa, stage, lane);
#pragma unroll
        for (int j = HB; j < BPW; ++j) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                asm volatile("" : "+v"(fa[j][mt]));
            }
        }
    };
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));

    // This lane's outputs of a tile (MFMA layout): rows mt * 16 + fg * 4 + r, column fr. D and C
    // are addressed through buffer resources based at this workgroup's first row and ending at
    // its last row (the launcher keeps 32 rows of either under 2^31 bytes): each output's offset
    // is (row * ld + column) elements, and an output in a row past m or a column past n gets the
    // resource's size as its offset, which the range check drops, so no output is guarded by a
    // branch.
    constexpr uint32_t kOutBytes = OUT == OUT_F32 ? 4u : 2u;
    const uint32_t rows_here = static_cast<uint32_t>(min(kMRows, a.M - mg0));
    const uint32_t d_bytes = rows_here * static_cast<uint32_t>(a.ldd) * kOutBytes;
    const uint32_t c_bytes = rows_here * static_cast<uint32_t>(a.ldc) * kOutBytes;
    const __amdgpu_buffer_rsrc_t d_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        static_cast<uint8_t *>(a.D) + static_cast<long long>(mg0) * a.ldd * kOutBytes, 0,
        static_cast<int>(d_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t c_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void *>(a.C) == nullptr
            ? static_cast<void *>(a.D)
            : static_cast<uint8_t *>(const_cast<void *>(a.C)) +
                  static_cast<long long>(mg0) * a.ldc * kOutBytes,
        0, static_cast<int>(a.C ? c_bytes : 0u), 0x00020000);

    // One tile; tile 0 (FIRST, peeled off the loop) brings in the second half of A on the way.
    auto tile = [&](int tl, auto first) {
        constexpr bool FIRST = decltype(first)::value;
        const int sl = tl % NSLOT;
        // this wave's loads of tile tl have landed (later ones may still be in flight; for tile
        // 0, the second half of A too)
        wait_vm_upto(FIRST ? BPW + (npro - 1) * NDW : min(ntl - 1 - tl, NSLOT - 1) * NDW);
        const int8_t *slot = &s_ring[wave][sl][0];
        const bool panel = packed_tile(t_begin + tl);
        f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int q = 0; q < NG; ++q) {
            if constexpr (FIRST) {
                if (q == NG / 2) {
                    second_half();  // before the first group that uses it
                }
            }
            const int j = 4 * q + fg;
            int off;
            if constexpr (BPW == 8) {
                off = panel ? j * 256 + fr * 16 : fr * CB + ((j ^ (fr & 7)) << 4);
            } else {
                off = panel ? j * 256 + fr * 16 : fr * CB + ((j ^ (fr & 3)) << 4);
            }
            const u32x4 wv = *reinterpret_cast<const u32x4 *>(slot + off);
            const uint64_t sc =
                *reinterpret_cast<const uint64_t *>(slot + WSLOT + fr * (2 * BPW) + q * 8);
            uint32_t p[4] = {wv[0], wv[1], wv[2], wv[3]};
            if constexpr ((PK & PK_B) == 0) {
                transpose_lane_groups(p);  // packed weights are stored transposed already
            }
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                f16x8 wq = unpack_q8_lds(p[jj], magic);
                // this block's MFMAs after the previous block's FMAs: one block's partials live
                // at a time (four waves per SIMD hide the MFMA -> FMA latency instead)
                asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(wq));
                const uint16_t sbits = static_cast<uint16_t>(sc >> (16 * jj));
                const float sf = static_cast<float>(__builtin_bit_cast(_Float16, sbits));
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) {
                    const f32x4 part = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        fa[4 * q + jj][mt], wq, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        acc[mt][r] = __builtin_fmaf(part[r], sf, acc[mt][r]);
                    }
                }
            }
        }
        // this wave has read its slot (the MFMAs consumed it): refill it with the tile NSLOT
        // ahead
        if (tl + NSLOT < ntl) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue(tl + NSLOT, sl);
        }
        // Add this wave's partials into the tile's f64 sums and count the wave in; no wave waits
        // for another. The sums of the 16 f32 partials are exact in f64 (unless their exponents
        // span more than 25 binades), so the order in which the waves add does not change them.
        double *sum = &s_acc[tl][0];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                __hip_atomic_fetch_add(&sum[(mt * 4 + r) * 64 + lane],
                                       static_cast<double>(acc[mt][r]), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) {
            __hip_atomic_fetch_add(&s_arrived[tl], 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    };
    // Tile tl's outputs, once all 16 waves have added their partials: the sums rounded to f32
    // once, then C, bias, clamp. `counted`: false when the arrival wait gave up, and then every
    // output of the tile is written as NaN, so a lost count-in cannot leave stale outputs.
    // Each output's whole offset is the lane's vector offset (scalar offset 0): an output row
    // past m or a column past n gets the resource's size, which the range check drops.
    auto finish = [&](int tl, bool counted) {
        const double *sum = &s_acc[tl][0];
        const int gn = (t_begin + tl) * kNTile + fr;
        const float bias = a.bias ? s_bias[tl * kNTile + fr] : 0.f;
        const bool col_ok = gn < a.N;
        // all eight sums read at once (one LDS round trip), rounded to f32
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            v[e] = static_cast<float>(sum[e * 64 + lane]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t row = static_cast<uint32_t>(fg * 4 + (e >> 2) * 16 + (e & 3));
            const bool ok = col_ok && row < rows_here;
            const uint32_t d_off =
                ok ? (row * static_cast<uint32_t>(a.ldd) + static_cast<uint32_t>(gn)) * kOutBytes
                   : d_bytes;
            float x = v[e];
            if (a.C) {
                const uint32_t c_off =
                    ok ? (row * static_cast<uint32_t>(a.ldc) + static_cast<uint32_t>(gn)) * kOutBytes
                       : c_bytes;
                x += load_out_buf<OUT>(c_rsrc, c_off, 0u);
            }
            if (a.bias) {
                x += bias;
            }
            x = fmaxf(x, a.cmin);
            x = fminf(x, a.cmax);
            store_out_buf<OUT>(d_rsrc, d_off, 0u,
                               counted ? x : __builtin_bit_cast(float, 0x7fc00000u));
        }
    };
    tile(0, std::true_type{});
#pragma unroll 1
    for (int tl = 1; tl < ntl; ++tl) {
        tile(tl, std::false_type{});
    }
    // Wave w < ntl finishes tile w once the last wave has counted itself in. Waves 0-3 get their
    // A first and finish their own tiles first, so the tiles' epilogues overlap the slower
    // waves' math; only the last tile's stays on the path. Every wave counts itself in for every
    // tile without waiting for anyone, so the wait ends; the iteration cap only bounds it, and a
    // tile whose count never completes is written as NaN (the parity checks then fail).
    if (wave < ntl) {
        uint32_t in = 0;
        for (int it = 0; it < (1 << 24); ++it) {
            in = __hip_atomic_load(&s_arrived[wave], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (in == NW) {
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        asm volatile("" ::: "memory");
        finish(wave, in == NW);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm0(0));
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
    // (the strip kernels address 32 rows of D and C through 32-bit buffer offsets)
    const bool strip = bl == 32 && (k == 2048 || k == 3072 || k == 4096) && layout_fast &&
                       ldsb % 8 == 0 && aligned16(A) && aligned16(B) && aligned16(scale_b) &&
                       ldd < (1ull << 24) && ldc < (1ull << 24);
    if (strip) {
        const int cus = device_cu_count();  // the current device, per call (no cached state)
        const long long need = (a.ntiles + kStripTiles - 1) / kStripTiles;
        const long long nwg = need > cus ? need : (a.ntiles < cus ? a.ntiles : cus);
        const unsigned long long gy = (m + kMRows - 1) / kMRows;
        TQT_REQUIRE(gy < 65536 && nwg < (1ll << 31), "grid too large");
        const dim3 grid(static_cast<unsigned>(nwg), static_cast<unsigned>(gy));
        const int nw = static_cast<int>(nwg);
        // k 2048 / 4096: weights staged through LDS; k 3072: the register strip kernel (8 waves)
        if (packed) {
            if (k == 4096) {
                hipLaunchKernelGGL((w4a16_lds_kernel<4096, PK_AB, OUT>), grid, dim3(1024), 0, s, a, nw);
            } else if (k == 3072) {
                hipLaunchKernelGGL((w4a16_regs_kernel<3072, PK_AB, OUT, 8>), grid, dim3(512), 0, s, a, nw);
            } else {
                hipLaunchKernelGGL((w4a16_lds_kernel<2048, PK_AB, OUT>), grid, dim3(1024), 0, s, a, nw);
            }
        } else {
            if (k == 4096) {
                hipLaunchKernelGGL((w4a16_lds_kernel<4096, PK_NONE, OUT>), grid, dim3(1024), 0, s, a, nw);
            } else if (k == 3072) {
                hipLaunchKernelGGL((w4a16_regs_kernel<3072, PK_NONE, OUT, 8>), grid, dim3(512), 0, s, a, nw);
            } else {
                hipLaunchKernelGGL((w4a16_lds_kernel<2048, PK_NONE, OUT>), grid, dim3(1024), 0, s, a, nw);
            }
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

static const size_t kW4A16MStep = 32;
static const size_t kW4A16NStep = 16;

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
