// gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt (W4A8) on gfx950.
//
// m = 1 with k = 2048 or 4096 (plain layouts): the decode strip kernel, wavefront per N-strip
// with v_dot8_u32_u4 and DPP / lane-swap reductions (described above w4a8_strip_kernel).
//
// Fast path (decode-shaped, any m in chunks of 15 rows, k % 256 == 0): one workgroup of 8
// wave64s owns a 16-channel weight tile (16 rows of B) for one chunk of up to 15 activation
// rows; wave w owns one eighth of k.
//   * Plain weights stream in 128-bit loads shaped 8 rows x 128 bytes per wave instruction
//     (whole cache lines), are staged through wave-private LDS (16-byte chunks XOR-swizzled by
//     row) and read back in the MFMA B-operand layout. Packed weights (16-byte chunks stored
//     chunk-major in 16-row panels) load straight into the B-operand layout, 1 KB contiguous
//     per instruction, with no staging (measured faster; for the plain layout the same direct
//     loads, 16 rows x 64 bytes per instruction, are slower than the staged whole lines). Each
//     128-byte-per-row "pair" of k (two MFMA steps) is consumed as soon as its two loads land,
//     so compute overlaps the stream.
//   * Nibbles become signed bytes in two bit operations each: ((w << 4) & 0xf0f0f0f0) ^
//     0x80808080 is the byte 16 * (lo - 8) and (w & 0xf0f0f0f0) ^ 0x80808080 is 16 * (hi - 8).
//     v_mfma_i32_16x16x64_i8 then accumulates exactly 16 * sum_k a * (q - 8); the workgroup
//     sum is shifted right by 4 (exact: |16 * sum| < 2^31 for k <= 65536).
//   * Activation row `rows` of the 16-row A operand is all ones, so that accumulator row is
//     16 * sum_k (q - 8), the rsum_b of the reference; rows past it are zero.
//   * Activations are permuted to the (even k, odd k) byte order of the decoded weights. Each
//     wave stages the activation rows of its own k-slice in LDS once (up to 8 16-byte loads per
//     lane, only the chunk's real rows, issued before the weights; row slices XOR-swizzled by
//     row so the operand reads are conflict-free), with no workgroup barrier: a wave reads back
//     only what it wrote. Slices too large for that are loaded per step from global memory.
// The eight waves' partial sums meet in LDS and the reference's f32 epilogue (zero-point
// correction, two scale multiplies, C, bias, clamp; no FMA) runs per output.
#include <cfloat>

#include "tqt_hip_common.hpp"
#include "tqt_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950.h"
#include "tqt_quantize_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_gfx950.h"
#include "tqt_quantize_qai8dx_gfx950.h"

namespace tqt {
namespace {

constexpr int kRowsPerChunk = 15;  // activation rows per workgroup (one more row holds ones)
constexpr int kNTile = 16;         // weight channels per workgroup
constexpr int kWaves = 8;          // k is split eight ways inside the workgroup
constexpr int kPairK = 256;        // k values per pair (128 bytes per weight row, 2 MFMA steps)
constexpr int kPairsPerBatch = 2;  // pairs whose loads are in flight together per wave

struct W4A8Args
{
    int M, N, K;
    const int8_t *A;
    long long lda;
    const uint8_t *B;
    long long bstride;  // bytes between weight rows (= ldb / 2)
    const void *C;  // f32, f16 or bf16 elements (the kernel's OUT)
    long long ldc;
    void *D;
    long long ldd;
    const void *bias;
    float cmin, cmax;
    const float *scale_a;
    const int32_t *zp_a;
    const float *scale_b;
    PackDesc pa, pb;  // packed A / B of the p-variant (read when the kernel's PK bit is set)
};

// reference tqt_kernel_gemm_i8_i4_4x1vl_rvv.h:234-419: zp correction (int32), RNE convert, two
// separate multiplies, C then bias (separate adds), vfmax then vfmin.
__device__ __forceinline__ float epilogue_f32(int32_t acc, int32_t rsum, int32_t zp, float sa,
                                              float sb, const float *c, const float *bias,
                                              float cmin, float cmax)
{
    // Rounds after every operation: the library is built with -ffp-contract=off, since hipcc
    // would otherwise fuse a * b + c (__fmul_rn / __fadd_rn do not prevent it).
    const int32_t v = static_cast<int32_t>(static_cast<uint32_t>(acc) -
                                           static_cast<uint32_t>(zp) * static_cast<uint32_t>(rsum));
    float f = __int2float_rn(v);
    f = __fmul_rn(f, sa);
    f = __fmul_rn(f, sb);
    if (c) {
        f = __fadd_rn(f, *c);
    }
    if (bias) {
        f = __fadd_rn(f, *bias);
    }
    f = fmaxf(f, cmin);
    f = fminf(f, cmax);
    return f;
}

// 16 activation bytes -> the byte order of the decoded weights within each 8-byte group:
// (even k of bytes 0-7, odd k of bytes 0-7, even k of bytes 8-15, odd k of bytes 8-15).
__device__ __forceinline__ i32x4 permute_act16(const i32x4 v)
{
    return i32x4{static_cast<int32_t>(__builtin_amdgcn_perm(v[1], v[0], 0x06040200u)),
                 static_cast<int32_t>(__builtin_amdgcn_perm(v[1], v[0], 0x07050301u)),
                 static_cast<int32_t>(__builtin_amdgcn_perm(v[3], v[2], 0x06040200u)),
                 static_cast<int32_t>(__builtin_amdgcn_perm(v[3], v[2], 0x07050301u))};
}

// 32 activation bytes (k = 0..31 of this lane's slice) -> two MFMA operands in the byte order
// of the decoded weights: (even k of bytes 0-7, odd k of bytes 0-7, even k 8-15, odd k 8-15).
__device__ __forceinline__ void permute_act(const i32x4 v0, const i32x4 v1, i32x4 &x0, i32x4 &x1)
{
    const uint32_t b0 = v0[0], b1 = v0[1], b2 = v0[2], b3 = v0[3];
    const uint32_t b4 = v1[0], b5 = v1[1], b6 = v1[2], b7 = v1[3];
    x0[0] = static_cast<int32_t>(__builtin_amdgcn_perm(b1, b0, 0x06040200u));
    x0[1] = static_cast<int32_t>(__builtin_amdgcn_perm(b1, b0, 0x07050301u));
    x0[2] = static_cast<int32_t>(__builtin_amdgcn_perm(b3, b2, 0x06040200u));
    x0[3] = static_cast<int32_t>(__builtin_amdgcn_perm(b3, b2, 0x07050301u));
    x1[0] = static_cast<int32_t>(__builtin_amdgcn_perm(b5, b4, 0x06040200u));
    x1[1] = static_cast<int32_t>(__builtin_amdgcn_perm(b5, b4, 0x07050301u));
    x1[2] = static_cast<int32_t>(__builtin_amdgcn_perm(b7, b6, 0x06040200u));
    x1[3] = static_cast<int32_t>(__builtin_amdgcn_perm(b7, b6, 0x07050301u));
}

// 16 weight bytes (32 nibbles, low nibble = even k) -> signed bytes 16 * (q - 8), as two MFMA
// operands (lo nibbles then hi nibbles of bytes 0-7, then of bytes 8-15).
__device__ __forceinline__ void decode_w16(const u32x4 w, i32x4 &q0, i32x4 &q1)
{
    q0[0] = static_cast<int32_t>(((w[0] << 4) & 0xf0f0f0f0u) ^ 0x80808080u);
    q0[1] = static_cast<int32_t>((w[0] & 0xf0f0f0f0u) ^ 0x80808080u);
    q0[2] = static_cast<int32_t>(((w[1] << 4) & 0xf0f0f0f0u) ^ 0x80808080u);
    q0[3] = static_cast<int32_t>((w[1] & 0xf0f0f0f0u) ^ 0x80808080u);
    q1[0] = static_cast<int32_t>(((w[2] << 4) & 0xf0f0f0f0u) ^ 0x80808080u);
    q1[1] = static_cast<int32_t>((w[2] & 0xf0f0f0f0u) ^ 0x80808080u);
    q1[2] = static_cast<int32_t>(((w[3] << 4) & 0xf0f0f0f0u) ^ 0x80808080u);
    q1[3] = static_cast<int32_t>((w[3] & 0xf0f0f0f0u) ^ 0x80808080u);
}

// Dynamic LDS of the activation-staging path: kWaves slices of act_slice_bytes() bytes.
constexpr int kMaxActLoads = 8;  // 16-byte activation loads per lane, at most

__host__ __device__ inline int act_slice_bytes(int rows_max, int ppw)
{
    return rows_max * ppw * kPairK;
}

template <int kActLoads, int PK, int OUT>
__global__ __launch_bounds__(kWaves * 64) void w4a8_mfma_kernel(W4A8Args a)
{
    constexpr bool kDirect = (PK & PK_B) != 0;  // weights straight into operand registers
    constexpr bool kActInLds = kActLoads > 0;
    // per wave: one pair of staged weights (16 rows x 128 bytes), reused pair after pair; after
    // the main loop it holds the wave's 16 x 16 int32 partial sums
    __shared__ __attribute__((aligned(16))) uint8_t s_w[kWaves][2 * 1024];
    // activations of each wave's k-slice: rows_max rows of ppw * 256 bytes (dynamic size)
    extern __shared__ __attribute__((aligned(16))) int8_t s_dyn[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int fr = lane & 15;  // A-operand row (activation) / B-operand column (channel)
    const int fg = lane >> 4;  // 16-k slot group of the MFMA step
    // weight load roles: row within an 8-row load and 16-byte chunk within a 128-byte row
    // segment; 8 consecutive lanes read one row's 128 bytes, or for packed weights (16-byte chunks
    // stored chunk-major in the panel) one chunk of 8 consecutive rows
    const int r8 = (PK & PK_B) ? (lane & 7) : (lane >> 3);
    const int c8 = (PK & PK_B) ? (lane >> 3) : (lane & 7);
    const int n0 = blockIdx.x * kNTile;
    const int m0 = blockIdx.y * kRowsPerChunk;
    const int rows = min(kRowsPerChunk, a.M - m0);

    // Epilogue operands of output (orow, ocol), fetched first so they are in flight with the
    // weight stream.
    const int orow = tid >> 4;
    const int ocol = tid & 15;
    const bool out_ok = tid < 256 && orow < rows && n0 + ocol < a.N;
    float p_sb = 0.f, p_sa = 0.f, p_bias = 0.f, p_c = 0.f;
    int32_t p_za = 0;
    // output rows are addressed as the workgroup's first row (uniform, 64-bit) plus a 24-bit
    // per-thread offset (the launcher keeps ldc, ldd, lda and the weight row stride < 2^24)
    if (out_ok) {
        const int gm = m0 + orow, gn = n0 + ocol;
        p_sb = a.scale_b[gn];
        p_sa = a.scale_a[gm];
        p_za = a.zp_a[gm];
        if (a.bias) {
            p_bias = load_out<OUT>(a.bias, gn);
        }
        if (a.C) {
            p_c = load_out<OUT>(a.C, static_cast<long long>(m0) * a.ldc +
                                         __umul24(orow, static_cast<uint32_t>(a.ldc)) + gn);
        }
    }

    const int npairs = a.K / kPairK;
    const int ppw = (npairs + kWaves - 1) / kWaves;
    const int p_begin = min(npairs, wave * ppw);
    const int p_end = min(npairs, p_begin + ppw);

    const i32x4 ones = i32x4{0x01010101, 0x01010101, 0x01010101, 0x01010101};
    const i32x4 zero = i32x4{0, 0, 0, 0};
    const bool a_real = fr < rows;
    const bool a_ones = fr == rows;

    // LDS path: this wave's activation slice, rows x [p_begin, p_end) pairs (row stride
    // npw * 256 bytes), 16-byte chunk q at lane q % 64, load q / 64. Chunk c of row r is stored
    // at slot c ^ (r & 7) of the row, so the 8 lanes of a ds_read_b128 phase (rows 0-7 or 8-15,
    // same chunk) hit 8 different 16-byte slots. The loads are issued before the weights, so the
    // ds_writes below wait for these loads only (loads complete in order).
    const int npw = p_end - p_begin;
    const int a_chunks = rows * npw * 16;
    // row of chunk q (rows of npw * 16 chunks) without an integer division. On the LDS path
    // q < 64 kActLoads <= 512, so x = q / 16 < 32 and npw <= 32: (x + 0.5) / npw sits at least
    // 1/64 from the next integer while the float error is below 2^-18, and the truncation is
    // exact
    const float inv_npw = 1.0f / static_cast<float>(npw > 0 ? npw : 1);
    auto chunk_row = [&](int q) {
        return static_cast<int>((static_cast<float>(q >> 4) + 0.5f) * inv_npw);
    };
    int8_t *s_a = s_dyn + wave * act_slice_bytes(min(kRowsPerChunk, a.M), ppw);
    i32x4 a_chunk[kActInLds ? kActLoads : 1];
    if constexpr (kActInLds) {
        if (a_chunks > 0) {
#pragma unroll
            for (int j = 0; j < kActLoads; ++j) {
                // unconditional: chunks past the slice reload its last chunk (not stored)
                const int q = min(lane + 64 * j, a_chunks - 1);
                const int r = chunk_row(q);
                const int off = (q - static_cast<int>(__umul24(r, npw)) * 16) * 16;
                int mul = 1;  // k multiplier of a packed row (its panel width)
                long long base;
                if constexpr ((PK & PK_A) != 0) {
                    base = pack_row_fixed<kPackW4A8MStep>(a.pa, m0 + r, mul);
                } else {
                    base = static_cast<long long>(m0) * a.lda +
                           __umul24(r, static_cast<uint32_t>(a.lda));
                }
                a_chunk[j] = *reinterpret_cast<const i32x4 *>(
                    a.A + base +
                    pack_k<kPackW4A8Chunk, (PK & PK_A) != 0>(p_begin * kPairK + off, mul));
            }
        }
    }
    // register path: this lane's activation row (row rows - 1 for the ones/zero lanes) and the
    // two weight rows it loads
    int a_mul = 1;
    const int8_t *a_rowp = a.A;
    if constexpr (!kActInLds) {
        const int r = m0 + min(fr, rows - 1);
        if constexpr ((PK & PK_A) != 0) {
            a_rowp = a.A + pack_row_fixed<kPackW4A8MStep>(a.pa, r, a_mul);
        } else {
            a_rowp = a.A + static_cast<long long>(r) * a.lda;
        }
    }
    // staged path: rows 8 * h + r8; direct path: row fr, chunks 4 * h + fg of each pair
    const uint8_t *w_rowp[2];
    int w_mul[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int row = kDirect ? fr : 8 * h + r8;
        const int grow = n0 + row < a.N ? n0 + row : n0;
        w_mul[h] = 1;
        if constexpr ((PK & PK_B) != 0) {
            w_rowp[h] = a.B + pack_row_fixed<kPackW4A8NStep>(a.pb, grow, w_mul[h]);
        } else {
            w_rowp[h] = a.B + static_cast<long long>(n0) * a.bstride +
                        __umul24(grow - n0, static_cast<uint32_t>(a.bstride));
        }
    }

    i32x4 acc0 = zero, acc1 = zero;
    for (int pb = p_begin; pb < p_end; pb += kPairsPerBatch) {
        // activations of this batch (register path): 32 bytes per lane per step
        i32x4 av[2 * kPairsPerBatch][2];
        if constexpr (!kActInLds) {
#pragma unroll
            for (int s = 0; s < 2 * kPairsPerBatch; ++s) {
                // unconditional loads from a valid row (row rows - 1 for the ones/zero lanes)
                const int pair = min(pb + (s >> 1), p_end - 1);
                const int kb = pair * kPairK + (s & 1) * 128 + fg * 32;
                const i32x4 v0 = *reinterpret_cast<const i32x4 *>(
                    a_rowp + pack_k<kPackW4A8Chunk, (PK & PK_A) != 0>(kb, a_mul));
                const i32x4 v1 = *reinterpret_cast<const i32x4 *>(
                    a_rowp + pack_k<kPackW4A8Chunk, (PK & PK_A) != 0>(kb + 16, a_mul));
                const i32x4 fill = a_ones ? ones : zero;
                av[s][0] = a_real ? v0 : fill;
                av[s][1] = a_real ? v1 : fill;
            }
        }
        // weights of this batch: load j covers rows 8 * (j & 1) .. +8, pair pb + j / 2. The
        // loads are unconditional (a pair past the slice reloads the last one; its MFMAs are
        // skipped), so that no branch makes the compiler wait for all of them at once.
        u32x4 wr[2 * kPairsPerBatch];
#pragma unroll
        for (int j = 0; j < 2 * kPairsPerBatch; ++j) {
            const int pair = min(pb + (j >> 1), p_end - 1);
            const int chunk = kDirect ? 4 * (j & 1) + fg : c8;
            wr[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(
                w_rowp[j & 1] + pack_k<kPackW4A8Chunk, (PK & PK_B) != 0>(
                                    pair * (kPairK / 2) + chunk * 16, w_mul[j & 1])));
        }
        // keep every load of the batch ahead of the compute (the scheduler would sink them to
        // their uses and serialize the stream); emits no instruction
        asm volatile("" ::: "memory");
        if constexpr (kActInLds) {
            if (pb == p_begin) {
#pragma unroll
                for (int j = 0; j < kActLoads; ++j) {
                    const int q = lane + 64 * j;
                    if (q < a_chunks) {
                        const int r = chunk_row(q);
                        const int rn = static_cast<int>(__umul24(r, npw));
                        const int c = q - rn * 16;
                        // stored in the decoded weights' byte order (the MFMA operand as is)
                        *reinterpret_cast<i32x4 *>(&s_a[rn * 256 + ((c ^ (r & 7)) << 4)]) =
                            permute_act16(a_chunk[j]);
                    }
                }
            }
        }
#pragma unroll
        for (int pp = 0; pp < kPairsPerBatch; ++pp) {
            const int pair = pb + pp;
            if (pair >= p_end) {
                break;
            }
            // stage this pair: (row, chunk) at row * 128 + ((chunk ^ (row & 7)) << 4), rows 8-15
            // in the second KiB. The buffer is the previous pair's: this wave's LDS accesses run
            // in program order, so these writes follow its reads of that pair.
            if constexpr (!kDirect) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    *reinterpret_cast<u32x4 *>(&s_w[wave][h * 1024 + r8 * 128 + ((c8 ^ r8) << 4)]) =
                        wr[2 * pp + h];
                }
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                i32x4 v0, v1;
                if constexpr (kActInLds) {
                    if (a_real) {
                        const int c0 = ((pair - p_begin) * kPairK + h * 128 + fg * 32) >> 4;
                        const int8_t *row = &s_a[__umul24(fr, npw) * kPairK];
                        v0 = *reinterpret_cast<const i32x4 *>(row + ((c0 ^ (fr & 7)) << 4));
                        v1 = *reinterpret_cast<const i32x4 *>(row + (((c0 + 1) ^ (fr & 7)) << 4));
                    } else {
                        v0 = a_ones ? ones : zero;
                        v1 = v0;
                    }
                } else {
                    v0 = av[2 * pp + h][0];
                    v1 = av[2 * pp + h][1];
                }
                i32x4 x0, x1, q0, q1;
                if constexpr (kActInLds) {
                    x0 = v0;  // staged in operand order already
                    x1 = v1;
                } else {
                    permute_act(v0, v1, x0, x1);
                }
                if constexpr (kDirect) {
                    decode_w16(wr[2 * pp + h], q0, q1);
                } else {
                    const int rr = fr & 7;
                    const int c = 4 * h + fg;
                    decode_w16(*reinterpret_cast<const u32x4 *>(
                                   &s_w[wave][(fr >> 3) * 1024 + rr * 128 + ((c ^ rr) << 4)]),
                               q0, q1);
                }
                acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, q0, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, q1, acc1, 0, 0, 0);
            }
        }
    }

    // lane holds rows 4 * fg + r, column fr of this wave's 16x16 partial; it goes to the wave's
    // own weight buffer (its last reads of it precede these writes in program order)
    int32_t(*s_part)[16][16] = reinterpret_cast<int32_t(*)[16][16]>(&s_w[0][0]);
    constexpr int kPartStride = 2 * 1024 / (16 * 16 * 4);  // partial tiles per wave buffer
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        s_part[wave * kPartStride][4 * fg + r][fr] = acc0[r] + acc1[r];
    }
    __syncthreads();
    if (out_ok) {
        uint32_t tot = 0, rs = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            tot += static_cast<uint32_t>(s_part[w * kPartStride][orow][ocol]);
            rs += static_cast<uint32_t>(s_part[w * kPartStride][rows][ocol]);
        }
        const int gn = n0 + ocol;
        store_out<OUT>(a.D, static_cast<long long>(m0) * a.ldd +
                                __umul24(orow, static_cast<uint32_t>(a.ldd)) + gn,
                       epilogue_f32(static_cast<int32_t>(tot) >> 4, static_cast<int32_t>(rs) >> 4,
                                    p_za, p_sa, p_sb, a.C ? &p_c : nullptr,
                                    a.bias ? &p_bias : nullptr, a.cmin, a.cmax));
    }
}

// ---------------------------------------------------------------------------------------------
// Decode strip kernel (m = 1, k = 2048 or 4096, plain layouts): wavefront per N-strip.
// Wave w of the grid owns kStripC = 4 consecutive output channels over all of k and reads each
// channel's weight row with 16-byte loads, 1 KiB contiguous per wave instruction; lane l holds
// k in [2048 j + 32 l, +32) of load j for every channel, so its activations are fixed for the
// whole wave and are decoded once. The contraction runs on v_dot8_u32_u4 (eight unsigned 4-bit
// products per instruction), on the nibbles as stored:
//   * a weight nibble is u = q + 8 in [0, 15]; an activation a becomes a + 128 = 16 h + l with
//     h, l in [0, 15], packed in the weight dword's nibble order;
//   * over a lane's n terms, with H = sum u h, L = sum u l, U = sum u and S = sum a,
//     sum q a - zp sum q = 16 H + L - (128 + zp) U + 8 (zp n - S)
//     (exact in wrapping 32-bit arithmetic), so each weight dword costs three dot8 and no decode.
// The four channels' lane partials are summed across the wave together: the 32-lane swap
// folds channels (0, 2) and (1, 3) into the two halves, the 16-lane swap leaves channel c in
// row c, and four DPP steps reduce each row; lane 16 c then runs the f32 epilogue of channel c.
// No LDS, no barrier. All sums are exact, so results are bit-identical to the MFMA kernel's.
// Issue order: the zero point as a scalar load (its own counter), the activations, the
// weights, then the epilogue operands; each channel's math waits only for its own loads.
// Measured (same box, M = 1, K 4096, N 11008): 5.70 us against 6.11 us for the MFMA k-split
// kernel; 2 or 8 channels per wave, 1, 2 or 8 waves per workgroup and channels interleaved
// across the waves were slower or equal, and at m = 2 the MFMA kernel is faster (6.14 vs 6.38),
// as the dot8 work grows with the rows while the MFMA's does not.
// ---------------------------------------------------------------------------------------------
constexpr int kStripWaves = 4;  // waves per workgroup (independent; no LDS, no barrier)
constexpr int kStripC = 4;      // output channels per wave (one per row of 16 lanes)
constexpr int kStripK = 2048;   // k covered by one 16-byte load per lane (64 lanes x 32 k)

// Row sums: every lane of each row of 16 lanes gets the sum of its row (quad swaps, half-row
// mirror, row mirror).
__device__ __forceinline__ uint32_t row16_sum_u32(uint32_t v)
{
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xb1, 0xf, 0xf,
                                                           false));  // quad_perm [1,0,3,2]
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4e, 0xf, 0xf,
                                                           false));  // quad_perm [2,3,0,1]
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x141, 0xf,
                                                           0xf, false));  // row_half_mirror
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x140, 0xf,
                                                           0xf, false));  // row_mirror
    return v;
}

// Minimum / maximum of v over the 64 lanes, wave-uniform (exact: any order): DPP steps inside
// each row of 16 lanes, then the four row results read by readlane. (With the same value in
// both operands of v_permlane{16,32}_swap, the compiler dropped the min / max that combines the
// swapped halves, so the rows are combined through scalar reads instead.)
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float x)
{
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xf, 0xf, false));
}

template <bool kMax>
__device__ __forceinline__ float wave_minmax_f32(float v)
{
    auto op = [](float x, float y) { return kMax ? fmaxf(x, y) : fminf(x, y); };
    v = op(v, dpp_f32<0xb1>(v));   // quad_perm [1,0,3,2]
    v = op(v, dpp_f32<0x4e>(v));   // quad_perm [2,3,0,1]
    v = op(v, dpp_f32<0x141>(v));  // row_half_mirror
    v = op(v, dpp_f32<0x140>(v));  // row_mirror
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return op(op(r0, r1), op(r2, r3));
}
__device__ __forceinline__ float wave_min_f32(float v)
{
    return wave_minmax_f32<false>(v);
}
__device__ __forceinline__ float wave_max_f32(float v)
{
    return wave_minmax_f32<true>(v);
}

// Four per-lane values -> row c of the result holds the 64-lane sum of v[c] in every lane.
__device__ __forceinline__ uint32_t wave_sum4_u32(const uint32_t (&v)[4])
{
    // p02: lanes 0-31 hold v0 folded over the two halves, lanes 32-63 v2 (p13: v1, v3)
    const auto p02 = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
    const auto p13 = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
    const uint32_t s02 = p02[0] + p02[1];
    const uint32_t s13 = p13[0] + p13[1];
    // rows (0, 1, 2, 3) <- (v0, v1, v2, v3), each folded over four lanes
    const auto p = __builtin_amdgcn_permlane16_swap(s02, s13, false, false);
    return row16_sum_u32(p[0] + p[1]);
}

// Activation bytes k 0-3 (x0) and k 4-7 (x1) -> the nibbles of a + 128 in the weight dword's
// order (byte b: k 2b in the low nibble, k 2b + 1 in the high one): h = (a + 128) >> 4 and
// l = a & 15.
__device__ __forceinline__ void act_nibbles(uint32_t x0, uint32_t x1, uint32_t &h, uint32_t &l)
{
    const uint32_t e = __builtin_amdgcn_perm(x1, x0, 0x06040200u);  // k 0, 2, 4, 6
    const uint32_t o = __builtin_amdgcn_perm(x1, x0, 0x07050301u);  // k 1, 3, 5, 7
    h = (((e >> 4) & 0x0f0f0f0fu) | (o & 0xf0f0f0f0u)) ^ 0x88888888u;
    l = (e & 0x0f0f0f0fu) | ((o << 4) & 0xf0f0f0f0u);
}

// The strip kernel's math and epilogue for one wave: its lanes' activation bytes av (load j:
// k = 2048 j + 32 lane + 0..31), its channels' weight loads wv (channel n0 + c, load j), the
// row's zero point and scale and this lane's epilogue operands (channel n0 + lane / 16).
template <int L, int OUT>
__device__ __forceinline__ void strip_finish(const W4A8Args &a, int n0, int lane,
                                             const u32x4 (&av)[L][2], u32x4 (&wv)[kStripC][L],
                                             int32_t zp, float p_sa, float p_sb, float p_bias,
                                             float p_c)
{
    static_assert(kStripC == 4, "one channel per row of 16 lanes");
    constexpr uint32_t kTerms = 32 * L;  // k values per lane
    // activation nibbles and the constant 8 (zp n - S) of this lane
    uint32_t ah[L][4], al[L][4];
    int32_t sa = 0;
#pragma unroll
    for (int j = 0; j < L; ++j) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const u32x4 &v = av[j][d >> 1];
            const uint32_t x0 = v[2 * (d & 1)], x1 = v[2 * (d & 1) + 1];
            act_nibbles(x0, x1, ah[j][d], al[j][d]);
            sa = __builtin_amdgcn_sdot4(static_cast<int32_t>(x0), 0x01010101, sa, false);
            sa = __builtin_amdgcn_sdot4(static_cast<int32_t>(x1), 0x01010101, sa, false);
        }
    }
    const uint32_t cst = 8u * (static_cast<uint32_t>(zp) * kTerms - static_cast<uint32_t>(sa));

    uint32_t part[kStripC];
#pragma unroll
    for (int c = 0; c < kStripC; ++c) {
        // channel c's math starts after channel c - 1's: the empty asm takes the previous
        // partial and hands channel c's weights on, so the scheduler cannot hoist this
        // channel's math (and the wait for its loads) above the previous channel's
#pragma unroll
        for (int j = 0; j < L; ++j) {
            asm volatile("" : "+v"(wv[c][j]) : "v"(part[c > 0 ? c - 1 : 0]));
        }
        uint32_t hs = 0, ls = 0, us = 0;
#pragma unroll
        for (int j = 0; j < L; ++j) {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t w = wv[c][j][d];
                us = __builtin_amdgcn_udot8(w, 0x11111111u, us, false);
                hs = __builtin_amdgcn_udot8(w, ah[j][d], hs, false);
                ls = __builtin_amdgcn_udot8(w, al[j][d], ls, false);
            }
        }
        // 16 H + L - (128 + zp) U + 8 (zp n - S), wrapping (any int32 zero point)
        part[c] = (hs << 4) + ls + cst - (128u + static_cast<uint32_t>(zp)) * us;
    }
    // acc - zp rsum of the reference (mod 2^32) of channel n0 + lane / 16
    const uint32_t tot = wave_sum4_u32(part);
    const int oc = lane >> 4;
    if ((lane & 15) == 0 && n0 + oc < a.N) {
        store_out<OUT>(a.D, n0 + oc,
                       epilogue_f32(static_cast<int32_t>(tot), 0, 0, p_sa, p_sb,
                                    a.C ? &p_c : nullptr, a.bias ? &p_bias : nullptr, a.cmin,
                                    a.cmax));
    }
}

// This wave's weight loads: channel c, load j: 16 bytes at byte 1024 j + 16 lane of its row
// (channels past n reload the last channel; their outputs are not stored).
template <int L>
__device__ __forceinline__ void strip_load_weights(const W4A8Args &a, int n0, int lane,
                                                   u32x4 (&wv)[kStripC][L])
{
#pragma unroll
    for (int c = 0; c < kStripC; ++c) {
        const uint8_t *p =
            a.B + static_cast<long long>(min(n0 + c, a.N - 1)) * a.bstride + 16 * lane;
#pragma unroll
        for (int j = 0; j < L; ++j) {
            wv[c][j] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4 *>(p + j * (kStripK / 2)));
        }
    }
}

template <int L, int OUT>
__global__ __launch_bounds__(kStripWaves * 64) void w4a8_strip_kernel(W4A8Args a)
{
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = (blockIdx.x * kStripWaves + wave) * kStripC;
    if (n0 >= a.N) {
        return;  // a whole wave past the last channel (waves never wait for each other)
    }

    // the zero point (a wave-uniform scalar load: it waits on its own counter, so the vector
    // loads below are not held behind it)
    const int32_t zp = a.zp_a[0];
    // activations first, then the weights, so that the activations are decoded while the
    // weights stream (vector loads complete in order): load j holds the 32 bytes at
    // k = 2048 j + 32 lane
    u32x4 av[L][2];
    const int8_t *ap = a.A + 32 * lane;
#pragma unroll
    for (int j = 0; j < L; ++j) {
        av[j][0] = *reinterpret_cast<const u32x4 *>(ap + j * kStripK);
        av[j][1] = *reinterpret_cast<const u32x4 *>(ap + j * kStripK + 16);
    }
    u32x4 wv[kStripC][L];
    strip_load_weights<L>(a, n0, lane, wv);
    // keep every weight load ahead of what follows (the scheduler would sink them to their
    // uses and serialize the stream); emits no instruction
    asm volatile("" ::: "memory");

    // epilogue operands of channel n0 + lane / 16 (stored by lane 16 c), requested behind the
    // stream since they are needed last (channels past n read the last channel, not stored)
    const int gn = min(n0 + (lane >> 4), a.N - 1);
    const float p_sb = a.scale_b[gn];
    const float p_sa = a.scale_a[0];
    const float p_bias = a.bias ? load_out<OUT>(a.bias, gn) : 0.f;
    const float p_c = a.C ? load_out<OUT>(a.C, gn) : 0.f;
    strip_finish<L, OUT>(a, n0, lane, av, wv, zp, p_sa, p_sb, p_bias, p_c);
}

// ---------------------------------------------------------------------------------------------
// Fused decode step (m = 1, k = 2048 or 4096): the row's qai8dx quantization and the strip
// kernel in one launch. Each workgroup requests the f32 row (8 L floats per thread) ahead of its
// weights, reduces the row's minimum and maximum (wave shuffles, then LDS across the four waves),
// computes the scale and zero point exactly as tqt_run_quantize_qai8dx_f32 does, quantizes its
// threads' values into an LDS copy of the int8 row, and after one more barrier each wave reads
// its lanes' activation bytes from that copy and runs the strip math. Every workgroup computes
// the same row (min and max are exact, the per-value steps are elementwise); workgroup 0 also
// writes it, with its scale and zero point, to the caller's A_q, scale_a and zero_point_a. The
// weight loads are in flight throughout. Measured (one box, M = 1, K 4096, N 11008): 7.49 us
// against 8.3-8.5 us for the two launches and 5.6 us for the GEMV alone; the redundant per-
// workgroup quantization is what remains (16 correctly rounded divisions per thread, about
// 1 us: a copy with a plain conversion in their place took 6.5 us); a multiply by the rounded
// reciprocal with a division only near rounding ties measured slower (8.0 us, divergent
// branches), and shuffles through ds_bpermute for the min / max 0.1 us slower than DPP.
// ---------------------------------------------------------------------------------------------
template <int L, int OUT>
__global__ __launch_bounds__(kStripWaves * 64) void w4a8_qstrip_kernel(W4A8Args a,
                                                                       const float *X,
                                                                       int8_t *Aq, float *sa_out,
                                                                       int32_t *za_out)
{
    constexpr int kThreads = kStripWaves * 64;
    constexpr int kF4 = kStripK * L / (4 * kThreads);  // float4 of the row per thread
    __shared__ float s_lo[kStripWaves], s_hi[kStripWaves];
    __shared__ __attribute__((aligned(16))) int8_t s_q[kStripK * L];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    // waves past the last channel still take part in the workgroup's barriers (they reload
    // the last channel and store nothing)
    const int n0 = (blockIdx.x * kStripWaves + wave) * kStripC;

    // the f32 row first (its wait then leaves the weights in flight): float4 tid + 256 j
    f32x4 xv[kF4];
#pragma unroll
    for (int j = 0; j < kF4; ++j) {
        xv[j] = reinterpret_cast<const f32x4 *>(X)[tid + kThreads * j];
    }
    u32x4 wv[kStripC][L];
    strip_load_weights<L>(a, n0, lane, wv);
    asm volatile("" ::: "memory");
    const int gn = min(n0 + (lane >> 4), a.N - 1);
    const float p_sb = a.scale_b[gn];
    const float p_bias = a.bias ? load_out<OUT>(a.bias, gn) : 0.f;
    const float p_c = a.C ? load_out<OUT>(a.C, gn) : 0.f;

    // the row's minimum and maximum (exact: any order)
    float lo = FLT_MAX, hi = -FLT_MAX;
#pragma unroll
    for (int j = 0; j < kF4; ++j) {
        const f32x4 v = xv[j];
        lo = fminf(lo, fminf(fminf(v[0], v[1]), fminf(v[2], v[3])));
        hi = fmaxf(hi, fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
    }
    lo = wave_min_f32(lo);
    hi = wave_max_f32(hi);
    if (lane == 0) {
        s_lo[wave] = lo;
        s_hi[wave] = hi;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    lo = s_lo[0];
    hi = s_hi[0];
#pragma unroll
    for (int w = 1; w < kStripWaves; ++w) {
        lo = fminf(lo, s_lo[w]);
        hi = fmaxf(hi, s_hi[w]);
    }
    float s;
    int32_t zp;
    const bool nonzero = qai8dx_row_params(lo, hi, s, zp);
    const float zpf = static_cast<float>(zp);
    const bool writer = blockIdx.x == 0;
#pragma unroll
    for (int j = 0; j < kF4; ++j) {
        uint32_t word = 0;
        if (nonzero) {
            const f32x4 v = xv[j];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                word |= static_cast<uint32_t>(static_cast<uint8_t>(qai8dx_quantize(v[e], s, zpf)))
                        << (8 * e);
            }
        }
        const int i = tid + kThreads * j;
        *reinterpret_cast<uint32_t *>(&s_q[4 * i]) = word;
        if (writer) {
            reinterpret_cast<uint32_t *>(Aq)[i] = word;
        }
    }
    if (writer && tid == 0) {
        sa_out[0] = s;
        za_out[0] = zp;
    }
    // LDS stores visible to every wave; the weight loads stay in flight (a __syncthreads()
    // would wait for them too)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    u32x4 av[L][2];
#pragma unroll
    for (int j = 0; j < L; ++j) {
        av[j][0] = *reinterpret_cast<const u32x4 *>(&s_q[j * kStripK + 32 * lane]);
        av[j][1] = *reinterpret_cast<const u32x4 *>(&s_q[j * kStripK + 32 * lane + 16]);
    }
    strip_finish<L, OUT>(a, n0, lane, av, wv, zp, s, p_sb, p_bias, p_c);
}

// Launches the strip kernel when m and k suit it (m = 1, k = 2048 or 4096); false otherwise.
template <int OUT>
bool launch_w4a8_strip(const W4A8Args &a, hipStream_t s)
{
    if (a.M != 1 || a.K % kStripK != 0) {
        return false;
    }
    const int per_block = kStripWaves * kStripC;
    const dim3 grid(static_cast<unsigned>((a.N + per_block - 1) / per_block));
    const dim3 block(kStripWaves * 64);
    switch (a.K / kStripK) {
    case 1: hipLaunchKernelGGL((w4a8_strip_kernel<1, OUT>), grid, block, 0, s, a); return true;
    case 2: hipLaunchKernelGGL((w4a8_strip_kernel<2, OUT>), grid, block, 0, s, a); return true;
    default: return false;
    }
}

// Launches the fused decode step when it applies (m = 1, k = 2048 or 4096); false otherwise.
template <int OUT>
bool launch_w4a8_qstrip(const W4A8Args &a, const float *X, int8_t *Aq, float *sa, int32_t *za,
                        hipStream_t s)
{
    if (a.M != 1 || a.K % kStripK != 0 || a.K / kStripK > 2) {
        return false;
    }
    const int per_block = kStripWaves * kStripC;
    const dim3 grid(static_cast<unsigned>((a.N + per_block - 1) / per_block));
    const dim3 block(kStripWaves * 64);
    if (a.K == kStripK) {
        hipLaunchKernelGGL((w4a8_qstrip_kernel<1, OUT>), grid, block, 0, s, a, X, Aq, sa, za);
    } else {
        hipLaunchKernelGGL((w4a8_qstrip_kernel<2, OUT>), grid, block, 0, s, a, X, Aq, sa, za);
    }
    return true;
}

// Generic path: one thread per output, any alignment, any even k.
template <int PK, int OUT>
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
    // packed operands: the run functions describe an unpacked one with step 0 (row-major)
    const PackRow ra = pack_row_info(a.pa, gm);
    const PackRow rb = pack_row_info(a.pb, gn);
    uint32_t acc = 0, rsum = 0;
    for (int k = 0; k < a.K; k += 2) {
        const uint8_t byte = (PK & PK_B) ? a.B[pack_row_byte(rb, k >> 1)] : brow[k >> 1];
        const int32_t lo = static_cast<int32_t>(byte & 0xf) - 8;
        const int32_t hi = static_cast<int32_t>(byte >> 4) - 8;
        rsum += static_cast<uint32_t>(lo + hi);
        const int32_t a0 = (PK & PK_A) ? a.A[pack_row_byte(ra, k)] : arow[k];
        const int32_t a1 = (PK & PK_A) ? a.A[pack_row_byte(ra, k + 1)] : arow[k + 1];
        acc += static_cast<uint32_t>(a0 * lo);
        acc += static_cast<uint32_t>(a1 * hi);
    }
    const float c = a.C ? load_out<OUT>(a.C, static_cast<long long>(gm) * a.ldc + gn) : 0.f;
    const float b = a.bias ? load_out<OUT>(a.bias, gn) : 0.f;
    store_out<OUT>(a.D, static_cast<long long>(gm) * a.ldd + gn,
                   epilogue_f32(static_cast<int32_t>(acc), static_cast<int32_t>(rsum), a.zp_a[gm],
                                a.scale_a[gm], a.scale_b[gn], a.C ? &c : nullptr,
                                a.bias ? &b : nullptr, a.cmin, a.cmax));
}

template <int kActLoads, int OUT>
void launch_w4a8(dim3 grid, dim3 block, size_t lds, hipStream_t s, const W4A8Args &a, bool packed)
{
    if (packed) {
        hipLaunchKernelGGL((w4a8_mfma_kernel<kActLoads, PK_AB, OUT>), grid, block, lds, s, a);
    } else {
        hipLaunchKernelGGL((w4a8_mfma_kernel<kActLoads, PK_NONE, OUT>), grid, block, lds, s, a);
    }
}

// Shared body of the W4A8 runs. `packed`: A and B are in the packed layout (A rows of k bytes,
// B rows of k/2 bytes; k_idx_a / k_idx_b apply the packers' tail rule).
template <int OUT>
void w4a8_run(size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a,
              const void *B, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
              size_t ldd, const void *bias, float clamp_min, float clamp_max,
              const struct tqt_qai8dx_qsi4cx_params *params, bool packed, hipStream_t s,
              const char *where)
{
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
    a.C = C;
    a.ldc = static_cast<long long>(ldc);
    a.D = D;
    a.ldd = static_cast<long long>(ldd);
    a.bias = bias;
    a.cmin = clamp_min;
    a.cmax = clamp_max;
    a.scale_a = params->scale_a;
    a.zp_a = params->zero_point_a;
    a.scale_b = params->scale_b;
    bool layout_fast;
    if (packed) {
        TQT_REQUIRE(lda >= k && ldb >= k && ldb % 2 == 0 && k_idx_b % 2 == 0,
                    "packed W4A8 needs lda, ldb >= k and even ldb, k_idx_b");
        a.pa = make_pack(kPackW4A8MStep, kPackW4A8Chunk, m, lda, k, k_idx_a);
        a.pb = make_pack(kPackW4A8NStep, kPackW4A8Chunk, n, ldb / 2, k / 2, k_idx_b / 2);
        // every 16-byte chunk of a packed row starts 16-byte aligned
        layout_fast = (k_idx_a % 16 == 0) && ((k_idx_b / 2) % 16 == 0);
    } else {
        a.pa = make_pack(0, kPackW4A8Chunk, m, lda, k, 0);
        a.pb = make_pack(0, kPackW4A8Chunk, n, ldb / 2, k / 2, 0);
        layout_fast = (lda % 16 == 0) && ((ldb / 2) % 16 == 0);
    }
    // (the fast kernel forms row offsets with 24-bit multiplies)
    const bool fast = (k % kPairK == 0) && k <= 65536 && layout_fast && aligned16(A) &&
                      aligned16(B) && (m + kRowsPerChunk - 1) / kRowsPerChunk < 65536 &&
                      lda < (1u << 24) && ldb / 2 < (1u << 24) && ldc < (1u << 24) &&
                      ldd < (1u << 24);
    if (fast && !packed && launch_w4a8_strip<OUT>(a, s)) {
        // decode strip kernel (m = 1, k = 2048 or 4096)
    } else if (fast) {
        const unsigned gx = static_cast<unsigned>((n + kNTile - 1) / kNTile);
        const unsigned long long gy = (m + kRowsPerChunk - 1) / kRowsPerChunk;
        const size_t rows_max = m < static_cast<size_t>(kRowsPerChunk) ? m : kRowsPerChunk;
        const size_t npairs = k / kPairK;
        const size_t ppw = (npairs + kWaves - 1) / kWaves;
        const dim3 grid(gx, static_cast<unsigned>(gy));
        // activation staging: each wave's slice is rows_max x ppw * 256 bytes, 16 bytes per
        // lane per load; up to kMaxActLoads loads per lane, else loaded per step
        const size_t act_loads = (rows_max * ppw * 16 + 63) / 64;
        const size_t lds = static_cast<size_t>(kWaves) *
                           act_slice_bytes(static_cast<int>(rows_max), static_cast<int>(ppw));
        const dim3 block(kWaves * 64);
        if (act_loads <= 1) {
            launch_w4a8<1, OUT>(grid, block, lds, s, a, packed);
        } else if (act_loads <= 2) {
            launch_w4a8<2, OUT>(grid, block, lds, s, a, packed);
        } else if (act_loads <= 4) {
            launch_w4a8<4, OUT>(grid, block, lds, s, a, packed);
        } else if (act_loads <= static_cast<size_t>(kMaxActLoads)) {
            launch_w4a8<kMaxActLoads, OUT>(grid, block, lds, s, a, packed);
        } else {
            launch_w4a8<0, OUT>(grid, block, 0, s, a, packed);
        }
    } else {
        const long long total = static_cast<long long>(m) * static_cast<long long>(n);
        const long long blocks = (total + 255) / 256;
        TQT_REQUIRE(blocks < (1ll << 31), "grid too large");
        if (packed) {
            hipLaunchKernelGGL((w4a8_generic_kernel<PK_AB, OUT>), dim3(static_cast<unsigned>(blocks)),
                               dim3(256), 0, s, a);
        } else {
            hipLaunchKernelGGL((w4a8_generic_kernel<PK_NONE, OUT>),
                               dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, a);
        }
    }
    check_launch(where);
}

}  // namespace
}  // namespace tqt

using namespace tqt;

extern "C" {

// Steps set only a caller's tile stride and the getters' alignment check (the run accepts any m
// and n), so they are launch-sized: 16 rows (a decode batch) by 16384 channels, one launch for
// the decode GEMV where 16-channel tiles took 688 synchronous calls (9.7 ms against 5.3 us).
static const size_t kW4A8MStep = 16;
static const size_t kW4A8NStep = 16384;

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
    w4a8_run<OUT_F32>(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias, clamp_min,
                      clamp_max, params, false, as_stream(stream),
             "tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    float clamp_min, float clamp_max, const struct tqt_qai8dx_qsi4cx_params *params)
{
    if (!params) {
        return;
    }
    if (m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950_async(
        m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias, clamp_min, clamp_max,
        params, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950");
}

// gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp (reference …qai8dxp_qsi4cxp_4x1vl_rvv.cpp:113-190; its
// geometry getters and packers are in packing.hip). The reference run reads tile bases as
// m_idx * k and n_idx * k / 2 and ignores k_idx; this run reads panels with lda / ldb and the
// k_idx tail rule, as the packers write them (the same bytes for the packers' lda = k, k_idx = 0).
void tqt_run_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, float clamp_min, float clamp_max,
    const struct tqt_qai8dx_qsi4cx_params *params, void *stream)
{
    w4a8_run<OUT_F32>(m, n, k, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, C, ldc, D, ldd,
                      bias, clamp_min, clamp_max, params, true, as_stream(stream),
             "tqt_run_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, float clamp_min, float clamp_max,
    const struct tqt_qai8dx_qsi4cx_params *params)
{
    if (!params || m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950_async(
        m, n, k, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, C, ldc, D, ldd, bias, clamp_min,
        clamp_max, params, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950");
}

// The fused decode step (include/tqt_quantize_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_gfx950.h):
// tqt_run_quantize_qai8dx_f32 of A into A_q, scale_a, zero_point_a, then the W4A8 GEMV on them,
// in one launch when m = 1 and k = 2048 or 4096 (16-byte aligned A and B, 4-byte aligned A_q,
// ldb / 2 a multiple of 16), else as those two launches; the results are the same either way.
void tqt_run_quantize_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_gfx950_async(
    size_t m, size_t n, size_t k, const float *A, size_t lda, int8_t *A_q, size_t lda_q,
    float *scale_a, int32_t *zero_point_a, const void *B, size_t ldb, const void *C, size_t ldc,
    void *D, size_t ldd, const void *bias, float clamp_min, float clamp_max,
    const float *scale_b, void *stream)
{
    static const char *where = "tqt_run_quantize_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_gfx950";
    if (m == 0) {
        return;
    }
    TQT_REQUIRE(k % 2 == 0, "k % 2 == 0");
    TQT_REQUIRE(m < (1u << 31) && n < (1u << 31) && k < (1u << 31), "dimension exceeds 2^31-1");
    TQT_REQUIRE(scale_a != nullptr && zero_point_a != nullptr && (scale_b != nullptr || n == 0),
                "scale_a / zero_point_a / scale_b == NULL");
    TQT_REQUIRE((A != nullptr && A_q != nullptr && (B != nullptr || n == 0)) || k == 0,
                "A / A_q / B == NULL");
    TQT_REQUIRE(D != nullptr || n == 0, "D == NULL");
    TQT_REQUIRE(lda >= k && lda_q >= k, "lda or lda_q < k");
    const hipStream_t s = as_stream(stream);
    if (n > 0 && m == 1 && aligned16(A) && aligned16(B) && (reinterpret_cast<uintptr_t>(A_q) & 3) == 0 &&
        (ldb / 2) % 16 == 0) {
        W4A8Args a = {};
        a.M = 1;
        a.N = static_cast<int>(n);
        a.K = static_cast<int>(k);
        a.A = A_q;
        a.lda = static_cast<long long>(lda_q);
        a.B = static_cast<const uint8_t *>(B);
        a.bstride = static_cast<long long>(ldb / 2);
        a.C = C;
        a.ldc = static_cast<long long>(ldc);
        a.D = D;
        a.ldd = static_cast<long long>(ldd);
        a.bias = bias;
        a.cmin = clamp_min;
        a.cmax = clamp_max;
        a.scale_a = scale_a;
        a.zp_a = zero_point_a;
        a.scale_b = scale_b;
        if (launch_w4a8_qstrip<OUT_F32>(a, A, A_q, scale_a, zero_point_a, s)) {
            check_launch(where);
            return;
        }
    }
    tqt_run_quantize_qai8dx_f32_gfx950_async(m, k, A, lda, A_q, lda_q, scale_a, zero_point_a,
                                             stream);
    if (n > 0) {
        const struct tqt_qai8dx_qsi4cx_params p = {scale_a, zero_point_a, scale_b};
        tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_mfma_gfx950_async(
            m, n, k, A_q, lda_q, 0, B, ldb, 0, C, ldc, D, ldd, bias, clamp_min, clamp_max, &p,
            stream);
    }
}

void tqt_run_quantize_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_gfx950(
    size_t m, size_t n, size_t k, const float *A, size_t lda, int8_t *A_q, size_t lda_q,
    float *scale_a, int32_t *zero_point_a, const void *B, size_t ldb, const void *C, size_t ldc,
    void *D, size_t ldd, const void *bias, float clamp_min, float clamp_max,
    const float *scale_b)
{
    if (m == 0) {
        return;
    }
    tqt_run_quantize_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_gfx950_async(
        m, n, k, A, lda, A_q, lda_q, scale_a, zero_point_a, B, ldb, C, ldc, D, ldd, bias,
        clamp_min, clamp_max, scale_b, nullptr);
    finish_sync(nullptr, "tqt_run_quantize_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_gfx950");
}

// =============================================================================================
// Output-type siblings: W4A8 with f16 or bf16 D, C and bias (reference
// …/gemm_1xnbias_clamp_{f16,bf16}_qai8dx_qsi4cxt/…_4x1vl_rvv.cpp and their packed siblings
// …_{f16,bf16}_qai8dxp_qsi4cxp; epilogue tqt_kernel_gemm_i8_i4_4x1vl_rvv.h:428-628: the f32
// epilogue with C and bias widened from the output type, the clamp bounds widened to f32, one
// round-to-nearest-even narrowing at the store). Packers and packed getters are in packing.hip.
// =============================================================================================

#define TQT_W4A8_OUT_GETTERS(T, ES)                                                               \
    size_t tqt_get_m_step_##T##_mfma_gfx950(void) { return kW4A8MStep; }                         \
    size_t tqt_get_n_step_##T##_mfma_gfx950(void) { return kW4A8NStep; }                         \
    size_t tqt_get_a_offset_##T##_mfma_gfx950(size_t m_idx, size_t k_idx, size_t lda)            \
    {                                                                                             \
        TQT_REQUIRE(m_idx % kW4A8MStep == 0, "m_idx % m_step == 0");                             \
        return m_idx * lda + k_idx;                                                               \
    }                                                                                             \
    size_t tqt_get_b_offset_##T##_mfma_gfx950(size_t n_idx, size_t k_idx, size_t ldb)            \
    {                                                                                             \
        TQT_REQUIRE(n_idx % kW4A8NStep == 0, "n_idx % n_step == 0");                             \
        TQT_REQUIRE(k_idx % 2 == 0, "k_idx % 2 == 0");                                           \
        return n_idx * (ldb / 2) + k_idx / 2;                                                     \
    }                                                                                             \
    size_t tqt_get_c_offset_##T##_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldc)            \
    {                                                                                             \
        TQT_REQUIRE(m_idx % kW4A8MStep == 0, "m_idx % m_step == 0");                             \
        TQT_REQUIRE(n_idx % kW4A8NStep == 0, "n_idx % n_step == 0");                             \
        return (m_idx * ldc + n_idx) * (ES);                                                      \
    }                                                                                             \
    size_t tqt_get_bias_offset_##T##_mfma_gfx950(size_t n_idx)                                   \
    {                                                                                             \
        TQT_REQUIRE(n_idx % kW4A8NStep == 0, "n_idx % n_step == 0");                             \
        return n_idx * (ES);                                                                      \
    }                                                                                             \
    size_t tqt_get_d_offset_##T##_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldd)            \
    {                                                                                             \
        TQT_REQUIRE(m_idx % kW4A8MStep == 0, "m_idx % m_step == 0");                             \
        TQT_REQUIRE(n_idx % kW4A8NStep == 0, "n_idx % n_step == 0");                             \
        return (m_idx * ldd + n_idx) * (ES);                                                      \
    }                                                                                             \
    size_t tqt_get_d_size_##T##_mfma_gfx950(size_t m, size_t n) { return m * n * (ES); }

// The run pair (synchronous and stream-ordered) of a W4A8 output sibling.
#define TQT_W4A8_OUT_RUNS(T, CT, OUT, PACKED)                                                     \
    void tqt_run_##T##_mfma_gfx950_async(                                                         \
        size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,   \
        size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd,               \
        const void *bias, CT clamp_min, CT clamp_max,                                             \
        const struct tqt_qai8dx_qsi4cx_params *params, void *stream)                              \
    {                                                                                             \
        w4a8_run<OUT>(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias,            \
                      static_cast<float>(clamp_min), static_cast<float>(clamp_max), params,       \
                      PACKED, as_stream(stream), "tqt_run_" #T "_mfma_gfx950");                   \
    }                                                                                             \
    void tqt_run_##T##_mfma_gfx950(size_t m, size_t n, size_t k, const void *A, size_t lda,       \
                                   size_t k_idx_a, const void *B, size_t ldb, size_t k_idx_b,     \
                                   const void *C, size_t ldc, void *D, size_t ldd,                \
                                   const void *bias, CT clamp_min, CT clamp_max,                  \
                                   const struct tqt_qai8dx_qsi4cx_params *params)                 \
    {                                                                                             \
        if (!params || m == 0 || n == 0) {                                                        \
            return;                                                                               \
        }                                                                                         \
        tqt_run_##T##_mfma_gfx950_async(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D,     \
                                        ldd, bias, clamp_min, clamp_max, params, nullptr);        \
        finish_sync(nullptr, "tqt_run_" #T "_mfma_gfx950");                                       \
    }

TQT_W4A8_OUT_GETTERS(gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt, sizeof(float16_t))
TQT_W4A8_OUT_RUNS(gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt, float16_t, OUT_F16, false)
TQT_W4A8_OUT_GETTERS(gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt, sizeof(bfloat16_t))
TQT_W4A8_OUT_RUNS(gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt, bfloat16_t, OUT_BF16, false)
TQT_W4A8_OUT_RUNS(gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp, float16_t, OUT_F16, true)
TQT_W4A8_OUT_RUNS(gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp, bfloat16_t, OUT_BF16, true)

}  // extern "C"
