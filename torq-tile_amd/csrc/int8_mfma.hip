// int8 x int8 -> int32 contraction on gfx950 int8 MFMA, shared by these kernel types:
//   gemm_clamp_i32_i8_i8                                (B is [k, n] row-major, int32 out)
//   gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt     (B is [n, k], requantized int8 out)
//   igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt  (A gathered from an NDHWC image)
//   gemm_1xnbias_clamp_{f32,f16}_qai8dx_qsi8cxt         (per-row dynamically quantized A,
//                                                        f32 / f16 out)
//   gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8      (weights x [k, n] activations, per-row
//                                                        bias and requantization)
//   igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8   (B gathered from an NCDHW image)
// and their packed siblings.
//
// Four kernels, chosen per call:
//   * conv_halo_kernel (igemmcl, plain or packed weights, 3 x 3 "same" convolution with stride 1
//     and 128 channels per group: the benchmark's): each workgroup loads the input rows its 256
//     output pixels touch into LDS once and forms the nine taps from them (described at the
//     kernel);
//   * int8_stream_kernel (plain A, B = [n, k], k % 128 == 0: W8A8 at its config; the other
//     igemmcl geometries whose group channel count is a multiple of 128): 8 wave64s, a 4-deep
//     ring of LDS stages filled by direct global->LDS loads, v_mfma_i32_32x32x32_i8, XCD-aware
//     tile order (described at the kernel);
//   * int8_mfma_kernel (igemmcl, the other 16-byte-aligned shapes, clamp_i32's [k, n] B): 256 threads
//     (4 wave64s in a 2x2 grid) on a BM x 128 tile, k in steps of 64 bytes through double-buffered
//     LDS tiles, v_mfma_i32_16x16x64_i8;
//   * int8_generic_kernel: one thread per output for unaligned pointers or strides, k not a
//     multiple of 16, or channel counts not a multiple of 16.
// All four accumulate exactly in int32 and fuse the epilogue (C, bias, requantization,
// saturation, clamp) into the store.
#include <type_traits>

#include "tqt_hip_common.hpp"
#include "tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950.h"
#include "tqt_gemm_clamp_i32_i8_i8_mfma_gfx950.h"
#include "tqt_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_clamp_i32_i8p_i8p_mfma_gfx950.h"
#include "tqt_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950.h"
#include "tqt_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950.h"
#include "tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950.h"
#include "tqt_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950.h"

namespace tqt {
namespace {

constexpr int kThreads = 256;
constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kPrefetch = 4;  // k-steps in flight in registers (int8_mfma_kernel)
constexpr int kConvMaxChunks = 1024;  // fast implicit convolution: k <= 16384

enum AMode { A_MATRIX = 0, A_CONV_CL = 1 };
// B_CF: B is the channel-first im2col [K, N] of an NCDHW input, gathered on the fly
// (k = (ic, kd, kh, kw), n = output pixel p0 + column)
enum BMode { B_NK = 0, B_KN = 1, B_CF = 2 };
// EPI_REQUANT_ROW: the requantization of EPI_REQUANT_I8 with its bias and multiplier per row
// (gemm_mx1bias: the scale array belongs to A, the scalar scale to B)
// s_waitcnt immediate waiting for vmcnt <= vm and lgkmcnt == 0.
__host__ __device__ constexpr int waitcnt_vm_lgkm0(int vm)
{
    // s_waitcnt immediate (gfx9): vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14
    return (vm & 15) | (7 << 4) | ((vm >> 4) << 14);
}

enum EpiMode {
    EPI_CLAMP_I32 = 0,
    EPI_REQUANT_I8 = 1,
    EPI_DYN_F32 = 2,
    EPI_DYN_F16 = 3,
    EPI_REQUANT_ROW = 4
};

__host__ __device__ constexpr bool is_dyn(int epi)
{
    return epi == EPI_DYN_F32 || epi == EPI_DYN_F16;
}

// Zero points for which q_a - zp fits 16 bits for every int8 q_a: there the reference's
// sum of int16(q_a - zp) * q_b equals sum q_a * q_b - zp * sum q_b (mod 2^32), which the MFMA
// kernels compute. Any other zero point takes an exact per-output loop.
constexpr int32_t kDynZpMin = -32640;
constexpr int32_t kDynZpMax = 32640;

struct ConvGeom
{
    int ID, IH, IW;
    int OH, OW;
    int KD, KH, KW;
    int SD, SH, SW;
    int DD, DH, DW;
    int PD, PH, PW;
    int IC;   // channel stride of the NDHWC input
    int ICg;  // channels per group (K = KD*KH*KW*ICg)
};

struct Int8Args
{
    int M, N, K;
    const int8_t *A;  // matrix A, or the group's channel base of the NDHWC input
    long long lda;
    const int8_t *B;  // matrix B, or (B_CF) the group's base of the NCDHW input
    long long ldb;
    const int32_t *C;
    long long ldc;
    void *D;
    long long ldd;
    long long d_row0;  // igemmcl: D row of local pixel 0 (= m_idx); 0 otherwise
    long long p0;      // igemmcl / igemmcf: global pixel index of local pixel 0
    int conv_bytes;    // igemmcl streaming path: input bytes from A to the end of the input
    const int32_t *bias;
    int32_t cmin, cmax;
    // requantization: multiplier of column j (row i for EPI_REQUANT_ROW) from
    // scale_a * scale_b[j or 0] / scale_d (quant_channel_b == 1: index 0)
    float scale_a;
    const float *scale_b;
    int32_t quant_channel_b;
    float scale_d;
    int32_t zp_d;
    ConvGeom cv;
    PackDesc pa, pb;  // packed A / B of the p-variants (read when the kernel's PK bit is set)
    // qai8dx x qsi8cx: per-row scale / zero point of A (scale_b above is per channel), an f32
    // or f16 bias, and the clamp bounds widened to f32
    const float *dyn_sa;
    const int32_t *dyn_za;
    const void *fbias;
    float fcmin, fcmax;
};

// The reference's accumulator of one output, sum_k int16(q_a - zp) * q_b in wrapping int32
// (tqt_kernel_gemm_qai8dx_qsi8cx_4x1vl_rvv.h:95-140: vwmacc.vx at SEW 16 takes the low 16 bits
// of the scalar q_a - zp), summed directly.
template <int PK>
__device__ uint32_t dyn_exact_acc(const Int8Args &a, int gm, int gn, int32_t zp)
{
    const PackRow ra = pack_row_info(a.pa, gm);
    const PackRow rb = pack_row_info(a.pb, gn);
    uint32_t acc = 0;
    for (int k = 0; k < a.K; ++k) {
        const int32_t av = (PK & PK_A) ? a.A[pack_row_byte(ra, k)]
                                       : a.A[static_cast<long long>(gm) * a.lda + k];
        const int32_t bv = (PK & PK_B) ? a.B[pack_row_byte(rb, k)]
                                       : a.B[static_cast<long long>(gn) * a.ldb + k];
        const uint32_t d = static_cast<uint32_t>(av) - static_cast<uint32_t>(zp);
        const int32_t a16 = static_cast<int16_t>(static_cast<uint16_t>(d & 0xffffu));
        acc += static_cast<uint32_t>(a16 * bv);
    }
    return acc;
}

// Epilogue of the qai8dx x qsi8cx types for one output from its accumulator x
// (tqt_kernel_gemm_qai8dx_qsi8cx_4x1vl_rvv.h): f32 D (dequant_fp32 :145-215): f32(x) * (sb * sa),
// + bias (+0 without one), vfmax, vfmin; f16 D (dequant_fp16 :217-330): the same f32 product
// rounded to f16, + the f16 bias in f16, then the bounds. Every step rounds once (the library is
// built without contraction).
template <int EPI>
__device__ __forceinline__ void dyn_finish_v(const Int8Args &a, int gn, long long drow, uint32_t x,
                                             float sb, float sa, float fb)
{
    const float sigma = __fmul_rn(sb, sa);
    const float f = __fmul_rn(static_cast<float>(static_cast<int32_t>(x)), sigma);
    if constexpr (EPI == EPI_DYN_F32) {
        float v = __fadd_rn(f, fb);
        v = rv_fmaxf(v, a.fcmin);
        v = rv_fminf(v, a.fcmax);
        static_cast<float *>(a.D)[drow * a.ldd + gn] = v;
    } else {
        // The product must be rounded to f32 before the f16 conversion (vfmul then vfncvt):
        // without this register barrier the compiler folds both into one v_fma_mixlo_f16, which
        // rounds the exact product to f16 once.
        float fr = f;
        asm volatile("" : "+v"(fr));
        const _Float16 h = static_cast<_Float16>(fr);
        const _Float16 b = static_cast<_Float16>(fb);  // exact: fb holds a binary16 value
        const _Float16 hs = h + b;  // one binary16 rounding
        float v = rv_fmaxf(static_cast<float>(hs), a.fcmin);  // exact on binary16 values
        v = rv_fminf(v, a.fcmax);
        store_out<OUT_F16>(a.D, drow * a.ldd + gn, v);
    }
}

__device__ __forceinline__ bool dyn_zp_in_range(int32_t zp)
{
    return zp >= kDynZpMin && zp <= kDynZpMax;
}

// The column's bias as f32 (an f16 bias converts exactly); +0 without a bias.
template <int EPI>
__device__ __forceinline__ float dyn_bias(const Int8Args &a, int gn)
{
    if (!a.fbias) {
        return 0.0f;
    }
    if constexpr (EPI == EPI_DYN_F32) {
        return static_cast<const float *>(a.fbias)[gn];
    } else {
        return static_cast<float>(static_cast<const _Float16 *>(a.fbias)[gn]);
    }
}

// One output from memory-held inputs (the exact per-output path).
template <int EPI>
__device__ __forceinline__ void dyn_finish(const Int8Args &a, int gm, int gn, long long drow,
                                           uint32_t x)
{
    dyn_finish_v<EPI>(a, gn, drow, x, a.scale_b[gn], a.dyn_sa[gm], dyn_bias<EPI>(a, gn));
}

// The MFMA kernels' epilogues load every per-row (zero point, scale) and per-column (scale, bias)
// input of a lane's outputs before its first store and wait for them once: stores count in
// vmcnt, so a load between two stores would make the compiler's wait for it drain the earlier
// store as well, serializing the lane's stores.

// LDS tile of R rows x 64 bytes. The 16-byte column chunk of row r is XOR-swizzled with
// (r >> 2) & 3 so that the 16 rows read by one 16-lane group of ds_read_b128 hit distinct
// banks.
__device__ __forceinline__ int lds_off(int row, int chunk)
{
    return row * kBK + ((chunk ^ ((row >> 2) & 3)) << 4);
}

// Byte (k, pixel (od, oh, ow)) of the channel-first im2col of the input at a.B (0 for a padding
// tap). Every load reads valid memory: a padding tap reads the plane's first byte.
__device__ __forceinline__ uint32_t cf_byte(const Int8Args &a, const int8_t *plane, int kd,
                                            int kh, int kw, int od, int oh, int ow, bool ok)
{
    const ConvGeom &g = a.cv;
    const int id = od * g.SD + kd * g.DD - g.PD;
    const int ih = oh * g.SH + kh * g.DH - g.PH;
    const int iw = ow * g.SW + kw * g.DW - g.PW;
    ok = ok && id >= 0 && id < g.ID && ih >= 0 && ih < g.IH && iw >= 0 && iw < g.IW;
    const long long off = ok ? (static_cast<long long>(id) * g.IH + ih) * g.IW + iw : 0;
    const uint32_t v = static_cast<uint8_t>(plane[off]);
    return ok ? v : 0u;
}

// Tap of channel-first im2col row k: the input channel's plane and (kd, kh, kw).
__device__ __forceinline__ const int8_t *cf_tap(const Int8Args &a, int k, int &kd, int &kh,
                                                int &kw)
{
    const ConvGeom &g = a.cv;
    const int khw = g.KH * g.KW;
    const int kdhw = g.KD * khw;
    const int ic = k / kdhw;
    int r = k - ic * kdhw;
    kd = r / khw;
    r -= kd * khw;
    kh = r / g.KW;
    kw = r - kh * g.KW;
    return a.B + static_cast<long long>(ic) * g.ID * g.IH * g.IW;
}

template <int BM, int AM, int BMd, int EPI, int PK>
__global__ __launch_bounds__(kThreads) void int8_mfma_kernel(Int8Args a)
{
    constexpr int WM = BM / 2;        // rows per wave
    constexpr int MT = WM / 16;       // 16-row sub-tiles per wave
    constexpr int NT = 4;             // 16-col sub-tiles per wave (64 columns)
    constexpr int A_CHUNKS = BM * 4 / kThreads;  // 16-byte chunks per thread per A tile
    constexpr int B_CHUNKS = kBN * 4 / kThreads;

    __shared__ __attribute__((aligned(16))) int8_t lds_a[2][BM * kBK];
    __shared__ __attribute__((aligned(16))) int8_t lds_b[2][kBN * kBK];
    __shared__ int32_t s_mult[kBN];
    __shared__ int32_t s_shift[kBN];
    // implicit convolution: per 16-byte k-chunk, the tap's input offset from the output pixel's
    // base and its (kd * DD, kh * DH, kw * DW) packed 10 bits each
    __shared__ int2 s_tap[AM == A_CONV_CL ? kConvMaxChunks : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1;
    const int wn = wave & 1;

    if constexpr (AM == A_CONV_CL) {
        const ConvGeom &g = a.cv;
        for (int c = tid; c < a.K / 16; c += kThreads) {
            const int k = 16 * c;
            const int tap = k / g.ICg;
            const int ic = k - tap * g.ICg;
            const int kw = tap % g.KW;
            const int t2 = tap / g.KW;
            const int kh = t2 % g.KH;
            const int kd = t2 / g.KH;
            const int dd = kd * g.DD, dh = kh * g.DH, dw = kw * g.DW;
            const int off = ((dd * g.IH + dh) * g.IW + dw) * g.IC + ic;
            s_tap[c] = int2{off, dd | (dh << 10) | (dw << 20)};
        }
        __syncthreads();
    }

    const int tiles_n = (a.N + kBN - 1) / kBN;
    const int tile_m = blockIdx.x / tiles_n;
    const int tile_n = blockIdx.x - tile_m * tiles_n;
    const int m0 = tile_m * BM;
    const int n0 = tile_n * kBN;

    if constexpr (EPI == EPI_REQUANT_I8) {
        if (tid < kBN && n0 + tid < a.N) {
            column_multiplier_dev(a.scale_a, a.scale_b, a.quant_channel_b, a.scale_d, n0 + tid,
                                  s_mult[tid], s_shift[tid]);
        }
    } else if constexpr (EPI == EPI_REQUANT_ROW) {
        if (tid < BM && m0 + tid < a.M) {
            column_multiplier_dev(a.scale_a, a.scale_b, a.quant_channel_b, a.scale_d, m0 + tid,
                                  s_mult[tid], s_shift[tid]);
        }
    }

    // Per-thread load assignment (fixed across the K loop): 4 consecutive threads read one row's
    // 64 bytes of a plain operand; for a packed one (16-byte chunks stored chunk-major in the
    // panel) consecutive threads take consecutive rows of one chunk, so a wave reads 64 rows x
    // 16 contiguous bytes.
    int a_row[A_CHUNKS], a_chk[A_CHUNKS], a_mul[A_CHUNKS];
    bool a_ok[A_CHUNKS];
    int a_od[A_CHUNKS], a_oh[A_CHUNKS], a_ow[A_CHUNKS];
    const int8_t *a_ptr[A_CHUNKS];
#pragma unroll
    for (int j = 0; j < A_CHUNKS; ++j) {
        const int c = tid + j * kThreads;
        a_row[j] = (PK & PK_A) ? c % BM : c >> 2;
        a_chk[j] = (PK & PK_A) ? c / BM : c & 3;
        const int gm = m0 + a_row[j];
        a_ok[j] = gm < a.M;
        a_mul[j] = 1;  // k multiplier of a packed row (its panel width)
        if constexpr (AM == A_MATRIX) {
            const int r = a_ok[j] ? gm : 0;
            long long base;
            if constexpr ((PK & PK_A) != 0) {
                base = pack_row_fixed<kPackI8MStep>(a.pa, r, a_mul[j]);
            } else {
                base = static_cast<long long>(r) * a.lda;
            }
            a_ptr[j] = a.A + base + pack_k<kPackI8Chunk, (PK & PK_A) != 0>(a_chk[j] * 16, a_mul[j]);
            a_od[j] = a_oh[j] = a_ow[j] = 0;
        } else {
            // a_od/a_oh/a_ow hold the first input coordinate of the output pixel's window
            const ConvGeom &g = a.cv;
            const long long p = a.p0 + (a_ok[j] ? gm : 0);
            const long long ohw = static_cast<long long>(g.OH) * g.OW;
            a_od[j] = static_cast<int>(p / ohw) * g.SD - g.PD;
            a_oh[j] = static_cast<int>((p / g.OW) % g.OH) * g.SH - g.PH;
            a_ow[j] = static_cast<int>(p % g.OW) * g.SW - g.PW;
            a_ptr[j] = a.A + ((static_cast<long long>(a_od[j]) * g.IH + a_oh[j]) * g.IW + a_ow[j]) *
                                 g.IC;
        }
    }
    int b_row[B_CHUNKS], b_chk[B_CHUNKS], b_mul[B_CHUNKS];
    bool b_ok[B_CHUNKS];
    const int8_t *b_ptr[B_CHUNKS];
    [[maybe_unused]] int b_od[B_CHUNKS], b_oh[B_CHUNKS], b_ow[B_CHUNKS];
#pragma unroll
    for (int j = 0; j < B_CHUNKS; ++j) {
        const int c = tid + j * kThreads;
        if constexpr (BMd == B_NK) {
            b_row[j] = (PK & PK_B) ? c % kBN : c >> 2;  // n within the tile
            b_chk[j] = (PK & PK_B) ? c / kBN : c & 3;   // 16-byte k chunk
            const int gn = n0 + b_row[j];
            b_ok[j] = gn < a.N;
            const int r = b_ok[j] ? gn : 0;
            long long base;
            b_mul[j] = 1;
            if constexpr ((PK & PK_B) != 0) {
                base = pack_row_fixed<kPackI8NStep>(a.pb, r, b_mul[j]);
            } else {
                base = static_cast<long long>(r) * a.ldb;
            }
            b_ptr[j] = a.B + base + pack_k<kPackI8Chunk, (PK & PK_B) != 0>(b_chk[j] * 16, b_mul[j]);
        } else {
            // one wave covers 64 consecutive k of one 16-column chunk, so each byte store of
            // the transpose below writes 64 consecutive bytes of one LDS row (no bank conflicts
            // beyond the four lanes that share a dword)
            b_row[j] = c & 63;  // k within the tile
            b_chk[j] = c >> 6;  // 16-column chunk
            const int gn = n0 + b_chk[j] * 16;
            b_ok[j] = gn < a.N;
            b_mul[j] = 1;
            b_ptr[j] = a.B + (b_ok[j] ? gn : 0);
            if constexpr (BMd == B_CF) {
                // output pixel of the chunk's first column
                const long long p = a.p0 + (b_ok[j] ? gn : 0);
                const long long ohw = static_cast<long long>(a.cv.OH) * a.cv.OW;
                b_od[j] = static_cast<int>(p / ohw);
                b_oh[j] = static_cast<int>((p / a.cv.OW) % a.cv.OH);
                b_ow[j] = static_cast<int>(p % a.cv.OW);
            }
        }
    }

    // One k-step of operands in registers: raw 16-byte loads plus a validity bit per chunk.
    // Every load reads valid memory (an out-of-range chunk reads the operand's first 16 bytes
    // instead) and the mask is applied when the step is stored to LDS, so no load sits in
    // a branch (the compiler would wait for it at the join, serializing the stream).
    struct Step
    {
        i32x4 a[A_CHUNKS];
        i32x4 b[B_CHUNKS];
        uint32_t am, bm;
    };
    auto load_tile = [&](int k0, Step &st) {
        st.am = 0;
        st.bm = 0;
#pragma unroll
        for (int j = 0; j < A_CHUNKS; ++j) {
            const int k = k0 + a_chk[j] * 16;
            bool ok = a_ok[j] && k < a.K;
            const int8_t *src;
            if constexpr (AM == A_MATRIX) {
                src = ok ? a_ptr[j] + pack_k<kPackI8Chunk, (PK & PK_A) != 0>(k0, a_mul[j]) : a.A;
            } else {
                const ConvGeom &g = a.cv;
                const int2 t = s_tap[ok ? k >> 4 : 0];
                const int id = a_od[j] + (t.y & 1023);
                const int ih = a_oh[j] + ((t.y >> 10) & 1023);
                const int iw = a_ow[j] + ((t.y >> 20) & 1023);
                ok = ok && id >= 0 && id < g.ID && ih >= 0 && ih < g.IH && iw >= 0 && iw < g.IW;
                src = ok ? a_ptr[j] + t.x : a.A;
            }
            st.a[j] = *reinterpret_cast<const i32x4 *>(src);
            st.am |= ok ? (1u << j) : 0u;
        }
#pragma unroll
        for (int j = 0; j < B_CHUNKS; ++j) {
            if constexpr (BMd == B_NK) {
                const int k = k0 + b_chk[j] * 16;
                const bool ok = b_ok[j] && k < a.K;
                st.b[j] = *reinterpret_cast<const i32x4 *>(
                    ok ? b_ptr[j] + pack_k<kPackI8Chunk, (PK & PK_B) != 0>(k0, b_mul[j]) : a.B);
                st.bm |= ok ? (1u << j) : 0u;
            } else if constexpr (BMd == B_KN) {
                const int k = k0 + b_row[j];
                const int gn = n0 + b_chk[j] * 16;
                const bool ok = b_ok[j] && k < a.K;
                const int8_t *src = b_ptr[j] + static_cast<long long>(ok ? k : 0) * a.ldb;
                if (gn + 16 <= a.N) {  // uniform per wave (one column chunk per wave)
                    st.b[j] = *reinterpret_cast<const i32x4 *>(src);
                } else {
                    i32x4 tmp = i32x4{0, 0, 0, 0};
                    int8_t *tb = reinterpret_cast<int8_t *>(&tmp);
                    for (int i = 0; i < 16 && gn + i < a.N; ++i) {
                        tb[i] = src[i];
                    }
                    st.b[j] = tmp;
                }
                st.bm |= ok ? (1u << j) : 0u;
            } else {
                // 16 consecutive output pixels of one channel-first im2col row, gathered
                const int k = k0 + b_row[j];
                const int gn = n0 + b_chk[j] * 16;
                const bool ok = b_ok[j] && k < a.K;
                int kd, kh, kw;
                const int8_t *plane = cf_tap(a, ok ? k : 0, kd, kh, kw);
                int od = b_od[j], oh = b_oh[j], ow = b_ow[j];
                uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    w[i >> 2] |= cf_byte(a, plane, kd, kh, kw, od, oh, ow, ok && gn + i < a.N)
                                 << (8 * (i & 3));
                    if (++ow == a.cv.OW) {
                        ow = 0;
                        if (++oh == a.cv.OH) {
                            oh = 0;
                            ++od;
                        }
                    }
                }
                st.b[j] = i32x4{static_cast<int>(w[0]), static_cast<int>(w[1]),
                                static_cast<int>(w[2]), static_cast<int>(w[3])};
                st.bm |= ok ? (1u << j) : 0u;
            }
        }
    };

    auto store_tile = [&](int buf, const Step &st) {
        const i32x4 z = i32x4{0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < A_CHUNKS; ++j) {
            *reinterpret_cast<i32x4 *>(&lds_a[buf][lds_off(a_row[j], a_chk[j])]) =
                (st.am >> j) & 1u ? st.a[j] : z;
        }
#pragma unroll
        for (int j = 0; j < B_CHUNKS; ++j) {
            const i32x4 v = (st.bm >> j) & 1u ? st.b[j] : z;
            if constexpr (BMd == B_NK) {
                *reinterpret_cast<i32x4 *>(&lds_b[buf][lds_off(b_row[j], b_chk[j])]) = v;
            } else {
                // Transpose 16 consecutive n of one k into the [n][k] tile. Lane k of the wave
                // holds column bytes n = 16 chunk + 4p + b of row k in dword p; a 4x4 byte
                // transpose inside each quad of lanes (k = 4q .. 4q + 3: the quad's dwords p by
                // broadcast DPP, then two byte permutes) leaves lane 4q + i with the four k-bytes
                // of column 16 chunk + 4p + i, stored as one dword. For each p the wave's 64
                // stores cover 256 bytes of distinct banks (16 byte stores per lane with four
                // lanes per dword took 11 us per 64x256x512 launch).
                const int kq = b_row[j] & ~3;
                const uint32_t qi = static_cast<uint32_t>(b_row[j] & 3);
                const uint32_t sel01 = qi | ((4u + qi) << 8) | 0x0c0c0000u;
                const uint32_t sel23 = 0x00000c0cu | (qi << 16) | ((4u + qi) << 24);
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const int x0 = __builtin_amdgcn_mov_dpp(v[p], 0x00, 0xf, 0xf, false);
                    const int x1 = __builtin_amdgcn_mov_dpp(v[p], 0x55, 0xf, 0xf, false);
                    const int x2 = __builtin_amdgcn_mov_dpp(v[p], 0xaa, 0xf, 0xf, false);
                    const int x3 = __builtin_amdgcn_mov_dpp(v[p], 0xff, 0xf, 0xf, false);
                    const uint32_t o =
                        __builtin_amdgcn_perm(static_cast<uint32_t>(x1), static_cast<uint32_t>(x0),
                                              sel01) |
                        __builtin_amdgcn_perm(static_cast<uint32_t>(x3), static_cast<uint32_t>(x2),
                                              sel23);
                    const int n = b_chk[j] * 16 + 4 * p + static_cast<int>(qi);
                    *reinterpret_cast<uint32_t *>(&lds_b[buf][lds_off(n, kq >> 4) + (kq & 15)]) = o;
                }
            }
        }
    };

    i32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            acc[i][j] = i32x4{0, 0, 0, 0};
        }
    }
    // qai8dx x qsi8cx: this lane's share of sum_k q_b for its column (16 of every 64 k)
    [[maybe_unused]] int32_t rs[NT] = {};

    const int nk = (a.K + kBK - 1) / kBK;
    const int frag_row = lane & 15;
    const int frag_chk = lane >> 4;

    auto compute_step = [&](int buf) {
        i32x4 fa[MT], fb[NT];
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            const int r = wm * WM + i * 16 + frag_row;
            fa[i] = *reinterpret_cast<const i32x4 *>(&lds_a[buf][lds_off(r, frag_chk)]);
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int r = wn * 64 + j * 16 + frag_row;
            fb[j] = *reinterpret_cast<const i32x4 *>(&lds_b[buf][lds_off(r, frag_chk)]);
        }
#pragma unroll
        for (int i = 0; i < MT; ++i) {
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
            }
        }
        if constexpr (is_dyn(EPI)) {
#pragma unroll
            for (int j = 0; j < NT; ++j) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    rs[j] = __builtin_amdgcn_sdot4(fb[j][q], 0x01010101, rs[j], false);
                }
            }
        }
    };

    // k-steps stream through registers PF steps ahead of the LDS pair (register set s holds
    // step j with j % PF == s; the sets rotate by unrolling, since a register copy would wait
    // for the load still filling it). Loads past the last step reload it, so every load is
    // unconditional and the compiler tracks each set's loads exactly.
    // [k, n] and channel-first B: two steps ahead (four measured slower: 9.4-9.7 vs 9.1 us per
    // 64x256x512 clamp launch)
    constexpr int PF = BMd != B_NK ? 2 : kPrefetch;
    Step ps[PF];
    auto step_k0 = [&](int st) { return min(st, nk - 1) * kBK; };
    if (nk > 0) {
#pragma unroll
        for (int st = 0; st < PF; ++st) {
            load_tile(step_k0(st), ps[st]);
        }
        store_tile(0, ps[0]);
        load_tile(step_k0(PF), ps[0]);
    }
    __syncthreads();

    // Step kt: compute from LDS buffer kt & 1, store step kt + 1 (set (kt + 1) % PF) into the
    // other buffer, refill that set with step kt + 1 + PF. A store past the last step writes a
    // buffer nobody reads. Whole groups of PF steps run without branches (a join inside the
    // group makes the compiler wait for every load in flight); the last nk % PF steps follow.
    auto step = [&](int kt, Step &set) {
        compute_step(kt & 1);
        store_tile((kt + 1) & 1, set);
        load_tile(step_k0(kt + 1 + PF), set);
        __syncthreads();
    };
    int kt0 = 0;
    for (; kt0 + PF <= nk; kt0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            step(kt0 + u, ps[(u + 1) % PF]);
        }
    }
#pragma unroll
    for (int u = 0; u < PF - 1; ++u) {
        if (kt0 + u < nk) {
            step(kt0 + u, ps[(u + 1) % PF]);
        }
    }

    if constexpr (is_dyn(EPI)) {
        // the four lanes of a column (lane % 16) each summed one 16-byte chunk of every k-step
        int32_t rsum[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int32_t t = rs[j] + __shfl_xor(rs[j], 16);
            rsum[j] = t + __shfl_xor(t, 32);
        }
        int32_t zr[MT][4];
        float sar[MT][4];
        float sbc[NT], fbc[NT];
        bool in_range = true;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int gm = m0 + wm * WM + i * 16 + 4 * (lane >> 4) + r;
                zr[i][r] = gm < a.M ? a.dyn_za[gm] : 0;
                sar[i][r] = gm < a.M ? a.dyn_sa[gm] : 0.0f;
                in_range = in_range && dyn_zp_in_range(zr[i][r]);
            }
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int gn = n0 + wn * 64 + j * 16 + (lane & 15);
            sbc[j] = gn < a.N ? a.scale_b[gn] : 0.0f;
            fbc[j] = gn < a.N ? dyn_bias<EPI>(a, gn) : 0.0f;
        }
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));  // the compiler then adds no waits below
        if (in_range) {
#pragma unroll
            for (int i = 0; i < MT; ++i) {
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    const int gn = n0 + wn * 64 + j * 16 + (lane & 15);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int gm = m0 + wm * WM + i * 16 + 4 * (lane >> 4) + r;
                        if (gm < a.M && gn < a.N) {
                            const uint32_t x = static_cast<uint32_t>(acc[i][j][r]) -
                                               static_cast<uint32_t>(zr[i][r]) *
                                                   static_cast<uint32_t>(rsum[j]);
                            dyn_finish_v<EPI>(a, gn, a.d_row0 + gm, x, sbc[j], sar[i][r], fbc[j]);
                        }
                    }
                }
            }
        } else {
            // a zero point beyond 16 bits: this lane's outputs summed term by term
            for (int e = 0; e < MT * NT * 4; ++e) {
                const int i = e / (NT * 4), j = (e / 4) % NT, r = e % 4;
                const int gn = n0 + wn * 64 + j * 16 + (lane & 15);
                const int gm = m0 + wm * WM + i * 16 + 4 * (lane >> 4) + r;
                if (gm < a.M && gn < a.N) {
                    dyn_finish<EPI>(a, gm, gn, a.d_row0 + gm,
                                    dyn_exact_acc<PK>(a, gm, gn, a.dyn_za[gm]));
                }
            }
        }
        return;
    }

    // Epilogue: lane holds D[4 * (lane / 16) + r][lane % 16] of every 16x16 sub-tile. C and the
    // bias of every output of the lane are loaded first and waited for once (stores count in
    // vmcnt: a load between stores would make its wait drain them).
    constexpr bool kRow = EPI == EPI_REQUANT_ROW;
    uint32_t add[MT][NT][4];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int gn = n0 + wn * 64 + j * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int gm = m0 + wm * WM + i * 16 + 4 * (lane >> 4) + r;
                uint32_t v = 0;
                if (gm < a.M && gn < a.N) {
                    if (a.C) {
                        v += static_cast<uint32_t>(a.C[static_cast<long long>(gm) * a.ldc + gn]);
                    }
                    if (a.bias) {
                        v += static_cast<uint32_t>(a.bias[kRow ? gm : gn]);
                    }
                }
                add[i][j][r] = v;
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));  // the compiler then adds no waits below
    // A lane's output rows are row_l plus compile-time offsets: one per-lane base plus multiples
    // of the uniform ldd; whole row tiles skip the per-output row check.
    const int row_l = m0 + wm * WM + 4 * (lane >> 4);
    const long long d_l = (a.d_row0 + row_l) * a.ldd;
    auto epilogue = [&](auto checked) {
        constexpr bool kChecked = decltype(checked)::value;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const int lc = wn * 64 + j * 16 + (lane & 15);
                const int gn = n0 + lc;
                if (gn >= a.N) {
                    continue;
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int dr = i * 16 + r;
                    const int gm = row_l + dr;
                    if (kChecked && gm >= a.M) {
                        continue;
                    }
                    const uint32_t v = static_cast<uint32_t>(acc[i][j][r]) + add[i][j][r];
                    const long long e = d_l + dr * a.ldd + gn;
                    if constexpr (EPI == EPI_CLAMP_I32) {
                        int32_t x = static_cast<int32_t>(v);
                        x = x < a.cmin ? a.cmin : x;
                        x = x > a.cmax ? a.cmax : x;
                        static_cast<int32_t *>(a.D)[e] = x;
                    } else {
                        const int q = kRow ? gm - m0 : lc;
                        static_cast<int8_t *>(a.D)[e] = requant_dev(
                            static_cast<int32_t>(v), s_mult[q], s_shift[q], a.zp_d, a.cmin, a.cmax);
                    }
                }
            }
        }
    };
    if (m0 + BM <= a.M) {
        epilogue(std::false_type{});
    } else {
        epilogue(std::true_type{});
    }
}

// ---------------------------------------------------------------------------------------------
// Streaming kernel for plain A and B = [n, k] (W8A8 and its packed siblings), k % 128 == 0, and
// for the implicit convolution (igemmcl) when the group channel count is a multiple of 128: a
// stage is then 128 channels of one tap, each A row the 128 contiguous input bytes of its output
// pixel's tap, read through a buffer resource whose range check returns zeros for padding taps.
//
// A workgroup of 8 wave64s (2 x 4, each BM/2 x 32) owns a BM x 128 output tile (BM = 64 or
// 128) and walks k in stages of 128 bytes through a 4-deep ring of LDS stages filled by direct
// global->LDS loads, every wave issuing an equal share of each stage's loads
// (global_load_lds_dwordx4: lane i of an instruction writes 16 bytes at LDS base + 16 * i, so
// no VGPRs carry the tiles). Each LDS row holds 128 k-bytes of one A row or one B row; its eight
// 16-byte chunks are stored XOR-swizzled with (row >> 1) & 7, which makes both the loads (8 rows
// x 128 B per instruction, whole cache lines) and the MFMA operand reads (ds_read_b128 of 32
// rows) conflict-free. Waves wait for their own loads with an explicit vmcnt and meet at a plain
// s_barrier: __syncthreads() would also drain every load still in flight for later stages.
// v_mfma_i32_32x32x32_i8 accumulates exactly in int32; the epilogue is fused into the store.
// Workgroups are ordered for the 8 XCDs: block b runs on XCD b % 8, and each XCD receives a
// contiguous range of tiles (M fastest), so its workgroups share their B rows (and A) in the
// XCD's L2.
// ---------------------------------------------------------------------------------------------
constexpr int kSK = 128;  // k bytes per pipeline stage

// dma_lds16 / dma_lds16_buf (tqt_hip_common.hpp) fill the ring with direct global -> LDS loads.

// Streaming kernel layout: kStreamWaves waves per workgroup each issue an equal share of every
// stage's 1 KiB load blocks and compute a BM/2 x 32 sub-tile (2 x 4 waves). Measured on MI355X
// (lab kernels, all 256 CUs busy): a CU sustains about 41 B/clk of L2 -> LDS traffic with eight
// waves issuing a few LDS-DMA loads each, against 24 B/clk with four waves issuing many, and
// ds_read_b128 reaches about 180 B/clk with eight waves reading against 105 B/clk with four; with
// two compute waves per SIMD one wave's LDS reads overlap the other's MFMAs.
constexpr int kStreamWaves = 8;
constexpr int kStreamWavesN = 4;  // waves along N (each 32 columns of the 128)
constexpr int kStreamThreads = kStreamWaves * 64;

// LDS ring depth of the streaming kernel (stages of 128 bytes of k for BM + 128 rows). Four
// stages: a 5- or 6-stage ring (which 64-row tiles would fit) measured no faster at the W8A8
// configuration (cold operands 17.6-18.0 us with four, 18.2 with six), and three slower (17.6-17.7
// vs 16.8 us).
constexpr int kStreamStages = 4;

template <int BM, int EPI, int PK, bool kConv = false>
__global__ __launch_bounds__(kStreamThreads) void int8_stream_kernel(Int8Args a, int tiles_m,
                                                                     int tiles, int per_xcd)
{
    constexpr int WM = BM / (kStreamWaves / kStreamWavesN);  // rows per wave
    constexpr int WN = kBN / kStreamWavesN;                   // columns per wave
    constexpr int MF = WM / 32;            // 32-row fragments per wave
    constexpr int NF = WN / 32;            // 32-column fragments per wave
    constexpr int A_DMA = BM / (8 * kStreamWaves);   // 1 KB (8-row) loads per wave per stage
    constexpr int B_DMA = kBN / (8 * kStreamWaves);
    static_assert(A_DMA >= 1 && B_DMA >= 1, "every wave loads A and B blocks");
    constexpr int PER_STAGE = A_DMA + B_DMA;
    constexpr int SA = BM * kSK;
    constexpr int SB = kBN * kSK;

    // ring of NS stages (A rows then B rows each); NS - 1 stages are in flight while one is read
    constexpr int NS = kStreamStages;
    __shared__ __attribute__((aligned(16))) int8_t ring[NS][SA + SB];
    __shared__ int32_t s_mult[kBN];
    __shared__ int32_t s_shift[kBN];

    const int t = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (t >= tiles) {
        return;
    }
    const int tile_m = t % tiles_m;
    const int m0 = tile_m * BM;
    const int n0 = (t / tiles_m) * kBN;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / kStreamWavesN;
    const int wn = wave % kStreamWavesN;

    // Epilogue inputs are loaded now and used after the main loop, so their latency hides under
    // it: the per-row multipliers' scale_b (EPI_REQUANT_ROW: finished into s_mult / s_shift
    // after the loop: computing them here would hold back this wave's first loads by a memory
    // round trip; the per-column ones are below) and the biases.
    constexpr bool kRow = EPI == EPI_REQUANT_ROW;
    [[maybe_unused]] float pre_sb = 0.f;
    [[maybe_unused]] int32_t pre_rbias = 0;  // per-row bias (EPI_REQUANT_ROW)
    [[maybe_unused]] uint32_t pre_cbias[NF] = {};
    [[maybe_unused]] const bool mult_lane = kRow ? (tid < BM && m0 + tid < a.M)
                                                 : (tid < kBN && n0 + tid < a.N);
    // Per-column requantization (W8A8, the convolution mode): the tile's 128 weight scales come
    // into LDS by LDS-DMA from waves 0 and 1 ahead of their ring loads (the first stage's wait
    // covers them, and the compiler places no wait of its own), and those lanes turn them into
    // multipliers after stage 1's compute, while its MFMAs run.
    __shared__ __attribute__((aligned(16))) float s_sbv[EPI == EPI_REQUANT_I8 ? kBN : 1];
    if constexpr (EPI == EPI_REQUANT_I8) {
        if (tid < kBN) {  // whole waves: kBN is a multiple of 64
            const int idx = min(n0 + tid, a.N - 1);
            dma_lds4(a.scale_b + (a.quant_channel_b == 1 ? 0 : idx),
                     reinterpret_cast<int8_t *>(s_sbv) + (tid & ~63) * 4);
        }
    } else if constexpr (kRow) {
        if (mult_lane) {
            const int idx = m0 + tid;
            pre_sb = a.scale_b[a.quant_channel_b == 1 ? 0 : idx];
            if (a.bias) {
                pre_rbias = a.bias[idx];
            }
        }
    }
    if constexpr (!is_dyn(EPI) && !kRow) {
        if (a.bias) {
#pragma unroll
            for (int j = 0; j < NF; ++j) {
                const int gn = n0 + wn * WN + 32 * j + (lane & 31);
                pre_cbias[j] = gn < a.N ? static_cast<uint32_t>(a.bias[gn]) : 0u;
            }
        }
    }
    __shared__ int32_t s_rbias[kRow ? BM : 1];

    // Load-side lane roles. Plain rows: lane = 8 * row-in-block + LDS slot, the slot holding
    // k-chunk slot ^ ((row >> 1) & 7) of that row, so 8 consecutive lanes read one row's 128
    // bytes. Packed rows (16-byte chunks stored chunk-major in the panel): lane = 8 * slot +
    // row-in-block, so 8 consecutive lanes read one chunk of 8 consecutive rows (128 contiguous
    // bytes), and an 8-row block of LDS holds its chunks chunk-major, chunk c in slot
    // c ^ (block & 1) (lds_pos below).
    constexpr bool kAP = (PK & PK_A) != 0;
    constexpr bool kBP = (PK & PK_B) != 0;
    const int8_t *a_row[A_DMA];
    int a_mul[A_DMA];
    // Implicit convolution (NDHWC input, ICg % 128 == 0): stage st is 128 channels of one tap,
    // so row r of a stage is 128 contiguous input bytes of output pixel p0 + m0 + r's window
    // (zeros for a padding tap, read through the buffer resource's range check). c_o* is the
    // window's first input coordinate, c_base the byte offset of that pixel plus the lane's
    // 16-byte chunk.
    [[maybe_unused]] int c_od[A_DMA], c_oh[A_DMA], c_ow[A_DMA], c_base[A_DMA];
    [[maybe_unused]] i32x4 c_rsrc;
#pragma unroll
    for (int j = 0; j < A_DMA; ++j) {
        const int blk = wave * A_DMA + j;
        const int r = 8 * blk + (kAP ? (lane & 7) : (lane >> 3));
        const int chunk = kAP ? ((lane >> 3) ^ (blk & 1)) : ((lane & 7) ^ ((r >> 1) & 7));
        const int gm = min(m0 + r, a.M - 1);
        long long base;
        a_mul[j] = 1;  // k multiplier of a packed row (its panel width)
        if constexpr (kConv) {
            const ConvGeom &g = a.cv;
            // p0 + M < 2^31 on this path: 32-bit unsigned divisions
            const uint32_t p = static_cast<uint32_t>(a.p0) + static_cast<uint32_t>(gm);
            const uint32_t q1 = p / static_cast<uint32_t>(g.OW);
            const uint32_t q2 = q1 / static_cast<uint32_t>(g.OH);
            c_od[j] = static_cast<int>(q2) * g.SD - g.PD;
            c_oh[j] = static_cast<int>(q1 - q2 * static_cast<uint32_t>(g.OH)) * g.SH - g.PH;
            c_ow[j] = static_cast<int>(p - q1 * static_cast<uint32_t>(g.OW)) * g.SW - g.PW;
            // unsigned (wrapping) arithmetic: for a padding position the partial offsets leave
            // the input; once a tap is in range the sum is its true offset (< 2^31)
            c_base[j] = static_cast<int>(
                ((static_cast<uint32_t>(c_od[j]) * g.IH + static_cast<uint32_t>(c_oh[j])) * g.IW +
                 static_cast<uint32_t>(c_ow[j])) *
                    g.IC +
                chunk * 16u);
            base = 0;
        } else if constexpr (kAP) {
            base = pack_row_fixed<kPackI8MStep>(a.pa, gm, a_mul[j]);
        } else {
            base = static_cast<long long>(gm) * a.lda;
        }
        a_row[j] = a.A + base + pack_k<kPackI8Chunk, kAP>(chunk * 16, a_mul[j]);
    }
    if constexpr (kConv) {
        const uint64_t ab = reinterpret_cast<uint64_t>(a.A);
        c_rsrc[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(ab & 0xffffffffu));
        c_rsrc[1] = __builtin_amdgcn_readfirstlane(static_cast<int>((ab >> 32) & 0xffffu));
        c_rsrc[2] = __builtin_amdgcn_readfirstlane(a.conv_bytes);  // num_records
        c_rsrc[3] = 0x00020000;                                    // raw 32-bit dwords
    }
    // tap cursor of the next stage to issue (stages are issued in order)
    [[maybe_unused]] int t_ic = 0, t_kw = 0, t_kh = 0, t_kd = 0;
    const int8_t *b_row[B_DMA];
    int b_mul[B_DMA];
#pragma unroll
    for (int j = 0; j < B_DMA; ++j) {
        const int blk = wave * B_DMA + j;
        const int r = 8 * blk + (kBP ? (lane & 7) : (lane >> 3));
        const int chunk = kBP ? ((lane >> 3) ^ (blk & 1)) : ((lane & 7) ^ ((r >> 1) & 7));
        const int gn = min(n0 + r, a.N - 1);
        long long base;
        b_mul[j] = 1;
        if constexpr (kBP) {
            base = pack_row_fixed<kPackI8NStep>(a.pb, gn, b_mul[j]);
        } else {
            base = static_cast<long long>(gn) * a.ldb;
        }
        b_row[j] = a.B + base + pack_k<kPackI8Chunk, kBP>(chunk * 16, b_mul[j]);
    }

    auto issue = [&](int st, int8_t *sa, int8_t *sb) {
        const int k0 = st * kSK;
        if constexpr (kConv) {
            const ConvGeom &g = a.cv;
            const int dd = t_kd * g.DD, dh = t_kh * g.DH, dw = t_kw * g.DW;
            const uint32_t toff =
                ((static_cast<uint32_t>(dd) * g.IH + dh) * g.IW + dw) * g.IC + t_ic;
#pragma unroll
            for (int j = 0; j < A_DMA; ++j) {
                const int id = c_od[j] + dd, ih = c_oh[j] + dh, iw = c_ow[j] + dw;
                const bool ok = id >= 0 && id < g.ID && ih >= 0 && ih < g.IH && iw >= 0 &&
                                iw < g.IW;
                dma_lds16_buf(c_rsrc,
                              ok ? static_cast<int>(static_cast<uint32_t>(c_base[j]) + toff)
                                 : a.conv_bytes,
                              sa + (wave * A_DMA + j) * 1024);
            }
            t_ic += kSK;
            if (t_ic == g.ICg) {
                t_ic = 0;
                if (++t_kw == g.KW) {
                    t_kw = 0;
                    if (++t_kh == g.KH) {
                        t_kh = 0;
                        ++t_kd;
                    }
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < A_DMA; ++j) {
                dma_lds16(a_row[j] + pack_k<kPackI8Chunk, kAP>(k0, a_mul[j]),
                          sa + (wave * A_DMA + j) * 1024);
            }
        }
#pragma unroll
        for (int j = 0; j < B_DMA; ++j) {
            dma_lds16(b_row[j] + pack_k<kPackI8Chunk, kBP>(k0, b_mul[j]),
                      sb + (wave * B_DMA + j) * 1024);
        }
    };

    i32x16 acc[MF][NF];
#pragma unroll
    for (int i = 0; i < MF; ++i) {
#pragma unroll
        for (int j = 0; j < NF; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                acc[i][j][r] = 0;
            }
        }
    }
    // qai8dx x qsi8cx: this lane's share of sum_k q_b for its column (half of every 32 k)
    [[maybe_unused]] int32_t rs[NF] = {};

    // MFMA operand lanes: row r32 of a 32-row fragment, k-chunk 2 * step + h. LDS position of
    // (row, chunk) in a stage: plain rows keep 128 bytes per row, chunks XOR-swizzled; packed
    // rows keep 8-row blocks of chunk-major 16-byte slots (the 16 rows one ds_read_b128 pass
    // reads fall in two blocks whose slots sit 128 bytes apart modulo 256: no bank conflict).
    const int r32 = lane & 31;
    const int h = lane >> 5;
    auto lds_pos = [](bool packed, int row, int c) {
        return packed ? (row >> 3) * 1024 + ((((c ^ ((row >> 3) & 1)) << 3) + (row & 7)) << 4)
                      : row * kSK + ((c ^ ((row >> 1) & 7)) << 4);
    };
    constexpr int KS = kSK / 32;  // MFMA k-steps per stage
    auto compute = [&](const int8_t *sa, const int8_t *sb) {
        i32x4 fa[KS][MF], fb[KS][NF];
        auto read_step = [&](int step) {
            const int c = 2 * step + h;
#pragma unroll
            for (int i = 0; i < MF; ++i) {
                const int row = wm * WM + 32 * i + r32;
                fa[step][i] = *reinterpret_cast<const i32x4 *>(sa + lds_pos(kAP, row, c));
            }
#pragma unroll
            for (int j = 0; j < NF; ++j) {
                const int row = wn * WN + 32 * j + r32;
                fb[step][j] = *reinterpret_cast<const i32x4 *>(sb + lds_pos(kBP, row, c));
            }
        };
#pragma unroll
        for (int step = 0; step < KS; ++step) {
            read_step(step);
        }
#pragma unroll
        for (int step = 0; step < KS; ++step) {
#pragma unroll
            for (int i = 0; i < MF; ++i) {
#pragma unroll
                for (int j = 0; j < NF; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[step][i], fb[step][j],
                                                                      acc[i][j], 0, 0, 0);
                }
            }
        }
        if constexpr (is_dyn(EPI)) {
#pragma unroll
            for (int step = 0; step < KS; ++step) {
#pragma unroll
                for (int j = 0; j < NF; ++j) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        rs[j] = __builtin_amdgcn_sdot4(fb[step][j][q], 0x01010101, rs[j], false);
                    }
                }
            }
        }
        // Instruction order: the operands of k-step 0 first, then the operands of each next
        // k-step between the MFMAs of the current one, so LDS latency hides under the MFMAs.
        __builtin_amdgcn_sched_group_barrier(0x100, MF + NF, 0);
#pragma unroll
        for (int step = 1; step < KS; ++step) {
            __builtin_amdgcn_sched_group_barrier(0x100, MF + NF, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, MF * NF, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, MF * NF, 0);
    };

    const int nst = a.K / kSK;
    // One pipeline step: wait until this wave's loads of stage st landed (the stages issued after
    // it may stay in flight), meet the other waves, refill the buffer everyone finished reading
    // in the previous step with stage st + NS - 1, then compute stage st.
    auto step = [&](int st, const int8_t *cur, int8_t *nxt) {
        if (st >= nst) {
            return;
        }
        const int ahead = min(NS - 2, nst - 1 - st);
        static_assert(NS >= 3 && NS <= 6, "ring depth");
        if (ahead >= 4) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(4 * PER_STAGE));
        } else if (ahead == 3) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(3 * PER_STAGE));
        } else if (ahead == 2) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(2 * PER_STAGE));
        } else if (ahead == 1) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(PER_STAGE));
        } else {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (st + NS - 1 < nst) {
            issue(st + NS - 1, nxt, nxt + SA);
        }
        compute(cur, cur + SA);
        if constexpr (EPI == EPI_REQUANT_I8) {
            if (st == 1 && tid < kBN) {
                column_multiplier_val(a.scale_a, s_sbv[tid], a.scale_d, s_mult[tid], s_shift[tid]);
            }
        }
    };

#pragma unroll
    for (int i = 0; i < NS - 1; ++i) {
        if (nst > i) {
            issue(i, ring[i], ring[i] + SA);
        }
    }
    for (int st = 0; st < nst; st += NS) {
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            step(st + i, ring[i], ring[(i + NS - 1) % NS]);
        }
    }
    // Every load of this wave has landed (the last step waits for vmcnt(0)); saying so here lets
    // the compiler's own wait tracking drop the vmcnt(0) it would otherwise place before each
    // output of the epilogue for the epilogue inputs loaded above. Stores count in vmcnt too, so
    // each of those waits would drain the previous output's store (measured: 4.5 us of a
    // 22.4 us W8A8 M512 launch).
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    if constexpr (EPI == EPI_REQUANT_I8) {
        // With three stages or more, stage 2's wait (lgkmcnt(0)) and barrier already order the
        // multipliers' LDS stores before every wave's epilogue (no barrier here: 0.47 us less per
        // W8A8 M512 launch with the multipliers moved into the loop); shorter k computes them
        // here.
        if (nst < 2 && tid < kBN) {
            column_multiplier_val(a.scale_a, s_sbv[tid], a.scale_d, s_mult[tid], s_shift[tid]);
        }
        if (nst < 3) {
            __syncthreads();
        }
    } else {
        if constexpr (kRow) {
            if (mult_lane) {
                column_multiplier_val(a.scale_a, pre_sb, a.scale_d, s_mult[tid], s_shift[tid]);
                s_rbias[tid] = pre_rbias;
            }
        }
        __syncthreads();  // s_mult / s_shift / s_rbias visible to every wave
    }

    if constexpr (is_dyn(EPI)) {
        // lanes r32 and r32 + 32 summed the two 16-byte halves of every k-step of column r32
        int32_t rsum[NF];
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            rsum[j] = rs[j] + __shfl_xor(rs[j], 32);
        }
        int32_t zr[MF][16];
        float sar[MF][16];
        float sbc[NF], fbc[NF];
        bool in_range = true;
#pragma unroll
        for (int i = 0; i < MF; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int gm = m0 + wm * WM + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                zr[i][r] = gm < a.M ? a.dyn_za[gm] : 0;
                sar[i][r] = gm < a.M ? a.dyn_sa[gm] : 0.0f;
                in_range = in_range && dyn_zp_in_range(zr[i][r]);
            }
        }
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            const int gn = n0 + wn * WN + 32 * j + r32;
            sbc[j] = gn < a.N ? a.scale_b[gn] : 0.0f;
            fbc[j] = gn < a.N ? dyn_bias<EPI>(a, gn) : 0.0f;
        }
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));  // the compiler then adds no waits below
        if (in_range) {
#pragma unroll
            for (int j = 0; j < NF; ++j) {
                const int gn = n0 + wn * WN + 32 * j + r32;
#pragma unroll
                for (int i = 0; i < MF; ++i) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int gm = m0 + wm * WM + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                        if (gm < a.M && gn < a.N) {
                            const uint32_t x = static_cast<uint32_t>(acc[i][j][r]) -
                                               static_cast<uint32_t>(zr[i][r]) *
                                                   static_cast<uint32_t>(rsum[j]);
                            dyn_finish_v<EPI>(a, gn, a.d_row0 + gm, x, sbc[j], sar[i][r], fbc[j]);
                        }
                    }
                }
            }
        } else {
            // a zero point beyond 16 bits: this lane's outputs summed term by term
            for (int e = 0; e < NF * MF * 16; ++e) {
                const int j = e / (MF * 16), i = (e / 16) % MF, r = e % 16;
                const int gn = n0 + wn * WN + 32 * j + r32;
                const int gm = m0 + wm * WM + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                if (gm < a.M && gn < a.N) {
                    dyn_finish<EPI>(a, gm, gn, a.d_row0 + gm,
                                    dyn_exact_acc<PK>(a, gm, gn, a.dyn_za[gm]));
                }
            }
        }
        return;
    }

    // Epilogue: lane holds D[8 * (r / 4) + 4 * h + r % 4][r32] of each 32 x 32 fragment. Every
    // output's address is a wave-uniform base -- the wave's first row plus a compile-time row
    // offset, times the row stride, plus the fragment's first column: scalar arithmetic -- plus
    // the lane's 32-bit offset 4 h ld + r32, so stores and C loads take the SGPR-base form with
    // no per-output 64-bit VALU arithmetic (the launcher checks 4 ld + 32 < 2^31). Whole row
    // tiles skip the per-output row check.
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const int wm_u = wave_u / kStreamWavesN;
    const int wn_u = wave_u % kStreamWavesN;
    const int row_w = m0 + wm_u * WM;                   // the wave's first row (A / C rows)
    const long long drow_w = a.d_row0 + row_w;          // the same row of D
    constexpr int kES = EPI == EPI_CLAMP_I32 ? 4 : 1;   // bytes per D element
    const int ldd32 = static_cast<int>(a.ldd);          // 136 ldd kES < 2^31 (launch_stream)
    const uint32_t voff_d = (static_cast<uint32_t>(4 * h) * static_cast<uint32_t>(ldd32) + r32) * kES;
    const uint32_t voff_c = static_cast<uint32_t>(4 * h) * static_cast<uint32_t>(a.ldc) + r32;
    // D through a buffer resource based at the wave's first row and the tile's first column:
    // each store is the lane's offset plus a scalar offset (row and fragment column)
    const __amdgpu_buffer_rsrc_t d_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        static_cast<int8_t *>(a.D) + (drow_w * a.ldd + n0) * kES, 0, 0x7fffffff, 0x00020000);
    auto epilogue = [&](auto checked) {
        constexpr bool kChecked = decltype(checked)::value;
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            const int lc0 = wn_u * WN + 32 * j;  // the fragment's first column (uniform)
            const int lc = lc0 + r32;
            const int gn = n0 + lc;
            if (gn >= a.N) {
                continue;
            }
            const uint32_t bias = pre_cbias[j];  // 0 without a bias and for kRow
            int32_t mult = 0, shift = 0;
            if constexpr (EPI == EPI_REQUANT_I8) {
                mult = s_mult[lc];
                shift = s_shift[lc];
            }
            // C (optional) for every output of this column first, so the compiler waits for
            // them once rather than between stores
            uint32_t cv[MF][16] = {};
            if (a.C) {
#pragma unroll
                for (int i = 0; i < MF; ++i) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int dr = 32 * i + 8 * (r >> 2) + (r & 3);
                        if (!kChecked || row_w + 4 * h + dr < a.M) {
                            const int32_t *cp =
                                a.C + (static_cast<long long>(row_w + dr) * a.ldc + n0 + lc0);
                            cv[i][r] = static_cast<uint32_t>(cp[voff_c]);
                        }
                    }
                }
                __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));  // no compiler waits below
            }
#pragma unroll
            for (int i = 0; i < MF; ++i) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int dr = 32 * i + 8 * (r >> 2) + (r & 3);
                    const int gm = row_w + 4 * h + dr;
                    if (kChecked && gm >= a.M) {
                        continue;
                    }
                    uint32_t v = static_cast<uint32_t>(acc[i][j][r]) + bias + cv[i][r];
                    if constexpr (kRow) {
                        mult = s_mult[gm - m0];
                        shift = s_shift[gm - m0];
                        v += static_cast<uint32_t>(s_rbias[gm - m0]);  // 0 without a bias
                    }
                    const int soff = (dr * ldd32 + lc0) * kES;
                    if constexpr (EPI == EPI_CLAMP_I32) {
                        int32_t x = static_cast<int32_t>(v);
                        x = x < a.cmin ? a.cmin : x;
                        x = x > a.cmax ? a.cmax : x;
                        __builtin_amdgcn_raw_buffer_store_b32(x, d_rsrc, static_cast<int>(voff_d),
                                                              soff, 0);
                    } else {
                        const int8_t q = requant_dev(static_cast<int32_t>(v), mult, shift, a.zp_d,
                                                     a.cmin, a.cmax);
                        __builtin_amdgcn_raw_buffer_store_b8(static_cast<uint8_t>(q), d_rsrc,
                                                             static_cast<int>(voff_d), soff, 0);
                    }
                }
            }
        }
    };
    if (m0 + BM <= a.M) {
        epilogue(std::false_type{});
    } else {
        epilogue(std::true_type{});
    }
}

// Generic path: one thread per output, any strides and any K.
template <int AM, int BMd, int EPI, int PK>
__global__ __launch_bounds__(256) void int8_generic_kernel(Int8Args a)
{
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    const long long total = static_cast<long long>(a.M) * a.N;
    if (idx >= total) {
        return;
    }
    const int gm = static_cast<int>(idx / a.N);
    const int gn = static_cast<int>(idx - static_cast<long long>(gm) * a.N);
    if constexpr (is_dyn(EPI)) {
        dyn_finish<EPI>(a, gm, gn, a.d_row0 + gm, dyn_exact_acc<PK>(a, gm, gn, a.dyn_za[gm]));
        return;
    }
    uint32_t acc = 0;
    if constexpr (AM == A_MATRIX) {
        if constexpr (PK == PK_NONE) {
            const int8_t *arow = a.A + static_cast<long long>(gm) * a.lda;
            if constexpr (BMd == B_CF) {
                const long long p = a.p0 + gn;
                const long long ohw = static_cast<long long>(a.cv.OH) * a.cv.OW;
                const int od = static_cast<int>(p / ohw);
                const int oh = static_cast<int>((p / a.cv.OW) % a.cv.OH);
                const int ow = static_cast<int>(p % a.cv.OW);
                for (int k = 0; k < a.K; ++k) {
                    int kd, kh, kw;
                    const int8_t *plane = cf_tap(a, k, kd, kh, kw);
                    const int32_t bv = static_cast<int8_t>(
                        static_cast<uint8_t>(cf_byte(a, plane, kd, kh, kw, od, oh, ow, true)));
                    acc += static_cast<uint32_t>(static_cast<int32_t>(arow[k]) * bv);
                }
            } else {
                for (int k = 0; k < a.K; ++k) {
                    const int32_t bv = (BMd == B_NK) ? a.B[static_cast<long long>(gn) * a.ldb + k]
                                                     : a.B[static_cast<long long>(k) * a.ldb + gn];
                    acc += static_cast<uint32_t>(static_cast<int32_t>(arow[k]) * bv);
                }
            }
        } else {
            // packed operands (B_NK): the same sum, addressed through the panel layout; the run
            // functions of the p-variants describe an unpacked operand with step 0 (row-major)
            const PackRow ra = pack_row_info(a.pa, gm);
            const PackRow rb = pack_row_info(a.pb, gn);
            if constexpr (BMd == B_CF) {
                // packed weights (A) times the gathered channel-first im2col
                const long long p = a.p0 + gn;
                const long long ohw = static_cast<long long>(a.cv.OH) * a.cv.OW;
                const int od = static_cast<int>(p / ohw);
                const int oh = static_cast<int>((p / a.cv.OW) % a.cv.OH);
                const int ow = static_cast<int>(p % a.cv.OW);
                for (int k = 0; k < a.K; ++k) {
                    int kd, kh, kw;
                    const int8_t *plane = cf_tap(a, k, kd, kh, kw);
                    const int32_t bv = static_cast<int8_t>(
                        static_cast<uint8_t>(cf_byte(a, plane, kd, kh, kw, od, oh, ow, true)));
                    acc += static_cast<uint32_t>(
                        static_cast<int32_t>(a.A[pack_row_byte(ra, k)]) * bv);
                }
            } else {
                for (int k = 0; k < a.K; ++k) {
                    acc += static_cast<uint32_t>(
                        static_cast<int32_t>(a.A[pack_row_byte(ra, k)]) *
                        static_cast<int32_t>(a.B[pack_row_byte(rb, k)]));
                }
            }
        }
    } else {
        const ConvGeom &g = a.cv;
        const long long p = a.p0 + gm;
        const long long ohw = static_cast<long long>(g.OH) * g.OW;
        const int od = static_cast<int>(p / ohw);
        const int oh = static_cast<int>((p / g.OW) % g.OH);
        const int ow = static_cast<int>(p % g.OW);
        const int8_t *w = a.B + static_cast<long long>(gn) * a.ldb;
        const PackRow rw = pack_row_info(a.pb, gn);  // used when the weights are packed
        long long kb = 0;                            // k of the current tap's first channel
        const int taps = a.K / g.ICg;
        for (int tap = 0; tap < taps; ++tap) {
            const int kw = tap % g.KW;
            const int kh = (tap / g.KW) % g.KH;
            const int kd = tap / (g.KW * g.KH);
            const int id = od * g.SD + kd * g.DD - g.PD;
            const int ih = oh * g.SH + kh * g.DH - g.PH;
            const int iw = ow * g.SW + kw * g.DW - g.PW;
            const bool inb = id >= 0 && id < g.ID && ih >= 0 && ih < g.IH && iw >= 0 && iw < g.IW;
            const int8_t *src =
                inb ? a.A + ((static_cast<long long>(id) * g.IH + ih) * g.IW + iw) * g.IC : nullptr;
            for (int ic = 0; ic < g.ICg; ++ic) {
                const int32_t av = src ? static_cast<int32_t>(src[ic]) : 0;
                const int32_t wv = (PK & PK_B) ? static_cast<int32_t>(a.B[pack_row_byte(rw, kb + ic)])
                                               : static_cast<int32_t>(w[ic]);
                acc += static_cast<uint32_t>(av * wv);
            }
            w += g.ICg;
            kb += g.ICg;
        }
    }
    if (a.C) {
        acc += static_cast<uint32_t>(a.C[static_cast<long long>(gm) * a.ldc + gn]);
    }
    constexpr bool kRow = EPI == EPI_REQUANT_ROW;
    if (a.bias) {
        acc += static_cast<uint32_t>(a.bias[kRow ? gm : gn]);
    }
    const long long drow = a.d_row0 + gm;
    if constexpr (EPI == EPI_CLAMP_I32) {
        int32_t x = static_cast<int32_t>(acc);
        x = x < a.cmin ? a.cmin : x;
        x = x > a.cmax ? a.cmax : x;
        static_cast<int32_t *>(a.D)[drow * a.ldd + gn] = x;
    } else {
        int32_t mult, shift;
        column_multiplier_dev(a.scale_a, a.scale_b, a.quant_channel_b, a.scale_d, kRow ? gm : gn,
                              mult, shift);
        static_cast<int8_t *>(a.D)[drow * a.ldd + gn] =
            requant_dev(static_cast<int32_t>(acc), mult, shift, a.zp_d, a.cmin, a.cmax);
    }
}

// The streaming kernel's epilogue addresses D (and C) with 32-bit offsets from a tile's first row:
// 136 rows of either must span less than 2 GiB.
inline bool stream_offsets_fit(const Int8Args &a, int d_bytes)
{
    return 136ll * a.ldd * d_bytes < (1ll << 31) && (a.C == nullptr || 136ll * a.ldc * 4 < (1ll << 31));
}

template <int EPI, int PK, bool kConv = false>
void launch_stream(const Int8Args &a, hipStream_t stream)
{
    const long long tiles_n = (a.N + kBN - 1) / kBN;
    const long long tm128 = (a.M + 127) / 128;
    const long long tm64 = (a.M + 63) / 64;
    // 128-row tiles when they still give most of the 256 CUs a workgroup.
    const bool big = tm128 * tiles_n >= 160;
    const long long tiles_m = big ? tm128 : tm64;
    const long long tiles = tiles_m * tiles_n;
    const long long per_xcd = (tiles + 7) / 8;
    TQT_REQUIRE(tiles < (1ll << 30), "grid too large");
    if (big) {
        hipLaunchKernelGGL((int8_stream_kernel<128, EPI, PK, kConv>), dim3(8 * per_xcd),
                           dim3(kStreamThreads), 0, stream, a, static_cast<int>(tiles_m),
                           static_cast<int>(tiles), static_cast<int>(per_xcd));
    } else {
        hipLaunchKernelGGL((int8_stream_kernel<64, EPI, PK, kConv>), dim3(8 * per_xcd),
                           dim3(kStreamThreads), 0, stream, a, static_cast<int>(tiles_m),
                           static_cast<int>(tiles), static_cast<int>(per_xcd));
    }
}

// ---------------------------------------------------------------------------------------------
// Implicit convolution through an LDS input halo (igemmcl, plain or packed weights; 2-D: one
// depth tap, depth stride 1, no depth padding; 3 x 3 taps, stride 1, dilation 1, padding 1 in h
// and w, so OH = IH and OW = IW; 128 channels per group).
//
// Output pixels are numbered row by row through the depth (batch) axis. With these geometries
// "stacked" output row R = od * OH + oh reads stacked input rows R - 1 .. R + 1 (input row
// od * IH + ih), so a tile of 256 consecutive pixels spanning stacked output rows R0 .. R1 reads
// stacked input rows R0 - 1 .. R1 + 1 only: the tile's halo, NR rows of IW + 2 pixels (the two
// border columns, and rows outside the input, zero) at a row pitch HC >= IW + 2 (below). A tap
// whose input row belongs to the previous or next image (the padding row between images) reads
// a zero line instead of the halo row. Every input byte a tile needs is loaded into LDS once: at
// the benchmark geometry (56 x 56 x 128, 256 x 64 tiles) 58 KiB of halo and 72 KiB of weights per
// workgroup, against 288 KiB of per-tap rows and weights for the streaming kernel's 128 x 128
// tiles.
//
// Every load moves whole 128-byte lines (a pixel's 128 channels, or one tap's 128 channels of a
// weight row): the memory system moves whole lines, so a split of each line over several stages
// would fetch it once per stage. The k loop therefore runs tap by tap, in stages of one kernel
// row (3 taps). The epilogue inputs and the whole halo are requested first, then each tap's
// weights (64 rows x 128 bytes: one 1 KiB block per wave), kHaloAhead stages ahead of the compute:
// every wave has the same loads outstanding behind each stage, so each stage's wait is a constant
// vmcnt (runtime counts would need a compare-and-branch tree of waits per stage: measured 3x
// slower), and stage 0 waits for the halo as well. Everything stays resident (no buffer is
// reused): no barrier other than each stage's arrival. A tap is 4 MFMA k-steps (32 channels
// each); a stage's 12 k-steps run as one software pipeline.
//
// MFMA operands: the weights are the 32-row operand and the pixels the 32-column operand, so the
// accumulator of a lane is one pixel (its column) and 16 channels in four runs of four consecutive
// channels (rows 8 g + 4 h + e): the epilogue writes 4 requantized channels per dword store.
//
// LDS: a pixel (or weight row) is 8 units of 16 bytes; chunk c of pixel q sits in unit
// 8 q + (c ^ ((q >> 1) & 7)), so any 16 consecutive pixels (or weight rows) a ds_read_b128 pass
// reads fall in 16 distinct 16-byte slots modulo 256 bytes: no bank conflicts (the halo pitch
// keeps consecutive output pixels consecutive modulo 16 across a row change where the halo still
// fits that way; counters: 416 conflict cycles per launch against 190 K). Loads are LDS-DMA:
// a load block fills 1 KiB (64 lanes x 16 bytes, 8 pixels) in lane order, each lane fetching the
// global chunk its position holds; 8 consecutive lanes read one pixel's 128 bytes.
constexpr int kHaloPix = 256;               // output pixels per workgroup
constexpr int kHaloCh = 64;                 // output channels per workgroup
constexpr int kHaloTaps = 9;                // 3 x 3
constexpr int kHaloWBlocks = 8;             // 1 KiB weight load blocks per tap (64 x 128 B)
constexpr int kHaloLdsBytes = 152 * 1024;   // halo + weights + a zero line
constexpr int kHaloTPS = 3;                 // taps per stage (one kernel row)
constexpr int kHaloStages = kHaloTaps / kHaloTPS;
constexpr int kHaloAhead = 2;               // stages in flight ahead of the one computed
constexpr int kHaloReadAhead = 2;           // k-steps of operands read ahead of the MFMAs

struct HaloPlan
{
    int HC;       // halo row pitch in pixels (>= IW + 2; the pixels past IW + 1 zero)
    int NRHC;     // halo pixels (NR rows)
    int HB;       // halo blocks
    int b_bytes;  // bytes of B from its base through the last weight byte
    int tiles_c;  // 64-channel tiles
    int tiles;    // workgroups with work
    int per_xcd;  // tiles per XCD (grid = 8 per_xcd)
};

// Raw buffer resource (stride 0, 32-bit dwords format): offsets at or past num_records read zeros.
__device__ __forceinline__ i32x4 raw_rsrc(const void *base, int num_records)
{
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    i32x4 r;
    r[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(b & 0xffffffffu));
    r[1] = __builtin_amdgcn_readfirstlane(static_cast<int>((b >> 32) & 0xffffu));
    r[2] = __builtin_amdgcn_readfirstlane(num_records);
    r[3] = 0x00020000;
    return r;
}

template <int PK>
__global__ __launch_bounds__(kStreamThreads) void conv_halo_kernel(Int8Args a, HaloPlan hp)
{
    static_assert(PK == PK_NONE || PK == PK_B, "plain or packed weights");
    __shared__ __attribute__((aligned(128))) int8_t lds[kHaloLdsBytes];
    __shared__ __attribute__((aligned(16))) int32_t s_mult[kHaloCh];
    __shared__ __attribute__((aligned(16))) int32_t s_shift[kHaloCh];
    __shared__ __attribute__((aligned(16))) int32_t s_bias[kHaloCh];
    __shared__ __attribute__((aligned(16))) float s_sb[kHaloCh];

    const int t = (blockIdx.x & 7) * hp.per_xcd + (blockIdx.x >> 3);
    if (t >= hp.tiles) {
        return;
    }
    // the two channel tiles of a pixel tile are neighbours in t, so they run on one XCD and
    // share the halo through its L2
    const int tile_c = t % hp.tiles_c;
    const int m0 = (t / hp.tiles_c) * kHaloPix;
    const int n0 = tile_c * kHaloCh;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const ConvGeom &g = a.cv;
    const int w_base = hp.HB * 1024;                     // weights: 9 taps x 8 blocks
    const int zero_base = w_base + kHaloTaps * kHaloWBlocks * 1024;  // 128 zero bytes

    // Epilogue inputs (the 64 channels' weight scales and biases; channels past N repeat the
    // last, and are not stored) by LDS-DMA ahead of everything else: the first stage's wait
    // covers them, and the compiler places no wait of its own for them.
    if (wave == 0) {
        const int ch = min(n0 + lane, a.N - 1);
        dma_lds4(a.scale_b + (a.quant_channel_b == 1 ? 0 : ch), reinterpret_cast<int8_t *>(s_sb));
        if (a.bias) {
            dma_lds4(a.bias + ch, reinterpret_cast<int8_t *>(s_bias));
        } else {
            s_bias[lane] = 0;
        }
    }
    if (tid < 8) {
        *reinterpret_cast<i32x4 *>(lds + zero_base + 16 * tid) = i32x4{0, 0, 0, 0};
    }

    // p0 + M < 2^31 on this path (launcher): 32-bit unsigned divisions
    const uint32_t OW = static_cast<uint32_t>(g.OW);
    const uint32_t IH = static_cast<uint32_t>(g.IH);
    const int R0 = static_cast<int>((static_cast<uint32_t>(a.p0) + static_cast<uint32_t>(m0)) / OW);
    const int nrows = g.ID * g.IH;  // stacked input rows
    const i32x4 a_rsrc = raw_rsrc(a.A, a.conv_bytes);
    const i32x4 b_rsrc = raw_rsrc(a.B, hp.b_bytes);
    const int slot = lane & 7;
    const int sub = lane >> 3;  // pixel (weight row) of a block this lane's 8-lane group reads

    // The halo: blocks wave, wave + 8, ... (8 pixels each); pixels past the halo's NR rows,
    // border columns and rows outside the input read zeros (offset past the resource). A lane's
    // pixel advances by 64 per block: its halo row, column and input offset step by uniform
    // amounts (one wrap at most: 64 mod HC < HC), so the loop needs no division or multiply.
    {
        const int q0 = wave * 8 + sub;
        int jr = q0 / hp.HC;
        int col = q0 - jr * hp.HC;
        const int djr = 64 / hp.HC;
        const int dcol = 64 - djr * hp.HC;
        // input offset of (row R0 - 1 + jr, column col - 1): row-major pixels, IC bytes each;
        // unsigned (wrapping) arithmetic: outside the input (row -1, rows past the last, the
        // border columns) the value is not used, and where it is used it is below 2^31
        uint32_t off = (static_cast<uint32_t>(R0 - 1 + jr) * static_cast<uint32_t>(g.IW) +
                        static_cast<uint32_t>(col - 1)) *
                           static_cast<uint32_t>(g.IC) +
                       static_cast<uint32_t>((slot ^ ((q0 >> 1) & 7)) * 16);
        const uint32_t doff = static_cast<uint32_t>((djr * g.IW + dcol) * g.IC);
        // a row wrap: HC pixels back, IW forward
        const uint32_t wrap = static_cast<uint32_t>((g.IW - hp.HC) * g.IC);
        for (int hb = wave; hb < hp.HB; hb += 8) {
            const int G = R0 - 1 + jr;
            const bool in = hb * 8 + sub < hp.NRHC && G >= 0 && G < nrows && col >= 1 &&
                            col <= g.IW;
            dma_lds16_buf(a_rsrc, in ? static_cast<int>(off) : a.conv_bytes, lds + hb * 1024);
            jr += djr;
            col += dcol;
            off += doff;
            if (col >= hp.HC) {
                col -= hp.HC;
                ++jr;
                off += wrap;
            }
        }
    }
    // Weights: block `wave` of tap t is rows 8 wave .. 8 wave + 7 of the tile's 64, tap t's 128
    // channels (bytes 128 t of the row), read as 8 whole 128-byte lines, one per 8-lane group
    // (LDS-DMA puts lane i's 16 bytes at byte 16 i of the block). Plain weights: group `sub`
    // reads row 8 wave + sub, its chunks in slots XOR-swizzled by the row. Packed weights
    // (panels of 128 rows, 16-byte chunks chunk-major: chunk c of row r at the row's base plus
    // 16 c w, w = the panel's height; the tile's 64 rows lie in one panel): group `sub` reads
    // chunk sub ^ (wave & 1) of the 8 rows, which lie side by side, so the block is chunk-major
    // with its 128-byte chunk pairs swapped in odd blocks; a tap steps by 128 w.
    int w_off, w_tap;
    if constexpr (PK == PK_B) {
        const int w_row = min(n0 + wave * 8 + slot, a.N - 1);
        int mul;
        w_off = static_cast<int>(pack_row_fixed<kPackI8NStep>(a.pb, w_row, mul)) +
                (sub ^ (wave & 1)) * 16 * mul;
        w_tap = g.ICg * mul;
    } else {
        const int w_nr = wave * 8 + sub;
        const int w_row = min(n0 + w_nr, a.N - 1);
        w_off = w_row * static_cast<int>(a.ldb) + (slot ^ ((w_nr >> 1) & 7)) * 16;
        w_tap = g.ICg;
    }
    auto issue_w = [&](int tp) {
        dma_lds16_buf(b_rsrc, w_off + tp * w_tap, lds + w_base + (tp * kHaloWBlocks + wave) * 1024);
    };
    auto issue_stage = [&](int st) {
#pragma unroll
        for (int tt = 0; tt < kHaloTPS; ++tt) {
            issue_w(st * kHaloTPS + tt);
        }
    };

    // Compute roles: wave (wc = wave >> 2, wp = wave & 3) computes channels 32 wc .. 32 wc + 31
    // x pixels 64 wp .. 64 wp + 63 of the tile (1 x 2 fragments) over the four k-steps of every
    // tap; the two waves of a SIMD (w and w + 4) hold the two channel halves. Lane (r32, h)
    // supplies row / column r32 and channel half h of each 32-channel k-step (chunk 2 k + h of
    // the 8).
    constexpr int KPW = 4;  // k-steps per tap
    constexpr int RW = 1;   // 32-channel fragments per wave
    constexpr int RP = 2;   // 32-pixel fragments per wave
    const int wp = wave & 3;
    const int jbase = wave >> 2;
    const int r32 = lane & 31;
    const int h = lane >> 5;
    // the lane's unit of k-step k is (address ^ 32 k) in a pixel row and (address ^ WKX k) in
    // a weight block: the XOR touches the chunk bits above h's only. A 16-lane pass of a
    // ds_read_b128 (16 rows of one chunk) covers the 16 slots of 256 bytes once in either
    // weight layout.
    constexpr int WKX = PK == PK_B ? 256 : 32;
    int w_addr[RW];  // + 8192 tap
#pragma unroll
    for (int jj = 0; jj < RW; ++jj) {
        const int nr = (jbase + jj) * 32 + r32;
        if constexpr (PK == PK_B) {
            const int blk = nr >> 3;
            w_addr[jj] = w_base + blk * 1024 + (h ^ (blk & 1)) * 128 + (nr & 7) * 16;
        } else {
            w_addr[jj] = w_base + nr * 128 + ((16 * h) ^ (16 * ((nr >> 1) & 7)));
        }
    }
    // per fragment: the halo pixel of tap (0, 0), and whether the top / bottom kernel rows lie in
    // this pixel's image
    int qb[RP];
    bool ok_top[RP], ok_bot[RP];
#pragma unroll
    for (int i = 0; i < RP; ++i) {
        const int pl = min(m0 + wp * 64 + 32 * i + r32, a.M - 1);  // rows past M: any valid pixel
        const uint32_t p = static_cast<uint32_t>(a.p0) + static_cast<uint32_t>(pl);
        const uint32_t R = p / OW;
        const int ow = static_cast<int>(p - R * OW);
        const int oh = static_cast<int>(R % IH);
        qb[i] = (static_cast<int>(R) - R0) * hp.HC + ow;
        ok_top[i] = oh > 0;
        ok_bot[i] = oh + 1 < g.IH;
    }

    i32x16 acc[RW][RP];  // [channel fragment][pixel fragment]
#pragma unroll
    for (int jj = 0; jj < RW; ++jj) {
#pragma unroll
        for (int i = 0; i < RP; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                acc[jj][i][r] = 0;
            }
        }
    }
#pragma unroll
    for (int st = 0; st < kHaloAhead; ++st) {
        issue_stage(st);
    }
#pragma unroll
    for (int st = 0; st < kHaloStages; ++st) {
        // this wave's loads up to stage st's weights have landed once at most the weight blocks
        // issued after them are outstanding (the epilogue inputs and the halo were requested
        // first); then every wave's have, after the barrier (the LDS stores of the zero line
        // and of a null bias too: lgkmcnt(0))
        const int later = kHaloTPS * min(kHaloAhead - 1, kHaloStages - 1 - st);
        static_assert(kHaloTPS * (kHaloAhead - 1) <= 8, "wait counts below");
        if (later == 8) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(8));
        } else if (later == 6) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(6));
        } else if (later == 4) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(4));
        } else if (later == 3) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(3));
        } else if (later == 2) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(2));
        } else if (later == 1) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(1));
        } else {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (st + kHaloAhead < kHaloStages) {
            issue_stage(st + kHaloAhead);
        }
        // pixel operand addresses of the stage's taps (a padding-row tap reads the zero line)
        int pa[kHaloTPS][RP];
#pragma unroll
        for (int tt = 0; tt < kHaloTPS; ++tt) {
            const int s = st * kHaloTPS + tt;
            const int kh = s / 3;
            const int tap_q = kh * hp.HC + (s - 3 * kh);
#pragma unroll
            for (int i = 0; i < RP; ++i) {
                const int q = qb[i] + tap_q;
                const bool ok = kh == 0 ? ok_top[i] : kh == 2 ? ok_bot[i] : true;
                pa[tt][i] = ok ? q * 128 + ((16 * h) ^ (16 * ((q >> 1) & 7))) : zero_base + 16 * h;
            }
        }
        // the stage's k-steps (its taps' KPW steps each) as one pipeline: the operands of step
        // u + 1 are read between the MFMAs of step u
        constexpr int NSTEP = kHaloTPS * KPW;
        i32x4 fw[NSTEP][RW], fp[NSTEP][RP];
#pragma unroll
        for (int u = 0; u < NSTEP; ++u) {
            const int tt = u / KPW;
            const int kx = 32 * (u % KPW);
#pragma unroll
            for (int jj = 0; jj < RW; ++jj) {
                fw[u][jj] = *reinterpret_cast<const i32x4 *>(
                    lds + ((w_addr[jj] + (st * kHaloTPS + tt) * 8192) ^ (WKX * (u % KPW))));
            }
#pragma unroll
            for (int i = 0; i < RP; ++i) {
                fp[u][i] = *reinterpret_cast<const i32x4 *>(lds + (pa[tt][i] ^ kx));
            }
        }
#pragma unroll
        for (int u = 0; u < NSTEP; ++u) {
#pragma unroll
            for (int jj = 0; jj < RW; ++jj) {
#pragma unroll
                for (int i = 0; i < RP; ++i) {
                    acc[jj][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[u][jj], fp[u][i],
                                                                       acc[jj][i], 0, 0, 0);
                }
            }
        }
        // reads run kHaloReadAhead steps ahead of the MFMAs (1 to 4 steps measured the same: the
        // loop is bound by the LDS read rate while MFMAs run, not by the read latency)
        __builtin_amdgcn_sched_group_barrier(0x100, (RW + RP) * kHaloReadAhead, 0);
#pragma unroll
        for (int u = 0; u < NSTEP; ++u) {
            if (u + kHaloReadAhead < NSTEP) {
                __builtin_amdgcn_sched_group_barrier(0x100, RW + RP, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, RW * RP, 0);
        }
        if (st == 1 && wave == 0) {
            // the channels' requantization multipliers, while this stage's MFMAs run
            int32_t mult, shift;
            column_multiplier_val(a.scale_a, s_sb[lane], a.scale_d, mult, shift);
            s_mult[lane] = mult;
            s_shift[lane] = shift;
        }
    }

    // No barrier here: wave 0 wrote the multipliers in stage 1, and stage 2's wait (lgkmcnt(0))
    // and barrier order those LDS stores before every wave's epilogue reads (a barrier here
    // measured 0.2 µs slower: it held each wave's epilogue until the slowest wave's last MFMA).
    static_assert(kHaloStages >= 3, "a stage barrier follows the multipliers' stage");

    // Epilogue: lane holds pixel m0 + 64 wp + 32 i + r32 and channels n0 + cb + 8 g + e.
    const int cb = jbase * 32 + 4 * h;
    i32x4 em[4], es[4], eb[4];
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
        em[gq] = *reinterpret_cast<const i32x4 *>(&s_mult[cb + 8 * gq]);
        es[gq] = *reinterpret_cast<const i32x4 *>(&s_shift[cb + 8 * gq]);
        eb[gq] = *reinterpret_cast<const i32x4 *>(&s_bias[cb + 8 * gq]);
    }
    // Four requantized channels go into one dword with two byte permutes and an OR.
    const int32_t lo = min(a.cmin, a.cmax);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int pl = m0 + wp * 64 + 32 * i + r32;
        if (pl >= a.M) {
            continue;
        }
        int8_t *drow = static_cast<int8_t *>(a.D) + (a.d_row0 + pl) * a.ldd + n0 + cb;
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
            uint32_t y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t v = static_cast<uint32_t>(acc[0][i][4 * gq + e]) +
                                   static_cast<uint32_t>(eb[gq][e]);
                y[e] = static_cast<uint32_t>(requant_clamped_dev(
                    static_cast<int32_t>(v), em[gq][e], es[gq][e], a.zp_d, lo, a.cmax));
            }
            // v_perm_b32 byte k of {S0, S1} (S1 bytes 0-3): low bytes of y0, y1 | y2, y3
            const uint32_t packed = __builtin_amdgcn_perm(y[1], y[0], 0x0c0c0400u) |
                                    __builtin_amdgcn_perm(y[3], y[2], 0x04000c0cu);
            const int ch = n0 + cb + 8 * gq;
            if (ch + 3 < a.N) {
                *reinterpret_cast<uint32_t *>(drow + 8 * gq) = packed;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (ch + e < a.N) {
                        drow[8 * gq + e] = static_cast<int8_t>(packed >> (8 * e));
                    }
                }
            }
        }
    }
}

// The halo kernel's plan for this call, or false when its geometry or sizes do not fit it.
bool halo_plan(const Int8Args &a, bool packed, HaloPlan &hp)
{
    const ConvGeom &g = a.cv;
    if (g.KD != 1 || g.PD != 0 || g.SD != 1 || g.KH != 3 || g.KW != 3 || g.SH != 1 || g.SW != 1 ||
        g.DH != 1 || g.DW != 1 || g.PH != 1 || g.PW != 1 || g.OH != g.IH || g.OW != g.IW) {
        return false;
    }
    if (g.ICg != 128 || a.conv_bytes <= 0) {
        return false;
    }
    // dword stores of 4 channels; pixel offsets of a tile and the B offsets fit 31 bits
    if ((reinterpret_cast<uintptr_t>(a.D) & 3u) != 0 || a.ldd % 4 != 0 ||
        static_cast<long long>(kHaloPix) * a.ldd >= (1ll << 31)) {
        return false;
    }
    // bytes of B the loads may address: plain rows, or whole 128-row panels when packed
    const long long b_bytes =
        packed ? static_cast<long long>((a.N + kPackI8NStep - 1) / kPackI8NStep) * kPackI8NStep * a.ldb
               : static_cast<long long>(a.N - 1) * a.ldb + a.K;
    if (a.ldb < a.K || b_bytes >= (1ll << 31)) {
        return false;
    }
    const long long RS = (g.OW - 1 + kHaloPix - 1) / g.OW + 1;  // most output rows per tile
    // Row pitch: with pitch = OW modulo 16, the 16 consecutive output pixels of a ds_read_b128
    // pass sit at 16 consecutive halo pixels modulo 16 across a change of output row too (no
    // bank conflict; with pitch IW + 2 such a pass puts two pairs of lanes on one slot). Taken
    // when the halo still fits; IW + 2 otherwise.
    const long long HCmin = static_cast<long long>(g.IW) + 2;
    const long long HCcf = HCmin + ((g.OW - HCmin) & 15);
    auto fits = [&](long long hc) {
        return ((RS + 2) * hc + 7) / 8 + kHaloTaps * kHaloWBlocks <= (kHaloLdsBytes - 128) / 1024;
    };
    const long long HC = fits(HCcf) ? HCcf : HCmin;
    if (!fits(HC)) {
        return false;
    }
    const long long NRHC = (RS + 2) * HC;
    const long long HB = (NRHC + 7) / 8;
    // stacked row indices and halo offsets in 32 bits
    if (static_cast<long long>(g.ID) * g.IH >= (1ll << 30) || a.p0 + a.M >= (1ll << 31)) {
        return false;
    }
    hp.HC = static_cast<int>(HC);
    hp.NRHC = static_cast<int>(NRHC);
    hp.HB = static_cast<int>(HB);
    hp.b_bytes = static_cast<int>(b_bytes);
    hp.tiles_c = (a.N + kHaloCh - 1) / kHaloCh;
    const long long tiles = static_cast<long long>((a.M + kHaloPix - 1) / kHaloPix) * hp.tiles_c;
    if (tiles >= (1ll << 30)) {
        return false;
    }
    hp.tiles = static_cast<int>(tiles);
    hp.per_xcd = static_cast<int>((tiles + 7) / 8);
    return true;
}

// ---------------------------------------------------------------------------------------------
// Small clamp_i32 problems ([k, n] B; M, N multiples of 32, k % 128 == 0, k <= 2048) that would
// give int8_mfma_kernel's 64 x 128 tiles only a few workgroups (the reference's shape list and
// the 64 x 256 x 512 configuration: 2): 32 x 32 output tiles, and the four waves of a workgroup
// split k, so every load of the workgroup is issued at once. Wave w takes k in
// [w k / 4, (w + 1) k / 4): A fragments straight from global memory (lane (r, h): 16 bytes of
// row r per 32-k step), B rows (32 columns x 32 bytes) loaded whole and transposed byte by byte
// into the wave's own [n][k] LDS block, read back as the MFMA's 16-k column slices;
// v_mfma_i32_32x32x32_i8. The four int32 partial tiles are added in LDS (exact: wrapping int32),
// then C, the reference's max-then-min clamp, int32 stores.
// ---------------------------------------------------------------------------------------------
constexpr int kSmallT = 32;                    // output tile edge
constexpr int kSmallMaxK = 2048;               // k per workgroup
constexpr int kSmallKW = kSmallMaxK / 4;       // k per wave at most
constexpr int kSmallPitch = kSmallKW + 16;     // bytes per LDS column row (16-byte aligned)

__global__ __launch_bounds__(256) void int8_small_clamp_kernel(Int8Args a)
{
    __shared__ __attribute__((aligned(16))) int8_t s_b[4][kSmallT][kSmallPitch];
    __shared__ __attribute__((aligned(16))) int32_t s_part[4][kSmallT * kSmallT];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int tiles_n = a.N / kSmallT;
    const int m0 = (blockIdx.x / tiles_n) * kSmallT;
    const int n0 = (blockIdx.x % tiles_n) * kSmallT;
    const int kw = a.K / 4;          // a multiple of 32
    const int k0 = wave * kw;
    const int steps = kw / 32;       // 1 .. 16
    const int r32 = lane & 31;
    const int h = lane >> 5;

    // A fragments of this wave's k-slice, and its B rows (lane: row k0 + 32 it + lane / 2,
    // columns n0 + 16 (lane & 1) .. + 15), all requested before any is used
    i32x4 fa[kSmallKW / 32];
    i32x4 bb[kSmallKW / 32];
    const int8_t *arow = a.A + static_cast<long long>(m0 + r32) * a.lda + k0 + 16 * h;
    const int8_t *bcol = a.B + static_cast<long long>(k0 + (lane >> 1)) * a.ldb + n0 + 16 * (lane & 1);
#pragma unroll
    for (int st = 0; st < kSmallKW / 32; ++st) {
        if (st < steps) {
            fa[st] = *reinterpret_cast<const i32x4 *>(arow + 32 * st);
            bb[st] = *reinterpret_cast<const i32x4 *>(bcol + static_cast<long long>(32 * st) * a.ldb);
        }
    }
    // B transposed into this wave's [n][k] block: byte j of the lane's chunk is column
    // 16 (lane & 1) + j of row 32 st + lane / 2
    int8_t(*sb)[kSmallPitch] = s_b[wave];
#pragma unroll
    for (int st = 0; st < kSmallKW / 32; ++st) {
        if (st < steps) {
            const int kk = 32 * st + (lane >> 1);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                sb[16 * (lane & 1) + j][kk] =
                    static_cast<int8_t>(static_cast<uint32_t>(bb[st][j >> 2]) >> (8 * (j & 3)));
            }
        }
    }
    // the wave reads back only what it wrote: its own LDS stores are in order, no barrier
    i32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        acc[r] = 0;
    }
#pragma unroll
    for (int st = 0; st < kSmallKW / 32; ++st) {
        if (st < steps) {
            const i32x4 fb = *reinterpret_cast<const i32x4 *>(&sb[r32][32 * st + 16 * h]);
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[st], fb, acc, 0, 0, 0);
        }
    }
    // lane (column r32, half h) holds rows 8 g + 4 h + e, e < 4, of its column
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        s_part[wave][(8 * (i >> 2) + 4 * h + (i & 3)) * kSmallT + r32] = acc[i];
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kSmallT * kSmallT / 256; ++q) {
        const int o = tid + 256 * q;
        const int row = o / kSmallT, col = o % kSmallT;
        uint32_t v = static_cast<uint32_t>(s_part[0][o]) + static_cast<uint32_t>(s_part[1][o]) +
                     static_cast<uint32_t>(s_part[2][o]) + static_cast<uint32_t>(s_part[3][o]);
        if (a.C) {
            v += static_cast<uint32_t>(a.C[static_cast<long long>(m0 + row) * a.ldc + n0 + col]);
        }
        int32_t x = static_cast<int32_t>(v);
        x = x < a.cmin ? a.cmin : x;
        x = x > a.cmax ? a.cmax : x;
        static_cast<int32_t *>(a.D)[static_cast<long long>(m0 + row) * a.ldd + n0 + col] = x;
    }
}

// The small clamp_i32 kernel when the shape fits it and the regular tiles would be few.
bool launch_small_clamp(const Int8Args &a, hipStream_t stream)
{
    const long long regular = ((a.M + 63) / 64) * static_cast<long long>((a.N + kBN - 1) / kBN);
    if (regular >= 64 || a.M % kSmallT != 0 || a.N % kSmallT != 0 || a.K % 128 != 0 ||
        a.K > kSmallMaxK || a.K == 0) {
        return false;
    }
    const long long blocks = static_cast<long long>(a.M / kSmallT) * (a.N / kSmallT);
    hipLaunchKernelGGL(int8_small_clamp_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       stream, a);
    return true;
}

template <int AM, int BMd, int EPI, int PK = PK_NONE>
void launch_int8(const Int8Args &a, bool fast, hipStream_t stream, const char *where)
{
    if (a.M <= 0 || a.N <= 0) {
        return;
    }
    // The streaming kernel takes plain (or packed) matrices and the implicit convolution whose
    // group channel count is a multiple of its 128-byte stage (conv_bytes > 0, set by the
    // convolution's run when its geometry allows).
    if constexpr (BMd == B_NK && AM == A_MATRIX) {
        if (fast && a.K % kSK == 0 && stream_offsets_fit(a, EPI == EPI_CLAMP_I32 ? 4 : 1)) {
            launch_stream<EPI, PK>(a, stream);
            check_launch(where);
            return;
        }
    }
    if constexpr (BMd == B_NK && AM == A_CONV_CL && EPI == EPI_REQUANT_I8 &&
                  (PK == PK_NONE || PK == PK_B)) {
        HaloPlan hp;
        if (fast && halo_plan(a, PK == PK_B, hp)) {
            hipLaunchKernelGGL(conv_halo_kernel<PK>, dim3(8 * hp.per_xcd), dim3(kStreamThreads),
                               0, stream, a, hp);
            check_launch(where);
            return;
        }
    }
    if constexpr (BMd == B_NK && AM == A_CONV_CL && EPI == EPI_REQUANT_I8) {
        if (fast && a.conv_bytes > 0 && a.cv.ICg % kSK == 0 && stream_offsets_fit(a, 1)) {
            launch_stream<EPI, PK, true>(a, stream);
            check_launch(where);
            return;
        }
    }
    if constexpr (AM == A_MATRIX && BMd == B_KN && EPI == EPI_CLAMP_I32 && PK == PK_NONE) {
        if (fast && a.d_row0 == 0 && launch_small_clamp(a, stream)) {
            check_launch(where);
            return;
        }
    }
    if (fast) {
        const int tiles_n = (a.N + kBN - 1) / kBN;
        const long long tiles_m128 = (a.M + 127) / 128;
        // Use 64-row tiles when 128-row tiles would leave most of the 256 CUs idle.
        if (tiles_m128 * tiles_n >= 256) {
            const long long blocks = tiles_m128 * tiles_n;
            TQT_REQUIRE(blocks < (1ll << 31), "grid too large");
            hipLaunchKernelGGL((int8_mfma_kernel<128, AM, BMd, EPI, PK>), dim3(blocks), dim3(kThreads),
                               0, stream, a);
        } else {
            const long long blocks = ((a.M + 63) / 64) * static_cast<long long>(tiles_n);
            TQT_REQUIRE(blocks < (1ll << 31), "grid too large");
            hipLaunchKernelGGL((int8_mfma_kernel<64, AM, BMd, EPI, PK>), dim3(blocks), dim3(kThreads),
                               0, stream, a);
        }
    } else {
        const long long total = static_cast<long long>(a.M) * a.N;
        const long long blocks = (total + 255) / 256;
        TQT_REQUIRE(blocks < (1ll << 31), "grid too large");
        hipLaunchKernelGGL((int8_generic_kernel<AM, BMd, EPI, PK>), dim3(blocks), dim3(256), 0, stream,
                           a);
    }
    check_launch(where);
}

Int8Args base_args(size_t m, size_t n, size_t k)
{
    TQT_REQUIRE(m < (1u << 31) && n < (1u << 31) && k < (1u << 31), "dimension exceeds 2^31-1");
    Int8Args a = {};
    a.M = static_cast<int>(m);
    a.N = static_cast<int>(n);
    a.K = static_cast<int>(k);
    return a;
}


// Shared body of the igemmcl runs: fills the arguments from the conv geometry and launches.
// `packed`: the weights are in the packed layout (k_idx_b applies the tail rule).
void igemm_run(size_t m, size_t n, const void *input, size_t group_idx, size_t m_idx,
               const void *B, size_t ldb, size_t k_idx_b, void *D, size_t ldd, const void *bias,
               int8_t clamp_min, int8_t clamp_max, const tqt_conv_params *conv_params,
               const struct tqt_qai8_qai8_qsi8cx_params *quant_params, bool packed,
               hipStream_t stream, const char *where)
{
    if (!conv_params || !quant_params) {
        return;  // reference …igemmcl…cpp:206-208
    }
    if (m == 0 || n == 0) {
        return;
    }
    const tqt_conv_params &p = *conv_params;
    TQT_REQUIRE(p.groups >= 1 && p.input_channel % p.groups == 0, "input_channel % groups != 0");
    TQT_REQUIRE(quant_params->scale_b != nullptr, "quant_params->scale_b == NULL");
    TQT_REQUIRE(input != nullptr && B != nullptr && D != nullptr, "NULL tensor pointer");
    const size_t icg = p.input_channel / p.groups;
    const size_t kfull = p.kernel_shape[0] * p.kernel_shape[1] * p.kernel_shape[2] * icg;
    for (int i = 0; i < 3; ++i) {
        TQT_REQUIRE(p.input_shape[i] < (1u << 30) && p.output_shape[i] < (1u << 30) &&
                        p.kernel_shape[i] < (1u << 15) && p.stride[i] < (1u << 15) &&
                        p.dilation[i] < (1u << 15) && p.pad[i] < (1u << 15),
                    "conv geometry out of range");
    }
    TQT_REQUIRE(p.input_channel < (1u << 30), "input_channel out of range");
    Int8Args a = base_args(m, n, kfull);
    a.A = static_cast<const int8_t *>(input) + group_idx * icg;
    a.B = static_cast<const int8_t *>(B);
    a.ldb = static_cast<long long>(ldb);
    a.D = D;
    a.ldd = static_cast<long long>(ldd);
    a.d_row0 = static_cast<long long>(m_idx);
    a.p0 = static_cast<long long>(m_idx);
    a.bias = static_cast<const int32_t *>(bias);
    a.cmin = clamp_min;
    a.cmax = clamp_max;
    a.scale_a = quant_params->scale_a;
    a.scale_b = quant_params->scale_b;
    a.quant_channel_b = quant_params->quant_channel_b;
    a.scale_d = quant_params->scale_d;
    a.zp_d = quant_params->zero_point_d;
    ConvGeom &g = a.cv;
    g.ID = static_cast<int>(p.input_shape[0]);
    g.IH = static_cast<int>(p.input_shape[1]);
    g.IW = static_cast<int>(p.input_shape[2]);
    g.OH = static_cast<int>(p.output_shape[1]);
    g.OW = static_cast<int>(p.output_shape[2]);
    g.KD = static_cast<int>(p.kernel_shape[0]);
    g.KH = static_cast<int>(p.kernel_shape[1]);
    g.KW = static_cast<int>(p.kernel_shape[2]);
    g.SD = static_cast<int>(p.stride[0]);
    g.SH = static_cast<int>(p.stride[1]);
    g.SW = static_cast<int>(p.stride[2]);
    g.DD = static_cast<int>(p.dilation[0]);
    g.DH = static_cast<int>(p.dilation[1]);
    g.DW = static_cast<int>(p.dilation[2]);
    g.PD = static_cast<int>(p.pad[0]);
    g.PH = static_cast<int>(p.pad[1]);
    g.PW = static_cast<int>(p.pad[2]);
    g.IC = static_cast<int>(p.input_channel);
    g.ICg = static_cast<int>(icg);
    TQT_REQUIRE(g.OH > 0 && g.OW > 0 && icg > 0, "empty conv geometry");
    // fast path: 16-byte channel runs, a tap table that fits LDS, tap extents that pack into
    // 10 bits each, and input offsets that fit 31 bits
    const size_t in_bytes = p.input_shape[0] * p.input_shape[1] * p.input_shape[2] *
                            static_cast<size_t>(p.input_channel);
    // streaming path: the input from the group's base must fit the buffer resource's 31-bit
    // offsets
    a.conv_bytes = (in_bytes < (1ull << 31) && m_idx + m < (1ull << 31))
                       ? static_cast<int>(in_bytes - group_idx * icg)
                       : 0;
    const bool geo_fast = (icg % 16 == 0) && (p.input_channel % 16 == 0) && aligned16(a.A) &&
                          aligned16(B) && kfull / 16 <= kConvMaxChunks &&
                          (p.kernel_shape[0] - 1) * p.dilation[0] < 1024 &&
                          (p.kernel_shape[1] - 1) * p.dilation[1] < 1024 &&
                          (p.kernel_shape[2] - 1) * p.dilation[2] < 1024 && in_bytes < (1ull << 31);
    if (packed) {
        TQT_REQUIRE(ldb >= kfull, "ldb < k");
        a.pb = make_pack(kPackI8NStep, kPackI8Chunk, n, ldb, kfull, k_idx_b);
        launch_int8<A_CONV_CL, B_NK, EPI_REQUANT_I8, PK_B>(
            a, geo_fast && kfull % kPackI8Chunk == 0 && kfull < (1u << 24) && k_idx_b % 16 == 0,
            stream, where);
    } else {
        launch_int8<A_CONV_CL, B_NK, EPI_REQUANT_I8>(a, geo_fast && ldb % 16 == 0, stream, where);
    }
}

// Requantization parameters of the qai8 x qsi8cx kernels.
void set_requant(Int8Args &a, const void *bias, int8_t clamp_min, int8_t clamp_max,
                 const struct tqt_qai8_qai8_qsi8cx_params *params)
{
    a.bias = static_cast<const int32_t *>(bias);
    a.cmin = clamp_min;
    a.cmax = clamp_max;
    a.scale_a = params->scale_a;
    a.scale_b = params->scale_b;
    a.quant_channel_b = params->quant_channel_b;
    a.scale_d = params->scale_d;
    a.zp_d = params->zero_point_d;
}

// Shared body of the packed int8 GEMM runs: A packed when a_packed (else row-major with lda),
// B always packed; k_idx_a / k_idx_b apply the packers' tail rule.
template <int EPI>
void packed_gemm_run(size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a,
                     bool a_packed, const void *B, size_t ldb, size_t k_idx_b, const void *C,
                     size_t ldc, void *D, size_t ldd, Int8Args a, hipStream_t stream,
                     const char *where)
{
    TQT_REQUIRE(A != nullptr || k == 0, "A == NULL");
    TQT_REQUIRE(B != nullptr || k == 0, "B == NULL");
    TQT_REQUIRE(D != nullptr, "D == NULL");
    TQT_REQUIRE(ldb >= k && lda >= k, "lda or ldb < k");
    a.A = static_cast<const int8_t *>(A);
    a.lda = static_cast<long long>(lda);
    a.B = static_cast<const int8_t *>(B);
    a.ldb = static_cast<long long>(ldb);
    a.C = static_cast<const int32_t *>(C);
    a.ldc = static_cast<long long>(ldc);
    a.D = D;
    a.ldd = static_cast<long long>(ldd);
    a.pa = make_pack(a_packed ? kPackI8MStep : 0, kPackI8Chunk, m, lda, k,
                     a_packed ? k_idx_a : 0);
    a.pb = make_pack(kPackI8NStep, kPackI8Chunk, n, ldb, k, k_idx_b);
    // fast paths: whole chunks, every 16-byte load aligned, packed k offsets within 24 bits
    const bool fast = (k % kPackI8Chunk == 0) && k < (1u << 24) && aligned16(A) && aligned16(B) &&
                      (k_idx_b % 16 == 0) && (a_packed ? k_idx_a % 16 == 0 : lda % 16 == 0);
    if (a_packed) {
        launch_int8<A_MATRIX, B_NK, EPI, PK_AB>(a, fast, stream, where);
    } else {
        launch_int8<A_MATRIX, B_NK, EPI, PK_B>(a, fast, stream, where);
    }
}

// Shared body of the qai8dx x qsi8cx runs (f32 / f16 D, plain or packed A and B). C is not an
// input: the reference ignores it (…qai8dx_qsi8cxt_4x1vl_rvv.cpp TQT_UNUSED(C)).
template <int EPI>
void dyn_run(size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a,
             const void *B, size_t ldb, size_t k_idx_b, void *D, size_t ldd, const void *bias,
             float clamp_min, float clamp_max, const struct tqt_qai8dxp_qsi8cxp_params *params,
             bool packed, hipStream_t stream, const char *where)
{
    if (!params) {
        return;  // reference …qai8dx_qsi8cxt_4x1vl_rvv.cpp run: if (!params) return
    }
    if (m == 0 || n == 0) {
        return;
    }
    TQT_REQUIRE(params->scale_a && params->zero_point_a && params->scale_b,
                "params arrays must be non-NULL");
    Int8Args a = base_args(m, n, k);
    a.scale_b = params->scale_b;
    a.dyn_sa = params->scale_a;
    a.dyn_za = params->zero_point_a;
    a.fbias = bias;
    a.fcmin = clamp_min;
    a.fcmax = clamp_max;
    if (packed) {
        packed_gemm_run<EPI>(m, n, k, A, lda, k_idx_a, true, B, ldb, k_idx_b, nullptr, 0, D, ldd,
                             a, stream, where);
        return;
    }
    TQT_REQUIRE(A != nullptr || k == 0, "A == NULL");
    TQT_REQUIRE(B != nullptr || k == 0, "B == NULL");
    TQT_REQUIRE(D != nullptr, "D == NULL");
    a.A = static_cast<const int8_t *>(A);
    a.lda = static_cast<long long>(lda);
    a.B = static_cast<const int8_t *>(B);
    a.ldb = static_cast<long long>(ldb);
    a.D = D;
    a.ldd = static_cast<long long>(ldd);
    const bool fast = (k % 16 == 0) && (lda % 16 == 0) && (ldb % 16 == 0) && aligned16(A) &&
                      aligned16(B);
    launch_int8<A_MATRIX, B_NK, EPI>(a, fast, stream, where);
}

// Requantization fields of the mx1bias types: the per-row scale array (weights, A) takes the
// place of the per-column one, the activation's scalar scale that of scale_a, so that
// column_multiplier_dev computes scale_a[i] * scale_b / scale_d (reference
// …mx1bias…qsi8dx_qai8_4x1vl_rvv.cpp run: tqt_quantize_multiplier per row, shift = -shift - 1).
void set_mx1bias(Int8Args &a, const void *bias, int8_t clamp_min, int8_t clamp_max,
                 const struct tqt_qai8_qsi8dx_qai8_params *p)
{
    TQT_REQUIRE(p->scale_a != nullptr, "params->scale_a == NULL");
    a.bias = static_cast<const int32_t *>(bias);
    a.cmin = clamp_min;
    a.cmax = clamp_max;
    a.scale_a = p->scale_b;
    a.scale_b = p->scale_a;
    a.quant_channel_b = p->quant_channel_a;
    a.scale_d = p->scale_d;
    a.zp_d = p->zero_point_d;
}

// Shared body of the igemmcf runs: output channels m (rows of the weights) times output pixels
// [n_idx, n_idx + n) of the channel-first im2col of group group_idx, gathered from the NCDHW
// input; D rows at D + i * ldd + n_idx. `packed`: the weights are in the packed layout.
void igemmcf_run(size_t m, size_t n, const void *input, size_t group_idx, size_t n_idx,
                 const void *A, size_t lda, size_t k_idx_a, void *D, size_t ldd, const void *bias,
                 int8_t clamp_min, int8_t clamp_max, const tqt_conv_params *conv_params,
                 const struct tqt_qai8_qsi8dx_qai8_params *quant_params, bool packed,
                 hipStream_t stream, const char *where)
{
    if (!conv_params || !quant_params) {
        return;  // reference …igemmcf…qsi8dx_qai8_1vlx4_rvv.cpp run: !conv_params || !params
    }
    if (m == 0 || n == 0) {
        return;
    }
    const tqt_conv_params &p = *conv_params;
    TQT_REQUIRE(p.groups >= 1 && p.input_channel % p.groups == 0, "input_channel % groups != 0");
    TQT_REQUIRE(input != nullptr && A != nullptr && D != nullptr, "NULL tensor pointer");
    for (int i = 0; i < 3; ++i) {
        TQT_REQUIRE(p.input_shape[i] < (1u << 30) && p.output_shape[i] < (1u << 30) &&
                        p.kernel_shape[i] < (1u << 15) && p.stride[i] < (1u << 15) &&
                        p.dilation[i] < (1u << 15) && p.pad[i] < (1u << 15),
                    "conv geometry out of range");
    }
    const size_t icg = p.input_channel / p.groups;
    const size_t plane = p.input_shape[0] * p.input_shape[1] * p.input_shape[2];
    const size_t kfull = p.kernel_shape[0] * p.kernel_shape[1] * p.kernel_shape[2] * icg;
    const size_t npix = p.output_shape[0] * p.output_shape[1] * p.output_shape[2];
    TQT_REQUIRE(n_idx + n <= npix, "n_idx + n exceeds the output pixels");
    Int8Args a = base_args(m, n, kfull);
    a.A = static_cast<const int8_t *>(A);
    a.lda = static_cast<long long>(lda);
    a.B = static_cast<const int8_t *>(input) + group_idx * icg * plane;
    a.D = static_cast<int8_t *>(D) + n_idx;
    a.ldd = static_cast<long long>(ldd);
    a.p0 = static_cast<long long>(n_idx);
    set_mx1bias(a, bias, clamp_min, clamp_max, quant_params);
    ConvGeom &g = a.cv;
    g.ID = static_cast<int>(p.input_shape[0]);
    g.IH = static_cast<int>(p.input_shape[1]);
    g.IW = static_cast<int>(p.input_shape[2]);
    g.OH = static_cast<int>(p.output_shape[1]);
    g.OW = static_cast<int>(p.output_shape[2]);
    g.KD = static_cast<int>(p.kernel_shape[0]);
    g.KH = static_cast<int>(p.kernel_shape[1]);
    g.KW = static_cast<int>(p.kernel_shape[2]);
    g.SD = static_cast<int>(p.stride[0]);
    g.SH = static_cast<int>(p.stride[1]);
    g.SW = static_cast<int>(p.stride[2]);
    g.DD = static_cast<int>(p.dilation[0]);
    g.DH = static_cast<int>(p.dilation[1]);
    g.DW = static_cast<int>(p.dilation[2]);
    g.PD = static_cast<int>(p.pad[0]);
    g.PH = static_cast<int>(p.pad[1]);
    g.PW = static_cast<int>(p.pad[2]);
    g.IC = static_cast<int>(p.input_channel);
    g.ICg = static_cast<int>(icg);
    TQT_REQUIRE(g.OH > 0 && g.OW > 0 && kfull > 0, "empty conv geometry");
    // fast path: whole 16-byte weight chunks (the gathered B side has no alignment needs)
    if (packed) {
        TQT_REQUIRE(lda >= kfull, "lda < k");
        a.pa = make_pack(kPackI8MStep, kPackI8Chunk, m, lda, kfull, k_idx_a);
        const bool fast = kfull % 16 == 0 && kfull < (1u << 24) && aligned16(A) &&
                          k_idx_a % 16 == 0;
        launch_int8<A_MATRIX, B_CF, EPI_REQUANT_ROW, PK_A>(a, fast, stream, where);
    } else {
        const bool fast = kfull % 16 == 0 && lda % 16 == 0 && aligned16(A);
        launch_int8<A_MATRIX, B_CF, EPI_REQUANT_ROW>(a, fast, stream, where);
    }
}

}  // namespace
}  // namespace tqt

using namespace tqt;

// =============================================================================================
// gemm_clamp_i32_i8_i8 (reference …/gemm_clamp_i32_i8_i8_4x1vl_rvv.cpp:25-146)
// =============================================================================================
extern "C" {

// Steps of a non-packed type set only a caller's tile stride and the getters' alignment check
// (the run accepts any m and n), so they are launch-sized: one step fills the GPU, and a caller
// that walks m_step x n_step tiles the reference's way (test/common/gemm_test_runner.h:314-340)
// makes one launch where 128 x 128 tiles took 128 synchronous calls (measured 3.0 ms against
// 17.6 us for one W8A8 M512 call).
static const size_t kClampMStep = 512;
static const size_t kClampNStep = 4096;

size_t tqt_get_m_step_gemm_clamp_i32_i8_i8_mfma_gfx950(void)
{
    return kClampMStep;
}
size_t tqt_get_n_step_gemm_clamp_i32_i8_i8_mfma_gfx950(void)
{
    return kClampNStep;
}
size_t tqt_get_a_offset_gemm_clamp_i32_i8_i8_mfma_gfx950(size_t m_idx, size_t k_idx, size_t lda)
{
    TQT_REQUIRE(m_idx % kClampMStep == 0, "m_idx % m_step == 0");
    return (m_idx * lda + k_idx) * sizeof(int8_t);
}
size_t tqt_get_b_offset_gemm_clamp_i32_i8_i8_mfma_gfx950(size_t n_idx, size_t k_idx, size_t ldb)
{
    TQT_REQUIRE(n_idx % kClampNStep == 0, "n_idx % n_step == 0");
    return (k_idx * ldb + n_idx) * sizeof(int8_t);
}
size_t tqt_get_c_offset_gemm_clamp_i32_i8_i8_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldc)
{
    TQT_REQUIRE(m_idx % kClampMStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kClampNStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldc + n_idx) * sizeof(int32_t);
}
size_t tqt_get_d_offset_gemm_clamp_i32_i8_i8_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldd)
{
    TQT_REQUIRE(m_idx % kClampMStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kClampNStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldd + n_idx) * sizeof(int32_t);
}
size_t tqt_get_d_size_gemm_clamp_i32_i8_i8_mfma_gfx950(size_t m, size_t n)
{
    return m * n * sizeof(int32_t);
}

void tqt_run_gemm_clamp_i32_i8_i8_mfma_gfx950_async(size_t m, size_t n, size_t k, const void *A,
                                                    size_t lda, size_t k_idx_a, const void *B,
                                                    size_t ldb, size_t k_idx_b, const void *C,
                                                    size_t ldc, void *D, size_t ldd,
                                                    int32_t clamp_min, int32_t clamp_max,
                                                    void *stream)
{
    (void)k_idx_a;
    (void)k_idx_b;
    if (m == 0 || n == 0) {
        return;
    }
    TQT_REQUIRE(A != nullptr || k == 0, "A == NULL");
    TQT_REQUIRE(B != nullptr || k == 0, "B == NULL");
    TQT_REQUIRE(D != nullptr, "D == NULL");
    Int8Args a = base_args(m, n, k);
    a.A = static_cast<const int8_t *>(A);
    a.lda = static_cast<long long>(lda);
    a.B = static_cast<const int8_t *>(B);
    a.ldb = static_cast<long long>(ldb);
    a.C = static_cast<const int32_t *>(C);
    a.ldc = static_cast<long long>(ldc);
    a.D = D;
    a.ldd = static_cast<long long>(ldd);
    a.cmin = clamp_min;
    a.cmax = clamp_max;
    const bool fast = (k % 16 == 0) && (lda % 16 == 0) && (ldb % 16 == 0) && aligned16(A) &&
                      aligned16(B);
    launch_int8<A_MATRIX, B_KN, EPI_CLAMP_I32>(a, fast, as_stream(stream),
                                                "tqt_run_gemm_clamp_i32_i8_i8_mfma_gfx950");
}

void tqt_run_gemm_clamp_i32_i8_i8_mfma_gfx950(size_t m, size_t n, size_t k, const void *A,
                                              size_t lda, size_t k_idx_a, const void *B,
                                              size_t ldb, size_t k_idx_b, const void *C,
                                              size_t ldc, void *D, size_t ldd, int32_t clamp_min,
                                              int32_t clamp_max)
{
    if (m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_clamp_i32_i8_i8_mfma_gfx950_async(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C,
                                                   ldc, D, ldd, clamp_min, clamp_max, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_clamp_i32_i8_i8_mfma_gfx950");
}

// =============================================================================================
// gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt (reference …qsi8cxt_4x1vl_rvv.cpp:26-198)
// =============================================================================================

// launch-sized steps (see kClampMStep)
static const size_t kReqMStep = 512;
static const size_t kReqNStep = 4096;

size_t tqt_get_m_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(void)
{
    return kReqMStep;
}
size_t tqt_get_n_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(void)
{
    return kReqNStep;
}
size_t tqt_get_a_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t m_idx,
                                                                                    size_t k_idx,
                                                                                    size_t lda)
{
    TQT_REQUIRE(m_idx % kReqMStep == 0, "m_idx % m_step == 0");
    return (m_idx * lda + k_idx) * sizeof(int8_t);
}
size_t tqt_get_b_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t n_idx,
                                                                                    size_t k_idx,
                                                                                    size_t ldb)
{
    TQT_REQUIRE(n_idx % kReqNStep == 0, "n_idx % n_step == 0");
    return (n_idx * ldb + k_idx) * sizeof(int8_t);
}
size_t tqt_get_c_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t m_idx,
                                                                                    size_t n_idx,
                                                                                    size_t ldc)
{
    TQT_REQUIRE(m_idx % kReqMStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kReqNStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldc + n_idx) * sizeof(int32_t);
}
size_t tqt_get_bias_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t n_idx)
{
    TQT_REQUIRE(n_idx % kReqNStep == 0, "n_idx % n_step == 0");
    return n_idx * sizeof(int32_t);
}
size_t tqt_get_d_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t m_idx,
                                                                                    size_t n_idx,
                                                                                    size_t ldd)
{
    TQT_REQUIRE(m_idx % kReqMStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kReqNStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldd + n_idx) * sizeof(int8_t);
}
size_t tqt_get_d_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t m,
                                                                                  size_t n)
{
    return m * n * sizeof(int8_t);
}

void tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qai8_qsi8cx_params *params,
    void *stream)
{
    (void)k_idx_a;
    (void)k_idx_b;
    if (!params) {
        return;  // reference …qsi8cxt_4x1vl_rvv.cpp:148-150
    }
    if (m == 0 || n == 0) {
        return;
    }
    TQT_REQUIRE(params->scale_b != nullptr, "params->scale_b == NULL");
    TQT_REQUIRE(A != nullptr || k == 0, "A == NULL");
    TQT_REQUIRE(B != nullptr || k == 0, "B == NULL");
    TQT_REQUIRE(D != nullptr, "D == NULL");
    Int8Args a = base_args(m, n, k);
    a.A = static_cast<const int8_t *>(A);
    a.lda = static_cast<long long>(lda);
    a.B = static_cast<const int8_t *>(B);
    a.ldb = static_cast<long long>(ldb);
    a.C = static_cast<const int32_t *>(C);
    a.ldc = static_cast<long long>(ldc);
    a.D = D;
    a.ldd = static_cast<long long>(ldd);
    a.bias = static_cast<const int32_t *>(bias);
    a.cmin = clamp_min;
    a.cmax = clamp_max;
    a.scale_a = params->scale_a;
    a.scale_b = params->scale_b;
    a.quant_channel_b = params->quant_channel_b;
    a.scale_d = params->scale_d;
    a.zp_d = params->zero_point_d;
    const bool fast = (k % 16 == 0) && (lda % 16 == 0) && (ldb % 16 == 0) && aligned16(A) &&
                      aligned16(B);
    launch_int8<A_MATRIX, B_NK, EPI_REQUANT_I8>(
        a, fast, as_stream(stream),
        "tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qai8_qsi8cx_params *params)
{
    if (!params) {
        return;
    }
    if (m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950_async(
        m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias, clamp_min, clamp_max,
        params, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950");
}

// =============================================================================================
// igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt (reference …igemmcl…_4x1vl_rvv.cpp:26-286)
// =============================================================================================

static const size_t kConvMStep = 128;
static const size_t kConvNStep = 128;

size_t tqt_get_m_step_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(void)
{
    return kConvMStep;
}
size_t tqt_get_n_step_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(void)
{
    return kConvNStep;
}
size_t tqt_get_b_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb)
{
    TQT_REQUIRE(n_idx % kConvNStep == 0, "n_idx % n_step == 0");
    return (n_idx * ldb + k_idx) * sizeof(int8_t);
}
size_t tqt_get_c_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc)
{
    TQT_REQUIRE(n_idx % kConvNStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldc + n_idx) * sizeof(int32_t);
}
size_t tqt_get_bias_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t n_idx)
{
    TQT_REQUIRE(n_idx % kConvNStep == 0, "n_idx % n_step == 0");
    return n_idx * sizeof(int32_t);
}
size_t tqt_get_d_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd)
{
    TQT_REQUIRE(n_idx % kConvNStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldd + n_idx) * sizeof(int8_t);
}
size_t tqt_get_d_size_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t m,
                                                                                    size_t n)
{
    return m * n * sizeof(int8_t);
}

void tqt_run_igemm_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *input, size_t group_idx, size_t m_idx,
    size_t k_idx_a, const void *B, size_t ldb, size_t k_idx_b, const void *C, size_t ldc,
    void *D, size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const tqt_conv_params *conv_params, const struct tqt_qai8_qai8_qsi8cx_params *quant_params,
    void *stream)
{
    (void)k;
    (void)k_idx_a;
    (void)C;
    (void)ldc;
    igemm_run(m, n, input, group_idx, m_idx, B, ldb, k_idx_b, D, ldd, bias, clamp_min, clamp_max,
              conv_params, quant_params, false, as_stream(stream),
              "tqt_run_igemm_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950");
}

void tqt_run_igemm_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *input, size_t group_idx, size_t m_idx,
    size_t k_idx_a, const void *B, size_t ldb, size_t k_idx_b, const void *C, size_t ldc,
    void *D, size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const tqt_conv_params *conv_params, const struct tqt_qai8_qai8_qsi8cx_params *quant_params)
{
    if (!conv_params || !quant_params) {
        return;
    }
    if (m == 0 || n == 0) {
        return;
    }
    tqt_run_igemm_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950_async(
        m, n, k, input, group_idx, m_idx, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias,
        clamp_min, clamp_max, conv_params, quant_params, nullptr);
    finish_sync(nullptr,
                "tqt_run_igemm_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950");
}

// =============================================================================================
// Packed int8 runs (geometry getters and packers: packing.hip). The reference runs walk
// m_step x n_step tiles of panel pointers (…gemm_clamp_i32_i8p_i8p_4x1vl_rvv.cpp,
// …qai8_qai8_qsi8cxp…cpp, …qai8_qai8p_qsi8cxp…cpp, igemmcl…qsi8cxp…cpp:202-300); here one
// launch covers the problem and each row finds its panel. Panel 0 is never shifted by k_idx
// (the packers' rule; the reference's runs would read before the buffer for n < n_step).
// =============================================================================================

void tqt_run_gemm_clamp_i32_i8p_i8p_mfma_gfx950_async(size_t m, size_t n, size_t k,
                                                      const void *A_packed, size_t lda,
                                                      size_t k_idx_a, const void *B_packed,
                                                      size_t ldb, size_t k_idx_b, const void *C,
                                                      size_t ldc, void *D, size_t ldd,
                                                      int32_t clamp_min, int32_t clamp_max,
                                                      void *stream)
{
    if (m == 0 || n == 0) {
        return;
    }
    Int8Args a = base_args(m, n, k);
    a.cmin = clamp_min;
    a.cmax = clamp_max;
    packed_gemm_run<EPI_CLAMP_I32>(m, n, k, A_packed, lda, k_idx_a, true, B_packed, ldb, k_idx_b,
                                   C, ldc, D, ldd, a, as_stream(stream),
                                   "tqt_run_gemm_clamp_i32_i8p_i8p_mfma_gfx950");
}

void tqt_run_gemm_clamp_i32_i8p_i8p_mfma_gfx950(size_t m, size_t n, size_t k, const void *A_packed,
                                                size_t lda, size_t k_idx_a, const void *B_packed,
                                                size_t ldb, size_t k_idx_b, const void *C,
                                                size_t ldc, void *D, size_t ldd,
                                                int32_t clamp_min, int32_t clamp_max)
{
    if (m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_clamp_i32_i8p_i8p_mfma_gfx950_async(m, n, k, A_packed, lda, k_idx_a, B_packed,
                                                     ldb, k_idx_b, C, ldc, D, ldd, clamp_min,
                                                     clamp_max, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_clamp_i32_i8p_i8p_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B_packed,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qai8_qsi8cx_params *params,
    void *stream)
{
    if (!params) {
        return;  // reference …qai8_qai8_qsi8cxp…cpp (as …qsi8cxt…cpp:148-150)
    }
    if (m == 0 || n == 0) {
        return;
    }
    TQT_REQUIRE(params->scale_b != nullptr, "params->scale_b == NULL");
    Int8Args a = base_args(m, n, k);
    set_requant(a, bias, clamp_min, clamp_max, params);
    packed_gemm_run<EPI_REQUANT_I8>(
        m, n, k, A, lda, k_idx_a, false, B_packed, ldb, k_idx_b, C, ldc, D, ldd, a,
        as_stream(stream), "tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B_packed,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qai8_qsi8cx_params *params)
{
    if (!params || m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950_async(
        m, n, k, A, lda, k_idx_a, B_packed, ldb, k_idx_b, C, ldc, D, ldd, bias, clamp_min,
        clamp_max, params, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const struct tqt_qai8_qai8_qsi8cx_params *params, void *stream)
{
    if (!params) {
        return;  // reference …qai8_qai8p_qsi8cxp…cpp (as …qsi8cxt…cpp:148-150)
    }
    if (m == 0 || n == 0) {
        return;
    }
    TQT_REQUIRE(params->scale_b != nullptr, "params->scale_b == NULL");
    Int8Args a = base_args(m, n, k);
    set_requant(a, bias, clamp_min, clamp_max, params);
    packed_gemm_run<EPI_REQUANT_I8>(
        m, n, k, A_packed, lda, k_idx_a, true, B_packed, ldb, k_idx_b, C, ldc, D, ldd, a,
        as_stream(stream), "tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const struct tqt_qai8_qai8_qsi8cx_params *params)
{
    if (!params || m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(
        m, n, k, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, C, ldc, D, ldd, bias, clamp_min,
        clamp_max, params, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950");
}

void tqt_run_igemm_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *input, size_t group_idx, size_t m_idx,
    size_t k_idx_a, const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc,
    void *D, size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const tqt_conv_params *conv_params, const struct tqt_qai8_qai8_qsi8cx_params *quant_params,
    void *stream)
{
    (void)k;
    (void)k_idx_a;
    (void)C;
    (void)ldc;
    igemm_run(m, n, input, group_idx, m_idx, B_packed, ldb, k_idx_b, D, ldd, bias, clamp_min,
              clamp_max, conv_params, quant_params, true, as_stream(stream),
              "tqt_run_igemm_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950");
}

void tqt_run_igemm_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *input, size_t group_idx, size_t m_idx,
    size_t k_idx_a, const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc,
    void *D, size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const tqt_conv_params *conv_params, const struct tqt_qai8_qai8_qsi8cx_params *quant_params)
{
    if (!conv_params || !quant_params || m == 0 || n == 0) {
        return;
    }
    tqt_run_igemm_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950_async(
        m, n, k, input, group_idx, m_idx, k_idx_a, B_packed, ldb, k_idx_b, C, ldc, D, ldd, bias,
        clamp_min, clamp_max, conv_params, quant_params, nullptr);
    finish_sync(nullptr,
                "tqt_run_igemm_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950");
}

// =============================================================================================
// gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8 (reference …/gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_4x1vl_rvv.cpp): weights A [m, k] (per-row
// scale) times activations B [k, n], int32 C (optional) and Mx1 bias, per-row requantization
// =============================================================================================
// launch-sized steps (see kClampMStep)
static const size_t kMx1MStep = 512;
static const size_t kMx1NStep = 4096;

size_t tqt_get_m_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(void)
{
    return kMx1MStep;
}
size_t tqt_get_n_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(void)
{
    return kMx1NStep;
}
size_t tqt_get_a_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m_idx, size_t k_idx, size_t lda)
{
    TQT_REQUIRE(m_idx % kMx1MStep == 0, "m_idx % m_step == 0");
    return (m_idx * lda + k_idx) * sizeof(int8_t);
}
size_t tqt_get_b_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t n_idx, size_t k_idx, size_t ldb)
{
    TQT_REQUIRE(n_idx % kMx1NStep == 0, "n_idx % n_step == 0");
    return (k_idx * ldb + n_idx) * sizeof(int8_t);
}
size_t tqt_get_c_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldc)
{
    TQT_REQUIRE(m_idx % kMx1MStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kMx1NStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldc + n_idx) * sizeof(int32_t);
}
size_t tqt_get_bias_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m_idx)
{
    TQT_REQUIRE(m_idx % kMx1MStep == 0, "m_idx % m_step == 0");
    return m_idx * sizeof(int32_t);
}
size_t tqt_get_d_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldd)
{
    TQT_REQUIRE(m_idx % kMx1MStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kMx1NStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldd + n_idx) * sizeof(int8_t);
}
size_t tqt_get_d_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m, size_t n)
{
    return m * n * sizeof(int8_t);
}

void tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qsi8dx_qai8_params *params,
    void *stream)
{
    (void)k_idx_a;
    (void)k_idx_b;
    if (!params) {
        return;  // reference …mx1bias…qsi8dx_qai8_4x1vl_rvv.cpp run: if (!params) return
    }
    if (m == 0 || n == 0) {
        return;
    }
    TQT_REQUIRE(A != nullptr || k == 0, "A == NULL");
    TQT_REQUIRE(B != nullptr || k == 0, "B == NULL");
    TQT_REQUIRE(D != nullptr, "D == NULL");
    Int8Args a = base_args(m, n, k);
    a.A = static_cast<const int8_t *>(A);
    a.lda = static_cast<long long>(lda);
    a.B = static_cast<const int8_t *>(B);
    a.ldb = static_cast<long long>(ldb);
    a.C = static_cast<const int32_t *>(C);
    a.ldc = static_cast<long long>(ldc);
    a.D = D;
    a.ldd = static_cast<long long>(ldd);
    set_mx1bias(a, bias, clamp_min, clamp_max, params);
    const bool fast = (k % 16 == 0) && (lda % 16 == 0) && (ldb % 16 == 0) && aligned16(A) &&
                      aligned16(B);
    launch_int8<A_MATRIX, B_KN, EPI_REQUANT_ROW>(a, fast, as_stream(stream),
                                                 "tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950");
}

void tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qsi8dx_qai8_params *params)
{
    if (!params || m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950_async(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd,
                                    bias, clamp_min, clamp_max, params, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950");
}

// =============================================================================================
// gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p (reference …/gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_4x1vl_rvv.cpp): the packed layout and packers of
// gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp (weights are the packed A rows, activations the packed B rows)
// =============================================================================================
size_t tqt_get_m_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(void)
{
    return kPackI8MStep;
}
size_t tqt_get_n_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(void)
{
    return kPackI8NStep;
}
size_t tqt_get_a_packed_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t m_idx, size_t k_idx, size_t lda,
                                                  size_t actual_m)
{
    return tqt_get_a_packed_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(m_idx, k_idx, lda, actual_m);
}
size_t tqt_get_b_packed_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t n_idx, size_t k_idx, size_t ldb,
                                                  size_t actual_n)
{
    return tqt_get_b_packed_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(n_idx, k_idx, ldb, actual_n);
}
size_t tqt_get_c_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldc)
{
    TQT_REQUIRE(m_idx % kPackI8MStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kPackI8NStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldc + n_idx) * sizeof(int32_t);
}
size_t tqt_get_bias_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t m_idx)
{
    TQT_REQUIRE(m_idx % kPackI8MStep == 0, "m_idx % m_step == 0");
    return m_idx * sizeof(int32_t);
}
size_t tqt_get_d_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldd)
{
    TQT_REQUIRE(m_idx % kPackI8MStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kPackI8NStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldd + n_idx) * sizeof(int8_t);
}
size_t tqt_get_d_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t m, size_t n)
{
    return m * n * sizeof(int8_t);
}
size_t tqt_get_a_packed_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t m, size_t k)
{
    return m * k;
}
size_t tqt_get_b_packed_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t n, size_t k)
{
    return n * k;
}
#define TQT_MX1_PACKER(ACTION, R)                                                                  \
    void tqt_##ACTION##_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950_async(                            \
        size_t R, size_t k, size_t ld, size_t ld_packed, size_t k_idx, const void *src, void *dst, \
        void *stream)                                                                              \
    {                                                                                              \
        tqt_##ACTION##_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(R, k, ld, ld_packed, k_idx,    \
                                                                       src, dst, stream);          \
    }                                                                                              \
    void tqt_##ACTION##_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t R, size_t k, size_t ld,    \
                                                                     size_t ld_packed,             \
                                                                     size_t k_idx,                 \
                                                                     const void *src, void *dst)   \
    {                                                                                              \
        tqt_##ACTION##_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(R, k, ld, ld_packed, k_idx, src,     \
                                                                 dst);                             \
    }
TQT_MX1_PACKER(run_a_pack, m)
TQT_MX1_PACKER(run_b_pack, n)
TQT_MX1_PACKER(run_bt_pack, n)
#undef TQT_MX1_PACKER

void tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const struct tqt_qai8_qsi8dx_qai8_params *params, void *stream)
{
    if (!params) {
        return;
    }
    if (m == 0 || n == 0) {
        return;
    }
    Int8Args a = base_args(m, n, k);
    set_mx1bias(a, bias, clamp_min, clamp_max, params);
    packed_gemm_run<EPI_REQUANT_ROW>(m, n, k, A_packed, lda, k_idx_a, true, B_packed, ldb,
                                     k_idx_b, C, ldc, D, ldd, a, as_stream(stream),
                                     "tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950");
}

void tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const struct tqt_qai8_qsi8dx_qai8_params *params)
{
    if (!params || m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950_async(m, n, k, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, C,
                                     ldc, D, ldd, bias, clamp_min, clamp_max, params, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950");
}

// =============================================================================================
// igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8 (reference …/igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_1vlx4_rvv.cpp) and its packed-weights
// sibling igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8: the mx1bias GEMM with B gathered from the
// channel-first input
// =============================================================================================
size_t tqt_get_m_step_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(void)
{
    return kMx1MStep;
}
size_t tqt_get_n_step_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(void)
{
    return kMx1NStep;
}
size_t tqt_get_a_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m_idx, size_t k_idx, size_t lda)
{
    TQT_REQUIRE(m_idx % kMx1MStep == 0, "m_idx % m_step == 0");
    return (m_idx * lda + k_idx) * sizeof(int8_t);
}
size_t tqt_get_c_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldc)
{
    TQT_REQUIRE(m_idx % kMx1MStep == 0, "m_idx % m_step == 0");
    return (m_idx * ldc + n_idx) * sizeof(int32_t);
}
size_t tqt_get_bias_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m_idx)
{
    TQT_REQUIRE(m_idx % kMx1MStep == 0, "m_idx % m_step == 0");
    return m_idx * sizeof(int32_t);
}
size_t tqt_get_d_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldd)
{
    TQT_REQUIRE(m_idx % kMx1MStep == 0, "m_idx % m_step == 0");
    return (m_idx * ldd + n_idx) * sizeof(int8_t);
}
size_t tqt_get_d_size_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m, size_t n)
{
    return m * n * sizeof(int8_t);
}

void tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *input, size_t group_idx, size_t n_idx,
    size_t k_idx_b, const void *A, size_t lda, size_t k_idx_a, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const tqt_conv_params *conv_params, const struct tqt_qai8_qsi8dx_qai8_params *quant_params,
    void *stream)
{
    (void)k;
    (void)k_idx_b;
    (void)k_idx_a;
    (void)C;
    (void)ldc;
    igemmcf_run(m, n, input, group_idx, n_idx, A, lda, 0, D, ldd, bias, clamp_min, clamp_max,
                conv_params, quant_params, false, as_stream(stream),
                "tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950");
}

void tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *input, size_t group_idx, size_t n_idx,
    size_t k_idx_b, const void *A, size_t lda, size_t k_idx_a, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const tqt_conv_params *conv_params, const struct tqt_qai8_qsi8dx_qai8_params *quant_params)
{
    if (!conv_params || !quant_params || m == 0 || n == 0) {
        return;
    }
    tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950_async(m, n, k, input, group_idx, n_idx, k_idx_b, A, lda,
                                           k_idx_a, C, ldc, D, ldd, bias, clamp_min, clamp_max,
                                           conv_params, quant_params, nullptr);
    finish_sync(nullptr, "tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950");
}

size_t tqt_get_m_step_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(void)
{
    return kPackI8MStep;
}
size_t tqt_get_n_step_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(void)
{
    return kMx1NStep;
}
size_t tqt_get_a_packed_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(size_t m_idx, size_t k_idx, size_t lda,
                                                   size_t actual_m)
{
    return tqt_get_a_packed_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(m_idx, k_idx, lda, actual_m);
}
size_t tqt_get_c_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldc)
{
    TQT_REQUIRE(m_idx % kPackI8MStep == 0, "m_idx % m_step == 0");
    return (m_idx * ldc + n_idx) * sizeof(int32_t);
}
size_t tqt_get_bias_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(size_t m_idx)
{
    TQT_REQUIRE(m_idx % kPackI8MStep == 0, "m_idx % m_step == 0");
    return m_idx * sizeof(int32_t);
}
size_t tqt_get_d_offset_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldd)
{
    TQT_REQUIRE(m_idx % kPackI8MStep == 0, "m_idx % m_step == 0");
    return (m_idx * ldd + n_idx) * sizeof(int8_t);
}
size_t tqt_get_d_size_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(size_t m, size_t n)
{
    return m * n * sizeof(int8_t);
}
size_t tqt_get_a_packed_size_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(size_t m, size_t k)
{
    return m * k;
}
void tqt_run_a_pack_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950_async(size_t m, size_t k, size_t ldw, size_t ldw_packed,
                                              size_t k_idx, const void *weight,
                                              void *weight_packed, void *stream)
{
    tqt_run_a_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(m, k, ldw, ldw_packed, k_idx, weight, weight_packed,
                                             stream);
}
void tqt_run_a_pack_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(size_t m, size_t k, size_t ldw, size_t ldw_packed,
                                        size_t k_idx, const void *weight, void *weight_packed)
{
    tqt_run_a_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(m, k, ldw, ldw_packed, k_idx, weight, weight_packed);
}

void tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *input, size_t group_idx, size_t n_idx,
    size_t k_idx_b, const void *A_packed, size_t lda, size_t k_idx_a, const void *C, size_t ldc,
    void *D, size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const tqt_conv_params *conv_params, const struct tqt_qai8_qsi8dx_qai8_params *quant_params,
    void *stream)
{
    (void)k;
    (void)k_idx_b;
    (void)C;
    (void)ldc;
    igemmcf_run(m, n, input, group_idx, n_idx, A_packed, lda, k_idx_a, D, ldd, bias, clamp_min,
                clamp_max, conv_params, quant_params, true, as_stream(stream),
                "tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950");
}

void tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *input, size_t group_idx, size_t n_idx,
    size_t k_idx_b, const void *A_packed, size_t lda, size_t k_idx_a, const void *C, size_t ldc,
    void *D, size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const tqt_conv_params *conv_params, const struct tqt_qai8_qsi8dx_qai8_params *quant_params)
{
    if (!conv_params || !quant_params || m == 0 || n == 0) {
        return;
    }
    tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950_async(m, n, k, input, group_idx, n_idx, k_idx_b, A_packed,
                                            lda, k_idx_a, C, ldc, D, ldd, bias, clamp_min,
                                            clamp_max, conv_params, quant_params, nullptr);
    finish_sync(nullptr, "tqt_run_igemm_igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8_mfma_gfx950");
}

// launch-sized steps (see kClampMStep)
static const size_t kDynMStep = 512;
static const size_t kDynNStep = 4096;

// =============================================================================================
// gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt (reference …/gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_4x1vl_rvv.cpp; kernel semantics
// tqt_kernel_gemm_qai8dx_qsi8cx_4x1vl_rvv.h)
// =============================================================================================
size_t tqt_get_m_step_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(void)
{
    return kDynMStep;
}
size_t tqt_get_n_step_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(void)
{
    return kDynNStep;
}
size_t tqt_get_a_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(size_t m_idx, size_t k_idx, size_t lda)
{
    TQT_REQUIRE(m_idx % kDynMStep == 0, "m_idx % m_step == 0");
    return (m_idx * lda + k_idx) * sizeof(int8_t);
}
size_t tqt_get_b_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(size_t n_idx, size_t k_idx, size_t ldb)
{
    TQT_REQUIRE(n_idx % kDynNStep == 0, "n_idx % n_step == 0");
    return (n_idx * ldb + k_idx) * sizeof(int8_t);
}
size_t tqt_get_c_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldc)
{
    TQT_REQUIRE(m_idx % kDynMStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kDynNStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldc + n_idx) * sizeof(float);
}
size_t tqt_get_bias_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(size_t n_idx)
{
    TQT_REQUIRE(n_idx % kDynNStep == 0, "n_idx % n_step == 0");
    return n_idx * sizeof(float);
}
size_t tqt_get_d_offset_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldd)
{
    TQT_REQUIRE(m_idx % kDynMStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kDynNStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldd + n_idx) * sizeof(float);
}
size_t tqt_get_d_size_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(size_t m, size_t n)
{
    return m * n * sizeof(float);
}

void tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    float clamp_min, float clamp_max, const struct tqt_qai8dxp_qsi8cxp_params *params,
    void *stream)
{
    (void)k_idx_a;
    (void)k_idx_b;
    (void)C;
    (void)ldc;
    dyn_run<EPI_DYN_F32>(m, n, k, A, lda, 0, B, ldb, 0, D, ldd, bias, clamp_min, clamp_max,
                         params, false, as_stream(stream),
                         "tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    float clamp_min, float clamp_max, const struct tqt_qai8dxp_qsi8cxp_params *params)
{
    if (!params || m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950_async(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd,
                                    bias, clamp_min, clamp_max, params, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt_mfma_gfx950");
}

// gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp (reference …/gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_4x1vl_rvv.cpp; geometry getters and
// packers in packing.hip)
void tqt_run_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, float clamp_min, float clamp_max,
    const struct tqt_qai8dxp_qsi8cxp_params *params, void *stream)
{
    (void)C;
    (void)ldc;
    dyn_run<EPI_DYN_F32>(m, n, k, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, D, ldd, bias,
                         clamp_min, clamp_max, params, true, as_stream(stream),
                         "tqt_run_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, float clamp_min, float clamp_max,
    const struct tqt_qai8dxp_qsi8cxp_params *params)
{
    if (!params || m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950_async(m, n, k, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, C,
                                     ldc, D, ldd, bias, clamp_min, clamp_max, params, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950");
}

// =============================================================================================
// gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt (reference …/gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_4x1vl_rvv.cpp; kernel semantics
// tqt_kernel_gemm_qai8dx_qsi8cx_4x1vl_rvv.h)
// =============================================================================================
size_t tqt_get_m_step_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950(void)
{
    return kDynMStep;
}
size_t tqt_get_n_step_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950(void)
{
    return kDynNStep;
}
size_t tqt_get_a_offset_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950(size_t m_idx, size_t k_idx, size_t lda)
{
    TQT_REQUIRE(m_idx % kDynMStep == 0, "m_idx % m_step == 0");
    return (m_idx * lda + k_idx) * sizeof(int8_t);
}
size_t tqt_get_b_offset_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950(size_t n_idx, size_t k_idx, size_t ldb)
{
    TQT_REQUIRE(n_idx % kDynNStep == 0, "n_idx % n_step == 0");
    return (n_idx * ldb + k_idx) * sizeof(int8_t);
}
size_t tqt_get_c_offset_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldc)
{
    TQT_REQUIRE(m_idx % kDynMStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kDynNStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldc + n_idx) * sizeof(float16_t);
}
size_t tqt_get_bias_offset_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950(size_t n_idx)
{
    TQT_REQUIRE(n_idx % kDynNStep == 0, "n_idx % n_step == 0");
    return n_idx * sizeof(float16_t);
}
size_t tqt_get_d_offset_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldd)
{
    TQT_REQUIRE(m_idx % kDynMStep == 0, "m_idx % m_step == 0");
    TQT_REQUIRE(n_idx % kDynNStep == 0, "n_idx % n_step == 0");
    return (m_idx * ldd + n_idx) * sizeof(float16_t);
}
size_t tqt_get_d_size_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950(size_t m, size_t n)
{
    return m * n * sizeof(float16_t);
}

void tqt_run_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    float16_t clamp_min, float16_t clamp_max, const struct tqt_qai8dxp_qsi8cxp_params *params,
    void *stream)
{
    (void)k_idx_a;
    (void)k_idx_b;
    (void)C;
    (void)ldc;
    dyn_run<EPI_DYN_F16>(m, n, k, A, lda, 0, B, ldb, 0, D, ldd, bias,
                         static_cast<float>(clamp_min), static_cast<float>(clamp_max), params,
                         false, as_stream(stream),
                         "tqt_run_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    float16_t clamp_min, float16_t clamp_max, const struct tqt_qai8dxp_qsi8cxp_params *params)
{
    if (!params || m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950_async(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd,
                                    bias, clamp_min, clamp_max, params, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt_mfma_gfx950");
}

// gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp (reference …/gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_4x1vl_rvv.cpp; geometry getters and
// packers in packing.hip)
void tqt_run_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, float16_t clamp_min, float16_t clamp_max,
    const struct tqt_qai8dxp_qsi8cxp_params *params, void *stream)
{
    (void)C;
    (void)ldc;
    dyn_run<EPI_DYN_F16>(m, n, k, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, D, ldd, bias,
                         static_cast<float>(clamp_min), static_cast<float>(clamp_max), params,
                         true, as_stream(stream),
                         "tqt_run_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950");
}

void tqt_run_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, float16_t clamp_min, float16_t clamp_max,
    const struct tqt_qai8dxp_qsi8cxp_params *params)
{
    if (!params || m == 0 || n == 0) {
        return;
    }
    tqt_run_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950_async(m, n, k, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, C,
                                     ldc, D, ldd, bias, clamp_min, clamp_max, params, nullptr);
    finish_sync(nullptr, "tqt_run_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950");
}

const char *tqt_gfx950_target(void)
{
    return "gfx950";
}

}  // extern "C"
