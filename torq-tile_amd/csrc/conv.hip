// Explicit-im2col convolution on gfx950.
//   convcl: the im2col of a channel-last (NDHWC) int8 activation into the [M, K] matrix A of the
//   W8A8 GEMM (M = OD*OH*OW output pixels, K = KD*KH*KW*IC_per_group in (kd, kh, kw, ic) order),
//   row-major or written straight into the packed layout of
//   gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp;
//   convcf: the im2col of a channel-first (NCDHW) activation into the [K, N] matrix B of the
//   mx1bias GEMM (K = IC_per_group*KD*KH*KW in (ic, kd, kh, kw) order, N = output pixels),
//   row-major or written transposed (pixel rows) into the packed B layout of
//   gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p.
// The convolution itself is that GEMM (the reference's run_conv forwards to the GEMM run, as
// here).
//
// The transform is pure byte movement, bound by HBM: one thread per 16-byte chunk of an output
// row. When the group's channel run is a whole number of 16-byte chunks (IC_per_group % 16 == 0,
// 16-byte aligned rows), a chunk lies inside one tap and moves as one 16-byte load and store;
// otherwise each byte finds its own tap. Padding taps write zeros.
#include "tqt_hip_common.hpp"
#include "tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950.h"
#include "tqt_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950.h"
#include "tqt_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950.h"
#include "tqt_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950.h"
#include "tqt_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950.h"
#include "tqt_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950.h"

namespace tqt {
namespace {

struct ConvShape
{
    int ID, IH, IW;
    int OD, OH, OW;
    int KD, KH, KW;
    int SD, SH, SW;
    int DD, DH, DW;
    int PD, PH, PW;
    int IC;   // channel stride of the input (all groups)
    int ICg;  // channels per group
    int c0;   // first channel of the group
    int M, K;
};

ConvShape conv_shape(size_t group_idx, const tqt_conv_params *p)
{
    TQT_REQUIRE(p != nullptr, "params == NULL");
    TQT_REQUIRE(p->groups >= 1 && p->input_channel % p->groups == 0,
                "input_channel % groups != 0");
    TQT_REQUIRE(group_idx < p->groups, "group_idx >= groups");
    for (int i = 0; i < 3; ++i) {
        TQT_REQUIRE(p->input_shape[i] < (1u << 30) && p->output_shape[i] < (1u << 30) &&
                        p->kernel_shape[i] < (1u << 15) && p->stride[i] < (1u << 15) &&
                        p->dilation[i] < (1u << 15) && p->pad[i] < (1u << 15),
                    "conv geometry out of range");
    }
    ConvShape g;
    g.ID = static_cast<int>(p->input_shape[0]);
    g.IH = static_cast<int>(p->input_shape[1]);
    g.IW = static_cast<int>(p->input_shape[2]);
    g.OD = static_cast<int>(p->output_shape[0]);
    g.OH = static_cast<int>(p->output_shape[1]);
    g.OW = static_cast<int>(p->output_shape[2]);
    g.KD = static_cast<int>(p->kernel_shape[0]);
    g.KH = static_cast<int>(p->kernel_shape[1]);
    g.KW = static_cast<int>(p->kernel_shape[2]);
    g.SD = static_cast<int>(p->stride[0]);
    g.SH = static_cast<int>(p->stride[1]);
    g.SW = static_cast<int>(p->stride[2]);
    g.DD = static_cast<int>(p->dilation[0]);
    g.DH = static_cast<int>(p->dilation[1]);
    g.DW = static_cast<int>(p->dilation[2]);
    g.PD = static_cast<int>(p->pad[0]);
    g.PH = static_cast<int>(p->pad[1]);
    g.PW = static_cast<int>(p->pad[2]);
    const size_t icg = p->input_channel / p->groups;
    TQT_REQUIRE(p->input_channel < (1u << 30), "input_channel out of range");
    g.IC = static_cast<int>(p->input_channel);
    g.ICg = static_cast<int>(icg);
    g.c0 = static_cast<int>(group_idx * icg);
    const size_t m = p->output_shape[0] * p->output_shape[1] * p->output_shape[2];
    const size_t k = p->kernel_shape[0] * p->kernel_shape[1] * p->kernel_shape[2] * icg;
    TQT_REQUIRE(m < (1u << 31) && k < (1u << 31), "im2col matrix too large");
    g.M = static_cast<int>(m);
    g.K = static_cast<int>(k);
    return g;
}

// Input byte offset of (output pixel p, im2col column k), or -1 for a padding tap.
__device__ __forceinline__ long long cl_src(const ConvShape &g, int od, int oh, int ow, int k)
{
    const int tap = k / g.ICg;
    const int ic = k - tap * g.ICg;
    const int kw = tap % g.KW;
    const int kh = (tap / g.KW) % g.KH;
    const int kd = tap / (g.KW * g.KH);
    const int id = od * g.SD + kd * g.DD - g.PD;
    const int ih = oh * g.SH + kh * g.DH - g.PH;
    const int iw = ow * g.SW + kw * g.DW - g.PW;
    if (id < 0 || id >= g.ID || ih < 0 || ih >= g.IH || iw < 0 || iw >= g.IW) {
        return -1;
    }
    return ((static_cast<long long>(id) * g.IH + ih) * g.IW + iw) * g.IC + g.c0 + ic;
}

// Input byte offset of channel-first im2col element (k, output pixel (od, oh, ow)), or -1 for a
// padding tap: k = (ic, kd, kh, kw) of the group, the input plane of channel c0 + ic.
__device__ __forceinline__ long long cf_src(const ConvShape &g, int od, int oh, int ow, int k)
{
    const int khw = g.KH * g.KW;
    const int kdhw = g.KD * khw;
    const int ic = k / kdhw;
    int r = k - ic * kdhw;
    const int kd = r / khw;
    r -= kd * khw;
    const int kh = r / g.KW;
    const int kw = r - kh * g.KW;
    const int id = od * g.SD + kd * g.DD - g.PD;
    const int ih = oh * g.SH + kh * g.DH - g.PH;
    const int iw = ow * g.SW + kw * g.DW - g.PW;
    if (id < 0 || id >= g.ID || ih < 0 || ih >= g.IH || iw < 0 || iw >= g.IW) {
        return -1;
    }
    return static_cast<long long>(g.c0 + ic) * g.ID * g.IH * g.IW +
           (static_cast<long long>(id) * g.IH + ih) * g.IW + iw;
}

// One thread per 16-byte chunk (p, c) of the [M, K] pixel-row matrix: the channel-last im2col
// (kCF false) or the transposed channel-first im2col (kCF true: row p holds (ic, kd, kh, kw));
// kPacked writes the chunk at its place in the packed layout `pd`, else at p * K + 16 c. kVec
// (channel-last only): the chunk is one tap's 16 channels and both ends are 16-byte aligned.
template <bool kCF, bool kPacked, bool kVec>
__global__ __launch_bounds__(256) void im2col_rows_kernel(ConvShape g, const int8_t *in,
                                                          int8_t *out, PackDesc pd, long long nchunks,
                                                          int row0)
{
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= nchunks) {
        return;
    }
    const int cpr = (g.K + 15) / 16;
    const int pr = static_cast<int>(idx / cpr);
    const int p = row0 + pr;
    const int c = static_cast<int>(idx - static_cast<long long>(pr) * cpr);
    const int k0 = 16 * c;
    const int cw = min(16, g.K - k0);
    const int ow = p % g.OW;
    const int oh = (p / g.OW) % g.OH;
    const int od = p / (g.OW * g.OH);
    long long dst;
    if constexpr (kPacked) {
        dst = pack_row_byte(pack_row_info(pd, p), k0);  // the chunk's cw bytes are contiguous
    } else {
        dst = static_cast<long long>(p) * g.K + k0;
    }
    if constexpr (kVec && !kCF) {
        const long long s = cl_src(g, od, oh, ow, k0);
        const i32x4 v = s >= 0 ? *reinterpret_cast<const i32x4 *>(in + s) : i32x4{0, 0, 0, 0};
        *reinterpret_cast<i32x4 *>(out + dst) = v;
    } else {
        for (int b = 0; b < cw; ++b) {
            const long long s = kCF ? cf_src(g, od, oh, ow, k0 + b) : cl_src(g, od, oh, ow, k0 + b);
            out[dst + b] = s >= 0 ? in[s] : static_cast<int8_t>(0);
        }
    }
}

// Channel-first im2col into row-major [K, N]: one thread per (row k, 16 consecutive pixels).
__global__ __launch_bounds__(256) void im2col_cf_kernel(ConvShape g, const int8_t *in, int8_t *out,
                                                        long long nchunks)
{
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= nchunks) {
        return;
    }
    const int cpr = (g.M + 15) / 16;  // g.M = output pixels
    const int k = static_cast<int>(idx / cpr);
    const int p0 = 16 * static_cast<int>(idx - static_cast<long long>(k) * cpr);
    const int cw = min(16, g.M - p0);
    int ow = p0 % g.OW;
    int oh = (p0 / g.OW) % g.OH;
    int od = p0 / (g.OW * g.OH);
    int8_t *o = out + static_cast<long long>(k) * g.M + p0;
    for (int b = 0; b < cw; ++b) {
        const long long s = cf_src(g, od, oh, ow, k);
        o[b] = s >= 0 ? in[s] : static_cast<int8_t>(0);
        if (++ow == g.OW) {
            ow = 0;
            if (++oh == g.OH) {
                oh = 0;
                ++od;
            }
        }
    }
}

// Pixel-row im2col of one group (channel-last, or the transposed channel-first one when cf) into
// row-major [M, K] (packed == false) or into the packed layout with leading dimension
// lda_packed, panel height `step` and the packers' k_idx tail rule (packed == true).
void im2col_rows_run(size_t group_idx, const void *activation, void *out, bool cf, bool packed,
                     size_t step, size_t lda_packed, size_t k_idx, const tqt_conv_params *params,
                     hipStream_t s, const char *where)
{
    const ConvShape g = conv_shape(group_idx, params);
    if (g.M == 0 || g.K == 0) {
        return;
    }
    TQT_REQUIRE(activation != nullptr && out != nullptr, "NULL tensor pointer");
    PackDesc pd = {};
    bool vec = !cf && g.ICg % 16 == 0 && g.IC % 16 == 0 && aligned16(activation) &&
               aligned16(out);
    if (packed) {
        TQT_REQUIRE(lda_packed >= static_cast<size_t>(g.K), "ld_packed < k");
        pd = make_pack(step, kPackI8Chunk, static_cast<size_t>(g.M), lda_packed,
                       static_cast<size_t>(g.K), k_idx);
        vec = vec && lda_packed % 16 == 0 && k_idx % 16 == 0;
    }
    const int8_t *in = static_cast<const int8_t *>(activation);
    int8_t *o = static_cast<int8_t *>(out);
    // a narrow last panel moved back onto the previous one is written after it, as the
    // reference's panel-by-panel packing leaves it
    const int split = packed ? tail_panel_start(pd) : g.M;
    for (int part = 0; part < 2; ++part) {
        const int row0 = part == 0 ? 0 : split;
        const int rows = part == 0 ? split : g.M - split;
        if (rows <= 0) {
            continue;
        }
        const long long nchunks = static_cast<long long>(rows) * ((g.K + 15) / 16);
        const long long blocks = (nchunks + 255) / 256;
        TQT_REQUIRE(blocks < (1ll << 31), "grid too large");
        const dim3 grid(static_cast<unsigned>(blocks));
        if (cf) {
            if (packed) {
                hipLaunchKernelGGL((im2col_rows_kernel<true, true, false>), grid, dim3(256), 0, s,
                                   g, in, o, pd, nchunks, row0);
            } else {
                hipLaunchKernelGGL((im2col_rows_kernel<true, false, false>), grid, dim3(256), 0,
                                   s, g, in, o, pd, nchunks, row0);
            }
        } else if (packed) {
            if (vec) {
                hipLaunchKernelGGL((im2col_rows_kernel<false, true, true>), grid, dim3(256), 0, s,
                                   g, in, o, pd, nchunks, row0);
            } else {
                hipLaunchKernelGGL((im2col_rows_kernel<false, true, false>), grid, dim3(256), 0,
                                   s, g, in, o, pd, nchunks, row0);
            }
        } else {
            if (vec) {
                hipLaunchKernelGGL((im2col_rows_kernel<false, false, true>), grid, dim3(256), 0,
                                   s, g, in, o, pd, nchunks, row0);
            } else {
                hipLaunchKernelGGL((im2col_rows_kernel<false, false, false>), grid, dim3(256), 0,
                                   s, g, in, o, pd, nchunks, row0);
            }
        }
    }
    check_launch(where);
}

// Channel-first im2col of one group into row-major [K, N].
void im2col_cf_run(size_t group_idx, const void *activation, void *out,
                   const tqt_conv_params *params, hipStream_t s, const char *where)
{
    const ConvShape g = conv_shape(group_idx, params);
    if (g.M == 0 || g.K == 0) {
        return;
    }
    TQT_REQUIRE(activation != nullptr && out != nullptr, "NULL tensor pointer");
    const long long nchunks = static_cast<long long>(g.K) * ((g.M + 15) / 16);
    const long long blocks = (nchunks + 255) / 256;
    TQT_REQUIRE(blocks < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(im2col_cf_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, g,
                       static_cast<const int8_t *>(activation), static_cast<int8_t *>(out),
                       nchunks);
    check_launch(where);
}

}  // namespace
}  // namespace tqt

using namespace tqt;

extern "C" {

// =============================================================================================
// convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt (reference …qai8_qai8_qsi8cxt_4x1vl_rvv.cpp):
// im2col + gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt
// =============================================================================================
size_t tqt_get_m_step_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(void)
{
    return tqt_get_m_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950();
}
size_t tqt_get_n_step_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(void)
{
    return tqt_get_n_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950();
}
size_t tqt_get_b_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t n_idx,
                                                                                      size_t k_idx,
                                                                                      size_t ldb)
{
    return tqt_get_b_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(n_idx, k_idx,
                                                                                        ldb);
}
size_t tqt_get_c_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t m_idx,
                                                                                      size_t n_idx,
                                                                                      size_t ldc)
{
    return tqt_get_c_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(m_idx, n_idx,
                                                                                        ldc);
}
size_t tqt_get_bias_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t n_idx)
{
    return tqt_get_bias_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(n_idx);
}
size_t tqt_get_d_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t m_idx,
                                                                                      size_t n_idx,
                                                                                      size_t ldd)
{
    return tqt_get_d_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(m_idx, n_idx,
                                                                                        ldd);
}
size_t tqt_get_d_size_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(size_t m,
                                                                                    size_t n)
{
    return tqt_get_d_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(m, n);
}
size_t tqt_get_a_im2col_size_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m, size_t k)
{
    return m * k * sizeof(int8_t);
}
size_t tqt_get_a_im2col_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m_idx, size_t k_idx, size_t lda_im2col)
{
    return (m_idx * lda_im2col + k_idx) * sizeof(int8_t);
}

void tqt_run_im2col_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950_async(
    size_t group_idx, const void *activation, void *im2col_buf, const tqt_conv_params *params,
    void *stream)
{
    im2col_rows_run(group_idx, activation, im2col_buf, false, false, 0, 0, 0, params,
                    as_stream(stream),
                    "tqt_run_im2col_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950");
}

void tqt_run_im2col_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t group_idx, const void *activation, void *im2col_buf, const tqt_conv_params *params)
{
    tqt_run_im2col_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950_async(
        group_idx, activation, im2col_buf, params, nullptr);
    finish_sync(nullptr,
                "tqt_run_im2col_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950");
}

void tqt_run_conv_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qai8_qsi8cx_params *params,
    void *stream)
{
    tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950_async(
        m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias, clamp_min, clamp_max,
        params, stream);
}

void tqt_run_conv_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qai8_qsi8cx_params *params)
{
    tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt_mfma_gfx950(
        m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias, clamp_min, clamp_max,
        params);
}

// =============================================================================================
// convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp (reference …qai8_qai8p_qsi8cxp_4x1vl_rvv.cpp):
// im2col fused with the A packing of gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp, and that
// GEMM
// =============================================================================================
size_t tqt_get_m_step_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(void)
{
    return tqt_get_m_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950();
}
size_t tqt_get_n_step_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(void)
{
    return tqt_get_n_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950();
}
size_t tqt_get_a_im2colpack_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t m_idx, size_t k_idx, size_t lda, size_t actual_m)
{
    return tqt_get_a_packed_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
        m_idx, k_idx, lda, actual_m);
}
size_t tqt_get_b_packed_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb, size_t actual_n)
{
    return tqt_get_b_packed_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
        n_idx, k_idx, ldb, actual_n);
}
size_t tqt_get_c_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc)
{
    return tqt_get_c_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(m_idx,
                                                                                         n_idx, ldc);
}
size_t tqt_get_bias_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t n_idx)
{
    return tqt_get_bias_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(n_idx);
}
size_t tqt_get_d_offset_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd)
{
    return tqt_get_d_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(m_idx,
                                                                                         n_idx, ldd);
}
size_t tqt_get_d_size_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(size_t m,
                                                                                     size_t n)
{
    return tqt_get_d_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(m, n);
}
size_t tqt_get_a_im2colpack_size_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t m, size_t k)
{
    return tqt_get_a_packed_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(m, k);
}
size_t tqt_get_b_packed_size_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t n, size_t k)
{
    return tqt_get_b_packed_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(n, k);
}

void tqt_run_bt_pack_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed,
    void *stream)
{
    tqt_run_bt_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(
        n, k, ldb, ldb_packed, k_idx, B, B_packed, stream);
}

void tqt_run_bt_pack_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed)
{
    tqt_run_bt_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
        n, k, ldb, ldb_packed, k_idx, B, B_packed);
}

void tqt_run_a_im2colpack_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(
    size_t group_idx, const void *activation, size_t lda_packed, size_t k_idx, void *A_packed,
    const tqt_conv_params *params, void *stream)
{
    im2col_rows_run(
        group_idx, activation, A_packed, false, true, kPackI8MStep, lda_packed, k_idx, params,
        as_stream(stream),
        "tqt_run_a_im2colpack_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950");
}

void tqt_run_a_im2colpack_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t group_idx, const void *activation, size_t lda_packed, size_t k_idx, void *A_packed,
    const tqt_conv_params *params)
{
    tqt_run_a_im2colpack_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(
        group_idx, activation, lda_packed, k_idx, A_packed, params, nullptr);
    finish_sync(
        nullptr,
        "tqt_run_a_im2colpack_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950");
}

void tqt_run_conv_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const struct tqt_qai8_qai8_qsi8cx_params *params, void *stream)
{
    tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(
        m, n, k, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, C, ldc, D, ldd, bias, clamp_min,
        clamp_max, params, stream);
}

void tqt_run_conv_convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const struct tqt_qai8_qai8_qsi8cx_params *params)
{
    tqt_run_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
        m, n, k, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, C, ldc, D, ldd, bias, clamp_min,
        clamp_max, params);
}

// =============================================================================================
// convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8 (reference …/convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_4x1vl_rvv.cpp): channel-first im2col
// B [K, N] + gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8 with the weights as A [OC_per_group, K]
// =============================================================================================
size_t tqt_get_m_step_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(void)
{
    return tqt_get_m_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950();
}
size_t tqt_get_n_step_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(void)
{
    return tqt_get_n_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950();
}
size_t tqt_get_a_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m_idx, size_t k_idx, size_t lda)
{
    return tqt_get_a_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(m_idx, k_idx, lda);
}
size_t tqt_get_c_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldc)
{
    return tqt_get_c_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(m_idx, n_idx, ldc);
}
size_t tqt_get_bias_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m_idx)
{
    return tqt_get_bias_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(m_idx);
}
size_t tqt_get_d_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldd)
{
    return tqt_get_d_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(m_idx, n_idx, ldd);
}
size_t tqt_get_d_size_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t m, size_t n)
{
    return tqt_get_d_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(m, n);
}
size_t tqt_get_b_im2col_size_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t k, size_t n)
{
    return k * n * sizeof(int8_t);
}
size_t tqt_get_b_im2col_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t n_idx, size_t k_idx, size_t ldb_im2col)
{
    return (k_idx * ldb_im2col + n_idx) * sizeof(int8_t);
}

void tqt_run_im2col_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950_async(size_t group_idx, const void *activation,
                                            void *im2col_buf, const tqt_conv_params *params,
                                            void *stream)
{
    im2col_cf_run(group_idx, activation, im2col_buf, params, as_stream(stream),
                  "tqt_run_im2col_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950");
}

void tqt_run_im2col_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(size_t group_idx, const void *activation,
                                      void *im2col_buf, const tqt_conv_params *params)
{
    tqt_run_im2col_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950_async(group_idx, activation, im2col_buf, params, nullptr);
    finish_sync(nullptr, "tqt_run_im2col_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950");
}

void tqt_run_conv_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qsi8dx_qai8_params *params,
    void *stream)
{
    tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950_async(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd,
                                    bias, clamp_min, clamp_max, params, stream);
}

void tqt_run_conv_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A, size_t lda, size_t k_idx_a, const void *B,
    size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D, size_t ldd, const void *bias,
    int8_t clamp_min, int8_t clamp_max, const struct tqt_qai8_qsi8dx_qai8_params *params)
{
    tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8_mfma_gfx950(m, n, k, A, lda, k_idx_a, B, ldb, k_idx_b, C, ldc, D, ldd, bias,
                              clamp_min, clamp_max, params);
}

// =============================================================================================
// convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p (reference …/convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_4x1vl_rvv.cpp): the channel-first
// im2col written transposed (pixel rows) into the packed B layout of gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p,
// the weights packed as its A, and that GEMM
// =============================================================================================
size_t tqt_get_m_step_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(void)
{
    return tqt_get_m_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950();
}
size_t tqt_get_n_step_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(void)
{
    return tqt_get_n_step_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950();
}
size_t tqt_get_a_packed_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t m_idx, size_t k_idx, size_t lda,
                                                  size_t actual_m)
{
    return tqt_get_a_packed_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(m_idx, k_idx, lda, actual_m);
}
size_t tqt_get_b_im2colpack_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t n_idx, size_t k_idx, size_t ldb,
                                                      size_t actual_n)
{
    return tqt_get_b_packed_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(n_idx, k_idx, ldb, actual_n);
}
size_t tqt_get_c_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldc)
{
    return tqt_get_c_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(m_idx, n_idx, ldc);
}
size_t tqt_get_bias_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t m_idx)
{
    return tqt_get_bias_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(m_idx);
}
size_t tqt_get_d_offset_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldd)
{
    return tqt_get_d_offset_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(m_idx, n_idx, ldd);
}
size_t tqt_get_d_size_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t m, size_t n)
{
    return tqt_get_d_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(m, n);
}
size_t tqt_get_a_packed_size_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t m, size_t k)
{
    return tqt_get_a_packed_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(m, k);
}
size_t tqt_get_b_im2colpack_size_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t n, size_t k)
{
    return tqt_get_b_packed_size_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(n, k);
}

void tqt_run_a_pack_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950_async(size_t m, size_t k, size_t lda, size_t lda_packed,
                                             size_t k_idx, const void *A, void *A_packed,
                                             void *stream)
{
    tqt_run_a_pack_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950_async(m, k, lda, lda_packed, k_idx, A, A_packed, stream);
}
void tqt_run_a_pack_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t m, size_t k, size_t lda, size_t lda_packed,
                                       size_t k_idx, const void *A, void *A_packed)
{
    tqt_run_a_pack_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(m, k, lda, lda_packed, k_idx, A, A_packed);
}

void tqt_run_b_im2colpack_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950_async(size_t group_idx, const void *activation,
                                                   size_t ldb_packed, size_t k_idx,
                                                   void *B_packed,
                                                   const tqt_conv_params *params, void *stream)
{
    im2col_rows_run(group_idx, activation, B_packed, true, true, kPackI8NStep, ldb_packed, k_idx,
                    params, as_stream(stream), "tqt_run_b_im2colpack_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950");
}

void tqt_run_b_im2colpack_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(size_t group_idx, const void *activation,
                                             size_t ldb_packed, size_t k_idx, void *B_packed,
                                             const tqt_conv_params *params)
{
    tqt_run_b_im2colpack_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950_async(group_idx, activation, ldb_packed, k_idx,
                                                  B_packed, params, nullptr);
    finish_sync(nullptr, "tqt_run_b_im2colpack_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950");
}

void tqt_run_conv_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950_async(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const struct tqt_qai8_qsi8dx_qai8_params *params, void *stream)
{
    tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950_async(m, n, k, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, C,
                                     ldc, D, ldd, bias, clamp_min, clamp_max, params, stream);
}

void tqt_run_conv_convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(
    size_t m, size_t n, size_t k, const void *A_packed, size_t lda, size_t k_idx_a,
    const void *B_packed, size_t ldb, size_t k_idx_b, const void *C, size_t ldc, void *D,
    size_t ldd, const void *bias, int8_t clamp_min, int8_t clamp_max,
    const struct tqt_qai8_qsi8dx_qai8_params *params)
{
    tqt_run_gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p_mfma_gfx950(m, n, k, A_packed, lda, k_idx_a, B_packed, ldb, k_idx_b, C, ldc, D,
                               ldd, bias, clamp_min, clamp_max, params);
}

}  // extern "C"
