// Packers and geometry getters of the packed (p) kernel types on gfx950:
//   gemm_clamp_i32_i8p_i8p, gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp,
//   gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp, gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp,
//   gemm_1xnbias_clamp_f16_f16p_qsi4c2p, igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp,
//   and the output-type siblings gemm_1xnbias_clamp_{f16,bf16}_qai8dxp_qsi4cxp,
//   gemm_1xnbias_clamp_f32_f16p_qsi4c2p and gemm_1xnbias_clamp_{f32,f16}_qai8dxp_qsi8cxp (same
//   layouts as the types they share a mainloop with).
// Their run functions live beside the mainloops they share (int8_mfma.hip, gemm_i8_i4.hip,
// gemm_f16_i4.hip). The layout (PackDesc, pack_offset) is defined in tqt_hip_common.hpp; the
// reference's packers are the permutations of tqt_gemm_pack_rvv.h:354-398, 542-567, 740-856.
//
// A packer is one GPU kernel: one thread per 16-byte piece of a row gathers its bytes from the
// source row (k-contiguous [rows, k] sources) or column ([k, n] sources). Chunks are multiples of
// 16 bytes, so a piece never straddles two chunks and its bytes are contiguous in the output.
#include "tqt_hip_common.hpp"
#include "tqt_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_clamp_i32_i8p_i8p_mfma_gfx950.h"
#include "tqt_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp_mfma_gfx950.h"
#include "tqt_gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp_mfma_gfx950.h"

namespace tqt {
namespace {

// Byte kb of source row r is at p + r * rs + kb * cs (cs = 1: k-contiguous rows; rs = 1 and
// cs = ld: an int8 [k, n] matrix whose columns are the packed rows).
struct PackSrc
{
    const uint8_t *p;
    long long rs, cs;
};

template <bool kFrag>
__global__ __launch_bounds__(256) void pack_kernel(PackSrc s, uint8_t *dst, PackDesc d,
                                                   long long nchunks, long long total, int row0)
{
    const long long idx = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) {
        return;
    }
    const int rr = static_cast<int>(idx / nchunks);
    const int r = row0 + rr;
    const long long kb0 = 16 * (idx - static_cast<long long>(rr) * nchunks);
    const long long rem = d.kbytes - kb0;
    const int cw = rem < 16 ? static_cast<int>(rem) : 16;
    uint8_t *o = dst + pack_offset(d, r, kb0);  // the piece's cw bytes are contiguous
    const uint8_t *row = s.p + static_cast<long long>(r) * s.rs;
    if (!kFrag && s.cs == 1 && cw == 16 &&
        ((reinterpret_cast<uintptr_t>(row + kb0) | reinterpret_cast<uintptr_t>(o)) & 15) == 0) {
        *reinterpret_cast<u32x4 *>(o) = *reinterpret_cast<const u32x4 *>(row + kb0);
        return;
    }
    for (int i = 0; i < cw; ++i) {
        // stored position kb0 + i holds logical byte w4a16_frag_pos(kb0 + i) (an involution)
        const long long kb = kFrag ? w4a16_frag_pos(kb0 + i, d.kbytes) : kb0 + i;
        o[i] = row[kb * s.cs];
    }
}

// Packs `d.rows` rows of `d.kbytes` bytes from `src` into `dst`. A narrow last panel moved back
// by the k_idx tail rule can overlap the end of the panel before it; the reference packs panel
// after panel, so the last panel's bytes win there: it is then written by a second launch,
// ordered after the first on the stream.
void pack_rows(const void *src, long long rs, long long cs, void *dst, const PackDesc &d,
               bool frag, void *stream, bool sync, const char *where)
{
    if (d.rows <= 0 || d.kbytes <= 0) {
        return;
    }
    TQT_REQUIRE(src != nullptr && dst != nullptr, "NULL pack buffer");
    const long long nchunks = (d.kbytes + 15) / 16;
    const PackSrc s = {static_cast<const uint8_t *>(src), rs, cs};
    hipStream_t st = as_stream(stream);
    const int split = tail_panel_start(d);
    for (int part = 0; part < 2; ++part) {
        const int row0 = part == 0 ? 0 : split;
        const int rows = part == 0 ? split : d.rows - split;
        if (rows <= 0) {
            continue;
        }
        const long long total = nchunks * rows;
        const long long blocks = (total + 255) / 256;
        TQT_REQUIRE(blocks < (1ll << 31), "pack grid too large");
        if (frag) {
            hipLaunchKernelGGL(pack_kernel<true>, dim3(blocks), dim3(256), 0, st, s,
                               static_cast<uint8_t *>(dst), d, nchunks, total, row0);
        } else {
            hipLaunchKernelGGL(pack_kernel<false>, dim3(blocks), dim3(256), 0, st, s,
                               static_cast<uint8_t *>(dst), d, nchunks, total, row0);
        }
    }
    if (sync) {
        finish_sync(st, where);
    } else {
        check_launch(where);
    }
}

// Packer argument conventions of the reference (tqt_gemm_pack_rvv.h): (rows, k, ld, ld_packed,
// k_idx) in elements of `esize` bytes; int4 operands pass esize 0 (two elements per byte).
void pack_nk(size_t rows, size_t k, size_t ld, size_t ld_packed, size_t k_idx, size_t step,
             int kc, int esize, bool frag, const void *src, void *dst, void *stream, bool sync,
             const char *where)
{
    if (esize == 0) {
        TQT_REQUIRE(k % 2 == 0 && ld % 2 == 0 && ld_packed % 2 == 0 && k_idx % 2 == 0,
                    "int4 packing needs even k, ld, ld_packed and k_idx");
    }
    TQT_REQUIRE(ld >= k && ld_packed >= k, "ld < k");
    auto bytes = [esize](size_t e) { return esize == 0 ? e / 2 : e * esize; };
    const PackDesc d = make_pack(step, kc, rows, bytes(ld_packed), bytes(k), bytes(k_idx));
    pack_rows(src, static_cast<long long>(bytes(ld)), 1, dst, d, frag, stream, sync, where);
}

// int8 B given as [k, n] row-major (ldb >= n): packed rows are its columns.
void pack_kn_i8(size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, size_t step,
                const void *src, void *dst, void *stream, bool sync, const char *where)
{
    TQT_REQUIRE(ldb >= n && ldb_packed >= k, "ldb < n or ldb_packed < k");
    const PackDesc d = make_pack(step, kPackI8Chunk, n, ldb_packed, k, k_idx);
    pack_rows(src, 1, static_cast<long long>(ldb), dst, d, false, stream, sync, where);
}

size_t packed_offset(size_t idx, size_t k_idx, size_t ld, size_t actual, size_t step,
                     size_t esize)
{
    return (idx * ld + k_idx * (actual < step ? actual : step)) * esize;
}

}  // namespace
}  // namespace tqt

using namespace tqt;

#define TQT_REQ_M(step) TQT_REQUIRE(m_idx % (step) == 0, "m_idx % m_step == 0")
#define TQT_REQ_N(step) TQT_REQUIRE(n_idx % (step) == 0, "n_idx % n_step == 0")

extern "C" {

// =============================================================================================
// gemm_clamp_i32_i8p_i8p (reference …/gemm_clamp_i32_i8p_i8p/…_4x1vl_rvv.cpp)
// =============================================================================================
size_t tqt_get_m_step_gemm_clamp_i32_i8p_i8p_mfma_gfx950(void)
{
    return kPackI8MStep;
}
size_t tqt_get_n_step_gemm_clamp_i32_i8p_i8p_mfma_gfx950(void)
{
    return kPackI8NStep;
}
size_t tqt_get_a_packed_offset_gemm_clamp_i32_i8p_i8p_mfma_gfx950(size_t m_idx, size_t k_idx,
                                                                   size_t lda, size_t actual_m)
{
    TQT_REQ_M(kPackI8MStep);
    return packed_offset(m_idx, k_idx, lda, actual_m, kPackI8MStep, 1);
}
size_t tqt_get_b_packed_offset_gemm_clamp_i32_i8p_i8p_mfma_gfx950(size_t n_idx, size_t k_idx,
                                                                   size_t ldb, size_t actual_n)
{
    TQT_REQ_N(kPackI8NStep);
    return packed_offset(n_idx, k_idx, ldb, actual_n, kPackI8NStep, 1);
}
size_t tqt_get_c_offset_gemm_clamp_i32_i8p_i8p_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldc)
{
    TQT_REQ_M(kPackI8MStep);
    TQT_REQ_N(kPackI8NStep);
    return (m_idx * ldc + n_idx) * sizeof(int32_t);
}
size_t tqt_get_d_offset_gemm_clamp_i32_i8p_i8p_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldd)
{
    TQT_REQ_M(kPackI8MStep);
    TQT_REQ_N(kPackI8NStep);
    return (m_idx * ldd + n_idx) * sizeof(int32_t);
}
size_t tqt_get_d_size_gemm_clamp_i32_i8p_i8p_mfma_gfx950(size_t m, size_t n)
{
    return m * n * sizeof(int32_t);
}
size_t tqt_get_a_packed_size_gemm_clamp_i32_i8p_i8p_mfma_gfx950(size_t m, size_t k)
{
    return m * k;
}
size_t tqt_get_b_packed_size_gemm_clamp_i32_i8p_i8p_mfma_gfx950(size_t n, size_t k)
{
    return n * k;
}
void tqt_run_a_pack_gemm_clamp_i32_i8p_i8p_mfma_gfx950_async(size_t m, size_t k, size_t lda,
                                                             size_t lda_packed, size_t k_idx,
                                                             const void *A, void *A_packed,
                                                             void *stream)
{
    pack_nk(m, k, lda, lda_packed, k_idx, kPackI8MStep, kPackI8Chunk, 1, false, A, A_packed, stream, false,
            "tqt_run_a_pack_gemm_clamp_i32_i8p_i8p_mfma_gfx950");
}
void tqt_run_a_pack_gemm_clamp_i32_i8p_i8p_mfma_gfx950(size_t m, size_t k, size_t lda,
                                                       size_t lda_packed, size_t k_idx,
                                                       const void *A, void *A_packed)
{
    pack_nk(m, k, lda, lda_packed, k_idx, kPackI8MStep, kPackI8Chunk, 1, false, A, A_packed, nullptr, true,
            "tqt_run_a_pack_gemm_clamp_i32_i8p_i8p_mfma_gfx950");
}
void tqt_run_b_pack_gemm_clamp_i32_i8p_i8p_mfma_gfx950_async(size_t n, size_t k, size_t ldb,
                                                             size_t ldb_packed, size_t k_idx,
                                                             const void *B, void *B_packed,
                                                             void *stream)
{
    pack_kn_i8(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, B, B_packed, stream, false,
               "tqt_run_b_pack_gemm_clamp_i32_i8p_i8p_mfma_gfx950");
}
void tqt_run_b_pack_gemm_clamp_i32_i8p_i8p_mfma_gfx950(size_t n, size_t k, size_t ldb,
                                                       size_t ldb_packed, size_t k_idx,
                                                       const void *B, void *B_packed)
{
    pack_kn_i8(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, B, B_packed, nullptr, true,
               "tqt_run_b_pack_gemm_clamp_i32_i8p_i8p_mfma_gfx950");
}
void tqt_run_bt_pack_gemm_clamp_i32_i8p_i8p_mfma_gfx950_async(size_t n, size_t k, size_t ldb,
                                                              size_t ldb_packed, size_t k_idx,
                                                              const void *B, void *B_packed,
                                                              void *stream)
{
    pack_nk(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, kPackI8Chunk, 1, false, B, B_packed, stream, false,
            "tqt_run_bt_pack_gemm_clamp_i32_i8p_i8p_mfma_gfx950");
}
void tqt_run_bt_pack_gemm_clamp_i32_i8p_i8p_mfma_gfx950(size_t n, size_t k, size_t ldb,
                                                        size_t ldb_packed, size_t k_idx,
                                                        const void *B, void *B_packed)
{
    pack_nk(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, kPackI8Chunk, 1, false, B, B_packed, nullptr, true,
            "tqt_run_bt_pack_gemm_clamp_i32_i8p_i8p_mfma_gfx950");
}

// =============================================================================================
// gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp (reference …qai8_qai8_qsi8cxp_4x1vl_rvv.cpp)
// =============================================================================================
size_t tqt_get_m_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(void)
{
    return kPackI8MStep;
}
size_t tqt_get_n_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(void)
{
    return kPackI8NStep;
}
size_t tqt_get_a_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(size_t m_idx,
                                                                                    size_t k_idx,
                                                                                    size_t lda)
{
    TQT_REQ_M(kPackI8MStep);
    return m_idx * lda + k_idx;
}
size_t tqt_get_b_packed_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb, size_t actual_n)
{
    TQT_REQ_N(kPackI8NStep);
    return packed_offset(n_idx, k_idx, ldb, actual_n, kPackI8NStep, 1);
}
size_t tqt_get_c_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(size_t m_idx,
                                                                                    size_t n_idx,
                                                                                    size_t ldc)
{
    TQT_REQ_M(kPackI8MStep);
    TQT_REQ_N(kPackI8NStep);
    return (m_idx * ldc + n_idx) * sizeof(int32_t);
}
size_t tqt_get_bias_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(
    size_t n_idx)
{
    TQT_REQ_N(kPackI8NStep);
    return n_idx * sizeof(int32_t);
}
size_t tqt_get_d_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(size_t m_idx,
                                                                                    size_t n_idx,
                                                                                    size_t ldd)
{
    TQT_REQ_M(kPackI8MStep);
    TQT_REQ_N(kPackI8NStep);
    return m_idx * ldd + n_idx;
}
size_t tqt_get_d_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(size_t m,
                                                                                  size_t n)
{
    return m * n;
}
size_t tqt_get_b_packed_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(size_t n,
                                                                                         size_t k)
{
    return n * k;
}
void tqt_run_b_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950_async(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed,
    void *stream)
{
    pack_kn_i8(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, B, B_packed, stream, false,
               "tqt_run_b_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950");
}
void tqt_run_b_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed)
{
    pack_kn_i8(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, B, B_packed, nullptr, true,
               "tqt_run_b_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950");
}
void tqt_run_bt_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950_async(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed,
    void *stream)
{
    pack_nk(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, kPackI8Chunk, 1, false, B, B_packed, stream, false,
            "tqt_run_bt_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950");
}
void tqt_run_bt_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed)
{
    pack_nk(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, kPackI8Chunk, 1, false, B, B_packed, nullptr, true,
            "tqt_run_bt_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950");
}

// =============================================================================================
// gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp (reference …qai8_qai8p_qsi8cxp_4x1vl_rvv.cpp)
// =============================================================================================
size_t tqt_get_m_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(void)
{
    return kPackI8MStep;
}
size_t tqt_get_n_step_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(void)
{
    return kPackI8NStep;
}
size_t tqt_get_a_packed_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t m_idx, size_t k_idx, size_t lda, size_t actual_m)
{
    TQT_REQ_M(kPackI8MStep);
    return packed_offset(m_idx, k_idx, lda, actual_m, kPackI8MStep, 1);
}
size_t tqt_get_b_packed_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb, size_t actual_n)
{
    TQT_REQ_N(kPackI8NStep);
    return packed_offset(n_idx, k_idx, ldb, actual_n, kPackI8NStep, 1);
}
size_t tqt_get_c_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(size_t m_idx,
                                                                                     size_t n_idx,
                                                                                     size_t ldc)
{
    TQT_REQ_M(kPackI8MStep);
    TQT_REQ_N(kPackI8NStep);
    return (m_idx * ldc + n_idx) * sizeof(int32_t);
}
size_t tqt_get_bias_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t n_idx)
{
    TQT_REQ_N(kPackI8NStep);
    return n_idx * sizeof(int32_t);
}
size_t tqt_get_d_offset_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(size_t m_idx,
                                                                                     size_t n_idx,
                                                                                     size_t ldd)
{
    TQT_REQ_M(kPackI8MStep);
    TQT_REQ_N(kPackI8NStep);
    return m_idx * ldd + n_idx;
}
size_t tqt_get_d_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(size_t m,
                                                                                   size_t n)
{
    return m * n;
}
size_t tqt_get_a_packed_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t m, size_t k)
{
    return m * k;
}
size_t tqt_get_b_packed_size_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t n, size_t k)
{
    return n * k;
}
void tqt_run_a_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(
    size_t m, size_t k, size_t lda, size_t lda_packed, size_t k_idx, const void *A, void *A_packed,
    void *stream)
{
    pack_nk(m, k, lda, lda_packed, k_idx, kPackI8MStep, kPackI8Chunk, 1, false, A, A_packed, stream, false,
            "tqt_run_a_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950");
}
void tqt_run_a_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t m, size_t k, size_t lda, size_t lda_packed, size_t k_idx, const void *A, void *A_packed)
{
    pack_nk(m, k, lda, lda_packed, k_idx, kPackI8MStep, kPackI8Chunk, 1, false, A, A_packed, nullptr, true,
            "tqt_run_a_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950");
}
void tqt_run_b_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed,
    void *stream)
{
    pack_kn_i8(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, B, B_packed, stream, false,
               "tqt_run_b_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950");
}
void tqt_run_b_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed)
{
    pack_kn_i8(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, B, B_packed, nullptr, true,
               "tqt_run_b_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950");
}
void tqt_run_bt_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950_async(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed,
    void *stream)
{
    pack_nk(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, kPackI8Chunk, 1, false, B, B_packed, stream, false,
            "tqt_run_bt_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950");
}
void tqt_run_bt_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed)
{
    pack_nk(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, kPackI8Chunk, 1, false, B, B_packed, nullptr, true,
            "tqt_run_bt_pack_gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp_mfma_gfx950");
}

// =============================================================================================
// gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp (reference …qai8dxp_qsi4cxp_4x1vl_rvv.cpp:25-111)
// =============================================================================================
size_t tqt_get_m_step_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950(void)
{
    return kPackW4A8MStep;
}
size_t tqt_get_n_step_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950(void)
{
    return kPackW4A8NStep;
}
size_t tqt_get_a_packed_offset_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950(size_t m_idx,
                                                                                  size_t k_idx,
                                                                                  size_t lda,
                                                                                  size_t actual_m)
{
    TQT_REQ_M(kPackW4A8MStep);
    return packed_offset(m_idx, k_idx, lda, actual_m, kPackW4A8MStep, 1);
}
size_t tqt_get_b_packed_offset_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950(size_t n_idx,
                                                                                  size_t k_idx,
                                                                                  size_t ldb,
                                                                                  size_t actual_n)
{
    TQT_REQ_N(kPackW4A8NStep);
    TQT_REQUIRE(k_idx % 2 == 0, "k_idx % 2 == 0");
    const size_t w = actual_n < kPackW4A8NStep ? actual_n : kPackW4A8NStep;
    return n_idx * (ldb / 2) + (k_idx / 2) * w;
}
size_t tqt_get_c_offset_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950(size_t m_idx,
                                                                           size_t n_idx,
                                                                           size_t ldc)
{
    TQT_REQ_M(kPackW4A8MStep);
    TQT_REQ_N(kPackW4A8NStep);
    return (m_idx * ldc + n_idx) * sizeof(float);
}
size_t tqt_get_bias_offset_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950(size_t n_idx)
{
    TQT_REQ_N(kPackW4A8NStep);
    return n_idx * sizeof(float);
}
size_t tqt_get_d_offset_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950(size_t m_idx,
                                                                           size_t n_idx,
                                                                           size_t ldd)
{
    TQT_REQ_M(kPackW4A8MStep);
    TQT_REQ_N(kPackW4A8NStep);
    return (m_idx * ldd + n_idx) * sizeof(float);
}
size_t tqt_get_d_size_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950(size_t m, size_t n)
{
    return m * n * sizeof(float);
}
size_t tqt_get_a_packed_size_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950(size_t m,
                                                                                size_t k)
{
    return m * k;
}
size_t tqt_get_b_packed_size_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950(size_t n,
                                                                                size_t k)
{
    return n * k / 2;
}
void tqt_run_a_pack_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950_async(
    size_t m, size_t k, size_t lda, size_t lda_packed, size_t k_idx, const void *A, void *A_packed,
    void *stream)
{
    pack_nk(m, k, lda, lda_packed, k_idx, kPackW4A8MStep, kPackW4A8Chunk, 1, false, A, A_packed, stream, false,
            "tqt_run_a_pack_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950");
}
void tqt_run_a_pack_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950(
    size_t m, size_t k, size_t lda, size_t lda_packed, size_t k_idx, const void *A, void *A_packed)
{
    pack_nk(m, k, lda, lda_packed, k_idx, kPackW4A8MStep, kPackW4A8Chunk, 1, false, A, A_packed, nullptr, true,
            "tqt_run_a_pack_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950");
}
void tqt_run_bt_pack_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950_async(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed,
    void *stream)
{
    pack_nk(n, k, ldb, ldb_packed, k_idx, kPackW4A8NStep, kPackW4A8Chunk, 0, false, B, B_packed, stream, false,
            "tqt_run_bt_pack_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950");
}
void tqt_run_bt_pack_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed)
{
    pack_nk(n, k, ldb, ldb_packed, k_idx, kPackW4A8NStep, kPackW4A8Chunk, 0, false, B, B_packed, nullptr, true,
            "tqt_run_bt_pack_gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp_mfma_gfx950");
}

// =============================================================================================
// gemm_1xnbias_clamp_f16_f16p_qsi4c2p (reference …f16p_qsi4c2p_8x2vl_rvv.cpp:25-119)
// =============================================================================================
size_t tqt_get_m_step_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(void)
{
    return kPackW4A16MStep;
}
size_t tqt_get_n_step_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(void)
{
    return kPackW4A16NStep;
}
size_t tqt_get_a_packed_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(size_t m_idx,
                                                                               size_t k_idx,
                                                                               size_t lda,
                                                                               size_t actual_m)
{
    TQT_REQ_M(kPackW4A16MStep);
    return packed_offset(m_idx, k_idx, lda, actual_m, kPackW4A16MStep, sizeof(uint16_t));
}
size_t tqt_get_b_packed_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(size_t n_idx,
                                                                               size_t k_idx,
                                                                               size_t ldb,
                                                                               size_t actual_n)
{
    TQT_REQ_N(kPackW4A16NStep);
    const size_t w = actual_n < kPackW4A16NStep ? actual_n : kPackW4A16NStep;
    return n_idx * (ldb / 2) + (k_idx / 2) * w;
}
size_t tqt_get_scale_b_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(size_t n_idx,
                                                                              size_t b_idx,
                                                                              size_t ldsb)
{
    TQT_REQ_N(kPackW4A16NStep);
    return (n_idx * ldsb + b_idx) * sizeof(uint16_t);
}
size_t tqt_get_c_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(size_t m_idx, size_t n_idx,
                                                                        size_t ldc)
{
    TQT_REQ_M(kPackW4A16MStep);
    TQT_REQ_N(kPackW4A16NStep);
    return (m_idx * ldc + n_idx) * sizeof(uint16_t);
}
size_t tqt_get_bias_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(size_t n_idx)
{
    TQT_REQ_N(kPackW4A16NStep);
    return n_idx * sizeof(uint16_t);
}
size_t tqt_get_d_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(size_t m_idx, size_t n_idx,
                                                                        size_t ldd)
{
    TQT_REQ_M(kPackW4A16MStep);
    TQT_REQ_N(kPackW4A16NStep);
    return (m_idx * ldd + n_idx) * sizeof(uint16_t);
}
size_t tqt_get_d_size_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(size_t m, size_t n)
{
    return m * n * sizeof(uint16_t);
}
size_t tqt_get_a_packed_size_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(size_t m, size_t k)
{
    return m * k * sizeof(uint16_t);
}
size_t tqt_get_b_packed_size_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(size_t n, size_t k)
{
    return n * k / 2;
}
void tqt_run_a_pack_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950_async(
    size_t m, size_t k, size_t lda, size_t lda_packed, size_t k_idx, const void *A, void *A_packed,
    void *stream)
{
    pack_nk(m, k, lda, lda_packed, k_idx, kPackW4A16MStep, kPackW4A16Chunk, 2, false, A, A_packed, stream, false,
            "tqt_run_a_pack_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950");
}
void tqt_run_a_pack_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(
    size_t m, size_t k, size_t lda, size_t lda_packed, size_t k_idx, const void *A, void *A_packed)
{
    pack_nk(m, k, lda, lda_packed, k_idx, kPackW4A16MStep, kPackW4A16Chunk, 2, false, A, A_packed, nullptr, true,
            "tqt_run_a_pack_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950");
}
void tqt_run_bt_pack_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950_async(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed,
    void *stream)
{
    pack_nk(n, k, ldb, ldb_packed, k_idx, kPackW4A16NStep, kPackW4A16Chunk, 0, true, B, B_packed, stream, false,
            "tqt_run_bt_pack_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950");
}
void tqt_run_bt_pack_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed)
{
    pack_nk(n, k, ldb, ldb_packed, k_idx, kPackW4A16NStep, kPackW4A16Chunk, 0, true, B, B_packed, nullptr, true,
            "tqt_run_bt_pack_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950");
}

// =============================================================================================
// gemm_1xnbias_clamp_{f32,f16}_qai8dxp_qsi8cxp (reference …qai8dxp_qsi8cxp_4x1vl_rvv.cpp): the
// layout and packers of qai8_qai8p_qsi8cxp; bias and D are f32 / f16 (ES bytes per element).
// =============================================================================================
#define TQT_DYNP(T, ES)                                                                            \
    size_t tqt_get_m_step_##T##_mfma_gfx950(void) { return kPackI8MStep; }                         \
    size_t tqt_get_n_step_##T##_mfma_gfx950(void) { return kPackI8NStep; }                         \
    size_t tqt_get_a_packed_offset_##T##_mfma_gfx950(size_t m_idx, size_t k_idx, size_t lda,       \
                                                     size_t actual_m)                              \
    {                                                                                              \
        TQT_REQ_M(kPackI8MStep);                                                                   \
        return packed_offset(m_idx, k_idx, lda, actual_m, kPackI8MStep, 1);                        \
    }                                                                                              \
    size_t tqt_get_b_packed_offset_##T##_mfma_gfx950(size_t n_idx, size_t k_idx, size_t ldb,       \
                                                     size_t actual_n)                              \
    {                                                                                              \
        TQT_REQ_N(kPackI8NStep);                                                                   \
        return packed_offset(n_idx, k_idx, ldb, actual_n, kPackI8NStep, 1);                        \
    }                                                                                              \
    size_t tqt_get_c_offset_##T##_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldc)             \
    {                                                                                              \
        TQT_REQ_M(kPackI8MStep);                                                                   \
        TQT_REQ_N(kPackI8NStep);                                                                   \
        return (m_idx * ldc + n_idx) * (ES);                                                       \
    }                                                                                              \
    size_t tqt_get_bias_offset_##T##_mfma_gfx950(size_t n_idx)                                    \
    {                                                                                              \
        TQT_REQ_N(kPackI8NStep);                                                                   \
        return n_idx * (ES);                                                                       \
    }                                                                                              \
    size_t tqt_get_d_offset_##T##_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldd)             \
    {                                                                                              \
        TQT_REQ_M(kPackI8MStep);                                                                   \
        TQT_REQ_N(kPackI8NStep);                                                                   \
        return (m_idx * ldd + n_idx) * (ES);                                                       \
    }                                                                                              \
    size_t tqt_get_d_size_##T##_mfma_gfx950(size_t m, size_t n) { return m * n * (ES); }          \
    size_t tqt_get_a_packed_size_##T##_mfma_gfx950(size_t m, size_t k) { return m * k; }           \
    size_t tqt_get_b_packed_size_##T##_mfma_gfx950(size_t n, size_t k) { return n * k; }           \
    void tqt_run_a_pack_##T##_mfma_gfx950_async(size_t m, size_t k, size_t lda, size_t lda_packed, \
                                                size_t k_idx, const void *A, void *A_packed,       \
                                                void *stream)                                      \
    {                                                                                              \
        pack_nk(m, k, lda, lda_packed, k_idx, kPackI8MStep, kPackI8Chunk, 1, false, A, A_packed,   \
                stream, false, "tqt_run_a_pack_" #T "_mfma_gfx950");                               \
    }                                                                                              \
    void tqt_run_a_pack_##T##_mfma_gfx950(size_t m, size_t k, size_t lda, size_t lda_packed,       \
                                          size_t k_idx, const void *A, void *A_packed)             \
    {                                                                                              \
        pack_nk(m, k, lda, lda_packed, k_idx, kPackI8MStep, kPackI8Chunk, 1, false, A, A_packed,   \
                nullptr, true, "tqt_run_a_pack_" #T "_mfma_gfx950");                               \
    }                                                                                              \
    void tqt_run_b_pack_##T##_mfma_gfx950_async(size_t n, size_t k, size_t ldb, size_t ldb_packed, \
                                                size_t k_idx, const void *B, void *B_packed,       \
                                                void *stream)                                      \
    {                                                                                              \
        pack_kn_i8(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, B, B_packed, stream, false,         \
                   "tqt_run_b_pack_" #T "_mfma_gfx950");                                           \
    }                                                                                              \
    void tqt_run_b_pack_##T##_mfma_gfx950(size_t n, size_t k, size_t ldb, size_t ldb_packed,       \
                                          size_t k_idx, const void *B, void *B_packed)             \
    {                                                                                              \
        pack_kn_i8(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, B, B_packed, nullptr, true,         \
                   "tqt_run_b_pack_" #T "_mfma_gfx950");                                           \
    }                                                                                              \
    void tqt_run_bt_pack_##T##_mfma_gfx950_async(size_t n, size_t k, size_t ldb,                  \
                                                 size_t ldb_packed, size_t k_idx, const void *B,   \
                                                 void *B_packed, void *stream)                     \
    {                                                                                              \
        pack_nk(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, kPackI8Chunk, 1, false, B, B_packed,   \
                stream, false, "tqt_run_bt_pack_" #T "_mfma_gfx950");                              \
    }                                                                                              \
    void tqt_run_bt_pack_##T##_mfma_gfx950(size_t n, size_t k, size_t ldb, size_t ldb_packed,      \
                                           size_t k_idx, const void *B, void *B_packed)            \
    {                                                                                              \
        pack_nk(n, k, ldb, ldb_packed, k_idx, kPackI8NStep, kPackI8Chunk, 1, false, B, B_packed,   \
                nullptr, true, "tqt_run_bt_pack_" #T "_mfma_gfx950");                              \
    }

TQT_DYNP(gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp, sizeof(float))
TQT_DYNP(gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp, sizeof(uint16_t))

// =============================================================================================
// gemm_1xnbias_clamp_f32_f16p_qsi4c2p (reference …f32_f16p_qsi4c2p_8x2vl_rvv.cpp): the packed
// layout and packers of the f16 type; C, bias and D are f32.
// =============================================================================================
size_t tqt_get_m_step_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950(void)
{
    return kPackW4A16MStep;
}
size_t tqt_get_n_step_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950(void)
{
    return kPackW4A16NStep;
}
size_t tqt_get_a_packed_offset_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950(size_t m_idx,
                                                                               size_t k_idx,
                                                                               size_t lda,
                                                                               size_t actual_m)
{
    return tqt_get_a_packed_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(m_idx, k_idx,
                                                                                   lda, actual_m);
}
size_t tqt_get_b_packed_offset_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950(size_t n_idx,
                                                                               size_t k_idx,
                                                                               size_t ldb,
                                                                               size_t actual_n)
{
    return tqt_get_b_packed_offset_gemm_1xnbias_clamp_f16_f16p_qsi4c2p_mfma_gfx950(n_idx, k_idx,
                                                                                   ldb, actual_n);
}
size_t tqt_get_scale_b_offset_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950(size_t n_idx,
                                                                              size_t b_idx,
                                                                              size_t ldsb)
{
    TQT_REQ_N(kPackW4A16NStep);
    return (n_idx * ldsb + b_idx) * sizeof(uint16_t);
}
size_t tqt_get_c_offset_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950(size_t m_idx, size_t n_idx,
                                                                        size_t ldc)
{
    TQT_REQ_M(kPackW4A16MStep);
    TQT_REQ_N(kPackW4A16NStep);
    return (m_idx * ldc + n_idx) * sizeof(float);
}
size_t tqt_get_bias_offset_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950(size_t n_idx)
{
    TQT_REQ_N(kPackW4A16NStep);
    return n_idx * sizeof(float);
}
size_t tqt_get_d_offset_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950(size_t m_idx, size_t n_idx,
                                                                        size_t ldd)
{
    TQT_REQ_M(kPackW4A16MStep);
    TQT_REQ_N(kPackW4A16NStep);
    return (m_idx * ldd + n_idx) * sizeof(float);
}
size_t tqt_get_d_size_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950(size_t m, size_t n)
{
    return m * n * sizeof(float);
}
size_t tqt_get_a_packed_size_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950(size_t m, size_t k)
{
    return m * k * sizeof(uint16_t);
}
size_t tqt_get_b_packed_size_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950(size_t n, size_t k)
{
    return n * k / 2;
}
void tqt_run_a_pack_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950_async(
    size_t m, size_t k, size_t lda, size_t lda_packed, size_t k_idx, const void *A, void *A_packed,
    void *stream)
{
    pack_nk(m, k, lda, lda_packed, k_idx, kPackW4A16MStep, kPackW4A16Chunk, 2, false, A, A_packed, stream, false,
            "tqt_run_a_pack_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950");
}
void tqt_run_a_pack_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950(
    size_t m, size_t k, size_t lda, size_t lda_packed, size_t k_idx, const void *A, void *A_packed)
{
    pack_nk(m, k, lda, lda_packed, k_idx, kPackW4A16MStep, kPackW4A16Chunk, 2, false, A, A_packed, nullptr, true,
            "tqt_run_a_pack_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950");
}
void tqt_run_bt_pack_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950_async(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed,
    void *stream)
{
    pack_nk(n, k, ldb, ldb_packed, k_idx, kPackW4A16NStep, kPackW4A16Chunk, 0, true, B, B_packed, stream, false,
            "tqt_run_bt_pack_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950");
}
void tqt_run_bt_pack_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950(
    size_t n, size_t k, size_t ldb, size_t ldb_packed, size_t k_idx, const void *B, void *B_packed)
{
    pack_nk(n, k, ldb, ldb_packed, k_idx, kPackW4A16NStep, kPackW4A16Chunk, 0, true, B, B_packed, nullptr, true,
            "tqt_run_bt_pack_gemm_1xnbias_clamp_f32_f16p_qsi4c2p_mfma_gfx950");
}

// =============================================================================================
// igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp (reference …igemmcl…qsi8cxp_4x1vl_rvv.cpp)
// =============================================================================================
size_t tqt_get_m_step_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(void)
{
    return kPackI8MStep;
}
size_t tqt_get_n_step_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(void)
{
    return kPackI8NStep;
}
size_t tqt_get_b_packed_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(
    size_t n_idx, size_t k_idx, size_t ldb, size_t actual_n)
{
    TQT_REQ_N(kPackI8NStep);
    return packed_offset(n_idx, k_idx, ldb, actual_n, kPackI8NStep, 1);
}
size_t tqt_get_c_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldc)
{
    TQT_REQ_N(kPackI8NStep);
    return (m_idx * ldc + n_idx) * sizeof(int32_t);
}
size_t tqt_get_bias_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(
    size_t n_idx)
{
    TQT_REQ_N(kPackI8NStep);
    return n_idx * sizeof(int32_t);
}
size_t tqt_get_d_offset_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(
    size_t m_idx, size_t n_idx, size_t ldd)
{
    TQT_REQ_N(kPackI8NStep);
    return m_idx * ldd + n_idx;
}
size_t tqt_get_d_size_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(size_t m,
                                                                                    size_t n)
{
    return m * n;
}
size_t tqt_get_b_packed_size_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(
    size_t n, size_t k)
{
    return n * k;
}
void tqt_run_bt_pack_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950_async(
    size_t n, size_t k, size_t ldw, size_t ldw_packed, size_t k_idx, const void *weight,
    void *weight_packed, void *stream)
{
    pack_nk(n, k, ldw, ldw_packed, k_idx, kPackI8NStep, kPackI8Chunk, 1, false, weight, weight_packed, stream,
            false, "tqt_run_bt_pack_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950");
}
void tqt_run_bt_pack_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950(
    size_t n, size_t k, size_t ldw, size_t ldw_packed, size_t k_idx, const void *weight,
    void *weight_packed)
{
    pack_nk(n, k, ldw, ldw_packed, k_idx, kPackI8NStep, kPackI8Chunk, 1, false, weight, weight_packed, nullptr,
            true, "tqt_run_bt_pack_igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp_mfma_gfx950");
}

// =============================================================================================
// gemm_1xnbias_clamp_{f16,bf16}_qai8dxp_qsi4cxp (reference …_{f16,bf16}_qai8dxp_qsi4cxp_4x1vl_rvv.cpp):
// the packed layout and packers of qai8dxp_qsi4cxp with 2-byte C, bias and D elements.
// =============================================================================================
#define TQT_W4A8P_OUT(T)                                                                          \
    size_t tqt_get_m_step_##T##_mfma_gfx950(void) { return kPackW4A8MStep; }                     \
    size_t tqt_get_n_step_##T##_mfma_gfx950(void) { return kPackW4A8NStep; }                     \
    size_t tqt_get_a_packed_offset_##T##_mfma_gfx950(size_t m_idx, size_t k_idx, size_t lda,     \
                                                     size_t actual_m)                            \
    {                                                                                             \
        TQT_REQ_M(kPackW4A8MStep);                                                                \
        return packed_offset(m_idx, k_idx, lda, actual_m, kPackW4A8MStep, 1);                     \
    }                                                                                             \
    size_t tqt_get_b_packed_offset_##T##_mfma_gfx950(size_t n_idx, size_t k_idx, size_t ldb,     \
                                                     size_t actual_n)                            \
    {                                                                                             \
        TQT_REQ_N(kPackW4A8NStep);                                                                \
        TQT_REQUIRE(k_idx % 2 == 0, "k_idx % 2 == 0");                                           \
        const size_t w = actual_n < kPackW4A8NStep ? actual_n : kPackW4A8NStep;                   \
        return n_idx * (ldb / 2) + (k_idx / 2) * w;                                               \
    }                                                                                             \
    size_t tqt_get_c_offset_##T##_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldc)            \
    {                                                                                             \
        TQT_REQ_M(kPackW4A8MStep);                                                                \
        TQT_REQ_N(kPackW4A8NStep);                                                                \
        return (m_idx * ldc + n_idx) * sizeof(uint16_t);                                          \
    }                                                                                             \
    size_t tqt_get_bias_offset_##T##_mfma_gfx950(size_t n_idx)                                   \
    {                                                                                             \
        TQT_REQ_N(kPackW4A8NStep);                                                                \
        return n_idx * sizeof(uint16_t);                                                          \
    }                                                                                             \
    size_t tqt_get_d_offset_##T##_mfma_gfx950(size_t m_idx, size_t n_idx, size_t ldd)            \
    {                                                                                             \
        TQT_REQ_M(kPackW4A8MStep);                                                                \
        TQT_REQ_N(kPackW4A8NStep);                                                                \
        return (m_idx * ldd + n_idx) * sizeof(uint16_t);                                          \
    }                                                                                             \
    size_t tqt_get_d_size_##T##_mfma_gfx950(size_t m, size_t n) { return m * n * 2; }            \
    size_t tqt_get_a_packed_size_##T##_mfma_gfx950(size_t m, size_t k) { return m * k; }         \
    size_t tqt_get_b_packed_size_##T##_mfma_gfx950(size_t n, size_t k) { return n * k / 2; }     \
    void tqt_run_a_pack_##T##_mfma_gfx950_async(size_t m, size_t k, size_t lda,                  \
                                                size_t lda_packed, size_t k_idx, const void *A,   \
                                                void *A_packed, void *stream)                     \
    {                                                                                             \
        pack_nk(m, k, lda, lda_packed, k_idx, kPackW4A8MStep, kPackW4A8Chunk, 1, false, A,        \
                A_packed, stream, false, "tqt_run_a_pack_" #T "_mfma_gfx950");                    \
    }                                                                                             \
    void tqt_run_a_pack_##T##_mfma_gfx950(size_t m, size_t k, size_t lda, size_t lda_packed,      \
                                          size_t k_idx, const void *A, void *A_packed)            \
    {                                                                                             \
        pack_nk(m, k, lda, lda_packed, k_idx, kPackW4A8MStep, kPackW4A8Chunk, 1, false, A,        \
                A_packed, nullptr, true, "tqt_run_a_pack_" #T "_mfma_gfx950");                    \
    }                                                                                             \
    void tqt_run_bt_pack_##T##_mfma_gfx950_async(size_t n, size_t k, size_t ldb,                 \
                                                 size_t ldb_packed, size_t k_idx, const void *B,  \
                                                 void *B_packed, void *stream)                    \
    {                                                                                             \
        pack_nk(n, k, ldb, ldb_packed, k_idx, kPackW4A8NStep, kPackW4A8Chunk, 0, false, B,        \
                B_packed, stream, false, "tqt_run_bt_pack_" #T "_mfma_gfx950");                   \
    }                                                                                             \
    void tqt_run_bt_pack_##T##_mfma_gfx950(size_t n, size_t k, size_t ldb, size_t ldb_packed,     \
                                           size_t k_idx, const void *B, void *B_packed)           \
    {                                                                                             \
        pack_nk(n, k, ldb, ldb_packed, k_idx, kPackW4A8NStep, kPackW4A8Chunk, 0, false, B,        \
                B_packed, nullptr, true, "tqt_run_bt_pack_" #T "_mfma_gfx950");                   \
    }

TQT_W4A8P_OUT(gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp)
TQT_W4A8P_OUT(gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp)

}  // extern "C"
