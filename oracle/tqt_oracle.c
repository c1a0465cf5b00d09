/*
 * TEST INFRASTRUCTURE ONLY (see tqt_oracle.h). CPU restatement of the reference semantics of
 * the five TORQ-Tile kernel types built for gfx950. Compiled with -ffp-contract=off so that
 * every float operation written here rounds once, in the order written.
 *
 * The integer kernels keep the reference's output tiling (m_step = 4 rows by n_step = 16
 * columns, i.e. VLENB = 16 as on a VLEN = 128 core, cpp:16-20 of each reference kernel) so
 * the same code serves as the timed CPU baseline; the per-output arithmetic is independent
 * of the tiling.
 */
#include "tqt_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define TQTO_MR 4
#define TQTO_NR 16

static int g_threads = 1;

void tqto_set_threads(int n)
{
    g_threads = n < 1 ? 1 : n;
}

int tqto_get_threads(void)
{
    return g_threads;
}

/* ------------------------------------------------------------------------------------------
 * binary16 helpers
 * ---------------------------------------------------------------------------------------- */

float tqto_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    float f;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in binary32 */
        f = (float)m * 5.9604644775390625e-08f;
        return sign ? -f : f;
    }
    if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e - 15u + 127u) << 23) | (m << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

/* Round a value given as (sign, 64-bit significand `sig` with value sig * 2^exp2) to binary16,
 * nearest-even. Used for both the f32 and the f64 narrowing. */
static uint16_t round_to_f16(uint32_t sign16, uint64_t sig, int exp2)
{
    /* normalise sig so that bit 63 is set */
    if (sig == 0) {
        return (uint16_t)sign16;
    }
    while (!(sig >> 63)) {
        sig <<= 1;
        exp2 -= 1;
    }
    /* value = 1.xxx * 2^(exp2 + 63) */
    int e = exp2 + 63; /* unbiased exponent */
    uint64_t q;        /* integer result in units of the target quantum */
    int qexp;          /* quantum exponent */
    if (e >= -14) {
        qexp = e - 10; /* 11 significant bits */
    } else {
        qexp = -24; /* subnormal quantum */
    }
    int sh = qexp - exp2; /* bits to drop from sig (>= 53 for normal inputs) */
    if (sh >= 64) {
        /* everything below half a quantum unless sh == 64 handled by generic code */
        if (sh > 64) {
            return (uint16_t)sign16;
        }
        /* sh == 64: value in [2^63, 2^64) * 2^exp2 = [0.5, 1) quantum */
        q = 0;
        uint64_t half = (uint64_t)1 << 63;
        if (sig > half) {
            q = 1;
        }
        return (uint16_t)(sign16 | (uint16_t)q);
    }
    q = sig >> sh;
    uint64_t rem = sig & ((((uint64_t)1) << sh) - 1);
    uint64_t half = ((uint64_t)1) << (sh - 1);
    if (rem > half || (rem == half && (q & 1))) {
        q += 1;
    }
    if (qexp == -24) {
        /* subnormal (q may have rounded up to 0x400 = smallest normal: same encoding) */
        return (uint16_t)(sign16 | (uint16_t)q);
    }
    /* normal: q in [1024, 2048]; q == 2048 bumps the exponent */
    if (q == 2048) {
        q = 1024;
        e += 1;
    }
    if (e > 15) {
        return (uint16_t)(sign16 | 0x7c00u);
    }
    return (uint16_t)(sign16 | (uint16_t)((e + 15) << 10) | (uint16_t)(q - 1024));
}

float tqto_bf16_to_f32(uint16_t b)
{
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t tqto_f32_to_bf16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) {
        return 0x7fc0u;
    }
    /* round to nearest even on the 16 dropped bits */
    const uint32_t lsb = (x >> 16) & 1u;
    return (uint16_t)((x + 0x7fffu + lsb) >> 16);
}

uint16_t tqto_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign16 = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        if (ax > 0x7f800000u) {
            return (uint16_t)(sign16 | 0x7e00u | ((ax >> 13) & 0x3ffu));
        }
        return (uint16_t)(sign16 | 0x7c00u);
    }
    uint32_t e = ax >> 23;
    uint64_t sig = ax & 0x7fffffu;
    int exp2;
    if (e == 0) {
        exp2 = -149;
    } else {
        sig |= 0x800000u;
        exp2 = (int)e - 150;
    }
    return round_to_f16(sign16, sig, exp2);
}

static uint16_t f64_to_f16(double d)
{
    uint64_t x;
    memcpy(&x, &d, 8);
    uint32_t sign16 = (uint32_t)(x >> 48) & 0x8000u;
    uint64_t ax = x & 0x7fffffffffffffffull;
    if (ax >= 0x7ff0000000000000ull) {
        return (uint16_t)(sign16 | (ax > 0x7ff0000000000000ull ? 0x7e00u : 0x7c00u));
    }
    uint64_t e = ax >> 52;
    uint64_t sig = ax & 0xfffffffffffffull;
    int exp2;
    if (e == 0) {
        exp2 = -1074;
    } else {
        sig |= 0x10000000000000ull;
        exp2 = (int)e - 1075;
    }
    return round_to_f16(sign16, sig, exp2);
}

/* ------------------------------------------------------------------------------------------
 * Requantization multiplier: src/gemm/gemm_i8_i8/tqt_utils_i8_i8.h:16-132
 * ---------------------------------------------------------------------------------------- */

static int64_t integer_from_exp(double input, int32_t *shift)
{
    /* tqt_utils_i8_i8.h:16-91: Q31 fraction from the double's bits, frexp exponent convention */
    uint64_t u;
    memcpy(&u, &input, 8);
    const uint64_t sign_mask = 0x8000000000000000ull;
    if ((u & ~sign_mask) == 0) {
        *shift = 0;
        return 0;
    }
    const uint32_t exponent_part = (uint32_t)((u & 0x7ff0000000000000ull) >> 52);
    if (exponent_part == 0x7ffu) {
        *shift = 0x7fffffff;
        if (u & 0x000fffffffc00000ull) {
            return 0;
        }
        return (u & sign_mask) ? (int64_t)0x8000000000000000ull : (int64_t)0x7fffffffffffffffll;
    }
    *shift = (int32_t)(exponent_part - 1023u) + 1;
    int64_t fraction = 0x40000000 + (int64_t)((u & 0x000fffffffc00000ull) >> 22);
    if ((u & 0x003fffffull) > 0x00200000ull) {
        fraction += 1;
    }
    if (u & sign_mask) {
        fraction *= -1;
    }
    return fraction;
}

void tqto_quantize_multiplier(double x, int32_t *mult, int32_t *shift)
{
    /* tqt_utils_i8_i8.h:98-132 */
    if (x == 0.) {
        *mult = 0;
        *shift = 0;
        return;
    }
    int64_t q = integer_from_exp(x, shift);
    if (q == (1ll << 31)) {
        q /= 2;
        ++*shift;
    }
    if (*shift < -31) {
        *shift = 0;
        q = 0;
    }
    *mult = (int32_t)q;
}

/* Per-column (mult, stored shift) exactly as the run functions build their VLAs
 * (…qsi8cxt_4x1vl_rvv.cpp:158-176; igemmcl …cpp:233-251). */
static void column_multiplier(float scale_a, const float *scale_b, int32_t quant_channel_b,
                              float scale_d, size_t j, int32_t *mult, int32_t *shift)
{
    size_t src = (quant_channel_b == 1) ? 0 : j;
    double real_scale = (double)scale_a * (double)scale_b[src] / (double)scale_d;
    tqto_quantize_multiplier(real_scale, mult, shift);
    *shift = -*shift - 1;
}

int8_t tqto_requant_one(int32_t acc, int32_t mult, int32_t shift, int32_t zp, int8_t cmin,
                        int8_t cmax)
{
    /* vmulh.vv: high 32 bits of the signed 64-bit product (floor division by 2^32) */
    int64_t prod = (int64_t)acc * (int64_t)mult;
    int32_t y = (int32_t)(prod >> 32);
    /* vsra.vv: arithmetic shift by the low 5 bits of the shift operand */
    y = y >> (shift & 31);
    /* vadd.vx: 32-bit wrapping add of the output zero point */
    y = (int32_t)((uint32_t)y + (uint32_t)zp);
    /* vnclip.wx twice with shift 0: saturate to int16, then to int8 */
    if (y > 32767) {
        y = 32767;
    }
    if (y < -32768) {
        y = -32768;
    }
    if (y > 127) {
        y = 127;
    }
    if (y < -128) {
        y = -128;
    }
    /* clamp_i8: vmax.vx then vmin.vx (tqt_kernel_gemm_i8_i8_4x1vl_rvv.h:231-259) */
    int8_t r = (int8_t)y;
    if (r < cmin) {
        r = cmin;
    }
    if (r > cmax) {
        r = cmax;
    }
    return r;
}

/* ------------------------------------------------------------------------------------------
 * Tile iteration helper: every kernel below walks (m_step, n_step) tiles like the reference
 * run functions; OpenMP splits tiles across threads when tqto_set_threads(n > 1).
 * ---------------------------------------------------------------------------------------- */

#define TILE_LOOP_BEGIN(m, n)                                                        \
    {                                                                                \
        const long n_mt = (long)(((m) + TQTO_MR - 1) / TQTO_MR);                     \
        const long n_nt = (long)(((n) + TQTO_NR - 1) / TQTO_NR);                     \
        const long n_tiles = n_mt * n_nt;                                            \
        _Pragma("omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)") \
        for (long t = 0; t < n_tiles; ++t) {                                         \
            const size_t m0 = (size_t)(t / n_nt) * TQTO_MR;                          \
            const size_t n0 = (size_t)(t % n_nt) * TQTO_NR;                          \
            const size_t mr = ((m) - m0) < TQTO_MR ? ((m) - m0) : TQTO_MR;           \
            const size_t nr = ((n) - n0) < TQTO_NR ? ((n) - n0) : TQTO_NR;

#define TILE_LOOP_END \
    }                 \
    }

void tqto_gemm_clamp_i32_i8_i8(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                               const int8_t *B, size_t ldb, const int32_t *C, size_t ldc,
                               int32_t *D, size_t ldd, int32_t cmin, int32_t cmax)
{
    /* …gemm_clamp_i32_i8_i8_4x1vl_rvv.cpp:71-101: init from C or 0, per-k row of B times an
     * A scalar (i8*i8 exact in i16, widened into i32), then vmax(cmin), vmin(cmax). */
    TILE_LOOP_BEGIN(m, n)
    uint32_t acc[TQTO_MR][TQTO_NR];
    for (size_t i = 0; i < mr; ++i) {
        for (size_t j = 0; j < nr; ++j) {
            acc[i][j] = C ? (uint32_t)C[(m0 + i) * ldc + n0 + j] : 0u;
        }
    }
    for (size_t kk = 0; kk < k; ++kk) {
        const int8_t *brow = B + kk * ldb + n0;
        for (size_t i = 0; i < mr; ++i) {
            const int32_t a = A[(m0 + i) * lda + kk];
            for (size_t j = 0; j < nr; ++j) {
                acc[i][j] += (uint32_t)(int32_t)(int16_t)(a * brow[j]);
            }
        }
    }
    for (size_t i = 0; i < mr; ++i) {
        for (size_t j = 0; j < nr; ++j) {
            int32_t v = (int32_t)acc[i][j];
            v = v > cmin ? v : cmin;
            v = v < cmax ? v : cmax;
            D[(m0 + i) * ldd + n0 + j] = v;
        }
    }
    TILE_LOOP_END
}

void tqto_gemm_qsi8cxt_acc(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                           const int8_t *B, size_t ldb, const int32_t *C, size_t ldc,
                           const int32_t *bias, int32_t *out, size_t ldout)
{
    /* …qsi8cxt_4x1vl_rvv.cpp:86-113 (+ add_1xnbias, tqt_kernel_gemm_i8_i8_4x1vl_rvv.h:154-175):
     * acc = (C or 0) + sum_k A[m,k]*B[n,k] + bias[n], all int32 with wrap-around. */
    TILE_LOOP_BEGIN(m, n)
    uint32_t acc[TQTO_MR][TQTO_NR];
    for (size_t i = 0; i < mr; ++i) {
        for (size_t j = 0; j < nr; ++j) {
            acc[i][j] = C ? (uint32_t)C[(m0 + i) * ldc + n0 + j] : 0u;
        }
    }
    for (size_t i = 0; i < mr; ++i) {
        const int8_t *arow = A + (m0 + i) * lda;
        for (size_t j = 0; j < nr; ++j) {
            const int8_t *brow = B + (n0 + j) * ldb;
            int32_t s = 0;
            for (size_t kk = 0; kk < k; ++kk) {
                s += (int32_t)arow[kk] * (int32_t)brow[kk];
            }
            acc[i][j] += (uint32_t)s;
        }
    }
    for (size_t i = 0; i < mr; ++i) {
        for (size_t j = 0; j < nr; ++j) {
            uint32_t v = acc[i][j];
            if (bias) {
                v += (uint32_t)bias[n0 + j];
            }
            out[(m0 + i) * ldout + n0 + j] = (int32_t)v;
        }
    }
    TILE_LOOP_END
}

void tqto_gemm_qai8_qai8_qsi8cxt(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                                 const int8_t *B, size_t ldb, const int32_t *C, size_t ldc,
                                 int8_t *D, size_t ldd, const int32_t *bias, int8_t cmin,
                                 int8_t cmax, float scale_a, const float *scale_b,
                                 int32_t quant_channel_b, float scale_d, int32_t zero_point_d)
{
    /* …qsi8cxt_4x1vl_rvv.cpp:140-198 */
    TILE_LOOP_BEGIN(m, n)
    int32_t mult[TQTO_NR], shift[TQTO_NR];
    for (size_t j = 0; j < nr; ++j) {
        column_multiplier(scale_a, scale_b, quant_channel_b, scale_d, n0 + j, &mult[j],
                          &shift[j]);
    }
    int32_t acc[TQTO_MR * TQTO_NR];
    /* single-tile accumulate, written into a local tile (ldout = TQTO_NR) */
    {
        for (size_t i = 0; i < mr; ++i) {
            const int8_t *arow = A + (m0 + i) * lda;
            for (size_t j = 0; j < nr; ++j) {
                const int8_t *brow = B + (n0 + j) * ldb;
                uint32_t v = C ? (uint32_t)C[(m0 + i) * ldc + n0 + j] : 0u;
                int32_t s = 0;
                for (size_t kk = 0; kk < k; ++kk) {
                    s += (int32_t)arow[kk] * (int32_t)brow[kk];
                }
                v += (uint32_t)s;
                if (bias) {
                    v += (uint32_t)bias[n0 + j];
                }
                acc[i * TQTO_NR + j] = (int32_t)v;
            }
        }
    }
    for (size_t i = 0; i < mr; ++i) {
        for (size_t j = 0; j < nr; ++j) {
            D[(m0 + i) * ldd + n0 + j] = tqto_requant_one(acc[i * TQTO_NR + j], mult[j], shift[j],
                                                          zero_point_d, cmin, cmax);
        }
    }
    TILE_LOOP_END
}

void tqto_gemm_qai8dx_qsi4cxt_f32(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                                  const uint8_t *B, size_t ldb, const float *C, size_t ldc,
                                  float *D, size_t ldd, const float *bias, float cmin, float cmax,
                                  const float *scale_a, const int32_t *zero_point_a,
                                  const float *scale_b)
{
    /* …qai8dx_qsi4cxt_4x1vl_rvv.cpp:81-138 with tqt_kernel_gemm_i8_i4_4x1vl_rvv.h:
     *   dequant_bt :77-93 (lo = (b & 15) - 8 is the even k, hi = (b >> 4) - 8 the odd k),
     *   accum_rsum_b :139-146, vmacc_lo/hi :152-224, apply_zp_correction :234-259,
     *   dequant_acc_to_f32 :271-301 (vfcvt RNE, * scale_a, * scale_b), add_c_f32 :331-367,
     *   add_1xnbias_f32 :307-323, clamp_f32 :373-397 (vfmax then vfmin). */
    const size_t bstride = ldb / 2;
    TILE_LOOP_BEGIN(m, n)
    for (size_t j = 0; j < nr; ++j) {
        const uint8_t *brow = B + (n0 + j) * bstride;
        int32_t rsum = 0;
        uint32_t acc[TQTO_MR] = {0, 0, 0, 0};
        for (size_t kk = 0; kk < k; kk += 2) {
            const uint8_t byte = brow[kk / 2];
            const int32_t lo = (int32_t)(byte & 0xf) - 8;
            const int32_t hi = (int32_t)(byte >> 4) - 8;
            rsum += lo + hi;
            for (size_t i = 0; i < mr; ++i) {
                const int8_t *arow = A + (m0 + i) * lda;
                acc[i] += (uint32_t)((int32_t)arow[kk] * lo);
                acc[i] += (uint32_t)((int32_t)arow[kk + 1] * hi);
            }
        }
        for (size_t i = 0; i < mr; ++i) {
            const size_t mi = m0 + i;
            int32_t v = (int32_t)(acc[i] - (uint32_t)zero_point_a[mi] * (uint32_t)rsum);
            float f = (float)v;
            f = f * scale_a[mi];
            f = f * scale_b[n0 + j];
            if (C) {
                f = f + C[mi * ldc + n0 + j];
            }
            if (bias) {
                f = f + bias[n0 + j];
            }
            f = fmaxf(f, cmin);
            f = fminf(f, cmax);
            D[mi * ldd + n0 + j] = f;
        }
    }
    TILE_LOOP_END
}

void tqto_gemm_qai8dx_qsi4cxt_h16(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                                  const uint8_t *B, size_t ldb, const uint16_t *C, size_t ldc,
                                  uint16_t *D, size_t ldd, const uint16_t *bias, uint16_t cmin,
                                  uint16_t cmax, const float *scale_a,
                                  const int32_t *zero_point_a, const float *scale_b, int out_bf16)
{
    /* …_{f16,bf16}_qai8dx_qsi4cxt_4x1vl_rvv.cpp gemm_kernel: the f32 path of
     * tqto_gemm_qai8dx_qsi4cxt_f32 on widened C / bias / clamps (vfwcvt / vfwcvtbf16 are exact),
     * then tqt_store_narrow_{f16,bf16}_kernel (vfncvt.f.f.w / vfncvtbf16.f.f.w, RNE). */
    float (*widen)(uint16_t) = out_bf16 ? tqto_bf16_to_f32 : tqto_f16_to_f32;
    float *C32 = NULL, *bias32 = NULL;
    float *D32 = (float *)malloc(m * n * sizeof(float));
    if (C) {
        C32 = (float *)malloc(m * n * sizeof(float));
        for (size_t i = 0; i < m; ++i) {
            for (size_t j = 0; j < n; ++j) {
                C32[i * n + j] = widen(C[i * ldc + j]);
            }
        }
    }
    if (bias) {
        bias32 = (float *)malloc(n * sizeof(float));
        for (size_t j = 0; j < n; ++j) {
            bias32[j] = widen(bias[j]);
        }
    }
    tqto_gemm_qai8dx_qsi4cxt_f32(m, n, k, A, lda, B, ldb, C32, n, D32, n, bias32, widen(cmin),
                                 widen(cmax), scale_a, zero_point_a, scale_b);
    for (size_t i = 0; i < m; ++i) {
        for (size_t j = 0; j < n; ++j) {
            const float f = D32[i * n + j];
            uint16_t h;
            if (out_bf16) {
                h = tqto_f32_to_bf16(f);
            } else {
                h = f != f ? (uint16_t)0x7e00u : tqto_f32_to_f16(f);
            }
            D[i * ldd + j] = h;
        }
    }
    free(D32);
    free(C32);
    free(bias32);
}

/* The k loop of test/common/reference_gemm.cpp:148-164 for output (i, j), starting from acc:
 * acc += f32(A) * (f32(q - 8) * f32(scale)) in k order, each product and sum rounded. */
static float w4a16_dot(float acc, const uint16_t *arow, const uint8_t *brow,
                       const uint16_t *srow, size_t k, size_t bl)
{
    for (size_t p = 0; p < k; ++p) {
        const float a_val = tqto_f16_to_f32(arow[p]);
        const uint8_t byte_val = brow[p / 2];
        const int32_t b_raw =
            (p % 2 == 0) ? (int32_t)(byte_val & 0x0f) - 8 : (int32_t)(byte_val >> 4) - 8;
        const float scale_val = tqto_f16_to_f32(srow[p / bl]);
        const float b_dequant = (float)b_raw * scale_val;
        const float prod = a_val * b_dequant;
        acc = acc + prod;
    }
    return acc;
}

void tqto_gemm_f16_qsi4c2t_f32acc(size_t m, size_t n, size_t k, size_t bl, const uint16_t *A,
                                  size_t lda, const uint8_t *B, size_t ldb,
                                  const uint16_t *scale_b, size_t ldsb, const uint16_t *C,
                                  size_t ldc, uint16_t *D, size_t ldd, const uint16_t *bias,
                                  uint16_t cmin, uint16_t cmax)
{
    /* test/common/reference_gemm.cpp:132-179 (TA = TD = float16_t, BiasMode k1xN). */
    const size_t brow_bytes = ldb / 2;
    const float cminf = tqto_f16_to_f32(cmin);
    const float cmaxf = tqto_f16_to_f32(cmax);
    TILE_LOOP_BEGIN(m, n)
    for (size_t i = m0; i < m0 + mr; ++i) {
        for (size_t j = n0; j < n0 + nr; ++j) {
            float acc = C ? tqto_f16_to_f32(C[i * ldc + j]) : 0.0f;
            acc = w4a16_dot(acc, A + i * lda, B + j * brow_bytes, scale_b + j * ldsb, k, bl);
            if (bias) {
                acc = acc + tqto_f16_to_f32(bias[j]);
            }
            acc = (acc < cminf) ? cminf : acc; /* std::max(acc, clamp_min) */
            acc = (cmaxf < acc) ? cmaxf : acc; /* std::min(acc, clamp_max) */
            D[i * ldd + j] = tqto_f32_to_f16(acc);
        }
    }
    TILE_LOOP_END
}

void tqto_gemm_f16_qsi4c2t_f32out(size_t m, size_t n, size_t k, size_t bl, const uint16_t *A,
                                  size_t lda, const uint8_t *B, size_t ldb,
                                  const uint16_t *scale_b, size_t ldsb, const float *C, size_t ldc,
                                  float *D, size_t ldd, const float *bias, float cmin, float cmax)
{
    /* test/common/reference_gemm.cpp:132-179 (TA = float16_t, TD = float, BiasMode k1xN): the
     * oracle the reference test holds gemm_1xnbias_clamp_f32_f16_qsi4c2t to
     * (test/common/quantized_gemm_test_runner.h:1092-1095). */
    const size_t brow_bytes = ldb / 2;
    TILE_LOOP_BEGIN(m, n)
    for (size_t i = m0; i < m0 + mr; ++i) {
        for (size_t j = n0; j < n0 + nr; ++j) {
            float acc = C ? C[i * ldc + j] : 0.0f;
            acc = w4a16_dot(acc, A + i * lda, B + j * brow_bytes, scale_b + j * ldsb, k, bl);
            if (bias) {
                acc = acc + bias[j];
            }
            acc = (acc < cmin) ? cmin : acc; /* std::max(acc, clamp_min) */
            acc = (cmax < acc) ? cmax : acc; /* std::min(acc, clamp_max) */
            D[i * ldd + j] = acc;
        }
    }
    TILE_LOOP_END
}

/* exact binary16 fused multiply-add, rounded once (the products and sums below are exact in
 * binary64 for every operand magnitude this test data reaches) */
static uint16_t f16_fma(uint16_t a, uint16_t b, uint16_t c)
{
    const double r = (double)tqto_f16_to_f32(a) * (double)tqto_f16_to_f32(b) +
                     (double)tqto_f16_to_f32(c);
    return f64_to_f16(r);
}

static uint16_t f16_mul(uint16_t a, uint16_t b)
{
    return f64_to_f16((double)tqto_f16_to_f32(a) * (double)tqto_f16_to_f32(b));
}

static uint16_t f16_add(uint16_t a, uint16_t b)
{
    return f64_to_f16((double)tqto_f16_to_f32(a) + (double)tqto_f16_to_f32(b));
}

uint16_t tqto_f16_add(uint16_t a, uint16_t b)
{
    return f16_add(a, b);
}

/* ------------------------------------------------------------------------------------------
 * W8A8 with dynamic per-row activation quantization (qai8dx x qsi8cx -> f32 / f16):
 * src/gemm/gemm_i8_i8/tqt_kernel_gemm_qai8dx_qsi8cx_4x1vl_rvv.h
 * ---------------------------------------------------------------------------------------- */

/* RISC-V vfmax / vfmin (IEEE 754-2019 maximumNumber / minimumNumber): a NaN operand yields the
 * other one (the canonical NaN 0x7fc00000 if both are NaN), and -0 orders below +0. */
static float canonical_nan_f32(void)
{
    const uint32_t u = 0x7fc00000u;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float rv_fmax(float a, float b)
{
    if (a != a) {
        return b != b ? canonical_nan_f32() : b;
    }
    if (b != b) {
        return a;
    }
    if (a == b) {
        return signbit(a) ? b : a;
    }
    return a > b ? a : b;
}

static float rv_fmin(float a, float b)
{
    if (a != a) {
        return b != b ? canonical_nan_f32() : b;
    }
    if (b != b) {
        return a;
    }
    if (a == b) {
        return signbit(a) ? a : b;
    }
    return a < b ? a : b;
}

/* The k loop (vwmacc_zp :95-140): each A byte is loaded, zero_point_a is subtracted in a
 * scalar register, and vwmacc.vx at SEW=16 uses the low 16 bits of that difference, so
 * acc = sum_k int16(q_a - zp_a) * q_b, accumulated in int32 with wrap-around. */
static int32_t dyn_acc(const int8_t *arow, const int8_t *brow, size_t k, int32_t zp)
{
    uint32_t acc = 0;
    for (size_t p = 0; p < k; ++p) {
        const uint32_t d = (uint32_t)((int32_t)arow[p]) - (uint32_t)zp;
        const int32_t a16 = (int32_t)(int16_t)(uint16_t)(d & 0xffffu);
        acc += (uint32_t)(a16 * (int32_t)brow[p]);
    }
    return (int32_t)acc;
}

void tqto_gemm_qai8dx_qsi8cxt_f32(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                                  const int8_t *B, size_t ldb, float *D, size_t ldd,
                                  const float *bias, float cmin, float cmax,
                                  const float *scale_a, const int32_t *zero_point_a,
                                  const float *scale_b)
{
    /* dequant_fp32 :145-215: vfcvt.f.x (RNE), sigma = scale_b * scale_a, f * sigma, + bias
     * (a zero vector when bias is NULL), vfmax cmin, vfmin cmax. */
    TILE_LOOP_BEGIN(m, n)
    for (size_t i = m0; i < m0 + mr; ++i) {
        for (size_t j = n0; j < n0 + nr; ++j) {
            const int32_t acc = dyn_acc(A + i * lda, B + j * ldb, k, zero_point_a[i]);
            const float sigma = scale_b[j] * scale_a[i];
            float f = (float)acc * sigma;
            f = f + (bias ? bias[j] : 0.0f);
            f = rv_fmax(f, cmin);
            f = rv_fmin(f, cmax);
            D[i * ldd + j] = f;
        }
    }
    TILE_LOOP_END
}

/* -0 orders below +0 and a NaN operand yields the other, on binary16 patterns. */
static uint16_t rv_hmax(uint16_t a, uint16_t b)
{
    return tqto_f32_to_f16(rv_fmax(tqto_f16_to_f32(a), tqto_f16_to_f32(b)));
}

static uint16_t rv_hmin(uint16_t a, uint16_t b)
{
    return tqto_f32_to_f16(rv_fmin(tqto_f16_to_f32(a), tqto_f16_to_f32(b)));
}

static uint16_t canon_f16(uint16_t h)
{
    return ((h & 0x7fffu) > 0x7c00u) ? (uint16_t)0x7e00u : h;
}

void tqto_gemm_qai8dx_qsi8cxt_f16(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                                  const int8_t *B, size_t ldb, uint16_t *D, size_t ldd,
                                  const uint16_t *bias, uint16_t cmin, uint16_t cmax,
                                  const float *scale_a, const int32_t *zero_point_a,
                                  const float *scale_b)
{
    /* dequant_fp16 :217-330: the f32 product f32(acc) * sigma is narrowed to f16 (vfncvt.f.f.w,
     * RNE), the f16 bias (or a zero vector) is added in f16 (one rounding), then vfmax / vfmin
     * with the f16 bounds. RISC-V arithmetic returns the canonical NaN 0x7e00. */
    TILE_LOOP_BEGIN(m, n)
    for (size_t i = m0; i < m0 + mr; ++i) {
        for (size_t j = n0; j < n0 + nr; ++j) {
            const int32_t acc = dyn_acc(A + i * lda, B + j * ldb, k, zero_point_a[i]);
            const float sigma = scale_b[j] * scale_a[i];
            const float f = (float)acc * sigma;
            uint16_t h = canon_f16(tqto_f32_to_f16(f));
            h = canon_f16(f16_add(h, bias ? bias[j] : (uint16_t)0));
            h = canon_f16(rv_hmax(h, cmin));
            h = canon_f16(rv_hmin(h, cmax));
            D[i * ldd + j] = h;
        }
    }
    TILE_LOOP_END
}

void tqto_gemm_f16_qsi4c2t_rvv(size_t m, size_t n, size_t k, size_t bl, const uint16_t *A,
                               size_t lda, const uint8_t *B, size_t ldb, const uint16_t *scale_b,
                               size_t ldsb, const uint16_t *C, size_t ldc, uint16_t *D,
                               size_t ldd, const uint16_t *bias, uint16_t cmin, uint16_t cmax)
{
    /* tqt_kernel_gemm_f16_i4_8x2vl_rvv.h: init_c :99-164 (or zero), per block load_scale
     * :170-190, dequant_bt :199-260 (vfcvt i16->f16 exact, vfmul f16 rounds), vfmacc :364-478
     * (f16 fused multiply-add in k order), add_1xnbias :484-545 (f16 add), clamp :551-646
     * (vfmax then vfmin). */
    const size_t brow_bytes = ldb / 2;
    const float cminf = tqto_f16_to_f32(cmin);
    const float cmaxf = tqto_f16_to_f32(cmax);
    TILE_LOOP_BEGIN(m, n)
    for (size_t i = m0; i < m0 + mr; ++i) {
        for (size_t j = n0; j < n0 + nr; ++j) {
            uint16_t acc = C ? C[i * ldc + j] : (uint16_t)0;
            for (size_t p = 0; p < k; ++p) {
                const uint8_t byte_val = B[j * brow_bytes + p / 2];
                const int32_t q =
                    (p % 2 == 0) ? (int32_t)(byte_val & 0x0f) - 8 : (int32_t)(byte_val >> 4) - 8;
                const uint16_t wq = tqto_f32_to_f16((float)q);
                const uint16_t w = f16_mul(wq, scale_b[j * ldsb + p / bl]);
                acc = f16_fma(A[i * lda + p], w, acc);
            }
            if (bias) {
                acc = f16_add(acc, bias[j]);
            }
            float v = tqto_f16_to_f32(acc);
            v = fmaxf(v, cminf);
            v = fminf(v, cmaxf);
            D[i * ldd + j] = tqto_f32_to_f16(v);
        }
    }
    TILE_LOOP_END
}

/* ------------------------------------------------------------------------------------------
 * Convolution
 * ---------------------------------------------------------------------------------------- */

void tqto_im2col_cl_i8(size_t group_idx, const int8_t *input, int8_t *col,
                       const struct tqto_conv_params *p)
{
    /* src/common/tqt_conv.h:131-202: row = output pixel (od, oh, ow); columns ordered
     * (kd, kh, kw, ic); out-of-bounds taps are zero-filled. */
    const size_t ID = p->input_shape[0], IH = p->input_shape[1], IW = p->input_shape[2];
    const size_t OD = p->output_shape[0], OH = p->output_shape[1], OW = p->output_shape[2];
    const size_t KD = p->kernel_shape[0], KH = p->kernel_shape[1], KW = p->kernel_shape[2];
    const size_t ICg = p->input_channel / p->groups;
    const size_t Kc = KD * KH * KW * ICg;
    size_t row = 0;
    for (size_t od = 0; od < OD; ++od) {
        for (size_t oh = 0; oh < OH; ++oh) {
            for (size_t ow = 0; ow < OW; ++ow) {
                size_t cc = 0;
                for (size_t kd = 0; kd < KD; ++kd) {
                    const long id = (long)(od * p->stride[0] + kd * p->dilation[0]) - (long)p->pad[0];
                    for (size_t kh = 0; kh < KH; ++kh) {
                        const long ih =
                            (long)(oh * p->stride[1] + kh * p->dilation[1]) - (long)p->pad[1];
                        for (size_t kw = 0; kw < KW; ++kw) {
                            const long iw =
                                (long)(ow * p->stride[2] + kw * p->dilation[2]) - (long)p->pad[2];
                            int8_t *dst = col + row * Kc + cc;
                            if (id >= 0 && id < (long)ID && ih >= 0 && ih < (long)IH && iw >= 0 &&
                                iw < (long)IW) {
                                memcpy(dst,
                                       input + (((size_t)id * IH + (size_t)ih) * IW + (size_t)iw) *
                                                   p->input_channel +
                                           group_idx * ICg,
                                       ICg);
                            } else {
                                memset(dst, 0, ICg);
                            }
                            cc += ICg;
                        }
                    }
                }
                row++;
            }
        }
    }
}

void tqto_im2col_cf_i8(size_t group_idx, const int8_t *input, int8_t *col,
                       const struct tqto_conv_params *p)
{
    /* src/common/tqt_conv.h:51-119: channel-first (NCDHW) input; row = (ic, kd, kh, kw) of the
     * group, column = output pixel (od, oh, ow); out-of-bounds taps are zero. */
    const size_t ID = p->input_shape[0], IH = p->input_shape[1], IW = p->input_shape[2];
    const size_t OD = p->output_shape[0], OH = p->output_shape[1], OW = p->output_shape[2];
    const size_t KD = p->kernel_shape[0], KH = p->kernel_shape[1], KW = p->kernel_shape[2];
    const size_t ICg = p->input_channel / p->groups;
    const size_t N = OD * OH * OW;
    const int8_t *in = input + group_idx * ICg * ID * IH * IW;
    size_t row = 0;
    for (size_t ic = 0; ic < ICg; ++ic) {
        for (size_t kd = 0; kd < KD; ++kd) {
            for (size_t kh = 0; kh < KH; ++kh) {
                for (size_t kw = 0; kw < KW; ++kw) {
                    size_t colj = 0;
                    for (size_t od = 0; od < OD; ++od) {
                        const long id =
                            (long)(od * p->stride[0] + kd * p->dilation[0]) - (long)p->pad[0];
                        for (size_t oh = 0; oh < OH; ++oh) {
                            const long ih =
                                (long)(oh * p->stride[1] + kh * p->dilation[1]) - (long)p->pad[1];
                            for (size_t ow = 0; ow < OW; ++ow) {
                                const long iw = (long)(ow * p->stride[2] + kw * p->dilation[2]) -
                                                (long)p->pad[2];
                                int8_t v = 0;
                                if (id >= 0 && id < (long)ID && ih >= 0 && ih < (long)IH &&
                                    iw >= 0 && iw < (long)IW) {
                                    v = in[ic * ID * IH * IW + ((size_t)id * IH + (size_t)ih) * IW +
                                           (size_t)iw];
                                }
                                col[row * N + colj] = v;
                                colj++;
                            }
                        }
                    }
                    row++;
                }
            }
        }
    }
}

void tqto_gemm_mx1bias_qsi8dx(size_t m, size_t n, size_t k, const int8_t *A, size_t lda,
                              const int8_t *B, size_t ldb, const int32_t *C, size_t ldc,
                              int8_t *D, size_t ldd, const int32_t *bias, int8_t cmin,
                              int8_t cmax, const float *scale_a, int32_t quant_channel_a,
                              float scale_b, float scale_d, int32_t zp_d)
{
    /* src/gemm/gemm_i8_i8/gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8/…_4x1vl_rvv.cpp:
     * per-row multiplier from scale_a[i] * scale_b / scale_d (row 0's for all rows when
     * quant_channel_a == 1), shift = -shift - 1 (:150-166); acc = C (or 0) + sum_k A[i,k]*B[k,j]
     * in wrapping int32 (kernel :100-112, B [k, n] with row stride ldb), + bias[i]
     * (add_mx1bias), then the requantization and clamp of the W8A8 kernels. */
    for (size_t i = 0; i < m; ++i) {
        const size_t src = (quant_channel_a == 1) ? 0 : i;
        int32_t mult, shift;
        const double real_scale = (double)scale_a[src] * (double)scale_b / (double)scale_d;
        tqto_quantize_multiplier(real_scale, &mult, &shift);
        shift = -shift - 1;
        for (size_t j = 0; j < n; ++j) {
            uint32_t acc = C ? (uint32_t)C[i * ldc + j] : 0u;
            for (size_t p = 0; p < k; ++p) {
                acc += (uint32_t)((int32_t)A[i * lda + p] * (int32_t)B[p * ldb + j]);
            }
            if (bias) {
                acc += (uint32_t)bias[i];
            }
            D[i * ldd + j] = tqto_requant_one((int32_t)acc, mult, shift, zp_d, cmin, cmax);
        }
    }
}

void tqto_igemmcf_qsi8dx(size_t m, size_t n, const int8_t *input, size_t group_idx,
                         size_t n_idx, const int8_t *A, size_t lda, int8_t *D, size_t ldd,
                         const int32_t *bias, int8_t cmin, int8_t cmax,
                         const struct tqto_conv_params *p, const float *scale_a,
                         int32_t quant_channel_a, float scale_b, float scale_d, int32_t zp_d)
{
    /* src/conv/igemm_i8_i8/igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8/…_1vlx4_rvv.cpp
     * run_igemm: output channels m (rows of the weights A [m, K]) times output pixels
     * [n_idx, n_idx + n) of the channel-first im2col, C ignored, D rows at D + i * ldd + pixel:
     * the mx1bias GEMM on columns n_idx.. of the full channel-first im2col. */
    const size_t ICg = p->input_channel / p->groups;
    const size_t K = ICg * p->kernel_shape[0] * p->kernel_shape[1] * p->kernel_shape[2];
    const size_t N = p->output_shape[0] * p->output_shape[1] * p->output_shape[2];
    int8_t *col = (int8_t *)malloc((K * N) > 0 ? K * N : 1);
    tqto_im2col_cf_i8(group_idx, input, col, p);
    tqto_gemm_mx1bias_qsi8dx(m, n, K, A, lda, col + n_idx, N, NULL, 0, D + n_idx, ldd, bias, cmin,
                             cmax, scale_a, quant_channel_a, scale_b, scale_d, zp_d);
    free(col);
}

void tqto_igemmcl_qsi8cxt(size_t m, size_t n, const int8_t *input, size_t group_idx,
                          size_t m_idx, const int8_t *B, size_t ldb, int8_t *D, size_t ldd,
                          const int32_t *bias, int8_t cmin, int8_t cmax,
                          const struct tqto_conv_params *p, float scale_a, const float *scale_b,
                          int32_t quant_channel_b, float scale_d, int32_t zero_point_d)
{
    /* …igemmcl…qsi8cxt_4x1vl_rvv.cpp:81-151 (kernel) and :194-286 (run): output pixel
     * g = m_idx + i decomposes as od = g/(OH*OW), oh = (g/OW)%OH, ow = g%OW; the k loop runs
     * kd, kh, kw, ic with the weight pointer advancing by one per step; out-of-bounds
     * pixels contribute 0; then bias, requantize, clamp; D[g * ldd + j]. */
    const size_t ID = p->input_shape[0], IH = p->input_shape[1], IW = p->input_shape[2];
    const size_t OH = p->output_shape[1], OW = p->output_shape[2];
    const size_t KD = p->kernel_shape[0], KH = p->kernel_shape[1], KW = p->kernel_shape[2];
    const size_t ICg = p->input_channel / p->groups;
    const int8_t *in_g = input + group_idx * ICg;
    TILE_LOOP_BEGIN(m, n)
    int32_t mult[TQTO_NR], shift[TQTO_NR];
    for (size_t j = 0; j < nr; ++j) {
        column_multiplier(scale_a, scale_b, quant_channel_b, scale_d, n0 + j, &mult[j],
                          &shift[j]);
    }
    for (size_t i = 0; i < mr; ++i) {
        const size_t gp = m_idx + m0 + i;
        const long od = (long)(gp / (OH * OW));
        const long oh = (long)((gp / OW) % OH);
        const long ow = (long)(gp % OW);
        for (size_t j = 0; j < nr; ++j) {
            const int8_t *w = B + (n0 + j) * ldb;
            uint32_t acc = 0;
            for (size_t kd = 0; kd < KD; ++kd) {
                const long id = od * (long)p->stride[0] + (long)(kd * p->dilation[0]) - (long)p->pad[0];
                for (size_t kh = 0; kh < KH; ++kh) {
                    const long ih =
                        oh * (long)p->stride[1] + (long)(kh * p->dilation[1]) - (long)p->pad[1];
                    for (size_t kw = 0; kw < KW; ++kw) {
                        const long iw =
                            ow * (long)p->stride[2] + (long)(kw * p->dilation[2]) - (long)p->pad[2];
                        const int inb = id >= 0 && id < (long)ID && ih >= 0 && ih < (long)IH &&
                                        iw >= 0 && iw < (long)IW;
                        const int8_t *src =
                            inb ? in_g + (((size_t)id * IH + (size_t)ih) * IW + (size_t)iw) *
                                             p->input_channel
                                : NULL;
                        for (size_t ic = 0; ic < ICg; ++ic) {
                            const int32_t a = src ? (int32_t)src[ic] : 0;
                            acc += (uint32_t)(a * (int32_t)w[ic]);
                        }
                        w += ICg;
                    }
                }
            }
            if (bias) {
                acc += (uint32_t)bias[n0 + j];
            }
            D[gp * ldd + n0 + j] =
                tqto_requant_one((int32_t)acc, mult[j], shift[j], zero_point_d, cmin, cmax);
        }
    }
    TILE_LOOP_END
}

/* ------------------------------------------------------------------------------------------
 * Caller-side input preparation (reference test harness)
 * ---------------------------------------------------------------------------------------- */

int8_t tqto_quantize_i8(float val, float scale, int32_t zp)
{
    /* test/common/test_common.h:232-240 */
    float q = nearbyintf(val / scale) + (float)zp;
    if (q > 127.0f) {
        q = 127.0f;
    }
    if (q < -128.0f) {
        q = -128.0f;
    }
    return (int8_t)q;
}

int32_t tqto_quantize_bias_i32(float val, float input_scale)
{
    /* test/common/test_common.h:268-277 */
    float q = nearbyintf(val / input_scale);
    if (q > 2147483647.0f) {
        q = 2147483647.0f;
    }
    if (q < -2147483648.0f) {
        q = -2147483648.0f;
    }
    if (q >= 2147483648.0f) {
        return 2147483647; /* 2147483647.0f rounds to 2^31 in binary32 */
    }
    return (int32_t)q;
}

void tqto_fuse_zp_to_bias(int32_t *fused, const int32_t *bias, const int8_t *data, int32_t zp,
                          size_t channels, size_t channel_size)
{
    /* test/common/test_common.h:280-290 */
    for (size_t ch = 0; ch < channels; ++ch) {
        int32_t s = 0;
        for (size_t i = 0; i < channel_size; ++i) {
            s += (int32_t)data[ch * channel_size + i];
        }
        fused[ch] = (int32_t)((uint32_t)bias[ch] - (uint32_t)zp * (uint32_t)s);
    }
}

void tqto_compute_asym_quant_params_i8(const float *data, size_t size, float *scale,
                                       int32_t *zp)
{
    /* test/common/quantized_gemm_test_runner.h:37-63 */
    float fmin = FLT_MAX, fmax = -FLT_MAX;
    for (size_t i = 0; i < size; ++i) {
        if (data[i] < fmin) {
            fmin = data[i];
        }
        if (data[i] > fmax) {
            fmax = data[i];
        }
    }
    fmax = fmax > 0.0f ? fmax : 0.0f;
    fmin = fmin < 0.0f ? fmin : 0.0f;
    const float s = (fmax - fmin) / 255.0f;
    if (s == 0.0f) {
        *scale = 1.0f;
        *zp = 0;
        return;
    }
    const float zp_tmp = -128.0f - fmin / s;
    int32_t zp_val = (int32_t)nearbyintf(zp_tmp);
    if (zp_val == -128) {
        zp_val = -127;
    }
    *scale = s;
    *zp = zp_val;
}

void tqto_compute_sym_quant_params_i8(const float *data, size_t size, float *scale)
{
    /* test/common/quantized_gemm_test_runner.h:67-86 */
    float fmin = FLT_MAX, fmax = -FLT_MAX;
    for (size_t i = 0; i < size; ++i) {
        if (data[i] < fmin) {
            fmin = data[i];
        }
        if (data[i] > fmax) {
            fmax = data[i];
        }
    }
    const float abs_max = (fabsf(fmax) >= fabsf(fmin)) ? fabsf(fmax) : fabsf(fmin);
    float s = 2.0f * abs_max / 255.0f;
    if (s == 0.0f) {
        s = 1.0f;
    }
    *scale = s;
}

void tqto_quantize_a_per_row_asym(const float *A, size_t m, size_t k, int8_t *A_i8,
                                  float *scale_a, int32_t *zp_a)
{
    /* test/gemm/test_gemm_i8_i4_rvv.cpp:40-77 */
    for (size_t row = 0; row < m; ++row) {
        const float *r = A + row * k;
        float fmin = FLT_MAX, fmax = -FLT_MAX;
        for (size_t i = 0; i < k; ++i) {
            if (r[i] < fmin) {
                fmin = r[i];
            }
            if (r[i] > fmax) {
                fmax = r[i];
            }
        }
        fmax = fmax > 0.0f ? fmax : 0.0f;
        fmin = fmin < 0.0f ? fmin : 0.0f;
        const float s = (fmax - fmin) / 255.0f;
        if (s == 0.0f) {
            scale_a[row] = 1.0f;
            zp_a[row] = 0;
            for (size_t i = 0; i < k; ++i) {
                A_i8[row * k + i] = 0;
            }
            continue;
        }
        const float zp_tmp = -128.0f - fmin / s;
        int32_t zp = (int32_t)nearbyintf(zp_tmp);
        if (zp < -128) {
            zp = -128;
        }
        if (zp > 127) {
            zp = 127;
        }
        scale_a[row] = s;
        zp_a[row] = zp;
        for (size_t i = 0; i < k; ++i) {
            A_i8[row * k + i] = tqto_quantize_i8(r[i], s, zp);
        }
    }
}

void tqto_quantize_fp16_to_int4(size_t n, size_t k, size_t bl, const uint16_t *src,
                                uint8_t *dst, uint16_t *scale, size_t ld_scale)
{
    /* test/common/quantize_utils.h:34-72 */
    memset(dst, 0, n * (k / 2));
    for (size_t j = 0; j < n; ++j) {
        const size_t nb = k / bl;
        for (size_t b = 0; b < nb; ++b) {
            float max_value = 0.0f, abs_max_value = 0.0f;
            for (size_t t = 0; t < bl; ++t) {
                const float v = tqto_f16_to_f32(src[j * k + b * bl + t]);
                if (fabsf(v) > abs_max_value) {
                    abs_max_value = fabsf(v);
                    max_value = v;
                }
            }
            const float fp32_scale = max_value / -8.0f;
            const float inv_scale = (fp32_scale != 0.0f) ? (1.0f / fp32_scale) : 0.0f;
            scale[j * ld_scale + b] = tqto_f32_to_f16(fp32_scale);
            for (size_t t = 0; t < bl; t += 2) {
                const float v0 = tqto_f16_to_f32(src[j * k + b * bl + t]);
                const float v1 = tqto_f16_to_f32(src[j * k + b * bl + t + 1]);
                const float x0 = v0 * inv_scale + 8.5f;
                const float x1 = v1 * inv_scale + 8.5f;
                const uint8_t q0 = (uint8_t)fminf((float)(int8_t)x0, 15.0f);
                const uint8_t q1 = (uint8_t)fminf((float)(int8_t)x1, 15.0f);
                dst[j * (k / 2) + (b * bl + t) / 2] = (uint8_t)(q0 | (uint8_t)(q1 << 4));
            }
        }
    }
}
