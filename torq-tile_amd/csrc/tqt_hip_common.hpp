// Shared host/device helpers of the gfx950 TORQ-Tile library: error reporting, fragment
// types, the requantization multiplier and epilogue, and launch plumbing.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "tqt_gfx950_common.h"

// ---------------------------------------------------------------------------------------------
// Error convention (reference src/common/tqt_common.h:76-81, TQT_ERROR in a debug build):
// print "file:line message" to stderr and abort.
// ---------------------------------------------------------------------------------------------
#define TQT_FAIL(msg)                                                       \
    do {                                                                    \
        fflush(stdout);                                                     \
        fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, (msg));           \
        abort();                                                            \
    } while (0)

#define TQT_REQUIRE(cond, msg)    \
    do {                          \
        if (!(cond)) {            \
            TQT_FAIL(msg);        \
        }                         \
    } while (0)

#define TQT_HIP_CHECK(expr)                                                             \
    do {                                                                                \
        hipError_t tqt_err_ = (expr);                                                   \
        if (tqt_err_ != hipSuccess) {                                                   \
            fflush(stdout);                                                             \
            fprintf(stderr, "%s:%d HIP error %s: %s\n", __FILE__, __LINE__, #expr,      \
                    hipGetErrorString(tqt_err_));                                       \
            abort();                                                                    \
        }                                                                               \
    } while (0)

namespace tqt {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

// One global -> LDS load of 16 bytes per lane (lane i writes lds + 16 * i; lds is wave-uniform).
// It is inline asm rather than __builtin_amdgcn_global_load_lds on purpose: the compiler tracks
// the builtin's LDS write and, where its alias tracking of the ring stages is lost (the pipelined
// loop's back edge), guards the next LDS reads with vmcnt(0), which drains every stage in flight
// and serializes the stream (measured: 22.9 us -> 16 us per W8A8 M512 launch without it). The
// kernels order these writes themselves with explicit vmcnt waits and s_barrier; the "memory"
// clobber keeps the compiler's own LDS accesses on their side of each load. M0 carries the LDS
// base (the low 32 bits of a flat LDS address are its LDS offset); nothing else in these kernels
// uses M0. gfx9 needs one wait state between an SALU write of M0 and an LDS-DMA load that reads
// it; the compiler cannot insert it inside an asm block, so the asm carries its own s_nop 0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_lds16(const int8_t *src, int8_t *lds)
{
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t base =
        __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(base)
                 : "memory", "m0");
#else
    (void)src;
    (void)lds;
#endif
}

// 4 bytes per lane (lane i's dword at lds + 4 i): small rows such as per-block scales.
__device__ __forceinline__ void dma_lds4(const void *src, int8_t *lds)
{
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t base =
        __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(base)
                 : "memory", "m0");
#else
    (void)src;
    (void)lds;
#endif
}

// The same load through a buffer resource: voffset is a byte offset from the resource's base,
// and an offset at or past its num_records reads zeros (the implicit convolution's padding taps).
__device__ __forceinline__ void dma_lds16_buf(i32x4 rsrc, int voffset, int8_t *lds)
{
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t base =
        __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voffset),
                 "s"(rsrc), "s"(base)
                 : "memory", "m0");
#else
    (void)rsrc;
    (void)voffset;
    (void)lds;
#endif
}
#pragma clang diagnostic pop

inline bool aligned16(const void *p)
{
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

inline hipStream_t as_stream(void *s)
{
    return reinterpret_cast<hipStream_t>(s);
}

// Launch-error check after every kernel launch; the synchronous entry points also wait.
inline void check_launch(const char *where)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fflush(stdout);
        fprintf(stderr, "%s: kernel launch failed: %s\n", where, hipGetErrorString(e));
        abort();
    }
}

inline void finish_sync(hipStream_t stream, const char *where)
{
    check_launch(where);
    hipError_t e = hipStreamSynchronize(stream);
    if (e != hipSuccess) {
        fflush(stdout);
        fprintf(stderr, "%s: kernel execution failed: %s\n", where, hipGetErrorString(e));
        abort();
    }
}

// ---------------------------------------------------------------------------------------------
// Requantization multiplier, evaluated on the device from the same double bits the reference
// uses on the host (reference src/gemm/gemm_i8_i8/tqt_utils_i8_i8.h:16-132): the Q31 fraction
// is the top 30 mantissa bits of x plus the implicit bit, rounded up when the 22 dropped bits
// exceed one half; the exponent follows frexp's [0.5, 1) convention. The run functions then
// store shift = -exponent - 1 (…qsi8cxt_4x1vl_rvv.cpp:158-176).
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ void quantize_multiplier_dev(double x, int32_t &mult, int32_t &shift)
{
    if (x == 0.0) {
        mult = 0;
        shift = 0;
        return;
    }
    const uint64_t u = static_cast<uint64_t>(__double_as_longlong(x));
    const uint64_t sign_mask = 0x8000000000000000ull;
    int64_t q;
    int32_t e;
    if ((u & ~sign_mask) == 0) {
        e = 0;
        q = 0;
    } else {
        const uint32_t exponent_part = static_cast<uint32_t>((u & 0x7ff0000000000000ull) >> 52);
        if (exponent_part == 0x7ffu) {
            e = 0x7fffffff;
            if (u & 0x000fffffffc00000ull) {
                q = 0;
            } else {
                q = (u & sign_mask) ? static_cast<int64_t>(0x8000000000000000ull)
                                    : static_cast<int64_t>(0x7fffffffffffffffll);
            }
        } else {
            e = static_cast<int32_t>(exponent_part - 1023u) + 1;
            q = 0x40000000ll + static_cast<int64_t>((u & 0x000fffffffc00000ull) >> 22);
            if ((u & 0x003fffffull) > 0x00200000ull) {
                q += 1;
            }
            if (u & sign_mask) {
                q = -q;
            }
        }
    }
    if (q == (1ll << 31)) {
        q /= 2;
        e += 1;
    }
    if (e < -31) {
        e = 0;
        q = 0;
    }
    mult = static_cast<int32_t>(q);
    shift = -e - 1;
}

// Column multiplier exactly as the run functions compute it: double(scale_a) * double(scale_b)
// / double(scale_d), column 0 reused for every column when quant_channel_b == 1.
// column_multiplier_val takes the column's scale_b already loaded (kernels that load it early
// and finish the multiplier later).
__device__ __forceinline__ void column_multiplier_val(float scale_a, float scale_b_col,
                                                      float scale_d, int32_t &mult, int32_t &shift)
{
    const double real = static_cast<double>(scale_a) * static_cast<double>(scale_b_col) /
                        static_cast<double>(scale_d);
    quantize_multiplier_dev(real, mult, shift);
}

__device__ __forceinline__ void column_multiplier_dev(float scale_a, const float *scale_b,
                                                      int32_t quant_channel_b, float scale_d,
                                                      int col, int32_t &mult, int32_t &shift)
{
    const int src = (quant_channel_b == 1) ? 0 : col;
    column_multiplier_val(scale_a, scale_b[src], scale_d, mult, shift);
}

// ---------------------------------------------------------------------------------------------
// Packed operand layout of the p-variants (the reference's packers are permutations A [m, k] ->
// [m/MR, k, MR] and B^T [n, k] -> [n/vl, k, vl], tqt_gemm_pack_rvv.h:542-567, 740-856; this is
// the gfx950 one). Rows (m of A, n of B) form panels of `step` rows: panel p holds rows
// [p*step, p*step + w), w = min(step, rows - p*step), and starts at byte p*step*ld, moved back by
// shift*(step - w) bytes when a panel after the first is narrower (shift = k_idx in bytes: the
// reference's tail-tile rule, tqt_gemm_pack_rvv.h:314-318). Inside a panel each row is cut into
// chunks of kc bytes stored chunk-major: chunk c of local row r at kc*c*w + r*cw,
// cw = min(kc, kbytes - kc*c). kc is the k-extent one wave load instruction takes from a row:
// 128 bytes for the int8 and W4A8 mainloops (8 rows x 128 bytes per instruction: one contiguous
// KiB), 16 bytes - one MFMA lane fragment - for W4A16 (16 channels x 16 bytes per lane group).
// One k-step of a whole panel is thus one contiguous block in the order the lanes take it. When
// kbytes % kc == 0, byte kb of row r sits at row_base(r) + (kb - kb % kc) * w + kb % kc. A panel
// of w rows holds w * kbytes bytes, so the packed sizes are the unpacked ones (m*k, n*k, n*k/2).
// ---------------------------------------------------------------------------------------------
// Panel heights (m_step / n_step) and chunk sizes of the packed kernel types.
constexpr size_t kPackI8MStep = 128;   // int8 GEMMs and igemmcl (A and B panels)
constexpr size_t kPackI8NStep = 128;
constexpr int kPackI8Chunk = 16;
constexpr size_t kPackW4A8MStep = 16;  // W4A8: one 16-channel weight tile per panel
constexpr size_t kPackW4A8NStep = 16;
constexpr int kPackW4A8Chunk = 16;
constexpr size_t kPackW4A16MStep = 32; // W4A16: one 32-row activation group, 16 channels
constexpr size_t kPackW4A16NStep = 16;
constexpr int kPackW4A16Chunk = 16;

// Which operands of a kernel instance are in the packed layout; plain row-major otherwise.
enum PackMode { PK_NONE = 0, PK_A = 1, PK_B = 2, PK_AB = 3 };

struct PackDesc
{
    long long ld;      // bytes per row of panel stride: panel p starts at p * step * ld
    long long kbytes;  // bytes of each row held in the panels
    long long shift;   // k_idx in bytes (tail panels after the first start shift*(step-w) earlier)
    int step;          // rows per panel; 0 = plain row-major (row r at r * ld)
    int rows;          // rows of the operand
    int kc;            // chunk bytes (a power of two, >= 16)
};

__host__ __device__ inline long long pack_panel_base(const PackDesc &d, int p, int w)
{
    long long b = static_cast<long long>(p) * d.step * d.ld;
    if (p > 0 && w < d.step) {
        b -= d.shift * (d.step - w);
    }
    return b;
}

// Placement of one row: its panel's base, the panel width and the row's index in the panel
// (a plain row-major operand is the case w = 1, rl = 0, base = r * ld).
struct PackRow
{
    long long base;
    long long kbytes;
    int w, rl, kc;
};

__host__ __device__ inline PackRow pack_row_info(const PackDesc &d, int r)
{
    PackRow pr;
    pr.kbytes = d.kbytes;
    pr.kc = d.kc;
    if (d.step == 0) {
        pr.base = static_cast<long long>(r) * d.ld;
        pr.w = 1;
        pr.rl = 0;
        return pr;
    }
    const int p = r / d.step;
    const int left = d.rows - p * d.step;
    pr.w = left < d.step ? left : d.step;
    pr.rl = r - p * d.step;
    pr.base = pack_panel_base(d, p, pr.w);
    return pr;
}

// Byte offset of byte kb (any kb < kbytes) of the row.
__host__ __device__ inline long long pack_row_byte(const PackRow &pr, long long kb)
{
    const long long c0 = kb - kb % pr.kc;  // first byte of kb's chunk
    const long long rem = pr.kbytes - c0;
    const long long cw = rem < pr.kc ? rem : pr.kc;
    return pr.base + c0 * pr.w + pr.rl * cw + kb % pr.kc;
}

__host__ __device__ inline long long pack_offset(const PackDesc &d, int r, long long kb)
{
    return pack_row_byte(pack_row_info(d, r), kb);
}

// For kbytes % kc == 0: byte kb of row r is at the returned offset + pack_k(kb, mul, kc).
__host__ __device__ inline long long pack_row(const PackDesc &d, int r, int &mul)
{
    if (d.step == 0) {
        mul = 1;
        return static_cast<long long>(r) * d.ld;
    }
    const int p = r / d.step;
    const int left = d.rows - p * d.step;
    const int w = left < d.step ? left : d.step;
    mul = w;
    return pack_panel_base(d, p, w) + static_cast<long long>(d.kc) * (r - p * d.step);
}

// pack_row of a packed descriptor whose step is the compile-time STEP (a power of two; r >= 0):
// shifts and masks where pack_row divides by the run-time step.
template <int STEP>
__device__ __forceinline__ long long pack_row_fixed(const PackDesc &d, int r, int &mul)
{
    static_assert(STEP > 0 && (STEP & (STEP - 1)) == 0, "panel step");
    const int p = static_cast<int>(static_cast<unsigned>(r) / STEP);
    const int rl = static_cast<int>(static_cast<unsigned>(r) % STEP);
    const int left = d.rows - p * STEP;
    const int w = left < STEP ? left : STEP;
    mul = w;
    long long b = static_cast<long long>(p) * STEP * d.ld + static_cast<long long>(d.kc) * rl;
    if (p > 0 && w < STEP) {
        b -= d.shift * (STEP - w);
    }
    return b;
}

// Offset of byte kb from the row base pack_row returned (a plain row: kb itself). For a packed
// row kb < 2^24 and mul <= 2^7 (the launchers of the packed fast paths check kbytes < 2^24; panel
// heights are at most 128), so one 24-bit multiply gives it.
template <int KC, bool kPacked>
__device__ __forceinline__ uint32_t pack_k(uint32_t kb, int mul)
{
    if constexpr (!kPacked) {
        return kb;
    } else {
        return __umul24(kb & ~static_cast<uint32_t>(KC - 1), static_cast<uint32_t>(mul)) +
               (kb & static_cast<uint32_t>(KC - 1));
    }
}

// Host-side description of a packed operand: `rows` rows of `kbytes` bytes, panel height `step`
// (0: plain row-major), chunk bytes `kc`, leading dimension `ld_bytes`, k_idx `shift_bytes`.
inline PackDesc make_pack(size_t step, int kc, size_t rows, size_t ld_bytes, size_t kbytes,
                          size_t shift_bytes)
{
    TQT_REQUIRE(rows < (1u << 31), "dimension exceeds 2^31-1");
    PackDesc d;
    d.ld = static_cast<long long>(ld_bytes);
    d.kbytes = static_cast<long long>(kbytes);
    d.shift = static_cast<long long>(shift_bytes);
    d.step = static_cast<int>(step);
    d.rows = static_cast<int>(rows);
    d.kc = kc;
    return d;
}

// First row of the panel that must be written after the others: the narrow last panel when the
// k_idx tail rule moves it back onto the panel before it (d.rows when there is none).
inline int tail_panel_start(const PackDesc &d)
{
    if (d.step <= 0 || d.shift <= 0 || d.rows <= d.step || d.rows % d.step == 0) {
        return d.rows;
    }
    return d.rows - d.rows % d.step;
}

// Byte order inside one row of a packed W4A16 weight: each whole 64-byte group (four 32-k blocks
// of 16 bytes) is a 4 x 4 transpose of dwords, so 16-byte chunk c of the group holds dword c of
// blocks 0..3 - the 8-k slice lane group c feeds to the four MFMAs of the group. Bytes of a
// trailing partial group keep their place. Returns the stored position of logical byte kb.
__host__ __device__ inline long long w4a16_frag_pos(long long kb, long long kbytes)
{
    const long long g = kb >> 6;
    if (64 * (g + 1) > kbytes) {
        return kb;
    }
    const long long blk = (kb >> 4) & 3;  // 32-k block within the group
    const long long dw = (kb >> 2) & 3;   // 8-k dword within the block
    return 64 * g + 16 * dw + 4 * blk + (kb & 3);
}

// ---------------------------------------------------------------------------------------------
// Output element types of the float-output kernel types (f32, f16, bf16). Loads widen exactly;
// stores round to nearest even (the reference's vfncvt.f.f.w / vfncvtbf16.f.f.w under the
// default rounding mode) and write the canonical quiet NaN (0x7e00, 0x7fc0) for a NaN, as those
// RISC-V conversions do.
// ---------------------------------------------------------------------------------------------
enum OutType { OUT_F32 = 0, OUT_F16 = 1, OUT_BF16 = 2 };

__host__ __device__ inline float bf16_bits_to_f32(uint16_t b)
{
    uint32_t u = static_cast<uint32_t>(b) << 16;
    float f;
    __builtin_memcpy(&f, &u, 4);
    return f;
}

__host__ __device__ inline uint16_t f32_to_bf16_bits(float f)
{
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        return 0x7fc0;
    }
    return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

template <int OUT>
__device__ __forceinline__ float load_out(const void *p, long long i)
{
    if constexpr (OUT == OUT_F32) {
        return static_cast<const float *>(p)[i];
    } else if constexpr (OUT == OUT_F16) {
        return static_cast<float>(static_cast<const _Float16 *>(p)[i]);
    } else {
        return bf16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
    }
}

// load_out in two halves: the element's raw bits now, the conversion later. A kernel that reads
// its epilogue operands ahead of its main loads keeps the bits, so that no conversion (and no
// wait for the load) stands before those loads; all-zero bits are +0 in every output type.
template <int OUT>
__device__ __forceinline__ uint32_t load_out_bits(const void *p, long long i)
{
    if constexpr (OUT == OUT_F32) {
        return static_cast<const uint32_t *>(p)[i];
    } else {
        return static_cast<const uint16_t *>(p)[i];
    }
}

template <int OUT>
__device__ __forceinline__ float out_from_bits(uint32_t bits)
{
    if constexpr (OUT == OUT_F32) {
        return __builtin_bit_cast(float, bits);
    } else if constexpr (OUT == OUT_F16) {
        return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
    } else {
        return bf16_bits_to_f32(static_cast<uint16_t>(bits));
    }
}

template <int OUT>
__device__ __forceinline__ void store_out(void *p, long long i, float v)
{
    if constexpr (OUT == OUT_F32) {
        static_cast<float *>(p)[i] = v;
    } else if constexpr (OUT == OUT_F16) {
        const _Float16 h = static_cast<_Float16>(v);
        static_cast<uint16_t *>(p)[i] = v != v ? static_cast<uint16_t>(0x7e00)
                                               : __builtin_bit_cast(uint16_t, h);
    } else {
        static_cast<uint16_t *>(p)[i] = f32_to_bf16_bits(v);
    }
}

// The same conversions through a raw buffer resource: element at byte offset voff + soff (soff
// wave-uniform); an offset at or past the resource's num_records reads 0 / writes nothing.
template <int OUT>
__device__ __forceinline__ float load_out_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
    if constexpr (OUT == OUT_F32) {
        return __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(voff),
                                                        static_cast<int>(soff), 0));
    } else {
        const uint16_t bits = __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(voff),
                                                                   static_cast<int>(soff), 0);
        if constexpr (OUT == OUT_F16) {
            return static_cast<float>(__builtin_bit_cast(_Float16, bits));
        } else {
            return bf16_bits_to_f32(bits);
        }
    }
}

template <int OUT>
__device__ __forceinline__ void store_out_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                              float v)
{
    if constexpr (OUT == OUT_F32) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r,
                                              static_cast<int>(voff), static_cast<int>(soff), 0);
    } else {
        uint16_t bits;
        if constexpr (OUT == OUT_F16) {
            const _Float16 h = static_cast<_Float16>(v);
            bits = v != v ? static_cast<uint16_t>(0x7e00) : __builtin_bit_cast(uint16_t, h);
        } else {
            bits = f32_to_bf16_bits(v);
        }
        __builtin_amdgcn_raw_buffer_store_b16(bits, r, static_cast<int>(voff),
                                              static_cast<int>(soff), 0);
    }
}

// RISC-V vfmax / vfmin on f32 (IEEE 754-2019 maximumNumber / minimumNumber): a NaN operand
// yields the other one (the canonical quiet NaN when both are NaN), and -0 orders below +0.
__device__ __forceinline__ float rv_fmaxf(float a, float b)
{
    if (a != a) {
        return b != b ? __builtin_bit_cast(float, 0x7fc00000u) : b;
    }
    if (b != b) {
        return a;
    }
    if (a == b) {
        return (__builtin_bit_cast(uint32_t, a) >> 31) ? b : a;
    }
    return a > b ? a : b;
}

__device__ __forceinline__ float rv_fminf(float a, float b)
{
    if (a != a) {
        return b != b ? __builtin_bit_cast(float, 0x7fc00000u) : b;
    }
    if (b != b) {
        return a;
    }
    if (a == b) {
        return (__builtin_bit_cast(uint32_t, a) >> 31) ? a : b;
    }
    return a < b ? a : b;
}

// One output of the requantization epilogue (reference tqt_kernel_gemm_i8_i8_4x1vl_rvv.h:
// requantize_1xn :334-408 = vmulh, vsra by shift & 31, vadd zp, vnclip to i16 then i8;
// clamp_i8 :231-259 = vmax then vmin).
// cmin and cmax are int8 values (the run functions take them as int8_t): then the saturation to
// [-128, 127] followed by max(., cmin) and min(., cmax) equals max(., min(cmin, cmax)) followed
// by min(., cmax), which also covers cmin > cmax (every output is cmax); the first of those is
// uniform, so two operations per output remain.
// The same output before its int8 truncation: an int32 in [lo, cmax], lo = min(cmin, cmax).
__device__ __forceinline__ int32_t requant_clamped_dev(int32_t acc, int32_t mult, int32_t shift,
                                                       int32_t zp, int32_t lo, int32_t cmax)
{
    int32_t y = __mulhi(acc, mult);  // high 32 bits of the signed 64-bit product
    y = y >> (shift & 31);
    y = static_cast<int32_t>(static_cast<uint32_t>(y) + static_cast<uint32_t>(zp));
    // max(y, lo) then min(., cmax): with lo <= cmax that is the median of the three
#if defined(__HIP_DEVICE_COMPILE__)
    asm("v_med3_i32 %0, %1, %2, %3" : "=v"(y) : "v"(y), "v"(lo), "v"(cmax));
#else
    y = min(max(y, lo), cmax);
#endif
    return y;
}

__device__ __forceinline__ int8_t requant_dev(int32_t acc, int32_t mult, int32_t shift,
                                              int32_t zp, int32_t cmin, int32_t cmax)
{
    return static_cast<int8_t>(requant_clamped_dev(acc, mult, shift, zp, min(cmin, cmax), cmax));
}

// ---------------------------------------------------------------------------------------------
// qai8dx: dynamic per-row asymmetric int8 quantization of f32 activations (reference test-side
// quantize_a_per_row_asym, test/gemm/test_gemm_i8_i4_rvv.cpp:40-77, with quantize_i8 from
// test/common/test_common.h:232-240), in float arithmetic with correctly rounded divisions and
// round-half-even nearbyint (the library is built with -ffp-contract=off).
// ---------------------------------------------------------------------------------------------

// Scale and zero point of a row from its minimum and maximum; false when the scale is 0 (then
// the row quantizes to scale 1, zero point 0 and all-zero values).
__device__ __forceinline__ bool qai8dx_row_params(float lo, float hi, float &s, int32_t &zp)
{
    hi = hi > 0.0f ? hi : 0.0f;
    lo = lo < 0.0f ? lo : 0.0f;
    s = (hi - lo) / 255.0f;
    if (s == 0.0f) {
        s = 1.0f;
        zp = 0;
        return false;
    }
    zp = static_cast<int32_t>(__builtin_rintf(-128.0f - lo / s));
    zp = zp < -128 ? -128 : (zp > 127 ? 127 : zp);
    return true;
}

// One value: clamp(nearbyint(x / s) + zp, -128, 127) (rint: round half to even).
__device__ __forceinline__ int8_t qai8dx_quantize(float x, float s, float zpf)
{
    float q = __builtin_rintf(x / s) + zpf;
    q = q > 127.0f ? 127.0f : q;
    q = q < -128.0f ? -128.0f : q;
    return static_cast<int8_t>(q);
}

}  // namespace tqt
