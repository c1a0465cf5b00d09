"""Shared test harness: library loaders, the CPU oracle binding, and seeded input generators.

The oracle (oracle/liboracle.so) and the reference's own portable test code
(oracle/_ref/libtqt_ref.so) are checkers only: tests call them to produce expected outputs;
the product is reached exclusively through libtorq_tile_gfx950.so.
"""

import ctypes
import importlib.util
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libtqt_ref.so")
SHIM_SO = os.path.join(ROOT, "tests", "abi_shim", "libtqt_test_shim.so")
GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")

c_size = ctypes.c_size_t
c_vp = ctypes.c_void_p


def load_product_module():
    """Import torq-tile_amd/tqt_gfx950.py (the package directory name is not an identifier)."""
    path = os.path.join(ROOT, "torq-tile_amd", "tqt_gfx950.py")
    spec = importlib.util.spec_from_file_location("tqt_gfx950", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def ptr(a):
    """Address of a numpy array's data (None for None)."""
    if a is None:
        return None
    return a.ctypes.data


# ------------------------------------------------------------------------------------------
# Oracle binding
# ------------------------------------------------------------------------------------------

class ConvParamsC(ctypes.Structure):
    _fields_ = [
        ("input_shape", c_size * 3),
        ("output_shape", c_size * 3),
        ("kernel_shape", c_size * 3),
        ("stride", c_size * 3),
        ("dilation", c_size * 3),
        ("pad", c_size * 3),
        ("input_channel", c_size),
        ("output_channel", c_size),
        ("groups", c_size),
    ]


def make_conv(input_shape, kernel_shape, stride=(1, 1, 1), dilation=(1, 1, 1), pad=(0, 0, 0),
              ic=1, oc=1, groups=1, cls=ConvParamsC):
    p = cls()
    for i in range(3):
        p.input_shape[i] = input_shape[i]
        p.kernel_shape[i] = kernel_shape[i]
        p.stride[i] = stride[i]
        p.dilation[i] = dilation[i]
        p.pad[i] = pad[i]
        p.output_shape[i] = ((input_shape[i] + 2 * pad[i] - dilation[i] * (kernel_shape[i] - 1)
                              - 1) // stride[i] + 1)
    p.input_channel = ic
    p.output_channel = oc
    p.groups = groups
    return p


_ORACLE = None


def oracle():
    global _ORACLE
    if _ORACLE is not None:
        return _ORACLE
    if not os.path.exists(ORACLE_SO):
        raise RuntimeError("oracle not built: %s (run make -C oracle)" % ORACLE_SO)
    o = ctypes.CDLL(ORACLE_SO)
    f32, i32, i8, u16 = ctypes.c_float, ctypes.c_int32, ctypes.c_int8, ctypes.c_uint16
    sig = {
        "tqto_set_threads": (None, [ctypes.c_int]),
        "tqto_get_threads": (ctypes.c_int, []),
        "tqto_f16_to_f32": (f32, [u16]),
        "tqto_f32_to_f16": (u16, [f32]),
        "tqto_bf16_to_f32": (f32, [u16]),
        "tqto_f32_to_bf16": (u16, [f32]),
        "tqto_quantize_multiplier": (None, [ctypes.c_double, c_vp, c_vp]),
        "tqto_requant_one": (i8, [i32, i32, i32, i32, i8, i8]),
        "tqto_gemm_clamp_i32_i8_i8": (None, [c_size] * 3 + [c_vp, c_size, c_vp, c_size, c_vp,
                                              c_size, c_vp, c_size, i32, i32]),
        "tqto_gemm_qai8_qai8_qsi8cxt": (None, [c_size] * 3 + [c_vp, c_size, c_vp, c_size, c_vp,
                                                c_size, c_vp, c_size, c_vp, i8, i8, f32, c_vp,
                                                i32, f32, i32]),
        "tqto_gemm_qsi8cxt_acc": (None, [c_size] * 3 + [c_vp, c_size, c_vp, c_size, c_vp, c_size,
                                          c_vp, c_vp, c_size]),
        "tqto_gemm_qai8dx_qsi4cxt_f32": (None, [c_size] * 3 + [c_vp, c_size, c_vp, c_size, c_vp,
                                                 c_size, c_vp, c_size, c_vp, f32, f32, c_vp,
                                                 c_vp, c_vp]),
        "tqto_gemm_qai8dx_qsi4cxt_h16": (None, [c_size] * 3 + [c_vp, c_size, c_vp, c_size, c_vp,
                                                 c_size, c_vp, c_size, c_vp, u16, u16, c_vp,
                                                 c_vp, c_vp, ctypes.c_int]),
        "tqto_gemm_f16_qsi4c2t_f32acc": (None, [c_size] * 4 + [c_vp, c_size, c_vp, c_size, c_vp,
                                                 c_size, c_vp, c_size, c_vp, c_size, c_vp, u16,
                                                 u16]),
        "tqto_gemm_f16_qsi4c2t_f32out": (None, [c_size] * 4 + [c_vp, c_size, c_vp, c_size, c_vp,
                                                 c_size, c_vp, c_size, c_vp, c_size, c_vp,
                                                 ctypes.c_float, ctypes.c_float]),
        "tqto_f16_add": (u16, [u16, u16]),
        "tqto_gemm_qai8dx_qsi8cxt_f32": (None, [c_size] * 3 + [
            c_vp, c_size, c_vp, c_size, c_vp, c_size, c_vp, ctypes.c_float, ctypes.c_float,
            c_vp, c_vp, c_vp]),
        "tqto_gemm_qai8dx_qsi8cxt_f16": (None, [c_size] * 3 + [
            c_vp, c_size, c_vp, c_size, c_vp, c_size, c_vp, u16, u16, c_vp, c_vp, c_vp]),
        "tqto_gemm_f16_qsi4c2t_rvv": (None, [c_size] * 4 + [c_vp, c_size, c_vp, c_size, c_vp,
                                              c_size, c_vp, c_size, c_vp, c_size, c_vp, u16,
                                              u16]),
        "tqto_im2col_cl_i8": (None, [c_size, c_vp, c_vp, ctypes.POINTER(ConvParamsC)]),
        "tqto_im2col_cf_i8": (None, [c_size, c_vp, c_vp, ctypes.POINTER(ConvParamsC)]),
        "tqto_gemm_mx1bias_qsi8dx": (None, [c_size] * 3 + [c_vp, c_size, c_vp, c_size, c_vp,
                                                 c_size, c_vp, c_size, c_vp, i8, i8, c_vp, i32,
                                                 f32, f32, i32]),
        "tqto_igemmcf_qsi8dx": (None, [c_size, c_size, c_vp, c_size, c_size, c_vp, c_size, c_vp,
                                        c_size, c_vp, i8, i8, ctypes.POINTER(ConvParamsC), c_vp,
                                        i32, f32, f32, i32]),
        "tqto_igemmcl_qsi8cxt": (None, [c_size, c_size, c_vp, c_size, c_size, c_vp, c_size, c_vp,
                                         c_size, c_vp, i8, i8, ctypes.POINTER(ConvParamsC), f32,
                                         c_vp, i32, f32, i32]),
        "tqto_quantize_i8": (i8, [f32, f32, i32]),
        "tqto_quantize_bias_i32": (i32, [f32, f32]),
        "tqto_fuse_zp_to_bias": (None, [c_vp, c_vp, c_vp, i32, c_size, c_size]),
        "tqto_compute_asym_quant_params_i8": (None, [c_vp, c_size, c_vp, c_vp]),
        "tqto_compute_sym_quant_params_i8": (None, [c_vp, c_size, c_vp]),
        "tqto_quantize_a_per_row_asym": (None, [c_vp, c_size, c_size, c_vp, c_vp, c_vp]),
        "tqto_quantize_fp16_to_int4": (None, [c_size, c_size, c_size, c_vp, c_vp, c_vp, c_size]),
    }
    for name, (res, args) in sig.items():
        f = getattr(o, name)
        f.restype = res
        f.argtypes = args
    threads = int(os.environ.get("TQT_ORACLE_THREADS", str(min(16, os.cpu_count() or 1))))
    o.tqto_set_threads(threads)
    _ORACLE = o
    return o


_REF = None


def ref():
    """The reference's own portable test code, or None when it was not built here."""
    global _REF
    if _REF is not None:
        return _REF
    if not os.path.exists(REF_SO):
        return None
    r = ctypes.CDLL(REF_SO)
    f32, i32, i8, u16, u32 = (ctypes.c_float, ctypes.c_int32, ctypes.c_int8, ctypes.c_uint16,
                              ctypes.c_uint32)
    sig = {
        "tqtr_quantize_multiplier": (None, [ctypes.c_double, c_vp, c_vp]),
        "tqtr_reference_gemm_i32_i8": (None, [c_size] * 3 + [c_vp, c_size, c_vp, c_size,
                                               ctypes.c_int, c_vp, c_size, c_vp, c_size, i32,
                                               i32]),
        "tqtr_reference_gemm_f32": (None, [c_size] * 3 + [c_vp, c_size, c_vp, c_size,
                                            ctypes.c_int, c_vp, c_size, c_vp, c_size, c_vp, f32,
                                            f32]),
        "tqtr_reference_gemm_qw_mixed_f16": (None, [c_size] * 4 + [c_vp, c_size, c_vp, c_size,
                                                     c_vp, c_size, c_vp, c_size, c_vp, c_size,
                                                     c_vp, u16, u16]),
        "tqtr_reference_gemm_qw_mixed_f16_f32": (None, [c_size] * 4 + [
            c_vp, c_size, c_vp, c_size, c_vp, c_size, c_vp, c_size, c_vp, c_size, c_vp, f32,
            f32]),
        "tqtr_reference_conv_cl_f32": (None, [c_size, c_vp, c_vp, c_vp, c_vp,
                                               ctypes.POINTER(ConvParamsC), f32, f32]),
        "tqtr_im2col_cl_i8": (None, [c_size, c_vp, c_vp, ctypes.POINTER(ConvParamsC)]),
        "tqtr_im2col_cf_i8": (None, [c_size, c_vp, c_vp, ctypes.POINTER(ConvParamsC)]),
        "tqtr_fill_uniform_f32": (None, [f32, f32, u32, c_vp, c_size, c_size]),
        "tqtr_fill_uniform_f16": (None, [f32, f32, u32, c_vp, c_size, c_size]),
        "tqtr_fill_uniform_i8": (None, [i8, i8, u32, c_vp, c_size, c_size]),
        "tqtr_fill_uniform_i32": (None, [i32, i32, u32, c_vp, c_size, c_size]),
        "tqtr_quantize_i8": (i8, [f32, f32, i32]),
        "tqtr_quantize_bias_i32": (i32, [f32, f32]),
        "tqtr_fuse_zp_to_bias": (None, [c_vp, c_vp, c_vp, i32, c_size, c_size]),
        "tqtr_quantize_fp16_to_int4": (None, [c_size, c_size, c_size, c_vp, c_vp, c_vp, c_size]),
    }
    for name, (res, args) in sig.items():
        f = getattr(r, name)
        f.restype = res
        f.argtypes = args
    _REF = r
    return r


# ------------------------------------------------------------------------------------------
# Oracle wrappers on numpy arrays (row-major, dense leading dimensions unless given)
# ------------------------------------------------------------------------------------------

def oracle_clamp(A, B, C, cmin, cmax):
    m, k = A.shape
    n = B.shape[1]
    D = np.zeros((m, n), np.int32)
    oracle().tqto_gemm_clamp_i32_i8_i8(m, n, k, ptr(A), k, ptr(B), n, ptr(C), n, ptr(D), n,
                                       cmin, cmax)
    return D


def oracle_w8a8(A, B, C, bias, cmin, cmax, scale_a, scale_b, qcb, scale_d, zp_d):
    m, k = A.shape
    n = B.shape[0]
    D = np.zeros((m, n), np.int8)
    oracle().tqto_gemm_qai8_qai8_qsi8cxt(m, n, k, ptr(A), k, ptr(B), k, ptr(C), n, ptr(D), n,
                                         ptr(bias), cmin, cmax, scale_a, ptr(scale_b), qcb,
                                         scale_d, zp_d)
    return D


def oracle_w8a8_acc(A, B, C, bias):
    m, k = A.shape
    n = B.shape[0]
    out = np.zeros((m, n), np.int32)
    oracle().tqto_gemm_qsi8cxt_acc(m, n, k, ptr(A), k, ptr(B), k, ptr(C), n, ptr(bias),
                                   ptr(out), n)
    return out


def oracle_w4a8(A, Bp, C, bias, cmin, cmax, scale_a, zp_a, scale_b):
    m, k = A.shape
    n = Bp.shape[0]
    D = np.zeros((m, n), np.float32)
    oracle().tqto_gemm_qai8dx_qsi4cxt_f32(m, n, k, ptr(A), k, ptr(Bp), k, ptr(C), n, ptr(D), n,
                                          ptr(bias), cmin, cmax, ptr(scale_a), ptr(zp_a),
                                          ptr(scale_b))
    return D


def oracle_w4a8_h16(A, Bp, C16, bias16, cmin_bits, cmax_bits, scale_a, zp_a, scale_b, bf16):
    """W4A8 with f16 (bf16=False) or bf16 C, bias, clamps and D, as 16-bit patterns."""
    m, k = A.shape
    n = Bp.shape[0]
    D = np.zeros((m, n), np.uint16)
    oracle().tqto_gemm_qai8dx_qsi4cxt_h16(m, n, k, ptr(A), k, ptr(Bp), k, ptr(C16), n, ptr(D), n,
                                          ptr(bias16), cmin_bits, cmax_bits, ptr(scale_a),
                                          ptr(zp_a), ptr(scale_b), 1 if bf16 else 0)
    return D


def bf16_bits(x):
    """float32 values -> bfloat16 bit patterns, round to nearest even (integer arithmetic,
    independent of the oracle's C)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, np.uint16(0x7FC0), r)


def bits_bf16_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def oracle_w4a16(A16, Bp, S16, bl, C16, bias16, cmin_bits, cmax_bits, rvv=False):
    m, k = A16.shape
    n = Bp.shape[0]
    D = np.zeros((m, n), np.uint16)
    f = oracle().tqto_gemm_f16_qsi4c2t_rvv if rvv else oracle().tqto_gemm_f16_qsi4c2t_f32acc
    f(m, n, k, bl, ptr(A16), k, ptr(Bp), k, ptr(S16), k // bl, ptr(C16), n, ptr(D), n,
      ptr(bias16), cmin_bits, cmax_bits)
    return D


def oracle_w4a16_f32(A16, Bp, S16, bl, C, bias, cmin, cmax):
    """W4A16 with f32 C, bias, clamp bounds and D (the f32-output type's oracle)."""
    m, k = A16.shape
    n = Bp.shape[0]
    D = np.zeros((m, n), np.float32)
    C = None if C is None else np.ascontiguousarray(C, np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
    oracle().tqto_gemm_f16_qsi4c2t_f32out(m, n, k, bl, ptr(A16), k, ptr(Bp), k, ptr(S16), k // bl,
                                          ptr(C), n, ptr(D), n, ptr(bias), float(cmin),
                                          float(cmax))
    return D


def oracle_w8a8dyn(A, B, bias, cmin, cmax, scale_a, zp_a, scale_b, f16=False):
    """W8A8 with dynamic per-row A quantization: f32 D, or f16 D (bias, cmin, cmax then given as
    binary16 patterns)."""
    m, k = A.shape
    n = B.shape[0]
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(B, np.int8)
    sa = np.ascontiguousarray(scale_a, np.float32)
    za = np.ascontiguousarray(zp_a, np.int32)
    sb = np.ascontiguousarray(scale_b, np.float32)
    if f16:
        D = np.zeros((m, n), np.uint16)
        b = None if bias is None else np.ascontiguousarray(bias, np.uint16)
        oracle().tqto_gemm_qai8dx_qsi8cxt_f16(m, n, k, ptr(A), k, ptr(B), k, ptr(D), n, ptr(b),
                                              int(cmin), int(cmax), ptr(sa), ptr(za), ptr(sb))
    else:
        D = np.zeros((m, n), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        oracle().tqto_gemm_qai8dx_qsi8cxt_f32(m, n, k, ptr(A), k, ptr(B), k, ptr(D), n, ptr(b),
                                              float(cmin), float(cmax), ptr(sa), ptr(za), ptr(sb))
    return D


def gen_w8a8dyn(m, n, k, seed=42, zp_range=(-128, 127)):
    """Random qai8dx x qsi8cx operands: int8 A and B, per-row scale / zero point, per-channel
    scale, f32 bias."""
    rng = np.random.default_rng(seed)
    return dict(
        A=rng.integers(-128, 128, size=(m, k), dtype=np.int64).astype(np.int8),
        B=rng.integers(-127, 128, size=(n, k), dtype=np.int64).astype(np.int8),
        scale_a=rng.uniform(0.002, 0.02, size=m).astype(np.float32),
        zp_a=rng.integers(zp_range[0], zp_range[1] + 1, size=m).astype(np.int32),
        scale_b=rng.uniform(0.001, 0.01, size=n).astype(np.float32),
        bias=rng.uniform(-10, 10, size=n).astype(np.float32))


def oracle_im2col_cf(inp, conv, group_idx=0):
    """Channel-first im2col of one group: [ICg*KD*KH*KW, OD*OH*OW] int8."""
    icg = conv.input_channel // conv.groups
    K = icg * conv.kernel_shape[0] * conv.kernel_shape[1] * conv.kernel_shape[2]
    N = conv.output_shape[0] * conv.output_shape[1] * conv.output_shape[2]
    col = np.zeros((K, N), np.int8)
    oracle().tqto_im2col_cf_i8(group_idx, ptr(np.ascontiguousarray(inp)), ptr(col),
                               ctypes.byref(conv))
    return col


def oracle_mx1bias(A, B, C, bias, cmin, cmax, scale_a, qca, scale_b, scale_d, zp_d):
    """gemm_mx1bias: A [m, k] int8, B [k, n] int8, C int32 [m, n] or None, bias int32 [m]."""
    m, k = A.shape
    n = B.shape[1]
    D = np.zeros((m, n), np.int8)
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(B, np.int8)
    sa = np.ascontiguousarray(scale_a, np.float32)
    oracle().tqto_gemm_mx1bias_qsi8dx(m, n, k, ptr(A), k, ptr(B), n, ptr(C), n, ptr(D), n,
                                      ptr(bias), cmin, cmax, ptr(sa), qca, scale_b, scale_d, zp_d)
    return D


def gen_mx1bias(m, n, k, seed=42, with_c=False, qca=None):
    """Weights A [m, k] with per-row scales, activations B [k, n], int32 bias [m]."""
    rng = np.random.default_rng(seed)
    return dict(
        A=rng.integers(-127, 128, size=(m, k), dtype=np.int64).astype(np.int8),
        B=rng.integers(-128, 128, size=(k, n), dtype=np.int64).astype(np.int8),
        C=(rng.integers(-3000, 3001, size=(m, n), dtype=np.int64).astype(np.int32)
           if with_c else None),
        bias=rng.integers(-2000, 2001, size=m, dtype=np.int64).astype(np.int32),
        scale_a=rng.uniform(0.001, 0.01, size=m).astype(np.float32),
        qca=m if qca is None else qca,
        scale_b=np.float32(0.02), scale_d=np.float32(0.08), zp_d=-5)


def oracle_igemmcl(inp, W, bias, cmin, cmax, conv, scale_a, scale_b, qcb, scale_d, zp_d,
                   m=None, m_idx=0, group_idx=0, D=None):
    n = W.shape[0]
    M_all = conv.output_shape[0] * conv.output_shape[1] * conv.output_shape[2]
    if m is None:
        m = M_all - m_idx
    if D is None:
        D = np.zeros((M_all, n), np.int8)
    oracle().tqto_igemmcl_qsi8cxt(m, n, ptr(inp), group_idx, m_idx, ptr(W), W.shape[1], ptr(D),
                                  n, ptr(bias), cmin, cmax, ctypes.byref(conv), scale_a,
                                  ptr(scale_b), qcb, scale_d, zp_d)
    return D


def f16_bits(x):
    """numpy float -> binary16 bit patterns (numpy's own round-to-nearest-even)."""
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def bits_f16(b):
    return np.asarray(b, np.uint16).view(np.float16)


# ------------------------------------------------------------------------------------------
# Seeded synthetic inputs for the BASELINE.json configurations
# ------------------------------------------------------------------------------------------

def pack_int4(q):
    """q: int array [n, k] with values in [-8, 7] -> bytes [n, k/2], low nibble = even k."""
    u = (q.astype(np.int32) + 8).astype(np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)


def gen_clamp(m, n, k, seed=42, with_c=False, lo=-128, hi=127):
    rng = np.random.default_rng(seed)
    A = rng.integers(lo, hi + 1, size=(m, k), dtype=np.int64).astype(np.int8)
    B = rng.integers(lo, hi + 1, size=(k, n), dtype=np.int64).astype(np.int8)
    C = rng.integers(-1000, 1001, size=(m, n), dtype=np.int64).astype(np.int32) if with_c else None
    return A, B, C


def gen_w8a8(m, n, k, seed=42, with_c=False, scale_a=0.02, scale_d=0.05, zp_d=0):
    """BASELINE cfg 2 input recipe at any shape."""
    rng = np.random.default_rng(seed)
    zp_a = int(rng.integers(-20, 21))
    x = rng.standard_normal((m, k)).astype(np.float32)
    A = np.clip(np.rint(x / np.float32(scale_a)) + zp_a, -128, 127).astype(np.int8)
    B = rng.integers(-127, 128, size=(n, k), dtype=np.int64).astype(np.int8)
    scale_b = rng.uniform(0.001, 0.01, size=n).astype(np.float32)
    bias = rng.integers(-1000, 1001, size=n, dtype=np.int64).astype(np.int32)
    fused = np.zeros(n, np.int32)
    oracle().tqto_fuse_zp_to_bias(ptr(fused), ptr(bias), ptr(B), zp_a, n, k)
    C = rng.integers(-5000, 5001, size=(m, n), dtype=np.int64).astype(np.int32) if with_c else None
    return dict(A=A, B=B, C=C, bias=fused, scale_a=np.float32(scale_a), zp_a=zp_a,
                scale_b=scale_b, scale_d=np.float32(scale_d), zp_d=zp_d)


def gen_w4a8(m, n, k, seed=42, with_c=False, with_bias=True):
    """BASELINE cfg 3 input recipe at any shape."""
    rng = np.random.default_rng(seed)
    Af = rng.standard_normal((m, k)).astype(np.float32)
    A = np.zeros((m, k), np.int8)
    sa = np.zeros(m, np.float32)
    za = np.zeros(m, np.int32)
    oracle().tqto_quantize_a_per_row_asym(ptr(Af), m, k, ptr(A), ptr(sa), ptr(za))
    # two independent uniform nibbles per byte == uniform bytes; nibble - 8 is U[-8, 7]
    Bp = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    sb = rng.uniform(0.005, 0.02, size=n).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float32) if with_bias else None
    C = rng.uniform(-2.0, 2.0, size=(m, n)).astype(np.float32) if with_c else None
    return dict(A=A, Bp=Bp, scale_a=sa, zp_a=za, scale_b=sb, bias=bias, C=C)


def gen_w4a16(m, n, k, bl=32, seed=42, with_c=False, with_bias=True):
    """BASELINE cfg 4 input recipe at any shape (f16 tensors as bit patterns)."""
    rng = np.random.default_rng(seed)
    A16 = f16_bits(rng.standard_normal((m, k)))
    Bp = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    S16 = f16_bits(rng.uniform(0.005, 0.02, size=(n, k // bl)))
    bias16 = f16_bits(rng.standard_normal(n) * 0.1) if with_bias else None
    C16 = f16_bits(rng.uniform(-5.0, 5.0, size=(m, n))) if with_c else None
    return dict(A16=A16, Bp=Bp, S16=S16, bl=bl, bias16=bias16, C16=C16)


def gen_igemmcl(ID, IH, IW, IC, OC, KH, KW, stride=(1, 1), pad=(0, 0), dil=(1, 1), KD=1,
                seed=42, scale_a=0.02, zp_a=3, scale_d=0.05, zp_d=0):
    """BASELINE cfg 5 input recipe at any shape (batch folded into the depth dimension)."""
    rng = np.random.default_rng(seed)
    conv = make_conv((ID, IH, IW), (KD, KH, KW), (1, stride[0], stride[1]), (1, dil[0], dil[1]),
                     (0, pad[0], pad[1]), IC, OC, 1)
    K = KD * KH * KW * IC
    inp = rng.integers(-128, 128, size=(ID, IH, IW, IC), dtype=np.int64).astype(np.int8)
    W = rng.integers(-127, 128, size=(OC, K), dtype=np.int64).astype(np.int8)
    scale_b = rng.uniform(0.001, 0.01, size=OC).astype(np.float32)
    bias = rng.integers(-1000, 1001, size=OC, dtype=np.int64).astype(np.int32)
    fused = np.zeros(OC, np.int32)
    oracle().tqto_fuse_zp_to_bias(ptr(fused), ptr(bias), ptr(W), zp_a, OC, K)
    return dict(inp=inp, W=W, bias=fused, conv=conv, scale_a=np.float32(scale_a), zp_a=zp_a,
                scale_b=scale_b, scale_d=np.float32(scale_d), zp_d=zp_d)


# ------------------------------------------------------------------------------------------
# Packed layout of the p-variants, restated independently of the device code (the library's
# packers must produce exactly these bytes): panels of `step` rows, panel p at
# p * step * ld_packed (minus shift * (step - w) for a narrower panel after the first), chunks
# of `kc` bytes stored chunk-major inside a panel, the last chunk of a row narrower when the
# row length is not a multiple of kc. W4A16 weights are first permuted inside each whole
# 64-byte group of a row (4 x 4 transpose of 4-byte words).
# ------------------------------------------------------------------------------------------

# chunk bytes per packed kernel type (one MFMA lane fragment for every type)
PACK_CHUNK = {"clampp": 16, "w8a8pb": 16, "w8a8p": 16, "igemmclp": 16, "w4a8p": 16,
              "w4a16p": 16, "w4a16fp": 16, "w8dynp": 16, "w8dynhp": 16}


def frag_perm(kbytes):
    """perm[P] = logical byte stored at position P of a fragment-ordered W4A16 weight row."""
    P = np.arange(kbytes)
    g = P >> 6
    full = 64 * (g + 1) <= kbytes
    swapped = 64 * g + 16 * ((P >> 2) & 3) + 4 * ((P >> 4) & 3) + (P & 3)
    return np.where(full, swapped, P)


def pack_panels(X, step, kc=16, ld_packed=None, shift=0, frag=False, out=None, base=0):
    """X: [rows, kbytes] (any dtype of 1 byte, or an index array) -> flat packed buffer.
    ld_packed, shift: bytes. Writes into `out` at offset `base` when given."""
    X = np.asarray(X)
    rows, kb = X.shape
    if ld_packed is None:
        ld_packed = kb
    if frag:
        X = X[:, frag_perm(kb)]
    if out is None:
        out = np.zeros(rows * ld_packed if rows else 0, X.dtype)
    kfull = kb // kc * kc
    for p in range((rows + step - 1) // step):
        r0 = p * step
        w = min(step, rows - r0)
        pb = base + r0 * ld_packed
        if p > 0 and w < step:
            pb -= shift * (step - w)
        blk = X[r0:r0 + w]
        full = blk[:, :kfull].reshape(w, kfull // kc, kc).transpose(1, 0, 2).ravel()
        out[pb:pb + full.size] = full
        tail = blk[:, kfull:].ravel()
        out[pb + full.size:pb + full.size + tail.size] = tail
    return out
