"""ctypes binding of the gfx950 TORQ-Tile C ABI (libtorq_tile_gfx950.so).

This is the Python-side stub a framework maintainer would add to call the library. The function
signatures are not restated here: they are read from the C declarations in include/*.h, so the
headers stay the one definition of the ABI, and every declared function must be exported by the
library or loading fails. The parameter structs are mirrored field for field. Buffers are passed
as raw device addresses (int); torch tensors on a ROCm device provide them via
``tensor.data_ptr()``.

Loading fails loudly: there is no CPU fallback. ``load()`` raises if the shared library has not
been built (``make -C torq-tile_amd``).
"""

import ctypes
import glob
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtorq_tile_gfx950.so")
INCLUDE_DIR = os.path.join(os.path.dirname(_HERE), "include")

c_size = ctypes.c_size_t
c_vp = ctypes.c_void_p

VARIANT = "mfma_gfx950"
KERNELS = {
    "clamp": "gemm_clamp_i32_i8_i8",
    "w8a8": "gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt",
    "w4a8": "gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt",
    "w4a16": "gemm_1xnbias_clamp_f16_f16_qsi4c2t",
    "igemmcl": "igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt",
    # packed (p) siblings
    "clampp": "gemm_clamp_i32_i8p_i8p",
    "w8a8pb": "gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp",
    "w8a8p": "gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp",
    "w4a8p": "gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp",
    "w4a16p": "gemm_1xnbias_clamp_f16_f16p_qsi4c2p",
    "igemmclp": "igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp",
    # output-type siblings of the W4A8 types: f16 / bf16 D, C, bias and clamp bounds
    "w4a8h": "gemm_1xnbias_clamp_f16_qai8dx_qsi4cxt",
    "w4a8b": "gemm_1xnbias_clamp_bf16_qai8dx_qsi4cxt",
    "w4a8hp": "gemm_1xnbias_clamp_f16_qai8dxp_qsi4cxp",
    "w4a8bp": "gemm_1xnbias_clamp_bf16_qai8dxp_qsi4cxp",
    # f32-output siblings of the W4A16 types: f32 C, bias, clamp bounds and D
    "w4a16f": "gemm_1xnbias_clamp_f32_f16_qsi4c2t",
    "w4a16fp": "gemm_1xnbias_clamp_f32_f16p_qsi4c2p",
    # W8A8 with per-row dynamically quantized A (qai8dx x qsi8cx), f32 / f16 D
    "w8dyn": "gemm_1xnbias_clamp_f32_qai8dx_qsi8cxt",
    "w8dynp": "gemm_1xnbias_clamp_f32_qai8dxp_qsi8cxp",
    "w8dynh": "gemm_1xnbias_clamp_f16_qai8dx_qsi8cxt",
    "w8dynhp": "gemm_1xnbias_clamp_f16_qai8dxp_qsi8cxp",
    # explicit-im2col convolution (channel-last): im2col (or im2col + pack) and the W8A8 GEMM
    "convcl": "convcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt",
    "convclp": "convcl_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp",
    # channel-first int8: weights x [k, n] activations with per-row (Mx1) bias and requantization
    "mx1": "gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8",
    "mx1p": "gemm_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p",
    "convcf": "convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8",
    "convcfp": "convcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8p",
    "igemmcf": "igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dx_qai8",
    "igemmcfp": "igemmcf_mx1bias_reqi32toi8_clamp_qai8_qsi8dxp_qai8",
}


class QAI8QSI8CXParams(ctypes.Structure):
    """struct tqt_qai8_qai8_qsi8cx_params (reference tqt_params_i8_i8.h:16-24)."""

    _fields_ = [
        ("scale_a", ctypes.c_float),
        ("zero_point_a", ctypes.c_int32),
        ("scale_b", c_vp),
        ("quant_channel_b", ctypes.c_int32),
        ("scale_d", ctypes.c_float),
        ("zero_point_d", ctypes.c_int32),
    ]


class QAI8DXQSI4CXParams(ctypes.Structure):
    """struct tqt_qai8dx_qsi4cx_params (reference tqt_params_i8_i4.h:23-28)."""

    _fields_ = [("scale_a", c_vp), ("zero_point_a", c_vp), ("scale_b", c_vp)]


class QAI8DXPQSI8CXPParams(ctypes.Structure):
    """struct tqt_qai8dxp_qsi8cxp_params (reference tqt_params_i8_i8.h:45-50)."""

    _fields_ = [("scale_a", c_vp), ("zero_point_a", c_vp), ("scale_b", c_vp)]


class QAI8QSI8DXQAI8Params(ctypes.Structure):
    """struct tqt_qai8_qsi8dx_qai8_params (reference tqt_params_i8_i8.h:28-36)."""

    _fields_ = [
        ("scale_a", c_vp),
        ("quant_channel_a", ctypes.c_int32),
        ("scale_b", ctypes.c_float),
        ("zero_point_b", ctypes.c_int32),
        ("scale_d", ctypes.c_float),
        ("zero_point_d", ctypes.c_int32),
    ]


class ConvParams(ctypes.Structure):
    """struct tqt_conv_params (reference src/common/tqt_conv.h:20-31)."""

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


def conv_params(input_shape, kernel_shape, stride, dilation, pad, ic, oc, groups=1):
    """Build ConvParams with the output shape the reference test harness computes
    (test/common/conv_test_runner.h: (in + 2 pad - dil (k - 1) - 1) / stride + 1)."""
    p = ConvParams()
    out = [
        (input_shape[i] + 2 * pad[i] - dilation[i] * (kernel_shape[i] - 1) - 1) // stride[i] + 1
        for i in range(3)
    ]
    for i in range(3):
        p.input_shape[i] = input_shape[i]
        p.output_shape[i] = out[i]
        p.kernel_shape[i] = kernel_shape[i]
        p.stride[i] = stride[i]
        p.dilation[i] = dilation[i]
        p.pad[i] = pad[i]
    p.input_channel = ic
    p.output_channel = oc
    p.groups = groups
    return p


def _sym(kind, action):
    name = KERNELS[kind]
    if action.endswith("_async"):
        return _sym(kind, action[:-len("_async")]) + "_async"
    if action == "run":
        verb = "run_igemm" if name.startswith("igemmcl") else "run"
        return "tqt_%s_%s_%s" % (verb, name, VARIANT)
    return "tqt_%s_%s_%s" % (action, name, VARIANT)


# C type (as written in include/*.h, parameter name dropped) -> ctypes type.
_CTYPES = {
    "size_t": c_size,
    "int32_t": ctypes.c_int32,
    "int8_t": ctypes.c_int8,
    "float": ctypes.c_float,
    "const void *": c_vp,
    "void *": c_vp,
    "const float *": c_vp,
    "float *": c_vp,
    "int8_t *": c_vp,
    "int32_t *": c_vp,
    "const char *": ctypes.c_char_p,
    "const tqt_conv_params *": ctypes.POINTER(ConvParams),
    "const struct tqt_conv_params *": ctypes.POINTER(ConvParams),
    "const struct tqt_qai8_qai8_qsi8cx_params *": ctypes.POINTER(QAI8QSI8CXParams),
    "const struct tqt_qai8dx_qsi4cx_params *": ctypes.POINTER(QAI8DXQSI4CXParams),
    "const struct tqt_qai8dxp_qsi8cxp_params *": ctypes.POINTER(QAI8DXPQSI8CXPParams),
    "const struct tqt_qai8_qsi8dx_qai8_params *": ctypes.POINTER(QAI8QSI8DXQAI8Params),
}
# f16 / bf16 values are passed in SSE registers on x86-64, which ctypes cannot fill: functions
# taking them are checked for export but not bound (the test shim in tests/abi_shim calls them).
_UNBOUND = ("float16_t", "bfloat16_t")
_DECL = re.compile(r"^(size_t|void|const char \*)\s*(tqt_\w+)\s*\(([^;]*?)\)\s*;", re.M)


def declarations(include_dir=INCLUDE_DIR):
    """{symbol: (restype, argtypes)} for every function include/*.h declares; argtypes is None
    for a function with an argument ctypes cannot pass."""
    decls = {}
    for header in sorted(glob.glob(os.path.join(include_dir, "*.h"))):
        with open(header) as fh:
            text = re.sub(r"/\*.*?\*/", " ", fh.read(), flags=re.S)
        for ret, name, args in _DECL.findall(text):
            args = " ".join(args.split())
            params = [] if args in ("", "void") else [p.strip() for p in args.split(",")]
            types = [re.sub(r"\s*\b\w+$", "", p) for p in params]
            restype = None if ret == "void" else _CTYPES[ret]
            if any(t in _UNBOUND for t in types):
                decls[name] = (restype, None)
            else:
                decls[name] = (restype, [_CTYPES[t] for t in types])
    if not decls:
        raise RuntimeError("no tqt_ declarations found under %s" % include_dir)
    return decls


class Lib:
    """Typed access to every exported function: ``lib.fn(kind, action)``."""

    def __init__(self, path=LIB_PATH):
        if not os.path.exists(path):
            raise RuntimeError(
                "gfx950 library not built: %s missing (run make -C torq-tile_amd)" % path)
        self.path = path
        self.dll = ctypes.CDLL(path)
        self._decls = declarations()
        self._fns = {}
        for name, (res, args) in self._decls.items():
            f = getattr(self.dll, name)  # AttributeError: declared but not exported
            if args is None:
                continue
            f.restype = res
            f.argtypes = args
            self._fns[name] = f
        # dynamic per-row activation quantization (include/tqt_quantize_qai8dx_gfx950.h)
        self.quantize = self._fns["tqt_run_quantize_qai8dx_f32_gfx950"]
        self.quantize_async = self._fns["tqt_run_quantize_qai8dx_f32_gfx950_async"]
        # the fused decode step: quantization + W4A8 GEMV
        # (include/tqt_quantize_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_gfx950.h)
        self.quantize_gemm = self._fns[
            "tqt_run_quantize_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_gfx950"]
        self.quantize_gemm_async = self._fns[
            "tqt_run_quantize_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_gfx950_async"]

    def fn(self, kind, action):
        return self._fns[_sym(kind, action)]

    def symbol_names(self):
        return sorted(self._decls)


_LIB = None


def load():
    global _LIB
    if _LIB is None:
        _LIB = Lib()
    return _LIB
