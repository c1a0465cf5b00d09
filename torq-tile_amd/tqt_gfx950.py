"""ctypes binding of the gfx950 TORQ-Tile C ABI (libtorq_tile_gfx950.so).

This is the Python-side stub a framework maintainer would add to call the library: it declares
every exported symbol with its exact C signature (include/*.h) and mirrors the parameter
structs field for field. Buffers are passed as raw device addresses (int); torch tensors on a
ROCm device provide them via ``tensor.data_ptr()``.

Loading fails loudly: there is no CPU fallback. ``load()`` raises if the shared library has not
been built (``make -C torq-tile_amd``).
"""

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtorq_tile_gfx950.so")

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


# (action, restype, argtypes) per kernel type; float16 / bfloat16 clamps are not callable from
# ctypes and those runs are reached through the test shim instead.
_GEMM_I8_ARGS = [c_size, c_size, c_size, c_vp, c_size, c_size, c_vp, c_size, c_size, c_vp,
                 c_size, c_vp, c_size]
_SIGS = {
    "clamp": {
        "get_m_step": (c_size, []),
        "get_n_step": (c_size, []),
        "get_a_offset": (c_size, [c_size] * 3),
        "get_b_offset": (c_size, [c_size] * 3),
        "get_c_offset": (c_size, [c_size] * 3),
        "get_d_offset": (c_size, [c_size] * 3),
        "get_d_size": (c_size, [c_size] * 2),
        "run": (None, _GEMM_I8_ARGS + [ctypes.c_int32, ctypes.c_int32]),
        "run_async": (None, _GEMM_I8_ARGS + [ctypes.c_int32, ctypes.c_int32, c_vp]),
    },
    "w8a8": {
        "get_m_step": (c_size, []),
        "get_n_step": (c_size, []),
        "get_a_offset": (c_size, [c_size] * 3),
        "get_b_offset": (c_size, [c_size] * 3),
        "get_c_offset": (c_size, [c_size] * 3),
        "get_bias_offset": (c_size, [c_size]),
        "get_d_offset": (c_size, [c_size] * 3),
        "get_d_size": (c_size, [c_size] * 2),
        "run": (None, _GEMM_I8_ARGS + [c_vp, ctypes.c_int8, ctypes.c_int8,
                                       ctypes.POINTER(QAI8QSI8CXParams)]),
        "run_async": (None, _GEMM_I8_ARGS + [c_vp, ctypes.c_int8, ctypes.c_int8,
                                             ctypes.POINTER(QAI8QSI8CXParams), c_vp]),
    },
    "w4a8": {
        "get_m_step": (c_size, []),
        "get_n_step": (c_size, []),
        "get_a_offset": (c_size, [c_size] * 3),
        "get_b_offset": (c_size, [c_size] * 3),
        "get_c_offset": (c_size, [c_size] * 3),
        "get_bias_offset": (c_size, [c_size]),
        "get_d_offset": (c_size, [c_size] * 3),
        "get_d_size": (c_size, [c_size] * 2),
        "run": (None, _GEMM_I8_ARGS + [c_vp, ctypes.c_float, ctypes.c_float,
                                       ctypes.POINTER(QAI8DXQSI4CXParams)]),
        "run_async": (None, _GEMM_I8_ARGS + [c_vp, ctypes.c_float, ctypes.c_float,
                                             ctypes.POINTER(QAI8DXQSI4CXParams), c_vp]),
    },
    "w4a16": {
        "get_m_step": (c_size, []),
        "get_n_step": (c_size, []),
        "get_a_offset": (c_size, [c_size] * 4),
        "get_b_offset": (c_size, [c_size] * 4),
        "get_scale_b_offset": (c_size, [c_size] * 3),
        "get_c_offset": (c_size, [c_size] * 3),
        "get_bias_offset": (c_size, [c_size]),
        "get_d_offset": (c_size, [c_size] * 3),
        "get_d_size": (c_size, [c_size] * 2),
    },
    "igemmcl": {
        "get_m_step": (c_size, []),
        "get_n_step": (c_size, []),
        "get_b_offset": (c_size, [c_size] * 3),
        "get_c_offset": (c_size, [c_size] * 3),
        "get_bias_offset": (c_size, [c_size]),
        "get_d_offset": (c_size, [c_size] * 3),
        "get_d_size": (c_size, [c_size] * 2),
        "run": (None, [c_size, c_size, c_size, c_vp, c_size, c_size, c_size, c_vp, c_size, c_size,
                       c_vp, c_size, c_vp, c_size, c_vp, ctypes.c_int8, ctypes.c_int8,
                       ctypes.POINTER(ConvParams), ctypes.POINTER(QAI8QSI8CXParams)]),
        "run_async": (None, [c_size, c_size, c_size, c_vp, c_size, c_size, c_size, c_vp, c_size,
                             c_size, c_vp, c_size, c_vp, c_size, c_vp, ctypes.c_int8,
                             ctypes.c_int8, ctypes.POINTER(ConvParams),
                             ctypes.POINTER(QAI8QSI8CXParams), c_vp]),
    },
}


_PACK = [c_size] * 5 + [c_vp, c_vp]  # (rows, k, ld, ld_packed, k_idx, src, dst)
_OFFP = [c_size] * 4                  # (idx, k_idx, ld, actual)


def _packed_sigs(base, packers, run_args, offsets):
    sig = {
        "get_m_step": (c_size, []),
        "get_n_step": (c_size, []),
        "get_c_offset": (c_size, [c_size] * 3),
        "get_d_offset": (c_size, [c_size] * 3),
        "get_d_size": (c_size, [c_size] * 2),
    }
    for what in offsets:
        sig[what] = (c_size, _OFFP if "packed_offset" in what else
                     ([c_size] * 3 if what == "get_a_offset" else [c_size] * 2))
    if base != "clamp":
        sig["get_bias_offset"] = (c_size, [c_size])
    for pk in packers:
        sig[pk] = (None, _PACK)
        sig[pk + "_async"] = (None, _PACK + [c_vp])
    if run_args is not None:
        sig["run"] = (None, run_args)
        sig["run_async"] = (None, run_args + [c_vp])
    return sig


_I8_REQ = [c_vp, ctypes.c_int8, ctypes.c_int8, ctypes.POINTER(QAI8QSI8CXParams)]
_SIGS["clampp"] = _packed_sigs(
    "clamp", ["run_a_pack", "run_b_pack", "run_bt_pack"],
    _GEMM_I8_ARGS + [ctypes.c_int32, ctypes.c_int32],
    ["get_a_packed_offset", "get_b_packed_offset", "get_a_packed_size", "get_b_packed_size"])
_SIGS["w8a8pb"] = _packed_sigs(
    "w8a8", ["run_b_pack", "run_bt_pack"], _GEMM_I8_ARGS + _I8_REQ,
    ["get_a_offset", "get_b_packed_offset", "get_b_packed_size"])
_SIGS["w8a8p"] = _packed_sigs(
    "w8a8", ["run_a_pack", "run_b_pack", "run_bt_pack"], _GEMM_I8_ARGS + _I8_REQ,
    ["get_a_packed_offset", "get_b_packed_offset", "get_a_packed_size", "get_b_packed_size"])
_SIGS["w4a8p"] = _packed_sigs(
    "w4a8", ["run_a_pack", "run_bt_pack"],
    _GEMM_I8_ARGS + [c_vp, ctypes.c_float, ctypes.c_float, ctypes.POINTER(QAI8DXQSI4CXParams)],
    ["get_a_packed_offset", "get_b_packed_offset", "get_a_packed_size", "get_b_packed_size"])
# float16 clamps: the run is reached through the test shim (tqts_run_w4a16p)
_SIGS["w4a16p"] = _packed_sigs(
    "w4a16", ["run_a_pack", "run_bt_pack"], None,
    ["get_a_packed_offset", "get_b_packed_offset", "get_a_packed_size", "get_b_packed_size"])
_SIGS["w4a16p"]["get_scale_b_offset"] = (c_size, [c_size] * 3)
_SIGS["igemmclp"] = _packed_sigs(
    "igemmcl", ["run_bt_pack"], _SIGS["igemmcl"]["run"][1],
    ["get_b_packed_offset", "get_b_packed_size"])
# f16 / bf16 clamps: the runs are reached through the test shim (tqts_run_w4a8h)
for _kind in ("w4a8h", "w4a8b"):
    _SIGS[_kind] = {a: v for a, v in _SIGS["w4a8"].items() if not a.startswith("run")}
for _kind in ("w4a8hp", "w4a8bp"):
    _SIGS[_kind] = _packed_sigs(
        "w4a8", ["run_a_pack", "run_bt_pack"], None,
        ["get_a_packed_offset", "get_b_packed_offset", "get_a_packed_size", "get_b_packed_size"])
_W4A16F_RUN = ([c_size] * 4 + [c_vp, c_size, c_size] * 2 +
               [c_vp, c_size, c_vp, c_size, c_vp, c_size, c_vp, ctypes.c_float, ctypes.c_float])
_SIGS["w4a16f"] = dict(_SIGS["w4a16"], run=(None, _W4A16F_RUN),
                       run_async=(None, _W4A16F_RUN + [c_vp]))
_SIGS["w4a16fp"] = _packed_sigs(
    "w4a16", ["run_a_pack", "run_bt_pack"], _W4A16F_RUN,
    ["get_a_packed_offset", "get_b_packed_offset", "get_a_packed_size", "get_b_packed_size"])
_SIGS["w4a16fp"]["get_scale_b_offset"] = (c_size, [c_size] * 3)
_DYN_RUN = _GEMM_I8_ARGS + [c_vp, ctypes.c_float, ctypes.c_float,
                            ctypes.POINTER(QAI8DXPQSI8CXPParams)]
_SIGS["w8dyn"] = {a: v for a, v in _SIGS["w4a8"].items() if not a.startswith("run")}
_SIGS["w8dyn"].update(run=(None, _DYN_RUN), run_async=(None, _DYN_RUN + [c_vp]))
_SIGS["w8dynh"] = {a: v for a, v in _SIGS["w4a8"].items() if not a.startswith("run")}
_SIGS["w8dynp"] = _packed_sigs(
    "w8dyn", ["run_a_pack", "run_b_pack", "run_bt_pack"], _DYN_RUN,
    ["get_a_packed_offset", "get_b_packed_offset", "get_a_packed_size", "get_b_packed_size"])
_SIGS["w8dynhp"] = _packed_sigs(
    "w8dyn", ["run_a_pack", "run_b_pack", "run_bt_pack"], None,
    ["get_a_packed_offset", "get_b_packed_offset", "get_a_packed_size", "get_b_packed_size"])
_IM2COL = [c_size, c_vp, c_vp, ctypes.POINTER(ConvParams)]
_IM2COLPACK = [c_size, c_vp, c_size, c_size, c_vp, ctypes.POINTER(ConvParams)]
_SIGS["convcl"] = {
    "get_m_step": (c_size, []),
    "get_n_step": (c_size, []),
    "get_b_offset": (c_size, [c_size] * 3),
    "get_c_offset": (c_size, [c_size] * 3),
    "get_bias_offset": (c_size, [c_size]),
    "get_d_offset": (c_size, [c_size] * 3),
    "get_d_size": (c_size, [c_size] * 2),
    "get_a_im2col_size": (c_size, [c_size] * 2),
    "get_a_im2col_offset": (c_size, [c_size] * 3),
    "run_im2col": (None, _IM2COL),
    "run_im2col_async": (None, _IM2COL + [c_vp]),
    "run_conv": _SIGS["w8a8"]["run"],
    "run_conv_async": _SIGS["w8a8"]["run_async"],
}
_SIGS["convclp"] = {
    "get_m_step": (c_size, []),
    "get_n_step": (c_size, []),
    "get_a_im2colpack_offset": (c_size, _OFFP),
    "get_b_packed_offset": (c_size, _OFFP),
    "get_c_offset": (c_size, [c_size] * 3),
    "get_bias_offset": (c_size, [c_size]),
    "get_d_offset": (c_size, [c_size] * 3),
    "get_d_size": (c_size, [c_size] * 2),
    "get_a_im2colpack_size": (c_size, [c_size] * 2),
    "get_b_packed_size": (c_size, [c_size] * 2),
    "run_bt_pack": (None, _PACK),
    "run_bt_pack_async": (None, _PACK + [c_vp]),
    "run_a_im2colpack": (None, _IM2COLPACK),
    "run_a_im2colpack_async": (None, _IM2COLPACK + [c_vp]),
    "run_conv": _SIGS["w8a8p"]["run"],
    "run_conv_async": _SIGS["w8a8p"]["run_async"],
}
_MX1_REQ = [c_vp, ctypes.c_int8, ctypes.c_int8, ctypes.POINTER(QAI8QSI8DXQAI8Params)]
_SIGS["mx1"] = {a: v for a, v in _SIGS["w8a8"].items() if not a.startswith("run")}
_SIGS["mx1"].update(run=(None, _GEMM_I8_ARGS + _MX1_REQ),
                    run_async=(None, _GEMM_I8_ARGS + _MX1_REQ + [c_vp]))
_SIGS["mx1p"] = _packed_sigs(
    "mx1", ["run_a_pack", "run_b_pack", "run_bt_pack"], _GEMM_I8_ARGS + _MX1_REQ,
    ["get_a_packed_offset", "get_b_packed_offset", "get_a_packed_size", "get_b_packed_size"])
_SIGS["convcf"] = {
    "get_m_step": (c_size, []),
    "get_n_step": (c_size, []),
    "get_a_offset": (c_size, [c_size] * 3),
    "get_c_offset": (c_size, [c_size] * 3),
    "get_bias_offset": (c_size, [c_size]),
    "get_d_offset": (c_size, [c_size] * 3),
    "get_d_size": (c_size, [c_size] * 2),
    "get_b_im2col_size": (c_size, [c_size] * 2),
    "get_b_im2col_offset": (c_size, [c_size] * 3),
    "run_im2col": (None, _IM2COL),
    "run_im2col_async": (None, _IM2COL + [c_vp]),
    "run_conv": _SIGS["mx1"]["run"],
    "run_conv_async": _SIGS["mx1"]["run_async"],
}
_SIGS["convcfp"] = {
    "get_m_step": (c_size, []),
    "get_n_step": (c_size, []),
    "get_a_packed_offset": (c_size, _OFFP),
    "get_b_im2colpack_offset": (c_size, _OFFP),
    "get_c_offset": (c_size, [c_size] * 3),
    "get_bias_offset": (c_size, [c_size]),
    "get_d_offset": (c_size, [c_size] * 3),
    "get_d_size": (c_size, [c_size] * 2),
    "get_a_packed_size": (c_size, [c_size] * 2),
    "get_b_im2colpack_size": (c_size, [c_size] * 2),
    "run_a_pack": (None, _PACK),
    "run_a_pack_async": (None, _PACK + [c_vp]),
    "run_b_im2colpack": (None, _IM2COLPACK),
    "run_b_im2colpack_async": (None, _IM2COLPACK + [c_vp]),
    "run_conv": _SIGS["mx1p"]["run"],
    "run_conv_async": _SIGS["mx1p"]["run_async"],
}
_IGEMMCF = ([c_size] * 3 + [c_vp, c_size, c_size, c_size, c_vp, c_size, c_size, c_vp, c_size, c_vp,
                            c_size, c_vp, ctypes.c_int8, ctypes.c_int8,
                            ctypes.POINTER(ConvParams), ctypes.POINTER(QAI8QSI8DXQAI8Params)])
_SIGS["igemmcf"] = {
    "get_m_step": (c_size, []),
    "get_n_step": (c_size, []),
    "get_a_offset": (c_size, [c_size] * 3),
    "get_c_offset": (c_size, [c_size] * 3),
    "get_bias_offset": (c_size, [c_size]),
    "get_d_offset": (c_size, [c_size] * 3),
    "get_d_size": (c_size, [c_size] * 2),
    "run_igemm": (None, _IGEMMCF),
    "run_igemm_async": (None, _IGEMMCF + [c_vp]),
}
_SIGS["igemmcfp"] = {
    "get_m_step": (c_size, []),
    "get_n_step": (c_size, []),
    "get_a_packed_offset": (c_size, _OFFP),
    "get_c_offset": (c_size, [c_size] * 3),
    "get_bias_offset": (c_size, [c_size]),
    "get_d_offset": (c_size, [c_size] * 3),
    "get_d_size": (c_size, [c_size] * 2),
    "get_a_packed_size": (c_size, [c_size] * 2),
    "run_a_pack": (None, _PACK),
    "run_a_pack_async": (None, _PACK + [c_vp]),
    "run_igemm": (None, _IGEMMCF),
    "run_igemm_async": (None, _IGEMMCF + [c_vp]),
}
_SHIM_RUNS = ("w4a16", "w4a16p", "w4a8h", "w4a8b", "w4a8hp", "w4a8bp", "w8dynh", "w8dynhp")


class Lib:
    """Typed access to every exported function: ``lib.fn(kind, action)``."""

    def __init__(self, path=LIB_PATH):
        if not os.path.exists(path):
            raise RuntimeError(
                "gfx950 library not built: %s missing (run make -C torq-tile_amd)" % path)
        self.path = path
        self.dll = ctypes.CDLL(path)
        self._fns = {}
        for kind, actions in _SIGS.items():
            for action, (res, args) in actions.items():
                f = getattr(self.dll, _sym(kind, action))
                f.restype = res
                f.argtypes = args
                self._fns[(kind, action)] = f
        self.dll.tqt_gfx950_target.restype = ctypes.c_char_p
        self.dll.tqt_gfx950_target.argtypes = []
        # dynamic per-row activation quantization (include/tqt_quantize_qai8dx_gfx950.h)
        qargs = [c_size, c_size, c_vp, c_size, c_vp, c_size, c_vp, c_vp]
        self.quantize = self.dll.tqt_run_quantize_qai8dx_f32_gfx950
        self.quantize.restype = None
        self.quantize.argtypes = qargs
        self.quantize_async = self.dll.tqt_run_quantize_qai8dx_f32_gfx950_async
        self.quantize_async.restype = None
        self.quantize_async.argtypes = qargs + [c_vp]

    def fn(self, kind, action):
        return self._fns[(kind, action)]

    def symbol_names(self):
        names = [_sym(k, a) for (k, a) in self._fns]
        for kind in _SHIM_RUNS:
            names += [_sym(kind, "run"), _sym(kind, "run_async")]
        names += ["tqt_gfx950_target", "tqt_run_quantize_qai8dx_f32_gfx950",
                  "tqt_run_quantize_qai8dx_f32_gfx950_async"]
        return sorted(set(names))


_LIB = None


def load():
    global _LIB
    if _LIB is None:
        _LIB = Lib()
    return _LIB
