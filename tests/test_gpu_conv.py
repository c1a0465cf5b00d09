"""Explicit-im2col convolution (convcl) on the GPU.

* run_im2col: byte-exact against the oracle's im2col (tqto_im2col_cl_i8, itself pinned to the
  reference's tqt_im2col_cl through ref_im2col.npz), over strides, dilations, paddings, groups,
  channel counts on and off the 16-byte fast path, and a 3-D (batch-in-depth) input.
* run_a_im2colpack: byte-exact against the packed-layout restatement (pack_panels) of that
  im2col, with ld_packed and k_idx sub-buffers.
* the convolution: im2col (or im2col + pack) then run_conv, through the interface structs,
  bit-exact against the oracle's implicit GEMM (tqto_igemmcl_qsi8cxt, pinned as im2col + GEMM),
  including BASELINE cfg 5's shape.
"""

import ctypes

import numpy as np
import pytest

import tqt_testlib as T

pytestmark = pytest.mark.gpu

SENTINEL = 0x5A


def _g():
    import gpu_run

    return gpu_run


def _torch():
    import torch

    return torch


def lib_conv(conv):
    cp = _g()._mod.ConvParams()
    ctypes.memmove(ctypes.byref(cp), ctypes.byref(conv), ctypes.sizeof(cp))
    return cp


def oracle_im2col(inp, conv, group_idx=0):
    icg = conv.input_channel // conv.groups
    M = conv.output_shape[0] * conv.output_shape[1] * conv.output_shape[2]
    K = conv.kernel_shape[0] * conv.kernel_shape[1] * conv.kernel_shape[2] * icg
    out = np.zeros((M, K), np.int8)
    T.oracle().tqto_im2col_cl_i8(group_idx, T.ptr(np.ascontiguousarray(inp)), T.ptr(out),
                                 ctypes.byref(conv))
    return out


def gpu_im2col(inp, conv, group_idx=0, offset=0):
    torch = _torch()
    M = conv.output_shape[0] * conv.output_shape[1] * conv.output_shape[2]
    K = conv.kernel_shape[0] * conv.kernel_shape[1] * conv.kernel_shape[2] * (
        conv.input_channel // conv.groups)
    src = np.zeros(inp.size + offset, np.int8)
    src[offset:] = inp.ravel()
    dsrc = _g().dev(src)
    out = torch.full((M * K + offset,), SENTINEL, dtype=torch.int8, device="cuda:0")
    _g().lib().fn("convcl", "run_im2col")(group_idx, dsrc.data_ptr() + offset,
                                          out.data_ptr() + offset, ctypes.byref(lib_conv(conv)))
    o = out.cpu().numpy()
    assert (o[:offset] == SENTINEL).all()
    return o[offset:].reshape(M, K)


def gen_input(ID, IH, IW, IC, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(-128, 128, size=(ID, IH, IW, IC), dtype=np.int64).astype(np.int8)


# (ID, IH, IW, IC, groups, kernel (kd, kh, kw), stride, pad, dilation)
IM2COL_CASES = [
    (1, 8, 8, 3, 1, (1, 3, 3), (1, 1, 1), (0, 1, 1), (1, 1, 1)),
    (1, 8, 8, 16, 1, (1, 3, 3), (1, 1, 1), (0, 0, 0), (1, 1, 1)),
    (1, 9, 7, 32, 1, (1, 3, 5), (1, 2, 2), (0, 1, 2), (1, 1, 1)),
    (1, 16, 16, 64, 1, (1, 3, 3), (1, 1, 1), (0, 2, 2), (1, 2, 2)),
    (2, 10, 9, 48, 3, (1, 3, 3), (1, 1, 1), (0, 1, 1), (1, 1, 1)),
    (1, 7, 11, 24, 2, (1, 2, 3), (1, 2, 1), (0, 1, 0), (1, 1, 2)),
    (3, 6, 6, 16, 1, (2, 3, 3), (1, 1, 1), (1, 1, 1), (1, 1, 1)),
    (1, 5, 5, 7, 1, (1, 1, 1), (1, 1, 1), (0, 0, 0), (1, 1, 1)),
]


@pytest.mark.parametrize("ID,IH,IW,IC,groups,kern,stride,pad,dil", IM2COL_CASES)
def test_im2col_cl_matches_oracle(gpu, ID, IH, IW, IC, groups, kern, stride, pad, dil):
    inp = gen_input(ID, IH, IW, IC, seed=IC + IH)
    conv = T.make_conv((ID, IH, IW), kern, stride, dil, pad, IC, 8, groups)
    for g in range(groups):
        np.testing.assert_array_equal(gpu_im2col(inp, conv, g), oracle_im2col(inp, conv, g))
    # an unaligned source and destination take the byte path and must agree too
    np.testing.assert_array_equal(gpu_im2col(inp, conv, groups - 1, offset=3),
                                  oracle_im2col(inp, conv, groups - 1))


@pytest.mark.parametrize("ID,IH,IW,IC,groups,kern,stride,pad,dil", IM2COL_CASES[1:6])
def test_im2colpack_matches_packed_layout(gpu, ID, IH, IW, IC, groups, kern, stride, pad, dil):
    torch = _torch()
    inp = gen_input(ID, IH, IW, IC, seed=IC * 3 + IW)
    conv = T.make_conv((ID, IH, IW), kern, stride, dil, pad, IC, 8, groups)
    dsrc = _g().dev(inp)
    cp = lib_conv(conv)
    for g in range(groups):
        A = oracle_im2col(inp, conv, g)
        M, K = A.shape
        # k_idx moves a narrow last panel back by k_idx * (128 - w) bytes (the packers' tail
        # rule); the whole im2col row is written either way
        for ldp, k_idx in ((K, 0), (K + 32, 0), (K, 16)):
            n_out = M * ldp
            out = torch.full((n_out,), SENTINEL, dtype=torch.int8, device="cuda:0")
            _g().lib().fn("convclp", "run_a_im2colpack")(g, dsrc.data_ptr(), ldp, k_idx,
                                                        out.data_ptr(), ctypes.byref(cp))
            exp = T.pack_panels(A.view(np.uint8), 128, 16, ld_packed=ldp, shift=k_idx,
                                out=np.full(n_out, SENTINEL, np.uint8))
            np.testing.assert_array_equal(out.cpu().numpy().view(np.uint8), exp)


def run_convcl(shim, d, packed):
    torch = _torch()
    conv, W = d["conv"], d["W"]
    M = conv.output_shape[0] * conv.output_shape[1] * conv.output_shape[2]
    n, K = W.shape
    din = _g().dev(d["inp"])
    dbias, dsb = _g().dev(d["bias"]), _g().dev(d["scale_b"])
    if packed:
        dWs = _g().dev(W)
        dW = torch.empty(n * K, dtype=torch.int8, device="cuda:0")
        _g().lib().fn("convclp", "run_bt_pack")(n, K, K, K, 0, dWs.data_ptr(), dW.data_ptr())
    else:
        dW = _g().dev(W)
    Abuf = torch.empty(max(M * K, 1), dtype=torch.int8, device="cuda:0")
    dD = torch.zeros((M, n), dtype=torch.int8, device="cuda:0")
    p = _g().w8a8_params(dict(d, B=W), dsb)
    f = shim.tqts_run_convcl
    f.restype = None
    f.argtypes = [ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p,
                  ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int8,
                  ctypes.c_int8, ctypes.c_void_p]
    f(int(packed), 0, din.data_ptr(), Abuf.data_ptr(), ctypes.byref(lib_conv(conv)), M, n, K,
      dW.data_ptr(), dD.data_ptr(), dbias.data_ptr(), -128, 127, ctypes.byref(p))
    torch.cuda.synchronize()
    return dD.cpu().numpy()


CONV_CASES = [(1, 8, 8, 3, 16, 3, 3, (1, 1), (1, 1), (1, 1)),
              (1, 12, 10, 32, 40, 3, 3, (1, 1), (1, 1), (1, 1)),
              (2, 9, 9, 16, 24, 3, 3, (2, 2), (0, 0), (1, 1)),
              (1, 16, 16, 64, 128, 1, 1, (1, 1), (0, 0), (1, 1)),
              (1, 11, 13, 24, 33, 3, 5, (1, 2), (2, 1), (1, 2))]


@pytest.mark.parametrize("ID,IH,IW,IC,OC,KH,KW,stride,pad,dil", CONV_CASES)
@pytest.mark.parametrize("packed", [False, True], ids=["plain", "packed"])
def test_convcl_matches_implicit_gemm_oracle(gpu, shim, packed, ID, IH, IW, IC, OC, KH, KW,
                                             stride, pad, dil):
    d = T.gen_igemmcl(ID, IH, IW, IC, OC, KH, KW, stride=stride, pad=pad, dil=dil,
                      seed=IC + OC + IH)
    got = run_convcl(shim, d, packed)
    exp = T.oracle_igemmcl(d["inp"], d["W"], d["bias"], -128, 127, d["conv"], d["scale_a"],
                           d["scale_b"], OC, d["scale_d"], d["zp_d"])
    np.testing.assert_array_equal(got, exp)


def test_convcl_config5_shape(gpu, shim):
    """BASELINE cfg 5's shape (NHWC 8x56x56x128, 3x3, pad 1, OC 128) through explicit im2col:
    equal to the implicit-GEMM kernel's output, which test_gpu_parity.py holds to the oracle at
    this size."""
    d = T.gen_igemmcl(8, 56, 56, 128, 128, 3, 3, pad=(1, 1), seed=42)
    implicit = _g().run_igemmcl(d)
    for packed in (False, True):
        np.testing.assert_array_equal(run_convcl(shim, d, packed), implicit)
