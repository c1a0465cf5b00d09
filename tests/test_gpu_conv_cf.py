"""Channel-first int8 kernels on the GPU, bit-exact against the oracle:

* gemm_mx1bias (weights A [m, k] with per-row scale, activations B [k, n], per-row bias and
  requantization) and its packed sibling, on the streaming, double-buffered and generic paths;
  the oracle is pinned as the transposed W8A8 oracle (test_oracle.py);
* convcf: the channel-first im2col (byte-exact vs the oracle's, itself pinned to the
  reference's tqt_im2col_cf through ref_im2col_cf.npz), the fused im2col + pack of B, and the
  convolution through the interface structs;
* igemmcf: the implicit channel-first GEMM (B gathered from the NCDHW input), plain and packed
  weights, over pixel windows, groups, strides, dilation and padding, against the oracle's
  im2col + mx1bias composition.
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


def mx1_params(d, dsa):
    P = _g()._mod.QAI8QSI8DXQAI8Params
    return P(dsa.data_ptr(), int(d["qca"]), float(d["scale_b"]), 0, float(d["scale_d"]),
             int(d["zp_d"]))


def oracle(d):
    return T.oracle_mx1bias(d["A"], d["B"], d["C"], d["bias"], -128, 127, d["scale_a"], d["qca"],
                            d["scale_b"], d["scale_d"], d["zp_d"])


def run_mx1(d, packed):
    torch = _torch()
    g = _g()
    A, B = d["A"], d["B"]
    m, k = A.shape
    n = B.shape[1]
    dA, dB = g.dev(A), g.dev(B)
    if packed:
        pA = torch.empty(max(m * k, 1), dtype=torch.int8, device="cuda:0")
        pB = torch.empty(max(n * k, 1), dtype=torch.int8, device="cuda:0")
        g.lib().fn("mx1p", "run_a_pack")(m, k, k, k, 0, dA.data_ptr(), pA.data_ptr())
        g.lib().fn("mx1p", "run_b_pack")(n, k, n, k, 0, dB.data_ptr(), pB.data_ptr())
        dA, dB, ldb = pA, pB, k
    else:
        ldb = n
    dC, dbias, dsa = g.dev(d["C"]), g.dev(d["bias"]), g.dev(d["scale_a"])
    dD = torch.zeros((m, n), dtype=torch.int8, device="cuda:0")
    p = mx1_params(d, dsa)
    g.lib().fn("mx1p" if packed else "mx1", "run")(
        m, n, k, dA.data_ptr(), k, 0, dB.data_ptr(), ldb, 0, g.dp(dC), n, dD.data_ptr(), n,
        g.dp(dbias), -128, 127, ctypes.byref(p))
    return dD.cpu().numpy()


# (m, n, k, with_c): k % 128 == 0 takes the streaming kernel when packed, k % 16 == 0 the
# double-buffered one, other k the generic kernel; qca = 1 shares row 0's multiplier
MX1_SHAPES = [(128, 256, 512, False), (130, 260, 192, True), (64, 200, 1152, False),
              (37, 45, 70, True), (3, 8, 11, False), (257, 129, 256, True)]


@pytest.mark.parametrize("m,n,k,with_c", MX1_SHAPES)
@pytest.mark.parametrize("packed", [False, True], ids=["plain", "packed"])
def test_mx1bias_gemm(gpu, packed, m, n, k, with_c):
    d = T.gen_mx1bias(m, n, k, seed=m + n + k, with_c=with_c)
    np.testing.assert_array_equal(run_mx1(d, packed), oracle(d))
    d = T.gen_mx1bias(m, n, k, seed=m + n + k + 1, with_c=with_c, qca=1)
    np.testing.assert_array_equal(run_mx1(d, packed), oracle(d))


def gen_cf_input(IC, ID, IH, IW, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(-128, 128, size=(IC, ID, IH, IW), dtype=np.int64).astype(np.int8)


# (IC, ID, IH, IW, groups, kernel, stride, pad, dilation)
CF_CASES = [
    (3, 1, 8, 8, 1, (1, 3, 3), (1, 1, 1), (0, 1, 1), (1, 1, 1)),
    (16, 1, 9, 7, 2, (1, 3, 3), (1, 2, 1), (0, 1, 0), (1, 1, 2)),
    (8, 2, 10, 9, 1, (1, 3, 3), (1, 1, 1), (0, 1, 1), (1, 1, 1)),
    (12, 3, 6, 6, 3, (2, 3, 3), (1, 1, 1), (1, 1, 1), (1, 1, 1)),
    (32, 1, 16, 16, 1, (1, 1, 1), (1, 1, 1), (0, 0, 0), (1, 1, 1)),
]


@pytest.mark.parametrize("IC,ID,IH,IW,groups,kern,stride,pad,dil", CF_CASES)
def test_im2col_cf_and_fused_pack(gpu, IC, ID, IH, IW, groups, kern, stride, pad, dil):
    torch = _torch()
    inp = gen_cf_input(IC, ID, IH, IW, seed=IC + IH)
    conv = T.make_conv((ID, IH, IW), kern, stride, dil, pad, IC, 8, groups)
    cp = lib_conv(conv)
    dsrc = _g().dev(inp)
    for grp in range(groups):
        col = T.oracle_im2col_cf(inp, conv, grp)
        K, N = col.shape
        out = torch.full((K * N,), SENTINEL, dtype=torch.int8, device="cuda:0")
        _g().lib().fn("convcf", "run_im2col")(grp, dsrc.data_ptr(), out.data_ptr(),
                                              ctypes.byref(cp))
        np.testing.assert_array_equal(out.cpu().numpy().reshape(K, N), col)
        for ldp, k_idx in ((K, 0), (K + 16, 0), (K, 16)):
            if k_idx >= K:
                continue
            pk = torch.full((N * ldp,), SENTINEL, dtype=torch.int8, device="cuda:0")
            _g().lib().fn("convcfp", "run_b_im2colpack")(grp, dsrc.data_ptr(), ldp, k_idx,
                                                        pk.data_ptr(), ctypes.byref(cp))
            exp = T.pack_panels(np.ascontiguousarray(col.T).view(np.uint8), 128, 16,
                                ld_packed=ldp, shift=k_idx,
                                out=np.full(N * ldp, SENTINEL, np.uint8))
            np.testing.assert_array_equal(pk.cpu().numpy().view(np.uint8), exp)


def cf_problem(IC, OC, ID, IH, IW, groups, kern, stride, pad, dil, seed):
    rng = np.random.default_rng(seed)
    inp = gen_cf_input(IC, ID, IH, IW, seed)
    conv = T.make_conv((ID, IH, IW), kern, stride, dil, pad, IC, OC, groups)
    icg, ocg = IC // groups, OC // groups
    K = icg * kern[0] * kern[1] * kern[2]
    N = conv.output_shape[0] * conv.output_shape[1] * conv.output_shape[2]
    W = rng.integers(-127, 128, size=(ocg, K), dtype=np.int64).astype(np.int8)
    d = dict(inp=inp, conv=conv, W=W, K=K, N=N, ocg=ocg,
             bias=rng.integers(-3000, 3001, size=ocg, dtype=np.int64).astype(np.int32),
             scale_a=rng.uniform(0.001, 0.01, size=ocg).astype(np.float32), qca=ocg,
             scale_b=np.float32(0.02), scale_d=np.float32(0.07), zp_d=3)
    return d


def oracle_cf(d, grp, n_idx=0, n=None):
    n = d["N"] - n_idx if n is None else n
    D = np.zeros((d["ocg"], d["N"]), np.int8)
    sa = np.ascontiguousarray(d["scale_a"])
    T.oracle().tqto_igemmcf_qsi8dx(d["ocg"], n, T.ptr(d["inp"]), grp, n_idx, T.ptr(d["W"]), d["K"],
                                   T.ptr(D), d["N"], T.ptr(d["bias"]), -128, 127,
                                   ctypes.byref(d["conv"]), T.ptr(sa), d["qca"], d["scale_b"],
                                   d["scale_d"], d["zp_d"])
    return D


def run_cf(shim, d, grp, kind, packed, n_idx=0, n=None):
    torch = _torch()
    g = _g()
    n = d["N"] - n_idx if n is None else n
    m, K, N = d["ocg"], d["K"], d["N"]
    din, dW = g.dev(d["inp"]), g.dev(d["W"])
    Wbuf = torch.empty(max(m * K, 1), dtype=torch.int8, device="cuda:0")
    dbias, dsa = g.dev(d["bias"]), g.dev(d["scale_a"])
    dD = torch.zeros((m, N), dtype=torch.int8, device="cuda:0")
    p = mx1_params(d, dsa)
    cp = lib_conv(d["conv"])
    if kind == "convcf":
        Bbuf = torch.empty(max(K * N, 1), dtype=torch.int8, device="cuda:0")
        f = shim.tqts_run_convcf
        f.restype = None
        f.argtypes = [ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p,
                      ctypes.c_void_p] + [ctypes.c_size_t] * 3 + [ctypes.c_void_p] * 4 + [
                          ctypes.c_int8, ctypes.c_int8, ctypes.c_void_p]
        f(int(packed), grp, din.data_ptr(), Bbuf.data_ptr(), ctypes.byref(cp), m, N, K,
          dW.data_ptr(), Wbuf.data_ptr(), dD.data_ptr(), dbias.data_ptr(), -128, 127,
          ctypes.byref(p))
    else:
        f = shim.tqts_run_igemmcf
        f.restype = None
        f.argtypes = ([ctypes.c_int] + [ctypes.c_size_t] * 3 + [ctypes.c_void_p] +
                      [ctypes.c_size_t] * 2 + [ctypes.c_void_p] * 3 + [ctypes.c_size_t,
                                                                       ctypes.c_void_p,
                                                                       ctypes.c_int8,
                                                                       ctypes.c_int8,
                                                                       ctypes.c_void_p,
                                                                       ctypes.c_void_p])
        f(int(packed), m, n, K, din.data_ptr(), grp, n_idx, dW.data_ptr(), Wbuf.data_ptr(),
          dD.data_ptr(), N, dbias.data_ptr(), -128, 127, ctypes.byref(cp), ctypes.byref(p))
    torch.cuda.synchronize()
    return dD.cpu().numpy()


# (IC, OC, ID, IH, IW, groups, kernel, stride, pad, dilation)
CONV_CF = [
    (16, 32, 1, 8, 8, 1, (1, 3, 3), (1, 1, 1), (0, 1, 1), (1, 1, 1)),
    (32, 40, 1, 12, 10, 1, (1, 3, 3), (1, 1, 1), (0, 1, 1), (1, 1, 1)),
    (24, 16, 2, 9, 9, 2, (1, 3, 3), (1, 2, 2), (0, 0, 0), (1, 1, 1)),
    (3, 8, 1, 11, 13, 1, (1, 3, 5), (1, 1, 2), (0, 2, 1), (1, 1, 2)),
    (64, 128, 1, 16, 16, 1, (1, 1, 1), (1, 1, 1), (0, 0, 0), (1, 1, 1)),
]


@pytest.mark.parametrize("IC,OC,ID,IH,IW,groups,kern,stride,pad,dil", CONV_CF)
@pytest.mark.parametrize("packed", [False, True], ids=["plain", "packed"])
@pytest.mark.parametrize("kind", ["convcf", "igemmcf"])
def test_channel_first_convolution(gpu, shim, kind, packed, IC, OC, ID, IH, IW, groups, kern,
                                   stride, pad, dil):
    d = cf_problem(IC, OC, ID, IH, IW, groups, kern, stride, pad, dil, seed=IC + OC + IH)
    for grp in range(groups):
        np.testing.assert_array_equal(run_cf(shim, d, grp, kind, packed), oracle_cf(d, grp))


@pytest.mark.parametrize("packed", [False, True], ids=["plain", "packed"])
def test_igemmcf_pixel_windows(gpu, shim, packed):
    """run_igemm on a window [n_idx, n_idx + n) of the output pixels writes exactly those
    columns of D (at D + n_idx) and nothing else."""
    d = cf_problem(32, 48, 1, 14, 15, 1, (1, 3, 3), (1, 1, 1), (0, 1, 1), (1, 1, 1), seed=7)
    for n_idx, n in ((0, 100), (37, 150), (d["N"] - 5, 5)):
        got = run_cf(shim, d, 0, "igemmcf", packed, n_idx, n)
        np.testing.assert_array_equal(got, oracle_cf(d, 0, n_idx, n))


def test_channel_first_config5_shape(gpu, shim):
    """BASELINE cfg 5's convolution in channel-first form (input [128, 8, 56, 56], 3x3, pad 1,
    OC 128): implicit (plain and packed weights) and explicit paths agree bit for bit, and one
    image's worth of pixels matches the oracle."""
    d = cf_problem(128, 128, 8, 56, 56, 1, (1, 3, 3), (1, 1, 1), (0, 1, 1), (1, 1, 1), seed=42)
    base = run_cf(shim, d, 0, "igemmcf", False)
    for kind, packed in (("igemmcf", True), ("convcf", False), ("convcf", True)):
        np.testing.assert_array_equal(run_cf(shim, d, 0, kind, packed), base)
    one = 56 * 56
    np.testing.assert_array_equal(base[:, 3 * one:4 * one], oracle_cf(d, 0, 3 * one, one)[:, 3 * one:4 * one])
