"""W8A8 with per-row dynamically quantized activations on the GPU:
gemm_1xnbias_clamp_{f32,f16}_qai8dx_qsi8cxt and the packed …_qai8dxp_qsi8cxp, through the
reference-shaped interface structs (test shim), bit-exact against the oracle's restatement of
tqt_kernel_gemm_qai8dx_qsi8cx_4x1vl_rvv.h (tqto_gemm_qai8dx_qsi8cxt_{f32,f16}, pinned in
test_oracle.py to the reference test's own acceptance check on its own inputs).

Cases: the streaming kernel (k % 128 == 0), the double-buffered kernel (k % 16 == 0), the
generic kernel (other k, unaligned strides), partial tiles, M = 1, NULL and present bias,
finite and infinite bounds, zero points whose difference with q_a leaves 16 bits (the exact
per-output path), signed-zero and NaN corners, stream-ordered runs, and the reference runner's
own inputs."""

import ctypes
import os

import numpy as np
import pytest

import tqt_testlib as T

pytestmark = pytest.mark.gpu

F16_NINF, F16_INF = 0xFC00, 0x7C00


def _g():
    import gpu_run

    return gpu_run


def _torch():
    import torch

    return torch


def run_dyn(shim, d, f16, packed, cmin=-np.inf, cmax=np.inf, with_bias=True, stream=False,
            lda=None):
    torch = _torch()
    g = _g()
    A, B = d["A"], d["B"]
    m, k = A.shape
    n = B.shape[0]
    lda = k if lda is None else lda
    if packed:
        kind = "w8dynhp" if f16 else "w8dynp"
        dAs, dBs = g.dev(A), g.dev(B)
        dA = torch.empty(max(m * k, 1), dtype=torch.int8, device="cuda:0")
        dB = torch.empty(max(n * k, 1), dtype=torch.int8, device="cuda:0")
        g.lib().fn(kind, "run_a_pack")(m, k, k, k, 0, dAs.data_ptr(), dA.data_ptr())
        g.lib().fn(kind, "run_bt_pack")(n, k, k, k, 0, dBs.data_ptr(), dB.data_ptr())
        lda = k
    else:
        Ap = np.zeros((m, lda), np.int8)
        Ap[:, :k] = A
        dA, dB = g.dev(Ap), g.dev(B)
    if f16:
        bias = T.f16_bits(d["bias"]).view(np.int16) if with_bias else None
        cmin_bits, cmax_bits = ((F16_NINF, F16_INF) if np.isinf(cmin) and np.isinf(cmax) else
                                (int(T.f16_bits(cmin)), int(T.f16_bits(cmax))))
        dD = torch.full((m, n), 0x5555, dtype=torch.int16, device="cuda:0")
    else:
        bias = d["bias"] if with_bias else None
        cmin_bits = cmax_bits = 0
        dD = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
    dbias = g.dev(bias)
    dsa, dza, dsb = g.dev(d["scale_a"]), g.dev(d["zp_a"]), g.dev(d["scale_b"])
    p = g._mod.QAI8DXPQSI8CXPParams(dsa.data_ptr(), dza.data_ptr(), dsb.data_ptr())
    f = shim.tqts_run_w8dyn
    f.restype = None
    f.argtypes = ([ctypes.c_int, ctypes.c_int] + [ctypes.c_size_t] * 3 +
                  [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t] * 2 +
                  [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float,
                   ctypes.c_float, ctypes.c_uint16, ctypes.c_uint16, ctypes.c_void_p,
                   ctypes.c_void_p])
    s = torch.cuda.current_stream().cuda_stream if stream else None
    f(int(f16), int(packed), m, n, k, dA.data_ptr(), lda, 0, dB.data_ptr(), k, 0,
      dD.data_ptr(), n, g.dp(dbias), float(cmin), float(cmax), cmin_bits, cmax_bits,
      ctypes.byref(p), s)
    torch.cuda.synchronize()
    out = dD.cpu().numpy()
    return out.view(np.uint16) if f16 else out


def expected(d, f16, cmin=-np.inf, cmax=np.inf, with_bias=True):
    if f16:
        bias = T.f16_bits(d["bias"]) if with_bias else None
        lo, hi = ((F16_NINF, F16_INF) if np.isinf(cmin) and np.isinf(cmax) else
                  (int(T.f16_bits(cmin)), int(T.f16_bits(cmax))))
        return T.oracle_w8a8dyn(d["A"], d["B"], bias, lo, hi, d["scale_a"], d["zp_a"],
                                d["scale_b"], f16=True)
    bias = d["bias"] if with_bias else None
    return T.oracle_w8a8dyn(d["A"], d["B"], bias, cmin, cmax, d["scale_a"], d["zp_a"],
                            d["scale_b"])


def check(shim, d, f16, packed, **kw):
    exp_kw = {key: kw[key] for key in ("cmin", "cmax", "with_bias") if key in kw}
    got = run_dyn(shim, d, f16, packed, **kw)
    exp = expected(d, f16, **exp_kw)
    if f16:
        np.testing.assert_array_equal(got, exp)
    else:
        np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))
    return got


# (m, n, k): k % 128 == 0 takes the streaming kernel, other k % 16 == 0 the double-buffered
# kernel, the rest the generic one; m and n not multiples of the 128 tile leave partial tiles
SHAPES = [(64, 256, 512), (257, 129, 1024), (1, 128, 4096), (130, 260, 192), (60, 63, 128),
          (3, 8, 11), (60, 63, 127), (33, 70, 96),
          # stream kernel on 128-row tiles, ragged, three k-stages
          (1200, 2100, 384)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("packed", [False, True], ids=["plain", "packed"])
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
def test_w8a8_dyn_run(gpu, shim, f16, packed, m, n, k):
    d = T.gen_w8a8dyn(m, n, k, seed=m + 3 * n + k)
    check(shim, d, f16, packed)
    check(shim, d, f16, packed, cmin=-6.0, cmax=4.5, with_bias=False, stream=True)


@pytest.mark.parametrize("packed", [False, True], ids=["plain", "packed"])
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
def test_w8a8_dyn_zero_points_beyond_16_bits(gpu, shim, f16, packed):
    """Rows whose zero point makes q_a - zp leave 16 bits take the exact per-output path in
    every kernel; the other rows of the same tiles keep the MFMA sum."""
    for m, n, k in ((70, 130, 256), (40, 50, 64), (5, 9, 30)):
        d = T.gen_w8a8dyn(m, n, k, seed=k)
        d["zp_a"][[0, 3]] = [40000, -40001]
        d["zp_a"][-1] = 32640  # the last zero point the MFMA sum covers
        check(shim, d, f16, packed)


@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
def test_w8a8_dyn_strided_a(gpu, shim, f16):
    """Plain A with a row stride beyond k (aligned: MFMA kernels; unaligned: generic)."""
    d = T.gen_w8a8dyn(48, 96, 256, seed=9)
    check(shim, d, f16, False, lda=272)
    check(shim, d, f16, False, lda=259)


def test_w8a8_dyn_signed_zero_and_nan(gpu, shim):
    """The RISC-V corners the oracle restates: without a bias a -0 product gains +0; vfmax
    orders -0 below +0; a NaN scale gives a NaN that the bounds replace."""
    d = T.gen_w8a8dyn(32, 64, 256, seed=5)
    d["A"][:4] = 0
    d["zp_a"][:4] = 0
    d["scale_b"][:8] = -d["scale_b"][:8]  # -0 products in rows 0-3, columns 0-7
    check(shim, d, False, False, with_bias=False)
    check(shim, d, False, False, cmin=0.0, cmax=np.inf, with_bias=False)
    check(shim, d, True, False, cmin=0.0, cmax=65504.0, with_bias=False)
    d["scale_a"][5] = np.nan
    check(shim, d, False, True, cmin=-3.0, cmax=3.0)
    check(shim, d, True, True, cmin=-3.0, cmax=3.0)


def test_w8a8_dyn_reference_test_list(gpu, shim):
    """The reference runner's inputs (ref_w8a8dyn.npz: its generator, its quantizers) on its
    int8 shape list, f32 and f16 D, bit-exact vs the oracle."""
    with np.load(os.path.join(T.GOLDEN_DIR, "ref_w8a8dyn.npz"), allow_pickle=False) as z:
        g = {key: z[key] for key in z.files}
    fm = float(np.finfo(np.float32).max)
    for i in range(len(g["shapes"])):
        pre = "w8a8dyn_%d_" % i
        d = {key: g[pre + key] for key in ("A", "B", "scale_a", "zp_a", "scale_b", "bias")}
        check(shim, d, False, False, cmin=-fm, cmax=fm)
        check(shim, d, True, True)


def test_w8a8_dyn_config2_shape(gpu, shim):
    """BASELINE cfg 2's shape (M512 K4096 N4096) with dynamic A quantization and f32 D:
    bit-exact vs the oracle, plain and packed."""
    d = T.gen_w8a8dyn(512, 4096, 4096, seed=2)
    exp = expected(d, False)
    for packed in (False, True):
        got = run_dyn(shim, d, False, packed)
        np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))
