"""W4A8 output-type siblings on the GPU: gemm_1xnbias_clamp_{f16,bf16}_qai8dx_qsi4cxt and their
packed forms …_qai8dxp_qsi4cxp, called through the reference-shaped interface structs (the
test shim passes the 16-bit clamp bounds by value), bit-exact against the oracle
(tqto_gemm_qai8dx_qsi4cxt_h16: the f32 epilogue of …_{f16,bf16}_qai8dx_qsi4cxt_4x1vl_rvv.cpp
on widened C, bias and bounds, one rounding to nearest even at the store).

Cases: both fast-kernel shapes (activations held in registers or staged in LDS), the generic
kernel (k not a multiple of 256), with and without C and bias, infinite and finite bounds,
results that overflow the 16-bit range, NaN-free and NaN-carrying C, and the decode shape."""

import ctypes

import numpy as np
import pytest

import tqt_testlib as T

pytestmark = pytest.mark.gpu

F16_INF, F16_NINF = 0x7C00, 0xFC00
BF16_INF, BF16_NINF = 0x7F80, 0xFF80


def _g():
    import gpu_run

    return gpu_run


def _torch():
    import torch

    return torch


def to16(x, bf16):
    if x is None:
        return None
    return T.bf16_bits(x) if bf16 else T.f16_bits(x)


def bounds(bf16, lo=None, hi=None):
    if lo is None:
        return (BF16_NINF, BF16_INF) if bf16 else (F16_NINF, F16_INF)
    return int(to16(np.float32(lo), bf16)), int(to16(np.float32(hi), bf16))


def run_h16(shim, d, C16, bias16, cmin_bits, cmax_bits, bf16, packed, stream=False):
    torch = _torch()
    g = _g()
    A, Bp = d["A"], d["Bp"]
    m, k = A.shape
    n = Bp.shape[0]
    kind = ("w4a8bp" if bf16 else "w4a8hp") if packed else None
    if packed:
        dAsrc, dBsrc = g.dev(A), g.dev(Bp)
        dA = torch.empty(max(m * k, 1), dtype=torch.uint8, device="cuda:0")
        dB = torch.empty(max(n * k // 2, 1), dtype=torch.uint8, device="cuda:0")
        g.lib().fn(kind, "run_a_pack")(m, k, k, k, 0, dAsrc.data_ptr(), dA.data_ptr())
        g.lib().fn(kind, "run_bt_pack")(n, k, k, k, 0, dBsrc.data_ptr(), dB.data_ptr())
    else:
        dA, dB = g.dev(A), g.dev(Bp)
    dC = g.dev(None if C16 is None else C16.view(np.int16))
    dbias = g.dev(None if bias16 is None else bias16.view(np.int16))
    dsa, dza, dsb = g.dev(d["scale_a"]), g.dev(d["zp_a"]), g.dev(d["scale_b"])
    p = g._mod.QAI8DXQSI4CXParams(dsa.data_ptr(), dza.data_ptr(), dsb.data_ptr())
    dD = torch.full((m, n), 0x5555, dtype=torch.int16, device="cuda:0")
    f = shim.tqts_run_w4a8h
    f.restype = None
    f.argtypes = ([ctypes.c_int, ctypes.c_int] + [ctypes.c_size_t] * 3 +
                  [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t] * 2 +
                  [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t,
                   ctypes.c_void_p, ctypes.c_uint16, ctypes.c_uint16, ctypes.c_void_p,
                   ctypes.c_void_p])
    s = torch.cuda.current_stream().cuda_stream if stream else None
    f(int(bf16), int(packed), m, n, k, dA.data_ptr(), k, 0, dB.data_ptr(), k, 0, g.dp(dC), n,
      dD.data_ptr(), n, g.dp(dbias), cmin_bits, cmax_bits, ctypes.byref(p), s)
    torch.cuda.synchronize()
    return dD.cpu().numpy().view(np.uint16)


def check(shim, d, bf16, packed, lo=None, hi=None, with_bias=True, stream=False, cbits=None):
    C16 = to16(d["C"], bf16)
    bias16 = to16(d["bias"], bf16) if with_bias else None
    cmin, cmax = bounds(bf16, lo, hi) if cbits is None else cbits
    got = run_h16(shim, d, C16, bias16, cmin, cmax, bf16, packed, stream)
    exp = T.oracle_w4a8_h16(d["A"], d["Bp"], C16, bias16, cmin, cmax, d["scale_a"], d["zp_a"],
                            d["scale_b"], bf16)
    np.testing.assert_array_equal(got, exp)
    return got


# (m, n, k): m=1/4 at k=4096 keep activations in registers, 15/37 rows at k>=1024 stage them
# in LDS, k=100 and k=2 take the generic kernel; n not a multiple of 16 leaves a partial tile
SHAPES = [(1, 160, 4096), (4, 48, 1024), (8, 33, 512), (15, 40, 256), (37, 70, 1024),
          (5, 21, 100), (16, 16, 2)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("packed", [False, True], ids=["plain", "packed"])
@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
def test_w4a8_h16_run(gpu, shim, bf16, packed, m, n, k):
    d = T.gen_w4a8(m, n, k, seed=m * 7 + n + k, with_c=(m % 2 == 1))
    check(shim, d, bf16, packed)
    check(shim, d, bf16, packed, lo=-0.75, hi=0.5, with_bias=False, stream=True)


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
def test_w4a8_h16_overflow_and_nan(gpu, shim, bf16):
    """Products beyond the f16 range round to infinity unless a finite bound clamps them first
    (in f32, before the narrowing). A NaN from C meets the clamp's max/min, which return the
    non-NaN operand (RVV vfmax/vfmin, C fmaxf/fminf), so it becomes the lower bound; only with
    NaN bounds does it reach the store, which writes the canonical NaN pattern."""
    m, n, k = 6, 48, 512
    d = T.gen_w4a8(m, n, k, seed=3, with_c=True)
    d["scale_b"] = (d["scale_b"] * np.float32(4.0e5)).astype(np.float32)
    got = check(shim, d, bf16, False)
    if not bf16:
        assert np.any((got & 0x7FFF) == 0x7C00)  # some results overflowed to infinity
    check(shim, d, bf16, True, lo=-60000.0, hi=60000.0)
    d2 = T.gen_w4a8(m, n, k, seed=4, with_c=True)
    d2["C"][1, 3] = np.nan
    d2["C"][4, 17] = np.nan
    got = check(shim, d2, bf16, False, lo=-5.0, hi=5.0)
    assert got[1, 3] == bounds(bf16, -5.0, 5.0)[0]
    check(shim, d2, bf16, True)
    nan_bits = (0x7FC1, 0xFFC3) if bf16 else (0x7E01, 0xFE03)  # NaN bounds with payloads
    got = check(shim, d2, bf16, False, cbits=nan_bits)
    assert got[1, 3] == (0x7FC0 if bf16 else 0x7E00)
    check(shim, d2, bf16, True, cbits=nan_bits)


@pytest.mark.parametrize("m", [1, 8])
@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
def test_w4a8_h16_decode_shape(gpu, shim, bf16, m):
    """The decode shape K4096 N11008 with a 16-bit D."""
    d = T.gen_w4a8(m, 11008, 4096, seed=m, with_c=False)
    check(shim, d, bf16, False)
    check(shim, d, bf16, True)
