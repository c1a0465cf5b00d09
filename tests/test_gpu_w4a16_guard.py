"""W4A16 output bounds: rows past m and columns past n are never written.

D and C are allocated with 40 sentinel-filled rows after row m - 1 (and D's columns past n up
to ldd carry the sentinel too), every W4A16 kernel path that takes k 2048 / 4096 runs with m
not a multiple of 32 (1, 20, 33), and the sentinel bytes must come back untouched while rows
0 .. m - 1 pass the same bars as the ordinary parity tests (f16: <= 2 f16 ULP against the
golden-pinned oracle and exact math; f32: within the MFMA kernels' own rounding bound)."""

import ctypes

import numpy as np
import pytest

import tqt_testlib as T

pytestmark = pytest.mark.gpu

GUARD_ROWS = 40
SENTINEL16 = 0x5A5A
SENTINEL32 = 0x5A5A5A5A


def _torch():
    import torch

    return torch


def _g():
    import gpu_run

    return gpu_run


def _run(shim, d, out_f32, packed, ldd_extra):
    torch = _torch()
    g = _g()
    A16, Bsrc, S16, bl = d["A16"], d["Bp"], d["S16"], d["bl"]
    m, k = A16.shape
    n = Bsrc.shape[0]
    ldd = n + ldd_extra
    rows = m + GUARD_ROWS
    dA = g.dev(A16.view(np.int16))
    dB = g.dev(Bsrc)
    if packed:
        kind = "w4a16fp" if out_f32 else "w4a16p"
        pA = torch.empty(2 * m * k, dtype=torch.uint8, device="cuda:0")
        pB = torch.empty(n * k // 2, dtype=torch.uint8, device="cuda:0")
        g.lib().fn(kind, "run_a_pack")(m, k, k, k, 0, dA.data_ptr(), pA.data_ptr())
        g.lib().fn(kind, "run_bt_pack")(n, k, k, k, 0, dB.data_ptr(), pB.data_ptr())
        dA, dB = pA, pB
    dS = g.dev(S16.view(np.int16))
    if out_f32:
        dtype, sent = torch.int32, SENTINEL32
        C = None if d["C32"] is None else d["C32"]
        bias = d["bias32"]
    else:
        dtype, sent = torch.int16, SENTINEL16
        C = None if d["C16"] is None else d["C16"].view(np.int16)
        bias = None if d["bias16"] is None else d["bias16"].view(np.int16)
    dD = torch.full((rows, ldd), sent, dtype=dtype, device="cuda:0")
    dC = None
    if C is not None:
        Cg = np.zeros((rows, ldd), dtype=C.dtype)
        Cg[:m, :n] = C
        dC = g.dev(Cg)
    dbias = g.dev(bias)
    if out_f32:
        f = shim.tqts_run_w4a16f
        f.restype = None
        f.argtypes = ([ctypes.c_int] + [ctypes.c_size_t] * 4 +
                      [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t] * 2 +
                      [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t,
                       ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float,
                       ctypes.c_float])
        f(int(packed), m, n, k, bl, dA.data_ptr(), k, 0, dB.data_ptr(), k, 0, dS.data_ptr(),
          k // bl, g.dp(dC), ldd, dD.data_ptr(), ldd, g.dp(dbias), -np.inf, np.inf)
    else:
        cmin = int(T.f16_bits(-65504.0))
        cmax = int(T.f16_bits(65504.0))
        if packed:
            f = shim.tqts_run_w4a16p
            f.restype = None
            f.argtypes = ([ctypes.c_size_t] * 4 +
                          [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t] * 2 +
                          [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t,
                           ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_uint16,
                           ctypes.c_uint16, ctypes.c_void_p])
            f(m, n, k, bl, dA.data_ptr(), k, 0, dB.data_ptr(), k, 0, dS.data_ptr(), k // bl,
              g.dp(dC), ldd, dD.data_ptr(), ldd, g.dp(dbias), cmin, cmax, None)
        else:
            f = shim.tqts_run_w4a16
            f.restype = None
            f.argtypes = [ctypes.c_size_t] * 4 + [ctypes.c_void_p, ctypes.c_size_t,
                                                  ctypes.c_void_p, ctypes.c_size_t,
                                                  ctypes.c_void_p, ctypes.c_size_t,
                                                  ctypes.c_void_p, ctypes.c_size_t,
                                                  ctypes.c_void_p, ctypes.c_size_t,
                                                  ctypes.c_void_p, ctypes.c_uint16,
                                                  ctypes.c_uint16]
            f(m, n, k, bl, dA.data_ptr(), k, dB.data_ptr(), k, dS.data_ptr(), k // bl,
              g.dp(dC), ldd, dD.data_ptr(), ldd, g.dp(dbias), cmin, cmax)
    torch.cuda.synchronize()
    out = dD.cpu().numpy()
    return out.view(np.uint32 if out_f32 else np.uint16), sent


@pytest.mark.parametrize("out_f32", [False, True], ids=["f16", "f32"])
@pytest.mark.parametrize("packed", [False, True], ids=["plain", "packed"])
@pytest.mark.parametrize("m,n,k", [(1, 100, 4096), (20, 48, 2048), (33, 72, 4096),
                                   (1, 4104, 2048)])
def test_w4a16_rows_past_m_untouched(gpu, shim, out_f32, packed, m, n, k):
    d = T.gen_w4a16(m, n, k, bl=32, seed=7 * m + n + k, with_c=True, with_bias=True)
    d["C32"] = T.bits_f16(d["C16"]).astype(np.float32)
    d["bias32"] = T.bits_f16(d["bias16"]).astype(np.float32)
    ldd_extra = 24
    got, sent = _run(shim, d, out_f32, packed, ldd_extra)
    assert np.all(got[m:] == sent), "rows past m written: %d" % int((got[m:] != sent).sum())
    assert np.all(got[:m, n:] == sent), "columns past n written"
    core = np.ascontiguousarray(got[:m, :n])
    if out_f32:
        from test_gpu_w4a16_f32 import exact_and_scale

        exact, S = exact_and_scale(d, d["C32"], d["bias32"])
        val = core.view(np.float32).astype(np.float64)
        assert np.all(np.isfinite(val))
        tol = (32 + k // 32 + 16) * 2.0 ** -24 * S
        assert np.all(np.abs(val - exact) <= tol), np.max(np.abs(val - exact) / tol)
    else:
        from test_gpu_parity import check_w4a16

        cmin, cmax = int(T.f16_bits(-65504.0)), int(T.f16_bits(65504.0))
        exp = T.oracle_w4a16(d["A16"], d["Bp"], d["S16"], 32, d["C16"], d["bias16"], cmin, cmax)
        check_w4a16(core, exp, d, (-65504.0, 65504.0))
