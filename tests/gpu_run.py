"""Run the five gfx950 kernel types through the C ABI on numpy inputs (device copies via torch)."""

import ctypes

import numpy as np
import torch

import tqt_testlib as T

_mod = T.load_product_module()


def dev(x):
    if x is None:
        return None
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")


def dp(t):
    return None if t is None else t.data_ptr()


def lib():
    return _mod.load()


def run_clamp(A, B, C, cmin, cmax):
    m, k = A.shape
    n = B.shape[1]
    dA, dB, dC = dev(A), dev(B), dev(C)
    dD = torch.zeros((m, n), dtype=torch.int32, device="cuda:0")
    lib().fn("clamp", "run")(m, n, k, dp(dA), k, 0, dp(dB), n, 0, dp(dC), n, dp(dD), n, cmin, cmax)
    return dD.cpu().numpy()


def w8a8_params(d, scale_b_dev):
    p = _mod.QAI8QSI8CXParams()
    p.scale_a = float(d["scale_a"])
    p.zero_point_a = int(d["zp_a"])
    p.scale_b = scale_b_dev.data_ptr()
    p.quant_channel_b = int(d.get("qcb", d["B"].shape[0]))
    p.scale_d = float(d["scale_d"])
    p.zero_point_d = int(d["zp_d"])
    return p


def run_w8a8(d, cmin=-128, cmax=127):
    A, B = d["A"], d["B"]
    m, k = A.shape
    n = B.shape[0]
    dA, dB, dC, dbias, dsb = dev(A), dev(B), dev(d["C"]), dev(d["bias"]), dev(d["scale_b"])
    dD = torch.zeros((m, n), dtype=torch.int8, device="cuda:0")
    p = w8a8_params(d, dsb)
    lib().fn("w8a8", "run")(m, n, k, dp(dA), k, 0, dp(dB), k, 0, dp(dC), n, dp(dD), n, dp(dbias),
                            cmin, cmax, ctypes.byref(p))
    return dD.cpu().numpy()


def run_w4a8(d, cmin=-np.inf, cmax=np.inf):
    A, Bp = d["A"], d["Bp"]
    m, k = A.shape
    n = Bp.shape[0]
    dA, dB = dev(A), dev(Bp)
    dC, dbias = dev(d["C"]), dev(d["bias"])
    dsa, dza, dsb = dev(d["scale_a"]), dev(d["zp_a"]), dev(d["scale_b"])
    dD = torch.zeros((m, n), dtype=torch.float32, device="cuda:0")
    p = _mod.QAI8DXQSI4CXParams(dsa.data_ptr(), dza.data_ptr(), dsb.data_ptr())
    lib().fn("w4a8", "run")(m, n, k, dp(dA), k, 0, dp(dB), k, 0, dp(dC), n, dp(dD), n, dp(dbias),
                            float(cmin), float(cmax), ctypes.byref(p))
    return dD.cpu().numpy()


def run_w4a16(shim, d, cmin_bits, cmax_bits):
    A16, Bp, S16, bl = d["A16"], d["Bp"], d["S16"], d["bl"]
    m, k = A16.shape
    n = Bp.shape[0]
    dA, dB, dS = dev(A16.view(np.int16)), dev(Bp), dev(S16.view(np.int16))
    dC = dev(None if d["C16"] is None else d["C16"].view(np.int16))
    dbias = dev(None if d["bias16"] is None else d["bias16"].view(np.int16))
    dD = torch.zeros((m, n), dtype=torch.int16, device="cuda:0")
    f = shim.tqts_run_w4a16
    f.restype = None
    f.argtypes = [ctypes.c_size_t] * 4 + [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                          ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t,
                                          ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                          ctypes.c_size_t, ctypes.c_void_p, ctypes.c_uint16,
                                          ctypes.c_uint16]
    f(m, n, k, bl, dp(dA), k, dp(dB), k, dp(dS), k // bl, dp(dC), n, dp(dD), n, dp(dbias),
      cmin_bits, cmax_bits)
    return dD.cpu().numpy().view(np.uint16)


def run_igemmcl(d, cmin=-128, cmax=127, m=None, m_idx=0, D_init=None):
    conv = d["conv"]
    W = d["W"]
    n = W.shape[0]
    M_all = conv.output_shape[0] * conv.output_shape[1] * conv.output_shape[2]
    if m is None:
        m = M_all - m_idx
    din, dW, dbias, dsb = dev(d["inp"]), dev(W), dev(d["bias"]), dev(d["scale_b"])
    if D_init is None:
        dD = torch.zeros((M_all, n), dtype=torch.int8, device="cuda:0")
    else:
        dD = dev(D_init)
    p = w8a8_params(dict(d, B=W), dsb)
    cp = _mod.ConvParams()
    ctypes.memmove(ctypes.byref(cp), ctypes.byref(conv), ctypes.sizeof(cp))
    lib().fn("igemmcl", "run")(m, n, W.shape[1], dp(din), 0, m_idx, 0, dp(dW), W.shape[1], 0,
                               None, 0, dp(dD), n, dp(dbias), cmin, cmax, ctypes.byref(cp),
                               ctypes.byref(p))
    return dD.cpu().numpy()
