"""The stream-ordered entry points inside a captured HIP graph: one graph holding a launch of
every kernel type is replayed several times, with eager work (clearing the outputs) and
synchronizations between replays, and every replay must reproduce the oracle (bit-exact for the
integer and W4A8 outputs) or, for W4A16, the eager launch of the same kernel bit for bit. The
kernels allocate nothing and record no memset, so capture is legal; this checks that replays
after the first stay correct."""

import ctypes

import numpy as np
import pytest

import tqt_testlib as T

pytestmark = pytest.mark.gpu


def test_all_kernel_types_replay_in_a_hip_graph(gpu, shim):
    import torch

    import gpu_run as G

    # the params structs and the function types must come from the same module instance
    mod = G._mod
    lib = G.lib()
    s = torch.cuda.Stream()
    sh = s.cuda_stream
    dev = G.dev
    launches, outputs, expected = [], [], []

    # int8 x int8 -> int32 with clamp (K x N weights)
    clA, clB, _ = T.gen_clamp(64, 256, 512, seed=3)
    cA, cB = dev(clA), dev(clB)
    cD = torch.zeros((64, 256), dtype=torch.int32, device="cuda:0")
    f_cl = lib.fn("clamp", "run_async")
    launches.append(lambda: f_cl(64, 256, 512, cA.data_ptr(), 512, 0, cB.data_ptr(), 256, 0,
                                 None, 256, cD.data_ptr(), 256, -(2 ** 31), 2 ** 31 - 1, sh))
    outputs.append(cD)
    expected.append(T.oracle_clamp(clA, clB, None, -(2 ** 31), 2 ** 31 - 1))

    # W8A8, streaming kernel (k % 128 == 0)
    w8 = T.gen_w8a8(64, 256, 512, seed=4)
    wA, wB, wbias, wsb = dev(w8["A"]), dev(w8["B"]), dev(w8["bias"]), dev(w8["scale_b"])
    wD = torch.zeros((64, 256), dtype=torch.int8, device="cuda:0")
    p8 = G.w8a8_params(w8, wsb)
    f_w8 = lib.fn("w8a8", "run_async")
    launches.append(lambda: f_w8(64, 256, 512, wA.data_ptr(), 512, 0, wB.data_ptr(), 512, 0, None,
                                 256, wD.data_ptr(), 256, wbias.data_ptr(), -128, 127,
                                 ctypes.byref(p8), sh))
    outputs.append(wD)
    expected.append(T.oracle_w8a8(w8["A"], w8["B"], None, w8["bias"], -128, 127, w8["scale_a"],
                                  w8["scale_b"], 256, w8["scale_d"], w8["zp_d"]))

    # W4A8 decode path
    w4 = T.gen_w4a8(4, 160, 1024, seed=5)
    qA, qB, qbias = dev(w4["A"]), dev(w4["Bp"]), dev(w4["bias"])
    qsa, qza, qsb = dev(w4["scale_a"]), dev(w4["zp_a"]), dev(w4["scale_b"])
    qD = torch.zeros((4, 160), dtype=torch.float32, device="cuda:0")
    p4 = mod.QAI8DXQSI4CXParams(qsa.data_ptr(), qza.data_ptr(), qsb.data_ptr())
    f_w4 = lib.fn("w4a8", "run_async")
    launches.append(lambda: f_w4(4, 160, 1024, qA.data_ptr(), 1024, 0, qB.data_ptr(), 1024, 0,
                                 None, 160, qD.data_ptr(), 160, qbias.data_ptr(), -np.inf, np.inf,
                                 ctypes.byref(p4), sh))
    outputs.append(qD)
    expected.append(T.oracle_w4a8(w4["A"], w4["Bp"], None, w4["bias"], -np.inf, np.inf,
                                  w4["scale_a"], w4["zp_a"], w4["scale_b"]))

    # W4A16 strip kernel (k = 2048), compared with its own eager launch
    h = T.gen_w4a16(32, 96, 2048, seed=6)
    hA, hB, hS = dev(h["A16"].view(np.int16)), dev(h["Bp"]), dev(h["S16"].view(np.int16))
    hbias = dev(h["bias16"].view(np.int16))
    hD = torch.zeros((32, 96), dtype=torch.int16, device="cuda:0")
    f_h = shim.tqts_run_w4a16_async
    f_h.restype = None
    f_h.argtypes = [ctypes.c_size_t] * 4 + [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                            ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t,
                                            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                            ctypes.c_size_t, ctypes.c_void_p, ctypes.c_uint16,
                                            ctypes.c_uint16, ctypes.c_void_p]
    cmin = int(np.float16(-65504.0).view(np.uint16))
    cmax = int(np.float16(65504.0).view(np.uint16))
    launches.append(lambda: f_h(32, 96, 2048, 32, hA.data_ptr(), 2048, hB.data_ptr(), 2048,
                                hS.data_ptr(), 64, None, 96, hD.data_ptr(), 96, hbias.data_ptr(),
                                cmin, cmax, sh))
    outputs.append(hD)
    expected.append(None)  # filled from the eager launch below

    # igemmcl
    cv = T.gen_igemmcl(2, 9, 9, 32, 48, 3, 3, pad=(1, 1), seed=7)
    conv = cv["conv"]
    m = conv.output_shape[0] * conv.output_shape[1] * conv.output_shape[2]
    vin, vW, vbias, vsb = dev(cv["inp"]), dev(cv["W"]), dev(cv["bias"]), dev(cv["scale_b"])
    vD = torch.zeros((m, 48), dtype=torch.int8, device="cuda:0")
    pv = G.w8a8_params(dict(cv, B=cv["W"]), vsb)
    cp = mod.ConvParams()
    ctypes.memmove(ctypes.byref(cp), ctypes.byref(conv), ctypes.sizeof(cp))
    kconv = cv["W"].shape[1]
    f_v = lib.fn("igemmcl", "run_async")
    launches.append(lambda: f_v(m, 48, kconv, vin.data_ptr(), 0, 0, 0, vW.data_ptr(), kconv, 0,
                                None, 0, vD.data_ptr(), 48, vbias.data_ptr(), -128, 127,
                                ctypes.byref(cp), ctypes.byref(pv), sh))
    outputs.append(vD)
    expected.append(T.oracle_igemmcl(cv["inp"], cv["W"], cv["bias"], -128, 127, conv,
                                     cv["scale_a"], cv["scale_b"], 48, cv["scale_d"],
                                     cv["zp_d"]))

    with torch.cuda.stream(s):
        for f in launches:
            f()
    torch.cuda.synchronize()
    eager = [o.cpu().numpy().copy() for o in outputs]
    expected[3] = eager[3]
    for got, exp in zip(eager, expected):
        np.testing.assert_array_equal(got.view(np.uint8), np.asarray(exp).view(np.uint8))

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        for f in launches:
            f()
    for _ in range(3):
        for o in outputs:
            o.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o, exp in zip(outputs, expected):
            np.testing.assert_array_equal(o.cpu().numpy().view(np.uint8),
                                          np.asarray(exp).view(np.uint8))
