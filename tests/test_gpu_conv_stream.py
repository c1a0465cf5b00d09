"""The streaming implicit convolution (igemmcl with a group channel count that is a multiple of
128: each 128-byte pipeline stage is one tap's channels, gathered straight into LDS, padding
taps read as zeros through the buffer range check), bit-exact against the oracle's restatement
of the reference igemmcl (tqto_igemmcl_qsi8cxt, pinned in test_oracle.py as im2col + GEMM).

Cases: strides, paddings and dilations in every dimension, a 3-D kernel, partial row and
column tiles, two groups with the second group selected, the reference's m_step tiling with
m_idx (a ragged last tile), and plain and packed weights. The plain-weight 3 x 3 stride-1
"same" cases with 128 channels per group (case 0, the grouped case, the tiled calls, cfg 5
plain) are served by the halo kernel instead (test_gpu_conv_halo.py); their packed twins still
take the streaming kernel."""

import ctypes

import numpy as np
import pytest

import tqt_testlib as T

pytestmark = pytest.mark.gpu


def _g():
    import gpu_run

    return gpu_run


def _torch():
    import torch

    return torch


def gen(in_shape, kern, stride, pad, dil, ic, oc, groups, seed):
    rng = np.random.default_rng(seed)
    conv = T.make_conv(in_shape, kern, stride, dil, pad, ic, oc, groups)
    icg = ic // groups
    K = kern[0] * kern[1] * kern[2] * icg
    inp = rng.integers(-128, 128, size=tuple(in_shape) + (ic,), dtype=np.int64).astype(np.int8)
    W = rng.integers(-127, 128, size=(oc, K), dtype=np.int64).astype(np.int8)
    scale_b = rng.uniform(0.001, 0.01, size=oc).astype(np.float32)
    bias = rng.integers(-60000, 60001, size=oc, dtype=np.int64).astype(np.int32)
    return dict(inp=inp, W=W, bias=bias, conv=conv, scale_a=np.float32(0.02), zp_a=0,
                scale_b=scale_b, scale_d=np.float32(0.05), zp_d=0)


def run(d, packed, group_idx=0, m=None, m_idx=0, D_init=None):
    torch = _torch()
    g = _g()
    conv, W = d["conv"], d["W"]
    n, K = W.shape
    M_all = conv.output_shape[0] * conv.output_shape[1] * conv.output_shape[2]
    m = M_all - m_idx if m is None else m
    din, dbias, dsb = g.dev(d["inp"]), g.dev(d["bias"]), g.dev(d["scale_b"])
    if packed:
        dWs = g.dev(W)
        dW = torch.empty(n * K, dtype=torch.int8, device="cuda:0")
        g.lib().fn("igemmclp", "run_bt_pack")(n, K, K, K, 0, dWs.data_ptr(), dW.data_ptr())
    else:
        dW = g.dev(W)
    dD = (torch.zeros((M_all, n), dtype=torch.int8, device="cuda:0") if D_init is None
          else g.dev(D_init))
    p = g.w8a8_params(dict(d, B=W), dsb)
    cp = g._mod.ConvParams()
    ctypes.memmove(ctypes.byref(cp), ctypes.byref(conv), ctypes.sizeof(cp))
    g.lib().fn("igemmclp" if packed else "igemmcl", "run")(
        m, n, K, din.data_ptr(), group_idx, m_idx, 0, dW.data_ptr(), K, 0, None, 0,
        dD.data_ptr(), n, dbias.data_ptr(), -128, 127, ctypes.byref(cp), ctypes.byref(p))
    torch.cuda.synchronize()
    return dD.cpu().numpy()


def expected(d, group_idx=0, m=None, m_idx=0, D=None):
    return T.oracle_igemmcl(d["inp"], d["W"], d["bias"], -128, 127, d["conv"], d["scale_a"],
                            d["scale_b"], d["W"].shape[0], d["scale_d"], d["zp_d"], m=m,
                            m_idx=m_idx, group_idx=group_idx, D=D)


# (input (D, H, W), kernel, stride, pad, dilation, IC, OC, groups)
CASES = [
    ((1, 9, 11), (1, 3, 3), (1, 1, 1), (0, 1, 1), (1, 1, 1), 128, 96, 1),
    ((2, 7, 7), (1, 3, 3), (1, 2, 1), (0, 0, 2), (1, 1, 2), 256, 40, 1),
    ((1, 10, 10), (1, 1, 1), (1, 1, 1), (0, 0, 0), (1, 1, 1), 128, 130, 1),
    ((4, 6, 5), (2, 3, 2), (1, 1, 2), (1, 1, 0), (2, 1, 1), 128, 64, 1),
    ((1, 12, 9), (1, 5, 3), (1, 2, 2), (0, 2, 1), (1, 1, 1), 384, 136, 1),
    ((3, 8, 8), (1, 3, 3), (1, 1, 1), (0, 1, 1), (1, 1, 1), 256, 72, 2),
]


@pytest.mark.parametrize("packed", [False, True], ids=["plain", "packed"])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_conv_stream_matches_oracle(gpu, case, packed):
    in_shape, kern, stride, pad, dil, ic, oc, groups = CASES[case]
    d = gen(in_shape, kern, stride, pad, dil, ic, oc, groups, seed=case)
    for gi in range(groups):
        np.testing.assert_array_equal(run(d, packed, group_idx=gi), expected(d, group_idx=gi))


def test_conv_stream_tiled_calls(gpu):
    """The reference caller pattern: one run per 128-pixel tile with m_idx (a ragged last
    tile); D is addressed absolutely."""
    d = gen((2, 11, 9), (1, 3, 3), (1, 1, 1), (0, 1, 1), (1, 1, 1), 128, 48, 1, seed=7)
    conv = d["conv"]
    M = conv.output_shape[0] * conv.output_shape[1] * conv.output_shape[2]
    D = np.zeros((M, 48), np.int8)
    for m_idx in range(0, M, 128):
        D = run(d, False, m=min(128, M - m_idx), m_idx=m_idx, D_init=D)
    np.testing.assert_array_equal(D, expected(d))


def test_conv_stream_config5(gpu):
    """BASELINE cfg 5 (NHWC 8x56x56x128, 3x3, pad 1, OC 128), plain and packed weights."""
    d = T.gen_igemmcl(8, 56, 56, 128, 128, 3, 3, pad=(1, 1), seed=11)
    exp = T.oracle_igemmcl(d["inp"], d["W"], d["bias"], -128, 127, d["conv"], d["scale_a"],
                           d["scale_b"], 128, d["scale_d"], d["zp_d"])
    for packed in (False, True):
        np.testing.assert_array_equal(run(d, packed), exp)
