"""The halo implicit convolution (igemmcl with plain weights, 3 x 3 taps, stride 1, dilation 1,
padding 1 in h and w, one depth tap, 128 channels per group: each workgroup loads the input rows
its 256 output pixels touch once into LDS and forms the nine taps from them), bit-exact against the
oracle's restatement of the reference igemmcl (tqto_igemmcl_qsi8cxt, pinned in test_oracle.py as
im2col + GEMM).

Plain weights and the packed sibling (igemmcl...qsi8cxp: 128-row panels, 16-byte chunks
chunk-major; a partial last panel in the tiled-call test) through the same cases.

Cases: the bank-conflict-free halo row pitch (rows long enough for it to fit) and the plain pitch
IW + 2; images smaller than a tile, so one tile crosses many image boundaries (the padding rows
between images), down to one-row images; a wide image near the halo's size limit, and one too wide
(served by the other kernels); output channel counts that are not a multiple of 64 or of 4 (the
byte tail of the dword stores); two and three groups with each group selected; channel counts per
group other than 128 (the other kernels); the caller's m_idx tiling with tiles that do not start on
a 256-pixel boundary; a padded D row stride (the bytes past n stay untouched) and an odd one (not
dword-aligned: the other kernels); output zero point with a narrow clamp; a per-tensor weight
scale; no bias; accumulators near 2^24 from extreme inputs; a seeded sweep of random geometries,
channel counts, weight layouts and caller tilings."""

import ctypes

import numpy as np
import pytest

import tqt_testlib as T

pytestmark = pytest.mark.gpu

SENTINEL = 0x5A


def _g():
    import gpu_run

    return gpu_run


def gen(in_shape, ic, oc, groups, seed, extreme=False):
    rng = np.random.default_rng(seed)
    conv = T.make_conv(in_shape, (1, 3, 3), (1, 1, 1), (1, 1, 1), (0, 1, 1), ic, oc, groups)
    K = 9 * (ic // groups)
    if extreme:
        # every product at +-2^14: the accumulators reach the int32 range the kernel must carry
        inp = np.where(rng.random(tuple(in_shape) + (ic,)) < 0.5, -128, 127).astype(np.int8)
        W = np.where(rng.random((oc, K)) < 0.5, -127, 127).astype(np.int8)
    else:
        inp = rng.integers(-128, 128, size=tuple(in_shape) + (ic,), dtype=np.int64).astype(np.int8)
        W = rng.integers(-127, 128, size=(oc, K), dtype=np.int64).astype(np.int8)
    scale_b = rng.uniform(0.001, 0.01, size=oc).astype(np.float32)
    bias = rng.integers(-60000, 60001, size=oc, dtype=np.int64).astype(np.int32)
    return dict(inp=inp, W=W, bias=bias, conv=conv, scale_a=np.float32(0.02), zp_a=0,
                scale_b=scale_b, scale_d=np.float32(0.05), zp_d=0)


def m_all(conv):
    return conv.output_shape[0] * conv.output_shape[1] * conv.output_shape[2]


def run(d, group_idx=0, m=None, m_idx=0, ldd=None, bias=True, qcb=None, zp_d=0, cmin=-128,
        cmax=127, D=None, packed=False):
    """One igemmcl run on the GPU into D (M_all x ldd, sentinel-filled unless given); packed:
    the qsi8cxp sibling, weights packed on the GPU first."""
    import torch

    g = _g()
    conv, W = d["conv"], d["W"]
    n, K = W.shape
    ldd = n if ldd is None else ldd
    m = m_all(conv) - m_idx if m is None else m
    if D is None:
        D = np.full((m_all(conv), ldd), SENTINEL, np.int8)
    din, dD = g.dev(d["inp"]), g.dev(D)
    if packed:
        dWs = g.dev(W)
        dW = torch.empty(n * K, dtype=torch.int8, device="cuda:0")
        g.lib().fn("igemmclp", "run_bt_pack")(n, K, K, K, 0, dWs.data_ptr(), dW.data_ptr())
    else:
        dW = g.dev(W)
    dbias, dsb = g.dev(d["bias"]), g.dev(d["scale_b"])
    p = g.w8a8_params(dict(d, B=W, zp_d=zp_d, qcb=n if qcb is None else qcb), dsb)
    cp = g._mod.ConvParams()
    ctypes.memmove(ctypes.byref(cp), ctypes.byref(conv), ctypes.sizeof(cp))
    g.lib().fn("igemmclp" if packed else "igemmcl", "run")(
        m, n, K, din.data_ptr(), group_idx, m_idx, 0, dW.data_ptr(), K, 0, None, 0,
        dD.data_ptr(), ldd, dbias.data_ptr() if bias else None, cmin, cmax, ctypes.byref(cp),
        ctypes.byref(p))
    torch.cuda.synchronize()
    return dD.cpu().numpy()


def expected(d, group_idx=0, m=None, m_idx=0, ldd=None, bias=True, qcb=None, zp_d=0, cmin=-128,
             cmax=127, D=None):
    conv, W = d["conv"], d["W"]
    n, K = W.shape
    ldd = n if ldd is None else ldd
    m = m_all(conv) - m_idx if m is None else m
    D = np.full((m_all(conv), ldd), SENTINEL, np.int8) if D is None else D.copy()
    T.oracle().tqto_igemmcl_qsi8cxt(
        m, n, T.ptr(d["inp"]), group_idx, m_idx, T.ptr(W), K, T.ptr(D), ldd,
        T.ptr(d["bias"]) if bias else None, cmin, cmax, ctypes.byref(conv), d["scale_a"],
        T.ptr(d["scale_b"]), n if qcb is None else qcb, d["scale_d"], zp_d)
    return D


# (input (D, H, W), IC, OC, groups)
CASES = [
    ((2, 30, 40), 128, 64, 1),    # conflict-free pitch (56 for rows of 40)
    ((2, 13, 17), 128, 64, 1),    # conflict-free pitch (33 for rows of 17)
    ((3, 9, 10), 128, 72, 1),     # plain pitch IW + 2 (the other does not fit); 64 + 8 channels
    ((1, 20, 21), 128, 130, 1),   # 130 = 2 x 64 + 2 (byte tail)
    ((2, 14, 14), 128, 128, 1),
    ((9, 4, 3), 128, 64, 1),      # 12-pixel images: 21 image boundaries per tile
    ((40, 1, 7), 128, 66, 1),     # one-row images: every row is an image
    ((1, 6, 90), 128, 64, 1),     # wide rows near the halo's size limit
    ((1, 4, 200), 128, 64, 1),    # too wide for the halo: other kernels
    ((2, 8, 8), 256, 70, 2),      # two groups of 128 channels
    ((1, 10, 10), 384, 33, 3),    # three groups of 128 channels
    ((2, 9, 13), 64, 64, 1),      # 64 channels per group: other kernels
    ((1, 9, 9), 224, 24, 1),      # 224 channels per group: other kernels
]


@pytest.mark.parametrize("packed", [False, True], ids=["plain", "packed"])
@pytest.mark.parametrize("case", range(len(CASES)), ids=[
    "x".join(map(str, c[0])) + "_ic%d_oc%d_g%d" % c[1:] for c in CASES])
def test_conv_halo_matches_oracle(gpu, case, packed):
    in_shape, ic, oc, groups = CASES[case]
    d = gen(in_shape, ic, oc, groups, seed=100 + case)
    for gi in range(groups):
        np.testing.assert_array_equal(run(d, group_idx=gi, packed=packed),
                                      expected(d, group_idx=gi))


@pytest.mark.parametrize("packed", [False, True], ids=["plain", "packed"])
def test_conv_halo_tiled_calls(gpu, packed):
    """The reference caller pattern with tiles of 200 pixels: no call starts on a 256-pixel
    boundary of the image, and the last one is ragged; D is addressed absolutely."""
    d = gen((3, 17, 19), 128, 200, 1, seed=7)
    M = m_all(d["conv"])
    D = np.full((M, 200), SENTINEL, np.int8)
    E = D.copy()
    for m_idx in range(0, M, 200):
        m = min(200, M - m_idx)
        D = run(d, m=m, m_idx=m_idx, D=D, packed=packed)
        E = expected(d, m=m, m_idx=m_idx, D=E)
    np.testing.assert_array_equal(D, E)
    assert not (D == SENTINEL).all(axis=1).any()


@pytest.mark.parametrize("ldd", [72, 69], ids=["padded", "odd"])
def test_conv_halo_row_stride(gpu, ldd):
    """D rows wider than n: every byte past n keeps its value (dword stores never cross n);
    an odd stride is not dword-aligned and takes the other kernels."""
    d = gen((2, 9, 13), 128, 66, 1, seed=3)
    out = run(d, ldd=ldd)
    np.testing.assert_array_equal(out, expected(d, ldd=ldd))
    assert (out[:, 66:] == SENTINEL).all()


@pytest.mark.parametrize("opts", [
    dict(zp_d=-5, cmin=-20, cmax=40),
    dict(zp_d=7, cmin=50, cmax=-3),       # cmin > cmax: every output is cmax
    dict(qcb=1),                          # per-tensor weight scale
    dict(bias=False),
], ids=["zp_clamp", "clamp_inverted", "per_tensor_scale", "no_bias"])
def test_conv_halo_epilogue_options(gpu, opts):
    d = gen((2, 10, 11), 128, 64, 1, seed=5)
    np.testing.assert_array_equal(run(d, **opts), expected(d, **opts))


def test_conv_halo_extreme_accumulators(gpu):
    """Inputs and weights all at +-127/128: per-tap partial sums up to 2^21, totals up to
    2^24 ahead of the bias and the requantization multiply."""
    d = gen((2, 7, 9), 128, 64, 1, seed=9, extreme=True)
    np.testing.assert_array_equal(run(d), expected(d))


def test_conv_halo_random_geometries(gpu):
    """A seeded sweep over 3 x 3 "same" convolutions with 128 channels per group: image counts,
    heights and widths (rows up to the halo's width limit and past it), output channels, one or
    two groups, plain or packed weights, and the caller's pixel tiling (whole calls or tiles of a
    random size), each bit-exact against the oracle."""
    rng = np.random.default_rng(2024)
    for case in range(16):
        ID = int(rng.integers(1, 5))
        IH = int(rng.integers(1, 21))
        IW = int(rng.integers(1, 121))
        groups = int(rng.integers(1, 3))
        oc = groups * int(rng.integers(1, 97))
        packed = bool(rng.integers(0, 2))
        d = gen((ID, IH, IW), 128 * groups, oc, groups, seed=500 + case)
        M = m_all(d["conv"])
        tile = M if rng.integers(0, 2) else int(rng.integers(1, M + 1))
        gi = int(rng.integers(0, groups))
        print("case %d: %dx%dx%d oc %d groups %d (group %d) packed %d tile %d" % (
            case, ID, IH, IW, oc, groups, gi, packed, tile), flush=True)
        D = np.full((M, oc), SENTINEL, np.int8)
        E = D.copy()
        for m_idx in range(0, M, tile):
            m = min(tile, M - m_idx)
            D = run(d, group_idx=gi, m=m, m_idx=m_idx, D=D, packed=packed)
            E = expected(d, group_idx=gi, m=m, m_idx=m_idx, D=E)
        np.testing.assert_array_equal(D, E)


@pytest.mark.parametrize("oc", [200, 72])
def test_conv_halo_packed_k_idx(gpu, oc):
    """Packed weights that are the k-range [16, 16 + K) of a wider packed buffer (ld_packed =
    K + 16, packed with k_idx = 16, so a narrower last panel starts 16 * (128 - w) bytes earlier
    by the packers' tail rule), run with the same ldb and k_idx_b: the halo kernel's
    chunk-major weight loads address the shifted tail panel like the packers."""
    import torch

    g = _g()
    d = gen((2, 11, 13), 128, oc, 1, seed=31 + oc)
    conv, W = d["conv"], d["W"]
    n, K = W.shape
    kx = 16
    L = g.lib()
    ns = L.fn("igemmclp", "get_n_step")()
    Bp = torch.zeros(n * (K + kx), dtype=torch.int8, device="cuda:0")
    b_off = L.fn("igemmclp", "get_b_packed_offset")(0, kx, K + kx, min(n, ns))
    dW = g.dev(W)
    L.fn("igemmclp", "run_bt_pack")(n, K, K, K + kx, kx, dW.data_ptr(), Bp.data_ptr() + b_off)
    M = m_all(conv)
    dD = g.dev(np.full((M, n), SENTINEL, np.int8))
    din, dbias, dsb = g.dev(d["inp"]), g.dev(d["bias"]), g.dev(d["scale_b"])
    p = g.w8a8_params(dict(d, B=W), dsb)
    cp = g._mod.ConvParams()
    ctypes.memmove(ctypes.byref(cp), ctypes.byref(conv), ctypes.sizeof(cp))
    L.fn("igemmclp", "run")(M, n, K, din.data_ptr(), 0, 0, 0, Bp.data_ptr() + b_off, K + kx, kx,
                            None, 0, dD.data_ptr(), n, dbias.data_ptr(), -128, 127,
                            ctypes.byref(cp), ctypes.byref(p))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dD.cpu().numpy(), expected(d))
