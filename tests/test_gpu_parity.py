"""GPU parity: every kernel type through the C ABI against the CPU oracle on identical inputs.

Shapes: the reference's own test shape lists (test/gemm/test_gemm_i8_i8_rvv.cpp:31-41,
test/gemm/test_gemm_i8_i4_rvv.cpp:164-179, test/gemm/test_gemm_f16_i4_rvv.cpp:19-49,
test/conv/test_igemm_i8_i8_rvv.cpp:21-41), the BASELINE.json configurations at full size, and
extra ragged / aligned shapes that exercise both the MFMA fast paths and the generic paths.

Bar: bit-exact for int32 and int8 outputs and for the W4A8 f32 output (same operation order,
no FMA); W4A16 f16 output within 2 binary16 ULP of both the f32-accumulating reference oracle
and the exact (float64) result, the ULP taken at max(|expected|, 2^-14, 2^-13 * sum|a*w|)
(see ulp_distance_f16).
"""

import ctypes

import numpy as np
import pytest

import tqt_testlib as T

pytestmark = pytest.mark.gpu

INT8_REF_SHAPES = [(32, 32, 32, False), (3, 8, 11, False), (5, 11, 10, False), (9, 19, 23, False),
                   (15, 32, 25, False), (60, 63, 127, False), (32, 32, 32, True),
                   (60, 63, 127, True)]
INT8_FAST_SHAPES = [(64, 256, 512, False), (130, 260, 192, True), (200, 136, 80, False),
                    (1, 128, 64, False), (257, 129, 1024, True),
                    # stream kernel with 1, 2, 3 and 5 k-stages of 128 (the column multipliers
                    # after the loop, in the last stage, and the ring shorter than its depth)
                    (64, 256, 128, False), (96, 200, 256, True), (130, 260, 384, False),
                    (33, 129, 640, True),
                    # 128-row tiles (chosen once they still fill 160 or more CUs), ragged
                    (1200, 2100, 384, True)]


def _gr():
    import gpu_run

    return gpu_run


@pytest.mark.parametrize("m,n,k,with_c", INT8_REF_SHAPES + INT8_FAST_SHAPES)
def test_clamp_i32_parity(gpu, m, n, k, with_c):
    A, B, C = T.gen_clamp(m, n, k, seed=42 + m, with_c=with_c, lo=-50, hi=50)
    for cmin, cmax in [(-100000, 100000), (-2**31, 2**31 - 1)]:
        got = _gr().run_clamp(A, B, C, cmin, cmax)
        exp = T.oracle_clamp(A, B, C, cmin, cmax)
        np.testing.assert_array_equal(got, exp)


# The small-problem kernel (32 x 32 tiles, k split over the four waves; M, N multiples of 32,
# k % 128 == 0, k <= 2048, few regular tiles): one to sixteen 32-k steps per wave, with and
# without C, full-range and narrow clamps (and an inverted one: max then min leaves cmax).
@pytest.mark.parametrize("m,n,k,with_c", [(32, 32, 128, False), (32, 160, 384, True),
                                          (96, 64, 2048, True), (64, 256, 1152, False),
                                          (128, 96, 256, True)])
def test_clamp_i32_small_kernel(gpu, m, n, k, with_c):
    A, B, C = T.gen_clamp(m, n, k, seed=m + n + k, with_c=with_c)
    for cmin, cmax in [(-2**31, 2**31 - 1), (-50000, 70000), (1000, -1000)]:
        got = _gr().run_clamp(A, B, C, cmin, cmax)
        exp = T.oracle_clamp(A, B, C, cmin, cmax)
        np.testing.assert_array_equal(got, exp)


def test_clamp_i32_config1(gpu):
    """BASELINE cfg 1: A [64,512], B [512,256] uniform in [-128,127], no C, full int32 clamp."""
    A, B, C = T.gen_clamp(64, 256, 512, seed=42)
    got = _gr().run_clamp(A, B, None, -2**31, 2**31 - 1)
    exp = T.oracle_clamp(A, B, None, -2**31, 2**31 - 1)
    np.testing.assert_array_equal(got, exp)
    # closed form: int64 matrix product fits int32 here
    np.testing.assert_array_equal(got, (A.astype(np.int64) @ B.astype(np.int64)).astype(np.int32))


@pytest.mark.parametrize("m,n,k,with_c", INT8_REF_SHAPES + INT8_FAST_SHAPES)
def test_w8a8_parity(gpu, m, n, k, with_c):
    d = T.gen_w8a8(m, n, k, seed=7 + n, with_c=with_c)
    got = _gr().run_w8a8(d)
    exp = T.oracle_w8a8(d["A"], d["B"], d["C"], d["bias"], -128, 127, d["scale_a"], d["scale_b"],
                        n, d["scale_d"], d["zp_d"])
    np.testing.assert_array_equal(got, exp)


def test_w8a8_variants(gpu):
    """No bias, narrow clamp, nonzero output zero point, per-tensor scale (quant_channel_b=1),
    and a real scale >= 0.5 (negative stored shift, shifted by shift & 31)."""
    m, n, k = 96, 200, 320
    base = T.gen_w8a8(m, n, k, seed=11)
    cases = [
        dict(bias=None),
        dict(zp_d=17),
        dict(qcb=1),
        dict(scale_d=np.float32(1e-5)),
    ]
    for upd in cases:
        d = dict(base, **upd)
        cmin, cmax = (-20, 90) if "zp_d" in upd else (-128, 127)
        got = _gr().run_w8a8(d, cmin, cmax)
        exp = T.oracle_w8a8(d["A"], d["B"], d["C"], d["bias"], cmin, cmax, d["scale_a"],
                            d["scale_b"], d.get("qcb", n), d["scale_d"], d["zp_d"])
        np.testing.assert_array_equal(got, exp, err_msg=str(upd.keys()))


@pytest.mark.parametrize("m,n,k", [(64, 256, 512), (7, 9, 33)])
def test_w8a8_inverted_clamp(gpu, m, n, k):
    """clamp_min > clamp_max: the reference's max-then-min leaves clamp_max everywhere
    (stream kernel and generic kernel)."""
    d = T.gen_w8a8(m, n, k, seed=m + n)
    for cmin, cmax in ((50, -30), (127, -128), (-5, -5)):
        got = _gr().run_w8a8(d, cmin, cmax)
        exp = T.oracle_w8a8(d["A"], d["B"], d["C"], d["bias"], cmin, cmax, d["scale_a"],
                            d["scale_b"], n, d["scale_d"], d["zp_d"])
        np.testing.assert_array_equal(got, exp)
        if cmin > cmax:
            assert (got == cmax).all()


def test_w8a8_config2_full(gpu):
    """BASELINE cfg 2 at full size: M=512, K=4096, N=4096, bit-exact."""
    d = T.gen_w8a8(512, 4096, 4096, seed=42)
    got = _gr().run_w8a8(d)
    exp = T.oracle_w8a8(d["A"], d["B"], None, d["bias"], -128, 127, d["scale_a"], d["scale_b"],
                        4096, d["scale_d"], d["zp_d"])
    np.testing.assert_array_equal(got, exp)


W4A8_REF_SHAPES = [(8, 8, 8, dict()), (16, 16, 16, dict()), (32, 32, 32, dict()),
                   (5, 11, 16, dict()), (7, 3, 8, dict()), (17, 19, 24, dict()),
                   (31, 35, 64, dict()), (60, 61, 128, dict()),
                   (32, 32, 32, dict(bias=True)), (17, 19, 24, dict(bias=True)),
                   (32, 32, 32, dict(clamp=(-0.5, 0.5))), (32, 32, 32, dict(c=True)),
                   (32, 32, 32, dict(c=True, bias=True, clamp=(-0.5, 0.5)))]
# Decode path (k % 256 == 0): k in pairs of 256 split over 8 waves, including empty waves
# (k = 256, 768), a tail pair per wave (k = 2304, 4352), activations staged in LDS
# (rows * k <= 8192) or read per step, several 15-row chunks with a short last one, and n tails.
W4A8_FAST_SHAPES = [(1, 160, 256, dict(bias=True)), (4, 100, 512, dict(bias=True, c=True)),
                    (15, 48, 768, dict(bias=True)), (16, 64, 1024, dict(clamp=(-0.5, 0.5))),
                    (33, 37, 2304, dict(bias=True)), (3, 45, 4352, dict(c=True)),
                    (2, 17, 2048, dict(bias=True)), (31, 33, 512, dict(bias=True, c=True)),
                    (2, 24, 65536, dict()),
                    # k % 256 != 0 goes to the per-output path
                    (15, 48, 384, dict(bias=True)), (33, 37, 640, dict(bias=True))]
# Decode strip path (m = 1, k = 2048 or 4096): channel counts that leave a wave partly (n % 4)
# or wholly (n % 16) past n, C, bias, clamps; m = 2-4 at the same k take the MFMA kernel.
W4A8_STRIP_SHAPES = [(1, 1, 2048, dict()), (1, 5, 4096, dict(bias=True)),
                     (1, 37, 2048, dict(c=True, bias=True, clamp=(-0.25, 0.5))),
                     (1, 16, 4096, dict(c=True)), (1, 1000, 4096, dict(bias=True)),
                     (2, 18, 4096, dict(c=True)), (3, 53, 4096, dict(bias=True)),
                     (3, 64, 2048, dict(c=True, bias=True)), (4, 23, 4096, dict(clamp=(-1.0, 0.0))),
                     (4, 1000, 2048, dict(bias=True))]


@pytest.mark.parametrize("m,n,k,opt", W4A8_REF_SHAPES + W4A8_FAST_SHAPES + W4A8_STRIP_SHAPES)
def test_w4a8_parity(gpu, m, n, k, opt):
    d = T.gen_w4a8(m, n, k, seed=42 + k, with_c=opt.get("c", False),
                   with_bias=opt.get("bias", False))
    cmin, cmax = opt.get("clamp", (-np.inf, np.inf))
    got = _gr().run_w4a8(d, cmin, cmax)
    exp = T.oracle_w4a8(d["A"], d["Bp"], d["C"], d["bias"], cmin, cmax, d["scale_a"], d["zp_a"],
                        d["scale_b"])
    np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_w4a8_extreme_values(gpu):
    """Largest accumulator the decode path admits: k = 65536, a = -128, q = 0 (w = -8)."""
    m, n, k = 3, 32, 65536
    d = T.gen_w4a8(m, n, k, seed=7, with_bias=True)
    d["A"][:] = -128
    d["A"][1, ::2] = 127
    d["Bp"][:] = 0x00
    d["Bp"][5:9] = 0xff
    got = _gr().run_w4a8(d)
    exp = T.oracle_w4a8(d["A"], d["Bp"], None, d["bias"], -np.inf, np.inf, d["scale_a"],
                        d["zp_a"], d["scale_b"])
    np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))


@pytest.mark.parametrize("zp", [-128, 127, 2**31 - 1, -2**31])
def test_w4a8_strip_extreme_values(gpu, zp):
    """Decode strip path (m = 1) at its extremes: activations -128 / 127 against weights -8 / 7
    (the nibble split's widest terms), zero points at the int8 and int32 limits (the zero-point
    correction wraps in 32 bits as the reference's does), k = 4096."""
    n, k = 40, 4096
    d = T.gen_w4a8(1, n, k, seed=11, with_bias=True)
    d["A"][:] = -128
    d["A"][:, 1::2] = 127
    d["zp_a"][0] = zp
    d["Bp"][:] = 0x00
    d["Bp"][3:7] = 0xff
    d["Bp"][9] = 0x0f
    d["Bp"][10] = 0xf0
    got = _gr().run_w4a8(d)
    exp = T.oracle_w4a8(d["A"], d["Bp"], None, d["bias"], -np.inf, np.inf, d["scale_a"],
                        d["zp_a"], d["scale_b"])
    np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))


@pytest.mark.parametrize("m", [1, 4, 8])
def test_w4a8_config3_full(gpu, m):
    """BASELINE cfg 3 at full size: K=4096, N=11008, M in {1, 4, 8}; bit-exact f32."""
    d = T.gen_w4a8(m, 11008, 4096, seed=42)
    got = _gr().run_w4a8(d)
    exp = T.oracle_w4a8(d["A"], d["Bp"], None, d["bias"], -np.inf, np.inf, d["scale_a"],
                        d["zp_a"], d["scale_b"])
    np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))


def w4a16_exact_and_scale(d):
    """Exact (float64) result and S = sum_k |a_k * w_k| per output, w = (q - 8) * s exactly."""
    A = T.bits_f16(d["A16"]).astype(np.float64)
    Bp, bl = d["Bp"], d["bl"]
    S16 = T.bits_f16(d["S16"]).astype(np.float32)
    m, k = A.shape
    n = Bp.shape[0]
    exact = np.zeros((m, n))
    S = np.zeros((m, n))
    Aabs = np.abs(A)
    for j0 in range(0, n, 2048):
        j1 = min(n, j0 + 2048)
        q = np.empty((j1 - j0, k), np.float32)
        q[:, 0::2] = (Bp[j0:j1] & 15).astype(np.float32) - 8
        q[:, 1::2] = (Bp[j0:j1] >> 4).astype(np.float32) - 8
        W = (q * np.repeat(S16[j0:j1], bl, axis=1)).astype(np.float64)  # exact in f32
        exact[:, j0:j1] = A @ W.T
        S[:, j0:j1] = Aabs @ np.abs(W).T
    if d["C16"] is not None:
        exact += T.bits_f16(d["C16"]).astype(np.float64)
        S += np.abs(T.bits_f16(d["C16"]).astype(np.float64))
    if d["bias16"] is not None:
        exact += T.bits_f16(d["bias16"]).astype(np.float64)[None, :]
    return exact, S


def ulp_distance_f16(got_bits, exp_vals, S):
    """|got - expected| in binary16 ULPs of max(|expected|, 2^-14, 2^-13 * S).

    Below magnitude 2^-13 * sum|a*w| one f16 ULP is smaller than a single f32 rounding of the
    accumulated sum, so no f32-accumulating evaluation order can promise it; the reference's
    own test oracle (sequential f32 sum) is within 1 ULP of exact math under this floor."""
    g = T.bits_f16(got_bits).astype(np.float64)
    e = np.asarray(exp_vals, np.float64)
    mag = np.maximum(np.maximum(np.abs(e), 2.0 ** -14), 2.0 ** -13 * S)
    ulp = 2.0 ** (np.floor(np.log2(mag)) - 10)
    return np.abs(g - e) / ulp


def check_w4a16(got, exp, d, clamp):
    """<= 2 f16 ULP against the f32-accumulating oracle and against exact math, with the ULP
    floored at 2^-13 * sum|a*w|. The outputs that pass only because of that floor (more than
    2 ULP of max(|expected|, 2^-14) from the oracle) are counted, printed and held to at most
    0.1% of the outputs (and 8 at least), so the floor cannot hide a systematic error."""
    exact, S = w4a16_exact_and_scale(d)
    exact = np.clip(exact, clamp[0], clamp[1])
    e_oracle = T.bits_f16(exp).astype(np.float64)
    d_oracle = ulp_distance_f16(got, e_oracle, S)
    d_exact = ulp_distance_f16(got, exact.astype(np.float16).astype(np.float64), S)
    assert d_oracle.max() <= 2.0, "max ULP vs oracle %s" % d_oracle.max()
    assert d_exact.max() <= 2.0, "max ULP vs exact %s" % d_exact.max()
    d_plain = ulp_distance_f16(got, e_oracle, np.zeros_like(S))
    on_floor = int((d_plain > 2.0).sum())
    print("W4A16 %dx%d: %d of %d outputs within 2 ULP only on the 2^-13*sum|a*w| floor "
          "(max plain ULP %.1f)" % (got.shape[0], got.shape[1], on_floor, got.size,
                                   float(d_plain.max())))
    assert on_floor <= max(8, got.size // 1000), on_floor
    return d_oracle, d_exact


W4A16_REF_SHAPES = [(8, 8, 4, 2, {}), (16, 16, 8, 2, {}), (32, 32, 32, 2, {}), (32, 32, 32, 4, {}),
                    (32, 32, 32, 32, {}), (5, 11, 10, 2, {}), (7, 3, 10, 2, {}),
                    (17, 19, 24, 4, {}), (31, 35, 64, 32, {}), (60, 61, 128, 32, {}),
                    (32, 32, 32, 2, dict(bias=True)), (17, 19, 24, 4, dict(bias=True)),
                    (32, 32, 32, 4, dict(clamp=(-0.5, 0.5))), (32, 32, 32, 4, dict(c=True)),
                    (32, 32, 32, 4, dict(c=True, bias=True, clamp=(-0.5, 0.5)))]
W4A16_FAST_SHAPES = [(32, 256, 4096, 32, dict(bias=True)), (1, 48, 128, 32, dict(bias=True)),
                     (33, 40, 512, 32, dict(c=True, bias=True)),
                     (64, 160, 1152, 32, dict(clamp=(-0.5, 0.5))),
                     # LDS strip kernel with 2-3 tiles per workgroup, a partial last tile and
                     # rows past m (k 2048), and 1-2 tiles per workgroup ending in a partial
                     # tile (k 4096)
                     (33, 8200, 2048, 32, dict(c=True, bias=True)),
                     (20, 4104, 4096, 32, dict(bias=True, clamp=(-0.5, 0.5))),
                     # chunk kernel with two and three 512-k chunks (the ring not yet full)
                     (32, 96, 1024, 32, dict(bias=True)),
                     (17, 300, 1536, 32, dict(c=True, clamp=(-0.5, 0.5)))]


@pytest.mark.parametrize("m,n,k,bl,opt", W4A16_REF_SHAPES + W4A16_FAST_SHAPES)
def test_w4a16_parity(gpu, shim, m, n, k, bl, opt):
    d = T.gen_w4a16(m, n, k, bl=bl, seed=42 + k, with_c=opt.get("c", False),
                    with_bias=opt.get("bias", False))
    lo, hi = opt.get("clamp", (-65504.0, 65504.0))
    cmin, cmax = int(T.f16_bits(lo)), int(T.f16_bits(hi))
    got = _gr().run_w4a16(shim, d, cmin, cmax)
    exp = T.oracle_w4a16(d["A16"], d["Bp"], d["S16"], bl, d["C16"], d["bias16"], cmin, cmax)
    check_w4a16(got, exp, d, (lo, hi))
    # distance to the RVV kernel's own f16-accumulating numerics, reported only: the reference
    # test accepts up to 1.0 absolute between those and the f32 oracle
    rvv = T.oracle_w4a16(d["A16"], d["Bp"], d["S16"], bl, d["C16"], d["bias16"], cmin, cmax,
                         rvv=True)
    diff = np.abs(T.bits_f16(got).astype(np.float64) - T.bits_f16(rvv).astype(np.float64))
    assert diff.max() <= 1.0


def test_w4a16_config4_full(gpu, shim):
    """BASELINE cfg 4 at full size: M=32, K=4096, N=14336, bl=32; <= 2 f16 ULP."""
    d = T.gen_w4a16(32, 14336, 4096, bl=32, seed=42)
    cmin, cmax = int(T.f16_bits(-65504.0)), int(T.f16_bits(65504.0))
    got = _gr().run_w4a16(shim, d, cmin, cmax)
    exp = T.oracle_w4a16(d["A16"], d["Bp"], d["S16"], 32, None, d["bias16"], cmin, cmax)
    check_w4a16(got, exp, d, (-65504.0, 65504.0))


IGEMM_REF = [  # (IC, OC, IH, IW, KH, KW, stride, pad, dil)
    (3, 16, 8, 8, 3, 3, (1, 1), (0, 0), (1, 1)),
    (16, 32, 8, 8, 3, 3, (1, 1), (0, 0), (1, 1)),
    (16, 32, 8, 8, 1, 1, (1, 1), (0, 0), (1, 1)),
    (3, 16, 8, 8, 3, 3, (1, 1), (1, 1), (1, 1)),
    (3, 16, 8, 8, 3, 3, (2, 2), (0, 0), (1, 1)),
    (3, 16, 8, 8, 3, 3, (1, 1), (2, 2), (2, 2)),
    (3, 16, 8, 8, 3, 3, (2, 2), (1, 1), (1, 1)),
    (8, 16, 7, 11, 3, 5, (1, 1), (0, 0), (1, 1)),
    (64, 128, 4, 4, 1, 1, (1, 1), (0, 0), (1, 1)),
    (3, 32, 16, 16, 3, 3, (1, 1), (1, 1), (1, 1)),
    (3, 8, 6, 6, 3, 3, (1, 1), (0, 0), (1, 1)),
    (64, 32, 4, 4, 3, 3, (1, 1), (1, 1), (1, 1)),
]
IGEMM_FAST = [
    (32, 48, 9, 13, 3, 3, (1, 1), (1, 1), (1, 1)),
    (128, 128, 14, 14, 3, 3, (2, 2), (1, 1), (1, 1)),
    (16, 24, 12, 10, 5, 3, (1, 2), (2, 1), (1, 2)),
]


@pytest.mark.parametrize("ic,oc,ih,iw,kh,kw,stride,pad,dil", IGEMM_REF + IGEMM_FAST)
def test_igemmcl_parity(gpu, ic, oc, ih, iw, kh, kw, stride, pad, dil):
    d = T.gen_igemmcl(1, ih, iw, ic, oc, kh, kw, stride=stride, pad=pad, dil=dil, seed=ic + oc)
    got = _gr().run_igemmcl(d)
    exp = T.oracle_igemmcl(d["inp"], d["W"], d["bias"], -128, 127, d["conv"], d["scale_a"],
                           d["scale_b"], oc, d["scale_d"], d["zp_d"])
    np.testing.assert_array_equal(got, exp)


def test_igemmcl_tiled_calls(gpu):
    """The reference caller pattern: one run per m_step tile with m_idx (D addressed
    absolutely), covering a ragged last tile."""
    d = T.gen_igemmcl(2, 10, 9, 32, 40, 3, 3, pad=(1, 1), seed=5)
    conv = d["conv"]
    M = conv.output_shape[0] * conv.output_shape[1] * conv.output_shape[2]
    step = 64
    D = np.zeros((M, 40), np.int8)
    for m_idx in range(0, M, step):
        D = _gr().run_igemmcl(d, m=min(step, M - m_idx), m_idx=m_idx, D_init=D)
    exp = T.oracle_igemmcl(d["inp"], d["W"], d["bias"], -128, 127, conv, d["scale_a"],
                           d["scale_b"], 40, d["scale_d"], d["zp_d"])
    np.testing.assert_array_equal(D, exp)


def test_igemmcl_config5_full(gpu):
    """BASELINE cfg 5 at full size: NHWC 8x56x56x128 (batch as depth), 3x3, OC 128, pad 1."""
    d = T.gen_igemmcl(8, 56, 56, 128, 128, 3, 3, pad=(1, 1), seed=42)
    got = _gr().run_igemmcl(d)
    exp = T.oracle_igemmcl(d["inp"], d["W"], d["bias"], -128, 127, d["conv"], d["scale_a"],
                           d["scale_b"], 128, d["scale_d"], d["zp_d"])
    np.testing.assert_array_equal(got, exp)


def test_interfaces_and_null_params(gpu, shim, lib):
    """NULL params leave D untouched (reference run_* returns early)."""
    import torch

    D = torch.full((4, 4), 7, dtype=torch.int8, device="cuda:0")
    lib.fn("w8a8", "run")(4, 4, 16, None, 16, 0, None, 16, 0, None, 4, D.data_ptr(), 4, None,
                          -128, 127, None)
    assert int(D.sum().item()) == 7 * 16
