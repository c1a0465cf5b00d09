"""CPU checks that pin the oracle (oracle/tqt_oracle.c) before it is trusted as the checker.

Sources of truth, in order of strength:
  1. golden fixtures written by tests/golden/make_golden.py from the reference's own compiled
     test code (its RNG, reference_gemm_i32_i8, reference_gemm_quantized_weight_mixed,
     tqt_im2col_cl, tqt_quantize_multiplier, quantize helpers);
  2. the same reference code live (oracle/_ref/libtqt_ref.so) where it was built;
  3. independent closed forms (numpy int64 / float64 products, numpy float16 rounding);
  4. hand-computed known answers and invariants for the requantization epilogue, which only
     the RVV source text defines (tqt_kernel_gemm_i8_i8_4x1vl_rvv.h:334-408).
"""

import ctypes
import os

import numpy as np
import pytest

import tqt_testlib as T

G = T.GOLDEN_DIR


def golden(name):
    """All arrays of a fixture, loaded eagerly: an NpzFile re-reads each key on access, so a
    pointer taken from g[key] would outlive the temporary array it points into."""
    with np.load(os.path.join(G, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ------------------------------------------------------------------------------------------
# binary16 conversion helpers (checked against numpy's own rounding)
# ------------------------------------------------------------------------------------------

def test_f16_to_f32_exhaustive():
    o = T.oracle()
    bits = np.arange(65536, dtype=np.uint16)
    got = np.array([o.tqto_f16_to_f32(int(b)) for b in bits], np.float32)
    exp = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), exp[~nan].view(np.uint32))


def test_f32_to_f16_rounding():
    o = T.oracle()
    rng = np.random.default_rng(0)
    # every f16 value, every midpoint between neighbours (ties), neighbours of midpoints,
    # overflow boundary, subnormal range, random values
    h = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (h[:-1] + h[1:]) / 2
    vals = np.concatenate([h, mids, np.nextafter(mids, 0), np.nextafter(mids, 1), -mids,
                           [65504.0, 65519.99, 65520.0, 1e6, 2.0 ** -25, 2.0 ** -26, 3e-8],
                           rng.standard_normal(20000) * 10.0 ** rng.uniform(-8, 5, 20000)])
    vals = vals.astype(np.float32)
    got = np.array([o.tqto_f32_to_f16(float(v)) for v in vals], np.uint16)
    exp = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, exp)


def test_bf16_conversions():
    """bfloat16 widening is exact for every pattern; narrowing rounds to nearest even on the 16
    dropped bits (checked against an integer formulation of RNE and against the defining
    property: the result is a neighbour of x and the nearer one, ties to even), NaN -> 0x7fc0."""
    o = T.oracle()
    bits = np.arange(65536, dtype=np.uint16)
    got = np.array([o.tqto_bf16_to_f32(int(b)) for b in bits], np.float32)
    exp = (bits.astype(np.uint32) << 16).view(np.float32)
    nan = np.isnan(exp)
    assert np.array_equal(got[~nan].view(np.uint32), exp[~nan].view(np.uint32))
    rng = np.random.default_rng(1)
    u = np.concatenate([rng.integers(0, 2 ** 32, 40000, dtype=np.uint64).astype(np.uint32),
                        np.array([0x3f808000, 0x3f818000, 0x3f80ffff, 0x7f7fffff, 0x7f800000,
                                  0xff800000, 0x7fc00001, 0x00008000, 0x80018000], np.uint32)])
    vals = u.view(np.float32)
    got = np.array([o.tqto_f32_to_bf16(float(v)) for v in vals], np.uint16)
    np.testing.assert_array_equal(got, T.bf16_bits(vals))
    fin = np.isfinite(vals) & (np.abs(vals) < 3.38e38)
    x = vals[fin].astype(np.float64)
    y = T.bits_bf16_f32(got[fin]).astype(np.float64)
    lo = T.bits_bf16_f32((u[fin] >> 16).astype(np.uint16)).astype(np.float64)  # truncation
    step = np.abs(T.bits_bf16_f32(((u[fin] >> 16) + 1).astype(np.uint16)).astype(np.float64) - lo)
    assert np.all(np.abs(y - x) <= step / 2 + 0.0)
    ties = np.abs(np.abs(y - x) - step / 2) == 0
    assert np.all((got[fin][ties] & 1) == 0)
    assert all(o.tqto_f32_to_bf16(float("nan")) == 0x7FC0 for _ in range(1))


def test_w4a8_h16_is_f32_epilogue_then_narrowing():
    """The f16 / bf16 output siblings: the f32 oracle on widened C, bias and clamp bounds,
    rounded once (f16: numpy's RNE; bf16: the integer RNE above)."""
    m, n, k = 5, 40, 256
    d = T.gen_w4a8(m, n, k, seed=8, with_c=True)
    rng = np.random.default_rng(9)
    for bf16 in (False, True):
        if bf16:
            C16, b16 = T.bf16_bits(d["C"]), T.bf16_bits(d["bias"])
            w = T.bits_bf16_f32
            cmin, cmax = int(T.bf16_bits(np.float32(-3.0))), int(T.bf16_bits(np.float32(2.5)))
        else:
            C16, b16 = T.f16_bits(d["C"]), T.f16_bits(d["bias"])
            w = lambda b: T.bits_f16(b).astype(np.float32)
            cmin, cmax = int(T.f16_bits(-3.0)), int(T.f16_bits(2.5))
        got = T.oracle_w4a8_h16(d["A"], d["Bp"], C16, b16, cmin, cmax, d["scale_a"], d["zp_a"],
                                d["scale_b"], bf16)
        f32 = T.oracle_w4a8(d["A"], d["Bp"], w(C16), w(b16), float(w(np.uint16(cmin))),
                            float(w(np.uint16(cmax))), d["scale_a"], d["zp_a"], d["scale_b"])
        exp = T.bf16_bits(f32) if bf16 else f32.astype(np.float16).view(np.uint16)
        np.testing.assert_array_equal(got, exp)
    del rng


# ------------------------------------------------------------------------------------------
# Requantization multiplier
# ------------------------------------------------------------------------------------------

def qm(x):
    o = T.oracle()
    m, s = ctypes.c_int32(), ctypes.c_int32()
    o.tqto_quantize_multiplier(float(x), ctypes.byref(m), ctypes.byref(s))
    return m.value, s.value


def test_quantize_multiplier_known_answers():
    # frexp convention: x = (mult / 2^31) * 2^shift, mult in [2^30, 2^31)
    assert qm(0.5) == (1 << 30, 0)
    assert qm(0.25) == (1 << 30, -1)
    assert qm(1.0) == (1 << 30, 1)
    assert qm(0.0004)[1] == -11
    assert qm(0.0) == (0, 0)
    assert qm(2.0 ** -40) == (0, 0)  # shift < -31 flushes to zero
    assert qm(0.75) == (3 << 29, 0)
    # 2^30 + all-ones upper fraction rounds up to 2^31 -> halved, shift + 1
    assert qm(1.0 - 2.0 ** -53) == (1 << 30, 1)
    assert qm(-0.5) == (-(1 << 30), 0)


def test_quantize_multiplier_vs_reference_golden():
    g = golden("ref_qm.npz")
    got = np.array([qm(x) for x in g["x"]], np.int64)
    assert np.array_equal(got[:, 0], g["mult"])
    assert np.array_equal(got[:, 1], g["shift"])


def test_quantize_multiplier_closed_form():
    """For finite x in [2^-31, 2^31) the pair approximates x within half a Q31 step."""
    rng = np.random.default_rng(3)
    for x in 10.0 ** rng.uniform(-9, 6, 5000):
        m, s = qm(x)
        approx = m * 2.0 ** (s - 31)
        assert abs(approx - x) <= 2.0 ** (s - 31) * 0.5 + 1e-300
        assert (1 << 30) <= m < (1 << 31)


# ------------------------------------------------------------------------------------------
# Requantization epilogue (only the RVV text defines it: hand known-answers + invariants)
# ------------------------------------------------------------------------------------------

def rq(acc, mult, shift, zp=0, cmin=-128, cmax=127):
    return T.oracle().tqto_requant_one(acc, mult, shift, zp, cmin, cmax)


def test_requant_known_answers():
    M30 = 1 << 30
    assert rq(-5, M30, 0) == -2          # floor(-1.25): vmulh rounds toward -inf
    assert rq(5, M30, 0) == 1            # floor(1.25)
    assert rq(-1, M30, 0) == -1          # floor(-0.25)
    assert rq(100, M30, 1, 3) == 15      # 25 >> 1 = 12, + 3
    assert rq(-100, M30, 1) == -13       # -25 >> 1 = -13 (arithmetic shift)
    assert rq(1000000, M30, 0) == 127    # saturate high
    assert rq(-1000000, M30, 0) == -128  # saturate low
    assert rq(2**31 - 1, 2**31 - 1, 0, 2**31 - 1) == -128  # 32-bit wrap of the zp add
    assert rq(2**31 - 1, M30, -1) == 0   # stored shift -1 shifts by 31
    assert rq(40, M30, 0, 0, -5, 7) == 7  # clamp after saturation
    assert rq(-40, M30, 0, 0, -5, 7) == -5
    assert rq(12345, 0, 0, 9) == 9       # zero multiplier


def test_requant_invariants():
    rng = np.random.default_rng(5)
    for _ in range(200):
        mult = int(rng.integers(1 << 30, 1 << 31))
        shift = int(rng.integers(0, 12))
        zp = int(rng.integers(-20, 21))
        accs = np.sort(rng.integers(-(1 << 20), 1 << 20, 64))
        ys = [rq(int(a), mult, shift, zp) for a in accs]
        assert all(ys[i] <= ys[i + 1] for i in range(len(ys) - 1))  # monotone
        real = mult / 2.0 ** 32 / 2.0 ** shift
        for a, y in zip(accs, ys):
            exact = np.floor(np.floor(a * mult / 2.0 ** 32) / 2.0 ** shift) + zp
            assert y == int(np.clip(exact, -128, 127))
            if -128 < y < 127:
                assert a * real + zp - 1 < y <= a * real + zp + 1e-9  # floor, not round


# ------------------------------------------------------------------------------------------
# GEMM restatements vs the reference's own test code
# ------------------------------------------------------------------------------------------

def test_clamp_i32_vs_reference_golden():
    g = golden("ref_clamp_i32.npz")
    for i, (m, n, k, with_c) in enumerate(g["shapes"]):
        A, B, D = g["clamp_%d_A" % i], g["clamp_%d_B" % i], g["clamp_%d_D" % i]
        C = g["clamp_%d_C" % i] if with_c else None
        got = T.oracle_clamp(A, B, C, -100000, 100000)
        np.testing.assert_array_equal(got, D)
        ref64 = A.astype(np.int64) @ B.astype(np.int64) + (0 if C is None else C)
        np.testing.assert_array_equal(got, np.clip(ref64, -100000, 100000))


def test_w4a16_f32acc_vs_reference_golden():
    """The f32-accumulating W4A16 oracle reproduces reference_gemm_quantized_weight_mixed
    bit for bit on the reference's own test inputs (its RNG, its int4 quantizer)."""
    g = golden("ref_w4a16.npz")
    for i, (m, n, k, bl, bias, c, clamp) in enumerate(g["shapes"]):
        pre = "w4a16_%d_" % i
        C = g[pre + "C"] if c else None
        bv = g[pre + "bias"] if bias else None
        cmin, cmax = (int(v) for v in g[pre + "clamp"])
        got = T.oracle_w4a16(g[pre + "A"], g[pre + "Bp"], g[pre + "S"], int(bl), C, bv, cmin, cmax)
        np.testing.assert_array_equal(got, g[pre + "D"])


def test_w4a16_f32out_vs_reference_golden():
    """The f32-output W4A16 oracle reproduces reference_gemm_quantized_weight_mixed<f16, float>
    bit for bit on the reference runner's own inputs (f32 C and bias from its generator,
    +-FLT_MAX or +-0.5 clamps)."""
    g = golden("ref_w4a16_f32.npz")
    for i, (m, n, k, bl, bias, c, clamp) in enumerate(g["shapes"]):
        pre = "w4a16f_%d_" % i
        C = g[pre + "C"] if c else None
        bv = g[pre + "bias"] if bias else None
        lo, hi = (float(v) for v in g[pre + "clamp"])
        got = T.oracle_w4a16_f32(g[pre + "A"], g[pre + "Bp"], g[pre + "S"], int(bl), C, bv, lo,
                                 hi)
        np.testing.assert_array_equal(got.view(np.uint32), g[pre + "D"].view(np.uint32))


def test_w4a16_f32out_rounds_to_the_f16_oracle():
    """With f16-valued C, bias and bounds the two W4A16 oracles share every step up to the
    store, so the f16 one is the f32 one rounded to f16 (numpy RNE)."""
    d = T.gen_w4a16(9, 40, 256, bl=32, seed=11, with_c=True, with_bias=True)
    lo, hi = T.f16_bits(-3.0), T.f16_bits(2.5)
    h = T.oracle_w4a16(d["A16"], d["Bp"], d["S16"], 32, d["C16"], d["bias16"], int(lo), int(hi))
    f = T.oracle_w4a16_f32(d["A16"], d["Bp"], d["S16"], 32, T.bits_f16(d["C16"]),
                           T.bits_f16(d["bias16"]), -3.0, 2.5)
    np.testing.assert_array_equal(h, f.astype(np.float16).view(np.uint16))


def test_w4a16_f32out_closed_form():
    """Independent float64 evaluation: each of the k + 2 rounded additions and k products of
    the f32 loop moves the result by at most 2^-24 of the running magnitude, so the oracle is
    within (2k + 4) * 2^-24 * (sum|a*w| + |C| + |bias|) of exact math; a dropped term, wrong
    nibble order or wrong block index misses by far more."""
    m, n, k, bl = 6, 50, 512, 16
    d = T.gen_w4a16(m, n, k, bl=bl, seed=12, with_bias=False)
    rng = np.random.default_rng(13)
    C = rng.uniform(-5, 5, size=(m, n)).astype(np.float32)
    bias = rng.uniform(-0.5, 0.5, size=n).astype(np.float32)
    got = T.oracle_w4a16_f32(d["A16"], d["Bp"], d["S16"], bl, C, bias, -np.inf, np.inf)
    A = T.bits_f16(d["A16"]).astype(np.float64)
    q = np.empty((n, k))
    q[:, 0::2] = (d["Bp"] & 15) - 8.0
    q[:, 1::2] = (d["Bp"] >> 4) - 8.0
    W = q * np.repeat(T.bits_f16(d["S16"]).astype(np.float64), bl, axis=1)
    exact = A @ W.T + C + bias
    S = np.abs(A) @ np.abs(W).T + np.abs(C) + np.abs(bias)
    assert np.all(np.abs(got - exact) <= (2 * k + 4) * 2.0 ** -24 * S)
    assert np.abs(got - exact).max() > 0  # the f32 loop does round


def test_f16_add_is_correctly_rounded():
    """binary16 addition: the exact float64 sum rounded once by numpy's float64 -> float16
    conversion, over random normal, subnormal, huge and special patterns."""
    o = T.oracle()
    rng = np.random.default_rng(31)
    a = rng.integers(0, 65536, 6000).astype(np.uint16)
    b = rng.integers(0, 65536, 6000).astype(np.uint16)
    b[:2000] = (a[:2000] ^ rng.integers(0, 64, 2000).astype(np.uint16))  # close magnitudes
    got = np.array([o.tqto_f16_add(int(x), int(y)) for x, y in zip(a, b)], np.uint16)
    with np.errstate(all="ignore"):
        exp = (T.bits_f16(a).astype(np.float64) + T.bits_f16(b).astype(np.float64))
        exp = exp.astype(np.float16).view(np.uint16)
    nan = np.isnan(T.bits_f16(exp))
    assert np.array_equal(got[~nan], exp[~nan])
    assert np.all(np.isnan(T.bits_f16(got[nan])))


def _dyn_golden():
    g = golden("ref_w8a8dyn.npz")
    for i, (m, n, k, _c) in enumerate(g["shapes"]):
        pre = "w8a8dyn_%d_" % i
        yield {key: g[pre + key] for key in ("A", "B", "scale_a", "zp_a", "scale_b", "bias",
                                             "Dref")}


def test_w8a8dyn_within_reference_tolerance():
    """The dynamic-quantization oracle, on the reference runner's own inputs, passes the
    reference test's own check against reference_gemm<float> of the unquantized operands
    (quantized_gemm_test_runner.h:1414-1423: abs 1.5 / cosine 0.998 for f32, 2.5 / 0.997 for
    f16, bounds +-FLT_MAX converted to the output type)."""
    for d in _dyn_golden():
        ref = d["Dref"].astype(np.float64)
        for f16 in (False, True):
            if f16:
                got = T.oracle_w8a8dyn(d["A"], d["B"], T.f16_bits(d["bias"]), 0xFC00, 0x7C00,
                                       d["scale_a"], d["zp_a"], d["scale_b"], f16=True)
                got = T.bits_f16(got).astype(np.float64)
                tol, cos_min = 2.5, 0.997
            else:
                fm = float(np.finfo(np.float32).max)
                got = T.oracle_w8a8dyn(d["A"], d["B"], d["bias"], -fm, fm, d["scale_a"],
                                       d["zp_a"], d["scale_b"]).astype(np.float64)
                tol, cos_min = 1.5, 0.998
            assert np.abs(got - ref).max() <= tol
            cos = (got * ref).sum() / (np.linalg.norm(got) * np.linalg.norm(ref) + 1e-30)
            assert cos >= cos_min


def test_w8a8dyn_closed_form():
    """Independent evaluation: the int32 accumulator from an int64 matrix product of
    (A - zp_a) and B, then the f32 epilogue steps in numpy float32 (each rounded: f32(acc),
    sigma = sb * sa, product, + bias, clamp); and the f16 output as numpy's f16 rounding of that
    product, an exactly rounded f16 bias add, and the f16 clamp."""
    d = T.gen_w8a8dyn(7, 45, 300, seed=3)
    A64 = d["A"].astype(np.int64) - d["zp_a"].astype(np.int64)[:, None]
    acc = (A64 @ d["B"].astype(np.int64).T).astype(np.int32)
    sigma = d["scale_b"][None, :] * d["scale_a"][:, None]
    prod = acc.astype(np.float32) * sigma
    f = np.minimum(np.maximum(prod + d["bias"][None, :], np.float32(-40.0)), np.float32(35.0))
    got = T.oracle_w8a8dyn(d["A"], d["B"], d["bias"], -40.0, 35.0, d["scale_a"], d["zp_a"],
                           d["scale_b"])
    np.testing.assert_array_equal(got.view(np.uint32), f.view(np.uint32))
    b16 = T.f16_bits(d["bias"])
    h = prod.astype(np.float16).astype(np.float64) + T.bits_f16(b16).astype(np.float64)[None, :]
    h = np.minimum(np.maximum(h.astype(np.float16), np.float16(-40.0)), np.float16(35.0))
    got16 = T.oracle_w8a8dyn(d["A"], d["B"], b16, int(T.f16_bits(-40.0)),
                             int(T.f16_bits(35.0)), d["scale_a"], d["zp_a"], d["scale_b"],
                             f16=True)
    np.testing.assert_array_equal(got16, h.view(np.uint16))


def test_w8a8dyn_zero_point_shift_invariance():
    """Moving a row's int8 values and its zero point by the same c leaves every output bit
    unchanged (the correction enters as q_a - zp_a); a sign error in the correction fails."""
    d = T.gen_w8a8dyn(5, 30, 200, seed=4, zp_range=(-20, 20))
    A = np.clip(d["A"], -100, 100).astype(np.int8)
    base = T.oracle_w8a8dyn(A, d["B"], d["bias"], -np.inf, np.inf, d["scale_a"], d["zp_a"],
                            d["scale_b"])
    for c in (-27, 13):
        got = T.oracle_w8a8dyn((A.astype(np.int32) + c).astype(np.int8), d["B"], d["bias"],
                               -np.inf, np.inf, d["scale_a"], d["zp_a"] + c, d["scale_b"])
        np.testing.assert_array_equal(got.view(np.uint32), base.view(np.uint32))


def test_w8a8dyn_sixteen_bit_difference_and_signed_zero():
    """Hand-worked cases of the RVV steps: q_a - zp_a is used modulo 2^16 (vwmacc.vx at SEW 16),
    a NULL bias still adds +0 (so a -0 product becomes +0), and vfmax orders -0 below +0."""
    A = np.array([[5, -3]], np.int8)
    B = np.array([[2, 1]], np.int8)
    # zp = 40000: int16(5 - 40000) = 25541, int16(-3 - 40000) = 25533 -> 2*25541 + 25533 = 76615
    got = T.oracle_w8a8dyn(A, B, None, -np.inf, np.inf, [1.0], [40000], [1.0])
    assert got[0, 0] == np.float32(76615.0)
    Z = np.zeros((1, 2), np.int8)
    neg = T.oracle_w8a8dyn(Z, B, None, -np.inf, np.inf, [1.0], [0], [-1.0])
    assert neg.view(np.uint32)[0, 0] == 0  # -0 product + 0 = +0
    both = T.oracle_w8a8dyn(Z, B, np.array([-0.0], np.float32), 0.0, np.inf, [1.0], [0], [-1.0])
    assert both.view(np.uint32)[0, 0] == 0  # -0 + -0 = -0, then vfmax(-0, +0) = +0


def test_im2col_cf_vs_reference_golden():
    """The channel-first im2col restatement reproduces the reference's tqt_im2col_cf byte for
    byte on its conv shape list, every group."""
    g = golden("ref_im2col_cf.npz")
    for i, (IC, OC, IH, IW, KH, KW, SH, SW, PH, PW, DH, DW) in enumerate(g["shapes"]):
        groups = int(g["cf_%d_groups" % i][0])
        conv = T.make_conv((1, IH, IW), (1, KH, KW), (1, SH, SW), (1, DH, DW), (0, PH, PW),
                           int(IC), int(OC), groups)
        for grp in range(groups):
            np.testing.assert_array_equal(T.oracle_im2col_cf(g["cf_%d_input" % i], conv, grp),
                                          g["cf_%d_col_g%d" % (i, grp)])


def test_mx1bias_is_the_transposed_w8a8():
    """gemm_mx1bias (per-row weights scale, bias and requantization) equals the transpose of the
    pinned W8A8 oracle (per-column scale, bias and requantization) with the operands swapped:
    the same int32 sums, and multipliers from the same double product."""
    m, n, k = 37, 45, 70
    d = T.gen_mx1bias(m, n, k, seed=5, with_c=False)
    got = T.oracle_mx1bias(d["A"], d["B"], None, d["bias"], -100, 110, d["scale_a"], m,
                           d["scale_b"], d["scale_d"], d["zp_d"])
    exp = T.oracle_w8a8(np.ascontiguousarray(d["B"].T), d["A"], None, d["bias"], -100, 110,
                        d["scale_b"], d["scale_a"], m, d["scale_d"], d["zp_d"])
    np.testing.assert_array_equal(got, exp.T)
    # one shared multiplier (quant_channel_a == 1) and C
    d = T.gen_mx1bias(m, n, k, seed=6, with_c=True, qca=1)
    got = T.oracle_mx1bias(d["A"], d["B"], d["C"], d["bias"], -128, 127, d["scale_a"], 1,
                           d["scale_b"], d["scale_d"], d["zp_d"])
    exp = T.oracle_w8a8(np.ascontiguousarray(d["B"].T), d["A"], np.ascontiguousarray(d["C"].T),
                        d["bias"], -128, 127, d["scale_b"], d["scale_a"], 1, d["scale_d"],
                        d["zp_d"])
    np.testing.assert_array_equal(got, exp.T)


def test_igemmcf_is_im2col_cf_then_mx1bias():
    """The implicit channel-first oracle on a pixel window [n_idx, n_idx + n) equals the
    mx1bias GEMM on those columns of the (golden-pinned) channel-first im2col."""
    rng = np.random.default_rng(8)
    IC, OC, groups = 12, 10, 2
    conv = T.make_conv((2, 9, 8), (1, 3, 3), (1, 2, 1), (1, 1, 2), (0, 1, 1), IC, OC, groups)
    inp = rng.integers(-128, 128, size=(IC, 2, 9, 8), dtype=np.int64).astype(np.int8)
    icg = IC // groups
    K = icg * 9
    N = conv.output_shape[0] * conv.output_shape[1] * conv.output_shape[2]
    ocg = OC // groups
    W = rng.integers(-127, 128, size=(ocg, K), dtype=np.int64).astype(np.int8)
    bias = rng.integers(-500, 500, size=ocg, dtype=np.int64).astype(np.int32)
    sa = rng.uniform(0.002, 0.01, size=ocg).astype(np.float32)
    for grp in range(groups):
        for n_idx, nn in ((0, N), (5, N - 9)):
            D = np.zeros((ocg, N), np.int8)
            T.oracle().tqto_igemmcf_qsi8dx(ocg, nn, T.ptr(inp), grp, n_idx, T.ptr(W), K, T.ptr(D),
                                           N, T.ptr(bias), -128, 127, ctypes.byref(conv),
                                           T.ptr(sa), ocg, 0.03, 0.1, 4)
            col = T.oracle_im2col_cf(inp, conv, grp)
            exp = T.oracle_mx1bias(W, np.ascontiguousarray(col[:, n_idx:n_idx + nn]), None, bias,
                                   -128, 127, sa, ocg, 0.03, 0.1, 4)
            np.testing.assert_array_equal(D[:, n_idx:n_idx + nn], exp)
            assert not D[:, :n_idx].any() and not D[:, n_idx + nn:].any()


def test_w4a16_rvv_numerics_within_reference_tolerance():
    """The RVV-numerics restatement (f16 weights, f16 FMA chain) stays within the reference
    test's own tolerance (abs 1.0, cosine 0.9999) of the f32 oracle on the reference inputs."""
    g = golden("ref_w4a16.npz")
    for i, (m, n, k, bl, bias, c, clamp) in enumerate(g["shapes"]):
        pre = "w4a16_%d_" % i
        C = g[pre + "C"] if c else None
        bv = g[pre + "bias"] if bias else None
        cmin, cmax = (int(v) for v in g[pre + "clamp"])
        got = T.bits_f16(T.oracle_w4a16(g[pre + "A"], g[pre + "Bp"], g[pre + "S"], int(bl), C,
                                        bv, cmin, cmax, rvv=True)).astype(np.float64)
        ref = T.bits_f16(g[pre + "D"]).astype(np.float64)
        assert np.abs(got - ref).max() <= 1.0
        cos = (got * ref).sum() / (np.linalg.norm(got) * np.linalg.norm(ref) + 1e-30)
        assert cos >= 0.9999


def test_w4a16_f32acc_closed_form():
    """Independent float64 evaluation: the f32 oracle is within 2 f16 ULP (ULP floored at the
    f32 accumulation-noise scale 2^-13 * sum|a*w|) of exact math."""
    d = T.gen_w4a16(16, 96, 1024, bl=32, seed=9, with_c=True, with_bias=True)
    cmin, cmax = int(T.f16_bits(-65504.0)), int(T.f16_bits(65504.0))
    got = T.bits_f16(T.oracle_w4a16(d["A16"], d["Bp"], d["S16"], 32, d["C16"], d["bias16"], cmin,
                                    cmax)).astype(np.float64)
    A = T.bits_f16(d["A16"]).astype(np.float64)
    q = np.empty((96, 1024))
    q[:, 0::2] = (d["Bp"] & 15) - 8.0
    q[:, 1::2] = (d["Bp"] >> 4) - 8.0
    W = q * np.repeat(T.bits_f16(d["S16"]).astype(np.float64), 32, axis=1)
    exact = A @ W.T + T.bits_f16(d["C16"]) + T.bits_f16(d["bias16"])[None, :]
    S = np.abs(A) @ np.abs(W).T + np.abs(T.bits_f16(d["C16"]).astype(np.float64))
    mag = np.maximum(np.maximum(np.abs(exact), 2.0 ** -14), 2.0 ** -13 * S)
    ulp = 2.0 ** (np.floor(np.log2(mag)) - 10)
    assert (np.abs(got - exact.astype(np.float16).astype(np.float64)) / ulp).max() <= 2.0


def test_w4a16_rejects_dropped_scale():
    """A plausible mistake (scale of the wrong block) is caught by the closed-form check."""
    d = T.gen_w4a16(4, 16, 128, bl=32, seed=2, with_bias=False)
    cmin, cmax = int(T.f16_bits(-65504.0)), int(T.f16_bits(65504.0))
    ok = T.bits_f16(T.oracle_w4a16(d["A16"], d["Bp"], d["S16"], 32, None, None, cmin, cmax))
    bad_s = d["S16"].copy()
    bad_s[:, [0, 1]] = bad_s[:, [1, 0]]
    bad = T.bits_f16(T.oracle_w4a16(d["A16"], d["Bp"], bad_s, 32, None, None, cmin, cmax))
    assert np.abs(ok.astype(np.float64) - bad.astype(np.float64)).max() > 1e-2


def test_w8a8_accumulator_closed_form():
    d = T.gen_w8a8(37, 45, 96, seed=4, with_c=True)
    acc = T.oracle_w8a8_acc(d["A"], d["B"], d["C"], d["bias"])
    exp = (d["A"].astype(np.int64) @ d["B"].astype(np.int64).T + d["C"] + d["bias"][None, :])
    np.testing.assert_array_equal(acc, exp.astype(np.int32))


def test_w8a8_is_acc_then_requant():
    """The W8A8 oracle equals (closed-form int32 accumulator) -> per-column reference
    multiplier (golden-pinned) -> pinned requantization, element by element."""
    d = T.gen_w8a8(24, 40, 64, seed=8)
    d["scale_d"] = np.float32(0.2)  # keep most outputs unsaturated
    D = T.oracle_w8a8(d["A"], d["B"], None, d["bias"], -128, 127, d["scale_a"], d["scale_b"], 40,
                      d["scale_d"], 0)
    acc = d["A"].astype(np.int64) @ d["B"].astype(np.int64).T + d["bias"][None, :]
    r = T.ref()
    for j in range(40):
        real = float(np.float64(d["scale_a"]) * np.float64(d["scale_b"][j]) /
                     np.float64(d["scale_d"]))
        m, s = qm(real)
        if r is not None:
            mm, ss = ctypes.c_int32(), ctypes.c_int32()
            r.tqtr_quantize_multiplier(real, ctypes.byref(mm), ctypes.byref(ss))
            assert (mm.value, ss.value) == (m, s)
        for i in range(24):
            assert D[i, j] == rq(int(acc[i, j]), m, -s - 1)
    assert 0.2 < np.mean((D > -128) & (D < 127))


def test_w8a8_float_sanity_like_reference_test():
    """The reference test's own acceptance (test/common/quantized_gemm_test_runner.h:190-306):
    dequantized int8 output within 1.0 absolute and cosine 0.999 of the fp32 reference GEMM."""
    o = T.oracle()
    m, n, k = 32, 48, 64
    rng = np.random.default_rng(42)
    Af = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    Bf = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    bf = rng.uniform(-10, 10, n).astype(np.float32)
    sa, za = ctypes.c_float(), ctypes.c_int32()
    o.tqto_compute_asym_quant_params_i8(T.ptr(Af), m * k, ctypes.byref(sa), ctypes.byref(za))
    sb = np.zeros(n, np.float32)
    for ch in range(n):
        s = ctypes.c_float()
        o.tqto_compute_sym_quant_params_i8(T.ptr(Bf[ch]), k, ctypes.byref(s))
        sb[ch] = s.value
    A = np.array([[o.tqto_quantize_i8(float(v), sa.value, za.value) for v in row] for row in Af],
                 np.int8)
    B = np.array([[o.tqto_quantize_i8(float(v), float(sb[ch]), 0) for v in Bf[ch]]
                  for ch in range(n)], np.int8)
    bias = np.array([o.tqto_quantize_bias_i32(float(bf[ch]), sa.value * float(sb[ch]))
                     for ch in range(n)], np.int32)
    fused = np.zeros(n, np.int32)
    o.tqto_fuse_zp_to_bias(T.ptr(fused), T.ptr(bias), T.ptr(B), za.value, n, k)
    ref = Af.astype(np.float64) @ Bf.astype(np.float64).T + bf[None, :]
    sd, zd = ctypes.c_float(), ctypes.c_int32()
    ref32 = ref.astype(np.float32)
    o.tqto_compute_asym_quant_params_i8(T.ptr(ref32), m * n, ctypes.byref(sd), ctypes.byref(zd))
    D = T.oracle_w8a8(A, B, None, fused, -128, 127, sa.value, sb, n, sd.value, zd.value)
    deq = (D.astype(np.float64) - zd.value) * sd.value
    assert np.abs(deq - ref).max() <= 1.0
    cos = (deq * ref).sum() / (np.linalg.norm(deq) * np.linalg.norm(ref))
    assert cos >= 0.999


def test_w4a8_closed_form():
    """Integer part by numpy int64 products; f32 epilogue by numpy float32 single ops in the
    reference's order; and within 1e-5 relative of a float64 evaluation."""
    d = T.gen_w4a8(9, 70, 256, seed=6, with_c=True, with_bias=True)
    D = T.oracle_w4a8(d["A"], d["Bp"], d["C"], d["bias"], -np.inf, np.inf, d["scale_a"],
                      d["zp_a"], d["scale_b"])
    q = np.empty((70, 256), np.int64)
    q[:, 0::2] = (d["Bp"] & 15).astype(np.int64) - 8
    q[:, 1::2] = (d["Bp"] >> 4).astype(np.int64) - 8
    a = d["A"].astype(np.int64)
    acc = (a - d["zp_a"][:, None]) @ q.T  # sum (a - zp) * b == sum a*b - zp * sum b
    f = acc.astype(np.float32)
    f = (f * d["scale_a"][:, None]).astype(np.float32)
    f = (f * d["scale_b"][None, :]).astype(np.float32)
    f = (f + d["C"]).astype(np.float32)
    f = (f + d["bias"][None, :]).astype(np.float32)
    np.testing.assert_array_equal(D.view(np.uint32), f.view(np.uint32))
    exact = (acc.astype(np.float64) * d["scale_a"][:, None] * d["scale_b"][None, :] + d["C"] +
             d["bias"][None, :])
    assert np.allclose(D, exact, rtol=1e-5, atol=1e-6)


def test_w4a8_nibble_order_matters():
    """Swapping the nibble order (odd k in the low nibble) changes the result: the even-k-low
    convention of the reference (tqt_kernel_gemm_i8_i4_4x1vl_rvv.h:77-93) is what is pinned."""
    d = T.gen_w4a8(3, 20, 64, seed=1, with_bias=False)
    D = T.oracle_w4a8(d["A"], d["Bp"], None, None, -np.inf, np.inf, d["scale_a"], d["zp_a"],
                      d["scale_b"])
    swapped = ((d["Bp"] >> 4) | (d["Bp"] << 4)).astype(np.uint8)
    D2 = T.oracle_w4a8(d["A"], swapped, None, None, -np.inf, np.inf, d["scale_a"], d["zp_a"],
                       d["scale_b"])
    assert not np.array_equal(D, D2)


# ------------------------------------------------------------------------------------------
# Convolution restatement
# ------------------------------------------------------------------------------------------

def test_im2col_vs_reference_golden():
    g = golden("ref_im2col.npz")
    o = T.oracle()
    for i, (ic, oc, ih, iw, kh, kw, sh, sw, ph, pw, dh, dw) in enumerate(g["shapes"]):
        conv = T.make_conv((1, ih, iw), (1, kh, kw), (1, sh, sw), (1, dh, dw), (0, ph, pw), ic, oc)
        inp = g["im2col_%d_in" % i]
        col = np.zeros_like(g["im2col_%d_col" % i])
        o.tqto_im2col_cl_i8(0, T.ptr(inp), T.ptr(col), ctypes.byref(conv))
        np.testing.assert_array_equal(col, g["im2col_%d_col" % i])


def test_igemmcl_equals_im2col_then_gemm():
    """igemmcl == convcl: explicit im2col (reference tqt_im2col_cl, golden) followed by the
    W8A8 GEMM (src/conv/conv_i8_i8/convcl…qsi8cxt…cpp:76-91)."""
    g = golden("ref_im2col.npz")
    for i, (ic, oc, ih, iw, kh, kw, sh, sw, ph, pw, dh, dw) in enumerate(g["shapes"]):
        d = T.gen_igemmcl(1, ih, iw, ic, oc, kh, kw, stride=(sh, sw), pad=(ph, pw),
                          dil=(dh, dw), seed=i)
        inp = g["im2col_%d_in" % i].reshape(1, ih, iw, ic)
        col = g["im2col_%d_col" % i]
        D = T.oracle_igemmcl(inp, d["W"], d["bias"], -128, 127, d["conv"], d["scale_a"],
                             d["scale_b"], oc, d["scale_d"], d["zp_d"])
        G = T.oracle_w8a8(col, d["W"], None, d["bias"], -128, 127, d["scale_a"], d["scale_b"], oc,
                          d["scale_d"], d["zp_d"])
        np.testing.assert_array_equal(D, G)


def test_igemmcl_tiles_and_batch_depth():
    """Per-tile calls with m_idx reproduce one full call; a batch folded into depth equals
    separate per-image convolutions."""
    d = T.gen_igemmcl(3, 7, 9, 16, 24, 3, 3, pad=(1, 1), seed=12)
    full = T.oracle_igemmcl(d["inp"], d["W"], d["bias"], -128, 127, d["conv"], d["scale_a"],
                            d["scale_b"], 24, d["scale_d"], d["zp_d"])
    M = full.shape[0]
    D = np.zeros_like(full)
    for m_idx in range(0, M, 4):
        T.oracle_igemmcl(d["inp"], d["W"], d["bias"], -128, 127, d["conv"], d["scale_a"],
                         d["scale_b"], 24, d["scale_d"], d["zp_d"], m=min(4, M - m_idx),
                         m_idx=m_idx, D=D)
    np.testing.assert_array_equal(D, full)
    per = 7 * 9
    for img in range(3):
        single = T.make_conv((1, 7, 9), (1, 3, 3), (1, 1, 1), (1, 1, 1), (0, 1, 1), 16, 24)
        one = T.oracle_igemmcl(np.ascontiguousarray(d["inp"][img:img + 1]), d["W"], d["bias"],
                               -128, 127, single, d["scale_a"], d["scale_b"], 24, d["scale_d"],
                               d["zp_d"])
        np.testing.assert_array_equal(one, full[img * per:(img + 1) * per])


def test_igemmcl_float_sanity_like_reference_test():
    """Reference conv test acceptance (test/common/quantized_igemm_test_runner.h:359-469):
    dequantized output within 1.0 absolute / cosine 0.999 of reference_conv<float>."""
    r = T.ref()
    if r is None:
        pytest.skip("reference test code not built here")
    o = T.oracle()
    ic, oc, ih, iw = 16, 32, 8, 8
    conv = T.make_conv((1, ih, iw), (1, 3, 3), (1, 1, 1), (1, 1, 1), (0, 1, 1), ic, oc)
    K = 9 * ic
    act = np.zeros((ih * iw, ic), np.float32)
    r.tqtr_fill_uniform_f32(-1.0, 1.0, 42, T.ptr(act), ih * iw, ic)
    w = np.zeros((oc, K), np.float32)
    r.tqtr_fill_uniform_f32(-1.0, 1.0, 43, T.ptr(w), oc, K)
    bf = np.zeros(oc, np.float32)
    r.tqtr_fill_uniform_f32(-10.0, 10.0, 123, T.ptr(bf), 1, oc)
    M = conv.output_shape[1] * conv.output_shape[2]
    ref = np.zeros((M, oc), np.float32)
    r.tqtr_reference_conv_cl_f32(0, T.ptr(act), T.ptr(w), T.ptr(bf), T.ptr(ref),
                                 ctypes.byref(conv), -3.4e38, 3.4e38)
    sa, za = ctypes.c_float(), ctypes.c_int32()
    o.tqto_compute_asym_quant_params_i8(T.ptr(act), act.size, ctypes.byref(sa), ctypes.byref(za))
    sb = np.zeros(oc, np.float32)
    for ch in range(oc):
        s = ctypes.c_float()
        o.tqto_compute_sym_quant_params_i8(T.ptr(w[ch]), K, ctypes.byref(s))
        sb[ch] = s.value
    A = np.array([[o.tqto_quantize_i8(float(v), sa.value, za.value) for v in row] for row in act],
                 np.int8).reshape(1, ih, iw, ic)
    W = np.array([[o.tqto_quantize_i8(float(v), float(sb[ch]), 0) for v in w[ch]]
                  for ch in range(oc)], np.int8)
    bias = np.array([o.tqto_quantize_bias_i32(float(bf[ch]), sa.value * float(sb[ch]))
                     for ch in range(oc)], np.int32)
    fused = np.zeros(oc, np.int32)
    o.tqto_fuse_zp_to_bias(T.ptr(fused), T.ptr(bias), T.ptr(W), za.value, oc, K)
    sd, zd = ctypes.c_float(), ctypes.c_int32()
    o.tqto_compute_asym_quant_params_i8(T.ptr(ref), ref.size, ctypes.byref(sd), ctypes.byref(zd))
    D = T.oracle_igemmcl(A, W, fused, -128, 127, conv, sa.value, sb, oc, sd.value, zd.value)
    deq = (D.astype(np.float64) - zd.value) * sd.value
    # the reference pads with int8 0, not zero_point_a, while the bias fusion covers all of K:
    # border pixels carry a bias the fp32 reference does not have, as in the reference test
    assert np.abs(deq - ref).max() <= 1.0 + 2 * abs(za.value) * sa.value * float(sb.max()) * K
    cos = (deq * ref).sum() / (np.linalg.norm(deq) * np.linalg.norm(ref))
    assert cos >= 0.99


# ------------------------------------------------------------------------------------------
# Harness quantization helpers vs the reference's own code
# ------------------------------------------------------------------------------------------

def test_quant_helpers_vs_reference_golden():
    g = golden("ref_quant.npz")
    o = T.oracle()
    q8 = np.array([o.tqto_quantize_i8(float(v), float(s), int(z))
                   for v, s, z in zip(g["vals"], g["scales"], g["zps"])], np.int8)
    np.testing.assert_array_equal(q8, g["q8"])
    qb = np.array([o.tqto_quantize_bias_i32(float(v) * 100, float(s) * 1e-3)
                   for v, s in zip(g["vals"], g["scales"])], np.int32)
    np.testing.assert_array_equal(qb, g["qb"])
    fused = np.zeros(37, np.int32)
    o.tqto_fuse_zp_to_bias(T.ptr(fused), T.ptr(g["bias"]), T.ptr(g["Bf"]), -7, 37, 53)
    np.testing.assert_array_equal(fused, g["fused"])
    i4 = np.zeros((9, 32), np.uint8)
    i4s = np.zeros((9, 4), np.uint16)
    o.tqto_quantize_fp16_to_int4(9, 64, 16, T.ptr(g["src"]), T.ptr(i4), T.ptr(i4s), 4)
    np.testing.assert_array_equal(i4, g["i4"])
    np.testing.assert_array_equal(i4s, g["i4s"])


def test_live_reference_matches_golden():
    """Where the reference test code is built (the build container), recompute one golden
    vector live, so the fixtures cannot drift from the code that wrote them."""
    r = T.ref()
    if r is None:
        pytest.skip("reference test code not built here")
    g = golden("ref_clamp_i32.npz")
    m, n, k, _ = g["shapes"][5]
    A, B = g["clamp_5_A"], g["clamp_5_B"]
    D = np.zeros((m, n), np.int32)
    r.tqtr_reference_gemm_i32_i8(int(m), int(n), int(k), T.ptr(A), int(k), T.ptr(B), int(n), 0,
                                 None, int(n), T.ptr(D), int(n), -100000, 100000)
    np.testing.assert_array_equal(D, g["clamp_5_D"])


# ------------------------------------------------------------------------------------------
# Per-row asymmetric activation quantization (qai8dx; test/gemm/test_gemm_i8_i4_rvv.cpp:40-77)
# ------------------------------------------------------------------------------------------

def oracle_per_row(X):
    X = np.ascontiguousarray(X, np.float32)
    m, k = X.shape
    q = np.zeros((m, k), np.int8)
    s = np.zeros(m, np.float32)
    z = np.zeros(m, np.int32)
    T.oracle().tqto_quantize_a_per_row_asym(T.ptr(X), m, k, T.ptr(q), T.ptr(s), T.ptr(z))
    return q, s, z


def per_row_violations(X, q, s, z):
    """Properties that asymmetric per-row int8 quantization over [min(x, 0), max(x, 0)] must
    have, independent of how it is computed. Returns a list of violated properties (empty when
    all hold). Every element is checked against the golden-pinned quantize_i8 too."""
    bad = []
    o = T.oracle()
    for r in range(X.shape[0]):
        x = X[r].astype(np.float64)
        lo, hi = min(x.min(), 0.0), max(x.max(), 0.0)
        sr, zr, qr = float(s[r]), int(z[r]), q[r].astype(np.int64)
        if lo == hi == 0.0:
            if not (sr == 1.0 and zr == 0 and not qr.any()):
                bad.append("zero row")
            continue
        # the scale spreads [lo, hi] over the 255 steps of int8
        if abs(sr * 255.0 - (hi - lo)) > 4e-7 * (hi - lo) + 255 * 2.0 ** -149:
            bad.append("scale")
        if not -128 <= zr <= 127:
            bad.append("zero point range")
        if lo == 0.0 and zr != -128:
            bad.append("one-signed row (>= 0) zero point")
        if hi == 0.0 and zr != 127:
            bad.append("one-signed row (<= 0) zero point")
        # real zero is representable: x = 0 quantizes to the zero point
        if int(o.tqto_quantize_i8(0.0, sr, zr)) != zr:
            bad.append("zero not exact")
        # the row's extremes land on the ends of the int8 range (a negative minimum on -128, a
        # positive maximum on 127), unless x / s sits within 1e-3 of a rounding tie or the
        # scale is subnormal (then s no longer carries 24 bits, and 255 s != hi - lo)
        def near_tie(v):
            if sr < 2.0 ** -126:
                return True
            u = abs(float(np.float32(v) / np.float32(sr)))
            return abs(u - np.floor(u) - 0.5) < 1e-3

        if x.min() < 0 and not near_tie(x.min()) and qr[np.argmin(x)] != -128:
            bad.append("minimum not on -128")
        if x.max() > 0 and not near_tie(x.max()) and qr[np.argmax(x)] != 127:
            bad.append("maximum not on 127")
        # round to nearest: dequantized values lie within half a step, unless saturated
        deq = (qr - zr) * sr
        inner = (qr > -128) & (qr < 127)
        if np.any(np.abs(deq - x)[inner] > 0.5 * sr * (1 + 1e-5)):
            bad.append("rounding")
        if np.any(x[qr == -128] > (-128 - zr + 0.5) * sr * (1 + 1e-5) + 1e-30):
            bad.append("low saturation")
        if np.any(x[qr == 127] < (127 - zr - 0.5) * sr * (1 - 1e-5) - 1e-30):
            bad.append("high saturation")
        # monotone in x
        order = np.argsort(x, kind="stable")
        if np.any(np.diff(qr[order]) < 0):
            bad.append("monotone")
        # each element is the golden-pinned quantize_i8 step with this row's parameters
        if any(int(o.tqto_quantize_i8(float(v), sr, zr)) != int(w) for v, w in
               zip(X[r][:64], q[r][:64])):
            bad.append("quantize_i8 step")
    return bad


def test_per_row_quantize_known_answers():
    """Hand-worked rows whose range is 255 (or 510) in binary-exact values, so the scale is
    exactly 1 (or 2) and each zero point and value follows from nearbyint (half to even) alone:
      [-100.75, 154.25]: zp = nearbyint(-128 + 100.75 = -27.25) = -27 (floor would give -28);
      [-100.25, 154.75]: zp = nearbyint(-27.75) = -28 (truncation would give -27);
      [-100.5, 154.5]:   zp = nearbyint(-27.5) = -28 and 154.5 -> 154 (half to even);
      s = 2, [-201.5, 308.5]: zp = nearbyint(-128 + 100.75) = -27."""
    X = np.array([
        [-100.75, 0.0, 154.25, 10.5, 11.5, -3.5],
        [-100.25, 0.0, 154.75, 10.5, 11.5, -3.5],
        [-100.5, 0.0, 154.5, 10.5, 11.5, -3.5],
        [-201.5, 0.0, 308.5, 21.0, 23.0, -7.0],
    ], np.float32)
    q, s, z = oracle_per_row(X)
    np.testing.assert_array_equal(s, [1.0, 1.0, 1.0, 2.0])
    np.testing.assert_array_equal(z, [-27, -28, -28, -27])
    # value = nearbyint(x / s) + zp, saturated: -100.75 -> -101 - 27 = -128; 154.25 -> 127;
    # 10.5 -> 10 (even); 11.5 -> 12; -3.5 -> -4
    np.testing.assert_array_equal(q, [
        [-128, -27, 127, -17, -15, -31],
        [-128, -28, 127, -18, -16, -32],
        [-128, -28, 126, -18, -16, -32],
        [-128, -27, 127, -17, -15, -31],
    ])


def test_per_row_quantize_special_rows():
    X = np.array([
        [0.0] * 8,                                   # all zero -> (1.0, 0, zeros)
        [0.5, 1.0, 2.0, 0.25, 3.0, 0.125, 1.5, 0.0],  # all >= 0 -> zp -128
        [-0.5, -1.0, -2.0, -0.25, -3.0, 0.0, -1.5, -0.125],  # all <= 0 -> zp 127
        [7.0] * 8,                                   # constant positive: every value 127
        [-7.0] * 8,                                  # constant negative: every value -128
        [1e-40, -1e-40, 0, 0, 0, 0, 0, 1e-40],       # subnormal range
    ], np.float32)
    q, s, z = oracle_per_row(X)
    assert (s[0], z[0]) == (1.0, 0) and not q[0].any()
    assert z[1] == -128 and z[2] == 127
    assert (q[3] == 127).all() and z[3] == -128
    assert (q[4] == -128).all() and z[4] == 127
    assert per_row_violations(X, q, s, z) == []


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_per_row_quantize_properties(seed):
    rng = np.random.default_rng(seed)
    X = np.concatenate([
        rng.standard_normal((6, 512)),
        rng.standard_normal((2, 512)) * 1e-3 + 0.5,       # one-signed, narrow
        rng.uniform(-5, 1, (2, 512)),                      # skewed
        rng.standard_normal((2, 512)) * 1e4,
    ]).astype(np.float32)
    q, s, z = oracle_per_row(X)
    assert per_row_violations(X, q, s, z) == []


def test_per_row_quantize_properties_reject_planted_mistakes():
    """The property checker has teeth: quantizers with one step changed (restated in numpy on
    the CPU) each violate a property on ordinary rows."""
    rng = np.random.default_rng(7)
    X = rng.standard_normal((6, 256)).astype(np.float32)

    def quantizer(scale_div=255.0, zp_off=-128.0, round_zp=np.rint, clip=True):
        lo = np.minimum(X.min(axis=1), 0).astype(np.float32)
        hi = np.maximum(X.max(axis=1), 0).astype(np.float32)
        s = ((hi - lo) / np.float32(scale_div)).astype(np.float32)
        z = round_zp(np.float32(zp_off) - lo / s).astype(np.int64)
        if clip:
            z = np.clip(z, -128, 127)
        q = np.clip(np.rint(X / s[:, None]) + z[:, None], -128, 127).astype(np.int8)
        return q, s, z.astype(np.int32)

    assert per_row_violations(X, *quantizer()) == []          # the unplanted form passes
    for plant in (dict(scale_div=256.0), dict(zp_off=-127.0), dict(zp_off=0.0),
                  dict(round_zp=np.floor)):
        assert per_row_violations(X, *quantizer(**plant)), plant


# ------------------------------------------------------------------------------------------
# Tensor-wide quantization parameters of the reference runner
# (test/common/quantized_gemm_test_runner.h:37-63 asymmetric, :67-86 symmetric)
# ------------------------------------------------------------------------------------------

def oracle_asym_params(x):
    x = np.ascontiguousarray(x, np.float32)
    s, z = ctypes.c_float(), ctypes.c_int32()
    T.oracle().tqto_compute_asym_quant_params_i8(T.ptr(x), x.size, ctypes.byref(s),
                                                 ctypes.byref(z))
    return s.value, z.value


def oracle_sym_param(x):
    x = np.ascontiguousarray(x, np.float32)
    s = ctypes.c_float()
    T.oracle().tqto_compute_sym_quant_params_i8(T.ptr(x), x.size, ctypes.byref(s))
    return s.value


# Hand-worked inputs whose range is a binary-exact multiple of 255, so the scale is exact and
# the zero point follows from nearbyint (half to even) and the -128 -> -127 rule alone.
ASYM_KNOWN = [
    ([0.0] * 5, 1.0, 0),                  # all zero: (1, 0)
    ([-100.75, 3.0, 154.25], 1.0, -27),   # nearbyint(-27.25) = -27 (floor: -28)
    ([-100.25, 154.75], 1.0, -28),        # nearbyint(-27.75) = -28 (truncation: -27)
    ([-127.5, 127.5], 1.0, 0),            # nearbyint(-0.5) = -0 (half away from zero: -1)
    ([-1.5, 253.5], 1.0, -126),           # nearbyint(-126.5) = -126 (half away: -127)
    ([0.0, 17.0, 255.0], 1.0, -127),      # zp -128 becomes -127
    ([2.0, 510.0], 2.0, -127),            # all >= 0: the minimum clamps to 0, then -128 -> -127
    ([-510.0, -2.0], 2.0, 127),           # all <= 0: the maximum clamps to 0; -128 + 255
    ([-63.75, 63.75], 0.5, 0),            # s = 127.5 / 255 = 0.5
    ([-0.5, 63.25], 0.25, -126),          # s = 63.75 / 255 = 0.25; nearbyint(-128 + 2)
]
# Symmetric: s = 2 max|x| / 255 (1 for all zeros), whichever of the extremes is larger.
SYM_KNOWN = [
    ([0.0, 0.0, 0.0], 1.0),
    ([-127.5, 3.0], 1.0),
    ([1.0, 2.0, -255.0], 2.0),            # |min| > |max|
    ([255.0, -1.0], 2.0),                 # |max| > |min|
    ([-63.75, 63.75], 0.5),               # tie
    ([0.5, 25.5], float(np.float32(51.0) / np.float32(255.0))),     # positives only
    ([-25.5, -0.5], float(np.float32(51.0) / np.float32(255.0))),   # negatives only
]


def asym_known_failures(fn):
    return [x for x, s, z in ASYM_KNOWN if fn(np.array(x, np.float32)) != (s, z)]


def sym_known_failures(fn):
    return [x for x, s in SYM_KNOWN if fn(np.array(x, np.float32)) != s]


def test_asym_quant_params_known_answers():
    assert asym_known_failures(oracle_asym_params) == []


def test_sym_quant_params_known_answers():
    assert sym_known_failures(oracle_sym_param) == []


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_quant_params_properties(seed):
    """On random tensors: 255 s spans [min(x, 0), max(x, 0)] to f32 rounding, the zero point is
    within half a step of -128 - min / s (or is the -127 that replaces -128) and maps real 0
    exactly (golden-pinned quantize_i8); the symmetric scale covers max|x| with 127.5 steps."""
    rng = np.random.default_rng(seed)
    o = T.oracle()
    for x in (rng.standard_normal(4096), rng.uniform(-3, 9, 1000), rng.uniform(0.5, 2, 300),
              -rng.uniform(0.5, 2, 300), rng.standard_normal(77) * 1e5):
        x = x.astype(np.float32)
        lo, hi = min(float(x.min()), 0.0), max(float(x.max()), 0.0)
        s, z = oracle_asym_params(x)
        assert abs(255.0 * s - (hi - lo)) <= 4e-7 * (hi - lo)
        assert -127 <= z <= 127
        exact = -128.0 - lo / s
        assert abs(z - exact) <= 0.5 + 1e-6 or (z == -127 and abs(-128 - exact) <= 0.5 + 1e-6)
        assert int(o.tqto_quantize_i8(0.0, s, z)) == z
        amax = float(np.abs(x).max())
        ss = oracle_sym_param(x)
        assert abs(127.5 * ss - amax) <= 4e-7 * amax


def test_quant_params_known_answers_reject_planted_mistakes():
    """The known answers have teeth: restatements with one step changed (numpy, f32) each miss
    at least one of them, while the unplanted restatement meets all."""
    f32 = np.float32

    def asym(x, div=255.0, rnd=np.rint, rule=True, off=-128.0):
        lo, hi = min(f32(x.min()), f32(0)), max(f32(x.max()), f32(0))
        s = f32(f32(hi - lo) / f32(div))
        if s == 0:
            return 1.0, 0
        z = int(rnd(f32(f32(off) - f32(lo / s))))
        if rule and z == -128:
            z = -127
        return float(s), z

    def sym(x, div=255.0, mode="both"):
        a = {"both": max(abs(f32(x.max())), abs(f32(x.min()))), "max": abs(f32(x.max())),
             "min": abs(f32(x.min()))}[mode]
        s = f32(f32(2.0) * f32(a) / f32(div))
        return float(s) if s != 0 else 1.0

    assert asym_known_failures(asym) == []
    for plant in (dict(div=256.0), dict(rnd=np.floor), dict(rnd=np.trunc), dict(rule=False),
                  dict(off=-127.0), dict(rnd=lambda v: np.sign(v) * np.floor(abs(v) + 0.5))):
        assert asym_known_failures(lambda x: asym(x, **plant)), plant
    assert sym_known_failures(sym) == []
    for plant in (dict(div=254.0), dict(mode="max"), dict(mode="min")):
        assert sym_known_failures(lambda x: sym(x, **plant)), plant
