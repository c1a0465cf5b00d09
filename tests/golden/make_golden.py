#!/usr/bin/env python3
"""Write the golden fixtures under tests/golden/ (run in the build container, where the
reference tree exists and `make -C oracle` has built oracle/_ref/libtqt_ref.so).

Every vector whose expected output the reference's own code can compute comes from that code:
inputs from the reference's UniformRandomGenerator (std::mt19937, test/common/data_generator.*)
with the seeds its tests use, outputs from its portable test oracles
(test/common/reference_gemm.cpp, src/common/tqt_conv.h tqt_im2col_cl,
src/gemm/gemm_i8_i8/tqt_utils_i8_i8.h tqt_quantize_multiplier, test/common/quantize_utils.h,
test/common/test_common.h). Those files are compiled from where they lie into
oracle/_ref/libtqt_ref.so by oracle/Makefile; nothing of them is copied here.

Fixtures (numpy .npz, no pickles):
  ref_clamp_i32.npz    reference_gemm_i32_i8 on the reference's int8 shape list
  ref_w4a16.npz        reference_gemm_quantized_weight_mixed<f16,f16> on its W4A16 shape list
  ref_w4a16_f32.npz    reference_gemm_quantized_weight_mixed<f16,float> on the same list
  ref_w8a8dyn.npz      the qai8dx x qsi8cx runner's inputs on the reference's int8 shape list
                       (A, B from its generator; per-row / per-channel quantization restated
                       below, quantize_i8 from the reference) with reference_gemm<float,float>
                       of the unquantized f32 operands, the value its test compares against
  ref_im2col.npz       tqt_im2col_cl<int8_t> on the reference's igemm shape list
  ref_im2col_cf.npz    tqt_im2col_cf<int8_t> (channel-first) on the same list, with groups
  ref_qm.npz           tqt_quantize_multiplier on edge and random doubles
  ref_quant.npz        quantize_i8 / quantize_bias_i32 / fuse_zp_to_bias / quantize_fp16_to_int4
"""

import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import tqt_testlib as T  # noqa: E402

INT8_SHAPES = [(32, 32, 32, 0), (3, 8, 11, 0), (5, 11, 10, 0), (9, 19, 23, 0), (15, 32, 25, 0),
               (60, 63, 127, 0), (32, 32, 32, 1), (60, 63, 127, 1)]
W4A16_SHAPES = [(8, 8, 4, 2, 0, 0, 0), (16, 16, 8, 2, 0, 0, 0), (32, 32, 32, 2, 0, 0, 0),
                (32, 32, 32, 4, 0, 0, 0), (32, 32, 32, 32, 0, 0, 0), (5, 11, 10, 2, 0, 0, 0),
                (7, 3, 10, 2, 0, 0, 0), (17, 19, 24, 4, 0, 0, 0), (31, 35, 64, 32, 0, 0, 0),
                (60, 61, 128, 32, 0, 0, 0), (32, 32, 32, 2, 1, 0, 0), (17, 19, 24, 4, 1, 0, 0),
                (32, 32, 32, 4, 0, 0, 1), (32, 32, 32, 4, 0, 1, 0), (32, 32, 32, 4, 1, 1, 1)]
CONV_SHAPES = [  # IC, OC, IH, IW, KH, KW, SH, SW, PH, PW, DH, DW
    (3, 16, 8, 8, 3, 3, 1, 1, 0, 0, 1, 1), (16, 32, 8, 8, 3, 3, 1, 1, 0, 0, 1, 1),
    (16, 32, 8, 8, 1, 1, 1, 1, 0, 0, 1, 1), (3, 16, 8, 8, 3, 3, 1, 1, 1, 1, 1, 1),
    (3, 16, 8, 8, 3, 3, 2, 2, 0, 0, 1, 1), (3, 16, 8, 8, 3, 3, 1, 1, 2, 2, 2, 2),
    (3, 16, 8, 8, 3, 3, 2, 2, 1, 1, 1, 1), (8, 16, 7, 11, 3, 5, 1, 1, 0, 0, 1, 1),
    (64, 128, 4, 4, 1, 1, 1, 1, 0, 0, 1, 1), (3, 32, 16, 16, 3, 3, 1, 1, 1, 1, 1, 1),
    (3, 8, 6, 6, 3, 3, 1, 1, 0, 0, 1, 1), (64, 32, 4, 4, 3, 3, 1, 1, 1, 1, 1, 1)]


def asym_quant_params_i8(x):
    """test/common/quantized_gemm_test_runner.h:37-67 compute_asym_quant_params_i8 (float32
    arithmetic; that header needs gtest, so it cannot be compiled here)."""
    f32 = np.float32
    fmax = max(f32(x.max()), f32(0.0))
    fmin = min(f32(x.min()), f32(0.0))
    scale = f32(f32(fmax - fmin) / f32(255.0))
    if scale == 0:
        return f32(1.0), 0
    zp = int(np.rint(f32(f32(-128.0) - f32(fmin / scale))))
    if zp == -128:
        zp = -127
    return scale, zp


def sym_quant_params_i8(x):
    """test/common/quantized_gemm_test_runner.h:69-85 compute_sym_quant_params_i8."""
    f32 = np.float32
    fmax, fmin = f32(x.max()), f32(x.min())
    amax = abs(fmax) if abs(fmax) >= abs(fmin) else abs(fmin)
    scale = f32(f32(f32(2.0) * amax) / f32(255.0))
    return f32(1.0) if scale == 0 else scale


def main():
    r = T.ref()
    if r is None:
        sys.exit("oracle/_ref/libtqt_ref.so is not built (needs the reference tree)")
    p = T.ptr
    out = {}

    # --- int8 -> int32 GEMM (test/common/quantized_gemm_test_runner.h:122-181) ---
    for i, (m, n, k, with_c) in enumerate(INT8_SHAPES):
        # the reference fills A then B from one generator object: reproduce by drawing
        # m*k + k*n values in one call and splitting
        AB = np.zeros(m * k + k * n, np.int8)
        r.tqtr_fill_uniform_i8(-50, 50, 42, p(AB), 1, AB.size)
        A = AB[:m * k].reshape(m, k).copy()
        B = AB[m * k:].reshape(k, n).copy()
        C = None
        if with_c:
            C = np.zeros((m, n), np.int32)
            r.tqtr_fill_uniform_i32(-1000, 1000, 42, p(C), m, n)
        D = np.zeros((m, n), np.int32)
        r.tqtr_reference_gemm_i32_i8(m, n, k, p(A), k, p(B), n, 0, p(C), n, p(D), n, -100000,
                                     100000)
        out["clamp_%d_A" % i] = A
        out["clamp_%d_B" % i] = B
        if C is not None:
            out["clamp_%d_C" % i] = C
        out["clamp_%d_D" % i] = D
    np.savez_compressed(os.path.join(HERE, "ref_clamp_i32.npz"),
                        shapes=np.array(INT8_SHAPES, np.int64), **out)

    # --- W4A16 (test/common/quantized_gemm_test_runner.h:1038-1112) ---
    out = {}
    for i, (m, n, k, bl, bias, c, clamp) in enumerate(W4A16_SHAPES):
        A = np.zeros((m, k), np.uint16)
        r.tqtr_fill_uniform_f16(-1.0, 1.0, 42, p(A), m, k)
        Bsrc = np.zeros((n, k), np.uint16)
        r.tqtr_fill_uniform_f16(-1.0, 1.0, 123, p(Bsrc), n, k)
        Bp = np.zeros((n, k // 2), np.uint8)
        S = np.zeros((n, k // bl), np.uint16)
        r.tqtr_quantize_fp16_to_int4(n, k, bl, p(Bsrc), p(Bp), p(S), k // bl)
        C = None
        if c:
            C = np.zeros((m, n), np.uint16)
            r.tqtr_fill_uniform_f16(-5.0, 5.0, 42, p(C), m, n)
        bvec = None
        if bias:
            bvec = np.zeros(n, np.uint16)
            r.tqtr_fill_uniform_f16(-0.5, 0.5, 7, p(bvec), 1, n)
        lo, hi = (-0.5, 0.5) if clamp else (-65504.0, 65504.0)
        cmin, cmax = int(T.f16_bits(lo)), int(T.f16_bits(hi))
        D = np.zeros((m, n), np.uint16)
        r.tqtr_reference_gemm_qw_mixed_f16(m, n, k, bl, p(A), k, p(Bp), k, p(S), k // bl, p(C), n,
                                           p(D), n, p(bvec), cmin, cmax)
        out["w4a16_%d_A" % i] = A
        out["w4a16_%d_Bsrc" % i] = Bsrc
        out["w4a16_%d_Bp" % i] = Bp
        out["w4a16_%d_S" % i] = S
        if C is not None:
            out["w4a16_%d_C" % i] = C
        if bvec is not None:
            out["w4a16_%d_bias" % i] = bvec
        out["w4a16_%d_clamp" % i] = np.array([cmin, cmax], np.uint16)
        out["w4a16_%d_D" % i] = D
    np.savez_compressed(os.path.join(HERE, "ref_w4a16.npz"),
                        shapes=np.array(W4A16_SHAPES, np.int64), **out)

    # --- W8A8 with dynamic A quantization, f32 / f16 D
    # (test/common/quantized_gemm_test_runner.h:1325-1425) ---
    out = {}
    for i, (m, n, k, _c) in enumerate(INT8_SHAPES):
        AB = np.zeros(m * k + n * k, np.float32)
        r.tqtr_fill_uniform_f32(-1.0, 1.0, 42, p(AB), 1, AB.size)
        Af = AB[:m * k].reshape(m, k).copy()
        Bf = AB[m * k:].reshape(n, k).copy()
        bias = np.zeros(n, np.float32)
        r.tqtr_fill_uniform_f32(-10.0, 10.0, 123, p(bias), 1, n)
        sa = np.zeros(m, np.float32)
        za = np.zeros(m, np.int32)
        for row in range(m):
            sa[row], za[row] = asym_quant_params_i8(Af[row])
        sb = np.array([sym_quant_params_i8(Bf[ch]) for ch in range(n)], np.float32)
        Aq = np.array([[r.tqtr_quantize_i8(float(v), float(sa[row]), int(za[row]))
                        for v in Af[row]] for row in range(m)], np.int8)
        Bq = np.array([[r.tqtr_quantize_i8(float(v), float(sb[ch]), 0) for v in Bf[ch]]
                       for ch in range(n)], np.int8)
        D = np.zeros((m, n), np.float32)
        flt_max = float(np.finfo(np.float32).max)
        r.tqtr_reference_gemm_f32(m, n, k, p(Af), k, p(Bf), k, 1, None, n, p(D), n, p(bias),
                                  -flt_max, flt_max)
        for key, v in (("A", Aq), ("B", Bq), ("scale_a", sa), ("zp_a", za), ("scale_b", sb),
                       ("bias", bias), ("Dref", D)):
            out["w8a8dyn_%d_%s" % (i, key)] = v
    np.savez_compressed(os.path.join(HERE, "ref_w8a8dyn.npz"),
                        shapes=np.array(INT8_SHAPES, np.int64), **out)

    # --- W4A16 with f32 C / bias / clamp / D (the same runner with TD = float; its
    # UniformRandomGenerator<float> draws C and bias, the clamp defaults to +-FLT_MAX) ---
    out = {}
    flt_max = float(np.finfo(np.float32).max)
    for i, (m, n, k, bl, bias, c, clamp) in enumerate(W4A16_SHAPES):
        A = np.zeros((m, k), np.uint16)
        r.tqtr_fill_uniform_f16(-1.0, 1.0, 42, p(A), m, k)
        Bsrc = np.zeros((n, k), np.uint16)
        r.tqtr_fill_uniform_f16(-1.0, 1.0, 123, p(Bsrc), n, k)
        Bp = np.zeros((n, k // 2), np.uint8)
        S = np.zeros((n, k // bl), np.uint16)
        r.tqtr_quantize_fp16_to_int4(n, k, bl, p(Bsrc), p(Bp), p(S), k // bl)
        C = None
        if c:
            C = np.zeros((m, n), np.float32)
            r.tqtr_fill_uniform_f32(-5.0, 5.0, 42, p(C), m, n)
        bvec = None
        if bias:
            bvec = np.zeros(n, np.float32)
            r.tqtr_fill_uniform_f32(-0.5, 0.5, 7, p(bvec), 1, n)
        lo, hi = (-0.5, 0.5) if clamp else (-flt_max, flt_max)
        D = np.zeros((m, n), np.float32)
        r.tqtr_reference_gemm_qw_mixed_f16_f32(m, n, k, bl, p(A), k, p(Bp), k, p(S), k // bl,
                                               p(C), n, p(D), n, p(bvec), ctypes.c_float(lo),
                                               ctypes.c_float(hi))
        out["w4a16f_%d_A" % i] = A
        out["w4a16f_%d_Bp" % i] = Bp
        out["w4a16f_%d_S" % i] = S
        if C is not None:
            out["w4a16f_%d_C" % i] = C
        if bvec is not None:
            out["w4a16f_%d_bias" % i] = bvec
        out["w4a16f_%d_clamp" % i] = np.array([lo, hi], np.float32)
        out["w4a16f_%d_D" % i] = D
    np.savez_compressed(os.path.join(HERE, "ref_w4a16_f32.npz"),
                        shapes=np.array(W4A16_SHAPES, np.int64), **out)

    # --- implicit im2col order (src/common/tqt_conv.h:131-202) ---
    out = {}
    for i, (ic, oc, ih, iw, kh, kw, sh, sw, ph, pw, dh, dw) in enumerate(CONV_SHAPES):
        conv = T.make_conv((1, ih, iw), (1, kh, kw), (1, sh, sw), (1, dh, dw), (0, ph, pw), ic, oc)
        inp = np.zeros((ih * iw, ic), np.int8)
        r.tqtr_fill_uniform_i8(-128, 127, 42, p(inp), ih * iw, ic)
        M = conv.output_shape[1] * conv.output_shape[2]
        col = np.zeros((M, kh * kw * ic), np.int8)
        r.tqtr_im2col_cl_i8(0, p(inp), p(col), ctypes.byref(conv))
        out["im2col_%d_in" % i] = inp
        out["im2col_%d_col" % i] = col
    np.savez_compressed(os.path.join(HERE, "ref_im2col.npz"),
                        shapes=np.array(CONV_SHAPES, np.int64), **out)

    # --- channel-first im2col (src/common/tqt_conv.h:51-119), two groups where IC allows ---
    out = {}
    for i, (IC, OC, IH, IW, KH, KW, SH, SW, PH, PW, DH, DW) in enumerate(CONV_SHAPES):
        groups = 2 if IC % 2 == 0 else 1
        conv = T.make_conv((1, IH, IW), (1, KH, KW), (1, SH, SW), (1, DH, DW), (0, PH, PW), IC,
                           OC, groups)
        inp = np.zeros((IC, IH, IW), np.int8)
        r.tqtr_fill_uniform_i8(-128, 127, 42, p(inp), IC, IH * IW)
        out["cf_%d_input" % i] = inp
        out["cf_%d_groups" % i] = np.array([groups], np.int64)
        for g in range(groups):
            icg = IC // groups
            K = icg * KH * KW
            N = conv.output_shape[1] * conv.output_shape[2]
            col = np.zeros((K, N), np.int8)
            r.tqtr_im2col_cf_i8(g, p(inp), p(col), ctypes.byref(conv))
            out["cf_%d_col_g%d" % (i, g)] = col
    np.savez_compressed(os.path.join(HERE, "ref_im2col_cf.npz"),
                        shapes=np.array(CONV_SHAPES, np.int64), **out)

    # --- requantization multiplier (src/gemm/gemm_i8_i8/tqt_utils_i8_i8.h:98-132) ---
    rng = np.random.default_rng(1234)
    edge = [0.0, -0.0, 0.5, 0.25, 0.0004, 1.0, 2.0, 0.999999999, 1.0 - 2.0 ** -53,
            0.75 + 2.0 ** -40, 2.0 ** -31, 2.0 ** -32, 2.0 ** -33, 3e-10, 5e-324, 1e-310,
            -0.5, -0.3, 1e10, 123456.789, np.inf, -np.inf,
            (1.0 + 2.0 ** -31) * 0.5, (1.0 + 3 * 2.0 ** -32) * 0.5]
    # the harness's own products: scale_a * scale_b / scale_d at the configuration ranges
    sa = np.float32(0.02)
    sb = rng.uniform(0.001, 0.01, 4000).astype(np.float32)
    cfg = (np.float64(sa) * sb.astype(np.float64) / np.float64(np.float32(0.05))).tolist()
    rnd = (10.0 ** rng.uniform(-12, 3, 20000)).tolist()
    # values whose 22 dropped mantissa bits sit exactly at / around the rounding threshold
    ties = []
    for _ in range(2000):
        hi_bits = int(rng.integers(0, 1 << 30))
        e = int(rng.integers(1000, 1030))
        for low in (0x1fffff, 0x200000, 0x200001):
            u = (e << 52) | (hi_bits << 22) | low
            ties.append(np.frombuffer(np.uint64(u).tobytes(), np.float64)[0])
    xs = np.array(edge + cfg + rnd + ties, np.float64)
    mult = np.zeros(xs.size, np.int32)
    shift = np.zeros(xs.size, np.int32)
    for j, x in enumerate(xs):
        mm, ss = ctypes.c_int32(), ctypes.c_int32()
        r.tqtr_quantize_multiplier(float(x), ctypes.byref(mm), ctypes.byref(ss))
        mult[j], shift[j] = mm.value, ss.value
    np.savez_compressed(os.path.join(HERE, "ref_qm.npz"), x=xs, mult=mult, shift=shift)

    # --- caller-side quantization helpers (test/common/test_common.h, quantize_utils.h) ---
    vals = np.concatenate([rng.uniform(-3, 3, 3000), np.array([0.0, 1.27, -1.28, 2.55, 0.005,
                                                               -0.015, 1e-3, 12.7])]).astype(
        np.float32)
    scales = rng.uniform(0.005, 0.05, vals.size).astype(np.float32)
    zps = rng.integers(-20, 21, vals.size).astype(np.int32)
    q8 = np.array([r.tqtr_quantize_i8(float(v), float(s), int(z))
                   for v, s, z in zip(vals, scales, zps)], np.int8)
    qb = np.array([r.tqtr_quantize_bias_i32(float(v) * 100, float(s) * 1e-3)
                   for v, s in zip(vals, scales)], np.int32)
    Bf = rng.integers(-127, 128, size=(37, 53)).astype(np.int8)
    bias = rng.integers(-1000, 1001, size=37).astype(np.int32)
    fused = np.zeros(37, np.int32)
    r.tqtr_fuse_zp_to_bias(p(fused), p(bias), p(Bf), -7, 37, 53)
    src = np.zeros((9, 64), np.uint16)
    r.tqtr_fill_uniform_f16(-1.0, 1.0, 99, p(src), 9, 64)
    src[0, :8] = T.f16_bits([0, 0, 0, 0, 0, 0, 0, 0])  # an all-zero block (scale 0 path)
    i4 = np.zeros((9, 32), np.uint8)
    i4s = np.zeros((9, 4), np.uint16)
    r.tqtr_quantize_fp16_to_int4(9, 64, 16, p(src), p(i4), p(i4s), 4)
    np.savez_compressed(os.path.join(HERE, "ref_quant.npz"), vals=vals, scales=scales, zps=zps,
                        q8=q8, qb=qb, Bf=Bf, bias=bias, fused=fused, src=src, i4=i4, i4s=i4s)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
