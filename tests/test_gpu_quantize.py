"""GPU dynamic per-row activation quantization (tqt_run_quantize_qai8dx_f32_gfx950) against the
oracle's restatement of the reference harness step (test/gemm/test_gemm_i8_i4_rvv.cpp:40-77,
itself pinned to the reference's golden vectors in test_oracle.py): int8 values, scales and zero
points bit-exact, on random rows, the special rows the formula branches on, round-half-even
ties, unaligned and strided rows; the decode pipeline quantize -> W4A8 GEMV against the
oracle's pipeline; and the fused decode step
(tqt_run_quantize_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_gfx950: one launch at m = 1, k = 2048 or
4096, else the two launches) against the same oracle pipeline, outputs and side outputs bit-exact."""

import ctypes

import numpy as np
import pytest

import tqt_testlib as T

pytestmark = pytest.mark.gpu


def _g():
    import gpu_run

    return gpu_run


def oracle_quant(X):
    m, k = X.shape
    X = np.ascontiguousarray(X, np.float32)
    q = np.zeros((m, k), np.int8)
    sa = np.zeros(m, np.float32)
    za = np.zeros(m, np.int32)
    T.oracle().tqto_quantize_a_per_row_asym(T.ptr(X), m, k, T.ptr(q), T.ptr(sa), T.ptr(za))
    return q, sa, za


def gpu_quant(X, lda=None, ldq=None, a_offset=0):
    """Quantize rows of X on the GPU; the source rows sit `a_offset` floats into their buffer."""
    import torch

    m, k = X.shape
    lda = k if lda is None else lda
    ldq = k if ldq is None else ldq
    src = np.zeros(a_offset + m * lda, np.float32)
    for r in range(m):
        src[a_offset + r * lda:a_offset + r * lda + k] = X[r]
    dA = _g().dev(src)
    dQ = torch.full((max(m * ldq, 1),), 77, dtype=torch.int8, device="cuda:0")
    dS = torch.zeros(m, dtype=torch.float32, device="cuda:0")
    dZ = torch.zeros(m, dtype=torch.int32, device="cuda:0")
    _g().lib().quantize(m, k, dA.data_ptr() + 4 * a_offset, lda, dQ.data_ptr(), ldq,
                        dS.data_ptr(), dZ.data_ptr())
    q = dQ.cpu().numpy()[:m * ldq].reshape(m, ldq)
    if ldq > k:
        assert (q[:, k:] == 77).all()  # padding untouched
    return q[:, :k], dS.cpu().numpy(), dZ.cpu().numpy()


def check(X, **kw):
    q, s, z = gpu_quant(X, **kw)
    eq, es, ez = oracle_quant(X)
    np.testing.assert_array_equal(q, eq)
    np.testing.assert_array_equal(s.view(np.uint32), es.view(np.uint32))
    np.testing.assert_array_equal(z, ez)


# k <= 4096 keeps the row in registers between the two passes; 4094 and 4101 sit either side
@pytest.mark.parametrize("m,k", [(1, 4096), (4, 4096), (8, 4096), (37, 100), (3, 7), (2, 1),
                                 (5, 65536), (2, 4094), (3, 4101)])
def test_random_rows(gpu, m, k):
    rng = np.random.default_rng(m * 1000 + k)
    check(rng.standard_normal((m, k)).astype(np.float32) * np.float32(rng.uniform(0.01, 50)))


def test_special_rows(gpu):
    k = 300
    rng = np.random.default_rng(5)
    rows = [
        np.zeros(k),                                    # s == 0: scale 1, zp 0, q 0
        np.abs(rng.standard_normal(k)) + 0.5,           # all positive: fmin clamps to 0
        -np.abs(rng.standard_normal(k)) - 0.5,          # all negative: fmax clamps to 0
        rng.standard_normal(k) * 1e-38,                 # subnormal range
        rng.standard_normal(k) * 1e30,                  # huge magnitudes
        np.where(np.arange(k) % 2 == 0, -0.0, 0.0),     # signed zeros only
        np.full(k, 3.0),                                # constant row
    ]
    X = np.stack(rows).astype(np.float32)
    check(X)


def test_round_half_even_ties(gpu):
    # min 0, max 255 -> s = 1, zp = -128: x = n + 0.5 rounds to the even neighbour
    x = np.concatenate([[0.0, 255.0], np.arange(0, 254) + 0.5]).astype(np.float32)
    q, s, z = gpu_quant(x[None, :])
    assert s[0] == 1.0 and z[0] == -128
    exp = (np.rint(x) - 128).astype(np.int8)
    np.testing.assert_array_equal(q[0], exp)
    check(x[None, :])


@pytest.mark.parametrize("lda,ldq,a_offset", [(4100, 4096, 0), (4096, 4104, 1), (4097, 4099, 3)])
def test_strided_and_unaligned_rows(gpu, lda, ldq, a_offset):
    rng = np.random.default_rng(lda + ldq)
    X = rng.standard_normal((6, 4096)).astype(np.float32)
    q, s, z = gpu_quant(X, lda=lda, ldq=ldq, a_offset=a_offset)
    eq, es, ez = oracle_quant(X)
    np.testing.assert_array_equal(q, eq)
    np.testing.assert_array_equal(s.view(np.uint32), es.view(np.uint32))
    np.testing.assert_array_equal(z, ez)


@pytest.mark.parametrize("m", [1, 4])
def test_decode_pipeline_quantize_then_w4a8(gpu, m):
    """f32 activations -> GPU quantize -> GPU W4A8 GEMV, all on the device, equals the oracle's
    quantize followed by the oracle's W4A8 bit for bit (the BASELINE cfg 3 shape)."""
    import torch

    n, k = 11008, 4096
    rng = np.random.default_rng(m)
    Af = rng.standard_normal((m, k)).astype(np.float32)
    Bp = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    sb = rng.uniform(0.005, 0.02, size=n).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float32)
    dAf, dB, dsb, dbias = _g().dev(Af), _g().dev(Bp), _g().dev(sb), _g().dev(bias)
    dQ = torch.empty((m, k), dtype=torch.int8, device="cuda:0")
    dS = torch.empty(m, dtype=torch.float32, device="cuda:0")
    dZ = torch.empty(m, dtype=torch.int32, device="cuda:0")
    dD = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    L = _g().lib()
    s = torch.cuda.current_stream().cuda_stream
    L.quantize_async(m, k, dAf.data_ptr(), k, dQ.data_ptr(), k, dS.data_ptr(), dZ.data_ptr(), s)
    p = _g()._mod.QAI8DXQSI4CXParams(dS.data_ptr(), dZ.data_ptr(), dsb.data_ptr())
    L.fn("w4a8", "run_async")(m, n, k, dQ.data_ptr(), k, 0, dB.data_ptr(), k, 0, None, n,
                              dD.data_ptr(), n, dbias.data_ptr(), -np.inf, np.inf,
                              ctypes.byref(p), s)
    torch.cuda.synchronize()
    eq, es, ez = oracle_quant(Af)
    exp = T.oracle_w4a8(eq, Bp, None, bias, -np.inf, np.inf, es, ez, sb)
    np.testing.assert_array_equal(dD.cpu().numpy().view(np.uint32), exp.view(np.uint32))


def run_fused(Af, Bp, sb, bias=None, C=None, cmin=-np.inf, cmax=np.inf, a_offset=0, ldq=None):
    """The fused decode step on the GPU: (D, A_q, scale_a, zero_point_a)."""
    import torch

    m, k = Af.shape
    n = Bp.shape[0]
    ldq = k if ldq is None else ldq
    src = np.zeros(a_offset + m * k, np.float32)
    src[a_offset:] = Af.reshape(-1)
    dA = _g().dev(src)
    dB, dsb = _g().dev(Bp), _g().dev(sb)
    dbias, dC = _g().dev(bias), _g().dev(C)
    dQ = torch.full((m * ldq,), 77, dtype=torch.int8, device="cuda:0")
    dS = torch.full((m,), -1.0, dtype=torch.float32, device="cuda:0")
    dZ = torch.full((m,), 999, dtype=torch.int32, device="cuda:0")
    dD = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
    _g().lib().quantize_gemm(m, n, k, dA.data_ptr() + 4 * a_offset, k, dQ.data_ptr(), ldq,
                             dS.data_ptr(), dZ.data_ptr(), dB.data_ptr(), k, _g().dp(dC), n,
                             dD.data_ptr(), n, _g().dp(dbias), float(cmin), float(cmax),
                             dsb.data_ptr())
    q = dQ.cpu().numpy().reshape(m, ldq)
    if ldq > k:
        assert (q[:, k:] == 77).all()
    return dD.cpu().numpy(), q[:, :k], dS.cpu().numpy(), dZ.cpu().numpy()


def check_fused(Af, Bp, sb, bias=None, C=None, cmin=-np.inf, cmax=np.inf, **kw):
    D, q, s, z = run_fused(Af, Bp, sb, bias, C, cmin, cmax, **kw)
    eq, es, ez = oracle_quant(Af)
    np.testing.assert_array_equal(q, eq)
    np.testing.assert_array_equal(s.view(np.uint32), es.view(np.uint32))
    np.testing.assert_array_equal(z, ez)
    exp = T.oracle_w4a8(eq, Bp, C, bias, cmin, cmax, es, ez, sb)
    np.testing.assert_array_equal(D.view(np.uint32), exp.view(np.uint32))


def fused_inputs(m, n, k, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    Af = (rng.standard_normal((m, k)) * scale).astype(np.float32)
    Bp = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    sb = rng.uniform(0.005, 0.02, size=n).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float32)
    return Af, Bp, sb, bias


# (m, n, k, extra): m = 1 with k = 2048 / 4096 takes the one-launch kernel (n tails that leave
# a wave partly or wholly past n, C, clamps, a strided A_q); the rest the two launches
FUSED_CASES = [(1, 11008, 4096, {}), (1, 37, 2048, dict(c=True, clamp=(-0.3, 0.4))),
               (1, 5, 4096, {}), (1, 1000, 2048, dict(c=True)), (1, 64, 4096, dict(ldq=4160)),
               (3, 40, 4096, dict(c=True)), (1, 48, 1024, {}), (2, 17, 2048, {})]


@pytest.mark.parametrize("m,n,k,opt", FUSED_CASES)
def test_fused_decode_step(gpu, m, n, k, opt):
    Af, Bp, sb, bias = fused_inputs(m, n, k, seed=m * 7 + k + n)
    C = (np.random.default_rng(n).uniform(-1, 1, (m, n)).astype(np.float32)
         if opt.get("c") else None)
    cmin, cmax = opt.get("clamp", (-np.inf, np.inf))
    check_fused(Af, Bp, sb, bias, C, cmin, cmax, ldq=opt.get("ldq"))


def test_fused_decode_step_special_rows(gpu):
    """The fused kernel's quantization branches: an all-zero row (scale 1, zero point 0, all-zero
    values), a one-signed row (zero point -128), exact half-step ties (round half to even), and a
    row whose f32 source is not 16-byte aligned (the two launches)."""
    n, k = 40, 2048
    _, Bp, sb, bias = fused_inputs(1, n, k, seed=5)
    check_fused(np.zeros((1, k), np.float32), Bp, sb, bias)
    pos = np.abs(np.random.default_rng(1).standard_normal((1, k))).astype(np.float32)
    check_fused(pos, Bp, sb, bias)
    ties = np.zeros((1, k), np.float32)
    ties[0, 0], ties[0, 1] = -127.5, 127.5  # s = 1: x / s lands on .5 exactly
    ties[0, 2:200] = np.arange(198, dtype=np.float32) * 0.5 - 49.5
    check_fused(ties, Bp, sb, bias)
    Af, _, _, _ = fused_inputs(1, n, k, seed=9)
    check_fused(Af, Bp, sb, bias, a_offset=1)
