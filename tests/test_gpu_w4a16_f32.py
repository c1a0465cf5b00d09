"""W4A16 with f32 output on the GPU: gemm_1xnbias_clamp_f32_f16_qsi4c2t and its packed sibling
…_f32_f16p_qsi4c2p, against the reference test's oracle for these types
(reference_gemm_quantized_weight_mixed<float16_t, float>, restated as
tqto_gemm_f16_qsi4c2t_f32out and pinned bit-exact to the reference's golden vectors).

Bars, written here:
  * the generic kernel (bl != 32, k % 128 != 0 or k > 4096) runs the oracle's operation order
    and must match it bit for bit;
  * the MFMA kernels sum each 32-k block exactly-multiplied in f32 and scale-accumulate the
    blocks, so against exact (float64) math they must stay within
    (bl + k/bl + 16) * 2^-24 * (sum|a*w| + |C| + |bias|) — a bound on their own rounding,
    far tighter than the reference test's 1.0 absolute tolerance; the oracle itself is within
    (2k + 4) * 2^-24 * the same sum (pinned in test_oracle.py), which bounds got - oracle.
"""

import ctypes
import os

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


def generic_path(k, bl):
    return not (bl == 32 and k % 128 == 0 and k <= 4096)


def run_f32(d, C, bias, cmin, cmax, packed=False, shim=None):
    torch = _torch()
    g = _g()
    A16, Bp, S16, bl = d["A16"], d["Bp"], d["S16"], d["bl"]
    m, k = A16.shape
    n = Bp.shape[0]
    kind = "w4a16fp" if packed else "w4a16f"
    dA, dB, dS = g.dev(A16.view(np.int16)), g.dev(Bp), g.dev(S16.view(np.int16))
    if packed:
        pA = torch.empty(max(2 * m * k, 1), dtype=torch.uint8, device="cuda:0")
        pB = torch.empty(max(n * k // 2, 1), dtype=torch.uint8, device="cuda:0")
        g.lib().fn(kind, "run_a_pack")(m, k, k, k, 0, dA.data_ptr(), pA.data_ptr())
        g.lib().fn(kind, "run_bt_pack")(n, k, k, k, 0, dB.data_ptr(), pB.data_ptr())
        dA, dB = pA, pB
    dC, dbias = g.dev(C), g.dev(bias)
    dD = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
    args = (m, n, k, bl, dA.data_ptr(), k, 0, dB.data_ptr(), k, 0, dS.data_ptr(), k // bl,
            g.dp(dC), n, dD.data_ptr(), n, g.dp(dbias), float(cmin), float(cmax))
    if shim is not None:
        f = shim.tqts_run_w4a16f
        f.restype = None
        f.argtypes = ([ctypes.c_int] + [ctypes.c_size_t] * 4 +
                      [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t] * 2 +
                      [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t,
                       ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float,
                       ctypes.c_float])
        f(int(packed), *args)
    else:
        g.lib().fn(kind, "run")(*args)
    torch.cuda.synchronize()
    return dD.cpu().numpy()


def exact_and_scale(d, C, bias):
    A = T.bits_f16(d["A16"]).astype(np.float64)
    Bp = d["Bp"]
    n, kb = Bp.shape
    q = np.empty((n, 2 * kb))
    q[:, 0::2] = (Bp & 15) - 8.0
    q[:, 1::2] = (Bp >> 4) - 8.0
    W = q * np.repeat(T.bits_f16(d["S16"]).astype(np.float64), d["bl"], axis=1)
    exact = A @ W.T
    S = np.abs(A) @ np.abs(W).T
    for t in (C, None if bias is None else bias[None, :]):
        if t is not None:
            exact = exact + t
            S = S + np.abs(t)
    return exact, S


def check(d, C, bias, cmin=-np.inf, cmax=np.inf, **kw):
    got = run_f32(d, C, bias, cmin, cmax, **kw)
    exp = T.oracle_w4a16_f32(d["A16"], d["Bp"], d["S16"], d["bl"], C, bias, cmin, cmax)
    k, bl = d["A16"].shape[1], d["bl"]
    if generic_path(k, bl):
        np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))
        return got
    exact, S = exact_and_scale(d, C, bias)
    exact = np.minimum(np.maximum(exact, cmin), cmax)
    assert np.all(np.isfinite(got))
    tol = (bl + k // bl + 16) * 2.0 ** -24 * S
    assert np.all(np.abs(got - exact) <= tol), np.max(np.abs(got - exact) / tol)
    assert np.all(np.abs(got - exp) <= tol + (2 * k + 4) * 2.0 ** -24 * S)
    return got


def gen(m, n, k, bl, seed, with_c, with_bias=True):
    d = T.gen_w4a16(m, n, k, bl=bl, seed=seed, with_bias=False)
    rng = np.random.default_rng(seed + 1)
    C = rng.uniform(-5, 5, size=(m, n)).astype(np.float32) if with_c else None
    bias = rng.uniform(-0.5, 0.5, size=n).astype(np.float32) if with_bias else None
    return d, C, bias


# (m, n, k, bl): the strip kernel (k 2048/3072/4096, bl 32), the block kernel (other k % 128,
# bl 32) and the generic kernel (bl 16, k not a multiple of 128)
SHAPES = [(32, 96, 4096, 32), (33, 40, 2048, 32), (7, 50, 3072, 32), (32, 48, 1024, 32),
          (5, 18, 384, 32), (9, 20, 64, 16), (6, 17, 96, 32), (3, 5, 10, 2),
          (33, 8200, 2048, 32)]


@pytest.mark.parametrize("m,n,k,bl", SHAPES)
@pytest.mark.parametrize("packed", [False, True], ids=["plain", "packed"])
def test_w4a16_f32_run(gpu, packed, m, n, k, bl):
    d, C, bias = gen(m, n, k, bl, seed=m + n + k, with_c=(m % 2 == 1))
    check(d, C, bias, packed=packed)
    check(d, None, None, cmin=-0.75, cmax=0.5, packed=packed)


def test_w4a16_f32_reference_test_list(gpu, shim):
    """The reference runner's own inputs and shape list (ref_w4a16_f32.npz, written by the
    reference's test oracle): bit-exact where the generic kernel runs, within the bound above
    on the MFMA path, through the interface struct."""
    with np.load(os.path.join(T.GOLDEN_DIR, "ref_w4a16_f32.npz"), allow_pickle=False) as z:
        g = {key: z[key] for key in z.files}
    for i, (m, n, k, bl, bias, c, clamp) in enumerate(g["shapes"]):
        pre = "w4a16f_%d_" % i
        d = dict(A16=g[pre + "A"], Bp=g[pre + "Bp"], S16=g[pre + "S"], bl=int(bl))
        C = g[pre + "C"] if c else None
        bv = g[pre + "bias"] if bias else None
        lo, hi = (float(v) for v in g[pre + "clamp"])
        got = check(d, C, bv, lo, hi, shim=shim)
        if generic_path(int(k), int(bl)):
            np.testing.assert_array_equal(got.view(np.uint32), g[pre + "D"].view(np.uint32))


def test_w4a16_f32_config4_shape(gpu):
    """BASELINE cfg 4 (M32 K4096 N14336 bl32) with f32 output, plain and packed."""
    d, C, bias = gen(32, 14336, 4096, 32, seed=4, with_c=False)
    a = check(d, C, bias)
    b = check(d, C, bias, packed=True)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_w4a16_f32_matches_f16_type_before_rounding(gpu, shim):
    """With f16-valued C and bias the f16-output type's result is this type's result rounded
    once to f16 (both run the same kernels; only the store differs)."""
    d, _, _ = gen(32, 64, 2048, 32, seed=21, with_c=False)
    rng = np.random.default_rng(22)
    C16 = T.f16_bits(rng.uniform(-5, 5, size=(32, 64)))
    b16 = T.f16_bits(rng.uniform(-0.5, 0.5, size=64))
    f32 = run_f32(d, T.bits_f16(C16).astype(np.float32), T.bits_f16(b16).astype(np.float32),
                  -np.inf, np.inf)
    h = _g().run_w4a16(shim, dict(d, C16=C16, bias16=b16), 0xFC00, 0x7C00)
    np.testing.assert_array_equal(h, f32.astype(np.float16).view(np.uint16))
