"""GPU parity on seeded random shapes: the W8A8, W4A8 and W4A16 runs through the C ABI against
the CPU oracle, over shapes drawn so that every kernel path of each type is taken (W8A8: the
stream kernel for k % 128 == 0, the double-buffered kernel for k % 16 == 0, the per-output kernel
otherwise; W4A8: the decode strip kernel at m = 1 with k = 2048 / 4096, the MFMA k-split kernel
for k % 256 == 0, the per-output kernel otherwise; W4A16: the chunk kernel for k % 512 == 0, the
MFMA kernel for k % 128 == 0, the per-output kernel otherwise), with ragged m and n, C, bias and
clamps. Same bar as test_gpu_parity: bit-exact for W8A8 and W4A8, within 2 f16 ULP for W4A16."""

import numpy as np
import pytest

import tqt_testlib as T
from test_gpu_parity import check_w4a16

pytestmark = pytest.mark.gpu

CASES = 12


def _gr():
    import gpu_run

    return gpu_run


def _w8a8_shape(i):
    r = np.random.default_rng(1000 + i)
    kind = i % 3
    if kind == 0:
        k = 128 * int(r.integers(1, 9))
    elif kind == 1:
        k = 16 * int(r.integers(1, 40))
        k += 16 if k % 128 == 0 else 0
    else:
        k = int(r.integers(1, 300))
    return int(r.integers(1, 300)), int(r.integers(1, 700)), k, bool(r.integers(0, 2))


@pytest.mark.parametrize("i", range(CASES))
def test_w8a8_sweep(gpu, i):
    m, n, k, with_c = _w8a8_shape(i)
    d = T.gen_w8a8(m, n, k, seed=2000 + i, with_c=with_c)
    cmin, cmax = (-128, 127) if i % 4 else (-60, 90)
    got = _gr().run_w8a8(d, cmin, cmax)
    exp = T.oracle_w8a8(d["A"], d["B"], d["C"], d["bias"], cmin, cmax, d["scale_a"],
                        d["scale_b"], n, d["scale_d"], d["zp_d"])
    np.testing.assert_array_equal(got, exp, err_msg="m=%d n=%d k=%d" % (m, n, k))


def _w4a8_shape(i):
    r = np.random.default_rng(3000 + i)
    kind = i % 3
    if kind == 0:
        m, k = 1, (2048, 4096)[i % 2]
    elif kind == 1:
        m, k = int(r.integers(2, 20)), 256 * int(r.integers(1, 12))
    else:
        m, k = int(r.integers(1, 20)), 2 * int(r.integers(1, 400))
        k += 2 if k % 256 == 0 else 0
    return m, int(r.integers(1, 600)), k


@pytest.mark.parametrize("i", range(CASES))
def test_w4a8_sweep(gpu, i):
    m, n, k = _w4a8_shape(i)
    d = T.gen_w4a8(m, n, k, seed=4000 + i, with_c=bool(i % 2), with_bias=bool(i % 3))
    cmin, cmax = (-np.inf, np.inf) if i % 4 else (-0.5, 1.0)
    got = _gr().run_w4a8(d, cmin, cmax)
    exp = T.oracle_w4a8(d["A"], d["Bp"], d["C"], d["bias"], cmin, cmax, d["scale_a"], d["zp_a"],
                        d["scale_b"])
    np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32),
                                  err_msg="m=%d n=%d k=%d" % (m, n, k))


def _w4a16_shape(i):
    r = np.random.default_rng(5000 + i)
    kind = i % 3
    if kind == 0:
        k = 512 * int(r.integers(1, 5))
    elif kind == 1:
        k = 128 * int(r.integers(1, 16))
        k += 128 if k % 512 == 0 else 0
    else:
        k = 32 * int(r.integers(1, 40))
        k += 32 if k % 128 == 0 else 0
    return int(r.integers(1, 70)), int(r.integers(1, 700)), k


@pytest.mark.parametrize("i", range(CASES))
def test_w4a16_sweep(gpu, shim, i):
    m, n, k = _w4a16_shape(i)
    bl = 32
    d = T.gen_w4a16(m, n, k, bl=bl, seed=6000 + i, with_c=bool(i % 2), with_bias=bool(i % 3))
    lo, hi = (-65504.0, 65504.0) if i % 4 else (-0.5, 0.75)
    cmin, cmax = int(T.f16_bits(lo)), int(T.f16_bits(hi))
    got = _gr().run_w4a16(shim, d, cmin, cmax)
    exp = T.oracle_w4a16(d["A16"], d["Bp"], d["S16"], bl, d["C16"], d["bias16"], cmin, cmax)
    check_w4a16(got, exp, d, (lo, hi))
