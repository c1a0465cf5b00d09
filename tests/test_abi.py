"""C-ABI checks that need no GPU: the library loads, exports exactly what include/*.h declares,
the offset getters follow the reference's formulas, the interface structs bind, and violated
preconditions abort (the reference's TQT_ASSUME) instead of returning garbage."""

import ctypes
import glob
import os
import re
import subprocess
import sys

import pytest

import tqt_testlib as T

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
V = "_mfma_gfx950"
TYPES = {
    "clamp": "gemm_clamp_i32_i8_i8",
    "w8a8": "gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt",
    "w4a8": "gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt",
    "w4a16": "gemm_1xnbias_clamp_f16_f16_qsi4c2t",
    "igemmcl": "igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt",
}


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(INC, "*.h")):
        text = open(h).read()
        names.update(re.findall(r"^(?:size_t|void|const char \*)\s*(tqt_\w+)\s*\(", text, re.M))
    return names


@pytest.fixture(scope="module")
def dll():
    lib = T.load_product_module().load()
    return lib.dll


def getter(dll, name, nargs):
    f = getattr(dll, name)
    f.restype = ctypes.c_size_t
    f.argtypes = [ctypes.c_size_t] * nargs
    return f


def test_exports_every_declared_function(dll):
    names = declared_functions()
    # five kernel types x (steps, offsets, d_size, run, run_async) + W4A16 scale_b offset
    assert len(names) >= 5 * 8 + 1
    missing = [n for n in sorted(names) if not hasattr(dll, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", T.load_product_module().LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\b(tqt_\w+)$", out, re.M))
    assert exported == names, (sorted(exported - names), sorted(names - exported))


def test_entry_points_follow_reference_names():
    names = declared_functions()
    for t in TYPES.values():
        for g in ("m_step", "n_step", "c_offset", "d_offset", "d_size", "b_offset"):
            assert "tqt_get_%s_%s%s" % (g, t, V) in names
        # clamp_i32 has no bias (…clamp_i32_i8_i8_4x1vl_rvv.h:36-108)
        assert (("tqt_get_bias_offset_%s%s" % (t, V)) in names) == (t != TYPES["clamp"])
        run = "run_igemm" if t.startswith("igemmcl") else "run"
        assert "tqt_%s_%s%s" % (run, t, V) in names
        assert "tqt_%s_%s%s_async" % (run, t, V) in names
        # igemmcl has no A offset in the reference (…igemmcl…qsi8cxt_4x1vl_rvv.h:26-71)
        assert (("tqt_get_a_offset_%s%s" % (t, V)) in names) == (not t.startswith("igemmcl"))
    assert "tqt_get_scale_b_offset_%s%s" % (TYPES["w4a16"], V) in names


def test_offsets_follow_reference_formulas(dll):
    ms = {k: getter(dll, "tqt_get_m_step_%s%s" % t, 0)() for k, t in
          ((k, (t, V)) for k, t in TYPES.items())}
    ns = {k: getter(dll, "tqt_get_n_step_%s%s" % t, 0)() for k, t in
          ((k, (t, V)) for k, t in TYPES.items())}
    for k in TYPES:
        assert ms[k] > 0 and ns[k] > 0
    g = lambda kind, what, n: getter(dll, "tqt_get_%s_%s%s" % (what, TYPES[kind], V), n)
    lda, ldb, ldc, ldd = 4160, 4352, 4608, 5120
    for i in range(3):
        m_idx, n_idx, k_idx = ms["clamp"] * i, ns["clamp"] * (i + 1), 64 * i
        # …clamp_i32_i8_i8_4x1vl_rvv.cpp:25-64: B is K x N row-major
        assert g("clamp", "a_offset", 3)(m_idx, k_idx, lda) == m_idx * lda + k_idx
        assert g("clamp", "b_offset", 3)(n_idx, k_idx, ldb) == k_idx * ldb + n_idx
        assert g("clamp", "c_offset", 3)(m_idx, n_idx, ldc) == 4 * (m_idx * ldc + n_idx)
        assert g("clamp", "d_offset", 3)(m_idx, n_idx, ldd) == 4 * (m_idx * ldd + n_idx)
        # …qsi8cxt_4x1vl_rvv.cpp:26-79: B^T is N x K
        m_idx, n_idx = ms["w8a8"] * i, ns["w8a8"] * i
        assert g("w8a8", "a_offset", 3)(m_idx, k_idx, lda) == m_idx * lda + k_idx
        assert g("w8a8", "b_offset", 3)(n_idx, k_idx, ldb) == n_idx * ldb + k_idx
        assert g("w8a8", "c_offset", 3)(m_idx, n_idx, ldc) == 4 * (m_idx * ldc + n_idx)
        assert g("w8a8", "bias_offset", 1)(n_idx) == 4 * n_idx
        assert g("w8a8", "d_offset", 3)(m_idx, n_idx, ldd) == m_idx * ldd + n_idx
        # …qai8dx_qsi4cxt_4x1vl_rvv.cpp:25-75: int4 B offset n*(ldb/2) + k/2
        m_idx, n_idx = ms["w4a8"] * i, ns["w4a8"] * i
        assert g("w4a8", "a_offset", 3)(m_idx, k_idx, lda) == m_idx * lda + k_idx
        assert g("w4a8", "b_offset", 3)(n_idx, k_idx, ldb) == n_idx * (ldb // 2) + k_idx // 2
        assert g("w4a8", "c_offset", 3)(m_idx, n_idx, ldc) == 4 * (m_idx * ldc + n_idx)
        assert g("w4a8", "bias_offset", 1)(n_idx) == 4 * n_idx
        assert g("w4a8", "d_offset", 3)(m_idx, n_idx, ldd) == 4 * (m_idx * ldd + n_idx)
        # …qsi4c2t_8x2vl_rvv.cpp:25-86: f16 A/C/D, int4 B, f16 scale_b [n, ldsb]
        m_idx, n_idx, bl = ms["w4a16"] * i, ns["w4a16"] * i, 32
        assert g("w4a16", "a_offset", 4)(m_idx, k_idx, lda, bl) == 2 * (m_idx * lda + k_idx)
        assert g("w4a16", "b_offset", 4)(n_idx, k_idx, ldb, bl) == n_idx * (ldb // 2) + k_idx // 2
        assert g("w4a16", "scale_b_offset", 3)(n_idx, i, 128) == 2 * (n_idx * 128 + i)
        assert g("w4a16", "c_offset", 3)(m_idx, n_idx, ldc) == 2 * (m_idx * ldc + n_idx)
        assert g("w4a16", "bias_offset", 1)(n_idx) == 2 * n_idx
        assert g("w4a16", "d_offset", 3)(m_idx, n_idx, ldd) == 2 * (m_idx * ldd + n_idx)
        # igemmcl…qsi8cxt_4x1vl_rvv.cpp:26-71
        m_idx, n_idx = ms["igemmcl"] * i, ns["igemmcl"] * i
        assert g("igemmcl", "b_offset", 3)(n_idx, k_idx, ldb) == n_idx * ldb + k_idx
        assert g("igemmcl", "d_offset", 3)(m_idx, n_idx, ldd) == m_idx * ldd + n_idx
    assert g("clamp", "d_size", 2)(64, 256) == 64 * 256 * 4
    assert g("w8a8", "d_size", 2)(512, 4096) == 512 * 4096
    assert g("w4a8", "d_size", 2)(8, 11008) == 8 * 11008 * 4
    assert g("w4a16", "d_size", 2)(32, 14336) == 32 * 14336 * 2
    assert g("igemmcl", "d_size", 2)(25088, 128) == 25088 * 128


def test_interface_structs_bind_the_gfx950_variant(dll, shim):
    out = (ctypes.c_size_t * 58)()  # five kernel types, then packed and output-type siblings
    shim.tqts_steps_via_interfaces(out)
    for t, kind in enumerate(TYPES):
        assert out[2 * t] == getter(dll, "tqt_get_m_step_%s%s" % (TYPES[kind], V), 0)()
        assert out[2 * t + 1] == getter(dll, "tqt_get_n_step_%s%s" % (TYPES[kind], V), 0)()


def test_target_is_gfx950(dll):
    f = dll.tqt_gfx950_target
    f.restype = ctypes.c_char_p
    assert f() == b"gfx950"


ABORT_CASES = [
    # (symbol, args): each violates a precondition the reference asserts with TQT_ASSUME
    ("tqt_get_a_offset_%s%s" % (TYPES["w8a8"], V), (1, 0, 16)),        # m_idx % m_step
    ("tqt_get_b_offset_%s%s" % (TYPES["w4a8"], V), (0, 3, 16)),        # odd k_idx for int4
    ("tqt_get_a_offset_%s%s" % (TYPES["w4a16"], V), (0, 16, 64, 32)),  # k_idx % bl
    ("tqt_get_b_offset_%s%s" % (TYPES["w4a16"], V), (0, 0, 64, 3)),    # odd bl
]


@pytest.mark.parametrize("sym,args", ABORT_CASES)
def test_violated_precondition_aborts(sym, args):
    code = ("import ctypes, sys; sys.path.insert(0, %r); import tqt_testlib as T; "
            "d = T.load_product_module().load().dll; f = getattr(d, %r); "
            "f.restype = ctypes.c_size_t; f.argtypes = [ctypes.c_size_t] * %d; f(*%r); "
            "print('returned')") % (os.path.dirname(os.path.abspath(__file__)), sym, len(args),
                                    args)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "returned" not in r.stdout
    assert "%" in r.stderr or "==" in r.stderr, r.stderr


def test_null_params_return_before_touching_the_gpu(dll):
    """Reference …qsi8cxt…cpp:148-150, …qai8dx_qsi4cxt…cpp:165-167, igemmcl :206-208: NULL
    params make run_* return at once. Here that holds before any HIP call, so it runs on a
    host without a GPU."""
    lib = T.load_product_module().load()
    lib.fn("w8a8", "run")(4, 4, 16, None, 16, 0, None, 16, 0, None, 4, None, 4, None, -128, 127,
                          None)
    lib.fn("w4a8", "run")(4, 4, 16, None, 16, 0, None, 16, 0, None, 4, None, 4, None, -1.0, 1.0,
                          None)


def test_empty_problem_is_a_no_op(dll):
    lib = T.load_product_module().load()
    lib.fn("clamp", "run")(0, 4, 16, None, 16, 0, None, 4, 0, None, 4, None, 4, -5, 5)
    lib.fn("clamp", "run")(4, 0, 16, None, 16, 0, None, 4, 0, None, 4, None, 4, -5, 5)
