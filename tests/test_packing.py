"""Packed (p) kernel types without a GPU: the numpy restatement of the packed layout against
hand-worked layouts, its permutation property, the offset getters against that restatement,
the entry points the reference's packed headers declare, and their interface structs.

The device packers and packed runs are checked against the same restatement, and against the
unpacked runs, in test_gpu_packed.py."""

import ctypes

import numpy as np
import pytest

import tqt_testlib as T

V = "_mfma_gfx950"
PACKED = {
    "clampp": "gemm_clamp_i32_i8p_i8p",
    "w8a8pb": "gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp",
    "w8a8p": "gemm_1xnbias_reqi32toi8_clamp_qai8_qai8p_qsi8cxp",
    "w4a8p": "gemm_1xnbias_clamp_f32_qai8dxp_qsi4cxp",
    "w4a16p": "gemm_1xnbias_clamp_f16_f16p_qsi4c2p",
    "igemmclp": "igemmcl_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxp",
}
# Functions each reference packed header declares (…_4x1vl_rvv.h / …_8x2vl_rvv.h).
REF_FUNCS = {
    "clampp": ["get_m_step", "get_n_step", "get_a_packed_offset", "get_b_packed_offset",
               "get_c_offset", "get_d_offset", "get_d_size", "get_a_packed_size",
               "get_b_packed_size", "run_a_pack", "run_b_pack", "run_bt_pack", "run"],
    "w8a8pb": ["get_m_step", "get_n_step", "get_a_offset", "get_b_packed_offset", "get_c_offset",
               "get_bias_offset", "get_d_offset", "get_d_size", "get_b_packed_size",
               "run_b_pack", "run_bt_pack", "run"],
    "w8a8p": ["get_m_step", "get_n_step", "get_a_packed_offset", "get_b_packed_offset",
              "get_c_offset", "get_bias_offset", "get_d_offset", "get_d_size",
              "get_a_packed_size", "get_b_packed_size", "run_a_pack", "run_b_pack",
              "run_bt_pack", "run"],
    "w4a8p": ["get_m_step", "get_n_step", "get_a_packed_offset", "get_b_packed_offset",
              "get_c_offset", "get_bias_offset", "get_d_offset", "get_d_size",
              "get_a_packed_size", "get_b_packed_size", "run_a_pack", "run_bt_pack", "run"],
    "w4a16p": ["get_m_step", "get_n_step", "get_a_packed_offset", "get_b_packed_offset",
               "get_scale_b_offset", "get_c_offset", "get_bias_offset", "get_d_offset",
               "get_d_size", "get_a_packed_size", "get_b_packed_size", "run_a_pack",
               "run_bt_pack", "run"],
    "w4a16fp": ["get_m_step", "get_n_step", "get_a_packed_offset", "get_b_packed_offset",
                "get_scale_b_offset", "get_c_offset", "get_bias_offset", "get_d_offset",
                "get_d_size", "get_a_packed_size", "get_b_packed_size", "run_a_pack",
                "run_bt_pack", "run"],
    "w8dynp": ["get_m_step", "get_n_step", "get_a_packed_offset", "get_b_packed_offset",
               "get_c_offset", "get_bias_offset", "get_d_offset", "get_d_size",
               "get_a_packed_size", "get_b_packed_size", "run_a_pack", "run_b_pack",
               "run_bt_pack", "run"],
    "w8dynhp": ["get_m_step", "get_n_step", "get_a_packed_offset", "get_b_packed_offset",
                "get_c_offset", "get_bias_offset", "get_d_offset", "get_d_size",
                "get_a_packed_size", "get_b_packed_size", "run_a_pack", "run_b_pack",
                "run_bt_pack", "run"],
    "igemmclp": ["get_m_step", "get_n_step", "get_b_packed_offset", "get_c_offset",
                 "get_bias_offset", "get_d_offset", "get_d_size", "get_b_packed_size",
                 "run_bt_pack", "run"],
}


@pytest.fixture(scope="module")
def mod():
    return T.load_product_module()


@pytest.fixture(scope="module")
def lib(mod):
    return mod.load()


def sym(mod, kind, action):
    return mod._sym(kind, action)


def test_layout_restatement_hand_worked():
    # 3 rows of 20 bytes, panels of 2 rows: panel 0 = chunk 0 of rows 0, 1, then the 4-byte
    # tails of rows 0, 1; panel 1 (one row) starts at 2 * 20
    X = np.arange(60).reshape(3, 20)
    exp = (list(range(0, 16)) + list(range(20, 36)) + [16, 17, 18, 19, 36, 37, 38, 39] +
           list(range(40, 56)) + [56, 57, 58, 59])
    np.testing.assert_array_equal(T.pack_panels(X, 2), exp)
    # a k_idx = 3 sub-buffer: the narrower panel 1 starts 3 * (2 - 1) bytes earlier
    out = np.full(80, -1)
    T.pack_panels(X[:, :4], 2, ld_packed=20, shift=3, out=out, base=3 * 2)
    assert list(out[6:14]) == [0, 1, 2, 3, 20, 21, 22, 23]
    assert list(out[6 + 40 - 3:6 + 40 - 3 + 4]) == [40, 41, 42, 43]


def test_layout_restatement_hand_worked_wide_chunks():
    # 2 rows of 200 bytes in one panel, 128-byte chunks: row 0 bytes 0-127, row 1 bytes
    # 0-127, then the 72-byte tails of rows 0 and 1
    X = np.arange(400).reshape(2, 200)
    exp = (list(range(0, 128)) + list(range(200, 328)) + list(range(128, 200)) +
           list(range(328, 400)))
    np.testing.assert_array_equal(T.pack_panels(X, 16, kc=128), exp)


@pytest.mark.parametrize("rows,kb,step,kc", [(1, 16, 16, 16), (37, 100, 16, 16),
                                             (130, 64, 128, 16), (5, 7, 4, 16),
                                             (256, 2048, 128, 128), (33, 8192, 32, 16),
                                             (300, 1000, 128, 128), (45, 2048, 16, 128)])
def test_layout_is_a_permutation(rows, kb, step, kc):
    idx = np.arange(rows * kb).reshape(rows, kb)
    out = T.pack_panels(idx, step, kc=kc)
    np.testing.assert_array_equal(np.sort(out), np.arange(rows * kb))
    # inverse: each element found where the chunk rule puts it
    rng = np.random.default_rng(rows + kb)
    for _ in range(200):
        r, c = int(rng.integers(rows)), int(rng.integers(kb))
        p, rl = divmod(r, step)
        w = min(step, rows - p * step)
        ch = c // kc
        cw = min(kc, kb - kc * ch)
        assert out[p * step * kb + kc * ch * w + rl * cw + c % kc] == r * kb + c


def test_fragment_order_is_an_involution_on_whole_groups():
    for kb in (64, 100, 128, 2048, 2050):
        p = T.frag_perm(kb)
        np.testing.assert_array_equal(np.sort(p), np.arange(kb))
        np.testing.assert_array_equal(p[p], np.arange(kb))
        np.testing.assert_array_equal(p[kb // 64 * 64:], np.arange(kb // 64 * 64, kb))
    # chunk c of a group holds 4-byte word c of each of the group's four 16-byte blocks
    p = T.frag_perm(64)
    for c in range(4):
        np.testing.assert_array_equal(p[16 * c:16 * c + 16],
                                      np.concatenate([np.arange(4) + 16 * b + 4 * c
                                                      for b in range(4)]))


def test_packed_entry_points_follow_reference_names(lib, mod):
    exported = set(lib.symbol_names())
    for kind, funcs in REF_FUNCS.items():
        for f in funcs:
            assert sym(mod, kind, f) in exported, (kind, f)
            if f.startswith("run"):
                assert sym(mod, kind, f + "_async") in exported


def _getter(lib, name, nargs):
    f = getattr(lib.dll, name)
    f.restype = ctypes.c_size_t
    f.argtypes = [ctypes.c_size_t] * nargs
    return f


# (kind, getter, element bytes (0 = int4), rows, k, step kind, frag)
OPERANDS = [
    ("clampp", "get_a_packed_offset", 1, 300, 192, "m", False),
    ("clampp", "get_b_packed_offset", 1, 260, 192, "n", False),
    ("w8a8pb", "get_b_packed_offset", 1, 129, 256, "n", False),
    ("w8a8p", "get_a_packed_offset", 1, 257, 320, "m", False),
    ("w8a8p", "get_b_packed_offset", 1, 200, 320, "n", False),
    ("w4a8p", "get_a_packed_offset", 1, 37, 512, "m", False),
    ("w4a8p", "get_b_packed_offset", 0, 45, 512, "n", False),
    ("w4a16p", "get_a_packed_offset", 2, 70, 384, "m", False),
    ("w4a16p", "get_b_packed_offset", 0, 40, 384, "n", True),
    ("w4a16fp", "get_a_packed_offset", 2, 70, 384, "m", False),
    ("w4a16fp", "get_b_packed_offset", 0, 40, 384, "n", True),
    ("w8dynp", "get_a_packed_offset", 1, 257, 320, "m", False),
    ("w8dynhp", "get_b_packed_offset", 1, 129, 256, "n", False),
    ("igemmclp", "get_b_packed_offset", 1, 200, 288, "n", False),
]


@pytest.mark.parametrize("kind,getter,esize,rows,k,which,frag", OPERANDS)
def test_packed_offsets_address_the_restated_layout(lib, mod, kind, getter, esize, rows, k,
                                                    which, frag):
    """get_{a,b}_packed_offset(idx, k_idx, ld = k, actual = rows - idx), the reference's formula
    (idx * ld + k_idx * min(actual, step)) in elements, lands on element (idx, k_idx) of the
    restated layout for every panel start and every chunk-aligned k_idx (whole 64-byte groups
    for the fragment-ordered W4A16 weights)."""
    step = _getter(lib, sym(mod, kind, "get_%s_step" % which), 0)()
    f = _getter(lib, sym(mod, kind, getter), 4)
    kbytes = k // 2 if esize == 0 else k * esize
    idx = np.arange(rows * kbytes).reshape(rows, kbytes)
    kc = T.PACK_CHUNK[kind]
    out = T.pack_panels(idx, step, kc=kc, frag=frag)
    kstep = 128 if frag else (2 * kc if esize == 0 else kc // esize)
    for r0 in range(0, rows, step):
        for k_idx in range(0, k, kstep):
            off = f(r0, k_idx, k, rows - r0)
            kb = k_idx // 2 if esize == 0 else k_idx * esize
            assert out[off] == r0 * kbytes + kb, (r0, k_idx)


def test_packed_sizes_equal_unpacked_sizes(lib, mod):
    m, n, k = 37, 91, 256
    g = lambda kind, what: _getter(lib, sym(mod, kind, what), 2)
    for kind in ("clampp", "w8a8p"):
        assert g(kind, "get_a_packed_size")(m, k) == m * k
        assert g(kind, "get_b_packed_size")(n, k) == n * k
    assert g("w8a8pb", "get_b_packed_size")(n, k) == n * k
    assert g("igemmclp", "get_b_packed_size")(n, k) == n * k
    assert g("w4a8p", "get_a_packed_size")(m, k) == m * k
    assert g("w4a8p", "get_b_packed_size")(n, k) == n * k // 2
    assert g("w4a16p", "get_a_packed_size")(m, k) == 2 * m * k
    assert g("w4a16p", "get_b_packed_size")(n, k) == n * k // 2
    assert g("clampp", "get_d_size")(m, n) == 4 * m * n
    assert g("w8a8p", "get_d_size")(m, n) == m * n
    assert g("w4a8p", "get_d_size")(m, n) == 4 * m * n
    assert g("w4a16p", "get_d_size")(m, n) == 2 * m * n
    assert g("w4a16fp", "get_a_packed_size")(m, k) == 2 * m * k
    assert g("w4a16fp", "get_b_packed_size")(n, k) == n * k // 2
    for kind in ("w4a16f", "w4a16fp"):
        ms = _getter(lib, sym(mod, kind, "get_m_step"), 0)()
        ns = _getter(lib, sym(mod, kind, "get_n_step"), 0)()
        assert (ms, ns) == ((_getter(lib, sym(mod, "w4a16", "get_m_step"), 0)(),
                             _getter(lib, sym(mod, "w4a16", "get_n_step"), 0)()) if kind == "w4a16f"
                            else (_getter(lib, sym(mod, "w4a16p", "get_m_step"), 0)(),
                                  _getter(lib, sym(mod, "w4a16p", "get_n_step"), 0)()))
        assert g(kind, "get_d_size")(m, n) == 4 * m * n
        assert _getter(lib, sym(mod, kind, "get_c_offset"), 3)(ms, ns, n) == 4 * (ms * n + ns)
        assert _getter(lib, sym(mod, kind, "get_bias_offset"), 1)(3 * ns) == 4 * 3 * ns
        base = "w4a16" if kind == "w4a16f" else "w4a16p"
        assert (_getter(lib, sym(mod, kind, "get_scale_b_offset"), 3)(ns, 3, 128) ==
                _getter(lib, sym(mod, base, "get_scale_b_offset"), 3)(ns, 3, 128))
    for kind in ("w8dynp", "w8dynhp"):
        assert g(kind, "get_a_packed_size")(m, k) == m * k
        assert g(kind, "get_b_packed_size")(n, k) == n * k
    for kind, es in (("w8dyn", 4), ("w8dynp", 4), ("w8dynh", 2), ("w8dynhp", 2)):
        ms = _getter(lib, sym(mod, kind, "get_m_step"), 0)()
        ns = _getter(lib, sym(mod, kind, "get_n_step"), 0)()
        assert g(kind, "get_d_size")(m, n) == es * m * n
        assert _getter(lib, sym(mod, kind, "get_d_offset"), 3)(ms, ns, n) == es * (ms * n + ns)
        assert _getter(lib, sym(mod, kind, "get_bias_offset"), 1)(2 * ns) == es * 2 * ns
    for kind in ("w4a8h", "w4a8b", "w4a8hp", "w4a8bp"):
        assert g(kind, "get_d_size")(m, n) == 2 * m * n
        ms = _getter(lib, sym(mod, kind, "get_m_step"), 0)()
        ns = _getter(lib, sym(mod, kind, "get_n_step"), 0)()
        # each output-type sibling advertises its f32 type's steps (plain or packed)
        base = "w4a8p" if kind.endswith("p") else "w4a8"
        assert (ms, ns) == (_getter(lib, sym(mod, base, "get_m_step"), 0)(),
                            _getter(lib, sym(mod, base, "get_n_step"), 0)())
        off = _getter(lib, sym(mod, kind, "get_d_offset"), 3)(3 * ms, 2 * ns, n)
        assert off == 2 * (3 * ms * n + 2 * ns)
        assert _getter(lib, sym(mod, kind, "get_bias_offset"), 1)(2 * ns) == 2 * 2 * ns


def test_packed_steps_via_interface_structs(lib, mod, shim):
    out = (ctypes.c_size_t * 58)()
    shim.tqts_steps_via_interfaces(out)
    kinds = (["clamp", "w8a8", "w4a8", "w4a16", "igemmcl"] + list(PACKED) +
             ["w4a8h", "w4a8hp", "w4a8b", "w4a8bp", "w4a16f", "w4a16fp", "w8dyn", "w8dynp",
              "w8dynh", "w8dynhp", "convcl", "convclp", "mx1", "mx1p", "convcf", "convcfp",
              "igemmcf", "igemmcfp"])
    for t, kind in enumerate(kinds):
        assert out[2 * t] == _getter(lib, sym(mod, kind, "get_m_step"), 0)()
        assert out[2 * t + 1] == _getter(lib, sym(mod, kind, "get_n_step"), 0)()
