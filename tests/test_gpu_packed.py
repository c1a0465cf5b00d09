"""GPU checks of the packed (p) kernel types through the C ABI.

* Packers: the bytes each run_{a,b,bt}_pack writes equal the layout restated in numpy
  (tqt_testlib.pack_panels), including tail panels, rows whose length is not a multiple of the
  16-byte chunk, ld_packed > k, and k_idx sub-buffers (the reference's tail rule).
* Packed runs: bit-exact against the CPU oracle (int32, int8 and W4A8 f32 outputs) or, for
  W4A16, bit-exact against the unpacked run of the same inputs - packing is a permutation, so a
  packed run must reproduce the unpacked result exactly - and within 2 f16 ULP of the oracle. The reference's own packed test drivers (quantized_gemm_test_runner.h:482-699:
  pack, walk m_step x n_step tiles through the packed offset getters, compare) are replayed.
* k_idx: a K split into sub-buffers packed with their k_idx and run one after the other with C
  accumulation reproduces the full product.
"""

import ctypes

import numpy as np
import pytest

import tqt_testlib as T

pytestmark = pytest.mark.gpu

SENTINEL = 0xA5


def _g():
    import gpu_run

    return gpu_run


def _torch():
    import torch

    return torch


def dbuf(nbytes):
    torch = _torch()
    t = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda:0")
    t.fill_(SENTINEL)
    return t


def host(t, nbytes=None):
    a = t.cpu().numpy().view(np.uint8)
    return a if nbytes is None else a[:nbytes]


def as_bytes(x):
    return np.ascontiguousarray(x).view(np.uint8).reshape(x.shape[0], -1)


def step_of(kind, which):
    return _g().lib().fn(kind, "get_%s_step" % which)()


def pack(kind, action, rows, k, ld, ldp, k_idx, src, dst, dst_off=0):
    _g().lib().fn(kind, action)(rows, k, ld, ldp, k_idx, src.data_ptr(),
                                dst.data_ptr() + dst_off)


# (kind, action, source kind, step kind): sources are int8 [rows, k] ("i8"), int8 [k, n]
# ("i8kn", packed rows are its columns), f16 [rows, k] ("f16"), int4 [rows, k/2] ("i4") and
# fragment-ordered int4 ("i4f")
PACKERS = [
    ("clampp", "run_a_pack", "i8", "m"),
    ("clampp", "run_b_pack", "i8kn", "n"),
    ("clampp", "run_bt_pack", "i8", "n"),
    ("w8a8pb", "run_b_pack", "i8kn", "n"),
    ("w8a8pb", "run_bt_pack", "i8", "n"),
    ("w8a8p", "run_a_pack", "i8", "m"),
    ("w8a8p", "run_b_pack", "i8kn", "n"),
    ("w8a8p", "run_bt_pack", "i8", "n"),
    ("w4a8p", "run_a_pack", "i8", "m"),
    ("w4a8p", "run_bt_pack", "i4", "n"),
    ("w4a16p", "run_a_pack", "f16", "m"),
    ("w4a16p", "run_bt_pack", "i4f", "n"),
    ("igemmclp", "run_bt_pack", "i8", "n"),
]
PACK_SHAPES = [(1, 16), (37, 100), (130, 256), (300, 1152), (17, 2)]


def make_source(src, rows, k, seed):
    """-> (device source, its leading dimension in elements, logical rows x bytes matrix)"""
    rng = np.random.default_rng(seed)
    if src == "i8":
        X = rng.integers(-128, 128, size=(rows, k), dtype=np.int64).astype(np.int8)
        return _g().dev(X), k, as_bytes(X)
    if src == "i8kn":
        X = rng.integers(-128, 128, size=(k, rows), dtype=np.int64).astype(np.int8)
        return _g().dev(X), rows, as_bytes(np.ascontiguousarray(X.T))
    if src == "f16":
        X = T.f16_bits(rng.standard_normal((rows, k)))
        return _g().dev(X.view(np.int16)), k, as_bytes(X)
    X = rng.integers(0, 256, size=(rows, k // 2), dtype=np.uint8)  # int4 pairs
    return _g().dev(X), k, X


def kbytes_of(src, k):
    return k // 2 if src.startswith("i4") else (2 * k if src == "f16" else k)


@pytest.mark.parametrize("rows,k", PACK_SHAPES)
@pytest.mark.parametrize("kind,action,src,which", PACKERS)
def test_packer_writes_restated_layout(gpu, kind, action, src, which, rows, k):
    if src.startswith("i4") and k % 2:
        pytest.skip("int4 packing needs an even k")
    step = step_of(kind, which)
    dsrc, ld, X = make_source(src, rows, k, seed=rows * 7 + k)
    kb = kbytes_of(src, k)
    dst = dbuf(rows * kb)
    pack(kind, action, rows, k, ld, k, 0, dsrc, dst)
    exp = T.pack_panels(X, step, kc=T.PACK_CHUNK[kind], frag=src == "i4f")
    np.testing.assert_array_equal(host(dst), exp)


@pytest.mark.parametrize("kind,action,src,which", PACKERS)
def test_packer_ld_packed_and_k_idx_sub_buffers(gpu, kind, action, src, which):
    """Two K halves packed as sub-buffers (k_idx = 0 and k_idx = K/2, dst at the getter's
    offset) into a buffer of leading dimension ld_packed > K write what packing the full
    matrix writes there, panel gaps untouched."""
    rows, k = 300, 512
    ldp = k + 64
    step = step_of(kind, which)
    dsrc, ld, X = make_source(src, rows, k, seed=3)
    kb, kbp = kbytes_of(src, k), kbytes_of(src, ldp)
    nbytes = (rows - 1) // step * step * kbp + min(step, rows - (rows - 1) // step * step) * kb
    full = dbuf(nbytes)
    pack(kind, action, rows, k, ld, ldp, 0, dsrc, full)
    exp = np.full(nbytes, SENTINEL, np.uint8)
    T.pack_panels(X, step, kc=T.PACK_CHUNK[kind], ld_packed=kbp, frag=src == "i4f", out=exp)
    np.testing.assert_array_equal(host(full), exp)

    # halves: the second starts at the offset of element (0, k/2); its source pointer moves
    # k/2 elements along the packed rows
    halves = dbuf(nbytes)
    h = k // 2
    getter = "get_%s_packed_offset" % ("a" if which == "m" else "b")
    off = _g().lib().fn(kind, getter)(0, h, ldp, min(rows, step))
    if src == "i8kn":
        src_off = h * ld  # int8 [k, n]: k rows down
    else:
        src_off = kbytes_of(src, h)
    pack(kind, action, rows, h, ld, ldp, 0, dsrc, halves)
    _g().lib().fn(kind, action)(rows, h, ld, ldp, h, dsrc.data_ptr() + src_off,
                                halves.data_ptr() + off)
    np.testing.assert_array_equal(host(halves), exp)


@pytest.mark.parametrize("kind,action,src,which", PACKERS)
def test_packer_overlapping_tail_panel(gpu, kind, action, src, which):
    """ld_packed = k with k_idx > 0 moves the narrow last panel back onto the end of the panel
    before it; the reference packs panel after panel, so those bytes hold the last panel's."""
    step = step_of(kind, which)
    rows, k = 2 * step + step // 3 + 1, 256
    dsrc, ld, X = make_source(src, rows, k, seed=11)
    kb = kbytes_of(src, k)
    k_idx = 32
    dst = dbuf(rows * kb)
    pack(kind, action, rows, k, ld, k, k_idx, dsrc, dst)
    exp = np.full(rows * kb, SENTINEL, np.uint8)
    T.pack_panels(X, step, kc=T.PACK_CHUNK[kind], ld_packed=kb, shift=kbytes_of(src, k_idx),
                  frag=src == "i4f", out=exp)
    np.testing.assert_array_equal(host(dst), exp)


# --------------------------------------------------------------------------------------------
# packed runs
# --------------------------------------------------------------------------------------------

INT8_SHAPES = [(64, 256, 512, False), (130, 260, 192, True), (200, 136, 80, False),
               (3, 8, 11, False), (60, 63, 127, True), (257, 129, 1024, True), (1, 128, 64, False),
               (64, 256, 128, False), (130, 260, 384, True), (1280, 2048, 256, False)]


def packed_i8(kind, action, M, rows, k):
    d = _g().dev(M)
    out = dbuf(rows * k)
    ld = M.shape[1]
    pack(kind, action, rows, k, ld, k, 0, d, out)
    return out


@pytest.mark.parametrize("m,n,k,with_c", INT8_SHAPES)
def test_clamp_i32_packed_run(gpu, m, n, k, with_c):
    A, B, C = T.gen_clamp(m, n, k, seed=m + n, with_c=with_c, lo=-50, hi=50)
    Ap = packed_i8("clampp", "run_a_pack", A, m, k)
    Bp = packed_i8("clampp", "run_b_pack", B, n, k)  # [k, n] source
    Bpt = packed_i8("clampp", "run_bt_pack", np.ascontiguousarray(B.T), n, k)
    np.testing.assert_array_equal(host(Bp), host(Bpt))
    torch = _torch()
    dC = _g().dev(C)
    for cmin, cmax in [(-100000, 100000), (-2 ** 31, 2 ** 31 - 1)]:
        dD = torch.zeros((m, n), dtype=torch.int32, device="cuda:0")
        _g().lib().fn("clampp", "run")(m, n, k, Ap.data_ptr(), k, 0, Bp.data_ptr(), k, 0,
                                       _g().dp(dC), n, dD.data_ptr(), n, cmin, cmax)
        np.testing.assert_array_equal(dD.cpu().numpy(), T.oracle_clamp(A, B, C, cmin, cmax))


def w8a8_run_packed(kind, d, a_packed):
    A, B = d["A"], d["B"]
    m, k = A.shape
    n = B.shape[0]
    dA = packed_i8(kind, "run_a_pack", A, m, k) if a_packed else _g().dev(A)
    dB = packed_i8(kind, "run_bt_pack", B, n, k)
    dC, dbias, dsb = _g().dev(d["C"]), _g().dev(d["bias"]), _g().dev(d["scale_b"])
    torch = _torch()
    dD = torch.zeros((m, n), dtype=torch.int8, device="cuda:0")
    p = _g().w8a8_params(d, dsb)
    _g().lib().fn(kind, "run")(m, n, k, dA.data_ptr(), k, 0, dB.data_ptr(), k, 0, _g().dp(dC), n,
                               dD.data_ptr(), n, _g().dp(dbias), -128, 127, ctypes.byref(p))
    return dD.cpu().numpy()


@pytest.mark.parametrize("m,n,k,with_c", INT8_SHAPES)
@pytest.mark.parametrize("kind,a_packed", [("w8a8pb", False), ("w8a8p", True)])
def test_w8a8_packed_run(gpu, kind, a_packed, m, n, k, with_c):
    d = T.gen_w8a8(m, n, k, seed=5 + m, with_c=with_c)
    got = w8a8_run_packed(kind, d, a_packed)
    exp = T.oracle_w8a8(d["A"], d["B"], d["C"], d["bias"], -128, 127, d["scale_a"], d["scale_b"],
                        n, d["scale_d"], d["zp_d"])
    np.testing.assert_array_equal(got, exp)


def test_w8a8_packed_config2_matches_unpacked(gpu):
    """BASELINE cfg 2 (M512 K4096 N4096): the packed run reproduces the unpacked run (which
    test_gpu_parity.py holds to the oracle at this size) bit for bit."""
    d = T.gen_w8a8(512, 4096, 4096, seed=42)
    got = w8a8_run_packed("w8a8p", d, True)
    np.testing.assert_array_equal(got, _g().run_w8a8(d))


W4A8_SHAPES = [(1, 160, 4096), (4, 48, 1024), (8, 33, 512), (15, 40, 256), (37, 70, 768),
               (5, 21, 100), (16, 16, 2)]


@pytest.mark.parametrize("m,n,k", W4A8_SHAPES)
def test_w4a8_packed_run(gpu, m, n, k):
    d = T.gen_w4a8(m, n, k, seed=m * 3 + n, with_c=(m % 2 == 1))
    Ap = packed_i8("w4a8p", "run_a_pack", d["A"], m, k)
    dBsrc = _g().dev(d["Bp"])
    Bp = dbuf(n * k // 2)
    pack("w4a8p", "run_bt_pack", n, k, k, k, 0, dBsrc, Bp)
    dC, dbias = _g().dev(d["C"]), _g().dev(d["bias"])
    dsa, dza, dsb = _g().dev(d["scale_a"]), _g().dev(d["zp_a"]), _g().dev(d["scale_b"])
    mod = _g()._mod
    p = mod.QAI8DXQSI4CXParams(dsa.data_ptr(), dza.data_ptr(), dsb.data_ptr())
    torch = _torch()
    dD = torch.zeros((m, n), dtype=torch.float32, device="cuda:0")
    _g().lib().fn("w4a8p", "run")(m, n, k, Ap.data_ptr(), k, 0, Bp.data_ptr(), k, 0, _g().dp(dC),
                                  n, dD.data_ptr(), n, _g().dp(dbias), -np.inf, np.inf,
                                  ctypes.byref(p))
    exp = T.oracle_w4a8(d["A"], d["Bp"], d["C"], d["bias"], -np.inf, np.inf, d["scale_a"],
                        d["zp_a"], d["scale_b"])
    np.testing.assert_array_equal(dD.cpu().numpy().view(np.uint32), exp.view(np.uint32))


W4A16_SHAPES = [(32, 96, 2048, 32), (32, 14336 // 64, 4096, 32), (33, 40, 3072, 32),
                (32, 48, 384, 32), (7, 20, 64, 16), (5, 18, 96, 32),
                (33, 8200, 2048, 32), (20, 4104, 4096, 32), (32, 96, 1024, 32),
                (17, 300, 1536, 32)]


def run_w4a16p(shim, d, lda_extra=0):
    A16, Bsrc, S16, bl = d["A16"], d["Bp"], d["S16"], d["bl"]
    m, k = A16.shape
    n = Bsrc.shape[0]
    lda = k + lda_extra
    dA = _g().dev(A16.view(np.int16))
    Ap = dbuf(2 * ((m - 1) // 32 * 32 * lda + min(32, m - (m - 1) // 32 * 32) * k))
    pack("w4a16p", "run_a_pack", m, k, k, lda, 0, dA, Ap)
    Bp = dbuf(n * k // 2)
    pack("w4a16p", "run_bt_pack", n, k, k, k, 0, _g().dev(Bsrc), Bp)
    dS = _g().dev(S16.view(np.int16))
    dC = _g().dev(None if d["C16"] is None else d["C16"].view(np.int16))
    dbias = _g().dev(None if d["bias16"] is None else d["bias16"].view(np.int16))
    torch = _torch()
    dD = torch.zeros((m, n), dtype=torch.int16, device="cuda:0")
    f = shim.tqts_run_w4a16p
    f.restype = None
    f.argtypes = ([ctypes.c_size_t] * 4 + [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
                                           ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
                                           ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                           ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t,
                                           ctypes.c_void_p, ctypes.c_uint16, ctypes.c_uint16,
                                           ctypes.c_void_p])
    cmin = int(np.float16(-65504.0).view(np.uint16))
    cmax = int(np.float16(65504.0).view(np.uint16))
    f(m, n, k, bl, Ap.data_ptr(), lda, 0, Bp.data_ptr(), k, 0, dS.data_ptr(), k // bl,
      _g().dp(dC), n, dD.data_ptr(), n, _g().dp(dbias), cmin, cmax, None)
    return dD.cpu().numpy().view(np.uint16), cmin, cmax


@pytest.mark.parametrize("m,n,k,bl", W4A16_SHAPES)
def test_w4a16_packed_run_matches_unpacked(gpu, shim, m, n, k, bl):
    """Bit-identical to the unpacked run, and both held to the golden-pinned f32 oracle with
    the same <= 2 f16 ULP bar as the unpacked parity tests."""
    from test_gpu_parity import check_w4a16

    d = T.gen_w4a16(m, n, k, bl=bl, seed=m + n + k, with_c=(n % 3 == 0))
    got, cmin, cmax = run_w4a16p(shim, d, lda_extra=(64 if m > 32 else 0))
    unpacked = _g().run_w4a16(shim, d, cmin, cmax)
    np.testing.assert_array_equal(got, unpacked)
    exp = T.oracle_w4a16(d["A16"], d["Bp"], d["S16"], bl, d["C16"], d["bias16"], cmin, cmax)
    check_w4a16(got, exp, d, (-65504.0, 65504.0))


def test_w4a16_packed_config4_full(gpu, shim):
    """BASELINE cfg 4 at full size (M=32, K=4096, N=14336, bl=32) through the packed type:
    <= 2 f16 ULP against the oracle."""
    from test_gpu_parity import check_w4a16

    d = T.gen_w4a16(32, 14336, 4096, bl=32, seed=42)
    got, cmin, cmax = run_w4a16p(shim, d)
    exp = T.oracle_w4a16(d["A16"], d["Bp"], d["S16"], 32, None, d["bias16"], cmin, cmax)
    check_w4a16(got, exp, d, (-65504.0, 65504.0))


IGEMM_SHAPES = [(32, 48, 9, 9, 3, 3, (1, 1), (1, 1), (1, 1)),
                (128, 128, 14, 14, 3, 3, (1, 1), (1, 1), (1, 1)),
                (16, 20, 7, 6, 3, 2, (2, 1), (0, 1), (1, 2)),
                (3, 5, 6, 6, 3, 3, (1, 1), (1, 1), (1, 1))]


@pytest.mark.parametrize("ic,oc,ih,iw,kh,kw,stride,pad,dil", IGEMM_SHAPES)
def test_igemmcl_packed_run(gpu, ic, oc, ih, iw, kh, kw, stride, pad, dil):
    d = T.gen_igemmcl(2, ih, iw, ic, oc, kh, kw, stride=stride, pad=pad, dil=dil, seed=ic + oc)
    conv, W = d["conv"], d["W"]
    K = W.shape[1]
    m = conv.output_shape[0] * conv.output_shape[1] * conv.output_shape[2]
    Wp = packed_i8("igemmclp", "run_bt_pack", W, oc, K)
    din, dbias, dsb = _g().dev(d["inp"]), _g().dev(d["bias"]), _g().dev(d["scale_b"])
    torch = _torch()
    dD = torch.zeros((m, oc), dtype=torch.int8, device="cuda:0")
    p = _g().w8a8_params(dict(d, B=W), dsb)
    mod = _g()._mod
    cp = mod.ConvParams()
    ctypes.memmove(ctypes.byref(cp), ctypes.byref(conv), ctypes.sizeof(cp))
    _g().lib().fn("igemmclp", "run")(m, oc, K, din.data_ptr(), 0, 0, 0, Wp.data_ptr(), K, 0, None,
                                     0, dD.data_ptr(), oc, dbias.data_ptr(), -128, 127,
                                     ctypes.byref(cp), ctypes.byref(p))
    exp = T.oracle_igemmcl(d["inp"], W, d["bias"], -128, 127, conv, d["scale_a"], d["scale_b"],
                           oc, d["scale_d"], d["zp_d"])
    np.testing.assert_array_equal(dD.cpu().numpy(), exp)


# --------------------------------------------------------------------------------------------
# the reference's packed test drivers, replayed (quantized_gemm_test_runner.h:482-699)
# --------------------------------------------------------------------------------------------

def test_reference_tile_loop_clamp_i32_packed(gpu):
    """run_packed_clamp_i32_i8_gemm_test: pack A and B ([k, n] via b_pack), then one run per
    m_step x n_step tile with pointers from get_{a,b}_packed_offset(idx, 0, k, m or n) and
    get_{c,d}_offset."""
    m, n, k = 300, 200, 96
    A, B, C = T.gen_clamp(m, n, k, seed=9, with_c=True, lo=-50, hi=50)
    L = _g().lib()
    Ap = packed_i8("clampp", "run_a_pack", A, m, k)
    Bp = packed_i8("clampp", "run_b_pack", B, n, k)
    torch = _torch()
    dC = _g().dev(C)
    dD = torch.zeros((m, n), dtype=torch.int32, device="cuda:0")
    ms, ns = L.fn("clampp", "get_m_step")(), L.fn("clampp", "get_n_step")()
    for m_idx in range(0, m, ms):
        for n_idx in range(0, n, ns):
            am, an = min(m - m_idx, ms), min(n - n_idx, ns)
            a_off = L.fn("clampp", "get_a_packed_offset")(m_idx, 0, k, m)
            b_off = L.fn("clampp", "get_b_packed_offset")(n_idx, 0, k, n)
            c_off = L.fn("clampp", "get_c_offset")(m_idx, n_idx, n)
            d_off = L.fn("clampp", "get_d_offset")(m_idx, n_idx, n)
            L.fn("clampp", "run")(am, an, k, Ap.data_ptr() + a_off, k, 0, Bp.data_ptr() + b_off,
                                  k, 0, dC.data_ptr() + c_off, n, dD.data_ptr() + d_off, n,
                                  -100000, 100000)
    np.testing.assert_array_equal(dD.cpu().numpy(), T.oracle_clamp(A, B, C, -100000, 100000))


def test_reference_tile_loop_w8a8_packed(gpu):
    """run_packed_1xnbias_reqi32toi8_gemm_test: A via a_pack, B [n, k] via bt_pack, tiles
    through the offset getters, bias tile from get_bias_offset. The run reads scale_b for the
    columns of its own call, so each tile's params point scale_b at the tile's first column
    (the reference driver hands every tile the same params, which agrees only for a
    per-tensor scale; its 1.0 tolerance after dequantization absorbs the rest)."""
    m, n, k = 150, 260, 128
    d = T.gen_w8a8(m, n, k, seed=21)
    L = _g().lib()
    Ap = packed_i8("w8a8p", "run_a_pack", d["A"], m, k)
    Bp = packed_i8("w8a8p", "run_bt_pack", d["B"], n, k)
    dbias, dsb = _g().dev(d["bias"]), _g().dev(d["scale_b"])
    torch = _torch()
    dD = torch.zeros((m, n), dtype=torch.int8, device="cuda:0")
    ms, ns = L.fn("w8a8p", "get_m_step")(), L.fn("w8a8p", "get_n_step")()
    for m_idx in range(0, m, ms):
        for n_idx in range(0, n, ns):
            am, an = min(m - m_idx, ms), min(n - n_idx, ns)
            # per-tile params: scale_b advanced to the tile's first column
            p = _g().w8a8_params(d, dsb)
            p.scale_b = dsb.data_ptr() + 4 * n_idx
            a_off = L.fn("w8a8p", "get_a_packed_offset")(m_idx, 0, k, m)
            b_off = L.fn("w8a8p", "get_b_packed_offset")(n_idx, 0, k, n)
            bias_off = L.fn("w8a8p", "get_bias_offset")(n_idx)
            d_off = L.fn("w8a8p", "get_d_offset")(m_idx, n_idx, n)
            L.fn("w8a8p", "run")(am, an, k, Ap.data_ptr() + a_off, k, 0, Bp.data_ptr() + b_off, k,
                                 0, None, n, dD.data_ptr() + d_off, n, dbias.data_ptr() + bias_off,
                                 -128, 127, ctypes.byref(p))
    exp = T.oracle_w8a8(d["A"], d["B"], None, d["bias"], -128, 127, d["scale_a"], d["scale_b"], n,
                        d["scale_d"], d["zp_d"])
    np.testing.assert_array_equal(dD.cpu().numpy(), exp)


@pytest.mark.parametrize("k1", [128, 40])
def test_k_split_sub_buffers_accumulate(gpu, k1):
    """K split at k1: both parts packed as sub-buffers of one ld_packed = K buffer (k_idx = 0
    and k_idx = k1, dst and src advanced as the reference's tail rule expects), D1 = A1 B1,
    then D = D1 + A2 B2 through C. k1 = 128 keeps every chunk aligned (MFMA path); k1 = 40 does
    not (generic path, tail panels shifted by 40 * (128 - w))."""
    m, n, k = 300, 200, 256
    A, B, C = T.gen_clamp(m, n, k, seed=k1, lo=-50, hi=50)
    L = _g().lib()
    dA, dBt = _g().dev(A), _g().dev(np.ascontiguousarray(B.T))
    Ap, Bp = dbuf(m * k), dbuf(n * k)
    ms, ns = L.fn("clampp", "get_m_step")(), L.fn("clampp", "get_n_step")()
    k2 = k - k1
    a2 = L.fn("clampp", "get_a_packed_offset")(0, k1, k, min(m, ms))
    b2 = L.fn("clampp", "get_b_packed_offset")(0, k1, k, min(n, ns))
    pack("clampp", "run_a_pack", m, k1, k, k, 0, dA, Ap)
    pack("clampp", "run_bt_pack", n, k1, k, k, 0, dBt, Bp)
    L.fn("clampp", "run_a_pack")(m, k2, k, k, k1, dA.data_ptr() + k1, Ap.data_ptr() + a2)
    L.fn("clampp", "run_bt_pack")(n, k2, k, k, k1, dBt.data_ptr() + k1, Bp.data_ptr() + b2)
    torch = _torch()
    D1 = torch.zeros((m, n), dtype=torch.int32, device="cuda:0")
    D = torch.zeros((m, n), dtype=torch.int32, device="cuda:0")
    big = 2 ** 31 - 1
    L.fn("clampp", "run")(m, n, k1, Ap.data_ptr(), k, 0, Bp.data_ptr(), k, 0, None, n,
                          D1.data_ptr(), n, -big - 1, big)
    L.fn("clampp", "run")(m, n, k2, Ap.data_ptr() + a2, k, k1, Bp.data_ptr() + b2, k, k1,
                          D1.data_ptr(), n, D.data_ptr(), n, -big - 1, big)
    np.testing.assert_array_equal(D.cpu().numpy(), T.oracle_clamp(A, B, None, -big - 1, big))
