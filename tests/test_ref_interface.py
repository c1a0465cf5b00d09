"""The drop-in boundary checked against the reference's own headers (CPU only).

For every `include/tqt_<type>_interface.h` of this build, the reference's interface header of the
same name (`/root/reference/src/.../tqt_<type>_interface.h`) is compiled in place, as C, with
this build's `tqt_<type>_mfma_gfx950.h` prototypes on top of it (as C++: the reference's
`tqt_conv.h` holds templates, and its library is C++ with C linkage):

  * the reference's `struct tqt_<type>_ukernel` is filled positionally, in the reference's member
    order, with the gfx950 functions (`tqt_<member>_<type>_mfma_gfx950`) -- a missing function,
    a member out of order or a prototype that differs from the reference's typedef fails to
    compile;
  * the reference struct and this build's struct have the same size and every member sits at
    the same offset (compile-time asserts in two translation units, one per header);
  * every member's typedef name in this build's header is the reference's name;
  * the parameter structs (`tqt_params_i8_i8.h`, `tqt_params_i8_i4.h`, `tqt_conv.h`) have the
    same size, field offsets and field types as this build's `tqt_gfx950_common.h`.

Skipped where the reference tree is absent (the GPU box). Reference headers are only compiled
here, never copied.
"""

import glob
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
REF = "/root/reference"
V = "_mfma_gfx950"
CXX = next((c for c in ("/opt/rocm/llvm/bin/clang++", shutil.which("clang++") or "") if c and
            os.path.exists(c)), None)

pytestmark = [
    pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src")),
                       reason="reference tree not present (only in the build container)"),
    pytest.mark.skipif(CXX is None, reason="clang++ not found (needed for _Float16 / __bf16)"),
]

CXXFLAGS = ["-x", "c++", "-std=c++17", "-Wall", "-Werror", "-Wno-unused-variable",
            "-Wno-unused-const-variable", "-fsyntax-only"]


def repo_types():
    out = []
    for h in sorted(glob.glob(os.path.join(INC, "tqt_*_interface.h"))):
        out.append(os.path.basename(h)[len("tqt_"):-len("_interface.h")])
    return out


def ref_header(t):
    hits = glob.glob(os.path.join(REF, "src", "**", "tqt_%s_interface.h" % t), recursive=True)
    assert len(hits) == 1, (t, hits)
    return os.path.relpath(hits[0], REF)


def strip_comments(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def struct_members(text, t):
    """[(typedef_name, member_name)] of struct tqt_<t>_ukernel in header text."""
    m = re.search(r"struct\s+tqt_%s_ukernel\s*\{(.*?)\}\s*;" % re.escape(t), strip_comments(text),
                  re.S)
    assert m, "no struct tqt_%s_ukernel" % t
    return re.findall(r"(\w+)\s+(\w+)\s*;", m.group(1))


def compile_cxx(src, tmp, name, extra=()):
    path = os.path.join(tmp, name)
    with open(path, "w") as fh:
        fh.write(src)
    r = subprocess.run([CXX] + CXXFLAGS + list(extra) + [path], capture_output=True, text=True)
    return r.returncode, r.stderr


def function_name(member, t):
    """The gfx950 function a ukernel member binds: tqt_<member>_<type>_mfma_gfx950, where a gemm
    type's run_gemm member is tqt_run_<type> (the type name already starts with gemm_)."""
    if member == "run_gemm" and t.startswith("gemm_"):
        return "tqt_run_%s%s" % (t, V)
    return "tqt_%s_%s%s" % (member, t, V)


TYPES = repo_types()


def test_every_repo_interface_has_a_reference_counterpart():
    assert len(TYPES) == 29
    for t in TYPES:
        ref_header(t)


@pytest.mark.parametrize("t", TYPES)
def test_reference_ukernel_binds_gfx950_variant(t, tmp_path):
    ref_rel = ref_header(t)
    ref_members = struct_members(open(os.path.join(REF, ref_rel)).read(), t)
    repo_members = struct_members(open(os.path.join(INC, "tqt_%s_interface.h" % t)).read(), t)
    # same typedef names and member names, in the same order
    assert repo_members == ref_members

    n = len(ref_members)
    inits = ",\n    ".join(function_name(mem, t) for _, mem in ref_members)
    asserts = "\n".join(
        "static_assert(offsetof(struct tqt_%s_ukernel, %s) == %d * sizeof(void (*)(void)), "
        "\"%s\");" % (t, mem, i, mem) for i, (_, mem) in enumerate(ref_members))
    size_assert = ("static_assert(sizeof(struct tqt_%s_ukernel) == %d * sizeof(void (*)(void)), "
                   "\"size\");" % (t, n))
    # (1) reference interface header + this build's prototypes (the reference's types stand in
    #     for tqt_gfx950_common.h's, whose guard is pre-defined). tqt_common.h comes first: some
    #     reference interface headers use its float16_t without including it.
    src_ref = """#include <stddef.h>
#include <type_traits>
#include "src/common/tqt_common.h"
#include "%s"
#define TQT_GFX950_COMMON_H 1
#include "tqt_%s%s.h"
static const struct tqt_%s_ukernel uk = {
    %s
};
%s
%s
""" % (ref_rel, t, V, t, inits, asserts, size_assert)
    rc, err = compile_cxx(src_ref, str(tmp_path), "ref_%s.cpp" % t, ["-I" + REF, "-I" + INC])
    assert rc == 0, err
    # (2) this build's interface header + prototypes: same layout, typedefs match the functions
    typed = "\n".join(
        "static_assert(std::is_same<%s, decltype(((struct tqt_%s_ukernel *)0)"
        "->%s)>::value, \"%s\");" % (td, t, mem, mem) for td, mem in ref_members)
    src_repo = """#include <stddef.h>
#include <type_traits>
#include "tqt_%s_interface.h"
#include "tqt_%s%s.h"
static const struct tqt_%s_ukernel uk = {
    %s
};
%s
%s
%s
""" % (t, t, V, t, inits, asserts, size_assert, typed)
    rc, err = compile_cxx(src_repo, str(tmp_path), "repo_%s.cpp" % t, ["-I" + INC])
    assert rc == 0, err


PARAM_STRUCTS = {
    "struct tqt_qai8_qai8_qsi8cx_params": (
        "src/gemm/gemm_i8_i8/tqt_params_i8_i8.h",
        ["scale_a", "zero_point_a", "scale_b", "quant_channel_b", "scale_d", "zero_point_d"]),
    "struct tqt_qai8_qsi8dx_qai8_params": (
        "src/gemm/gemm_i8_i8/tqt_params_i8_i8.h",
        ["scale_a", "quant_channel_a", "scale_b", "zero_point_b", "scale_d", "zero_point_d"]),
    "struct tqt_qai8dxp_qsi8cxp_params": (
        "src/gemm/gemm_i8_i8/tqt_params_i8_i8.h", ["scale_a", "zero_point_a", "scale_b"]),
    "struct tqt_qai8dx_qsi4cx_params": (
        "src/gemm/gemm_i8_i4/tqt_params_i8_i4.h", ["scale_a", "zero_point_a", "scale_b"]),
    "struct tqt_conv_params": (
        "src/common/tqt_conv.h",
        ["input_shape", "output_shape", "kernel_shape", "stride", "dilation", "pad",
         "input_channel", "output_channel", "groups"]),
}


TYPE_NAMES = ["float", "int32_t", "size_t", "float *", "int32_t *", "const float *",
              "const int32_t *", "size_t[3]"]


def layout_program(includes):
    """C++ source printing, per param struct, its size and each field's offset, size and type."""
    prog = ["#include <stdio.h>", "#include <stddef.h>", "#include <stdint.h>"]
    prog += ['#include "%s"' % h for h in includes]
    prog.append("template <typename T> const char *tn() { return \"?\"; }")
    for ty in TYPE_NAMES:
        prog.append('template <> const char *tn<%s>() { return "%s"; }' % (ty, ty))
    prog.append("int main() {")
    for s, (_, fields) in PARAM_STRUCTS.items():
        prog.append('printf("%s %%zu\\n", sizeof(%s));' % (s, s))
        for f in fields:
            prog.append('printf("%s.%s %%zu %%zu %%s\\n", offsetof(%s, %s), sizeof(((%s *)0)->%s), '
                        'tn<decltype(((%s *)0)->%s)>());' % (s, f, s, f, s, f, s, f))
    prog.append("return 0; }")
    return "\n".join(prog) + "\n"


def run_layout(tmp, name, includes, incdir):
    src = os.path.join(tmp, name + ".cpp")
    exe = os.path.join(tmp, name)
    with open(src, "w") as fh:
        fh.write(layout_program(includes))
    r = subprocess.run([CXX, "-std=c++17", "-I" + incdir, src, "-o", exe], capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stderr
    return subprocess.run([exe], capture_output=True, text=True, check=True).stdout


def test_param_structs_match_reference_layout(tmp_path):
    """Every param struct's size, and each field's offset, size and type, as the reference's
    headers lay them out (one program built on theirs, one on ours, outputs compared)."""
    ref = run_layout(str(tmp_path), "ref_params", sorted({h for h, _ in PARAM_STRUCTS.values()}),
                     REF)
    ours = run_layout(str(tmp_path), "repo_params", ["tqt_gfx950_common.h"], INC)
    assert "?" not in ref.split()
    assert ours == ref
