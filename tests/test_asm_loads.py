"""No inline-asm vector load into a VGPR is touched before a wait covers it (CPU; needs hipcc).

Every torq-tile_amd/csrc/*.hip file is compiled to gfx950 device assembly with the library's own
flags, and tests/asm_load_check.py follows each kernel's control flow: an instruction that reads
or writes the destination register of an inline-asm load still in flight fails the test (the
compiler treats such a register as written at issue, so it may copy or reuse it early; a late
return then corrupts a value, as a memory-aperture fault once showed). The checker itself is
pinned on small listings with planted mistakes."""

import concurrent.futures
import glob
import os
import shutil
import subprocess

import pytest

import asm_load_check as C

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "torq-tile_amd")
HIPCC = "/opt/rocm/bin/hipcc"
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-Xclang",
         "-target-feature", "-Xclang", "-packed-fp32-ops", "-I../include", "-Icsrc",
         "--offload-device-only", "-S"]


def _listing(body):
    return "\n".join(["_Z4testv:", *body, ".Lfunc_end0:"])


GOOD = [
    ";;#ASMSTART", "global_load_dwordx4 v[4:7], v[0:1], off", ";;#ASMEND",
    "global_load_dword v8, v[2:3], off",
    "s_waitcnt vmcnt(1)",
    "v_add_u32 v9, v4, v5",
    "s_endpgm",
]
# read before the covering wait (vmcnt(2) leaves the asm load in flight)
BAD_EARLY_READ = [
    ";;#ASMSTART", "global_load_dwordx4 v[4:7], v[0:1], off", ";;#ASMEND",
    "global_load_dword v8, v[2:3], off",
    "s_waitcnt vmcnt(2)",
    "v_mov_b32 v10, v6",
    "s_endpgm",
]
# the destination register reused by another value while the load is in flight
BAD_REUSE = [
    ";;#ASMSTART", "global_load_dword v4, v[0:1], off", ";;#ASMEND",
    "v_mov_b32 v4, 0",
    "s_waitcnt vmcnt(0)",
    "s_endpgm",
]
# covered on the fall-through path only: the branch target reads it first
BAD_BRANCH = [
    ";;#ASMSTART", "global_load_dword v4, v[0:1], off", ";;#ASMEND",
    "s_cbranch_scc1 .LBB0_2",
    "s_waitcnt vmcnt(0)",
    ".LBB0_2:",
    "v_add_u32 v5, v4, v4",
    "s_endpgm",
]
# a loop whose back edge brings the load (issued in the loop) around before its wait
BAD_LOOP = [
    ".LBB0_1:",
    "v_add_u32 v5, v4, 1",
    ";;#ASMSTART", "global_load_dword v4, v[0:1], off", ";;#ASMEND",
    "s_cbranch_scc1 .LBB0_1",
    "s_waitcnt vmcnt(0)",
    "s_endpgm",
]
# LDS-DMA writes no VGPR: its address register may be reused at once
LDS_DMA = [
    ";;#ASMSTART", "global_load_lds_dwordx4 v[0:1], off", ";;#ASMEND",
    "v_mov_b32 v0, 0",
    "s_endpgm",
]


def test_checker_pins():
    good, n = C.check_asm(_listing(GOOD))
    assert n == 1 and good == {"_Z4testv": []}
    for bad in (BAD_EARLY_READ, BAD_REUSE, BAD_BRANCH, BAD_LOOP):
        res, n = C.check_asm(_listing(bad))
        assert n == 1 and len(res["_Z4testv"]) >= 1, bad
    res, n = C.check_asm(_listing(LDS_DMA))
    assert n == 0 and res == {"_Z4testv": []}


def _compile(src, out_dir):
    out = os.path.join(out_dir, os.path.basename(src)[:-4] + ".s")
    subprocess.run([HIPCC, *FLAGS, "-o", out, src], cwd=PKG, check=True,
                   stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    return src, out


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_no_asm_load_register_touched_in_flight(tmp_path):
    srcs = sorted(glob.glob(os.path.join(PKG, "csrc", "*.hip")))
    assert srcs
    bad = []
    total = 0
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        for src, out in ex.map(lambda s: _compile(s, str(tmp_path)), srcs):
            with open(out) as f:
                res, n = C.check_asm(f.read())
            total += n
            for kern, v in res.items():
                for ld, line, text in v[:4]:
                    bad.append("%s %s: load at line %d, %s at line %d" % (
                        os.path.basename(src), kern[:60], ld, text, line))
    print("inline-asm VGPR loads checked: %d" % total)
    assert not bad, "\n".join(bad[:20])
    shutil.rmtree(str(tmp_path), ignore_errors=True)
