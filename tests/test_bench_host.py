"""Host logic of bench.py that needs no GPU: which bench leg each product kernel's counters are
attributed to (the HBM traffic and counter summaries sum per leg by demangled kernel name), and
the launch shapes the empty-launch floors use."""

import os
import sys

import pytest

sys.path.insert(0, os.path.join(os.path.dirname(__file__), ".."))
import bench  # noqa: E402

NS = "tqt::(anonymous namespace)::"


@pytest.mark.parametrize("name,leg", [
    ("void %sconv_halo_kernel<0>(%sInt8Args, %sHaloPlan)" % (NS, NS, NS), "conv"),
    ("void %sconv_halo_kernel<2>(%sInt8Args, %sHaloPlan)" % (NS, NS, NS), "conv"),
    ("void %sint8_stream_kernel<128, 1, 0, true>(%sInt8Args, int, int, int)" % (NS, NS), "conv"),
    ("void %sint8_stream_kernel<64, 1, 0, false>(%sInt8Args, int, int, int)" % (NS, NS), "w8a8"),
    ("void %sw4a8_mfma_kernel<1, 0, 0>(%sW4A8Args)" % (NS, NS), "w4a8"),
    ("void %sw4a8_strip_kernel<2, 0>(%sW4A8Args)" % (NS, NS), "w4a8"),
    # the fused decode step is not one of the traffic legs
    ("void %sw4a8_qstrip_kernel<2, 0>(%sW4A8Args, float const*, signed char*, float*, int*)"
     % (NS, NS), None),
    ("void %sw4a16_chunk_kernel<0, 1, 3>(%sW4A16Args, int)" % (NS, NS), "w4a16"),
    ("void at::native::vectorized_elementwise_kernel<4, at::native::bitwise_not_kernel_cuda>",
     "copy"),
    ("void %squantize_qai8dx_kernel(float const*)" % NS, None),
])
def test_leg_of_kernel(name, leg):
    assert bench.leg_of_kernel(name) == leg


def test_launch_shapes_mi355x():
    """The launch shapes at the bench configurations on 256 CUs: W4A8 strip kernel 11008 / 16
    workgroups of 4 waves; W4A16 chunk kernel one 1024-thread workgroup per CU (896 tiles need
    224) with its 3 x 50 KiB ring; igemmcl halo kernel 196 tiles rounded up to the 8 XCDs (200)
    with 152 KiB + 1 KiB of LDS."""
    shapes = bench.launch_shapes(256)
    assert shapes == {
        "w4a8 strip (M=1)": (688, 256, 0),
        "w4a16 chunk": (256, 1024, 153600),
        "igemmcl halo": (200, 512, 156672),
    }
    # fewer CUs than W4A16 workgroups needed: one per 64 channels
    assert bench.launch_shapes(200)["w4a16 chunk"][0] == 224
