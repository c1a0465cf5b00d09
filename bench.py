#!/usr/bin/env python3
"""Benchmark of the gfx950 TORQ-Tile quantized micro-kernels on one MI355X.

Headline (BASELINE.json metric "W4A8 GEMV HBM GB/s (M=1) + W8A8 GEMM int8 TOPS (M=512),
% roofline"):
  * value   = W8A8 GEMM int8 TOPS on configs[1] (gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt,
              M=512, K=4096, N=4096), with its MFMA roofline;
  * w4a8    = W4A8 decode GEMV HBM GB/s on configs[2] at M=1 (K=4096, N=11008), with its HBM
              roofline; M=4 and M=8 are reported beside it.
The remaining configurations (int8->int32 GEMM, W4A16, int8 implicit-GEMM conv), the packed
siblings of W8A8, W4A8, W4A16 and igemmcl on the same shapes (operands packed by the library's packers
before timing), and the W4A8 decode step with its activation quantization on the GPU, are timed
the same way and reported under "configs".

A step is one launch of the kernel over one batch of synthetic inputs already resident in
HBM. Each launch reads a different copy of the weights (and activations): the copies together
exceed the 256 MB Infinity Cache, so the GB/s figures are HBM figures. Kernel time comes from
HIP events recorded on the stream the kernels are launched on, around exactly `--steps`
back-to-back launches after `--warmup` untimed ones; the timed launches are captured into one
HIP graph and replayed (`--no-graphs`: issued one by one; the headline legs report both).

cpu_baseline: the portable C restatement of the reference kernel (oracle/, the same tile loop
the reference runs with VLENB = 16), timed on this host's cores over a bounded sample.
"""

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA
F16_PEAK_TFLOPS = 2500.0     # MI355X dense fp16 MFMA
CACHE_BYTES = 256 << 20      # Infinity Cache (MALL)

W8A8 = dict(m=512, n=4096, k=4096)
W4A8 = dict(m=1, n=11008, k=4096)
W4A16 = dict(m=32, n=14336, k=4096, bl=32)
CONV = dict(ID=8, IH=56, IW=56, IC=128, OC=128, KH=3, KW=3, pad=1)
CLAMP = dict(m=64, n=256, k=512)
# W4A8 M=1 algorithmic bytes: B n*k/2 + scale_b 4n + bias 4n + A m*k + 8m + D 4mn
W4A8_BYTES = 11008 * 4096 // 2 + 8 * 11008 + 4096 + 8 + 4 * 11008


def load_lib():
    import importlib.util

    spec = importlib.util.spec_from_file_location(
        "tqt_gfx950", os.path.join(ROOT, "torq-tile_amd", "tqt_gfx950.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod, mod.load()


def copies_for(bytes_per_copy):
    return max(2, int(math.ceil(1.25 * CACHE_BYTES / max(1, bytes_per_copy))) + 1)


class Timer:
    """HIP events on the launch stream around exactly `steps` launches.

    Default: the `steps` launches (each on its own weight copy) are captured once into a HIP
    graph and the graph is replayed between the two events, so the figure is the kernels'
    back-to-back cost without per-launch host overhead. `stream_ms` also times the same launches
    issued one by one on the stream.

    Cache state: right before the start event, a kernel reads a buffer of twice the Infinity
    Cache (MALL), so no timed launch finds a copy that warm-up or an earlier replay left in the
    MALL or an L2 (a read, so no dirty lines are left whose write-back the timed launches would
    pay); inside the timed region a copy is read again only after `copies` launches, which
    together read more than the MALL holds (copies_for)."""

    def __init__(self, torch, stream, graphs=True):
        self.torch = torch
        self.stream = stream
        self.graphs = graphs
        self.sup = load_support()
        self.flush_buf = torch.zeros(2 * CACHE_BYTES, dtype=torch.uint8, device="cuda")
        self.flush_sink = torch.zeros(2 * CACHE_BYTES // (8 * 4096), dtype=torch.int32,
                                      device="cuda")

    def flush(self):
        """Read (not write) 2x the MALL on the timing stream: evicts the operands from the MALL
        and the L2s and leaves no dirty lines whose write-back the timed launches would pay."""
        if self.sup.tqtb_read_floor_async(self.flush_buf.data_ptr(), self.flush_buf.numel(),
                                          self.flush_sink.data_ptr(), self.flush_sink.numel(), 8,
                                          self.stream.cuda_stream):
            raise RuntimeError("cache flush launch failed")

    def _events(self):
        torch = self.torch
        return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def stream_ms(self, launch, copies, warmup, steps):
        torch = self.torch
        for i in range(warmup):
            launch(i % copies)
        torch.cuda.synchronize()
        self.flush()
        start, end = self._events()
        start.record(self.stream)
        for i in range(steps):
            launch((warmup + i) % copies)
        end.record(self.stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps  # ms per launch

    def run(self, launch, copies, warmup, steps):
        if not self.graphs:
            return self.stream_ms(launch, copies, warmup, steps)
        torch = self.torch
        for i in range(warmup):
            launch(i % copies)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=self.stream):
            for i in range(steps):
                launch((warmup + i) % copies)
        graph.replay()  # untimed: first replay uploads the graph
        torch.cuda.synchronize()
        self.flush()
        start, end = self._events()
        start.record(self.stream)
        graph.replay()
        end.record(self.stream)
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / steps
        del graph
        return ms  # ms per launch


# ------------------------------------------------------------------------------------------
# Synthetic inputs (BASELINE.json recipes; numpy only, seeded)
# ------------------------------------------------------------------------------------------

def inputs_w8a8(rng, m, n, k):
    zp_a = int(rng.integers(-20, 21))
    x = rng.standard_normal((m, k), dtype=np.float32)
    A = np.clip(np.rint(x / np.float32(0.02)) + zp_a, -128, 127).astype(np.int8)
    B = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    scale_b = rng.uniform(0.001, 0.01, size=n).astype(np.float32)
    bias = rng.integers(-1000, 1001, size=n).astype(np.int64)
    fused = (bias - zp_a * B.astype(np.int64).sum(axis=1)).astype(np.int32)
    return A, B, scale_b, fused, zp_a


def inputs_w4a8(rng, m, n, k):
    Af = rng.standard_normal((m, k), dtype=np.float32)
    fmax = np.maximum(Af.max(axis=1), 0).astype(np.float32)
    fmin = np.minimum(Af.min(axis=1), 0).astype(np.float32)
    s = ((fmax - fmin) / np.float32(255.0)).astype(np.float32)
    zp = np.clip(np.rint(np.float32(-128.0) - fmin / s), -128, 127).astype(np.int32)
    A = np.clip(np.rint(Af / s[:, None]) + zp[:, None], -128, 127).astype(np.int8)
    Bp = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    sb = rng.uniform(0.005, 0.02, size=n).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float32)
    return A, Bp, s, zp, sb, bias


# ------------------------------------------------------------------------------------------
# Per-config measurements
# ------------------------------------------------------------------------------------------

def pack_dev(torch, lib, kind, action, rows, k, src, nbytes):
    """One packed copy of `src` (device tensor) by the library's packer (synchronous)."""
    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    lib.fn(kind, action)(rows, k, k, k, 0, src.data_ptr(), dst.data_ptr())
    return dst


def bench_w8a8(torch, mod, lib, timer, warmup, steps, rng, packed=False):
    """packed: the qai8_qai8p_qsi8cxp sibling on the same inputs, A and B packed once by the
    library's packers before timing."""
    m, n, k = W8A8["m"], W8A8["n"], W8A8["k"]
    A, B, sb, bias, zp_a = inputs_w8a8(rng, m, n, k)
    per_copy = A.nbytes + B.nbytes
    nc = copies_for(per_copy)
    dA = [torch.from_numpy(A).cuda()]
    dB = [torch.from_numpy(B).cuda()]
    if packed:
        dA = [pack_dev(torch, lib, "w8a8p", "run_a_pack", m, k, dA[0], A.nbytes)]
        dB = [pack_dev(torch, lib, "w8a8p", "run_bt_pack", n, k, dB[0], B.nbytes)]
    for _ in range(nc - 1):
        dA.append(dA[0].clone())
        dB.append(dB[0].clone())
    dsb = torch.from_numpy(sb).cuda()
    dbias = torch.from_numpy(bias).cuda()
    dD = torch.empty((m, n), dtype=torch.int8, device="cuda")
    p = mod.QAI8QSI8CXParams(0.02, zp_a, dsb.data_ptr(), n, 0.05, 0)
    f = lib.fn("w8a8p" if packed else "w8a8", "run_async")
    s = timer.stream.cuda_stream

    def launch(i):
        f(m, n, k, dA[i].data_ptr(), k, 0, dB[i].data_ptr(), k, 0, None, n, dD.data_ptr(), n,
          dbias.data_ptr(), -128, 127, ctypes.byref(p), s)

    ms = timer.run(launch, nc, warmup, steps)
    ms_stream = timer.stream_ms(launch, nc, warmup, steps) if timer.graphs else ms
    ops = 2.0 * m * n * k
    algo_bytes = A.nbytes + B.nbytes + 4 * n + 4 * n + m * n
    tops = ops / (ms * 1e-3) / 1e12
    return dict(ms=ms, ms_stream=ms_stream, tops=tops, gbs=algo_bytes / (ms * 1e-3) / 1e9, ops=ops,
                bytes=algo_bytes, copies=nc, inputs=(A, B, sb, bias, zp_a))


def bench_w4a8(torch, mod, lib, timer, warmup, steps, rng, m, packed=False, dynq=False):
    """packed: the qai8dxp_qsi4cxp sibling on the same inputs (packed once before timing).
    dynq: each step is the decode step "quantize the f32 activations on the GPU, then the W4A8
    GEMV": "fused" through tqt_run_quantize_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_gfx950 (one
    launch at M = 1), any other true value as the two launches (tqt_run_quantize_qai8dx_f32_gfx950
    + the W4A8 run), both on the stream."""
    n, k = W4A8["n"], W4A8["k"]
    A, Bp, sa, za, sb, bias = inputs_w4a8(rng, m, n, k)
    nc = copies_for(Bp.nbytes)
    dB = [torch.from_numpy(Bp).cuda()]
    dA0 = torch.from_numpy(A).cuda()
    if packed:
        dB = [pack_dev(torch, lib, "w4a8p", "run_bt_pack", n, k, dB[0], Bp.nbytes)]
        dA0 = pack_dev(torch, lib, "w4a8p", "run_a_pack", m, k, dA0, A.nbytes)
    for _ in range(nc - 1):
        dB.append(dB[0].clone())
    dA = [dA0.clone() for _ in range(nc)]
    dsa, dza, dsb = (torch.from_numpy(x).cuda() for x in (sa, za, sb))
    dbias = torch.from_numpy(bias).cuda()
    dD = torch.empty((m, n), dtype=torch.float32, device="cuda")
    p = mod.QAI8DXQSI4CXParams(dsa.data_ptr(), dza.data_ptr(), dsb.data_ptr())
    f = lib.fn("w4a8p" if packed else "w4a8", "run_async")
    s = timer.stream.cuda_stream
    if dynq:
        Af = rng.standard_normal((m, k), dtype=np.float32)
        dAf = [torch.from_numpy(Af).cuda() for _ in range(nc)]

    def launch(i):
        if dynq == "fused":
            lib.quantize_gemm_async(m, n, k, dAf[i].data_ptr(), k, dA[i].data_ptr(), k,
                                    dsa.data_ptr(), dza.data_ptr(), dB[i].data_ptr(), k, None, n,
                                    dD.data_ptr(), n, dbias.data_ptr(), -math.inf, math.inf,
                                    dsb.data_ptr(), s)
            return
        if dynq:
            lib.quantize_async(m, k, dAf[i].data_ptr(), k, dA[i].data_ptr(), k, dsa.data_ptr(),
                               dza.data_ptr(), s)
        f(m, n, k, dA[i].data_ptr(), k, 0, dB[i].data_ptr(), k, 0, None, n, dD.data_ptr(), n,
          dbias.data_ptr(), -math.inf, math.inf, ctypes.byref(p), s)

    ms = timer.run(launch, nc, warmup, steps)
    ms_stream = timer.stream_ms(launch, nc, warmup, steps) if timer.graphs else ms
    # B n*k/2 + scale_b 4n + bias 4n + A m*k + scale_a/zp_a 8m + D 4mn (+ the f32 A the
    # quantization reads, 4mk, when it runs in the step)
    algo_bytes = n * k // 2 + 4 * n + 4 * n + m * k + 8 * m + 4 * m * n + (4 * m * k if dynq else 0)
    return dict(ms=ms, ms_stream=ms_stream, gbs=algo_bytes / (ms * 1e-3) / 1e9, bytes=algo_bytes,
                ops=2.0 * m * n * k, copies=nc, inputs=(A, Bp, sa, za, sb, bias))


def load_support():
    """libtqt_bench_support.so: the read-floor kernel and the W4A16 forwarders that take the f16
    clamp bounds as bit patterns (ctypes cannot pass _Float16 by value)."""
    path = os.path.join(ROOT, "torq-tile_amd", "libtqt_bench_support.so")
    if not os.path.exists(path):
        raise RuntimeError("bench support library not built: %s (make -C torq-tile_amd)" % path)
    sup = ctypes.CDLL(path)
    sz, vp = ctypes.c_size_t, ctypes.c_void_p
    sup.tqtb_read_floor_async.restype = ctypes.c_int
    sup.tqtb_read_floor_async.argtypes = [vp, sz, vp, sz, ctypes.c_int, vp]
    sup.tqtb_stream_floor_async.restype = ctypes.c_int
    sup.tqtb_stream_floor_async.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, vp, sz, vp]
    sup.tqtb_empty_async.restype = ctypes.c_int
    sup.tqtb_empty_async.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp]
    sup.tqtb_stream_lds_bytes.restype = ctypes.c_int
    sup.tqtb_stream_lds_bytes.argtypes = []
    sup.tqtb_run_w4a16_async.restype = None
    sup.tqtb_run_w4a16_async.argtypes = ([sz] * 4 + [vp, sz, vp, sz, vp, sz, vp, sz, vp, sz, vp,
                                                    ctypes.c_uint16, ctypes.c_uint16, vp])
    sup.tqtb_run_w4a16p_async.restype = None
    sup.tqtb_run_w4a16p_async.argtypes = sup.tqtb_run_w4a16_async.argtypes
    return sup


def bench_w4a16(torch, mod, lib, timer, warmup, steps, rng, packed=False):
    """packed: the f16p_qsi4c2p sibling on the same inputs (packed once before timing)."""
    m, n, k, bl = W4A16["m"], W4A16["n"], W4A16["k"], W4A16["bl"]
    A = rng.standard_normal((m, k)).astype(np.float16)
    Bp = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    S = rng.uniform(0.005, 0.02, size=(n, k // bl)).astype(np.float16)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float16)
    nc = copies_for(Bp.nbytes + S.nbytes)
    dB = [torch.from_numpy(Bp).cuda()]
    dS = [torch.from_numpy(S).cuda()]
    dA = torch.from_numpy(A).cuda()
    if packed:
        dB = [pack_dev(torch, lib, "w4a16p", "run_bt_pack", n, k, dB[0], Bp.nbytes)]
        dA = pack_dev(torch, lib, "w4a16p", "run_a_pack", m, k, dA, A.nbytes)
    for _ in range(nc - 1):
        dB.append(dB[0].clone())
        dS.append(dS[0].clone())
    dbias = torch.from_numpy(bias).cuda()
    dD = torch.empty((m, n), dtype=torch.float16, device="cuda")
    sup = load_support()
    f = sup.tqtb_run_w4a16p_async if packed else sup.tqtb_run_w4a16_async
    cmin = int(np.float16(-65504.0).view(np.uint16))
    cmax = int(np.float16(65504.0).view(np.uint16))
    s = timer.stream.cuda_stream

    def launch(i):
        f(m, n, k, bl, dA.data_ptr(), k, dB[i].data_ptr(), k, dS[i].data_ptr(), k // bl, None, n,
          dD.data_ptr(), n, dbias.data_ptr(), cmin, cmax, s)

    ms = timer.run(launch, nc, warmup, steps)
    algo_bytes = Bp.nbytes + S.nbytes + A.nbytes + bias.nbytes + 2 * m * n
    flops = 2.0 * m * n * k
    return dict(ms=ms, gbs=algo_bytes / (ms * 1e-3) / 1e9, tflops=flops / (ms * 1e-3) / 1e12,
                bytes=algo_bytes, ops=flops, copies=nc)


FLOOR_LOADS = (1, 2, 4, 8, 16)


def bench_floor(torch, timer, warmup, steps, nbytes):
    """Single-launch HBM read floor for `nbytes` (the W4A8 M=1 operand bytes): one launch of a
    plain streaming read per step (each workgroup reads loads x 4 KiB contiguous, all its loads
    issued at once), over rotating copies like the kernel legs, for each per-lane load count in
    FLOOR_LOADS; the fastest is the floor."""
    sup = load_support()
    nbytes = (nbytes + 15) // 16 * 16
    nc = copies_for(nbytes)
    src = [torch.zeros(nbytes, dtype=torch.uint8, device="cuda") for _ in range(nc)]
    sink_words = nbytes // 4096 + 1
    sink = torch.zeros(sink_words, dtype=torch.int32, device="cuda")
    s = timer.stream.cuda_stream
    per_loads = {}
    for loads in FLOOR_LOADS:
        def launch(i, loads=loads):
            if sup.tqtb_read_floor_async(src[i].data_ptr(), nbytes, sink.data_ptr(), sink_words,
                                         loads, s):
                raise RuntimeError("read floor launch failed")

        per_loads[loads] = timer.run(launch, nc, warmup, steps)
    best = min(per_loads, key=per_loads.get)
    ms = per_loads[best]
    return dict(ms=ms, gbs=nbytes / (ms * 1e-3) / 1e9, bytes=nbytes, copies=nc, loads=best,
                us_by_loads={b: round(v * 1e3, 3) for b, v in per_loads.items()})


def bench_stream_floor(torch, timer, warmup, steps, resident=False):
    """The W8A8 stream kernel's load schedule alone (tqtb_stream_floor_async: same grid, tile
    order, LDS-DMA roles, four-slot ring, waits and barriers; no MFMA, no epilogue) on cfg 2's
    A and B: the per-CU L2 -> LDS stream floor of that kernel's shape. Cold: rotating copies
    like the W8A8 leg; resident: every workgroup reads the first tile's 192 rows (768 KiB, held
    in each XCD's L2 after first touch)."""
    sup = load_support()
    m, n, k = W8A8["m"], W8A8["n"], W8A8["k"]
    nc = 1 if resident else copies_for((m + n) * k)
    dA = [torch.zeros((m, k), dtype=torch.int8, device="cuda") for _ in range(nc)]
    dB = [torch.zeros((n, k), dtype=torch.int8, device="cuda") for _ in range(nc)]
    sink_words = 8 * ((m // 64) * (n // 128) // 8 + 1)
    sink = torch.zeros(sink_words, dtype=torch.int32, device="cuda")
    s = timer.stream.cuda_stream

    def launch(i):
        if sup.tqtb_stream_floor_async(dA[i].data_ptr(), dB[i].data_ptr(), m, n, k,
                                       1 if resident else 0, sink.data_ptr(), sink_words, s):
            raise RuntimeError("stream floor launch failed")

    ms = timer.run(launch, nc, warmup, steps)
    per_cu = (64 + 128) * k
    return dict(ms=ms, bytes=per_cu, copies=nc, per_cu_bytes=per_cu,
                per_cu_gbs=per_cu / (ms * 1e-3) / 1e9)


def bench_empty(torch, timer, warmup, steps, blocks=256, threads=512, lds=None):
    """An empty kernel with a kernel's launch shape (default: the W8A8 stream kernel's, 256
    workgroups of 512 threads and its LDS size): the per-launch cost of that shape in a graph."""
    sup = load_support()
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    if lds is None:
        lds = sup.tqtb_stream_lds_bytes() + 1536  # the ring and the multiplier arrays
    s = timer.stream.cuda_stream

    def launch(i):
        if sup.tqtb_empty_async(blocks, threads, lds, sink.data_ptr(), s):
            raise RuntimeError("empty launch failed")

    ms = timer.run(launch, 1, warmup, steps)
    return dict(ms=ms, bytes=0, copies=1)


def launch_shapes(cus):
    """Grid, block and LDS bytes of the other headline kernels at their configurations, as the
    library launches them: the W4A8 strip kernel (4 waves of 4 channels per workgroup, no LDS),
    the W4A16 chunk kernel (at most one 1024-thread workgroup per CU, a three-slot ring of
    50 KiB chunks) and the igemmcl halo kernel (256 pixels x 64 channels per workgroup, 152 KiB
    of halo and weights plus four 64-entry epilogue arrays). cus: the GPU's CU count."""
    w4a16_tiles = (W4A16["n"] + 15) // 16
    w4a16_wgs = max((w4a16_tiles + 3) // 4, min(w4a16_tiles, cus))
    conv_px = CONV["ID"] * CONV["IH"] * CONV["IW"]
    return {
        "w4a8 strip (M=1)": ((W4A8["n"] + 15) // 16, 256, 0),
        "w4a16 chunk": (w4a16_wgs, 1024, 3 * (32768 + 16384 + 2048)),
        "igemmcl halo": (8 * ((((conv_px + 255) // 256) * (CONV["OC"] // 64) + 7) // 8), 512,
                         152 * 1024 + 4 * 64 * 4),
    }


def bench_caller(torch, mod, lib, kind, reps=5):
    """The reference's caller pattern (test/common/quantized_gemm_test_runner.h:273-292,
    examples/gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_rvv/...rvv.cpp:194-210): walk the output in
    get_m_step() x get_n_step() tiles and call the synchronous run once per tile, with the
    tile's operands found by the offset getters (and the per-row / per-channel parameter arrays
    advanced to the tile, since a run indexes them from its own first row and column). kind:
    "w8a8" (cfg 2) or "w4a8" (cfg 3, M = 1). Host wall clock over whole GEMMs, warm operands;
    also the same tiles issued with the stream-ordered run and one synchronization per GEMM."""
    rng = np.random.default_rng(3)
    if kind == "w8a8":
        m, n, k = W8A8["m"], W8A8["n"], W8A8["k"]
        A, B, sb, bias, zp_a = inputs_w8a8(rng, m, n, k)
        dA, dB = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
        dsb, dbias = torch.from_numpy(sb).cuda(), torch.from_numpy(bias).cuda()
        dD = torch.empty((m, n), dtype=torch.int8, device="cuda")
    else:
        m, n, k = 1, W4A8["n"], W4A8["k"]
        A, Bp, sa, za, sb, bias = inputs_w4a8(rng, m, n, k)
        dA, dB = torch.from_numpy(A).cuda(), torch.from_numpy(Bp).cuda()
        dsa, dza = torch.from_numpy(sa).cuda(), torch.from_numpy(za).cuda()
        dsb, dbias = torch.from_numpy(sb).cuda(), torch.from_numpy(bias).cuda()
        dD = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ms_, ns_ = lib.fn(kind, "get_m_step")(), lib.fn(kind, "get_n_step")()
    a_off, b_off = lib.fn(kind, "get_a_offset"), lib.fn(kind, "get_b_offset")
    bias_off, d_off = lib.fn(kind, "get_bias_offset"), lib.fn(kind, "get_d_offset")
    tiles = []
    for mi in range(0, m, ms_):
        for ni in range(0, n, ns_):
            am, an = min(ms_, m - mi), min(ns_, n - ni)
            if kind == "w8a8":
                p = mod.QAI8QSI8CXParams(0.02, zp_a, dsb.data_ptr() + 4 * ni, n, 0.05, 0)
                args = (am, an, k, dA.data_ptr() + a_off(mi, 0, k), k, 0,
                        dB.data_ptr() + b_off(ni, 0, k), k, 0, None, n,
                        dD.data_ptr() + d_off(mi, ni, n), n, dbias.data_ptr() + bias_off(ni),
                        -128, 127)
            else:
                p = mod.QAI8DXQSI4CXParams(dsa.data_ptr() + 4 * mi, dza.data_ptr() + 4 * mi,
                                           dsb.data_ptr() + 4 * ni)
                args = (am, an, k, dA.data_ptr() + a_off(mi, 0, k), k, 0,
                        dB.data_ptr() + b_off(ni, 0, k), k, 0, None, n,
                        dD.data_ptr() + d_off(mi, ni, n), n, dbias.data_ptr() + bias_off(ni),
                        -math.inf, math.inf)
            tiles.append((args, p))
    run, run_async = lib.fn(kind, "run"), lib.fn(kind, "run_async")
    stream = torch.cuda.current_stream().cuda_stream

    def gemm_sync():
        for args, p in tiles:
            run(*args, ctypes.byref(p))

    def gemm_async():
        for args, p in tiles:
            run_async(*args, ctypes.byref(p), stream)
        torch.cuda.synchronize()

    out = {}
    for name, fn in (("sync", gemm_sync), ("async", gemm_async)):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        out[name] = (time.perf_counter() - t0) / reps
    return dict(ms=out["sync"] * 1e3, ms_async=out["async"] * 1e3, calls=len(tiles),
                m_step=ms_, n_step=ns_, bytes=0, copies=1)


def bench_conv(torch, mod, lib, timer, warmup, steps, rng, packed=False):
    """packed: the igemmcl...qsi8cxp sibling on the same inputs (weights packed once before
    timing)."""
    c = CONV
    ID, IH, IW, IC, OC, KH, KW, pad = (c["ID"], c["IH"], c["IW"], c["IC"], c["OC"], c["KH"],
                                       c["KW"], c["pad"])
    K = KH * KW * IC
    inp = rng.integers(-128, 128, size=(ID, IH, IW, IC), dtype=np.int8)
    W = rng.integers(-127, 128, size=(OC, K), dtype=np.int8)
    sb = rng.uniform(0.001, 0.01, size=OC).astype(np.float32)
    bias = (rng.integers(-1000, 1001, size=OC) - 3 * W.astype(np.int64).sum(axis=1)).astype(
        np.int32)
    conv = mod.conv_params((ID, IH, IW), (1, KH, KW), (1, 1, 1), (1, 1, 1), (0, pad, pad), IC, OC)
    M = conv.output_shape[0] * conv.output_shape[1] * conv.output_shape[2]
    nc = copies_for(inp.nbytes + W.nbytes)
    din = [torch.from_numpy(inp).cuda()]
    for _ in range(nc - 1):
        din.append(din[0].clone())
    dW = torch.from_numpy(W).cuda()
    if packed:
        dW = pack_dev(torch, lib, "igemmclp", "run_bt_pack", OC, K, dW, W.nbytes)
    dsb = torch.from_numpy(sb).cuda()
    dbias = torch.from_numpy(bias).cuda()
    dD = torch.empty((M, OC), dtype=torch.int8, device="cuda")
    p = mod.QAI8QSI8CXParams(0.02, 3, dsb.data_ptr(), OC, 0.05, 0)
    f = lib.fn("igemmclp" if packed else "igemmcl", "run_async")
    s = timer.stream.cuda_stream

    def launch(i):
        f(M, OC, K, din[i].data_ptr(), 0, 0, 0, dW.data_ptr(), K, 0, None, 0, dD.data_ptr(), OC,
          dbias.data_ptr(), -128, 127, ctypes.byref(conv), ctypes.byref(p), s)

    ms = timer.run(launch, nc, warmup, steps)
    ops = 2.0 * OC * M * K
    algo_bytes = inp.nbytes + W.nbytes + 4 * OC + 4 * OC + M * OC
    return dict(ms=ms, tops=ops / (ms * 1e-3) / 1e12, gbs=algo_bytes / (ms * 1e-3) / 1e9,
                bytes=algo_bytes, ops=ops, copies=nc)


def bench_clamp(torch, mod, lib, timer, warmup, steps, rng):
    m, n, k = CLAMP["m"], CLAMP["n"], CLAMP["k"]
    A = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    B = rng.integers(-128, 128, size=(k, n), dtype=np.int8)
    dA = torch.from_numpy(A).cuda()
    dB = torch.from_numpy(B).cuda()
    dD = torch.empty((m, n), dtype=torch.int32, device="cuda")
    f = lib.fn("clamp", "run_async")
    s = timer.stream.cuda_stream

    def launch(i):
        f(m, n, k, dA.data_ptr(), k, 0, dB.data_ptr(), n, 0, None, n, dD.data_ptr(), n,
          -2**31, 2**31 - 1, s)

    ms = timer.run(launch, 1, warmup, steps)
    ops = 2.0 * m * n * k
    return dict(ms=ms, tops=ops / (ms * 1e-3) / 1e12, bytes=A.nbytes + B.nbytes + 4 * m * n,
                ops=ops, copies=1)


def bench_copy(torch, timer, warmup, steps):
    """Plain streaming kernel of known traffic (bitwise_not over 256 MB of int32): reads and
    writes exactly `nbytes` each per launch; calibrates the FETCH_SIZE / WRITE_SIZE counters."""
    nbytes = 256 << 20
    src = torch.zeros(nbytes // 4, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)

    def launch(i):
        torch.bitwise_not(src, out=dst)

    ms = timer.run(launch, 1, warmup, steps)
    return dict(ms=ms, bytes=2 * nbytes, read=nbytes, write=nbytes, copies=1)


# ------------------------------------------------------------------------------------------
# HBM traffic per launch from rocprofv3 counters (FETCH_SIZE, then WRITE_SIZE)
# ------------------------------------------------------------------------------------------

PMC_LEGS = "w8a8,w4a8,w4a16,conv,copy"
TRAFFIC_LEGS = ("w8a8", "w4a8", "w4a16", "conv")


def leg_of_kernel(name):
    """Which bench leg a (demangled) kernel name belongs to, for the legs in PMC_LEGS."""
    if "bitwise_not" in name:
        return "copy"
    if "w4a8_mfma_kernel" in name or "w4a8_strip_kernel" in name:
        return "w4a8"
    if "w4a16_" in name:
        return "w4a16"
    if "conv_halo_kernel" in name:
        return "conv"
    if "int8_stream_kernel<" in name or "igemm" in name:
        # int8_stream_kernel<BM, EPI, PK, conv>: the convolution mode has conv = true
        head = name.split(">")[0].rstrip()
        return "conv" if (head.endswith("true") or "igemm" in name) else "w8a8"
    return None


def pmc_pass(counter, timeout_s=120):
    """One rocprofv3 --pmc run of this script's PMC_LEGS in a child process; returns
    {leg: mean counter value per dispatch (KiB)} or None."""
    import csv
    import glob
    import shutil
    import signal
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3")
    if prof is None:
        return None
    out = tempfile.mkdtemp(prefix="tqt_pmc_", dir="/tmp")
    cmd = [prof, "--pmc", counter, "-d", out, "-o", "pmc", "--output-format", "csv", "--",
           sys.executable, os.path.abspath(__file__), "--only", PMC_LEGS, "--steps", "6",
           "--warmup", "2", "--no-graphs"]
    env = dict(os.environ, TMPDIR="/tmp")
    proc = subprocess.Popen(cmd, cwd="/tmp", env=env, stdout=subprocess.DEVNULL,
                            stderr=subprocess.DEVNULL, start_new_session=True)
    try:
        proc.wait(timeout=timeout_s)
    except subprocess.TimeoutExpired:
        os.killpg(proc.pid, signal.SIGKILL)
        proc.wait()
        shutil.rmtree(out, ignore_errors=True)
        return None
    vals = {leg: [] for leg in PMC_LEGS.split(",")}
    for path in glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True):
        with open(path, newline="") as fh:
            for row in csv.DictReader(fh):
                if row.get("Counter_Name") != counter:
                    continue
                leg = leg_of_kernel(row.get("Kernel_Name", ""))
                if leg in vals:
                    vals[leg].append(float(row["Counter_Value"]))
    shutil.rmtree(out, ignore_errors=True)
    if not all(vals.values()):
        return None
    return {leg: sum(v) / len(v) for leg, v in vals.items()}


def hbm_traffic():
    """HBM bytes per launch of the W8A8, W4A8, W4A16 and igemmcl kernels: FETCH_SIZE and
    WRITE_SIZE (KiB per dispatch), each scaled by bytes / counter of the copy kernel, whose
    traffic is known."""
    fetch = pmc_pass("FETCH_SIZE")
    write = pmc_pass("WRITE_SIZE") if fetch else None
    if not fetch or not write:
        return None
    nbytes = 256 << 20
    f_scale = nbytes / fetch["copy"]
    w_scale = nbytes / write["copy"]
    res = {"fetch_scale_bytes_per_KiB": round(f_scale, 2),
           "write_scale_bytes_per_KiB": round(w_scale, 2)}
    for leg in TRAFFIC_LEGS:
        res[leg] = {"read": fetch[leg] * f_scale, "write": write[leg] * w_scale,
                    "total": fetch[leg] * f_scale + write[leg] * w_scale}
    return res


# ------------------------------------------------------------------------------------------
# CPU baseline (oracle restatement of the reference kernel; bounded sample)
# ------------------------------------------------------------------------------------------

def host_cpu():
    """(threads to use, description): this process's CPU affinity capped at 16 threads, the CPU
    share of one GPU on the GPU box (OMP_NUM_THREADS there), with nproc and the CPU model."""
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 1
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    threads = max(1, min(16, avail))
    return threads, dict(nproc=os.cpu_count(), affinity=avail, threads=threads, model=model)


def cpu_baseline(w8, w4, budget_s=8.0, single_budget_s=6.0):
    """The oracle's W8A8 and W4A8 (the reference's 4x16 tile loop in portable C, built with
    -O3 -ffp-contract=off -fopenmp) on the host cores: OpenMP over output tiles (the
    reference's threading model) on `threads` threads, and on one thread, each repeated over
    whole config-sized calls for a bounded time. value = W8A8 TOPS on all threads."""
    import tqt_testlib as T

    o = T.oracle()
    A, B, sb, bias, _ = w8["inputs"]
    m, n, k = W8A8["m"], W8A8["n"], W8A8["k"]
    D = np.empty((m, n), np.int8)
    A4, Bp4, sa4, za4, sb4, bias4 = w4["inputs"]
    n4, k4 = W4A8["n"], W4A8["k"]
    D4 = np.empty((1, n4), np.float32)

    def w8a8_call():
        o.tqto_gemm_qai8_qai8_qsi8cxt(m, n, k, T.ptr(A), k, T.ptr(B), k, None, n, T.ptr(D), n,
                                      T.ptr(bias), -128, 127, 0.02, T.ptr(sb), n, 0.05, 0)

    def w4a8_call():
        o.tqto_gemm_qai8dx_qsi4cxt_f32(1, n4, k4, T.ptr(A4), k4, T.ptr(Bp4), k4, None, n4,
                                       T.ptr(D4), n4, T.ptr(bias4), -np.inf, np.inf, T.ptr(sa4),
                                       T.ptr(za4), T.ptr(sb4))

    def timed(call, threads, budget):
        o.tqto_set_threads(threads)
        call()  # warm
        reps = 0
        t0 = time.perf_counter()
        while True:
            call()
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return reps, el

    threads, host = host_cpu()
    r8, e8 = timed(w8a8_call, threads, budget_s)
    r81, e81 = timed(w8a8_call, 1, single_budget_s)
    r4, e4 = timed(w4a8_call, threads, budget_s / 2)
    r41, e41 = timed(w4a8_call, 1, single_budget_s / 2)
    o.tqto_set_threads(threads)
    ops8 = 2.0 * m * n * k
    w4_bytes = w4["bytes"]
    return dict(value=round(r8 * ops8 / e8 / 1e12, 4), unit="TOPS", cores=threads, kind="port",
                value_single_thread=round(r81 * ops8 / e81 / 1e12, 4),
                w4a8={"value": round(r4 * w4_bytes / e4 / 1e9, 3), "unit": "GB/s",
                      "value_single_thread": round(r41 * w4_bytes / e41 / 1e9, 3),
                      "us_per_call": round(e4 / r4 * 1e6, 1)},
                host=host,
                sample="W8A8 M=512 K=4096 N=4096: %d calls on %d threads in %.1f s, %d on 1 thread "
                       "in %.1f s; W4A8 M=1 K=4096 N=11008: %d calls on %d threads in %.1f s, %d "
                       "on 1 thread in %.1f s (oracle/ portable C: the reference's 4x16 tile "
                       "loop, OpenMP over tiles, -O3 -ffp-contract=off)"
                       % (r8, threads, e8, r81, e81, r4, threads, e4, r41, e41))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 counter passes that measure HBM traffic")
    ap.add_argument("--no-graphs", action="store_true",
                    help="time launches issued one by one on the stream instead of a HIP graph")
    ap.add_argument("--only", default=None,
                    help="comma-separated legs (w8a8,w4a8,w4a8m2,w4a8m4,w4a8m8,w4a16,w8a8p,w4a8p,"
                         "w4a16p,w4a8dq,w4a8dqf,conv,convp,clamp,copy,floor,sfloor,sfloor_l2,empty,"
                         "caller_w8a8,caller_w4a8): "
                         "time just those and print one JSON line each (profiling runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: these kernels run on a single MI355X and this "
              "build has no multi-GPU path (use --gpus 1).", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    mod, lib = load_lib()
    stream = torch.cuda.Stream()
    timer = Timer(torch, stream, graphs=not args.no_graphs)
    rng = np.random.default_rng(42)
    K, W = args.steps, args.warmup

    if args.only:
        legs = {
            "w8a8": lambda: bench_w8a8(torch, mod, lib, timer, W, K, rng),
            "w4a8": lambda: bench_w4a8(torch, mod, lib, timer, W, K, rng, 1),
            "w4a8m2": lambda: bench_w4a8(torch, mod, lib, timer, W, K, rng, 2),
            "w4a8m4": lambda: bench_w4a8(torch, mod, lib, timer, W, K, rng, 4),
            "w4a8m8": lambda: bench_w4a8(torch, mod, lib, timer, W, K, rng, 8),
            "w4a16": lambda: bench_w4a16(torch, mod, lib, timer, W, K, rng),
            "w8a8p": lambda: bench_w8a8(torch, mod, lib, timer, W, K, rng, packed=True),
            "w4a8p": lambda: bench_w4a8(torch, mod, lib, timer, W, K, rng, 1, packed=True),
            "w4a16p": lambda: bench_w4a16(torch, mod, lib, timer, W, K, rng, packed=True),
            "w4a8dq": lambda: bench_w4a8(torch, mod, lib, timer, W, K, rng, 1, dynq=True),
            "w4a8dqf": lambda: bench_w4a8(torch, mod, lib, timer, W, K, rng, 1, dynq="fused"),
            "conv": lambda: bench_conv(torch, mod, lib, timer, W, K, rng),
            "convp": lambda: bench_conv(torch, mod, lib, timer, W, K, rng, packed=True),
            "clamp": lambda: bench_clamp(torch, mod, lib, timer, W, K, rng),
            "copy": lambda: bench_copy(torch, timer, W, K),
            "floor": lambda: bench_floor(torch, timer, W, K, W4A8_BYTES),
            "sfloor": lambda: bench_stream_floor(torch, timer, W, K),
            "sfloor_l2": lambda: bench_stream_floor(torch, timer, W, K, resident=True),
            "empty": lambda: bench_empty(torch, timer, W, K),
            "caller_w8a8": lambda: bench_caller(torch, mod, lib, "w8a8"),
            "caller_w4a8": lambda: bench_caller(torch, mod, lib, "w4a8"),
        }
        with torch.cuda.stream(stream):
            for leg in args.only.split(","):
                r = legs[leg]()
                line = {"leg": leg, "us_per_launch": round(r["ms"] * 1e3, 3),
                        "bytes": r["bytes"], "copies": r["copies"]}
                for key in ("us_by_loads", "calls", "m_step", "n_step", "per_cu_gbs"):
                    if key in r:
                        line[key] = r[key]
                if "ms_async" in r:
                    line["us_async"] = round(r["ms_async"] * 1e3, 3)
                print(json.dumps(line), flush=True)
        return

    def progress(name, r):
        print("bench: %s %.3f us per launch" % (name, r["ms"] * 1e3), file=sys.stderr,
              flush=True)
        return r

    with torch.cuda.stream(stream):
        w8 = progress("w8a8", bench_w8a8(torch, mod, lib, timer, W, K, rng))
        w4 = {mm: progress("w4a8 M=%d" % mm, bench_w4a8(torch, mod, lib, timer, W, K, rng, mm))
              for mm in (1, 4, 8)}
        w416 = progress("w4a16", bench_w4a16(torch, mod, lib, timer, W, K, rng))
        cv = progress("igemmcl", bench_conv(torch, mod, lib, timer, W, K, rng))
        cl = progress("clamp_i32", bench_clamp(torch, mod, lib, timer, W, K, rng))
        w8p = progress("w8a8 packed", bench_w8a8(torch, mod, lib, timer, W, K, rng, packed=True))
        w4p = progress("w4a8 packed",
                       bench_w4a8(torch, mod, lib, timer, W, K, rng, 1, packed=True))
        w416p = progress("w4a16 packed",
                         bench_w4a16(torch, mod, lib, timer, W, K, rng, packed=True))
        cvp = progress("igemmcl packed", bench_conv(torch, mod, lib, timer, W, K, rng,
                                                    packed=True))
        w4dq = progress("w4a8 decode step (two launches)",
                        bench_w4a8(torch, mod, lib, timer, W, K, rng, 1, dynq=True))
        w4dqf = progress("w4a8 decode step (fused)",
                         bench_w4a8(torch, mod, lib, timer, W, K, rng, 1, dynq="fused"))
        fl = progress("read floor", bench_floor(torch, timer, W, K, w4[1]["bytes"]))
        sf = progress("w8a8 stream floor", bench_stream_floor(torch, timer, W, K))
        sfr = progress("w8a8 stream floor L2-resident",
                       bench_stream_floor(torch, timer, W, K, resident=True))
        em = progress("empty launch", bench_empty(torch, timer, W, K))
        ems = {name: progress("empty launch " + name,
                              bench_empty(torch, timer, W, K, blocks=b, threads=t, lds=l))
               for name, (b, t, l) in launch_shapes(
                   torch.cuda.get_device_properties(0).multi_processor_count).items()}
        cw8 = progress("reference caller w8a8", bench_caller(torch, mod, lib, "w8a8"))
        cw4 = progress("reference caller w4a8", bench_caller(torch, mod, lib, "w4a8"))

    w41 = w4[1]
    traffic = None if args.no_traffic else hbm_traffic()
    print("bench: traffic counters %s" % ("done" if traffic else "skipped or unavailable"),
          file=sys.stderr, flush=True)
    tr = {leg: (round(traffic[leg]["total"]) if traffic else None) for leg in TRAFFIC_LEGS}
    out = {
        "metric": "W4A8 GEMV HBM GB/s (M=1) + W8A8 GEMM int8 TOPS (M=512), % roofline",
        "value": round(w8["tops"], 3),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(w8["ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded BASELINE.json recipes), %d rotating weight copies > 256 MB "
                "MALL" % w8["copies"],
        "timing": ("HIP events around one replay of a HIP graph holding exactly `steps` launches"
                   if not args.no_graphs else "HIP events around `steps` stream launches"),
        "ms_per_step_stream_launches": round(w8["ms_stream"], 6),
        "config": {"workload": "gemm_1xnbias_reqi32toi8_clamp_qai8_qai8_qsi8cxt M=512 K=4096 "
                               "N=4096 (W8A8 prefill, int8 requantized out)",
                   "M": 512, "K": 4096, "N": 4096},
        "roofline": {"bound": "mfma", "achieved": round(w8["tops"], 3), "peak": INT8_PEAK_TOPS,
                     "unit": "TOPS", "frac": round(w8["tops"] / INT8_PEAK_TOPS, 4),
                     "traffic": tr["w8a8"], "algorithmic_bytes": w8["bytes"]},
        # the W8A8 kernel's own load schedule alone (no MFMA, no epilogue), cold and with every
        # workgroup reading one L2-resident tile, and an empty launch of its shape
        "w8a8_floors": {
            "stream_us": round(sf["ms"] * 1e3, 3),
            "stream_per_cu_GBs": round(sf["per_cu_gbs"], 2),
            "stream_l2_resident_us": round(sfr["ms"] * 1e3, 3),
            "stream_l2_resident_per_cu_GBs": round(sfr["per_cu_gbs"], 2),
            "per_cu_bytes": sf["per_cu_bytes"],
            "empty_launch_us": round(em["ms"] * 1e3, 3),
            "frac_of_stream_floor": round(sf["ms"] / w8["ms"], 4),
        },
        # an empty kernel with each headline kernel's grid, block and LDS size, graph-replayed
        # like the kernels: the fixed per-launch cost inside each kernel's figure
        "launch_floors_us": dict([("w8a8 stream", round(em["ms"] * 1e3, 3))] +
                                 [(name, round(r["ms"] * 1e3, 3)) for name, r in ems.items()]),
        # the reference's caller pattern: one synchronous run per m_step x n_step tile
        # (host wall clock per whole GEMM, warm operands), and the same tiles through the
        # stream-ordered runs with one synchronization
        "reference_caller": {
            name: {"calls": r["calls"], "m_step": r["m_step"], "n_step": r["n_step"],
                   "us_sync": round(r["ms"] * 1e3, 2), "us_async": round(r["ms_async"] * 1e3, 2)}
            for name, r in (("w8a8 cfg2", cw8), ("w4a8 cfg3 M=1", cw4))},
        "w4a8": {
            "workload": "gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt M=1 K=4096 N=11008 (W4A8 decode)",
            "value": round(w41["gbs"], 2), "unit": "GB/s", "us_per_launch": round(w41["ms"] * 1e3, 3),
            "us_per_launch_stream_launches": round(w41["ms_stream"] * 1e3, 3),
            "roofline": {"bound": "hbm", "achieved": round(w41["gbs"], 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(w41["gbs"] / HBM_PEAK_GBS, 4),
                         "traffic": tr["w4a8"], "algorithmic_bytes": w41["bytes"]},
            # one launch of a plain 16-byte streaming read of the same bytes (rotating copies,
            # fastest of FLOOR_LOADS shapes): the single-launch HBM read floor on this GPU
            "read_floor": {"us": round(fl["ms"] * 1e3, 3), "GB/s": round(fl["gbs"], 2),
                           "frac": round(fl["gbs"] / HBM_PEAK_GBS, 4),
                           "loads_per_lane": fl["loads"], "us_by_loads": fl["us_by_loads"]},
            "frac_of_read_floor": round(fl["ms"] / w41["ms"], 4),
            "M4": {"GB/s": round(w4[4]["gbs"], 2), "us": round(w4[4]["ms"] * 1e3, 3),
                   "frac": round(w4[4]["gbs"] / HBM_PEAK_GBS, 4)},
            "M8": {"GB/s": round(w4[8]["gbs"], 2), "us": round(w4[8]["ms"] * 1e3, 3),
                   "frac": round(w4[8]["gbs"] / HBM_PEAK_GBS, 4)},
            "copies": w41["copies"],
        },
        "configs": {
            "gemm_clamp_i32_i8_i8 64x256x512": {"us": round(cl["ms"] * 1e3, 3),
                                                "TOPS": round(cl["tops"], 3)},
            "w4a16 32x14336x4096 bl32": {"us": round(w416["ms"] * 1e3, 3),
                                         "GB/s": round(w416["gbs"], 2),
                                         "hbm_frac": round(w416["gbs"] / HBM_PEAK_GBS, 4),
                                         "TFLOP/s": round(w416["tflops"], 2),
                                         "f16_mfma_frac": round(w416["tflops"] / F16_PEAK_TFLOPS, 4),
                                         "traffic": tr["w4a16"],
                                         "algorithmic_bytes": w416["bytes"]},
            "igemmcl 8x56x56x128 3x3 OC128": {"us": round(cv["ms"] * 1e3, 3),
                                              "TOPS": round(cv["tops"], 3),
                                              "mfma_frac": round(cv["tops"] / INT8_PEAK_TOPS, 4),
                                              "traffic": tr["conv"],
                                              "algorithmic_bytes": cv["bytes"]},
            # packed siblings on the same configurations (operands packed before timing)
            "packed qai8_qai8p_qsi8cxp 512x4096x4096": {
                "us": round(w8p["ms"] * 1e3, 3), "TOPS": round(w8p["tops"], 3),
                "mfma_frac": round(w8p["tops"] / INT8_PEAK_TOPS, 4)},
            "packed qai8dxp_qsi4cxp M=1 K=4096 N=11008": {
                "us": round(w4p["ms"] * 1e3, 3), "GB/s": round(w4p["gbs"], 2),
                "hbm_frac": round(w4p["gbs"] / HBM_PEAK_GBS, 4)},
            "W4A8 decode step with GPU activation quantization, M=1 K=4096 N=11008": {
                "us": round(w4dqf["ms"] * 1e3, 3), "GB/s": round(w4dqf["gbs"], 2),
                "hbm_frac": round(w4dqf["gbs"] / HBM_PEAK_GBS, 4),
                "entry_point": "tqt_run_quantize_gemm_1xnbias_clamp_f32_qai8dx_qsi4cxt_gfx950 "
                               "(one launch)",
                "two_launches_us": round(w4dq["ms"] * 1e3, 3)},
            "packed f16p_qsi4c2p 32x14336x4096 bl32": {
                "us": round(w416p["ms"] * 1e3, 3), "GB/s": round(w416p["gbs"], 2),
                "hbm_frac": round(w416p["gbs"] / HBM_PEAK_GBS, 4)},
            "packed igemmcl qsi8cxp 8x56x56x128 3x3 OC128": {
                "us": round(cvp["ms"] * 1e3, 3), "TOPS": round(cvp["tops"], 3),
                "mfma_frac": round(cvp["tops"] / INT8_PEAK_TOPS, 4)},
        },
    }
    if traffic:
        out["traffic_detail"] = {
            "source": "rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE (KiB per dispatch), scaled "
                      "by the counters of a 256 MB bitwise_not copy kernel",
            "fetch_scale_bytes_per_KiB": traffic["fetch_scale_bytes_per_KiB"],
            "write_scale_bytes_per_KiB": traffic["write_scale_bytes_per_KiB"],
        }
        for leg in TRAFFIC_LEGS:
            out["traffic_detail"][leg] = {k: round(v) for k, v in traffic[leg].items()}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(w8, w41)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
