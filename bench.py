#!/usr/bin/env python3
"""Benchmark of the MI355X `Hip` backend's hot path on one GPU.

The headline line is BASELINE.json's first metric on the configuration its
target names: a dense bf16 GEMM, M = N = K = 8192, through the C ABI's
`tc_matmul` (Kernels::matmul), in TFLOP/s.  A "step" is one such product over
one batch of synthetic input already resident in HBM.  The same JSON line
carries the other configurations' measurements under "workloads": the f32
and f16 GEMMs of the sweep, the axis reductions of configuration 2 (at the
stated [64,128,1024] and at the 512 MiB size its text quotes), the broadcast
chain and strided copies of configuration 3 — each with the roofline that
bounds it.

Timing: W untimed warmup steps, then exactly K steps between two HIP events
recorded on the library's own stream (the stream every kernel is launched
on), the stream synchronised on both sides.  The bandwidth workloads, whose
kernels take microseconds, capture their K calls into a HIP graph and time
its replay, so the figure is the kernels' and not this script's call rate.  The roofline's `achieved` is the
algorithmic work per launch of the dominant kernel over that kernel's own
event-timed duration.  The CPU baseline is the oracle's C restatement of the
reference Host (simd) algorithm, timed on a bounded sample on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""

from __future__ import annotations

import argparse
import ctypes
import itertools
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from tensorcrate_amd import halfconv, lib  # noqa: E402
from tensorcrate_amd.optim import Adam  # noqa: E402
from tensorcrate_amd.tensor import Tensor  # noqa: E402

HBM_PEAK = 8000.0  # GB/s, MI355X HBM3E
# HBM bytes per launch of the headline product, from `rocprofv3 --pmc
# FETCH_SIZE` and `--pmc WRITE_SIZE` runs of `bench.py --traffic-probe
# kernels`, scaled by what the counters read for a plain 1 GiB copy (fetch
# x 2.0, write x 0.998): the back-to-back launches' 1.617 GB read + 0.134 GB
# written (profiles/gemm_bf16_8192_traffic.md).
HEADLINE_TRAFFIC = 1.751e9
# HBM bytes per call of each other product, bandwidth workload (part
# "kernels" of the probe) and fused or training workload (part "programs"),
# from the same two counters with the same calibration
# (profiles/gemm_bf16_8192_traffic.md, profiles/bandwidth_traffic.md,
# profiles/fused_programs_traffic.md): the bandwidth workloads within 5% of
# their algorithmic bytes.
MEASURED_TRAFFIC = {
    "f16 GEMM 16384x1024x4096": 3.419e+08,
    "f32 GEMM 4096x4096x4096": 6.041e+08,
    "x*y, f32 [256,512,512] x [1,512,1]": 5.364e+08,
    "t+z, f32 [256,512,512] + [256,1,512]": 5.406e+08,
    "permute(0,2,1).contiguous, f32 [256,512,512]": 5.364e+08,
    "slice [:,128:384,:].contiguous, f32": 2.682e+08,
    "concat of two [256,256,512] halves on axis 1, f32": 5.366e+08,
    "same-shape add, f32 64 Mi elements": 8.048e+08,
    "sum_axes [2] of f32 [64x128x1024]": 3.366e+07,
    "var_axes [2] of f32 [64x128x1024]": 3.366e+07,
    "sum_axes [0, 1] of f32 [64x128x1024]": 3.415e+07,
    "var_axes [0, 1] of f32 [64x128x1024]": 3.523e+07,
    "argmax axis 1 of f32 [64x128x1024]": 3.387e+07,
    "sum_axes [2] of f32 [1024x128x1024]": 5.38e+08,
    "var_axes [2] of f32 [1024x128x1024]": 5.38e+08,
    "sum_axes [0, 1] of f32 [1024x128x1024]": 5.401e+08,
    "var_axes [0, 1] of f32 [1024x128x1024]": 5.465e+08,
    "argmax axis 1 of f32 [1024x128x1024]": 5.412e+08,
    "matvec, f32 [8192x8192] . [8192]": 2.688e+08,
    "vecmat, f32 [8192] . [8192x8192]": 2.71e+08,
    "dot, f32 64 Mi elements": 5.37e+08,
    "transpose, f32 [4096x4096]": 1.342e+08,
    "layer norm f32 [8192x8192] (fused_with_statistics), statistics and program in one kernel": 5.368e+08,
    "layer norm f32 [8192x8192] (fused_with_statistics), composed: row moments, then the program": 8.059e+08,
    "Adam update, 25175040 f32 parameters (fused program)": 7.043e+08,
    "MLP training step 1024-4096-4096-1024, batch 4096, f32, tape + Adam (configs[4])": 8.402e+09,
    "bf16 dense layer relu(x w + b) 8192x8192x8192, in the product's epilogue": 1.752e+09,
    "bf16 dense layer relu(x w + b) 8192x8192x8192, unfused: product, then program": 2.318e+09,
    "f32 dense layer relu(x w + b) 4096x1024x4096, in the product's epilogue": 2.015e+08,
    "f32 dense layer relu(x w + b) 4096x1024x4096, unfused: product, then program": 3.356e+08,
}
MFMA_PEAK = {"bf16": 2516.6, "f16": 2516.6, "f32": 157.3}  # dense TFLOP/s
KIND = {"bf16": lib.BF16, "f16": lib.F16, "f32": lib.F32}
METRIC = "GEMM TFLOP/s & %MFMA peak; reduce/elementwise/copy GB/s & %HBM peak"


def log(message: str) -> None:
    print(message, file=sys.stderr, flush=True)


class Timing(float):
    """Mean milliseconds per call over every timed call, carrying the spread
    the reference harness reports (benches/nn_ops.rs:185-252): the median
    and minimum of the samples, and their median absolute deviation as a
    fraction of the median."""

    median: float
    low: float
    mad: float
    samples: int

    @staticmethod
    def of(mean: float, samples: list[float]) -> "Timing":
        t = Timing(mean)
        ordered = sorted(samples)
        t.median = ordered[len(ordered) // 2]
        t.low = ordered[0]
        deviations = sorted(abs(x - t.median) for x in ordered)
        t.mad = deviations[len(deviations) // 2] / t.median if t.median > 0 else 0.0
        t.samples = len(ordered)
        return t


# Samples a graph-replayed workload is timed over (the reference harness
# takes 15, benches/nn_ops.rs).
SAMPLES = 15

_hip = None


def _hip_runtime() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        vp = ctypes.c_void_p
        _hip.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
        _hip.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
        _hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t]
        _hip.hipGraphLaunch.argtypes = [vp, vp]
        _hip.hipGraphExecDestroy.argtypes = [vp]
        _hip.hipGraphDestroy.argtypes = [vp]
        _hip.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        _hip.hipEventRecord.argtypes = [vp, vp]
        _hip.hipEventSynchronize.argtypes = [vp]
        _hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        _hip.hipEventDestroy.argtypes = [vp]
    return _hip


def _stream() -> ctypes.c_void_p:
    stream = ctypes.c_void_p()
    lib.call("tc_stream", ctypes.byref(stream))
    return stream


class _Marks:
    """HIP events recorded on the library's stream (the stream every kernel
    is launched on): mark i is recorded after the i-th timed unit."""

    def __init__(self, count: int):
        self.hip, self.stream = _hip_runtime(), _stream()
        self.events = []
        for _ in range(count):
            event = ctypes.c_void_p()
            if self.hip.hipEventCreate(ctypes.byref(event)) != 0:
                raise RuntimeError("hipEventCreate failed")
            self.events.append(event)

    def record(self, i: int) -> None:
        if self.hip.hipEventRecord(self.events[i], self.stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def between(self, i: int, j: int) -> float:
        ms = ctypes.c_float()
        if self.hip.hipEventElapsedTime(ctypes.byref(ms), self.events[i], self.events[j]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def finish(self) -> None:
        self.hip.hipEventSynchronize(self.events[-1])
        lib.sync()
        for event in self.events:
            self.hip.hipEventDestroy(event)


# How long a matrix-core line runs its call back to back before it is timed.
# The part runs its first dense products of a burst fast and then slows for
# a few dozen launches while its power controller settles the clock (an
# 8192^3 product: 0.74, then 0.95, then a steady 0.72 ms); 50 ms of the
# call covers that, so no line is timed inside the ramp.
SETTLE_SECONDS = 0.05


def settle(fn, seconds: float = SETTLE_SECONDS) -> None:
    """`fn` called back to back, untimed, for at least `seconds`."""
    start = time.perf_counter()
    while True:
        for _ in range(4):
            fn()
        lib.sync()
        if time.perf_counter() - start >= seconds:
            return


def timed(fn, steps: int, warmup: int) -> Timing:
    """`fn` called `warmup` times untimed, then exactly `steps` times between
    HIP events on the library's stream, with the stream synchronised before
    and after; an event after every call makes each call one sample."""
    for _ in range(warmup):
        fn()
    lib.sync()
    marks = _Marks(steps + 1)
    marks.record(0)
    for i in range(steps):
        fn()
        marks.record(i + 1)
    marks.hip.hipEventSynchronize(marks.events[-1])
    samples = [marks.between(i, i + 1) for i in range(steps)]
    total = marks.between(0, steps)
    marks.finish()
    return Timing.of(total / steps, samples)


def timed_graph(fn, steps: int, warmup: int) -> Timing:
    """Milliseconds per call of `fn`, with `steps` calls captured into one
    HIP graph on the library's stream and the graph replayed SAMPLES times
    between HIP events on that stream, each replay one sample: the kernels
    run back to back, as they would from a compiled caller, rather than
    paced by this script's per-call overhead.  Falls back to `timed` if the
    stream cannot be captured."""
    for _ in range(warmup):
        fn()
    lib.sync()
    hip, stream = _hip_runtime(), _stream()
    graph, graph_exec = ctypes.c_void_p(), ctypes.c_void_p()
    if hip.hipStreamBeginCapture(stream, 2) != 0:  # hipStreamCaptureModeRelaxed
        return timed(fn, steps, 0)
    for _ in range(steps):
        fn()
    if hip.hipStreamEndCapture(stream, ctypes.byref(graph)) != 0 or \
            hip.hipGraphInstantiate(ctypes.byref(graph_exec), graph, None, None, 0) != 0:
        return timed(fn, steps, 0)
    hip.hipGraphLaunch(graph_exec, stream)  # one untimed replay
    lib.sync()
    marks = _Marks(SAMPLES + 1)
    marks.record(0)
    for i in range(SAMPLES):
        hip.hipGraphLaunch(graph_exec, stream)
        marks.record(i + 1)
    hip.hipEventSynchronize(marks.events[-1])
    samples = [marks.between(i, i + 1) / steps for i in range(SAMPLES)]
    total = marks.between(0, SAMPLES)
    marks.finish()
    hip.hipGraphExecDestroy(graph_exec)
    hip.hipGraphDestroy(graph)
    # The graph is gone: the storage its captured calls used may serve
    # eager work again.
    lib.call("tc_release_graph_memory")
    return Timing.of(total / (SAMPLES * steps), samples)


def host_matrix(kind: str, rows: int, cols: int, rng, sigma=None) -> np.ndarray:
    if sigma is None:
        values = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
    else:
        values = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(sigma)
    if kind == "bf16":
        return halfconv.bf16_bits(values)
    if kind == "f16":
        return halfconv.f16(values)
    return values


class Product:
    """One product's operands, generated and uploaded to HBM, ready to time."""

    def __init__(self, kind: str, m: int, k: int, n: int, seed: int, sigma):
        rng = np.random.default_rng(seed)
        self.kind, self.m, self.k, self.n = kind, m, k, n
        self.a_host = host_matrix(kind, m, k, rng, sigma)
        self.b_host = host_matrix(kind, k, n, rng, sigma)
        self.a, self.b = lib.Buffer.of(self.a_host), lib.Buffer.of(self.b_host)
        self.c = lib.Buffer(m * n * (4 if kind == "f32" else 2))

    def time(self, steps: int, warmup: int, cpu: bool = False) -> dict:
        kind, m, k, n = self.kind, self.m, self.k, self.n
        a, b, c, code = self.a, self.b, self.c, KIND[kind]
        op = lambda: lib.call("tc_matmul", code, code, lib.PLAIN, 0, m, k, n, a.ptr, b.ptr, c.ptr)
        settle(op)
        ms = timed(op, steps, warmup)
        # The product is one kernel launch, so the call's event time is the
        # kernel's.
        kernel_ms = ms
        flops = 2.0 * m * n * k
        achieved = flops / (kernel_ms * 1e-3) / 1e12
        for buffer in (a, b, c):
            buffer.free()
        baseline = None
        if cpu:
            from oracle import binding as oracle  # the CPU baseline's restatement
            band = 64
            band_a, b_host = np.ascontiguousarray(self.a_host[:band]), self.b_host
            baseline = cpu_rate(lambda: oracle.matmul(code, band_a, b_host, band, k, n), 2.0 * band * k * n,
                                "TFLOP/s", f"rows 0..{band} of A times all of B: the oracle's widen + single-thread "
                                "AVX2 i-p-j FMA + round-once (compact.rs:232-262, simd_x86.rs:1302-1331), linear in M",
                                1e12, min_seconds=1.0)
        self.a_host = self.b_host = None
        return {
            "workload": f"{kind} GEMM {m}x{k}x{n}",
            "key": f"gemm {kind} {m}x{k}x{n}",
            "spread": spread(ms),
            "cpu_baseline": baseline,
            "value": flops / (ms * 1e-3) / 1e12,
            "unit": "TFLOP/s",
            "ms": ms,
            "roofline": {"bound": "mfma", "achieved": achieved, "peak": MFMA_PEAK[kind], "unit": "TFLOP/s",
                         "frac": achieved / MFMA_PEAK[kind],
                         "traffic": MEASURED_TRAFFIC.get(f"{kind} GEMM {m}x{k}x{n}"), "kernel_ms": kernel_ms,
                         "bytes": (m * k + k * n + m * n) * (4 if kind == "f32" else 2)},
        }


def gemm(kind: str, m: int, k: int, n: int, seed: int, sigma, steps: int, warmup: int, cpu: bool = False) -> dict:
    return Product(kind, m, k, n, seed, sigma).time(steps, warmup, cpu)


class DenseLayer:
    """relu(x . w + bias) over synthetic operands, as the calls the bench
    times: the program in the product kernel's epilogue
    (`tc_matmul_epilogue`, one kernel, the product never in HBM), unfused
    (`tc_matmul`, then `tc_fused` over the stored product), and the product
    alone."""

    def __init__(self, kind: str, m: int, k: int, n: int):
        rng = np.random.default_rng(11)
        code = KIND[kind]
        size = 4 if kind == "f32" else 2
        self.hx = host_matrix(kind, m, k, rng, 1 / np.sqrt(k))
        self.hw = host_matrix(kind, k, n, rng, 1 / np.sqrt(k))
        self.hbias = host_matrix(kind, 1, n, rng).reshape(n)
        x, w, bias = lib.Buffer.of(self.hx), lib.Buffer.of(self.hw), lib.Buffer.of(self.hbias)
        out, product = lib.Buffer(m * n * size), lib.Buffer(m * n * size)
        self.buffers = [x, w, bias, out, product]
        self.program = [(0, 0, 0, 0, code, 0, 0.0), (0, 1, 1, 1, code, 0, 0.0), (2, lib.ADD, 2, 0, 1, 0, 0.0),
                        (1, 0, 3, 0, 0, 0, 0.0), (4, lib.MAX, 4, 2, 3, 0, 0.0), (5, 0, 0, 4, code, 0, 0.0)]
        program = self.program
        enc, places = lib._program(program, [(0, 1, 1, [m], [n]), (0, 1, 0, [], [])])
        bias_in, bias_len = lib._buffers([(bias, n)])
        both_in, both_len = lib._buffers([(product, m * n), (bias, n)])
        outs, out_lens = lib._buffers([(out, m * n)])

        def fused():
            lib.call("tc_matmul_epilogue", code, enc, len(program), places, 2, m, k, n, x.ptr, w.ptr, bias_in,
                     bias_len, 1, outs, out_lens, 1)

        def unfused():
            lib.call("tc_matmul", code, code, lib.PLAIN, 0, m, k, n, x.ptr, w.ptr, product.ptr)
            lib.call("tc_fused", code, enc, len(program), places, 2, both_in, both_len, 2, outs, out_lens, 1, m, n)

        def product_only():
            lib.call("tc_matmul", code, code, lib.PLAIN, 0, m, k, n, x.ptr, w.ptr, product.ptr)

        self.fused, self.unfused, self.product_only = fused, unfused, product_only

    def free(self) -> None:
        for buffer in self.buffers:
            buffer.free()


def dense_layer(kind: str, m: int, k: int, n: int, steps: int, warmup: int) -> list[dict]:
    """relu(x . w + bias) two ways, and the product alone (`DenseLayer`).
    Every line counts the product's 2 m n k FLOP only."""
    from oracle import binding as oracle  # the CPU baseline's restatement

    layer = DenseLayer(kind, m, k, n)
    code = KIND[kind]
    hx, hw, hbias, program = layer.hx, layer.hw, layer.hbias, layer.program
    fused, unfused, product_only = layer.fused, layer.unfused, layer.product_only
    flops = 2.0 * m * n * k
    # The CPU baseline: the oracle's product-then-program (the Host's
    # run_matmul, fused/mod.rs:1143-1215) over a band of rows of x.
    band = 32 if kind != "f32" else 128
    band_x = np.ascontiguousarray(hx[:band])
    band_places = [(0, 1, 1, [band], [n]), (0, 1, 0, [], [])]
    band_out = np.empty(band * n, hx.dtype)
    baseline = cpu_rate(lambda: oracle.matmul_epilogue(code, program, band_places, band_x, hw, band, k, n, [hbias],
                                                       [band_out]),
                        2.0 * band * k * n, "TFLOP/s",
                        f"rows 0..{band} of x: the oracle's single-thread product, then the program, linear in M",
                        1e12, min_seconds=1.0)
    # x, w and the bias read once, relu(x w + b) written once.
    algorithmic = (m * k + k * n + n + m * n) * (4 if kind == "f32" else 2)
    # The programs compile on their second appearance; both compiles come
    # first, so that the idle time they take does not undo the clock's
    # settling, and each line is then timed after its call ran back to back.
    for _ in range(2):
        fused()
        unfused()
    lib.sync()
    lines = []
    for name, short, fn in (("in the product's epilogue", "epilogue", fused),
                            ("unfused: product, then program", "unfused", unfused),
                            ("the product alone", "product", product_only)):
        settle(fn)
        ms = timed(fn, steps, warmup)
        achieved = flops / (ms * 1e-3) / 1e12
        workload = f"{kind} dense layer relu(x w + b) {m}x{k}x{n}, {name}"
        lines.append({"workload": workload, "key": f"dense {kind} {m}x{k}x{n} {short}", "spread": spread(ms),
                      "value": achieved, "unit": "TFLOP/s", "ms": ms,
                      "roofline": {"bound": "mfma", "achieved": achieved, "peak": MFMA_PEAK[kind],
                                   "unit": "TFLOP/s", "frac": achieved / MFMA_PEAK[kind],
                                   "traffic": MEASURED_TRAFFIC.get(workload), "bytes": algorithmic},
                      "cpu_baseline": baseline})
    layer.free()
    return lines


class LayerNorm:
    """(x - mean) / sqrt(deviations / cols + 1e-5) * gamma over the rows of an
    f32 rows x cols matrix x, as the two calls the bench times on a given x:
    `one_kernel` (`tc_fused_with_statistics`, one compiled kernel from the
    program's second appearance) and `composed` (`tc_row_moments`, then
    `tc_fused`)."""

    def __init__(self, rows: int, cols: int, rng):
        self.hgamma = rng.uniform(0.5, 1.5, cols).astype(np.float32)
        gamma = lib.Buffer.of(self.hgamma)
        nbytes = rows * cols * 4
        out, means, devs = lib.Buffer(nbytes), lib.Buffer(rows * 4), lib.Buffer(rows * 4)
        self.buffers = [gamma, out, means, devs]
        f32 = lib.F32
        self.program = program = [
            (0, 0, 0, 0, f32, 0, 0.0), (0, 1, 1, 1, f32, 0, 0.0), (0, 2, 2, 2, f32, 0, 0.0),
            (0, 2, 3, 3, f32, 0, 0.0), (1, 0, 4, 0, 0, 0, float(np.float32(1.0 / cols))),
            (2, lib.MUL, 3, 3, 4, 0, 0.0), (1, 0, 4, 0, 0, 0, 1e-5), (2, lib.ADD, 3, 3, 4, 0, 0.0),
            (3, 13, 3, 3, 0, 0, 0.0), (2, lib.SUB, 0, 0, 2, 0, 0.0), (2, lib.DIV, 0, 0, 3, 0, 0.0),
            (2, lib.MUL, 0, 0, 1, 0, 0.0), (5, 0, 0, 0, f32, 0, 0.0)]
        whole = (0, 1, 1, [rows], [cols])
        place_list = [whole, (0, 1, 0, [], []), (0, 0, 1, [rows], [1])]
        enc, places = lib._program(program, place_list)
        _, whole_place = lib._program([], [whole])
        outs, out_lens = lib._buffers([(out, rows * cols)])

        def one_kernel(x):
            ins, in_lens = lib._buffers([(x, rows * cols), (gamma, cols)])
            stats = (lib.Statistic * 2)()
            for i, which in enumerate((lib.STAT_MEAN, lib.STAT_DEVIATIONS)):
                stats[i].source, stats[i].source_len, stats[i].source_dtype = x.ptr, rows * cols, f32
                stats[i].which, stats[i].place = which, whole_place[0]
            lib.call("tc_fused_with_statistics", f32, enc, len(program), places, 3, ins, in_lens, 2, outs, out_lens,
                     1, rows, cols, stats, 2)

        def composed(x):
            lib.call("tc_row_moments", f32, f32, x.ptr, rows * cols, whole_place, rows, cols, means.ptr, devs.ptr)
            ins, in_lens = lib._buffers([(x, rows * cols), (gamma, cols), (means, rows), (devs, rows)])
            lib.call("tc_fused", f32, enc, len(program), places, 3, ins, in_lens, 4, outs, out_lens, 1, rows, cols)

        self.one_kernel, self.composed = one_kernel, composed

    def free(self) -> None:
        for buffer in self.buffers:
            buffer.free()


def layer_norm(rows: int, cols: int, steps: int, warmup: int) -> list[dict]:
    """(x - mean) / sqrt(deviations / cols + 1e-5) * gamma over the rows of an
    f32 matrix, its row statistics read by the program (`fused_with_statistics`,
    kernels.rs:1103): one kernel computing each row's statistics and running
    the program over that row (`tc_fused_with_statistics`, compiled from the
    program's second appearance), against the trait's default composition
    (`tc_row_moments`, then `tc_fused`).  Both lines count x read once and
    the result written once; inputs rotate past the Infinity Cache."""
    from oracle import binding as oracle  # the CPU baseline's restatement

    f32 = lib.F32
    rng = np.random.default_rng(17)
    nbytes = rows * cols * 4
    xs = rotation(lambda: lib.Buffer.of(rng.uniform(-3, 3, rows * cols).astype(np.float32)), nbytes)
    norm = LayerNorm(rows, cols, rng)
    program, hgamma = norm.program, norm.hgamma
    one_kernel, composed = norm.one_kernel, norm.composed

    # The CPU baseline: the oracle's row moments, then its program, over a
    # band of rows.
    band = 64
    hx = rng.uniform(-3, 3, band * cols).astype(np.float32)
    band_whole = (0, 1, 1, [band], [cols])
    band_places = [band_whole, (0, 1, 0, [], []), (0, 0, 1, [band], [1])]
    band_out = np.empty(band * cols, np.float32)

    def cpu():
        m, d = oracle.row_moments(f32, f32, hx, band_whole, band, cols)
        oracle.fused(f32, program, band_places, [hx, hgamma, m, d], [band_out], band, cols)

    baseline = cpu_rate(cpu, 8.0 * band * cols, "GB/s",
                        f"rows 0..{band}: the oracle's row moments, then its program, one thread", 1e9)
    lines = []
    for name, short, fn in (("statistics and program in one kernel", "1 kernel", one_kernel),
                            ("composed: row moments, then the program", "composed", composed)):
        ms = timed_graph(rotating(xs, fn), steps, warmup)
        lines.append(with_cpu(hbm_line(f"layer norm f32 [{rows}x{cols}] (fused_with_statistics), {name}",
                                       2.0 * nbytes, ms, f"layernorm {short}"), baseline))
    for buffer in xs:
        buffer.free()
    norm.free()
    return lines


PCIE_PEAK = 64.0  # GB/s, PCIe 5.0 x16, one direction


def transfers() -> list[dict]:
    """Host to HBM and back, 1 GiB of pageable memory each way: the plain
    runtime copy (`tc_upload`) against the pinned double-buffered staging
    (`tc_upload_staged`), and a TCR1 record of 1 GiB loaded from a file in
    the page cache straight into HBM.  Wall time of each call, which returns
    only when its host side is free."""
    import tempfile

    from oracle import tcr1  # writes the record the loader reads

    nbytes = 1 << 30
    host = np.random.default_rng(5).integers(0, 256, nbytes, dtype=np.uint8)
    back = np.empty_like(host)
    dev = lib.Buffer(nbytes)

    def wall(fn, repeats=3):
        fn()
        lib.sync()
        best = float("inf")
        for _ in range(repeats):
            start = time.perf_counter()
            fn()
            lib.sync()
            best = min(best, time.perf_counter() - start)
        return best * 1e3

    def line(workload, ms, key):
        gbs = nbytes / (ms * 1e-3) / 1e9
        return {"workload": workload, "key": key, "value": gbs, "unit": "GB/s", "ms": ms,
                "roofline": {"bound": "pcie", "achieved": gbs, "peak": PCIE_PEAK, "unit": "GB/s",
                             "frac": gbs / PCIE_PEAK, "traffic": None}}

    lines = [
        line("upload 1 GiB pageable, runtime copy", wall(lambda: lib.call("tc_upload", dev.ptr, host.ctypes.data, nbytes)),
             "upload runtime"),
        line("upload 1 GiB pageable, pinned staging",
             wall(lambda: lib.call("tc_upload_staged", dev.ptr, host.ctypes.data, nbytes)), "upload staged"),
        line("download 1 GiB pageable, runtime copy",
             wall(lambda: lib.call("tc_download", back.ctypes.data, dev.ptr, nbytes)), "download runtime"),
        line("download 1 GiB pageable, pinned staging",
             wall(lambda: lib.call("tc_download_staged", back.ctypes.data, dev.ptr, nbytes)), "download staged"),
    ]
    with tempfile.TemporaryDirectory() as folder:
        path = os.path.join(folder, "x.tcr")
        tag = tcr1.tag("u8")
        with open(path, "wb") as f:
            f.write(tcr1.record(tcr1.VECTOR, [nbytes], tag, host.tobytes()))
        h = lib.Tcr1()
        lib.call("tc_tcr1_read_header", path.encode(), 0, tag, len(tag), tcr1.VECTOR, ctypes.byref(h))
        lines.append(line("TCR1 record of 1 GiB, page-cached file to HBM",
                          wall(lambda: lib.call("tc_tcr1_load", path.encode(), ctypes.byref(h), dev.ptr)), "tcr1 load"))
    dev.free()
    return lines


def spread(ms) -> dict | None:
    """The samples' median, minimum and MAD (a fraction of the median) of a
    `Timing`, as the reference harness reports them."""
    if not isinstance(ms, Timing):
        return None
    return {"samples": ms.samples, "median_ms": ms.median, "min_ms": ms.low, "mad": ms.mad}


def hbm_line(workload: str, nbytes: float, ms: float, key: str) -> dict:
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"workload": workload, "key": key, "value": gbs, "unit": "GB/s", "ms": ms, "spread": spread(ms),
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK, "unit": "GB/s", "frac": gbs / HBM_PEAK,
                         "traffic": MEASURED_TRAFFIC.get(workload)}}


def _host_cpu() -> tuple[str, int]:
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for text in f:
                if text.startswith("model name"):
                    model = text.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return model, len(os.sched_getaffinity(0))


CPU_MODEL, NPROC = _host_cpu()


# CPU baselines are measured after every GPU timing, so that the GPU runs
# its workloads back to back: each line's record is filled in then.
DEFERRED: list = []


# Threads for the Host paths that split over every core: the host's CPUs,
# at most the 16 a one-GPU box's share holds.
HOST_THREADS = max(1, min(NPROC, 16))


def cpu_rate(fn, work: float, unit: str, sample: str, scale: float, min_seconds: float = 0.4,
             chunks: int = 0) -> dict:
    """The oracle's C restatement of the Host (simd) algorithm run on this
    host: `fn` does `work` units of the line's metric per call; called until
    `min_seconds` pass after one untimed call, the rate is work x calls /
    seconds / `scale`.  With `chunks`, a call is `fn(i)` for every chunk i,
    spread over HOST_THREADS threads (the oracle's C calls release the
    interpreter's lock), as the Host splits its elementwise kernels and its
    fused interpreter over every core (parallel.rs:1-14, simd_dispatch.rs:54-75,
    fused/mod.rs:4255-4290).  Returns the line's record, filled in by
    `run_cpu_baselines`."""
    threads = HOST_THREADS if chunks else 1
    record = {"value": None, "unit": unit, "cores": threads, "kind": "port", "sample": sample, "cpu": CPU_MODEL,
              "nproc": NPROC}
    DEFERRED.append((record, fn, work, scale, min_seconds, chunks))
    return record


def run_cpu_baselines() -> None:
    from concurrent.futures import ThreadPoolExecutor

    with ThreadPoolExecutor(HOST_THREADS) as pool:
        while DEFERRED:
            record, fn, work, scale, min_seconds, chunks = DEFERRED.pop(0)
            call = (lambda: list(pool.map(fn, range(chunks)))) if chunks else fn
            call()
            calls, start = 0, time.perf_counter()
            while True:
                call()
                calls += 1
                elapsed = time.perf_counter() - start
                if elapsed >= min_seconds:
                    break
            record["value"] = work * calls / elapsed / scale


def with_cpu(line: dict, baseline: dict) -> dict:
    line["cpu_baseline"] = baseline
    return line


# Inputs smaller than the 256 MiB Infinity Cache would be read back from it
# by back-to-back calls; rotating over copies that together pass 512 MiB keeps
# every call's reads coming from HBM.
COLD_BYTES = 512 << 20


def rotation(make, nbytes: int) -> list:
    return [make() for _ in range(max(1, -(-COLD_BYTES // nbytes)))]


def rotating(inputs: list, call):
    """A zero-argument function calling `call` on the next of `inputs`."""
    turn = itertools.count()
    return lambda: call(inputs[next(turn) % len(inputs)])


def launch_floor(steps: int, warmup: int) -> dict:
    """What one graph-replayed launch costs with no work in it: a copy of one
    f32 element through `tc_strided_copy`, timed as the bandwidth lines are.
    A launch moving B bytes cannot take less than this plus B / 8 TB/s, so at
    32 MiB no single launch reaches more than about 70% of HBM."""
    src, dst = lib.Buffer(16), lib.Buffer(16)
    shape = lib.dims([1])
    at = lib.strided(0, [1])
    ms = timed_graph(lambda: lib.call("tc_strided_copy", 4, src.ptr, 1, 1, shape, ctypes.byref(at), dst.ptr),
                     steps, warmup)
    src.free()
    dst.free()
    us = ms * 1e3
    ceiling = (32 << 20) / ((32 << 20) / (HBM_PEAK * 1e9) + us * 1e-6) / 1e9
    return {"workload": "launch floor: a one-element copy, graph-replayed", "key": "launch floor", "value": us,
            "unit": "us/launch", "spread": spread(ms),
            "higher_is_better": False, "ms": ms,
            "roofline": {"bound": "launch", "achieved": None, "peak": None, "unit": "GB/s", "frac": None,
                         "traffic": None, "ceiling_32MiB_GBps": ceiling},
            "cpu_baseline": None}


def reductions(shape, seed: int, steps: int, warmup: int) -> list[dict]:
    from oracle import binding as oracle  # the CPU baselines' restatement

    rng = np.random.default_rng(seed)
    host = rng.standard_normal(shape, dtype=np.float32)
    n = int(np.prod(shape))
    xs = rotation(lambda: Tensor.from_numpy(host), 4 * n)
    lines = []
    tag = "x".join(map(str, shape))
    size = f"{4 * n >> 20}M"
    # The CPU baseline folds a leading slab of at most 8 Mi elements with the
    # same axes: the Host walk costs the same per element at any size.
    slab_rows = max(1, min(shape[0], (8 << 20) // (shape[1] * shape[2])))
    slab = np.ascontiguousarray(host[:slab_rows])
    slab_shape = [slab_rows, shape[1], shape[2]]
    strides = [shape[1] * shape[2], shape[2], 1]
    sample = f"the oracle's sequential Host walk over [{slab_rows},{shape[1]},{shape[2]}]" + \
        ("" if slab_rows == shape[0] else f", the leading slab of [{tag}]")
    fold_code = {"sum": (lib.FOLD, lib.SUM, 0), "max": (lib.FOLD, lib.RMAX, 0), "min": (lib.FOLD, lib.RMIN, 0)}
    for name, axes, results in [("sum", [2], n // shape[2]), ("max", [2], n // shape[2]),
                                ("min", [2], n // shape[2]), ("mean", [2], n // shape[2]), ("var", [2], n // shape[2]),
                                ("sum", [0, 1], shape[2]), ("max", [0, 1], shape[2]), ("var", [0, 1], shape[2])]:
        fn = rotating(xs, lambda x: getattr(x, f"{name}_axes")(axes))
        ms = timed_graph(fn, max(steps, 2 * len(xs)), warmup)
        line = hbm_line(f"{name}_axes {axes} of f32 [{tag}]", 4 * (n + results), ms,
                        f"{name}[{','.join(map(str, axes))}] {size}")
        depth = int(np.prod([slab_shape[a] for a in axes]))
        kind, op, divisor = fold_code.get(name, (lib.MEAN if name == "mean" else lib.VARIANCE, 0,
                                                 0 if name == "mean" else depth))
        slab_results = int(np.prod(slab_shape)) // depth
        work = 4.0 * (slab.size + slab_results)
        lines.append(with_cpu(line, cpu_rate(
            lambda: oracle.reduce(lib.F32, slab, slab_shape, 0, strides, axes, kind, op, divisor),
            work, "GB/s", sample, 1e9)))
    for name, op in (("argmax", lib.RMAX), ("argmin", lib.RMIN)):
        fn = rotating(xs, lambda x: getattr(x, name)(1))
        ms = timed_graph(fn, max(steps, 2 * len(xs)), warmup)
        line = hbm_line(f"{name} axis 1 of f32 [{tag}]", 4 * n + 4 * (n // shape[1]), ms, f"{name}[1] {size}")
        work = 4.0 * slab.size + 4.0 * (slab.size // shape[1])
        lines.append(with_cpu(line, cpu_rate(
            lambda: oracle.arg_reduce(lib.F32, slab, slab_shape, 0, strides, 1, op), work, "GB/s", sample, 1e9)))
    return lines


def broadcast_and_copies(steps: int, warmup: int) -> list[dict]:
    from oracle import binding as oracle  # the CPU baselines' restatement

    rng = np.random.default_rng(2)
    shape = (256, 512, 512)
    hx = rng.standard_normal(shape, dtype=np.float32)
    hy = rng.uniform(-1, 1, (1, 512, 1)).astype(np.float32)
    hz = rng.uniform(-1, 1, (256, 1, 512)).astype(np.float32)
    x, y, z = Tensor.from_numpy(hx), Tensor.from_numpy(hy), Tensor.from_numpy(hz)
    n = 256 * 512 * 512
    mib = 4 * n
    # CPU baselines run the oracle's Host restatements over the leading
    # [32,512,512] slab (an eighth; the walks cost the same per element).
    rows = 32
    sx, sz = np.ascontiguousarray(hx[:rows]), np.ascontiguousarray(hz[:rows])
    sn = rows * 512 * 512
    slab = f"the oracle's Host walk over the leading [{rows},512,512] slab"
    lines = []
    ms = timed_graph(lambda: x * y, steps, warmup)
    lines.append(with_cpu(hbm_line("x*y, f32 [256,512,512] x [1,512,1]", 2 * mib + 4 * 512, ms, "x*y"), cpu_rate(
        lambda: oracle.binary(lib.F32, lib.ARITHMETIC, lib.MUL, [rows, 512, 512], sx, 0, [262144, 512, 1], hy, 0,
                              [0, 1, 0]), 8.0 * sn + 4 * 512, "GB/s", slab + " (strided.rs:29-78)", 1e9)))
    t = x * y
    st = np.ascontiguousarray(t.to_numpy()[:rows])
    ms = timed_graph(lambda: t + z, steps, warmup)
    lines.append(with_cpu(hbm_line("t+z, f32 [256,512,512] + [256,1,512]", 2 * mib + 4 * 256 * 512, ms, "t+z"), cpu_rate(
        lambda: oracle.binary(lib.F32, lib.ARITHMETIC, lib.ADD, [rows, 512, 512], st, 0, [262144, 512, 1], sz, 0,
                              [512, 0, 1]), 8.0 * sn + 4 * rows * 512, "GB/s", slab + " (strided.rs:29-78)", 1e9)))
    out = t + z
    so = np.ascontiguousarray(out.to_numpy()[:rows])
    ms = timed_graph(lambda: out.permute([0, 2, 1]).contiguous(), steps, warmup)
    lines.append(with_cpu(hbm_line("permute(0,2,1).contiguous, f32 [256,512,512]", 2 * mib, ms, "permute"), cpu_rate(
        lambda: oracle.strided_copy(so, [rows, 512, 512], 0, [262144, 1, 512]), 8.0 * sn, "GB/s",
        slab + " (backend.rs:255-274)", 1e9)))
    p = out.permute([0, 2, 1]).contiguous()
    sp = np.ascontiguousarray(p.to_numpy()[:rows])
    # The slice reads 128 MiB, which the Infinity Cache could hold: rotate.
    sources = rotation(lambda: out.permute([0, 2, 1]).contiguous(), mib // 2)
    ms = timed_graph(rotating(sources, lambda q: q.slice(1, 128, 384).contiguous()), steps, warmup)
    lines.append(with_cpu(hbm_line("slice [:,128:384,:].contiguous, f32", mib, ms, "slice"), cpu_rate(
        lambda: oracle.strided_copy(sp, [rows, 256, 512], 128 * 512, [262144, 512, 1]), 4.0 * sn, "GB/s",
        slab + " (backend.rs:255-274)", 1e9)))
    del sources
    halves = p.chunk(1, 2)
    ms = timed_graph(lambda: Tensor.concat(halves, 1), steps, warmup)

    def assemble_slab():
        # backend.rs:303-323: each half's region copied into its place.
        target = np.empty((rows, 512, 512), np.float32)
        for half in range(2):
            oracle.strided_write(sp, target, [rows, 256, 512], half * 256 * 512, [262144, 512, 1], half * 256 * 512,
                                 [262144, 512, 1])
        return target
    lines.append(with_cpu(hbm_line("concat of two [256,256,512] halves on axis 1, f32", 2 * mib, ms, "concat"), cpu_rate(
        assemble_slab, 8.0 * sn, "GB/s", slab + " (backend.rs:303-323)", 1e9)))
    a, b = x.storage, t.storage
    dst = lib.Buffer(mib)
    ms = timed_graph(lambda: lib.call("tc_elementwise", lib.F32, lib.ADD, a.ptr, b.ptr, dst.ptr, n), steps, warmup)
    ea, eb = sx.reshape(-1), st.reshape(-1)
    # The Host splits a same-shape kernel into windows over every core
    # (simd_dispatch.rs:54-75; four chunks a thread, parallel.rs:28).
    pieces = 4 * HOST_THREADS
    bounds = [sn * i // pieces for i in range(pieces + 1)]
    lines.append(with_cpu(hbm_line("same-shape add, f32 64 Mi elements", 3 * mib, ms, "add"), cpu_rate(
        lambda i: oracle.elementwise(lib.F32, lib.ARITHMETIC, lib.ADD, ea[bounds[i]:bounds[i + 1]],
                                     eb[bounds[i]:bounds[i + 1]]), 12.0 * sn, "GB/s",
        f"the oracle's elementwise loop over {sn} elements in {pieces} windows on {HOST_THREADS} threads "
        "(simd_dispatch.rs:54-75)", 1e9, chunks=pieces)))
    return lines


def vector_products(steps: int, warmup: int) -> list[dict]:
    """GEMV, vecmat and dot at the bandwidth sizes of configs a11, and the
    4096 x 4096 transpose of a12; inputs rotate past the Infinity Cache."""
    from oracle import binding as oracle  # the CPU baselines' restatement

    rng = np.random.default_rng(5)
    rows = cols = 8192
    mbytes = 4 * rows * cols
    host = rng.standard_normal((rows, cols), dtype=np.float32)
    mats = rotation(lambda: lib.Buffer.of(host), mbytes)
    hv = rng.standard_normal(cols, dtype=np.float32)
    v = lib.Buffer.of(hv)
    y = lib.Buffer(4 * rows)
    band = 1024  # CPU baselines: a band of 1024 rows of the matrix
    hb = np.ascontiguousarray(host[:band])
    sample = f"the oracle's Host loop over rows 0..{band} of the [{rows}x{cols}] matrix"
    lines = []
    ms = timed_graph(rotating(mats, lambda m: lib.call("tc_matvec", lib.F32, 0, rows, cols, m.ptr, v.ptr, y.ptr)),
                     max(steps, 2 * len(mats)), warmup)
    lines.append(with_cpu(hbm_line(f"matvec, f32 [{rows}x{cols}] . [{cols}]", mbytes + 4 * (rows + cols), ms, "matvec"),
                          cpu_rate(lambda: oracle.matvec(lib.F32, hb, hv), 4.0 * (band * cols + band + cols), "GB/s",
                                   sample + " (simd_dispatch.rs:626-659)", 1e9)))
    ms = timed_graph(rotating(mats, lambda m: lib.call("tc_vecmat", lib.F32, rows, cols, v.ptr, m.ptr, y.ptr)),
                     max(steps, 2 * len(mats)), warmup)
    hw = np.ascontiguousarray(hv[:band])
    lines.append(with_cpu(hbm_line(f"vecmat, f32 [{rows}] . [{rows}x{cols}]", mbytes + 4 * (rows + cols), ms, "vecmat"),
                          cpu_rate(lambda: oracle.vecmat(lib.F32, hw, hb), 4.0 * (band * cols + band + cols), "GB/s",
                                   sample + " (vector.rs:491)", 1e9)))
    del mats
    n = 64 << 20
    ha, hb2 = rng.standard_normal(n, dtype=np.float32), rng.standard_normal(n, dtype=np.float32)
    a, b = lib.Buffer.of(ha), lib.Buffer.of(hb2)
    result = lib.Buffer(4)
    ms = timed_graph(lambda: lib.call("tc_dot", lib.F32, a.ptr, b.ptr, n, result.ptr), steps, warmup)
    da, db = np.ascontiguousarray(ha[: 8 << 20]), np.ascontiguousarray(hb2[: 8 << 20])
    lines.append(with_cpu(hbm_line("dot, f32 64 Mi elements", 8 * n, ms, "dot"),
                          cpu_rate(lambda: oracle.dot(lib.F32, da, db), 8.0 * da.size, "GB/s",
                                   "the oracle's eight-lane AVX2 dot (simd_x86.rs:57-101) over the first 8 Mi pairs",
                                   1e9)))
    del a, b
    side = 4096
    tbytes = 4 * side * side
    first = rng.standard_normal((side, side), dtype=np.float32)
    srcs = rotation(lambda: lib.Buffer.of(first), tbytes)
    dst = lib.Buffer(tbytes)
    ms = timed_graph(rotating(srcs, lambda m: lib.call("tc_transpose", 4, side, side, m.ptr, dst.ptr)),
                     max(steps, 2 * len(srcs)), warmup)
    lines.append(with_cpu(hbm_line(f"transpose, f32 [{side}x{side}]", 2 * tbytes, ms, "transpose"),
                          cpu_rate(lambda: oracle.transpose(first), 2.0 * tbytes, "GB/s",
                                   f"the oracle's transpose of the whole [{side}x{side}] matrix, one thread "
                                   "(the Host blocks 32 x 32 over all cores, matrix.rs:1173-1206)", 1e9)))
    return lines


def mlp_step(steps: int, warmup: int) -> list[dict]:
    """Configuration 5: the training step of the reference's harness
    (``mlp_step``, benches/nn_ops.rs:875-921) at 1024 -> 4096 -> 4096 -> 1024,
    batch 4096, on the C++ tape: forward, backward and an Adam update of
    every parameter, with nothing read back.  Its work is the 618.5 GFLOP of
    its nine f32 products; the Adam step alone is timed as its own line."""
    from oracle import mlp  # the synthetic network's generator only

    from oracle import binding as oracle  # the CPU baselines' restatement
    from tensorcrate_amd.optim import adam_program, identity_place

    widths, batch = (1024, 4096, 4096, 1024), 4096
    weights, biases = mlp.he_init(widths, 4)
    x, y = mlp.batch_of(widths, batch, 4)
    net = lib.Mlp(widths, batch, weights, biases, x, y, 1e-3)
    # Three steps compile the step's Adam programs (each on its second
    # appearance), then the step runs back to back until the clock settles.
    for _ in range(3):
        net.step()
    lib.sync()
    settle(net.step)
    ms = timed(net.step, steps, warmup)
    flops = sum(2.0 * widths[l] * widths[l + 1] * batch for l in range(3)) * 3
    net.close()
    achieved = flops / (ms * 1e-3) / 1e12
    # The CPU baseline: the step's first product (W0 . X) on a band of W0's
    # rows through the oracle's single-thread f32 Host product, its rate
    # scaled to the step's 618.5 GFLOP, which the nine products dominate.
    band = 64
    w_band = np.ascontiguousarray(weights[1][:band])
    right = np.ascontiguousarray(weights[1])  # a 4096 x 4096 operand of the step's largest products
    baseline = cpu_rate(lambda: oracle.matmul(lib.F32, w_band, right, band, widths[1], widths[2]),
                        2.0 * band * widths[1] * widths[2], "steps/s",
                        f"rows 0..{band} of W1 times a {widths[1]}x{widths[2]} operand: the oracle's single-thread "
                        "AVX2 i-p-j f32 product, its rate divided by the step's 618.5 GFLOP", flops, min_seconds=1.0)
    del weights, biases, x, y
    lines = [{"workload": "MLP training step 1024-4096-4096-1024, batch 4096, f32, tape + Adam (configs[4])",
              "key": "mlp step", "spread": spread(ms),
              "value": 1e3 / ms, "unit": "steps/s", "ms": ms,
              "roofline": {"bound": "mfma", "achieved": achieved, "peak": MFMA_PEAK["f32"], "unit": "TFLOP/s",
                           "frac": achieved / MFMA_PEAK["f32"],
                           "traffic": MEASURED_TRAFFIC.get("MLP training step 1024-4096-4096-1024, batch 4096, f32, "
                                                           "tape + Adam (configs[4])")},
              "cpu_baseline": baseline}]
    # The Adam step over all 25,175,040 parameters as one tensor: reads the
    # gradient, parameters and both moments, writes the last three.
    n = sum(widths[l] * widths[l + 1] + widths[l + 1] for l in range(3))
    params, grads = lib.Buffer(4 * n), lib.Buffer(4 * n)
    lib.call("tc_fill", params.ptr, n, 4, ctypes.byref(ctypes.c_float(0.5)))
    lib.call("tc_fill", grads.ptr, n, 4, ctypes.byref(ctypes.c_float(0.25)))
    rule = Adam(1e-3)
    rule.update(params, grads, 1, n)
    # Graph-captured like the other bandwidth lines: each captured update
    # keeps its own step's constants, and the replay times the kernels back
    # to back rather than this script's per-step host work.
    ms = timed_graph(lambda: rule.update(params, grads, 1, n), steps, warmup)
    # The CPU baseline: the oracle's interpreter over 8 Mi parameters, split
    # into windows over every core as the Host's tile interpreter splits a
    # program (fused/mod.rs:4255-4290).
    sample_n = 8 << 20
    pieces = 4 * HOST_THREADS
    window = -(-sample_n // pieces)
    code, loads = adam_program(True, lib.F32, 1e-3, 0.9, 0.999, 1e-8, 2)
    hp = np.full(sample_n, 0.5, np.float32)
    hg, hm, hv = np.full(sample_n, 0.25, np.float32), np.zeros(sample_n, np.float32), np.zeros(sample_n, np.float32)

    def adam_window(i):
        at = slice(i * window, min(sample_n, (i + 1) * window))
        count = at.stop - at.start
        if count > 0:
            views = [a[at] for a in (hg, hp, hm, hv)]
            oracle.fused(lib.F32, code, [identity_place(1, count)] * loads, views, views[1:], 1, count)
    lines.append(with_cpu(hbm_line(f"Adam update, {n} f32 parameters (fused program)", 7 * 4 * n, ms, "adam"), cpu_rate(
        adam_window, 7.0 * 4 * sample_n, "GB/s",
        f"the oracle's program interpreter over {sample_n} parameters in {pieces} windows on {HOST_THREADS} threads "
        "(fused/mod.rs:4255-4290)", 1e9, chunks=pieces)))
    return lines


def traffic_probe(part: str = "all") -> None:
    """A short run for ``rocprofv3 --pmc FETCH_SIZE`` / ``WRITE_SIZE``, each
    kernel launched eagerly so every dispatch is one workload's: three plain
    contiguous copies of 1 GiB through ``tc_strided_copy`` (the rows kernel;
    1 GiB read and 1 GiB written each, the counters' calibration), then
    (part "kernels" or "all") three launches of the headline product, three
    of the f16 16384 x 1024 x 4096 product, three each of the f32 4096^3
    product in its PLAIN, LEFT and RIGHT forms and one call of every
    bandwidth workload, then (part "programs" or "all") one call of every
    fused and training workload, in the order ``traffic_workloads`` lists
    them, each between two marker launches (a 1 x 1 ``tc_flip``) after its
    untimed calls.  The parts split the probe into two processes."""
    n = 1 << 28
    src, dst = lib.Buffer(4 * n), lib.Buffer(4 * n)
    lib.call("tc_fill", src.ptr, n, 4, ctypes.byref(ctypes.c_float(1.0)))
    shape = lib.dims([n])
    at = lib.strided(0, [1])
    for _ in range(3):
        lib.call("tc_strided_copy", 4, src.ptr, n, 1, shape, ctypes.byref(at), dst.ptr)
    lib.sync()
    src.free()
    dst.free()
    if part != "programs":
        product_probe()
    one, flipped = lib.Buffer(16), lib.Buffer(16)

    def marker():
        lib.call("tc_flip", 4, one.ptr, 1, 1, flipped.ptr)
        lib.sync()
    for workload, run, untimed in traffic_workloads(part):
        log(f"probe: {workload}")
        for _ in range(untimed):
            run()
        lib.sync()
        marker()
        run()
        lib.sync()
        marker()
    log("traffic probe done")


def product_probe() -> None:
    """The traffic probe's products, three eager launches each."""
    m = k = n = 8192
    rng = np.random.default_rng(3)
    a = lib.Buffer.of(host_matrix("bf16", m, k, rng, 1 / np.sqrt(k)))
    b = lib.Buffer.of(host_matrix("bf16", k, n, rng, 1 / np.sqrt(k)))
    c = lib.Buffer(m * n * 2)
    for _ in range(3):
        lib.call("tc_matmul", lib.BF16, lib.BF16, lib.PLAIN, 0, m, k, n, a.ptr, b.ptr, c.ptr)
    lib.sync()
    for buffer in (a, b, c):
        buffer.free()
    # The f16 skinny product of the sweep, as its workload line runs it.
    m, k, n = 16384, 1024, 4096
    a = lib.Buffer.of(host_matrix("f16", m, k, rng, 1 / np.sqrt(k)))
    b = lib.Buffer.of(host_matrix("f16", k, n, rng, 1 / np.sqrt(k)))
    c = lib.Buffer(m * n * 2)
    for _ in range(3):
        lib.call("tc_matmul", lib.F16, lib.F16, lib.PLAIN, 0, m, k, n, a.ptr, b.ptr, c.ptr)
    lib.sync()
    for buffer in (a, b, c):
        buffer.free()
    # The f32 4096^3 product in each form the MLP step's products take:
    # PLAIN (A.B), LEFT (A^T.B, the weight gradients), RIGHT (A.B^T).
    m = k = n = 4096
    a = lib.Buffer.of(host_matrix("f32", m, k, rng, None))
    b = lib.Buffer.of(host_matrix("f32", k, n, rng, None))
    c = lib.Buffer(m * n * 4)
    for form in (lib.PLAIN, lib.LEFT, lib.RIGHT):
        for _ in range(3):
            lib.call("tc_matmul", lib.F32, lib.F32, form, 0, m, k, n, a.ptr, b.ptr, c.ptr)
    lib.sync()
    for buffer in (a, b, c):
        buffer.free()


# Each workload's dispatches lie between two markers (a 1 x 1 flip, a kernel
# none of them uses), after its untimed calls: a workload of several kernels
# (the MLP step, the composed layer norm) is the sum between.
def traffic_workloads(part: str = "all"):
    """(workload, call, untimed calls first) for every bandwidth line (part
    "kernels") and the fused and training lines (part "programs"), in a
    fixed order, each call on inputs made beforehand (so the probe's
    dispatches are the calls')."""
    calls = []
    if part != "programs":
        calls += bandwidth_workloads()
    if part != "kernels":
        calls += program_workloads()
    return calls


def bandwidth_workloads():
    """The bandwidth lines' calls for the traffic probe."""
    rng = np.random.default_rng(2)
    x = Tensor.from_numpy(rng.standard_normal((256, 512, 512), dtype=np.float32))
    y = Tensor.from_numpy(rng.uniform(-1, 1, (1, 512, 1)).astype(np.float32))
    z = Tensor.from_numpy(rng.uniform(-1, 1, (256, 1, 512)).astype(np.float32))
    t = x * y
    out = t + z
    p = out.permute([0, 2, 1]).contiguous()
    halves = p.chunk(1, 2)
    n = 256 * 512 * 512
    dst = lib.Buffer(4 * n)
    small = Tensor.from_numpy(rng.standard_normal((64, 128, 1024), dtype=np.float32))
    large = Tensor.from_numpy(rng.standard_normal((1024, 128, 1024), dtype=np.float32))
    mat = lib.Buffer.of(rng.standard_normal((8192, 8192), dtype=np.float32))
    vec = lib.Buffer.of(rng.standard_normal(8192, dtype=np.float32))
    yv = lib.Buffer(4 * 8192)
    da = lib.Buffer.of(rng.standard_normal(64 << 20, dtype=np.float32))
    db = lib.Buffer.of(rng.standard_normal(64 << 20, dtype=np.float32))
    dot_out = lib.Buffer(4)
    sq = lib.Buffer.of(rng.standard_normal((4096, 4096), dtype=np.float32))
    sq_t = lib.Buffer(4 * 4096 * 4096)
    keep = (x, y, z, t, out, p, halves, dst, small, large, mat, vec, yv, da, db, dot_out, sq, sq_t)
    calls = [
        ("x*y, f32 [256,512,512] x [1,512,1]", lambda: x * y),
        ("t+z, f32 [256,512,512] + [256,1,512]", lambda: t + z),
        ("permute(0,2,1).contiguous, f32 [256,512,512]", lambda: out.permute([0, 2, 1]).contiguous()),
        ("slice [:,128:384,:].contiguous, f32", lambda: p.slice(1, 128, 384).contiguous()),
        ("concat of two [256,256,512] halves on axis 1, f32", lambda: Tensor.concat(halves, 1)),
        ("same-shape add, f32 64 Mi elements",
         lambda: lib.call("tc_elementwise", lib.F32, lib.ADD, x.storage.ptr, t.storage.ptr, dst.ptr, n)),
    ]
    for tag, tensor in (("64x128x1024", small), ("1024x128x1024", large)):
        calls += [
            (f"sum_axes [2] of f32 [{tag}]", lambda tensor=tensor: tensor.sum_axes([2])),
            (f"var_axes [2] of f32 [{tag}]", lambda tensor=tensor: tensor.var_axes([2])),
            (f"sum_axes [0, 1] of f32 [{tag}]", lambda tensor=tensor: tensor.sum_axes([0, 1])),
            (f"var_axes [0, 1] of f32 [{tag}]", lambda tensor=tensor: tensor.var_axes([0, 1])),
            (f"argmax axis 1 of f32 [{tag}]", lambda tensor=tensor: tensor.argmax(1)),
        ]
    # Plain 32 MiB streams beside the 32 MiB reductions: what one launch of
    # that size reaches when it only reads, or only copies.
    plain = lib.Buffer.of(rng.standard_normal(8 << 20, dtype=np.float32))
    plain_out, plain_sum = lib.Buffer(32 << 20), lib.Buffer(4)
    keep += (plain, plain_out, plain_sum)
    calls += [
        ("read of 32 MiB (vector_reduce sum), f32",
         lambda: lib.call("tc_vector_reduce", lib.F32, plain.ptr, 8 << 20, lib.SUM, plain_sum.ptr)),
        ("copy of 32 MiB, f32", lambda: lib.call("tc_copy", plain_out.ptr, plain.ptr, 32 << 20)),
    ]
    calls += [
        ("matvec, f32 [8192x8192] . [8192]",
         lambda: lib.call("tc_matvec", lib.F32, 0, 8192, 8192, mat.ptr, vec.ptr, yv.ptr)),
        ("vecmat, f32 [8192] . [8192x8192]",
         lambda: lib.call("tc_vecmat", lib.F32, 8192, 8192, vec.ptr, mat.ptr, yv.ptr)),
        ("dot, f32 64 Mi elements", lambda: lib.call("tc_dot", lib.F32, da.ptr, db.ptr, 64 << 20, dot_out.ptr)),
        ("transpose, f32 [4096x4096]", lambda: lib.call("tc_transpose", 4, 4096, 4096, sq.ptr, sq_t.ptr)),
    ]
    bandwidth_workloads.keep = keep
    return [(name, call, 0) for name, call in calls]


def program_workloads():
    """The workloads of several kernels or compiled programs, each run
    untimed first as many times as its timed line's warmup needs (the
    programs compile on their second appearance)."""
    rng = np.random.default_rng(2)
    norm = LayerNorm(8192, 8192, np.random.default_rng(17))
    ln_x = lib.Buffer.of(rng.uniform(-3, 3, 8192 * 8192).astype(np.float32))
    dense_bf16, dense_f32 = DenseLayer("bf16", 8192, 8192, 8192), DenseLayer("f32", 4096, 1024, 4096)
    from oracle import mlp  # the synthetic network's generator only

    widths = (1024, 4096, 4096, 1024)
    weights, biases = mlp.he_init(widths, 4)
    mx, my = mlp.batch_of(widths, 4096, 4)
    net = lib.Mlp(widths, 4096, weights, biases, mx, my, 1e-3)
    count = sum(widths[l] * widths[l + 1] + widths[l + 1] for l in range(3))
    params, grads = lib.Buffer(4 * count), lib.Buffer(4 * count)
    lib.call("tc_fill", params.ptr, count, 4, ctypes.byref(ctypes.c_float(0.5)))
    lib.call("tc_fill", grads.ptr, count, 4, ctypes.byref(ctypes.c_float(0.25)))
    rule = Adam(1e-3)
    program_workloads.keep = (norm, ln_x, dense_bf16, dense_f32, net, params, grads, rule)
    return [
        ("layer norm f32 [8192x8192] (fused_with_statistics), statistics and program in one kernel",
         lambda: norm.one_kernel(ln_x), 2),
        ("layer norm f32 [8192x8192] (fused_with_statistics), composed: row moments, then the program",
         lambda: norm.composed(ln_x), 2),
        ("Adam update, 25175040 f32 parameters (fused program)", lambda: rule.update(params, grads, 1, count), 3),
        ("MLP training step 1024-4096-4096-1024, batch 4096, f32, tape + Adam (configs[4])", net.step, 3),
        ("bf16 dense layer relu(x w + b) 8192x8192x8192, in the product's epilogue", dense_bf16.fused, 2),
        ("bf16 dense layer relu(x w + b) 8192x8192x8192, unfused: product, then program", dense_bf16.unfused, 2),
        ("f32 dense layer relu(x w + b) 4096x1024x4096, in the product's epilogue", dense_f32.fused, 2),
        ("f32 dense layer relu(x w + b) 4096x1024x4096, unfused: product, then program", dense_f32.unfused, 2),
    ]


def cpu_baseline(m: int, k: int, n: int) -> dict:
    """The oracle's restatement of the Host (simd) bf16 product —
    widen, i-p-j AVX2 FMA on one thread, round once (compact.rs:232-253,
    simd_x86.rs:1302-1327) — on a band of rows of A against all of B, scaled
    linearly in M (the i-p-j loop is linear in rows)."""
    from oracle import binding as oracle

    rng = np.random.default_rng(3)
    sigma = 1 / np.sqrt(k)
    b = halfconv.bf16_bits(rng.standard_normal((k, n), dtype=np.float32) * np.float32(sigma))
    rows = 2
    while True:
        a = halfconv.bf16_bits(rng.standard_normal((rows, k), dtype=np.float32) * np.float32(sigma))
        start = time.perf_counter()
        oracle.matmul(oracle.BF16, a, b, rows, k, n)
        seconds = time.perf_counter() - start
        if seconds >= 10.0 or rows >= m:
            break
        rows = min(m, max(rows * 2, int(rows * 12.0 / max(seconds, 1e-3))))
    flops = 2.0 * rows * k * n
    return {"value": flops / seconds / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"rows 0..{rows} of A ({rows} of {m}) times all of B, bf16 {m}x{k}x{n}: the oracle's "
                      f"widen + single-thread AVX2 i-p-j FMA + round-once, {seconds:.1f} s, scaled linearly in M",
            "cpu": CPU_MODEL, "nproc": NPROC}


def secondary(groups: set, steps: int, warmup: int) -> list[dict]:
    """The other configurations' lines, each with its own roofline."""
    workloads = []
    if "gemm" in groups:
        log("f32 GEMM 4096^3 ...")
        workloads.append(gemm("f32", 4096, 4096, 4096, 3, None, steps, warmup, cpu=True))
        log("f16 GEMM 16384x4096x1024 ...")
        workloads.append(gemm("f16", 16384, 1024, 4096, 3, 1 / np.sqrt(1024), steps, warmup, cpu=True))
    if "reductions" in groups:
        log("reductions ...")
        workloads.append(launch_floor(steps, warmup))
        workloads += reductions((64, 128, 1024), 1, steps, warmup)
        workloads += reductions((1024, 128, 1024), 1, max(steps // 2, 5), warmup)
    if "copies" in groups:
        log("broadcast chain and copies ...")
        workloads += broadcast_and_copies(steps, warmup)
    if "vectors" in groups:
        log("matvec, vecmat, dot, transpose ...")
        workloads += vector_products(steps, warmup)
    if "transfer" in groups:
        log("host transfers and TCR1 loads ...")
        workloads += transfers()
    if "mlp" in groups:
        log("MLP training step and Adam ...")
        # Three untimed steps: Adam's programs compile on their second
        # appearance, and the streaming one (the 4096 x 4096 weight) appears
        # once a step from the second step on.
        workloads += mlp_step(max(steps // 4, 3), 3)
    if "fusion" in groups:
        # Last: the bf16 8192^3 products, so that a headline timed next runs
        # in the power state of sustained matrix-core work.
        log("dense layers, fused and unfused ...")
        workloads += layer_norm(8192, 8192, steps, max(warmup, 3))
        workloads += dense_layer("f32", 4096, 1024, 4096, steps, warmup)
        workloads += dense_layer("bf16", 8192, 8192, 8192, steps, warmup)
    for line in workloads:
        frac = line["roofline"]["frac"]
        log(f"  {line['workload']}: {line['value']:.1f} {line['unit']}" + (f" ({frac * 100:.1f}%)" if frac else ""))
    return workloads


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    # The part ramps its clock over the first few dozen launches of a dense
    # product (1.01 ms, then 0.88 ms, for the headline): the untimed warmup
    # covers the ramp so the timed steps are the steady state.
    parser.add_argument("--warmup", type=int, default=30)
    parser.add_argument("--quick", action="store_true", help="headline only, no secondary workloads or CPU baseline")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--traffic-probe", nargs="?", const="all", choices=["all", "kernels", "programs"],
                        help="only the short run that HBM-traffic counters are read over (optionally one part: "
                             "the kernels' workloads or the compiled programs')")
    parser.add_argument("--only", default="",
                        help="comma-separated secondary groups to run alone (gemm, reductions, copies, vectors, fusion, transfer, mlp); "
                             "prints their lines as a JSON list instead of the headline line")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path, so --gpus must be 1", file=sys.stderr)
        return 2
    lib.call("tc_init", 0)
    name, arch = lib.device_info()
    log(f"device {name} {arch}")
    if args.traffic_probe:
        traffic_probe(args.traffic_probe)
        return 0

    if args.only:
        groups = set(args.only.split(","))
        unknown = groups - {"gemm", "reductions", "copies", "vectors", "fusion", "transfer", "mlp"}
        if unknown:
            print(f"bench.py: no workload group {sorted(unknown)}", file=sys.stderr)
            return 2
        workloads = secondary(groups, args.steps, args.warmup)
        if not args.no_cpu:
            run_cpu_baselines()
        print(json.dumps(workloads), flush=True)
        return 0

    m = k = n = 8192
    # The headline's operands are made and uploaded first; the other
    # workloads then run, the bf16 8192^3 dense layers last, and the
    # headline's W warmup and K timed steps follow them at once, so the timed
    # steps see the part's sustained-load clock rather than the ramp a cold
    # part goes through over its first few dozen dense products.
    head_operands = Product("bf16", m, k, n, 3, 1 / np.sqrt(k))
    workloads = []
    if not args.quick:
        workloads = secondary({"gemm", "reductions", "copies", "vectors", "fusion", "mlp"}, args.steps, args.warmup)
    log("bf16 GEMM 8192^3 ...")
    head = head_operands.time(args.steps, args.warmup)
    log(f"  {head['value']:.1f} TFLOP/s ({head['ms']:.3f} ms/step), kernel {head['roofline']['achieved']:.1f}")
    baseline = None
    if not args.quick and not args.no_cpu:
        log("CPU baselines ...")
        run_cpu_baselines()
        baseline = cpu_baseline(m, k, n)
        log(f"  {baseline['value'] * 1e3:.2f} GFLOP/s on one core")
    for w in workloads:
        if w.get("cpu_baseline") is not None and w["cpu_baseline"]["value"] is None:
            w["cpu_baseline"] = None
    # Every workload's full record goes to stderr as one JSON object; the
    # last stdout line is the compact headline.
    log("workloads: " + json.dumps(workloads))
    line = headline_line(head, baseline, workloads, args.steps, args.warmup, f"{name} {arch}")
    print(json.dumps(line, separators=(",", ":")), flush=True)
    return 0


# The fields of each entry of the headline line's "workloads" table.
WORKLOAD_FIELDS = ["value", "unit", "frac", "traffic_ratio", "mad", "cpu"]


def _round(value, digits=5):
    return None if value is None else float(f"{value:.{digits}g}")


def compact(line: dict) -> list:
    """A workload as one row of the headline's table: value, unit, fraction
    of its roofline, HBM traffic over algorithmic bytes, the samples' MAD as
    a fraction of their median, and the CPU baseline's value."""
    roof = line.get("roofline") or {}
    ratio = None
    if roof.get("traffic") and line.get("ms"):
        if roof.get("unit") == "GB/s" and roof.get("achieved"):
            ratio = roof["traffic"] / (roof["achieved"] * 1e9 * line["ms"] * 1e-3)
        elif roof.get("bytes"):
            ratio = roof["traffic"] / roof["bytes"]
    cpu = line.get("cpu_baseline") or {}
    return [_round(line["value"]), line["unit"], _round(roof.get("frac"), 3), _round(ratio, 3),
            _round((line.get("spread") or {}).get("mad"), 2), _round(cpu.get("value"), 3)]


def headline_line(head: dict, baseline: dict | None, workloads: list[dict], steps: int, warmup: int,
                  device: str) -> dict:
    """The one JSON line the driver reads: BASELINE.json's metric on the bf16
    8192^3 product, its roofline and CPU baseline, and every other workload
    as a compact row keyed by a short name (full records go to stderr)."""
    roof = {k: (_round(v) if isinstance(v, float) else v) for k, v in head["roofline"].items()}
    roof["traffic"] = HEADLINE_TRAFFIC
    cpu = None
    if baseline is not None:
        cpu = {k: (_round(v) if isinstance(v, float) else v) for k, v in baseline.items()}
    return {
        "metric": METRIC,
        "value": _round(head["value"], 5),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": _round(head["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: A, B ~ N(0, 1/sqrt(K)) bf16, seed 3, numpy PCG64",
        "config": {"workload": "dense GEMM bf16 M=N=K=8192, f32 accumulate, bf16 out (configs[3])",
                   "m": 8192, "n": 8192, "k": 8192, "device": device},
        "spread": {k: (_round(v) if isinstance(v, float) else v) for k, v in (head.get("spread") or {}).items()},
        "roofline": roof,
        "cpu_baseline": cpu,
        "workload_fields": WORKLOAD_FIELDS,
        "workloads": {w["key"]: compact(w) for w in workloads},
    }


if __name__ == "__main__":
    sys.exit(main())
