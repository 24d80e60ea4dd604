"""The matrix product's program epilogue (`tc_matmul_epilogue` through the
matrix-core kernels; `Kernels::matmul_epilogue`, kernels.rs:1142,
`Program::run_matmul`, fused/mod.rs:1143-1215) against the unfused
computation the host runs (`host_matmul`, fused/mod.rs:4751-4764): the
product rounded to the program's type, then the program.  The fused kernels
accumulate exactly as `tc_matmul` does and run the same interpreter, so the
two agree bit for bit, at every tile shape, edge and type."""

import ctypes

import numpy as np
import pytest

from tensorcrate_amd import lib
from tests.common import EXP, Code, column_broadcast, identity_place, row_broadcast, to_kind

pytestmark = pytest.mark.gpu

HOST = {lib.F32: np.float32, lib.F16: np.float16, lib.BF16: np.uint16}


def bias_relu(kind):
    code = Code()
    p = code.load(0, 0, kind)
    b = code.load(1, 1, kind)
    shifted = code.binary(lib.ADD, p, b)
    code.store(code.compare(lib.MAX, shifted, code.const(0.0)), kind, 0)
    return code.code, 1


def scaled_two_outputs(kind):
    # out0 = product * scale[row] + bias[col]; out1 = exp(product) in f32; the
    # product read twice.
    code = Code()
    p = code.load(0, 0, kind)
    s = code.load(2, 2, kind)
    b = code.load(1, 1, kind)
    code.store(code.binary(lib.ADD, code.binary(lib.MUL, p, s), b), kind, 0)
    again = code.load(0, 0, kind)
    code.store(code.unary(EXP, again), lib.F32, 1)
    return code.code, 2


PROGRAMS = {"bias_relu": bias_relu, "scaled_two_outputs": scaled_two_outputs}


def run_both(kind, program, m, k, n, seed):
    rng = np.random.default_rng(seed)
    a = to_kind(rng.uniform(-1, 1, (m, k)).astype(np.float32), kind)
    b = to_kind(rng.uniform(-1, 1, (k, n)).astype(np.float32), kind)
    bias = to_kind(rng.uniform(-1, 1, n).astype(np.float32), kind)
    scale = to_kind(rng.uniform(0.5, 2, m).astype(np.float32), kind)
    code, outputs = PROGRAMS[program](kind)
    places = [identity_place(m, n), row_broadcast(n), column_broadcast(m)]
    da, db, dbias, dscale = (lib.Buffer.of(x) for x in (a, b, bias, scale))
    inputs = [(dbias, n)] + ([(dscale, m)] if outputs == 2 else [])
    widths = [HOST[kind](0).itemsize, 4][:outputs]
    fused = [lib.Buffer(m * n * w) for w in widths]
    lib.matmul_epilogue(kind, code, places, da, db, m, k, n, inputs, [(f, m * n) for f in fused])
    # Unfused: the product in the program's type, then the program over it.
    product = lib.Buffer(m * n * widths[0])
    lib.call("tc_matmul", kind, kind, lib.PLAIN, 0, m, k, n, da.ptr, db.ptr, product.ptr)
    plain = [lib.Buffer(m * n * w) for w in widths]
    lib.fused(kind, code, places, [(product, m * n)] + inputs, [(p, m * n) for p in plain], m, n)
    dtypes = [HOST[kind], np.float32][:outputs]
    return ([f.download(t, m * n) for f, t in zip(fused, dtypes)],
            [p.download(t, m * n) for p, t in zip(plain, dtypes)])


SHAPES = [(8, 8, 8), (64, 64, 64), (300, 256, 520), (1024, 512, 1024), (4096, 64, 4096), (4100, 72, 4104)]


@pytest.mark.parametrize("kind", [lib.F32, lib.BF16, lib.F16])
@pytest.mark.parametrize("program", sorted(PROGRAMS))
@pytest.mark.parametrize("m,k,n", SHAPES)
def test_fused_epilogue_matches_the_unfused_computation(kind, program, m, k, n):
    fused, plain = run_both(kind, program, m, k, n, m + k + n + kind)
    for got, want in zip(fused, plain):
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8))


def test_the_reference_example_through_the_fused_kernel():
    # fused/mod.rs:1103-1125 at a size the matrix-core kernel takes: relu(x w
    # + bias) with x w exact in f32.
    m, k, n = 16, 8, 16
    x = np.zeros((m, k), np.float32)
    x[:2, :2] = [[1, 2], [3, 4]]
    w = np.zeros((k, n), np.float32)
    w[:2, :2] = [[1, -1], [0, 1]]
    bias = np.zeros(n, np.float32)
    bias[:2] = [0.5, -2.5]
    code, _ = bias_relu(lib.F32)
    out = lib.Buffer(m * n * 4)
    lib.matmul_epilogue(lib.F32, code, [identity_place(m, n), row_broadcast(n)], lib.Buffer.of(x), lib.Buffer.of(w),
                        m, k, n, [(lib.Buffer.of(bias), n)], [(out, m * n)])
    y = out.download(np.float32, m * n).reshape(m, n)
    assert y[:2, :2].tolist() == [[1.5, 0.0], [3.5, 0.0]]
    # The zero rows are relu(bias): 0.5 in column 0, zeros elsewhere.
    assert np.all(y[2:, 0] == 0.5) and np.all(y[2:, 1:] == 0) and np.all(y[:2, 2:] == 0)


def test_the_product_must_be_read_in_order():
    # fused/mod.rs:1185-1190.
    m, k, n = 16, 16, 16
    code, _ = bias_relu(lib.F32)
    transposed = (0, m, 1, [m], [1])
    a = lib.Buffer.of(np.ones((m, k), np.float32))
    out = lib.Buffer(m * n * 4)
    with pytest.raises(lib.HipError, match="the product is read through a remap"):
        lib.matmul_epilogue(lib.F32, code, [transposed, row_broadcast(n)], a, a, m, k, n,
                            [(lib.Buffer.of(np.ones(n, np.float32)), n)], [(out, m * n)])


@pytest.mark.parametrize("kind", [lib.F32, lib.BF16, lib.F16])
@pytest.mark.parametrize("m,k,n", [(520, 136, 1032), (4100, 136, 4104), (4100, 200, 4104), (4100, 256, 4104)],
                         ids=["small-tiles", "large-tiles", "persistent", "four-wave"])
def test_a_repeated_program_runs_compiled_with_the_same_bits(kind, m, k, n):
    # The first appearance of a program runs the interpreter epilogue; from
    # the second the program is compiled into the product kernel (as the
    # reference's Metal backend specializes a program seen before).  All
    # give the unfused bits: in the kernel for fewer 256 x 256 tiles than
    # CUs, in the one-tile kernel for more (17 x 17 tiles, ragged, three
    # steps), and, for 16-bit types with a whole pair of steps, in the
    # eight-wave persistent kernel, or with K a multiple of 128 in the
    # four-wave one.  Compiled kernels are cached by source, constants being
    # arguments, so each case has a program of its own shape: the bias added
    # for the small tiles, subtracted for the large ones, the scaled
    # product's maximum with the bias for the persistent ones, and the
    # minimum of product plus bias with a constant for the four-wave ones.
    code = Code()
    p = code.load(0, 0, kind)
    b = code.load(1, 1, kind)
    if k == 256:
        summed = code.binary(lib.ADD, p, b)
        code.store(code.compare(lib.MIN, summed, code.const(0.5 + kind)), kind, 0)
    elif k == 200:
        scaled = code.binary(lib.MUL, p, code.const(0.375 + kind))
        code.store(code.compare(lib.MAX, scaled, b), kind, 0)
    else:
        shifted = code.binary(lib.SUB if m > 1000 else lib.ADD, p, b)
        scaled = code.binary(lib.MUL, shifted, code.const(0.375 + kind))
        code.store(code.compare(lib.MAX, scaled, code.const(-0.25)), kind, 0)
    rng = np.random.default_rng(kind)
    a = to_kind(rng.uniform(-1, 1, (m, k)).astype(np.float32), kind)
    w = to_kind(rng.uniform(-1, 1, (k, n)).astype(np.float32), kind)
    bias = to_kind(rng.uniform(-1, 1, n).astype(np.float32), kind)
    places = [identity_place(m, n), row_broadcast(n)]
    da, dw, db = lib.Buffer.of(a), lib.Buffer.of(w), lib.Buffer.of(bias)
    width = HOST[kind](0).itemsize
    results = []
    compiled = []
    for _ in range(3):
        out = lib.Buffer(m * n * width)
        lib.matmul_epilogue(kind, code.code, places, da, dw, m, k, n, [(db, n)], [(out, m * n)])
        results.append(out.download(HOST[kind], m * n))
        count = ctypes.c_uint64()
        lib.call("tc_fused_compiled", ctypes.byref(count))
        compiled.append(count.value)
    assert compiled[1] == compiled[0] + 1 and compiled[2] == compiled[1]  # compiled once, on the second call
    product = lib.Buffer(m * n * width)
    lib.call("tc_matmul", kind, kind, lib.PLAIN, 0, m, k, n, da.ptr, dw.ptr, product.ptr)
    plain = lib.Buffer(m * n * width)
    lib.fused(kind, code.code, places, [(product, m * n), (db, n)], [(plain, m * n)], m, n)
    want = plain.download(HOST[kind], m * n)
    for got in results:
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8))


def residual_scaled(kind):
    # out0 = max(product * scale[row] + bias[col], 0) + residual[row, col];
    # out1 = the product in f32.  Every kind of load the four-wave kernel's
    # run form takes: a row-invariant run (the bias), one value a row (the
    # scale), a run a row (the residual), and a second output of another type.
    code = Code()
    p = code.load(0, 0, kind)
    s = code.load(2, 2, kind)
    b = code.load(1, 1, kind)
    r = code.load(3, 3, kind)
    y = code.compare(lib.MAX, code.binary(lib.ADD, code.binary(lib.MUL, p, s), b), code.const(0.0))
    code.store(code.binary(lib.ADD, y, r), kind, 0)
    code.store(code.load(0, 0, kind), lib.F32, 1)
    return code.code


@pytest.mark.parametrize("kind", [lib.BF16, lib.F16])
@pytest.mark.parametrize("m,k,n,skew", [(4100, 256, 4104, 0), (4100, 256, 4100, 0), (4100, 256, 4104, 1)],
                         ids=["runs", "columns-not-whole-runs", "misaligned-bias"])
def test_four_wave_epilogue_forms_give_the_unfused_bits(kind, m, k, n, skew):
    # With N a multiple of 8 and every operand 16-byte aligned the compiled
    # four-wave epilogue takes whole runs of eight columns (the bias loaded
    # once a half tile, 16-byte loads and stores); with N not a multiple of 8,
    # or a bias one element off 16 bytes, it takes the element form.  Both
    # give the unfused bits on every call, ragged tiles on both edges
    # included (17 x 17 tiles of 256).
    rng = np.random.default_rng(kind * 10 + skew + n)
    a = to_kind(rng.uniform(-1, 1, (m, k)).astype(np.float32), kind)
    w = to_kind(rng.uniform(-1, 1, (k, n)).astype(np.float32), kind)
    bias = to_kind(rng.uniform(-1, 1, n + skew).astype(np.float32), kind)
    scale = to_kind(rng.uniform(0.5, 2, m).astype(np.float32), kind)
    residual = to_kind(rng.uniform(-1, 1, (m, n)).astype(np.float32), kind)
    code = residual_scaled(kind)
    places = [identity_place(m, n), (skew, 1, 0, [], []), column_broadcast(m), identity_place(m, n)]
    da, dw, db, ds, dr = (lib.Buffer.of(x) for x in (a, w, bias, scale, residual))
    inputs = [(db, n + skew), (ds, m), (dr, m * n)]
    width = HOST[kind](0).itemsize
    results = []
    for _ in range(3):  # the interpreter, then compiled from the second call
        outs = [lib.Buffer(m * n * width), lib.Buffer(m * n * 4)]
        lib.matmul_epilogue(kind, code, places, da, dw, m, k, n, inputs, [(o, m * n) for o in outs])
        results.append((outs[0].download(HOST[kind], m * n), outs[1].download(np.float32, m * n)))
    product = lib.Buffer(m * n * width)
    lib.call("tc_matmul", kind, kind, lib.PLAIN, 0, m, k, n, da.ptr, dw.ptr, product.ptr)
    plain = [lib.Buffer(m * n * width), lib.Buffer(m * n * 4)]
    lib.fused(kind, code, places, [(product, m * n)] + inputs, [(p, m * n) for p in plain], m, n)
    want = (plain[0].download(HOST[kind], m * n), plain[1].download(np.float32, m * n))
    for call, got in enumerate(results):
        for g, wt in zip(got, want):
            assert np.array_equal(g.view(np.uint8), wt.view(np.uint8)), call
