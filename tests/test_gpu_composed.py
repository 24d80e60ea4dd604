"""The composed `Kernels` members on the GPU — `tc_row_moments`,
`tc_fused_sum`, `tc_matmul_epilogue`, and `fused_with_statistics` as the
trait's default composes it (kernels.rs:1090-1149) — against the oracle on
the same inputs, and against the reference's known answers.

Tolerances: moments and sums fold in a different order from the host's
left-to-right loop, so they are held to the accumulated-rounding bound
(2^-24 sqrt(n) of the magnitudes summed, plus the output's rounding); the
epilogue's product to the f32 product tolerance 1e-5 sqrt(K) of sum|a||b|,
the program after it then being the same arithmetic."""

import math

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib
from tests.common import EXP, Code, Lcg, column_broadcast, identity_place, row_broadcast, to_kind, widen
from tests.test_oracle_composed import PLACES, exp_program, layer_norm, oracle_at, relu_layer, statistic_operands

pytestmark = pytest.mark.gpu

UNIT = {lib.F32: 2.0 ** -24, lib.F16: 2.0 ** -11, lib.BF16: 2.0 ** -8}
HOST = {lib.F32: np.float32, lib.F16: np.float16, lib.BF16: np.uint16}


def device_moments(dtype, input_dtype, source, place, rows, cols):
    buf = lib.Buffer.of(source)
    size = 4 if dtype == lib.F32 else 2
    means, devs = lib.Buffer(max(rows, 1) * size), lib.Buffer(max(rows, 1) * size)
    lib.row_moments(dtype, input_dtype, buf, source.size, place, rows, cols, means, devs)
    return means.download(HOST[dtype], rows), devs.download(HOST[dtype], rows)


@pytest.mark.parametrize("name,make", PLACES)
@pytest.mark.parametrize("dtype,input_dtype", [(lib.F32, lib.F32), (lib.F32, lib.F16), (lib.BF16, lib.F32),
                                               (lib.F16, lib.F16), (lib.BF16, lib.BF16)])
@pytest.mark.parametrize("rows,cols", [(6, 37), (130, 1000), (3, 1)])
def test_row_moments_against_the_oracle(name, make, dtype, input_dtype, rows, cols):
    place, length = make(rows, cols)
    rng = np.random.default_rng(rows * cols + dtype * 7 + input_dtype)
    source = to_kind(rng.uniform(-3, 3, length), input_dtype)
    got_mean, got_dev = device_moments(dtype, input_dtype, source, place, rows, cols)
    want_mean, want_dev = oracle.row_moments(dtype, input_dtype, source, place, rows, cols)
    values = widen(input_dtype, source).astype(np.float64)
    scale = np.array([max(abs(values[oracle_at(place, r, c)]) for c in range(cols)) for r in range(rows)])
    gm, wm = widen(dtype, got_mean), widen(dtype, want_mean)
    gd, wd = widen(dtype, got_dev), widen(dtype, want_dev)
    root = np.sqrt(cols)
    assert np.all(np.abs(gm - wm) <= 4 * root * 2.0 ** -24 * scale + 2 * UNIT[dtype] * np.abs(wm) + 1e-30), name
    assert np.all(np.abs(gd - wd) <= 8 * cols * root * 2.0 ** -24 * scale ** 2 + 2 * UNIT[dtype] * wd + 1e-30), name


def test_row_moments_of_empty_rows_are_nans():
    got_mean, got_dev = device_moments(lib.F32, lib.F32, np.zeros(4, np.float32), identity_place(4, 0), 4, 0)
    assert np.all(np.isnan(got_mean)) and np.all(np.isnan(got_dev))


def device_fused_sum(dtype, code, places, inputs, rows, cols, axis):
    bufs = [(lib.Buffer.of(x), x.size) for x in inputs]
    n = rows if axis == 0 else cols
    out = lib.Buffer(max(n, 1) * (4 if dtype == lib.F32 else 2))
    lib.fused_sum(dtype, code, places, bufs, rows, cols, axis, out)
    return out.download(HOST[dtype], n)


def test_fused_sum_known_answer():
    x = np.array([0.0, 0.0, 1.0, 0.0], np.float32)
    sums = device_fused_sum(lib.F32, exp_program(), [identity_place(2, 2)], [x], 2, 2, 0)
    assert sums[0] == 2.0
    assert abs(sums[1] - (math.e + 1.0)) <= 2 * 2.0 ** -24 * (math.e + 1.0)


@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("rows,cols", [(1, 1), (33, 70), (1024, 512), (5, 100000)])
def test_fused_sum_against_the_oracle(axis, rows, cols):
    rng = np.random.default_rng(rows + cols + axis)
    x = rng.uniform(-1, 1, rows * cols).astype(np.float32)
    got = device_fused_sum(lib.F32, exp_program(), [identity_place(rows, cols)], [x], rows, cols, axis)
    want = oracle.fused_sum(lib.F32, exp_program(), [identity_place(rows, cols)], [x], rows, cols, axis)
    depth = cols if axis == 0 else rows
    magnitude = np.exp(x.reshape(rows, cols).astype(np.float64)).sum(1 - axis)
    assert np.all(np.abs(got - want) <= 4 * np.sqrt(depth) * 2.0 ** -24 * magnitude + 2.0 ** -24 * magnitude)


def test_fused_sum_over_empty_rows_is_zero():
    got = device_fused_sum(lib.F32, exp_program(), [identity_place(3, 0)], [np.zeros(1, np.float32)], 3, 0, 0)
    assert got.tolist() == [0.0, 0.0, 0.0]


def device_epilogue(code, places, a, b, m, k, n, inputs):
    da, db = lib.Buffer.of(a), lib.Buffer.of(b)
    bufs = [(lib.Buffer.of(x), x.size) for x in inputs]
    out = lib.Buffer(m * n * 4)
    lib.matmul_epilogue(lib.F32, code, places, da, db, m, k, n, bufs, [(out, m * n)])
    return out.download(np.float32, m * n)


def test_matmul_epilogue_known_answer():
    x = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    w = np.array([[1.0, -1.0], [0.0, 1.0]], np.float32)
    bias = np.array([0.5, -2.5], np.float32)
    y = device_epilogue(relu_layer(), [identity_place(2, 2), row_broadcast(2)], x, w, 2, 2, 2, [bias])
    assert y.reshape(2, 2).tolist() == [[1.5, 0.0], [3.5, 0.0]]


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 2), (16, 16, 16), (17, 33, 15), (65, 130, 67), (128, 7, 200),
                                   (1024, 512, 768)])
def test_matmul_epilogue_against_the_oracle(m, k, n):
    # The shapes of tests/fused.rs:1466-1475, and one past every tile edge.
    rng = Lcg(31 + m)
    a = rng.uniform(-1.0, 1.0, m * k).astype(np.float32)
    b = rng.uniform(-1.0, 1.0, k * n).astype(np.float32)
    bias = rng.uniform(-1.0, 1.0, n).astype(np.float32)
    places = [identity_place(m, n), row_broadcast(n)]
    got = device_epilogue(relu_layer(), places, a, b, m, k, n, [bias])
    want = np.zeros(m * n, np.float32)
    oracle.matmul_epilogue(lib.F32, relu_layer(), places, a, b, m, k, n, [bias], [want])
    scale = (np.abs(a.reshape(m, k).astype(np.float64)) @ np.abs(b.reshape(k, n))).reshape(-1) + np.abs(np.tile(bias, m))
    assert np.all(np.abs(got - want) <= 1e-5 * np.sqrt(k) * scale)


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 5), (9, 31), (17, 64), (40, 1000), (300, 7), (4096, 1024)])
def test_fused_with_statistics_against_the_oracle(rows, cols):
    # The layer norm of tests/fused.rs:1855-1879 with its statistics from
    # tc_row_moments (one computation per input), then tc_fused.
    rng = Lcg(5150 + rows)
    if rows * cols > 100000:
        np_rng = np.random.default_rng(rows)
        x = np_rng.uniform(-3, 3, rows * cols).astype(np.float32)
        gamma = np_rng.uniform(0.5, 1.5, cols).astype(np.float32)
        h = np_rng.uniform(-1, 1, rows * cols).astype(np.float16)
        start = np_rng.uniform(-1, 1, rows * cols).astype(np.float32)
    else:
        x, gamma, h, start = statistic_operands(rng, rows, cols)
    code, places = layer_norm(rows, cols)
    whole = identity_place(rows, cols)
    dx, dg, dh, dacc = (lib.Buffer.of(v) for v in (x, gamma, h, start))
    normalized = lib.Buffer(rows * cols * 4)
    lib.fused_with_statistics(lib.F32, code, places, [(dx, x.size), (dg, cols), (dh, h.size), (dacc, start.size)],
                              [(dacc, start.size), (normalized, rows * cols)], rows, cols,
                              [(dx, x.size, lib.F32, whole, "mean"), (dx, x.size, lib.F32, whole, "deviations"),
                               (dh, h.size, lib.F16, whole, "mean")])
    mean, devs = oracle.row_moments(lib.F32, lib.F32, x, whole, rows, cols)
    other, _ = oracle.row_moments(lib.F32, lib.F16, h, whole, rows, cols)
    acc = start.copy()
    want = np.zeros(rows * cols, np.float32)
    oracle.fused(lib.F32, code, places, [x, gamma, h, acc, mean, devs, other], [acc, want], rows, cols)
    got = normalized.download(np.float32, rows * cols)
    # Normalized values are O(1); the statistics' rounding moves them by a
    # few units of the mean's and the deviation's last places.
    tol = 64 * np.sqrt(cols) * 2.0 ** -24 * 4.0
    assert np.max(np.abs(got - want)) <= tol
    assert np.max(np.abs(dacc.download(np.float32, rows * cols) - acc)) <= 2 * tol


@pytest.mark.parametrize("dtype", [lib.F32, lib.BF16])
def test_row_sums_of_a_repeated_program_run_as_one_compiled_kernel(dtype):
    # From the program's second appearance its row sums are one kernel that
    # never stores the output; every run agrees with the oracle to the
    # summation bound.  exp(x) * 0.5 + 0.25 is this test's own program.
    import ctypes

    code = Code()
    x = code.load(0, 0, dtype)
    y = code.binary(lib.ADD, code.binary(lib.MUL, code.unary(EXP, x), code.const(0.5)), code.const(0.25))
    code.store(y, dtype, 0)
    rows, cols = 300, 5000
    rng = np.random.default_rng(dtype)
    values = to_kind(rng.uniform(-1, 1, rows * cols).astype(np.float32), dtype)
    want = widen(dtype, oracle.fused_sum(dtype, code.code, [identity_place(rows, cols)], [values], rows, cols, 0))
    exact = (np.exp(widen(dtype, values).astype(np.float64)) * 0.5 + 0.25).reshape(rows, cols).sum(1)
    unit = 2.0 ** -24 if dtype == lib.F32 else 2.0 ** -8
    counts = []
    for _ in range(3):
        got = widen(dtype, device_fused_sum(dtype, code.code, [identity_place(rows, cols)], [values], rows, cols, 0))
        # Per element: three operations rounded to the type (and exp's own
        # error); per sum: a lane's run of cols / 64 additions and a 64-lane
        # tree in f32, then the result rounded to the type.  The oracle sums
        # left to right, within cols 2^-24 of the exact sum.
        bound = (4 * unit + 2 * (cols / 64 + 8) * 2.0 ** -24) * exact + unit * exact
        assert np.all(np.abs(got - exact) <= bound)
        assert np.all(np.abs(got - want) <= bound + (4 * unit + cols * 2.0 ** -24) * exact)
        count = ctypes.c_uint64()
        lib.call("tc_fused_compiled", ctypes.byref(count))
        counts.append(count.value)
    assert counts[1] == counts[0] + 1 and counts[2] == counts[1]


@pytest.mark.parametrize("axis", [0, 1], ids=["row-sums", "column-sums"])
@pytest.mark.parametrize("dtype,rows,cols", [(lib.F32, 8192, 8192), (lib.BF16, 8192, 16384)])
def test_sums_of_a_program_over_256_mib_of_runs(dtype, rows, cols, axis):
    # Compiled row or column sums whose runs read 256 MiB or more load them
    # non-temporally; every call (the first may compose, later ones run
    # compiled) agrees with the oracle to the summation bound.
    # exp(x) * 0.5 - 0.25 is this test's own program.
    code = Code()
    x = code.load(0, 0, dtype)
    y = code.binary(lib.SUB, code.binary(lib.MUL, code.unary(EXP, x), code.const(0.5)), code.const(0.25))
    code.store(y, dtype, 0)
    rng = np.random.default_rng(dtype + axis)
    values = to_kind(rng.uniform(-1, 1, rows * cols).astype(np.float32), dtype)
    want = widen(dtype, oracle.fused_sum(dtype, code.code, [identity_place(rows, cols)], [values], rows, cols, axis))
    exact = (np.exp(widen(dtype, values).astype(np.float64)) * 0.5 - 0.25).reshape(rows, cols).sum(1 - axis)
    magnitude = (np.exp(widen(dtype, values).astype(np.float64)) * 0.5 + 0.25).reshape(rows, cols).sum(1 - axis)
    unit = 2.0 ** -24 if dtype == lib.F32 else 2.0 ** -8
    depth = cols if axis == 0 else rows
    # Per element: three operations rounded to the type (and exp's own
    # error); per sum: at most `depth` additions in f32, then the result
    # rounded to the type; the oracle within depth 2^-24 of the exact sum.
    bound = (4 * unit + 2 * (depth + 8) * 2.0 ** -24) * magnitude + unit * np.abs(exact)
    for _ in range(3):
        got = widen(dtype, device_fused_sum(dtype, code.code, [identity_place(rows, cols)], [values], rows, cols,
                                            axis))
        assert np.all(np.abs(got - exact) <= bound)
        assert np.all(np.abs(got - want) <= bound + (4 * unit + depth * 2.0 ** -24) * magnitude)


@pytest.mark.parametrize("dtype", [lib.F32, lib.BF16])
@pytest.mark.parametrize("rows,cols", [(300, 5000), (5000, 64), (33, 70), (7, 100000)],
                         ids=["wide", "tall-split-rows", "ragged", "few-rows"])
def test_column_sums_of_a_repeated_program_run_compiled(dtype, rows, cols):
    # From the program's second appearance its column sums are computed
    # without storing the output: a kernel over 64-column tiles, the rows
    # split over workgroups when the columns are few (5000 x 64), the splits'
    # sums added by a second kernel; every run agrees with the oracle to the
    # summation bound.
    import ctypes

    code = Code()
    x = code.load(0, 0, dtype)
    y = code.binary(lib.ADD, code.binary(lib.MUL, code.unary(EXP, x), code.const(0.5)), code.const(0.25))
    # A product by 1 per case (exact in every type), so each case's program
    # is its own source and compiles on its own second appearance.
    for _ in range([(300, 5000), (5000, 64), (33, 70), (7, 100000)].index((rows, cols))):
        y = code.binary(lib.MUL, y, code.const(1.0))
    code.store(y, dtype, 0)
    rng = np.random.default_rng(dtype + rows)
    values = to_kind(rng.uniform(-1, 1, rows * cols).astype(np.float32), dtype)
    want = widen(dtype, oracle.fused_sum(dtype, code.code, [identity_place(rows, cols)], [values], rows, cols, 1))
    exact = (np.exp(widen(dtype, values).astype(np.float64)) * 0.5 + 0.25).reshape(rows, cols).sum(0)
    unit = 2.0 ** -24 if dtype == lib.F32 else 2.0 ** -8
    counts = []
    for _ in range(3):
        got = widen(dtype, device_fused_sum(dtype, code.code, [identity_place(rows, cols)], [values], rows, cols, 1))
        # Per element: three operations rounded to the type (and exp's own
        # error); per sum: at most `rows` additions in f32, then the result
        # rounded to the type.  The oracle sums in its own order, within
        # rows 2^-24 of the exact sum.
        bound = (4 * unit + 2 * (rows + 8) * 2.0 ** -24) * exact + unit * exact
        assert np.all(np.abs(got - exact) <= bound)
        assert np.all(np.abs(got - want) <= bound + (4 * unit + rows * 2.0 ** -24) * exact)
        count = ctypes.c_uint64()
        lib.call("tc_fused_compiled", ctypes.byref(count))
        counts.append(count.value)
    assert counts[1] == counts[0] + 1 and counts[2] == counts[1]


@pytest.mark.parametrize("shape", [(300, 777), (40, 8300), (301, 1024), (64, 8192), (33, 4100), (41, 3000),
                                   (8, 33000)])
@pytest.mark.parametrize("dtype", [lib.F32, lib.BF16])
def test_fused_with_statistics_runs_as_one_compiled_kernel(dtype, shape):
    # From the program's second appearance its statistics and the program run
    # as one kernel (the statistics never stored): compiled once, and every
    # run, composed or compiled, within the statistics' rounding of the
    # oracle.  (x - mean) / (deviations / cols + 1) is this test's own
    # program; the moments fold in another order than the oracle's, which
    # moves the statistics by their last place at most.  Rows of 777 are
    # not whole 16-byte packs in f32, and rows of 33000 hold more than 64
    # values a lane over four waves: both take the general form.  The others
    # take the form that holds the row in registers and feeds the program's
    # load of x from them: a wave a row for 1024 (301 rows: the last
    # workgroup's four waves have one row), two for 3000 (41 rows: the last
    # workgroup's second pair of waves has none), four for 4100, 8192 and
    # 8300 (whose last packs fall past the row on some lanes).  A shape may
    # find its kernel compiled already; either way the last call is one
    # launch.
    check_one_kernel_statistics(dtype, *shape)


@pytest.mark.parametrize("dtype,rows,cols", [(lib.F32, 8192, 8192), (lib.BF16, 8192, 16384)])
def test_one_kernel_statistics_of_a_source_as_large_as_the_infinity_cache(dtype, rows, cols):
    # A source of 256 MiB or more is read with non-temporal loads, each row
    # once, and meets the same bound.
    check_one_kernel_statistics(dtype, rows, cols)


def check_one_kernel_statistics(dtype, rows, cols):
    """(x - mean) / (deviations / cols + 1) through fused_with_statistics,
    three calls, each within the statistics' rounding of the oracle; the
    last one launch."""
    import ctypes

    code = Code()
    x = code.load(0, 0, dtype)
    mean = code.load(1, 1, dtype)
    deviations = code.load(1, 2, dtype)
    centered = code.binary(lib.SUB, x, mean)
    scale = code.binary(lib.ADD, code.binary(lib.MUL, deviations, code.const(np.float32(1.0 / cols))),
                        code.const(1.0))
    code.store(code.binary(lib.DIV, centered, scale), dtype, 0)
    places = [identity_place(rows, cols), column_broadcast(rows)]
    whole = identity_place(rows, cols)
    xs = to_kind(np.random.default_rng(dtype).uniform(-3, 3, rows * cols).astype(np.float32), dtype)
    dx = lib.Buffer.of(xs)
    means, devs = oracle.row_moments(dtype, dtype, xs, whole, rows, cols)
    want = np.zeros(rows * cols, HOST[dtype])
    oracle.fused(dtype, code.code, places, [xs, means, devs], [want], rows, cols)
    want = widen(dtype, want).astype(np.float64)
    tol = 4 * UNIT[dtype] * np.max(np.abs(want)) + 64 * np.sqrt(cols) * 2.0 ** -24 * 4
    compiled = []
    for _ in range(3):
        out = lib.Buffer(rows * cols * np.dtype(HOST[dtype]).itemsize)
        before = lib.activity()[0]
        lib.fused_with_statistics(dtype, code.code, places, [(dx, xs.size)], [(out, rows * cols)], rows, cols,
                                  [(dx, xs.size, dtype, whole, "mean"), (dx, xs.size, dtype, whole, "deviations")])
        launches = lib.activity()[0] - before
        got = widen(dtype, out.download(HOST[dtype], rows * cols)).astype(np.float64)
        assert np.max(np.abs(got - want)) <= tol
        count = ctypes.c_uint64()
        lib.call("tc_fused_compiled", ctypes.byref(count))
        compiled.append(count.value)
    assert compiled[1] - compiled[0] in (0, 1) and compiled[2] == compiled[1]
    assert launches == 1


@pytest.mark.parametrize("cols", [777, 1024, 3000, 8192])
@pytest.mark.parametrize("offset", [1000.0, 10000.0])
def test_row_statistics_of_offset_rows_keep_two_pass_accuracy(offset, cols):
    # Rows whose mean is large against their spread (offset + U(-1, 1)): the
    # one-kernel statistics, in either of their forms (the row held in
    # registers by one, two or four waves for 1024, 3000 and 8192 columns,
    # the batched walk for 777), shift
    # each row by its first element, and are at least as close to the exact
    # moments as the reference's own two passes (the oracle's sequential f32
    # mean, then squared deviations from it, statistics/mod.rs:419-441), or
    # within 1e-5 of them relative.  The composition's moments (the first
    # call) come from the axis-reduction kernels' variance fold, which merges
    # unshifted chunk moments: it is held to the f32 accumulation bound
    # cols * 2^-24 of the deviations instead.
    import ctypes

    rows = 64
    rng = np.random.default_rng(int(offset) + cols)
    xs = (offset + rng.uniform(-1, 1, rows * cols)).astype(np.float32)
    code = Code()
    code.store(code.load(1, 1, lib.F32), lib.F32, 0)
    code.store(code.load(1, 2, lib.F32), lib.F32, 1)
    places = [identity_place(rows, cols), column_broadcast(rows)]
    whole = identity_place(rows, cols)
    dx = lib.Buffer.of(xs)
    exact = xs.reshape(rows, cols).astype(np.float64)
    exact_mean = exact.mean(axis=1)
    exact_dev = ((exact - exact_mean[:, None]) ** 2).sum(axis=1)
    ref_mean, ref_dev = oracle.row_moments(lib.F32, lib.F32, xs, whole, rows, cols)
    ref_mean_err = np.abs(ref_mean.astype(np.float64) - exact_mean)
    ref_dev_err = np.abs(ref_dev.astype(np.float64) - exact_dev)
    for call in range(2):  # composed, then the compiled kernel
        means, devs = lib.Buffer(rows * cols * 4), lib.Buffer(rows * cols * 4)
        lib.fused_with_statistics(lib.F32, code.code, places, [(dx, xs.size)], [(means, rows * cols),
                                                                               (devs, rows * cols)], rows, cols,
                                  [(dx, xs.size, lib.F32, whole, "mean"), (dx, xs.size, lib.F32, whole, "deviations")])
        got_mean = means.download(np.float32, rows * cols).reshape(rows, cols)[:, 0].astype(np.float64)
        got_dev = devs.download(np.float32, rows * cols).reshape(rows, cols)[:, 0].astype(np.float64)
        mean_err, dev_err = np.abs(got_mean - exact_mean), np.abs(got_dev - exact_dev)
        assert np.all(mean_err <= np.maximum(2 * ref_mean_err, 4 * np.spacing(np.float32(offset)))), call
        relative = 1e-5 if call else cols * 2.0 ** -24
        assert np.all(dev_err <= np.maximum(2 * ref_dev_err, relative * exact_dev)), \
            (call, dev_err.max(), ref_dev_err.max())


@pytest.mark.parametrize("cols", [1024, 3000, 8192])
@pytest.mark.parametrize("dtype", [lib.F32, lib.BF16])
def test_a_division_by_a_statistic_keeps_the_divisions_bits(dtype, cols):
    # The one-kernel form divides by a function of the row's statistics with
    # one reciprocal a row and a product an element (the f32 division kept
    # for any quotient not a normal float).  The program also stores the
    # statistics it read, so the oracle can run the same program on them:
    # every quotient must be its bits, for one, two and four waves a row,
    # and from the composed first call too.
    rows = 33
    code = Code()
    x = code.load(0, 0, dtype)
    mean = code.load(1, 1, dtype)
    deviations = code.load(1, 2, dtype)
    scale = code.binary(lib.MUL, deviations, code.const(np.float32(1.0 / cols)))
    code.store(code.binary(lib.DIV, code.binary(lib.SUB, x, mean), scale), dtype, 0)
    code.store(mean, dtype, 1)
    code.store(deviations, dtype, 2)
    places = [identity_place(rows, cols), column_broadcast(rows)]
    whole = identity_place(rows, cols)
    xs = to_kind(np.random.default_rng(cols).uniform(-3, 3, rows * cols).astype(np.float32), dtype)
    dx = lib.Buffer.of(xs)
    host = np.float32 if dtype == lib.F32 else np.uint16
    for call in range(3):
        out = [lib.Buffer(rows * cols * np.dtype(host).itemsize) for _ in range(3)]
        lib.fused_with_statistics(dtype, code.code, places, [(dx, xs.size)], [(o, rows * cols) for o in out],
                                  rows, cols,
                                  [(dx, xs.size, dtype, whole, "mean"), (dx, xs.size, dtype, whole, "deviations")])
        got = [o.download(host, rows * cols) for o in out]
        means = got[1].reshape(rows, cols)[:, 0].copy()
        devs = got[2].reshape(rows, cols)[:, 0].copy()
        want = np.zeros(rows * cols, host)
        oracle.fused(dtype, code.code[:-2], places, [xs, means, devs], [want], rows, cols)
        assert np.array_equal(got[0].view(np.uint32 if dtype == lib.F32 else np.uint16),
                              want.view(np.uint32 if dtype == lib.F32 else np.uint16)), call
