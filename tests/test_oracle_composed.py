"""The oracle's composed `Kernels` members — `row_moments`, `fused_sum`,
`matmul_epilogue` and the `fused_with_statistics` default (kernels.rs:
1090-1149) — pinned on the CPU against the reference's own known answers
(the `run_sum` and `run_matmul` examples, fused/mod.rs:1030-1040 and
:1103-1125; the layer-norm statistics test, tests/fused.rs:1855-1972),
against numpy in f64, and against their definitions as compositions."""

import math

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib
from tests.common import EXP, SQRT, Code, Lcg, column_broadcast, identity_place, row_broadcast, to_kind, widen


def test_row_moments_known_answer_and_empty_rows():
    x = np.array([1, 2, 3, 4, 5, 6], np.float32)
    means, devs = oracle.row_moments(lib.F32, lib.F32, x, identity_place(2, 3), 2, 3)
    assert means.tolist() == [2.0, 5.0] and devs.tolist() == [2.0, 2.0]
    means, devs = oracle.row_moments(lib.F32, lib.F32, x, identity_place(2, 0), 2, 0)
    assert np.all(np.isnan(means)) and np.all(np.isnan(devs))


def _pair(rows):
    return 2 if rows % 2 == 0 else 1


# Places over a rows x cols walk, and the length of input each reads.
PLACES = [
    ("rows", lambda r, c: ((0, 1, 1, [r], [c]), r * c)),
    ("every other column", lambda r, c: ((1, 2, 1, [r], [2 * c]), 2 * r * c + 1)),
    ("two lead axes", lambda r, c: ((0, 1, 2, [r // _pair(r), _pair(r)], [c * _pair(r), c]), r * c)),
    ("one repeated row", lambda r, c: ((0, 1, 0, [], []), c)),
    ("transposed", lambda r, c: ((0, r, 1, [r], [1]), r * c)),
]


@pytest.mark.parametrize("name,make", PLACES)
@pytest.mark.parametrize("dtype,input_dtype", [(lib.F32, lib.F32), (lib.F32, lib.F16), (lib.BF16, lib.F32),
                                               (lib.F16, lib.F16)])
def test_row_moments_against_f64(name, make, dtype, input_dtype):
    rows, cols = 6, 37
    place, length = make(rows, cols)
    rng = np.random.default_rng(rows * cols + dtype * 7 + input_dtype)
    source = to_kind(rng.uniform(-3, 3, length), input_dtype)
    means, devs = oracle.row_moments(dtype, input_dtype, source, place, rows, cols)
    # The matrix the place reads, converted to the program's type, in f64.
    values = widen(input_dtype, source).astype(np.float32)
    matrix = np.array([[values[oracle_at(place, r, c)] for c in range(cols)] for r in range(rows)], np.float32)
    matrix = widen(dtype, to_kind(matrix, dtype)).astype(np.float64)
    want_mean = matrix.mean(1)
    want_dev = ((matrix - want_mean[:, None]) ** 2).sum(1)
    unit = {lib.F32: 2.0 ** -24, lib.F16: 2.0 ** -11, lib.BF16: 2.0 ** -8}[dtype]
    scale = np.abs(matrix).max(1)
    assert np.all(np.abs(widen(dtype, means) - want_mean) <= cols * 2.0 ** -24 * scale + unit * np.abs(want_mean))
    assert np.all(np.abs(widen(dtype, devs) - want_dev) <= cols * 2.0 ** -22 * scale ** 2 + unit * want_dev)


def oracle_at(place, row, col):
    """`Place::at` (fused/mod.rs:3256-3268)."""
    offset, col_step, lead, dims, steps = place
    at = offset + col * col_step
    if lead > 0:
        for k in range(lead - 1, 0, -1):
            at += (row % dims[k]) * steps[k]
            row //= dims[k]
        at += row * steps[0]
    return at


def exp_program():
    code = Code()
    x = code.load(0, 0, lib.F32)
    code.store(code.unary(EXP, x), lib.F32, 0)
    return code.code


def test_fused_sum_known_answer():
    # fused/mod.rs:1030-1040: the row sums of exp over [[0, 0], [1, 0]] are
    # [2, e + 1].
    x = np.array([0.0, 0.0, 1.0, 0.0], np.float32)
    sums = oracle.fused_sum(lib.F32, exp_program(), [identity_place(2, 2)], [x], 2, 2, 0)
    assert sums[0] == 2.0
    assert sums[1] == np.float32(math.exp(1.0)) + np.float32(1.0)
    columns = oracle.fused_sum(lib.F32, exp_program(), [identity_place(2, 2)], [x], 2, 2, 1)
    assert columns.tolist() == [float(np.float32(1.0) + np.float32(math.exp(1.0))), 2.0]


@pytest.mark.parametrize("axis", [0, 1])
def test_fused_sum_is_the_output_summed(axis):
    rng = np.random.default_rng(3 + axis)
    rows, cols = 33, 70
    x = rng.uniform(-1, 1, rows * cols).astype(np.float32)
    out = np.zeros(rows * cols, np.float32)
    oracle.fused(lib.F32, exp_program(), [identity_place(rows, cols)], [x], [out], rows, cols)
    sums = oracle.fused_sum(lib.F32, exp_program(), [identity_place(rows, cols)], [x], rows, cols, axis)
    want = out.reshape(rows, cols).astype(np.float64).sum(1 - axis)
    assert np.allclose(sums, want, rtol=1e-5 * np.sqrt(cols if axis == 0 else rows))


def relu_layer():
    """relu(product + bias): the `run_matmul` example (fused/mod.rs:1103-1125)."""
    code = Code()
    p = code.load(0, 0, lib.F32)
    b = code.load(1, 1, lib.F32)
    shifted = code.binary(lib.ADD, p, b)
    zero = code.const(0.0)
    code.store(code.compare(lib.MAX, shifted, zero), lib.F32, 0)
    return code.code


def test_matmul_epilogue_known_answer():
    x = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    w = np.array([[1.0, -1.0], [0.0, 1.0]], np.float32)
    bias = np.array([0.5, -2.5], np.float32)
    y = np.zeros(4, np.float32)
    oracle.matmul_epilogue(lib.F32, relu_layer(), [identity_place(2, 2), row_broadcast(2)], x, w, 2, 2, 2, [bias],
                           [y])
    assert y.reshape(2, 2).tolist() == [[1.5, 0.0], [3.5, 0.0]]


def test_matmul_epilogue_is_the_product_then_the_program_bit_for_bit():
    # tests/fused.rs:1508-1530.
    rng = Lcg(31)
    for m, k, n in [(1, 1, 1), (3, 5, 2), (17, 33, 15), (65, 130, 67), (128, 7, 200)]:
        a = np.array(rng.uniform(-1.0, 1.0, m * k), np.float32)
        b = np.array(rng.uniform(-1.0, 1.0, k * n), np.float32)
        bias = np.array(rng.uniform(-1.0, 1.0, n), np.float32)
        places = [identity_place(m, n), row_broadcast(n)]
        fused = np.zeros(m * n, np.float32)
        oracle.matmul_epilogue(lib.F32, relu_layer(), places, a, b, m, k, n, [bias], [fused])
        product = oracle.matmul(lib.F32, a, b, m, k, n).reshape(-1)
        by_hand = np.zeros(m * n, np.float32)
        oracle.fused(lib.F32, relu_layer(), places, [product, bias], [by_hand], m, n)
        assert np.array_equal(fused.view(np.uint32), by_hand.view(np.uint32)), (m, k, n)


def layer_norm(rows, cols):
    """acc += γ·(x − mean)/√(dev/n + ε) + mean(h), and the normalized x
    (tests/fused.rs:1855-1879).  Slots: 0 x, 1 γ, 2 h (read only for its
    statistic), 3 acc (updated in place), then the statistics: 4 mean(x),
    5 deviations(x), 6 mean(h)."""
    places = [identity_place(rows, cols), row_broadcast(cols), column_broadcast(rows)]
    code = Code()
    x = code.load(0, 0, lib.F32)
    gamma = code.load(1, 1, lib.F32)
    acc = code.load(0, 3, lib.F32)
    mean = code.load(2, 4, lib.F32)
    deviations = code.load(2, 5, lib.F32)
    other = code.load(2, 6, lib.F32)
    variance = code.binary(lib.MUL, deviations, code.const(np.float32(1.0 / cols)))
    stabilized = code.binary(lib.ADD, variance, code.const(1e-5))
    deviation = code.unary(SQRT, stabilized)
    centered = code.binary(lib.SUB, x, mean)
    normalized = code.binary(lib.DIV, centered, deviation)
    scaled = code.binary(lib.MUL, normalized, gamma)
    shifted = code.binary(lib.ADD, scaled, other, dst=scaled)
    nxt = code.binary(lib.ADD, acc, shifted, dst=acc)
    code.store(nxt, lib.F32, 0)
    code.store(normalized, lib.F32, 1)
    return code.code, places


def statistic_operands(rng, rows, cols):
    h = np.array([np.float16(v) for v in rng.uniform(-1.0, 1.0, rows * cols)], np.float16)
    return (np.array(rng.uniform(-3.0, 3.0, rows * cols), np.float32), np.array(rng.uniform(0.5, 1.5, cols), np.float32),
            h, np.array(rng.uniform(-1.0, 1.0, rows * cols), np.float32))


def test_row_statistics_feed_the_program_as_the_hand_formula_says():
    # tests/fused.rs:1929-1971, on the oracle: the statistics computed by
    # row_moments, appended as inputs, and the program's bits equal to the
    # formula evaluated by hand in the program's order.
    rng = Lcg(5150)
    for rows, cols in [(1, 1), (3, 5), (9, 31), (17, 64), (40, 1000), (300, 7)]:
        x, gamma, h, start = statistic_operands(rng, rows, cols)
        code, places = layer_norm(rows, cols)
        mean, devs = oracle.row_moments(lib.F32, lib.F32, x, identity_place(rows, cols), rows, cols)
        other, _ = oracle.row_moments(lib.F32, lib.F16, h, identity_place(rows, cols), rows, cols)
        acc = start.copy()
        normalized = np.zeros(rows * cols, np.float32)
        oracle.fused(lib.F32, code, places, [x, gamma, h, acc, mean, devs, other], [acc, normalized], rows, cols)
        n = np.float32(cols)
        for r in range(rows):
            deviation = np.sqrt(devs[r] * (np.float32(1.0) / n) + np.float32(1e-5))
            for c in range(cols):
                i = r * cols + c
                want = (x[i] - mean[r]) / deviation
                assert normalized[i].view(np.uint32) == np.float32(want).view(np.uint32), (rows, cols, i)
                updated = start[i] + (np.float32(want) * gamma[c] + other[r])
                assert acc[i].view(np.uint32) == np.float32(updated).view(np.uint32), (rows, cols, i)


def test_moments_known_answers_and_against_f64():
    # statistics/mod.rs:419-441: mean = sum / n, then the deviations.
    assert oracle.moments(lib.F32, np.array([1, 2, 3, 4], np.float32)) == (2.5, 5.0)
    mean, devs = oracle.moments(lib.F32, np.zeros(0, np.float32))
    assert math.isnan(mean) and math.isnan(devs)
    rng = np.random.default_rng(21)
    x = rng.uniform(-3, 3, 100000).astype(np.float32)
    mean, devs = oracle.moments(lib.F32, x)
    wide = x.astype(np.float64)
    assert abs(mean - wide.mean()) <= 1e-4 * 3
    assert abs(devs - ((wide - wide.mean()) ** 2).sum()) <= 1e-3 * devs
