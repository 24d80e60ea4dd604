"""The oracle's analytic functions and powers (`vector_unary`,
`vector_unary_dual`, `vector_power*`, kernels.rs:876-895) pinned on the CPU:
the functions against numpy in f64, the derivatives against their closed
forms' known answers and central differences, and the power's fast
exponents bit for bit against the single operations they stand for
(tests/analytic.rs:285-345)."""

import math

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib
from tests.common import to_kind, ulps, widen

NUMPY_F64 = [np.sin, np.cos, np.tan, lambda x: 1 / np.cos(x), lambda x: 1 / np.sin(x), np.arcsin, np.arccos,
             np.arctan, np.exp, np.log, np.sinh, np.cosh, np.tanh, np.sqrt]
# Where each function is exercised: inside its domain, away from overflow.
DOMAINS = [(-20, 20), (-20, 20), (-1.4, 1.4), (-1.4, 1.4), (0.1, 3.0), (-0.999, 0.999), (-0.999, 0.999), (-50, 50),
           (-80, 80), (1e-3, 1e4), (-80, 80), (-80, 80), (-10, 10), (0, 1e6)]


@pytest.mark.parametrize("op", range(14))
def test_unary_against_f64(op):
    rng = np.random.default_rng(op)
    low, high = DOMAINS[op]
    x = rng.uniform(low, high, 4096).astype(np.float32)
    got = oracle.unary(lib.F32, op, x)
    want = NUMPY_F64[op](x.astype(np.float64)).astype(np.float32)
    assert ulps(got, want).max() <= 4, op
    for kind in (lib.F16, lib.BF16):
        xs = to_kind(x if op != 8 else x / 8, kind)
        got = oracle.unary(kind, op, xs)
        exact = NUMPY_F64[op](widen(kind, xs).astype(np.float64))
        assert ulps(got, to_kind(exact, kind)).max() <= 1, (op, kind)


def test_compact_secant_is_the_reciprocal_of_the_rounded_cosine():
    # vmath.rs:503-504: f16 and bf16 take 1/x in their own type.
    x = to_kind(np.linspace(-1.4, 1.4, 301), lib.F16)
    cos = to_kind(np.cos(widen(lib.F16, x).astype(np.float32)), lib.F16)
    want = to_kind(np.float32(1.0) / widen(lib.F16, cos).astype(np.float32), lib.F16)
    got = oracle.unary(lib.F16, 3, x)
    assert ulps(got, want).max() <= 1


def test_derivative_known_answers():
    x = np.array([0.0], np.float32)
    one = np.ones(1, np.float32)
    assert oracle.unary_dual(lib.F32, 0, x, one)[1].tolist() == [1.0]   # sin' = cos
    d = oracle.unary_dual(lib.F32, 1, x, one)[1]                        # cos' = -sin: -0
    assert d.tolist() == [0.0] and np.signbit(d[0])
    assert oracle.unary_dual(lib.F32, 8, x, one)[1].tolist() == [1.0]   # exp' = exp
    assert oracle.unary_dual(lib.F32, 12, x, one)[1].tolist() == [1.0]  # tanh'(0) = 1 - 0
    assert oracle.unary_dual(lib.F32, 7, x, one)[1].tolist() == [1.0]   # atan'(0) = 1
    four = np.array([4.0], np.float32)
    assert oracle.unary_dual(lib.F32, 13, four, one)[1].tolist() == [0.25]  # 1 / (2 sqrt 4)
    assert oracle.unary_dual(lib.F32, 9, four, one * 2)[1].tolist() == [0.5]  # (1/4) * 2


@pytest.mark.parametrize("op", range(14))
def test_derivatives_against_central_differences(op):
    rng = np.random.default_rng(100 + op)
    low, high = DOMAINS[op]
    low, high = (max(low, 0.2) if op in (9, 13) else low), min(high, 5.0)
    x = rng.uniform(low, high, 512).astype(np.float32)
    t = rng.uniform(-2, 2, 512).astype(np.float32)
    _, got = oracle.unary_dual(lib.F32, op, x, t)
    f, h = NUMPY_F64[op], 1e-6
    xd = x.astype(np.float64)
    slope = (f(xd + h) - f(xd - h)) / (2 * h)
    want = slope * t
    assert np.all(np.abs(got - want) <= 1e-4 * np.maximum(np.abs(want), 1.0)), op


def test_fast_exponents_are_exact():
    # tests/analytic.rs:285-345.
    values = np.concatenate([np.arange(-2000, 2000) * 0.017,
                             [0.0, -0.0, np.inf, -np.inf, np.nan, np.finfo(np.float32).tiny, -1.0]]).astype(np.float32)
    with np.errstate(all="ignore"):
        exact = {0.0: np.ones_like(values), 1.0: values, 2.0: values * values,
                 0.5: np.where(values == -np.inf, np.float32(np.inf), np.sqrt(values) + np.float32(0.0)),
                 -1.0: np.float32(1.0) / values}
    for exponent, want in exact.items():
        got = oracle.power_scalar(lib.F32, values, exponent, False)
        assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32)), exponent


def test_power_against_f64():
    rng = np.random.default_rng(7)
    a = rng.uniform(0.01, 20, 4096).astype(np.float32)
    b = rng.uniform(-8, 8, 4096).astype(np.float32)
    got = oracle.power(lib.F32, a, b)
    want = np.power(a.astype(np.float64), b.astype(np.float64)).astype(np.float32)
    assert ulps(got, want).max() <= 2
    got = oracle.power_scalar(lib.F32, b, 2.5, True)
    want = np.power(2.5, b.astype(np.float64)).astype(np.float32)
    assert ulps(got, want).max() <= 2
    got = oracle.power_scalar(lib.F32, a, 3.0, False)
    want = np.power(a.astype(np.float64), 3.0).astype(np.float32)
    assert ulps(got, want).max() <= 2
