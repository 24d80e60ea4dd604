"""Analytic functions and powers on the GPU (`tc_unary`, `tc_unary_dual`,
`tc_power`, `tc_power_scalar`; kernels.rs:876-895, :941-949) against the
oracle on the same inputs.

The device's f32 functions are not the host's `vmath` ones, so f32 results
are held to a few ulp of the oracle's libm (both are within a few ulp of the
exact value; tan, the least accurate, gets the widest bound).  f16 and bf16
results, rounded from f32, match to one ulp of their own type.  The power's
fast exponents are single IEEE operations and match bit for bit."""

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib
from tests.common import to_kind, ulps, widen
from tests.test_oracle_analytic import DOMAINS

pytestmark = pytest.mark.gpu

HOST = {lib.F32: np.float32, lib.F16: np.float16, lib.BF16: np.uint16}
F32_ULPS = {2: 8, 3: 8, 4: 8}  # tan, sec, csc near their poles


def operand(kind, op, n, seed):
    rng = np.random.default_rng(seed)
    low, high = DOMAINS[op]
    x = rng.uniform(low, high, n)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-30, -1e-30])
    x = np.concatenate([x, specials])
    return to_kind(x if kind == lib.F32 or op != 8 else x / 8, kind)


def device_unary(kind, op, x):
    a = lib.Buffer.of(x)
    out = lib.Buffer(max(x.nbytes, 1))
    lib.call("tc_unary", kind, op, a.ptr, out.ptr, x.size)
    return out.download(HOST[kind], x.size)


@pytest.mark.parametrize("kind", [lib.F32, lib.F16, lib.BF16])
@pytest.mark.parametrize("op", range(14))
def test_unary_against_the_oracle(kind, op):
    x = operand(kind, op, 100003, op)
    got = device_unary(kind, op, x)
    want = oracle.unary(kind, op, x)
    bound = F32_ULPS.get(op, 4) if kind == lib.F32 else 1
    worst = int(np.argmax(ulps(got, want)))
    assert ulps(got, want).max() <= bound, (op, kind, worst, widen(kind, x[worst:worst + 1]))


@pytest.mark.parametrize("kind", [lib.F32, lib.BF16])
@pytest.mark.parametrize("op", range(14))
def test_unary_dual_against_the_oracle(kind, op):
    x = operand(kind, op, 20001, 50 + op)
    rng = np.random.default_rng(op)
    t = to_kind(rng.uniform(-2, 2, x.size), kind)
    dv, dt, ov, ot = lib.Buffer.of(x), lib.Buffer.of(t), lib.Buffer(x.nbytes), lib.Buffer(x.nbytes)
    lib.call("tc_unary_dual", kind, op, dv.ptr, dt.ptr, ov.ptr, ot.ptr, x.size)
    want_value, want_tangent = oracle.unary_dual(kind, op, x, t)
    got_value, got_tangent = ov.download(HOST[kind], x.size), ot.download(HOST[kind], x.size)
    bound = F32_ULPS.get(op, 4) if kind == lib.F32 else 1
    assert ulps(got_value, want_value).max() <= bound, op
    # A derivative composes a few roundings of the function's value, and
    # some cancel (tanh' = 1 - tanh^2 near |tanh| = 1): each element is within
    # a few ulp, or within a few units of the value's own last place times
    # the tangent.
    unit = 2.0 ** -24 if kind == lib.F32 else 2.0 ** -8
    value = np.abs(widen(kind, want_value).astype(np.float64))
    slack = 32 * unit * np.abs(widen(kind, t).astype(np.float64)) * np.maximum(1.0, value) ** 2
    with np.errstate(invalid="ignore"):  # inf - inf where both are infinite: decided by ulps
        close = np.abs(widen(kind, got_tangent).astype(np.float64) - widen(kind, want_tangent)) <= slack
    assert np.all((ulps(got_tangent, want_tangent) <= (4 * bound if kind == lib.F32 else 3)) | close), op


def test_unary_and_dual_of_odd_lengths_and_offsets():
    # Unaligned views take the element-at-a-time path; the tail of the
    # 16-byte path is finished by the first block.
    rng = np.random.default_rng(3)
    x = rng.uniform(-2, 2, 1031).astype(np.float32)
    a = lib.Buffer.of(x)
    out = lib.Buffer(x.nbytes + 16)
    lib.call("tc_unary", lib.F32, 8, a.ptr + 4, out.ptr + 4, x.size - 1)
    got = out.download(np.float32, x.size)[1:]
    assert ulps(got, oracle.unary(lib.F32, 8, x[1:])).max() <= 4
    ov, ot = lib.Buffer(x.nbytes), lib.Buffer(x.nbytes)
    lib.call("tc_unary_dual", lib.F32, 0, a.ptr, a.ptr, ov.ptr, ot.ptr, 1027)
    want_value, want_tangent = oracle.unary_dual(lib.F32, 0, x[:1027], x[:1027])
    assert ulps(ov.download(np.float32, 1027), want_value).max() <= 4
    assert ulps(ot.download(np.float32, 1027), want_tangent).max() <= 16


def test_an_unknown_function_is_refused():
    a = lib.Buffer(16)
    with pytest.raises(lib.HipError, match="no Analytic 14"):
        lib.call("tc_unary", lib.F32, 14, a.ptr, a.ptr, 4)


@pytest.mark.parametrize("kind", [lib.F32, lib.F16, lib.BF16])
def test_power_against_the_oracle(kind):
    rng = np.random.default_rng(9)
    a = to_kind(np.concatenate([rng.uniform(0.01, 8, 50000), [0.0, -1.0, np.inf, np.nan, -0.0]]), kind)
    b = to_kind(np.concatenate([rng.uniform(-6, 6, 50000), [0.5, 3.0, -1.0, 2.0, -3.0]]), kind)
    da, db, out = lib.Buffer.of(a), lib.Buffer.of(b), lib.Buffer(a.nbytes)
    lib.call("tc_power", kind, da.ptr, db.ptr, out.ptr, a.size)
    bound = 2 if kind == lib.F32 else 1
    assert ulps(out.download(HOST[kind], a.size), oracle.power(kind, a, b)).max() <= bound
    for scalar, left in [(2.5, True), (3.0, False), (-2.5, False), (0.0, False), (1.0, False), (2.0, False),
                         (0.5, False), (-1.0, False)]:
        lib.call("tc_power_scalar", kind, da.ptr, scalar, int(left), out.ptr, a.size)
        got = out.download(HOST[kind], a.size)
        want = oracle.power_scalar(kind, a, scalar, left)
        exact = kind == lib.F32 and not left and scalar in (0.0, 1.0, 2.0, 0.5, -1.0)
        assert ulps(got, want).max() <= (0 if exact else bound), (scalar, left)
