"""The oracle's scalar-operand and clamp checkers pinned (CPU only).

``or_scalar`` is the checker of ``tc_broadcast`` and ``tc_compare_scalar``
(``Kernels::vector_broadcast`` / ``vector_compare_scalar``,
tensors/kernels.rs:838-855, host side :1208-1235): one operand is a scalar of
the element type, on the left when ``scalar_left``.  ``or_clamp`` is the
checker of ``tc_clamp`` (``Vector::clamp``, tensors/vector.rs:630-652:
``ordered_min(ordered_max(x, low), high)``; a NaN element clamps to ``low``
and a NaN bound is inert, tensors/shape.rs:30-43).

The references here are independent of the C restatement: torch's float32,
float16 and bfloat16 operators (each one operation rounded once), numpy's ``fmin``/``fmax`` for IEEE minNum/maxNum, and the
reference's documented known answers.  A swapped ``scalar_left``, a
remainder taken the wrong way round, a predicate true on NaN or a clamp that
propagates a NaN bound fails one of them.
"""

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib
from tests.common import KINDS, KIND_NAMES, same, to_kind, torch, widen

ARITHMETIC_OPS = [lib.ADD, lib.SUB, lib.MUL, lib.DIV, lib.REM]
COMPARE_OPS = [lib.MIN, lib.MAX, lib.MAX_SHARE, lib.LESS, lib.LESS_EQUAL, lib.GREATER, lib.GREATER_EQUAL]


def operands(kind):
    """Values of the type with NaN, infinities, signed zeros, ties with the
    scalars below and ordinary numbers of both signs."""
    rng = np.random.default_rng(7)
    special = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1.5, -1.5, 3.0, -2.25, 1e-3, 250.0], np.float32)
    values = np.concatenate([special, rng.standard_normal(2000).astype(np.float32) * 4])
    return to_kind(values, kind)


def torch_dtype(kind):
    return {lib.F32: torch.float32, lib.F16: torch.float16, lib.BF16: torch.bfloat16}[kind]


def as_torch(kind, host):
    """The host form of `kind` as a torch tensor of that type (bf16 from its bits)."""
    if kind == lib.BF16:
        return torch.from_numpy(host.astype(np.int16, copy=False).view(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(host)


def from_torch(kind, tensor):
    if kind == lib.BF16:
        return tensor.view(torch.int16).numpy().view(np.uint16)
    return tensor.numpy()


def arithmetic_reference(kind, op, x, scalar, scalar_left):
    """One rounded operation in the element type, by torch's own operators
    (the remainder is ``fmod``, Rust's truncating ``%``)."""
    t = as_torch(kind, x)
    s = torch.tensor(scalar, dtype=torch_dtype(kind))
    left, right = (s, t) if scalar_left else (t, s)
    out = {lib.ADD: torch.add, lib.SUB: torch.sub, lib.MUL: torch.mul, lib.DIV: torch.div,
           lib.REM: torch.fmod}[op](left.expand_as(t) if scalar_left else left,
                                     right.expand_as(t) if not scalar_left else right)
    return from_torch(kind, out)


def compare_reference(op, x, scalar, scalar_left):
    """`Compare::value` (kernels.rs:138-153) in float64 from the widened
    operands: minNum/maxNum, predicates false on NaN, the max share 1, 0 or
    one half otherwise (a NaN operand included)."""
    x = x.astype(np.float64)
    s = np.full_like(x, scalar)
    a, b = (s, x) if scalar_left else (x, s)
    with np.errstate(invalid="ignore"):
        if op == lib.MIN:
            return np.fmin(a, b)
        if op == lib.MAX:
            return np.fmax(a, b)
        if op == lib.MAX_SHARE:
            return np.where(a > b, 1.0, np.where(a < b, 0.0, 0.5))
        return {lib.LESS: a < b, lib.LESS_EQUAL: a <= b, lib.GREATER: a > b,
                lib.GREATER_EQUAL: a >= b}[op].astype(np.float64)


@pytest.mark.parametrize("kind", KINDS, ids=[KIND_NAMES[k] for k in KINDS])
@pytest.mark.parametrize("scalar_left", [False, True], ids=["scalar_right", "scalar_left"])
@pytest.mark.parametrize("op", ARITHMETIC_OPS, ids=["add", "sub", "mul", "div", "rem"])
def test_scalar_arithmetic_is_one_rounded_operation_on_the_right_side(kind, scalar_left, op):
    x = operands(kind)
    for scalar in (1.5, -2.25, 0.0, 3.0):
        got = oracle.scalar(kind, lib.ARITHMETIC, op, x, scalar, scalar_left)
        want = arithmetic_reference(kind, op, x, scalar, scalar_left)
        assert same(widen(kind, got), widen(kind, want)), (KIND_NAMES[kind], op, scalar, scalar_left)


def test_scalar_sides_differ_where_the_operation_is_not_symmetric():
    x = np.array([3.0, 8.0], np.float32)
    assert same(oracle.scalar(lib.F32, lib.ARITHMETIC, lib.SUB, x, 10.0, False), [-7.0, -2.0])
    assert same(oracle.scalar(lib.F32, lib.ARITHMETIC, lib.SUB, x, 10.0, True), [7.0, 2.0])
    assert same(oracle.scalar(lib.F32, lib.ARITHMETIC, lib.DIV, x, 2.0, True),
                np.float32([np.float32(2) / np.float32(3), 0.25]))
    # Rust's `%` truncates toward zero and keeps the dividend's sign.
    assert same(oracle.scalar(lib.F32, lib.ARITHMETIC, lib.REM, np.array([-7.5, 7.5], np.float32), 2.0, False),
                [-1.5, 1.5])
    assert same(oracle.scalar(lib.F32, lib.ARITHMETIC, lib.REM, np.array([2.0, -2.0], np.float32), -7.5, True),
                [-1.5, -1.5])


@pytest.mark.parametrize("kind", KINDS, ids=[KIND_NAMES[k] for k in KINDS])
@pytest.mark.parametrize("scalar_left", [False, True], ids=["scalar_right", "scalar_left"])
@pytest.mark.parametrize("op", COMPARE_OPS,
                         ids=["min", "max", "max_share", "less", "less_equal", "greater", "greater_equal"])
def test_scalar_comparisons_follow_compare_value(kind, scalar_left, op):
    x = operands(kind)
    for scalar in (1.5, -1.5, 0.0, float("nan")):
        got = widen(kind, oracle.scalar(kind, lib.COMPARE, op, x, scalar, scalar_left))
        want = compare_reference(op, widen(kind, x), scalar, scalar_left)
        assert same(got, want), (KIND_NAMES[kind], op, scalar, scalar_left)


def test_max_share_known_answers():
    # ∂max(a, s)/∂a: 1 above, 0 below, one half at a tie (kernels.rs:114-116).
    x = np.array([2.0, 0.0, 1.0], np.float32)
    assert same(oracle.scalar(lib.F32, lib.COMPARE, lib.MAX_SHARE, x, 1.0, False), [1.0, 0.0, 0.5])
    # With the scalar on the left it is ∂max(s, a)/∂s.
    assert same(oracle.scalar(lib.F32, lib.COMPARE, lib.MAX_SHARE, x, 1.0, True), [0.0, 1.0, 0.5])


def test_clamp_known_answers():
    # The reference's doc example (vector.rs:630-634).
    assert same(oracle.clamp(lib.F32, np.array([-2.0, 0.5, 7.0], np.float32), 0.0, 1.0), [0.0, 0.5, 1.0])
    # A NaN element clamps to `low` (vector.rs:638-639).
    assert same(oracle.clamp(lib.F32, np.array([np.nan], np.float32), -3.0, 4.0), [-3.0])
    # A NaN bound is inert (shape.rs:30-43): only the other bound applies.
    x = np.array([-5.0, 0.5, 5.0, np.nan], np.float32)
    assert same(oracle.clamp(lib.F32, x, np.nan, 1.0), [-5.0, 0.5, 1.0, 1.0])
    assert same(oracle.clamp(lib.F32, x, 0.0, np.nan), [0.0, 0.5, 5.0, 0.0])
    assert same(oracle.clamp(lib.F32, x, np.nan, np.nan), [-5.0, 0.5, 5.0, np.nan])


@pytest.mark.parametrize("kind", KINDS, ids=[KIND_NAMES[k] for k in KINDS])
def test_clamp_is_the_piecewise_definition(kind):
    x = operands(kind)
    wide = widen(kind, x).astype(np.float64)
    for low, high in ((-1.5, 1.5), (0.0, 0.0), (-np.inf, 0.5), (2.0, np.inf)):
        got = widen(kind, oracle.clamp(kind, x, low, high)).astype(np.float64)
        with np.errstate(invalid="ignore"):
            want = np.where(np.isnan(wide), low, np.where(wide < low, low, np.where(wide > high, high, wide)))
        assert same(got, want), (KIND_NAMES[kind], low, high)
        # torch's clamp agrees wherever the element is a number.
        ordered = ~np.isnan(wide)
        theirs = from_torch(kind, torch.clamp(as_torch(kind, x), low, high))
        assert same(got[ordered], widen(kind, theirs)[ordered]), (KIND_NAMES[kind], low, high)
