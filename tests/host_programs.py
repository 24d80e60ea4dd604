"""The programs the reference's Host backend interprets for the optimizer
steps, derived by the tests from the program as built and the restated
optimizer (`oracle/fusion.py`): the checker's side of the Adam parity tests.

`adam_graph` is `Adam::program` (optim.rs:1048-1100) as `build_with` hands
it to the optimizer (fused/mod.rs:2282-2435): the builder's nodes in the
order built, each uniform a named constant (`Node::Uniform`, :2407-2409),
the literal one kept as a literal (`placeholder`, :2588-2607), the loads
numbered by their distinct (slot, remap) in order of appearance, the stores
the in-place tensors first and then the outputs (:2300-2312).  `lower`
turns the optimizer's chosen code into this library's encoded instructions,
its constants evaluated in the element type as `evaluate` does
(:2618-2630)."""

from __future__ import annotations

import numpy as np

from oracle import binding as oracle
from oracle import fusion as F

LOAD, CONST, BINARY, UNARY, COMPARE, STORE = 0, 1, 2, 3, 4, 5
SIZES = {0: 4, 1: 2, 2: 2}  # F32, F16, BF16


def in_type(dtype: int, value) -> np.float32:
    """`value` rounded to the element type, held as an f32 (the oracle's
    narrowing: RNE, NaN kept)."""
    v = np.array([value], np.float32)
    if dtype == 0:
        return v[0]
    return oracle.widen(dtype, oracle.narrow(dtype, v))[0]


def powi(dtype: int, base, exponent: int) -> np.float32:
    """`Float::powi` in the element type: square and multiply from the low
    bit, each product rounded (compiler-rt's __powisf2)."""
    result, a, b = np.float32(1.0), in_type(dtype, base), abs(exponent)
    while True:
        if b & 1:
            result = in_type(dtype, result * a)
        b //= 2
        if b == 0:
            break
        a = in_type(dtype, a * a)
    return in_type(dtype, np.float32(1.0) / result) if exponent < 0 else result


# The uniforms of Adam::program, in declaration order (optim.rs:1052-1057).
RATE, FIRST_DECAY, SECOND_DECAY, EPSILON, FIRST_CORRECTION, SECOND_CORRECTION = range(6)


def adam_graph(resumed: bool, element_bytes: int) -> F.Graph:
    """Adam's program as the optimizer receives it."""
    named = [("const", ("named", i)) for i in range(6)]
    nodes = named + [
        ("load", 0, 0),              # 6: g (input 0)
        ("load", 1, 1),              # 7: p (update 0)
        ("const", F.lit(1.0)),       # 8: one
        ("bin", F.SUB, 8, 1),        # 9: 1 - beta1
        ("bin", F.SUB, 8, 2),        # 10: 1 - beta2
        ("bin", F.MUL, 6, 9),        # 11: g (1 - beta1)
        ("bin", F.MUL, 6, 6),        # 12: g g
        ("bin", F.MUL, 12, 10),      # 13: g g (1 - beta2)
    ]
    if resumed:
        nodes += [
            ("load", 2, 2),          # 14: m (update 1)
            ("load", 3, 3),          # 15: v (update 2)
            ("bin", F.MUL, 14, 1),   # 16: m beta1
            ("bin", F.MUL, 15, 2),   # 17: v beta2
            ("bin", F.ADD, 16, 11),  # 18: first moment
            ("bin", F.ADD, 17, 13),  # 19: second moment
        ]
        first, second = 18, 19
    else:
        first, second = 11, 13
    at = len(nodes)
    nodes += [
        ("bin", F.MUL, first, 4),      # corrected first
        ("bin", F.MUL, second, 5),     # corrected second
        ("un", F.SQRT, at + 1),        # root
        ("bin", F.ADD, at + 2, 3),     # denominator
        ("bin", F.DIV, at, at + 3),    # step
        ("bin", F.MUL, at + 4, 0),     # step rate
        ("bin", F.SUB, 7, at + 5),     # p - step rate
    ]
    inputs = 4 if resumed else 2
    return F.Graph(nodes, [(at + 6, 0), (first, 1), (second, 2)], [element_bytes] * inputs, [element_bytes] * 3)


def evaluate(dtype: int, scalar: tuple, named: list) -> np.float32:
    """A constant in the element type (fused/mod.rs:2618-2630): literals
    converted, named constants as given, folds one rounded operation each."""
    kind = scalar[0]
    if kind == "lit":
        return in_type(dtype, F.lit_value(scalar))
    if kind == "named":
        return named[scalar[1]]
    a, b = evaluate(dtype, scalar[2], named), evaluate(dtype, scalar[3], named)
    op = scalar[1]
    value = {F.ADD: a + b, F.SUB: a - b, F.MUL: a * b, F.DIV: a / b}[op]
    return in_type(dtype, value)


def lower(dtype: int, code: list, named: list) -> list:
    """The optimizer's allocated code as encoded instructions (`lower`,
    fused/mod.rs:2632-2680); a load's place is its remap code."""
    out = []
    for instr in code:
        kind = instr[0]
        if kind == "load":
            _, dst, slot, remap = instr
            out.append((LOAD, remap, dst, slot, dtype, 0, 0.0))
        elif kind == "const":
            out.append((CONST, 0, instr[1], 0, 0, 0, float(evaluate(dtype, instr[2], named))))
        elif kind == "bin":
            _, dst, op, a, b = instr
            out.append((BINARY, op, dst, a, b, 0, 0.0))
        elif kind == "un":
            _, dst, function, a = instr
            out.append((UNARY, function, dst, a, 0, 0, 0.0))
        elif kind == "cmp":
            _, dst, op, a, b = instr
            out.append((COMPARE, op, dst, a, b, 0, 0.0))
        else:
            _, src, output = instr
            out.append((STORE, 0, 0, src, dtype, output, 0.0))
    return out


def host_adam_program(resumed: bool, dtype: int, rate, first_decay, second_decay, epsilon, step: int,
                      reassociate: bool = True, model: F.CostModel = F.BALANCED_MODEL):
    """The Host's Adam step: the plan the optimizer chooses (under the
    balanced cost model `Step::of` builds with, optim.rs:739-746), lowered
    with this step's uniforms (`Adam::update`, optim.rs:1106-1124).  Returns
    (encoded program, number of loads, plan)."""
    plan = F.optimize(adam_graph(resumed, SIZES[dtype]), model, reassociate)
    one = np.float32(1.0)
    b1, b2 = in_type(dtype, first_decay), in_type(dtype, second_decay)
    named = [in_type(dtype, rate), b1, b2, in_type(dtype, epsilon),
             in_type(dtype, one / in_type(dtype, one - powi(dtype, b1, step))),
             in_type(dtype, one / in_type(dtype, one - powi(dtype, b2, step)))]
    loads = len({instr[3] for instr in plan.code if instr[0] == "load"})
    return lower(dtype, plan.code, named), loads, plan
