"""The Adam rule over Hip storage, as tensorcrate runs it: one fused program
per step (optim.rs:986-1136).

``adam_program`` encodes the program ``Adam::program`` builds
(optim.rs:1048-1100) as the Host runs it, with its uniforms bound to their
values: the coefficients, ``1 - beta`` folded into constants computed once in
the element type, and the bias corrections ``1 / (1 - beta^t)`` computed on
the host in the element type as ``update`` does (optim.rs:1106-1124).
``Adam.update`` runs it through ``tc_fused``.

The Host optimizes every built program before it runs it, under the
thread's ``Algebra`` (fused/mod.rs:2473-2491, optim.rs:716-745):

- ``EXACT``: only rewrites that keep every result's bits, so the program runs
  in its construction order: ``((m' c1) / (sqrt(v' c2) + eps)) rate``;
- ``REASSOCIATE``, the default: the optimizer (fusion/src/rewrite.rs:324-399)
  flattens the product chain ``m' . c1 / d . rate``, whose inner links nothing
  else reads, gathers its two constants into one folded in the element type,
  and rebuilds it as ``(m' . fl(c1 rate)) / d``, one instruction and one
  constant fewer; under every cost model the reference defines that plan is
  the cheapest (fusion/src/optimize.rs:152-215), so it is the one the Host
  interprets.  The other chains of the step (``g g (1 - beta2)``,
  ``m beta1 + g (1 - beta1)``, ``sqrt(.) + eps``, ``p - step``) rebuild as
  built.
"""

from __future__ import annotations

import numpy as np

from . import lib

SQRT = 13  # Analytic::Sqrt (kernels.rs:307)


def _in_type(dtype: int, value: float) -> np.float32:
    """`value` rounded to the element type, held as an f32."""
    v = np.float32(value)
    if dtype == lib.F16:
        return np.float32(np.float16(v))
    if dtype == lib.BF16:
        x = np.array([v], np.float32).view(np.uint32)[0]
        if (x & 0x7FFFFFFF) > 0x7F800000:
            bits = (x >> 16) | 0x40
        else:
            bits = (int(x) + 0x7FFF + ((int(x) >> 16) & 1)) >> 16
        return np.array([int(bits) << 16], np.uint32).view(np.float32)[0]
    return v


def powi(dtype: int, base, exponent: int) -> np.float32:
    """`Float::powi` in the element type: square and multiply from the low
    bit, each product rounded (LLVM compiler-rt's __powisf2, which Rust's
    f32::powi lowers to)."""
    result = np.float32(1.0)
    a = _in_type(dtype, base)
    b = abs(exponent)
    while True:
        if b & 1:
            result = _in_type(dtype, result * a)
        b //= 2
        if b == 0:
            break
        a = _in_type(dtype, a * a)
    return _in_type(dtype, np.float32(1.0) / result) if exponent < 0 else result


def identity_place(rows: int, cols: int):
    """A load of a rows x cols tensor in its own order (Place::grid)."""
    return (0, 1, 1, [rows], [cols])


EXACT, REASSOCIATE = "exact", "reassociate"  # `Algebra` (fused/mod.rs:2473-2491)


def adam_program(resumed: bool, dtype: int, rate, first_decay, second_decay, epsilon, step: int,
                 algebra: str = REASSOCIATE):
    """The encoded Adam step (optim.rs:1048-1100) as the Host runs it under
    `algebra`, and its load places' slots.  Inputs: 0 the gradient, 1 the
    parameters, then (resumed) 2 the first moment and 3 the second; outputs:
    0 the parameters, 1 the first moment, 2 the second."""
    if algebra not in (EXACT, REASSOCIATE):
        raise ValueError(f"no Algebra {algebra!r}")
    t = lambda v: float(_in_type(dtype, v))
    one = np.float32(1.0)
    b1, b2 = _in_type(dtype, first_decay), _in_type(dtype, second_decay)
    first_correction = _in_type(dtype, one / _in_type(dtype, one - powi(dtype, b1, step)))
    second_correction = _in_type(dtype, one / _in_type(dtype, one - powi(dtype, b2, step)))
    first_share, second_share = t(one - b1), t(one - b2)
    LOAD, CONST, BINARY, UNARY, STORE = 0, 1, 2, 3, 5
    code = [
        (LOAD, 0, 0, 0, dtype, 0, 0.0),              # r0 = g
        (CONST, 0, 1, 0, 0, 0, first_share),          # r1 = 1 - beta1
        (BINARY, lib.MUL, 2, 0, 1, 0, 0.0),           # r2 = g (1 - beta1)
        (BINARY, lib.MUL, 3, 0, 0, 0, 0.0),           # r3 = g g
        (CONST, 0, 4, 0, 0, 0, second_share),         # r4 = 1 - beta2
        (BINARY, lib.MUL, 5, 3, 4, 0, 0.0),           # r5 = g g (1 - beta2)
    ]
    if resumed:
        code += [
            (LOAD, 2, 6, 2, dtype, 0, 0.0),           # r6 = m
            (CONST, 0, 7, 0, 0, 0, float(b1)),
            (BINARY, lib.MUL, 6, 6, 7, 0, 0.0),       # m beta1
            (BINARY, lib.ADD, 6, 6, 2, 0, 0.0),       # first
            (LOAD, 3, 8, 3, dtype, 0, 0.0),           # r8 = v
            (CONST, 0, 9, 0, 0, 0, float(b2)),
            (BINARY, lib.MUL, 8, 8, 9, 0, 0.0),       # v beta2
            (BINARY, lib.ADD, 8, 8, 5, 0, 0.0),       # second
        ]
        first, second = 6, 8
    else:
        first, second = 2, 5
    if algebra == REASSOCIATE:
        # c1 and the rate gathered into one constant, folded in the type.
        folded = t(np.float32(first_correction) * np.float32(t(rate)))
        numerator = [(CONST, 0, 10, 0, 0, 0, folded),
                     (BINARY, lib.MUL, 11, first, 10, 0, 0.0)]    # m' fl(c1 rate)
    else:
        numerator = [(CONST, 0, 10, 0, 0, 0, float(first_correction)),
                     (BINARY, lib.MUL, 11, first, 10, 0, 0.0)]    # corrected first
    code += numerator + [
        (CONST, 0, 12, 0, 0, 0, float(second_correction)),
        (BINARY, lib.MUL, 13, second, 12, 0, 0.0),    # corrected second
        (UNARY, SQRT, 13, 13, 0, 0, 0.0),             # root
        (CONST, 0, 14, 0, 0, 0, t(epsilon)),
        (BINARY, lib.ADD, 13, 13, 14, 0, 0.0),        # denominator
        (BINARY, lib.DIV, 11, 11, 13, 0, 0.0),        # step
    ]
    if algebra == EXACT:
        code += [(CONST, 0, 15, 0, 0, 0, t(rate)),
                 (BINARY, lib.MUL, 11, 11, 15, 0, 0.0)]      # step rate
    code += [
        (LOAD, 1, 7, 1, dtype, 0, 0.0),               # r7 = p
        (BINARY, lib.SUB, 7, 7, 11, 0, 0.0),          # p - step rate
        (STORE, 0, 0, 7, dtype, 0, 0.0),
        (STORE, 0, 0, first, dtype, 1, 0.0),
        (STORE, 0, 0, second, dtype, 2, 0.0),
    ]
    loads = 4 if resumed else 2
    return code, loads


class Adam:
    """`Adam` (optim.rs:1001-1136) over device buffers of `len` elements."""

    def __init__(self, rate, dtype: int = lib.F32, algebra: str = REASSOCIATE):
        self.rate = rate
        self.first_decay, self.second_decay, self.epsilon = 0.9, 0.999, 1e-8
        self.dtype = dtype
        # Fixed when the rule is made, as `Step::default` takes the thread's
        # algebra (optim.rs:727-733).
        self.algebra = algebra
        self.steps = 0
        self.first = self.second = None

    def update(self, parameters: lib.Buffer, gradient: lib.Buffer, rows: int, cols: int) -> None:
        self.steps += 1
        resumed = self.first is not None
        code, loads = adam_program(resumed, self.dtype, self.rate, self.first_decay, self.second_decay,
                                   self.epsilon, self.steps, self.algebra)
        n = rows * cols
        places = [identity_place(rows, cols)] * loads
        if not resumed:
            size = lib.DTYPE_SIZE[self.dtype]
            self.first, self.second = lib.Buffer(n * size), lib.Buffer(n * size)
            inputs = [(gradient, n), (parameters, n)]
        else:
            inputs = [(gradient, n), (parameters, n), (self.first, n), (self.second, n)]
        outputs = [(parameters, n), (self.first, n), (self.second, n)]
        lib.fused(self.dtype, code, places, inputs, outputs, rows, cols)
