"""Tensor variables on the tape (host/tape.hpp's `TensorVar`, the C++ mirror
of src/tensors/tape/tensor.rs) on the GPU, operation by operation, as
tests/tensor_autodiff.rs:50-400 checks them in the reference; the matrix
and vector rules they pass through (`MatrixVar::matmul`, `matvec`,
`matvec_add`, `VectorVar`'s products) are checked the same way.

Each operation is written once against a small facade and run twice: on the
device tape (`lib.Tape`), which differentiates it with one backward pass from
a fixed seed, and in numpy f64, whose central differences of
``<op(inputs), seed>`` are the expected gradients.  The f32 gradients must
agree within 2e-4 of the largest expected magnitude, the reference's bound
for f32 against f64 (tensor_autodiff.rs:388-391).  The inputs are rounded to
f32 first, so both sides see the same values.  The harness itself is pinned
on the CPU against closed forms (`test_the_difference_harness_...`).

Every operation of the reference's table is covered.
"""

import numpy as np
import pytest

from tensorcrate_amd import lib
from tests.test_oracle_analytic import NUMPY_F64

X = (2, 3, 4, 5)


def filled(shape, seed, low, high):
    return np.random.default_rng(seed).uniform(low, high, shape).astype(np.float32).astype(np.float64)


class Np:
    """The facade in numpy f64: what each recorded operation computes."""

    def __init__(self, value):
        self.v = np.asarray(value, np.float64)

    def binary(self, other, op):
        a, b = self.v, other.v
        return Np({"add": np.add, "sub": np.subtract, "mul": np.multiply, "div": np.divide,
                   "maximum": np.maximum, "minimum": np.minimum, "power": np.power,
                   "matmul": np.matmul,
                   "vector_mul": lambda a, b: (a.ravel() * b.ravel()).reshape(a.shape),
                   "matvec": np.matmul}[op](a, b))

    def matvec_add(self, v, addend):
        return Np(self.v @ v.v + addend.v)

    __add__ = lambda self, o: self.binary(o, "add")
    __sub__ = lambda self, o: self.binary(o, "sub")
    __mul__ = lambda self, o: self.binary(o, "mul")
    __truediv__ = lambda self, o: self.binary(o, "div")

    def unary(self, op, first=0.0, second=0.0):
        x = self.v
        table = {"clamp_min": lambda: np.maximum(x, first), "clamp_max": lambda: np.minimum(x, first),
                 "clamp": lambda: np.clip(x, first, second), "relu": lambda: np.maximum(x, 0.0),
                 "abs": lambda: np.abs(x), "neg": lambda: -x, "scale": lambda: x * first,
                 "shift": lambda: x + first, "power_scalar": lambda: x ** first,
                 "power_scalar_left": lambda: first ** x, "contiguous": lambda: x.copy()}
        return Np(table[op]())

    def analytic(self, f):
        return Np(NUMPY_F64[f](self.v))

    def layout(self, op, values):
        x = self.v
        if op == "reshape":
            return Np(x.reshape(values))
        if op == "permute":
            return Np(np.transpose(x, values))
        if op == "transpose":
            return Np(np.swapaxes(x, *values))
        if op == "narrow":
            axis, start, length = values
            return Np(np.take(x, range(start, start + length), axis=axis))
        if op == "select":
            return Np(np.take(x, values[1], axis=values[0]))
        if op == "slice":
            axis, start, end = values
            return Np(np.take(x, range(start, end), axis=axis))
        if op == "squeeze":
            return Np(np.squeeze(x, axis=values[0]))
        if op == "unsqueeze":
            return Np(np.expand_dims(x, values[0]))
        return Np(np.broadcast_to(x, values).copy())

    def split(self, axis, sizes=None, parts=0):
        bounds = np.cumsum(sizes)[:-1] if sizes is not None else parts
        return [Np(p) for p in np.split(self.v, bounds, axis=axis)]

    def reduce(self, op, axes=(), keep_dims=False):
        x = self.v
        axes = (axes,) if isinstance(axes, int) else tuple(axes)
        if op == "sum":
            return Np(x.sum())
        if op == "mean":
            return Np(x.mean())
        fold = {"sum_axes": lambda: x.sum(axis=axes, keepdims=keep_dims),
                "mean_axes": lambda: x.mean(axis=axes, keepdims=keep_dims),
                "var_axes": lambda: x.var(axis=axes, keepdims=keep_dims),
                "var_axes_sample": lambda: x.var(axis=axes, ddof=1, keepdims=keep_dims),
                "max_axes": lambda: x.max(axis=axes, keepdims=keep_dims),
                "min_axes": lambda: x.min(axis=axes, keepdims=keep_dims)}
        return Np(fold[op]())


def join(op, pieces, axis):
    """`concat`/`stack` on either side of the facade."""
    if isinstance(pieces[0], Np):
        f = np.concatenate if op == "concat" else np.stack
        return Np(f([p.v for p in pieces], axis=axis))
    return pieces[0].tape.join(op, pieces, axis)


def positive(shape, seed):
    return filled(shape, seed, 0.5, 1.5)


def x():
    return filled(X, 1, -1.0, 1.0)


# The operations of tensor_autodiff.rs:52-270 this tape records: name,
# inputs, and the computation on recorded inputs `v`.
OPS = [
    ("add_same", lambda: [x(), filled(X, 2, -1, 1)], lambda v: v[0] + v[1]),
    ("add_broadcast", lambda: [x(), filled((4, 1), 2, -1, 1)], lambda v: v[0] + v[1]),
    ("sub_broadcast", lambda: [filled((3, 1, 5), 2, -1, 1), x()], lambda v: v[0] - v[1]),
    ("mul_broadcast", lambda: [filled((2, 1, 4, 1), 1, -1, 1), filled((1, 3, 1, 5), 2, -1, 1)],
     lambda v: v[0] * v[1]),
    ("div_broadcast", lambda: [x(), positive((5,), 2)], lambda v: v[0] / v[1]),
    ("div_left_broadcast", lambda: [filled((3, 1, 1), 2, -1, 1), positive(X, 3)], lambda v: v[0] / v[1]),
    ("scalar_operand", lambda: [x(), filled((), 2, 0.5, 1.5)], lambda v: (v[0] * v[1]) + v[1]),
    ("permuted_operand", lambda: [x(), filled((3, 1), 2, -1, 1)],
     lambda v: v[0].layout("permute", [0, 2, 1, 3]) * v[1]),
    ("maximum", lambda: [x(), filled((4, 5), 2, -1, 1)], lambda v: v[0].binary(v[1], "maximum")),
    ("minimum", lambda: [filled((3, 1, 5), 2, -1, 1), x()], lambda v: v[0].binary(v[1], "minimum")),
    ("power", lambda: [positive((2, 3, 4), 1), filled((4,), 2, -1, 2)], lambda v: v[0].binary(v[1], "power")),
    ("power_scalar", lambda: [positive(X, 1)], lambda v: v[0].unary("power_scalar", 2.5)),
    ("power_scalar_left", lambda: [x()], lambda v: v[0].unary("power_scalar_left", 1.7)),
    ("scale_shift_neg", lambda: [x()], lambda v: v[0].unary("scale", -1.5).unary("shift", 0.25).unary("neg")),
    ("abs", lambda: [x()], lambda v: v[0].unary("abs")),
    ("relu", lambda: [x()], lambda v: v[0].unary("relu")),
    ("clamp", lambda: [x()], lambda v: v[0].unary("clamp", -0.5, 0.4)),
    *[(f"analytic_{f}", lambda: [filled((2, 3, 4), 1, 0.15, 0.85)], (lambda f: lambda v: v[0].analytic(f))(f))
      for f in range(14)],
    ("reshape", lambda: [x()], lambda v: v[0].layout("reshape", [6, 20])),
    ("permute", lambda: [x()], lambda v: v[0].layout("permute", [0, 2, 3, 1])),
    ("transpose", lambda: [x()], lambda v: v[0].layout("transpose", [-1, 1])),
    ("squeeze_unsqueeze", lambda: [filled((2, 1, 4), 1, -1, 1)], lambda v: v[0].layout("reshape", [1, 2, 4, 1])),
    ("broadcast_to", lambda: [filled((3, 1, 5), 1, -1, 1)], lambda v: v[0].layout("broadcast_to", list(X))),
    ("contiguous", lambda: [x()], lambda v: v[0].unary("contiguous")),
    ("sum_axes", lambda: [x()], lambda v: v[0].reduce("sum_axes", [1, 3])),
    ("sum_axes_keep", lambda: [x()], lambda v: v[0].reduce("sum_axes", -2, True)),
    ("sum_all", lambda: [x()], lambda v: v[0].reduce("sum_axes", [0, 1, 2, 3])),
    ("mean_axes", lambda: [x()], lambda v: v[0].reduce("mean_axes", [0, 2], True)),
    ("var_axes_population", lambda: [x()], lambda v: v[0].reduce("var_axes", [1, 2])),
    ("var_axes_sample", lambda: [x()], lambda v: v[0].reduce("var_axes_sample", -1, True)),
    ("max_axes", lambda: [x()], lambda v: v[0].reduce("max_axes", [1, 3])),
    ("min_axes", lambda: [x()], lambda v: v[0].reduce("min_axes", -1, True)),
    ("matrix_round_trip", lambda: [filled((2, 3, 4), 1, -1, 1), filled((4, 5), 2, -1, 1)],
     lambda v: v[0].binary(v[1], "matmul").analytic(12)),
    ("narrowed_operand", lambda: [x(), filled((2, 1, 4, 5), 2, -1, 1)],
     lambda v: v[0].layout("narrow", [1, 1, 1]) * v[1]),
    ("narrow", lambda: [x()], lambda v: v[0].layout("narrow", [2, 1, 2])),
    ("slice", lambda: [x()], lambda v: v[0].layout("slice", [-1, 1, 4])),
    ("select", lambda: [x()], lambda v: v[0].layout("select", [1, 2])),
    ("split", lambda: [filled((2, 3, 4, 6), 1, -1, 1)],
     lambda v: (lambda p: p[0].reduce("sum_axes", -1, True) * p[1].analytic(12))(v[0].split(-1, sizes=[2, 4]))),
    ("chunk", lambda: [filled((2, 3, 4, 6), 1, -1, 1)],
     lambda v: (lambda p: (p[0] * p[1]) + p[2].analytic(0))(v[0].split(-1, parts=3))),
    ("concat", lambda: [filled((2, 3, 4, 2), 1, -1, 1), filled((2, 3, 4, 3), 2, -1, 1)],
     lambda v: join("concat", [v[1], v[0], v[1].unary("scale", 2.0)], -1)),
    ("stack", lambda: [filled((2, 3, 4), 1, -1, 1), filled((2, 3, 4), 2, -1, 1)],
     lambda v: join("stack", [v[0], v[1], v[0]], 1)),
    ("squeeze_unsqueeze_axes", lambda: [filled((2, 1, 4), 1, -1, 1)],
     lambda v: v[0].layout("squeeze", [1]).layout("unsqueeze", [0]).layout("unsqueeze", [-1])),
    # tensor_autodiff.rs:251-254: flat = x.to_vector(); (flat * flat).to_tensor([4, 6]).
    ("vector_round_trip", lambda: [filled((2, 3, 4), 1, -1, 1)],
     lambda v: v[0].binary(v[0], "vector_mul").layout("reshape", [4, 6])),
    ("vector_product", lambda: [filled((2, 3, 4), 1, -1, 1), positive((6, 4), 2)],
     lambda v: v[0].binary(v[1], "vector_mul")),
    ("matvec", lambda: [filled((5, 7), 1, -1, 1), filled((7,), 2, -1, 1)], lambda v: v[0].binary(v[1], "matvec")),
    ("matvec_add", lambda: [filled((5, 7), 1, -1, 1), filled((7,), 2, -1, 1), filled((5,), 3, -1, 1)],
     lambda v: v[0].matvec_add(v[1], v[2])),
    # A tensor used twice: the second rule adds into an adjoint already there.
    ("reused_operand", lambda: [x()], lambda v: v[0].reduce("sum_axes", 1, True) + (v[0] * v[0])),
    # The narrow's rule runs after the product's, so it adds into an adjoint
    # that is already there (tensor_autodiff.rs:254-258).
    ("slice_into_existing_adjoint", lambda: [x()],
     lambda v: v[0].layout("narrow", [1, 0, 2]).reduce("sum_axes", 1, True) + (v[0] * v[0])),
    # The product is recorded first, so the narrow's rule writes into zeros
    # and the product's adds to that (tensor_autodiff.rs:259-264).
    ("slice_before_other_use", lambda: [x()],
     lambda v: (lambda square: v[0].layout("narrow", [-1, 2, 3]).analytic(8).reduce("sum_axes", -1, True) + square)(
         v[0] * v[0])),
]


def seed_for(shape):
    return filled(shape, 7, -1.0, 1.0)


def projected(apply, inputs, seed):
    return float(np.sum(apply([Np(a) for a in inputs]).v * seed))


def differences(apply, inputs):
    """Central differences of <apply(inputs), seed> in f64, step
    1e-6·max(|x|, 1), as tensor_autodiff.rs:327-359 takes them."""
    seed = seed_for(apply([Np(a) for a in inputs]).v.shape)
    grads = []
    for which, a in enumerate(inputs):
        g = np.empty(a.size)
        for k in range(a.size):
            h = 1e-6 * max(abs(a.flat[k]), 1.0)
            moved = [b.copy() for b in inputs]
            moved[which].flat[k] = a.flat[k] + h
            up = projected(apply, moved, seed)
            moved[which].flat[k] = a.flat[k] - h
            g[k] = (up - projected(apply, moved, seed)) / (2 * h)
        grads.append(g.reshape(a.shape))
    return grads, seed


def assert_close(got, want, tolerance, what):
    scale = max(1.0, float(np.max(np.abs(want))) if want.size else 0.0)
    err = float(np.max(np.abs(np.asarray(got, np.float64) - want))) if want.size else 0.0
    assert err <= tolerance * scale, f"{what}: error {err} against scale {scale}"


def test_the_difference_harness_reproduces_closed_forms():
    """Pins the harness: d<a·b, s>/da = b·s summed over the broadcast,
    d<Σ_axis x, s>/dx = s spread, d<max(x,0), s>/dx = s·[x>0]."""
    a, b = filled((3, 1), 1, -1, 1), filled((3, 4), 2, -1, 1)
    (ga, gb), s = differences(lambda v: v[0] * v[1], [a, b])
    assert np.allclose(ga, (b * s).sum(axis=1, keepdims=True), atol=1e-8)
    assert np.allclose(gb, a * s, atol=1e-8)
    (gx,), s = differences(lambda v: v[0].reduce("sum_axes", 0), [b])
    assert np.allclose(gx, np.broadcast_to(s, b.shape), atol=1e-8)
    (gx,), s = differences(lambda v: v[0].unary("relu"), [b])
    assert np.allclose(gx, s * (b > 0), atol=1e-8)
    # A planted mistake (the wrong operand's value) is caught.
    assert not np.allclose(ga, (a * s).sum(axis=1, keepdims=True), atol=1e-3)


@pytest.mark.gpu
@pytest.mark.parametrize("name,inputs,apply", OPS, ids=[op[0] for op in OPS])
def test_every_operation_matches_finite_differences(name, inputs, apply):
    values = inputs()
    want, seed = differences(apply, values)
    tape = lib.Tape()
    leaves = [tape.tensor(a) for a in values]
    out = apply(leaves)
    expected = apply([Np(a) for a in values]).v
    assert out.shape == expected.shape, name
    assert_close(out.value(), expected, 1e-5, f"{name} value")
    out.backward(seed)
    for which, (leaf, g) in enumerate(zip(leaves, want)):
        got = leaf.grad()
        assert np.shape(got) == g.shape, f"{name}: gradient shape"
        assert_close(got, g, 2e-4, f"{name} d/d input{which}")
    tape.close()


@pytest.mark.gpu
def test_axis_extremes_share_the_adjoint_among_ties_and_skip_nans():
    # tensor_autodiff.rs:401-423
    tape = lib.Tape()
    x = tape.tensor(np.array([[1.0, 3.0, 3.0, 2.0], [np.nan, -1.0, 5.0, 5.0]]))
    top = x.reduce("max_axes", -1)
    assert np.array_equal(top.value(), [3.0, 5.0])
    top.reduce("sum").backward()
    assert np.array_equal(x.grad(), [[0, 0.5, 0.5, 0], [0, 0, 0.5, 0.5]])
    bottom = x.reduce("min_axes", [0, 1], True)
    assert np.array_equal(bottom.value(), [[-1.0]])
    bottom.reduce("sum").backward()
    assert np.array_equal(x.grad(), [[0, 0, 0, 0], [0, 1, 0, 0]])
    nans = tape.tensor(np.array([[np.nan, np.nan]]))
    nans.reduce("max_axes", 1).reduce("sum").backward()
    assert np.array_equal(nans.grad(), [[0.0, 0.0]])
    tape.close()


@pytest.mark.gpu
def test_elementwise_extremes_split_ties_and_sum_over_the_broadcast():
    # tensor_autodiff.rs:425-434
    tape = lib.Tape()
    x = tape.tensor(np.array([[1.0, 2.0], [3.0, 0.0]]))
    floor = tape.tensor(np.array([1.0, 1.0]))
    x.binary(floor, "maximum").reduce("sum").backward()
    assert np.array_equal(x.grad(), [[0.5, 1.0], [1.0, 0.0]])
    assert np.array_equal(floor.grad(), [0.5, 1.0])
    tape.close()


@pytest.mark.gpu
def test_whole_tensor_sums_and_means_are_lazy_scalars():
    # tensor_autodiff.rs:436-450
    tape = lib.Tape()
    values = filled((2, 3, 4), 1, -1, 1)
    x = tape.tensor(values)
    total, mean = x.reduce("sum"), x.reduce("mean")
    total.add_scalar(mean).backward()
    assert np.allclose(x.grad(), 1.0 + 1.0 / 24.0, rtol=0, atol=1e-7)
    assert abs(total.value() - values.sum()) <= 1e-5
    assert abs(mean.value() - values.sum() / 24) <= 1e-6
    tape.close()


@pytest.mark.gpu
def test_empty_and_unit_extents_differentiate():
    # After tensor_autodiff.rs:452-477: a [0, 3] tensor folds to zeros and
    # receives a [0, 3] gradient; the unit tensor's gradient is its partner.
    tape = lib.Tape()
    empty = tape.tensor(np.zeros((0, 3)))
    unit = tape.tensor(np.array([[[1.0], [2.0], [3.0]]]))
    folded = empty.reduce("sum_axes", 0)
    assert np.array_equal(folded.value(), [0.0, 0.0, 0.0])
    row = unit.layout("reshape", [3])
    ((folded + row) * row).reduce("sum").backward()
    assert empty.grad().shape == (0, 3)
    assert np.array_equal(unit.grad(), [[[2.0], [4.0], [6.0]]])
    # Narrowing to nothing sends nothing back, into an adjoint or not.
    x = tape.tensor(np.array([[1.0, 2.0], [3.0, 4.0]]))
    none = x.layout("narrow", [1, 1, 0])
    assert none.shape == (2, 0)
    (none.reduce("sum_axes", 1, True) + x).reduce("sum").backward()
    assert np.array_equal(x.grad(), np.ones((2, 2)))
    after = x.unary("scale", 2.0)
    (x.layout("narrow", [0, 2, 0]).reduce("sum_axes", 0) + after.reduce("sum_axes", 0)).reduce("sum").backward()
    assert np.array_equal(x.grad(), np.full((2, 2), 2.0))
    tape.close()


@pytest.mark.gpu
def test_a_second_backward_pass_gives_the_same_tensor_gradients():
    # tensor_autodiff.rs:484-496
    tape = lib.Tape()
    x = tape.tensor(filled((2, 3, 4), 1, -1, 1))
    loss = ((x * x.analytic(8)) + x.reduce("max_axes", 1, True)).reduce("sum")
    loss.backward()
    first = x.grad()
    loss.backward()
    assert np.array_equal(x.grad(), first)
    tape.zero_grad()
    assert not np.any(x.grad())
    tape.close()


@pytest.mark.gpu
def test_shapes_that_do_not_broadcast_are_rejected():
    # tensor_autodiff.rs:498-514
    tape = lib.Tape()
    a, b = tape.tensor(np.zeros((2, 3))), tape.tensor(np.zeros(4))
    with pytest.raises(lib.HipError, match=r"add: tensor shapes differ, \[2, 3\] and \[4\]"):
        a + b
    with pytest.raises(lib.HipError, match=r"sum_axes: axes \[1, -1\] are not distinct axes of shape \[2, 3\]"):
        a.reduce("sum_axes", [1, -1])
    with pytest.raises(lib.HipError, match=r"reshape: shape \[2, 3\] holds 6 elements"):
        a.layout("reshape", [4])
    with pytest.raises(lib.HipError, match=r"narrow: 2\.\.4 is out of range for axis 1 of shape \[2, 3\]"):
        a.layout("narrow", [1, 2, 2])
    with pytest.raises(lib.HipError, match=r"chunk: axis 1 of shape \[2, 3\] does not split into 2 equal parts"):
        a.split(1, parts=2)
    with pytest.raises(lib.HipError, match=r"concat: shapes \[2, 3\] and \[4\] differ off axis 0"):
        tape.join("concat", [a, b], 0)
    tape.close()
