"""The restated program optimizer (`oracle/fusion.py`) against the reference
crate's own tests (fusion/src/tests.rs), and the Host's Adam step it yields
against the product's encoded program.

The crate's tests fix what the restatement must do: rewrites without
reassociation leave every result's bits, with it stay within 1e-9 of an f64
evaluation; the chosen plan fits and never costs more than the program as
written; common subexpressions are merged; the exact identities remove
instructions; reassociation folds constants and saves divisions; a large
critical-path weight picks the balanced tree; register pressure falls to two
for a badly ordered sum.  The same random programs are generated from the
crate's LCG (tests.rs:105-163), so a mistake in a rewrite, a schedule, the
allocator or the cost that those tests would catch fails here too."""

import math

import numpy as np
import pytest

from oracle import binding as oracle
from oracle import fusion as F
from tensorcrate_amd import lib
from tensorcrate_amd.optim import EXACT, REASSOCIATE, adam_program, identity_place
from tests import host_programs as H

MASK = (1 << 64) - 1


class Lcg:
    """The crate tests' generator (tests.rs:105-122)."""

    def __init__(self, seed):
        self.state = seed

    def next(self):
        self.state = (self.state * 6364136223846793005 + 1442695040888963407) & MASK
        return self.state >> 33

    def below(self, n):
        return self.next() % n

    def unit(self):
        return self.next() / float(1 << 31)


def random_graph(rng, inputs, size, outputs):
    """tests.rs:124-163."""
    nodes = [("load", slot, 0) for slot in range(inputs)]
    for _ in range(size):
        n = len(nodes)

        def pick():
            return n - 1 - rng.below(min(n, 4))
        choice = rng.below(10)
        if choice == 0:
            c = rng.below(4)
            scalar = (F.lit(-1.0) if c == 0 else F.lit(1.0) if c == 1 else ("named", rng.below(3)) if c == 2
                      else F.lit(0.5 + rng.below(4)))
            node = ("const", scalar)
        elif choice == 1:
            f = [0, 8, 12, 13][rng.below(4)]
            node = ("un", f, pick())
        elif choice == 2:
            op = [F.MIN, F.MAX, F.LESS][rng.below(3)]
            a = pick()
            node = ("cmp", op, a, pick())
        elif choice == 3:
            a = pick()
            node = ("bin", F.DIV, a, pick())
        else:
            op = [F.ADD, F.SUB, F.MUL][rng.below(3)]
            a = pick()
            node = ("bin", op, a, rng.below(n))
        nodes.append(node)
    stores = [(len(nodes) - 1 - out * 2, out) for out in range(outputs)]
    return F.Graph(nodes, stores, [4] * inputs, [4] * outputs)


def f64_scalar(s, named):
    if s[0] == "lit":
        return F.lit_value(s)
    if s[0] == "named":
        return named[s[1]]
    return f64_binary(s[1], f64_scalar(s[2], named), f64_scalar(s[3], named))


def f64_binary(op, a, b):
    if op == F.ADD:
        return a + b
    if op == F.SUB:
        return a - b
    if op == F.MUL:
        return a * b
    if op == F.DIV:
        return a / b if b != 0 else (math.copysign(math.inf, a) * math.copysign(1, b) if a != 0 and a == a
                                     else math.nan)
    return math.fmod(a, b)


def f64_compare(op, a, b):
    if op == F.MIN:
        return b if a != a else (a if b != b else min(a, b))
    if op == F.MAX:
        return b if a != a else (a if b != b else max(a, b))
    if op == F.MAX_SHARE:
        return 1.0 if a > b else (0.0 if a < b else 0.5)
    flag = {F.LESS: a < b, F.LESS_EQUAL: a <= b, F.GREATER: a > b, F.GREATER_EQUAL: a >= b}[op]
    return 1.0 if flag else 0.0


def f64_unary(f, x):
    if f == 0:
        return math.sin(x) if math.isfinite(x) else math.nan
    if f == 8:
        try:
            return math.exp(x)
        except OverflowError:
            return math.inf
    if f == 12:
        return math.tanh(x)
    return math.sqrt(x) if x >= 0 else math.nan


def run_graph(graph, inputs, named):
    """tests.rs:61-77."""
    values = []
    for node in graph.nodes:
        kind = node[0]
        if kind == "load":
            values.append(inputs[node[1]])
        elif kind == "const":
            values.append(f64_scalar(node[1], named))
        elif kind == "bin":
            values.append(f64_binary(node[1], values[node[2]], values[node[3]]))
        elif kind == "un":
            values.append(f64_unary(node[1], values[node[2]]))
        else:
            values.append(f64_compare(node[1], values[node[2]], values[node[3]]))
    out = [math.nan] * len(graph.output_bytes)
    for value, output in graph.stores:
        out[output] = values[value]
    return out


def run_code(code, outputs, inputs, named):
    """tests.rs:80-103: the allocated code through its registers."""
    r = [math.nan] * 64
    out = [math.nan] * outputs
    for instr in code:
        kind = instr[0]
        if kind == "load":
            r[instr[1]] = inputs[instr[2]]
        elif kind == "const":
            r[instr[1]] = f64_scalar(instr[2], named)
        elif kind == "bin":
            r[instr[1]] = f64_binary(instr[2], r[instr[3]], r[instr[4]])
        elif kind == "un":
            r[instr[1]] = f64_unary(instr[2], r[instr[3]])
        elif kind == "cmp":
            r[instr[1]] = f64_compare(instr[2], r[instr[3]], r[instr[4]])
        else:
            out[instr[2]] = r[instr[1]]
    return out


def bits(values):
    return [np.float64(v).view(np.uint64) if v == v else "nan" for v in values]


def agree(a, b, tolerance):
    for x, y in zip(a, b):
        if x != x and y != y:
            continue
        if x == y:
            continue
        if not (abs(x - y) <= tolerance * (1.0 + max(abs(x), abs(y)))):
            return False
    return True


def test_every_candidate_computes_what_the_program_does():
    # tests.rs:173-221.
    rng = Lcg(7)
    for case in range(150):
        graph = random_graph(rng, 3, 6 + case % 14, 1 + case % 3)
        inputs = [1.0 + rng.unit() for _ in range(3)]
        named = [1.5, 0.25, 3.0]
        want = run_graph(graph, inputs, named)
        for plan in F.candidates(graph, reassociate=False):
            got = run_code(plan.code, len(graph.output_bytes), inputs, named)
            assert bits(got) == bits(want), (case, plan.variant)
            assert bits(run_graph(plan.graph, inputs, named)) == bits(got), (case, plan.variant)
        for plan in F.candidates(graph):
            got = run_code(plan.code, len(graph.output_bytes), inputs, named)
            assert agree(got, want, 1e-9), (case, plan.variant, got, want)


def test_the_chosen_program_fits_and_never_costs_more():
    # tests.rs:223-239.
    rng = Lcg(11)
    for case in range(100):
        graph = random_graph(rng, 4, 10 + case % 20, 2)
        written = F.cost(graph, F.BALANCED_MODEL)
        plan = F.optimize(graph)
        assert plan.registers <= 16
        assert plan.cost.total <= written.total + 1e-9, case


def one_store(nodes, store, inputs):
    return F.Graph(nodes, [(store, 0)], [4] * inputs, [4])


def test_common_subexpressions_are_computed_once():
    # tests.rs:260-287: exp(a + b) . exp(b + a).
    g = one_store([("load", 0, 0), ("load", 1, 0), ("bin", F.ADD, 0, 1), ("un", 8, 2), ("bin", F.ADD, 1, 0),
                   ("un", 8, 4), ("bin", F.MUL, 3, 5)], 6, 2)
    plan = F.optimize(g, reassociate=False)
    assert sum(1 for n in plan.graph.nodes if n[0] == "un") == 1
    assert plan.cost.special_ops == 1


def test_exact_identities_remove_instructions():
    # tests.rs:289-314: ((a . 1) - (b . -1)) / 1 = a + b.
    g = one_store([("load", 0, 0), ("load", 1, 0), ("const", F.lit(1.0)), ("const", F.lit(-1.0)),
                   ("bin", F.MUL, 0, 2), ("bin", F.MUL, 1, 3), ("bin", F.SUB, 4, 5), ("bin", F.DIV, 6, 2)], 7, 2)
    plan = F.optimize(g, reassociate=False)
    assert len(plan.graph.nodes) == 3
    assert plan.graph.nodes[2][:2] == ("bin", F.ADD)


def test_reassociation_folds_constants_and_saves_divisions():
    # tests.rs:316-357: ((x . 2) . 3) / y / z = x . (2 . 3) / (y . z).
    g = one_store([("load", 0, 0), ("load", 1, 0), ("load", 2, 0), ("const", F.lit(2.0)), ("const", F.lit(3.0)),
                   ("bin", F.MUL, 0, 3), ("bin", F.MUL, 5, 4), ("bin", F.DIV, 6, 1), ("bin", F.DIV, 7, 2)], 8, 3)
    plan = F.optimize(g)
    assert sum(1 for n in plan.graph.nodes if n[:2] == ("bin", F.DIV)) == 1
    constants = [n for n in plan.graph.nodes if n[0] == "const"]
    assert len(constants) == 1
    assert constants[0][1] == ("sbin", F.MUL, F.lit(2.0), F.lit(3.0))
    exact = F.optimize(g, reassociate=False)
    assert plan.cost.total < exact.cost.total


def test_a_balanced_sum_shortens_the_critical_path():
    # tests.rs:359-385.
    nodes = [("load", i, 0) for i in range(4)] + [("un", 8, i) for i in range(4)]
    nodes += [("bin", F.ADD, 4, 5), ("bin", F.ADD, 8, 6), ("bin", F.ADD, 9, 7)]
    g = one_store(nodes, 10, 4)
    model = F.CostModel(F.METAL.alpha, F.METAL.beta, 10.0, F.METAL.delta, F.METAL.epsilon)
    plan = F.optimize(g, model)
    assert plan.variant[0] == F.BALANCED
    assert plan.cost.critical_path < F.cost(g, model).critical_path


def test_register_pressure_is_minimized_and_limits_hold():
    # tests.rs:387-416.
    nodes = [("load", i, 0) for i in range(16)]
    acc = 0
    for i in range(1, 16):
        nodes.append(("bin", F.ADD, acc, i))
        acc = len(nodes) - 1
    g = one_store(nodes, acc, 16)
    assert F.cost(g, F.HOST).peak_registers >= 16
    assert F.optimize(g, reassociate=False).registers <= 2


# ---- the Host's Adam step ---------------------------------------------------------


@pytest.mark.parametrize("model", [F.BALANCED_MODEL, F.HOST, F.METAL], ids=["balanced", "host", "metal"])
@pytest.mark.parametrize("resumed", [False, True])
def test_the_optimizer_regroups_adams_step(model, resumed):
    # Under reassociation the chosen plan folds the first bias correction
    # and the rate into one constant and has one division; without it the
    # plan keeps both constants and the final product by the rate.
    plan = F.optimize(H.adam_graph(resumed, 4), model)
    assert plan.variant[0] in (F.LEFT_DEEP, F.BALANCED)
    folded = [n for n in plan.graph.nodes if n[0] == "const" and n[1][0] == "sbin" and n[1][1] == F.MUL]
    assert folded == [("const", ("sbin", F.MUL, ("named", H.FIRST_CORRECTION), ("named", H.RATE)))]
    assert not any(n == ("const", ("named", H.RATE)) for n in plan.graph.nodes)
    exact = F.optimize(H.adam_graph(resumed, 4), model, reassociate=False)
    assert exact.variant[0] == F.KEEP
    assert ("const", ("named", H.RATE)) in exact.graph.nodes
    assert plan.cost.total < exact.cost.total


def run_adam(dtype, code, grads, p0):
    """Steps of an encoded Adam program through the oracle's interpreter."""
    n = p0.size
    storage = {0: np.float32, 1: np.float16, 2: np.uint16}[dtype]
    p = p0.copy()
    m = v = None
    for code_at_step in code:
        places = [identity_place(1, n)] * code_at_step[1]
        if m is None:
            m, v = np.zeros(n, storage), np.zeros(n, storage)
            ins = [grads.pop(0), p]
        else:
            ins = [grads.pop(0), p, m, v]
        oracle.fused(dtype, code_at_step[0], places, ins, [p, m, v], 1, n)
    return p, m, v


@pytest.mark.parametrize("dtype,second_decay", [(lib.F32, 0.999), (lib.F16, 0.999), (lib.BF16, 0.99)])
@pytest.mark.parametrize("algebra", [REASSOCIATE, EXACT])
def test_the_products_adam_program_is_the_hosts(dtype, second_decay, algebra):
    # Four steps of the product's encoded step against the plan the restated
    # optimizer chooses for Adam::program, both interpreted by the oracle:
    # the same bits for parameters and both moments.
    rng = np.random.default_rng(31 + dtype)
    n = 4099
    storage = {0: np.float32, 1: np.float16, 2: np.uint16}[dtype]

    def to_storage(x):
        return x.astype(np.float32) if dtype == 0 else oracle.narrow(dtype, x.astype(np.float32))
    p0 = to_storage(rng.standard_normal(n))
    grads = [to_storage(rng.standard_normal(n) * 10.0 ** rng.integers(-3, 3, n)) for _ in range(4)]
    ours, host = [], []
    for step in range(1, 5):
        resumed = step > 1
        code, loads = adam_program(resumed, dtype, 1e-3, 0.9, second_decay, 1e-8, step, algebra)
        ours.append((code, loads))
        hcode, hloads, _ = H.host_adam_program(resumed, dtype, 1e-3, 0.9, second_decay, 1e-8, step,
                                               reassociate=algebra == REASSOCIATE)
        host.append((hcode, hloads))
    got = run_adam(dtype, ours, list(grads), p0)
    want = run_adam(dtype, host, list(grads), p0)
    for g, w in zip(got, want):
        assert g.dtype == storage
        assert np.array_equal(g.view(np.uint8), w.view(np.uint8))


def test_the_two_algebras_differ():
    # The regrouping is not exact: over many parameters some bits differ, and
    # every difference is within a few ulps of the step (about the rate) plus
    # a few of the parameter.
    rng = np.random.default_rng(5)
    n = 1 << 16
    p0 = rng.standard_normal(n).astype(np.float32)
    grads = [rng.standard_normal(n).astype(np.float32) for _ in range(3)]
    results = {}
    for algebra in (REASSOCIATE, EXACT):
        code = [adam_program(step > 1, lib.F32, 1e-3, 0.9, 0.999, 1e-8, step, algebra) for step in (1, 2, 3)]
        results[algebra] = run_adam(lib.F32, code, list(grads), p0)[0]
    a, b = results[REASSOCIATE], results[EXACT]
    differ = a != b
    assert differ.any()
    step_ulp = np.spacing(np.float32(1e-3))
    assert np.all(np.abs(a - b) <= 3 * 4 * step_ulp + 4 * np.spacing(np.maximum(np.abs(a), np.abs(b))))
