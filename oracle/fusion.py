"""The reference's fused-program optimizer, restated in Python: TEST
INFRASTRUCTURE ONLY.  Nothing in the product imports it.

The Host backend runs every program built with a `fused::Builder` (the
optimizers' steps among them) through the `tensorcrate-fusion` crate before
interpreting it (`build_with`, src/tensors/fused/mod.rs:2282-2470;
`optimized`, :2549-2586).  Under the default `Algebra::Reassociate`
(fused/mod.rs:2473-2491) the crate may regroup associative chains and fold
their constants, so the bits the Host computes are those of the plan the
crate chooses, not of the program as built.  This module restates that
choice so the tests can derive the Host's program for a given graph:

- `rewrite` (fusion/src/rewrite.rs:36-437): hash-consing, canonical operand
  order, the exact identities, and chains flattened and rebuilt left-deep or
  balanced with their constants folded into one;
- `rematerialize` (rewrite.rs:439-549);
- the schedules (fusion/src/schedule.rs:131-340) and register allocation
  (:342-408);
- the cost (fusion/src/cost.rs, optimize.rs:96-150) and the candidates,
  sorted by cost with ties kept in their order (optimize.rs:152-215).

Graphs are lists of nodes, tuples of
  ("load", slot, remap) | ("const", scalar) | ("bin", op, a, b)
  | ("un", function, a) | ("cmp", op, a, b)
and scalars tuples of ("lit", value) | ("named", index) | ("sbin", op, a, b).
Operation codes are the reference's (`Bin`, `Cmp`, graph.rs:12-75).
"""

from __future__ import annotations

import math
import struct
from dataclasses import dataclass, field

ADD, SUB, MUL, DIV, REM = range(5)
MIN, MAX, MAX_SHARE, LESS, LESS_EQUAL, GREATER, GREATER_EQUAL = range(7)
SQRT = 13

KEEP, LEFT_DEEP, BALANCED = "keep", "left_deep", "balanced"
NOTHING, CONSTANTS, CONSTANTS_AND_LOADS = "nothing", "constants", "constants_and_loads"
AS_BUILT, DEPTH_FIRST, LEAST_LIVE, CRITICAL_PATH, EXHAUSTIVE = (
    "as_built", "depth_first", "least_live", "critical_path", "exhaustive")


def lit(value: float) -> tuple:
    """A literal scalar, kept as its f64 bits so -0.0 and 0.0 differ
    (`Scalar::literal`, graph.rs:110-113)."""
    return ("lit", struct.unpack("<Q", struct.pack("<d", float(value)))[0])


def lit_value(scalar: tuple) -> float | None:
    if scalar[0] != "lit":
        return None
    return struct.unpack("<d", struct.pack("<Q", scalar[1]))[0]


def scalar_is(scalar: tuple, value: float) -> bool:
    """`Scalar::is` (graph.rs:123-127): a literal with exactly these bits."""
    return scalar[0] == "lit" and scalar == lit(value)


@dataclass
class Graph:
    """`Graph` (graph.rs:185-196)."""
    nodes: list
    stores: list  # (value, output)
    input_bytes: list
    output_bytes: list

    def stored(self) -> list:
        out = [False] * len(self.nodes)
        for value, _ in self.stores:
            out[value] = True
        return out

    def users(self) -> list:
        """Each value's readers, in order, without repeats (graph.rs:207-218)."""
        users = [[] for _ in self.nodes]
        for at, node in enumerate(self.nodes):
            for operand in operands(node):
                if at not in users[operand]:
                    users[operand].append(at)
        return users

    def key(self) -> tuple:
        return (tuple(self.nodes), tuple(self.stores), tuple(self.input_bytes), tuple(self.output_bytes))


def operands(node: tuple) -> list:
    kind = node[0]
    if kind in ("bin", "cmp"):
        return [node[2], node[3]]
    if kind == "un":
        return [node[2]]
    return []


def remapped(node: tuple, f) -> tuple:
    kind = node[0]
    if kind in ("bin", "cmp"):
        return (kind, node[1], f(node[2]), f(node[3]))
    if kind == "un":
        return (kind, node[1], f(node[2]))
    return node


def distinct(node: tuple) -> list:
    """Operands with an immediate repeat removed (`distinct`, schedule.rs:82-86)."""
    out = []
    for operand in operands(node):
        if not out or out[-1] != operand:
            out.append(operand)
    return out


def commutes(op: int) -> bool:
    return op in (ADD, MUL)


def mirrored(op: int):
    return {MIN: MIN, MAX: MAX, LESS: GREATER, LESS_EQUAL: GREATER_EQUAL, GREATER: LESS,
            GREATER_EQUAL: LESS_EQUAL}.get(op)


# ---- rewrite.rs ----------------------------------------------------------------


class Rebuilder:
    """`Rebuilder` (rewrite.rs:53-234): nodes hash-consed as they are built,
    commutative operands in canonical order, exact identities applied."""

    def __init__(self, relaxed: bool):
        self.nodes: list = []
        self.index: dict = {}
        self.relaxed = relaxed

    def push(self, node: tuple) -> int:
        found = self.index.get(node)
        if found is not None:
            return found
        self.nodes.append(node)
        self.index[node] = len(self.nodes) - 1
        return len(self.nodes) - 1

    def constant(self, scalar: tuple) -> int:
        return self.push(("const", scalar))

    def scalar(self, value: int):
        node = self.nodes[value]
        return node[1] if node[0] == "const" else None

    def is_constant(self, value: int, of: float) -> bool:
        s = self.scalar(value)
        return s is not None and scalar_is(s, of)

    def negation_of(self, value: int):
        node = self.nodes[value]
        if node[0] == "bin" and node[1] == MUL:
            if self.is_constant(node[3], -1.0):
                return node[2]
            if self.is_constant(node[2], -1.0):
                return node[3]
        return None

    def negate(self, value: int) -> int:
        return self.binary(MUL, value, self.constant(lit(-1.0)))

    def binary(self, op: int, a: int, b: int) -> int:
        x, y = self.scalar(a), self.scalar(b)
        if x is not None and y is not None:
            return self.constant(("sbin", op, x, y))
        if op == MUL:
            if self.is_constant(b, 1.0):
                return a
            if self.is_constant(a, 1.0):
                return b
            if self.is_constant(b, -1.0):
                n = self.negation_of(a)
                if n is not None:
                    return n
            if self.is_constant(a, -1.0):
                n = self.negation_of(b)
                if n is not None:
                    return n
        elif op == DIV and self.is_constant(b, 1.0):
            return a
        elif op == SUB:
            if self.is_constant(b, 0.0):
                return a
            n = self.negation_of(b)
            if n is not None:
                return self.binary(ADD, a, n)
        elif op == ADD:
            if self.is_constant(b, -0.0):
                return a
            if self.is_constant(a, -0.0):
                return b
            n = self.negation_of(b)
            if n is not None:
                return self.binary(SUB, a, n)
            n = self.negation_of(a)
            if n is not None:
                return self.binary(SUB, b, n)
        if commutes(op) and b < a:
            a, b = b, a
        return self.push(("bin", op, a, b))

    def compare(self, op: int, a: int, b: int) -> int:
        mirror = None if (op in (MIN, MAX) and not self.relaxed) else mirrored(op)
        if mirror is not None and b < a:
            return self.push(("cmp", mirror, b, a))
        return self.push(("cmp", op, a, b))

    def copy(self, node: tuple, mapping: list) -> int:
        kind = node[0]
        if kind == "bin":
            return self.binary(node[1], mapping[node[2]], mapping[node[3]])
        if kind == "cmp":
            return self.compare(node[1], mapping[node[2]], mapping[node[3]])
        if kind == "un":
            return self.push(("un", node[1], mapping[node[2]]))
        return self.push(node)

    def reduce_with(self, terms: list, association: str, combine) -> int:
        assert terms, "a chain has at least one term"
        level = list(terms)
        if association == BALANCED:
            while len(level) > 1:
                nxt = []
                for i in range(0, len(level), 2):
                    pair = level[i:i + 2]
                    nxt.append(combine(pair[0], pair[1]) if len(pair) == 2 else pair[0])
                level = nxt
            return level[0]
        acc = level[0]
        for term in level[1:]:
            acc = combine(acc, term)
        return acc

    def reduce(self, op: int, terms: list, association: str) -> int:
        return self.reduce_with(terms, association, lambda a, b: self.binary(op, a, b))

    def split_constants(self, terms: list):
        values, constants = [], []
        for inverse, value in terms:
            s = self.scalar(value)
            if s is not None:
                constants.append((inverse, s))
            else:
                values.append((inverse, value))
        values.sort(key=lambda t: (t[1], t[0]))
        return values, constants


SUM, PRODUCT, FMIN, FMAX = "sum", "product", "min", "max"


def family(graph: Graph, value: int):
    node = graph.nodes[value]
    if node[0] == "bin" and node[1] in (ADD, SUB):
        return SUM
    if node[0] == "bin" and node[1] in (MUL, DIV):
        return PRODUCT
    if node[0] == "cmp" and node[1] == MIN:
        return FMIN
    if node[0] == "cmp" and node[1] == MAX:
        return FMAX
    return None


def source_negation(graph: Graph, value: int):
    def minus_one(v):
        n = graph.nodes[v]
        return n[0] == "const" and scalar_is(n[1], -1.0)
    node = graph.nodes[value]
    if node[0] == "bin" and node[1] == MUL:
        if minus_one(node[3]):
            return node[2]
        if minus_one(node[2]):
            return node[3]
    return None


def flatten(graph, absorbable, value, root, inverse, fam, out):
    """A chain's terms (rewrite.rs:272-322): flattened only through links that
    are the root or read by nothing else."""
    through = root or absorbable[value]
    node = graph.nodes[value]
    if fam == SUM and node[0] == "bin" and node[1] in (ADD, SUB) and through:
        flatten(graph, absorbable, node[2], False, inverse, fam, out)
        flatten(graph, absorbable, node[3], False, inverse ^ (node[1] == SUB), fam, out)
    elif fam == SUM and node[0] == "bin" and node[1] == MUL and through and \
            source_negation(graph, value) is not None:
        flatten(graph, absorbable, source_negation(graph, value), False, not inverse, fam, out)
    elif fam == PRODUCT and node[0] == "bin" and node[1] in (MUL, DIV) and through:
        flatten(graph, absorbable, node[2], False, inverse, fam, out)
        flatten(graph, absorbable, node[3], False, inverse ^ (node[1] == DIV), fam, out)
    elif ((fam == FMIN and node[0] == "cmp" and node[1] == MIN) or
          (fam == FMAX and node[0] == "cmp" and node[1] == MAX)) and through:
        flatten(graph, absorbable, node[2], False, False, fam, out)
        flatten(graph, absorbable, node[3], False, False, fam, out)
    else:
        out.append((inverse, value))


def reassociate(builder: Rebuilder, graph, absorbable, mapping, value, fam, association) -> int:
    """rewrite.rs:324-399."""
    terms: list = []
    flatten(graph, absorbable, value, True, False, fam, terms)
    mapped = [(inverse, mapping[v]) for inverse, v in terms]
    if fam in (FMIN, FMAX):
        op = MIN if fam == FMIN else MAX
        values = sorted(set(v for _, v in mapped))
        return builder.reduce_with(values, association, lambda x, y: builder.compare(op, x, y))
    values, constants = builder.split_constants(mapped)
    combine, invert = (ADD, SUB) if fam == SUM else (MUL, DIV)
    folded = None
    for inverse, s in constants:
        if folded is not None:
            folded = ("sbin", invert if inverse else combine, folded, s)
        elif not inverse:
            folded = s
        elif fam == SUM:
            folded = ("sbin", MUL, s, lit(-1.0))
        else:
            folded = ("sbin", DIV, lit(1.0), s)
    direct = [v for inv, v in values if not inv]
    inverted = [v for inv, v in values if inv]
    if folded is not None:
        direct.append(builder.constant(folded))
    if direct and not inverted:
        return builder.reduce(combine, direct, association)
    if direct and inverted:
        a = builder.reduce(combine, direct, association)
        b = builder.reduce(combine, inverted, association)
        return builder.binary(invert, a, b)
    assert inverted, "a chain has at least one term"
    b = builder.reduce(combine, inverted, association)
    if fam == SUM:
        return builder.negate(b)
    return builder.binary(DIV, builder.constant(lit(1.0)), b)


def rewrite(graph: Graph, association: str) -> Graph:
    """rewrite.rs:401-437."""
    relaxed = association != KEEP
    users = graph.users()
    stored = graph.stored()
    absorbable = [len(users[v]) == 1 and not stored[v] for v in range(len(graph.nodes))]
    builder = Rebuilder(relaxed)
    mapping: list = []
    for value, node in enumerate(graph.nodes):
        fam = family(graph, value)
        if fam is not None and relaxed:
            mapping.append(reassociate(builder, graph, absorbable, mapping, value, fam, association))
        else:
            mapping.append(builder.copy(node, mapping))
    stores = [(mapping[v], out) for v, out in graph.stores]
    return eliminate_dead(Graph(builder.nodes, stores, list(graph.input_bytes), list(graph.output_bytes)))


def eliminate_dead(graph: Graph) -> Graph:
    """rewrite.rs:439-472."""
    live = [False] * len(graph.nodes)
    for v, _ in graph.stores:
        live[v] = True
    for v in range(len(graph.nodes) - 1, -1, -1):
        if live[v]:
            for operand in operands(graph.nodes[v]):
                live[operand] = True
    renumber = [None] * len(graph.nodes)
    nodes = []
    for v, node in enumerate(graph.nodes):
        if live[v]:
            renumber[v] = len(nodes)
            nodes.append(remapped(node, lambda o: renumber[o]))
    return Graph(nodes, [(renumber[v], out) for v, out in graph.stores], graph.input_bytes, graph.output_bytes)


def rematerialize(graph: Graph, what: str) -> Graph:
    """rewrite.rs:474-549."""
    def chosen(node):
        if what == NOTHING:
            return False
        if node[0] == "const":
            return True
        return what == CONSTANTS_AND_LOADS and node[0] == "load"
    if what == NOTHING or not any(chosen(n) for n in graph.nodes):
        return Graph(list(graph.nodes), list(graph.stores), graph.input_bytes, graph.output_bytes)
    stored = graph.stored()
    nodes: list = []
    mapping = [None] * len(graph.nodes)
    for value, node in enumerate(graph.nodes):
        if chosen(node):
            if stored[value]:
                mapping[value] = len(nodes)
                nodes.append(node)
            continue
        copies: list = []
        for operand in operands(node):
            if chosen(graph.nodes[operand]) and not any(f == operand for f, _ in copies):
                copies.append((operand, len(nodes)))
                nodes.append(graph.nodes[operand])

        def at(operand, copies=copies):
            for f, t in copies:
                if f == operand:
                    return t
            return mapping[operand]
        mapping[value] = len(nodes)
        nodes.append(remapped(node, at))
    return Graph(nodes, [(mapping[v], out) for v, out in graph.stores], graph.input_bytes, graph.output_bytes)


# ---- schedule.rs -------------------------------------------------------------


def peak(graph: Graph, order: list) -> int:
    """schedule.rs:88-106."""
    users = [len(u) for u in graph.users()]
    stored = graph.stored()
    remaining = list(users)
    live = best = 0
    for value in order:
        dying = 0
        for operand in distinct(graph.nodes[value]):
            remaining[operand] -= 1
            if remaining[operand] == 0 and not stored[operand]:
                dying += 1
        live = live + 1 - dying
        best = max(best, live)
    return best


def finish_times(graph: Graph, latency) -> list:
    finish = [0.0] * len(graph.nodes)
    for value, node in enumerate(graph.nodes):
        start = max([finish[o] for o in operands(node)], default=0.0)
        finish[value] = start + latency(node)
    return finish


def heights(graph: Graph, latency) -> list:
    users = graph.users()
    height = [0.0] * len(graph.nodes)
    for value in range(len(graph.nodes) - 1, -1, -1):
        after = max([height[u] for u in users[value]], default=0.0)
        height[value] = after + latency(graph.nodes[value])
    return height


def needs(graph: Graph) -> list:
    """schedule.rs:154-173."""
    need = [1] * len(graph.nodes)
    for value, node in enumerate(graph.nodes):
        if node[0] == "un":
            need[value] = need[node[2]]
        elif node[0] in ("bin", "cmp"):
            a, b = node[2], node[3]
            if a == b:
                need[value] = need[a]
            elif need[a] == need[b]:
                need[value] = need[a] + 1
            else:
                need[value] = max(need[a], need[b])
    return need


def depth_first(graph: Graph) -> list:
    need = needs(graph)
    emitted = [False] * len(graph.nodes)
    order: list = []

    def visit(value):
        if emitted[value]:
            return
        ops = distinct(graph.nodes[value])
        ops = sorted(ops, key=lambda o: -need[o])  # stable, like Rust's sort_by_key
        for o in ops:
            visit(o)
        emitted[value] = True
        order.append(value)
    for v, _ in graph.stores:
        visit(v)
    return order


def list_schedule(graph: Graph, latency, critical_first: bool) -> list:
    """schedule.rs:205-263."""
    users_len = [len(u) for u in graph.users()]
    stored = graph.stored()
    height = heights(graph, latency)
    remaining = list(users_len)
    waiting = [len(distinct(n)) for n in graph.nodes]
    users = graph.users()
    ready = [v for v in range(len(graph.nodes)) if waiting[v] == 0]
    order: list = []

    def growth(value):
        dying = sum(1 for o in distinct(graph.nodes[value]) if remaining[o] == 1 and not stored[o])
        return 1 - dying

    def key(i):
        v = ready[i]
        # by growth: smaller first; by height: larger first; then the value.
        if critical_first:
            return (-height[v], growth(v), v)
        return (growth(v), -height[v], v)
    while ready:
        best = min(range(len(ready)), key=key)
        value = ready[best]
        # Vec::swap_remove: the last element takes the removed one's place.
        ready[best] = ready[-1]
        ready.pop()
        for o in distinct(graph.nodes[value]):
            remaining[o] -= 1
        order.append(value)
        for u in users[value]:
            waiting[u] -= 1
            if waiting[u] == 0:
                ready.append(u)
    return order


def exhaustive(graph: Graph):
    """Branch and bound over every order (schedule.rs:265-340)."""
    users = graph.users()
    stored = graph.stored()
    state = {"best_peak": math.inf, "best": None, "visited": 0}
    waiting = [len(distinct(n)) for n in graph.nodes]
    remaining = [len(u) for u in users]
    order: list = []

    def step(live, pk):
        state["visited"] += 1
        if pk >= state["best_peak"] or state["visited"] > 200_000:
            return
        if len(order) == len(graph.nodes):
            state["best_peak"] = pk
            state["best"] = list(order)
            return
        ready = [v for v in range(len(graph.nodes)) if waiting[v] == 0 and v not in order]
        for value in ready:
            ops = distinct(graph.nodes[value])
            dying = 0
            for o in ops:
                remaining[o] -= 1
                if remaining[o] == 0 and not stored[o]:
                    dying += 1
            now = live + 1 - dying
            for u in users[value]:
                waiting[u] -= 1
            order.append(value)
            step(now, max(pk, now))
            order.pop()
            for u in users[value]:
                waiting[u] += 1
            for o in ops:
                remaining[o] += 1
    step(0, 0)
    return state["best"]


def orders(graph: Graph, latency, exhaustive_limit: int) -> list:
    found: list = []

    def offer(schedule, order):
        if not any(existing == order for _, existing in found):
            found.append((schedule, order))
    offer(AS_BUILT, list(range(len(graph.nodes))))
    offer(DEPTH_FIRST, depth_first(graph))
    offer(LEAST_LIVE, list_schedule(graph, latency, False))
    offer(CRITICAL_PATH, list_schedule(graph, latency, True))
    if len(graph.nodes) <= exhaustive_limit:
        best = exhaustive(graph)
        if best is not None:
            offer(EXHAUSTIVE, best)
    return found


def allocate(graph: Graph, order: list):
    """Registers in `order` (schedule.rs:342-408): a result takes the register
    of its first dying operand, else the lowest free one, else a new one.
    Returns (code, registers); code entries are ("load", dst, slot, remap),
    ("const", dst, scalar), ("bin", dst, op, a, b), ("un", dst, f, a),
    ("cmp", dst, op, a, b) and ("store", src, output)."""
    users_len = [len(u) for u in graph.users()]
    stored = graph.stored()
    remaining = list(users_len)
    free: list = []
    nxt = 0
    assigned = [None] * len(graph.nodes)
    code = []
    for value in order:
        node = graph.nodes[value]
        released = []
        for o in distinct(node):
            remaining[o] -= 1
            if remaining[o] == 0 and not stored[o]:
                released.append(assigned[o])
        if released:
            dst = released[0]
        elif free:
            position = min(range(len(free)), key=lambda i: free[i])
            dst = free[position]
            free[position] = free[-1]
            free.pop()
        else:
            dst = nxt
            nxt += 1
        free.extend(released[1:])
        kind = node[0]
        if kind == "load":
            code.append(("load", dst, node[1], node[2]))
        elif kind == "const":
            code.append(("const", dst, node[1]))
        elif kind == "bin":
            code.append(("bin", dst, node[1], assigned[node[2]], assigned[node[3]]))
        elif kind == "un":
            code.append(("un", dst, node[1], assigned[node[2]]))
        else:
            code.append(("cmp", dst, node[1], assigned[node[2]], assigned[node[3]]))
        assigned[value] = dst
    for v, out in graph.stores:
        code.append(("store", assigned[v], out))
    return code, nxt


# ---- cost.rs, optimize.rs ---------------------------------------------------------


@dataclass(frozen=True)
class Latency:
    load: float = 4.0
    constant: float = 0.0
    arithmetic: float = 1.0
    divide: float = 4.0
    sqrt: float = 4.0
    transcendental: float = 16.0


@dataclass(frozen=True)
class CostModel:
    """`CostModel` (cost.rs:27-99): the three the reference defines."""
    alpha: float
    beta: float
    gamma: float
    delta: float
    epsilon: float
    latency: Latency = field(default_factory=Latency)


HOST = CostModel(1.0, 0.1, 0.05, 0.25, 4.0)
METAL = CostModel(0.25, 0.5, 0.25, 1.0, 2.0)
BALANCED_MODEL = CostModel(0.6, 0.3, 0.15, 0.6, 3.0)


def latency_of(model: CostModel):
    lat = model.latency

    def f(node):
        kind = node[0]
        if kind == "load":
            return lat.load
        if kind == "const":
            return lat.constant
        if kind == "bin" and node[1] in (DIV, REM):
            return lat.divide
        if kind in ("bin", "cmp"):
            return lat.arithmetic
        return lat.sqrt if node[1] == SQRT else lat.transcendental
    return f


@dataclass
class Cost:
    instructions: int
    peak_registers: int
    critical_path: float
    memory_bytes: int
    special_ops: int
    total: float


def cost_of(graph: Graph, registers: int, model: CostModel) -> Cost:
    """optimize.rs:96-130 and `Cost::weigh` (cost.rs:113-133)."""
    finish = finish_times(graph, latency_of(model))
    critical = max([finish[v] for v, _ in graph.stores], default=0.0)
    memory = special = 0
    for node in graph.nodes:
        if node[0] == "load":
            memory += graph.input_bytes[node[1]]
        elif (node[0] == "bin" and node[1] in (DIV, REM)) or node[0] == "un":
            special += 1
    for _, out in graph.stores:
        memory += graph.output_bytes[out]
    instructions = len(graph.nodes)
    total = (model.alpha * instructions + model.beta * registers + model.gamma * critical +
             model.delta * memory + model.epsilon * special)
    return Cost(instructions, registers, critical, memory, special, total)


def reorder(graph: Graph, order: list) -> Graph:
    position = [0] * len(graph.nodes)
    for at, value in enumerate(order):
        position[value] = at
    nodes = [remapped(graph.nodes[v], lambda o: position[o]) for v in order]
    return Graph(nodes, [(position[v], out) for v, out in graph.stores], graph.input_bytes, graph.output_bytes)


@dataclass
class Plan:
    graph: Graph
    code: list
    registers: int
    cost: Cost
    variant: tuple  # (association, rematerialize, schedule)


def candidates(graph: Graph, model: CostModel = BALANCED_MODEL, reassociate: bool = True,
               exhaustive_limit: int = 10) -> list:
    """Every equivalent program, cheapest first, ties in the order built
    (optimize.rs:152-205; Rust's `sort_by` is stable)."""
    latency = latency_of(model)
    associations = [KEEP] + ([LEFT_DEEP, BALANCED] if reassociate else [])
    written = eliminate_dead(Graph(list(graph.nodes), list(graph.stores), graph.input_bytes, graph.output_bytes))
    code, registers = allocate(written, list(range(len(written.nodes))))
    plans = [Plan(written, code, registers, cost_of(written, registers, model), (KEEP, NOTHING, AS_BUILT))]
    seen: list = []
    for association in associations:
        rewritten = rewrite(graph, association)
        for what in (NOTHING, CONSTANTS, CONSTANTS_AND_LOADS):
            variant = rematerialize(rewritten, what)
            if variant.key() in seen:
                continue
            seen.append(variant.key())
            for schedule, order in orders(variant, latency, exhaustive_limit):
                ordered = reorder(variant, order)
                code, registers = allocate(ordered, list(range(len(ordered.nodes))))
                plans.append(Plan(ordered, code, registers, cost_of(ordered, registers, model),
                                  (association, what, schedule)))
    plans.sort(key=lambda p: p.cost.total)
    return plans


def optimize(graph: Graph, model: CostModel = BALANCED_MODEL, reassociate: bool = True,
             max_registers: int = 16, max_instructions: int = 256) -> Plan:
    """The cheapest plan that fits (optimize.rs:207-215)."""
    for plan in candidates(graph, model, reassociate):
        if plan.registers <= max_registers and len(plan.code) <= max_instructions:
            return plan
    raise ValueError("no equivalent program fits the register and instruction limits")


def cost(graph: Graph, model: CostModel) -> Cost:
    """optimize.rs:217-223: the program as written."""
    written = eliminate_dead(Graph(list(graph.nodes), list(graph.stores), graph.input_bytes, graph.output_bytes))
    _, registers = allocate(written, list(range(len(written.nodes))))
    return cost_of(written, registers, model)
