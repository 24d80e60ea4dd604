"""The runtime under every entry point on the GPU: storage reuse fenced
against queued work and against captured graphs, and the counts of
operations queued and host waits (metal/pool.rs:34-48 and
src/counters.rs:33-135 are the reference's; metal/tests.rs:191-211,
:295-320 and :365-385 its tests)."""

import ctypes

import numpy as np
import pytest

from oracle import mlp
from tensorcrate_amd import lib
from tensorcrate_amd.tensor import Tensor

pytestmark = pytest.mark.gpu

TANH = 8  # Analytic::Tanh (kernels.rs:292-310)


class Graph:
    """A HIP graph captured from the library's stream (relaxed mode)."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so")
        vp = ctypes.c_void_p
        self.hip.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
        self.hip.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
        self.hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t]
        self.hip.hipGraphLaunch.argtypes = [vp, vp]
        self.hip.hipGraphExecDestroy.argtypes = [vp]
        self.hip.hipGraphDestroy.argtypes = [vp]
        self.stream = vp()
        lib.call("tc_stream", ctypes.byref(self.stream))
        self.graph, self.exec = vp(), vp()

    def __enter__(self):
        lib.sync()
        assert self.hip.hipStreamBeginCapture(self.stream, 2) == 0
        return self

    def __exit__(self, kind, value, trace):
        assert self.hip.hipStreamEndCapture(self.stream, ctypes.byref(self.graph)) == 0
        if kind is None:
            assert self.hip.hipGraphInstantiate(ctypes.byref(self.exec), self.graph, None, None, 0) == 0
        return False

    def replay(self):
        assert self.hip.hipGraphLaunch(self.exec, self.stream) == 0

    def destroy(self):
        self.hip.hipGraphExecDestroy(self.exec)
        self.hip.hipGraphDestroy(self.graph)


def test_a_recycled_allocation_is_never_clobbered_by_queued_work():
    # metal/tests.rs:191-211: queue a kernel, drop its output at once, and
    # upload into what may be the same storage; the upload must win.  Ten
    # rounds, since a race can be won by luck.
    source = lib.Buffer.of((np.arange(1 << 20) % 13 * 0.1).astype(np.float32))
    known = np.arange(1 << 20, dtype=np.float32)
    for round_ in range(10):
        out = lib.Buffer(4 << 20)
        lib.call("tc_unary", lib.F32, TANH, source.ptr, out.ptr, 1 << 20)
        out.free()
        fresh = lib.Buffer.of(known)
        assert np.array_equal(fresh.download(np.float32), known), round_
        fresh.free()


def test_storage_a_graph_touches_is_never_handed_to_eager_work():
    n = 1 << 18
    lib.call("tc_release_graph_memory")
    live0, retired0 = lib.graph_memory()
    assert (live0, retired0) == (0, 0)
    seven = ctypes.c_float(7.0)
    with Graph() as graph:
        # Allocated and freed inside the capture: its replays still write it.
        scratch = lib.Buffer(4 * n)
        lib.call("tc_fill", scratch.ptr, n, 4, ctypes.byref(seven))
        inside = scratch.ptr
        scratch.free()
        # Reused within the same capture: the graph's nodes keep their order.
        again = lib.Buffer(4 * n)
        assert again.ptr == inside
        lib.call("tc_fill", again.ptr, n, 4, ctypes.byref(seven))
        kept = again  # still live when the capture ends
    live, retired = lib.graph_memory()
    assert live >= 4 * n and retired == 0
    # Eager allocations of the same size get other storage, and keep what was
    # uploaded into them however often the graph replays.
    known = np.arange(n, dtype=np.float32)
    eager = [lib.Buffer.of(known) for _ in range(3)]
    assert all(buffer.ptr != inside for buffer in eager)
    for _ in range(3):
        graph.replay()
    lib.sync()
    for buffer in eager:
        assert np.array_equal(buffer.download(np.float32), known)
    assert np.all(kept.download(np.float32) == 7.0)
    # Freed after the capture, the graph's storage is retired, not cached.
    kept.free()
    live, retired = lib.graph_memory()
    assert live == 0 and retired >= 4 * n
    fresh = lib.Buffer(4 * n)
    assert fresh.ptr != inside
    # Once the caller says the graphs are gone, it is storage like any other.
    graph.destroy()
    lib.call("tc_release_graph_memory")
    assert lib.graph_memory() == (0, 0)
    for buffer in eager + [fresh]:
        buffer.free()


def test_copies_and_broadcasts_stay_queued_until_read():
    # metal/tests.rs:295-320 and :365-385: a broadcast, a permute, a concat
    # of two regions and a slice write queue their kernels without the host
    # waiting; only reading the result waits.
    x = Tensor.from_numpy(np.arange(2 * 3 * 4, dtype=np.float32).reshape(2, 3, 4))
    one = Tensor.from_numpy(np.ones((1, 3, 1), np.float32))
    lib.sync()
    dispatches, waits = lib.activity()
    y = x + one
    p = y.permute([2, 0, 1]).contiguous()
    joined = Tensor.concat([p, p], 0)
    joined.write_slice(0, 0, p)
    after, waited = lib.activity()
    assert waited == waits, "queued work waited on the host"
    assert after - dispatches >= 4
    got = joined.to_numpy()
    assert lib.activity()[1] > waits
    want = np.concatenate([(np.arange(24, dtype=np.float32).reshape(2, 3, 4) + 1).transpose(2, 0, 1)] * 2)
    assert np.array_equal(got, want)


def test_a_training_step_waits_only_when_its_loss_is_read():
    # tape/mod.rs:1286-1297: the loss is queued behind the step, and the
    # host blocks only when it asks for the value.
    widths, batch = (64, 128, 128, 32), 96
    weights, biases = mlp.he_init(widths, 3)
    x, y = mlp.batch_of(widths, batch, 3)
    net = lib.Mlp(widths, batch, weights, biases, x, y, 1e-3)
    net.step()
    net.loss()
    lib.sync()
    dispatches, waits = lib.activity()
    for _ in range(3):
        net.step()
    queued, waited = lib.activity()
    assert waited == waits, "a training step waited on the host"
    assert queued - dispatches >= 3 * 9, "nine products a step at least"
    loss = net.loss()
    assert np.isfinite(loss) and lib.activity()[1] == waits + 1
    net.close()


def test_a_split_reduction_replays_from_a_graph_like_its_eager_run():
    # A reduction over [0, 1] of [64, 128, 1024] splits each column's 8192
    # rows over blocks, whose partial states a second launch combines from
    # memory the runtime allocates; replays of a captured graph, with eager
    # work between them, must each give the eager result, bit for bit.
    rng = np.random.default_rng(21)
    host = rng.standard_normal((64, 128, 1024), dtype=np.float32)
    x = Tensor.from_numpy(host)
    eager = {name: getattr(x, f"{name}_axes")([0, 1]).to_numpy() for name in ("sum", "max", "var")}
    out = {}
    lib.call("tc_release_graph_memory")
    with Graph() as graph:
        for name in ("sum", "max", "var"):
            out[name] = getattr(x, f"{name}_axes")([0, 1])
    for replay in range(3):
        graph.replay()
        lib.sync()
        for name in ("sum", "max", "var"):
            assert np.array_equal(out[name].to_numpy(), eager[name]), (name, replay)
        # Eager work between the replays, allocating partials of its own.
        again = x.sum_axes([0, 1]).to_numpy()
        assert np.array_equal(again, eager["sum"])
    wide = host.astype(np.float64)
    assert np.allclose(eager["sum"], wide.sum((0, 1)), rtol=0, atol=1e-6 * np.sqrt(8192) * np.abs(wide).sum((0, 1)).max())
    assert np.array_equal(eager["max"], host.max((0, 1)))
    graph.destroy()
    del out
    lib.call("tc_release_graph_memory")


def test_compiled_programs_replay_from_a_graph_like_their_eager_runs():
    # The compiled forms of a program, captured once compiled: column sums
    # with their rows split (partial sums in memory the runtime allocates,
    # added by a second launch), row sums in runs, the one-kernel layer norm
    # (four waves a row, gamma loaded ahead) and a run-form program storing
    # f32.  Replays, with eager work between them, must each give the eager
    # result, bit for bit.
    from tests.common import EXP, Code, column_broadcast, identity_place, row_broadcast

    rng = np.random.default_rng(23)
    f32 = lib.F32
    # exp(x) * 0.5 + 0.25, summed along either axis of a 5000 x 64 matrix.
    code = Code()
    y = code.binary(lib.ADD, code.binary(lib.MUL, code.unary(EXP, code.load(0, 0, f32)), code.const(0.5)),
                    code.const(0.25))
    code.store(y, f32, 0)
    rows, cols = 5000, 64
    x = lib.Buffer.of(rng.uniform(-1, 1, rows * cols).astype(np.float32))
    place = [identity_place(rows, cols)]
    column_sums, row_sums = lib.Buffer(4 * cols), lib.Buffer(4 * rows)
    # (x - mean) / (deviations / cols + 1e-5) * gamma over 64 rows of 8192.
    ln_rows, ln_cols = 64, 8192
    ln = Code()
    centered = ln.binary(lib.SUB, ln.load(0, 0, f32), ln.load(1, 2, f32))
    scale = ln.binary(lib.ADD, ln.binary(lib.MUL, ln.load(1, 3, f32), ln.const(np.float32(1.0 / ln_cols))),
                      ln.const(1e-5))
    ln.store(ln.binary(lib.MUL, ln.binary(lib.DIV, centered, scale), ln.load(2, 1, f32)), f32, 0)
    ln_places = [identity_place(ln_rows, ln_cols), column_broadcast(ln_rows), row_broadcast(ln_cols)]
    whole = identity_place(ln_rows, ln_cols)
    lx = lib.Buffer.of(rng.uniform(-3, 3, ln_rows * ln_cols).astype(np.float32))
    gamma = lib.Buffer.of(rng.uniform(0.5, 1.5, ln_cols).astype(np.float32))
    normed = lib.Buffer(4 * ln_rows * ln_cols)
    stats = [(lx, ln_rows * ln_cols, f32, whole, "mean"), (lx, ln_rows * ln_cols, f32, whole, "deviations")]

    def run_all():
        lib.fused_sum(f32, code.code, place, [(x, rows * cols)], rows, cols, 1, column_sums)
        lib.fused_sum(f32, code.code, place, [(x, rows * cols)], rows, cols, 0, row_sums)
        lib.fused_with_statistics(f32, ln.code, ln_places, [(lx, ln_rows * ln_cols), (gamma, ln_cols)],
                                  [(normed, ln_rows * ln_cols)], ln_rows, ln_cols, stats)

    def read():
        return [column_sums.download(np.float32, cols), row_sums.download(np.float32, rows),
                normed.download(np.float32, ln_rows * ln_cols)]

    compiled = ctypes.c_uint64()
    run_all()
    run_all()  # the second appearance compiles each form
    lib.call("tc_fused_compiled", ctypes.byref(compiled))
    eager = read()
    for buffer, n in ((column_sums, cols), (row_sums, rows), (normed, ln_rows * ln_cols)):
        lib.call("tc_fill", buffer.ptr, n, 4, ctypes.byref(ctypes.c_float(0.0)))
    lib.call("tc_release_graph_memory")
    with Graph() as graph:
        run_all()
    for replay in range(3):
        graph.replay()
        lib.sync()
        got = read()
        for name, a, b in zip(("column sums", "row sums", "layer norm"), got, eager):
            assert np.array_equal(a, b), (name, replay)
        # Eager work between the replays, allocating partial sums of its own.
        lib.fused_sum(f32, code.code, place, [(x, rows * cols)], rows, cols, 1, column_sums)
        assert np.array_equal(column_sums.download(np.float32, cols), eager[0])
    after = ctypes.c_uint64()
    lib.call("tc_fused_compiled", ctypes.byref(after))
    assert after.value == compiled.value  # nothing compiled anew under capture
    graph.destroy()
    lib.call("tc_release_graph_memory")
