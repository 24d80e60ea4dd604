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
