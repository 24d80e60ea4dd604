"""Axis reductions and arg-reductions on the GPU against the oracle
(Kernels::reduce_axes / arg_reduce, kernels.rs:1175-1187; strided.rs:80-225;
tests/broadcast_reduce.rs:236-873 are the reference's versions).

max/min and the arg indices are bit-exact.  Sum, mean and variance fold in a
different order from the host's left-to-right loop, so they are held to a
tolerance against the f64 value: |got - want| <= tol * sqrt(depth) * sum|x|
(the scale a sum of `depth` roundings can reach), with tol the element
type's unit roundoff (f32 2^-24, f16 2^-11, bf16 2^-8) plus the final
rounding to the element type.
"""

import itertools

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib
from tensorcrate_amd.tensor import Tensor
from tests.common import KINDS, CapturedGraph, bits_equal, filler, same, to_kind, widen

pytestmark = pytest.mark.gpu

UNIT = {lib.F32: 2.0 ** -24, lib.F16: 2.0 ** -11, lib.BF16: 2.0 ** -8}
# Half the subnormal spacing: the absolute rounding error below the normals.
TINY = {lib.F32: 2.0 ** -150, lib.F16: 2.0 ** -25, lib.BF16: 2.0 ** -134}


def slices(x, axes):
    kept = [k for k in range(x.ndim) if k not in axes]
    moved = np.transpose(x, kept + list(axes))
    return moved.reshape(int(np.prod([x.shape[k] for k in kept], dtype=np.int64)), -1).astype(np.float64)


def check_sum_like(got, want, scale, depth, kind, what=""):
    """Within the accumulated-rounding bound, plus the output's rounding."""
    bound = 2.0 ** -24 * np.sqrt(max(depth, 1)) * 4 * scale + UNIT[kind] * np.abs(want) + TINY[kind]
    excess = np.abs(got.astype(np.float64) - want) - bound
    worst = int(np.argmax(excess))
    assert np.all(excess <= 0), (what, worst, float(got[worst]), float(want[worst]), float(excess[worst]))


def check_all_reductions(view, x_values, kind):
    """Every subset of axes, against the oracle (exact ops) and f64 (sums)."""
    host = view.storage.as_slice()
    for r in range(1, view.rank + 1):
        for axes in itertools.combinations(range(view.rank), r):
            axes = list(axes)
            s = slices(x_values, axes)
            depth = s.shape[1]
            for op, name in [(lib.RMAX, "max_axes"), (lib.RMIN, "min_axes")]:
                got = getattr(view, name)(axes).to_numpy()
                want = oracle.reduce(kind, host, list(view.shape), view.offset, list(view.strides), axes, lib.FOLD, op)
                assert bits_equal(got, want), (axes, name)
            scale = np.abs(s).sum(1)
            got = widen(kind, view.sum_axes(axes).to_numpy()).reshape(-1)
            check_sum_like(got, s.sum(1), scale, depth, kind, ("sum", axes))
            got = widen(kind, view.mean_axes(axes).to_numpy()).reshape(-1)
            check_sum_like(got, s.mean(1), scale / depth, depth, kind, ("mean", axes))
            for correction, divisor in [("population", depth), ("sample", depth - 1)]:
                if divisor < 1:
                    continue
                got = widen(kind, view.var_axes(axes, correction).to_numpy()).reshape(-1)
                dev = s - s.mean(1, keepdims=True)
                want = (dev ** 2).sum(1) / divisor
                check_sum_like(got, want, (dev ** 2).sum(1) / divisor + np.abs(s).max(1) ** 2 / divisor, depth, kind,
                               ("var", correction, axes))


@pytest.mark.parametrize("kind", KINDS)
def test_reductions_over_every_subset_of_axes(kind):
    # tests/broadcast_reduce.rs:387-399.
    x = filler([2, 3, 4, 5])
    t = Tensor.from_numpy(to_kind(x, kind), kind)
    check_all_reductions(t.view(), x, kind)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("shape", [[2, 3, 4, 5], [3, 2, 5, 70], [80, 3, 2, 4]])
def test_device_shapes_of_the_reference(kind, shape):
    # The shapes tests/broadcast_reduce.rs:776-786 checks Metal against Host on.
    rng = np.random.default_rng(sum(shape))
    x = to_kind(rng.standard_normal(shape).astype(np.float32), kind)
    xv = widen(kind, x).reshape(shape)
    t = Tensor.from_numpy(x, kind)
    check_all_reductions(t.view(), xv, kind)


def test_reductions_read_non_contiguous_views_in_place():
    # tests/broadcast_reduce.rs:401-415.
    x = filler([3, 4, 5, 6])
    t = Tensor.from_numpy(x)
    for view, values in [(t.permute([2, 0, 3, 1]), x.transpose(2, 0, 3, 1)),
                         (t.narrow(3, 1, 4).transpose(0, 2), x[:, :, :, 1:5].transpose(2, 1, 0, 3)),
                         (t.select(1, 2).slice(2, 1, 5), x[:, 2, :, 1:5])]:
        check_all_reductions(view, values, lib.F32)
    row = Tensor.from_numpy(filler([5]))
    repeated = row.broadcast_to([3, 5])
    assert repeated.sum_axes(0).to_numpy().tolist() == (3 * filler([5])).tolist()


def test_empty_and_single_element_reductions():
    # tests/broadcast_reduce.rs:450-492.
    empty = Tensor.filled([2, 0, 3], 0.0)
    assert empty.sum_axes(1).to_numpy().tolist() == [[0.0] * 3] * 2
    assert empty.max_axes(1, keep_dims=True).to_numpy().tolist() == [[[-np.inf] * 3]] * 2
    assert np.all(np.isnan(empty.mean_axes(1).to_numpy()))
    assert empty.sum_axes(2).shape == (2, 0)
    assert empty.argmax(2).shape == (2, 0)
    single = Tensor.from_numpy(filler([3, 1]))
    assert np.all(np.isnan(single.var_axes(1, "sample").to_numpy()))
    assert single.var_axes(1, "population").to_numpy().tolist() == [0.0, 0.0, 0.0]


def test_compact_sums_accumulate_in_f32():
    ones = Tensor.filled([2, 10000], 1.0, lib.F16)
    assert widen(lib.F16, ones.sum_axes(1).to_numpy()).tolist() == [10000.0, 10000.0]
    ones = Tensor.filled([3, 1000], 1.0, lib.BF16)
    assert widen(lib.BF16, ones.mean_axes(-1).to_numpy()).tolist() == [1.0, 1.0, 1.0]


def test_extremes_pass_over_nans():
    nan = np.nan
    x = Tensor.from_numpy(np.array([[1.0, nan, 3.0], [nan, nan, nan], [-2.0, 5.0, nan]], np.float32))
    assert x.max_axes(1).to_numpy().tolist() == [3.0, -np.inf, 5.0]
    assert x.min_axes(1).to_numpy().tolist() == [1.0, np.inf, -2.0]
    assert x.max_axes(0).to_numpy().tolist() == [1.0, 5.0, 3.0]
    assert x.argmax(1).to_numpy().tolist() == [2, 0, 1]
    assert x.argmin(1).to_numpy().tolist() == [0, 0, 0]
    assert x.argmax(0).to_numpy().tolist() == [0, 2, 0]
    assert np.isnan(x.sum_axes(1).to_numpy()[0])


def test_ties_go_to_the_first_position():
    tied = Tensor.from_numpy(np.array([[1.0, 7.0, 7.0, 2.0], [-3.0, -3.0, 0.0, -3.0]], np.float32))
    assert tied.argmax(1).to_numpy().tolist() == [1, 2]
    assert tied.argmin(1, keep_dims=True).to_numpy().tolist() == [[0], [0]]


@pytest.mark.parametrize("kind", KINDS)
def test_arg_extremes_along_every_axis(kind):
    # tests/broadcast_reduce.rs:553-562: many ties from the filler, long
    # contiguous and long strided axes, against the oracle.
    for shape, perm in [([2, 3, 4, 5], [3, 1, 0, 2]), ([3, 300, 2], [0, 1, 2]), ([4, 5, 130], [2, 0, 1]),
                        ([7, 1000], [1, 0])]:
        x = to_kind(filler(shape), kind)
        t = Tensor.from_numpy(x, kind).permute(perm)
        for axis in range(t.rank):
            for op, name in [(lib.RMAX, "argmax"), (lib.RMIN, "argmin")]:
                got = getattr(t, name)(axis).to_numpy()
                want = oracle.arg_reduce(kind, x, list(t.shape), t.offset, list(t.strides), axis, op)
                assert np.array_equal(got, want), (shape, perm, axis, name)


def test_arg_extremes_with_nans_in_long_slices():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((64, 300)).astype(np.float32)
    x[rng.random(x.shape) < 0.2] = np.nan
    x[5] = np.nan
    t = Tensor.from_numpy(x)
    for axis in (0, 1):
        for op, name in [(lib.RMAX, "argmax"), (lib.RMIN, "argmin")]:
            view = t.view()
            want = oracle.arg_reduce(lib.F32, x, [64, 300], 0, [300, 1], axis, op)
            assert np.array_equal(getattr(view, name)(axis).to_numpy(), want)


def test_config2_reductions():
    # [64, 128, 1024] N(0,1), seed 1: sum/max/min/mean/var over axis 2 and
    # over axes [0, 1]; argmax/argmin over axis 1.
    rng = np.random.default_rng(1)
    x = rng.standard_normal((64, 128, 1024), dtype=np.float32)
    t = Tensor.from_numpy(x)
    flat = x.reshape(-1)
    for axes in ([2], [0, 1]):
        for op, name in [(lib.RMAX, "max_axes"), (lib.RMIN, "min_axes")]:
            want = oracle.reduce(lib.F32, flat, [64, 128, 1024], 0, [131072, 1024, 1], axes, lib.FOLD, op)
            assert bits_equal(getattr(t, name)(axes).to_numpy(), want)
        s = slices(x, axes)
        depth = s.shape[1]
        scale = np.abs(s).sum(1)
        check_sum_like(t.sum_axes(axes).to_numpy().reshape(-1), s.sum(1), scale, depth, lib.F32)
        check_sum_like(t.mean_axes(axes).to_numpy().reshape(-1), s.mean(1), scale / depth, depth, lib.F32)
        dev = s - s.mean(1, keepdims=True)
        want = (dev ** 2).sum(1) / depth
        check_sum_like(t.var_axes(axes).to_numpy().reshape(-1), want, want + np.abs(s).max(1) ** 2 / depth, depth,
                       lib.F32)
        # The oracle's own sequential sum agrees with f64 to the same bound.
        mine = oracle.reduce(lib.F32, flat, [64, 128, 1024], 0, [131072, 1024, 1], axes, lib.FOLD, lib.SUM)
        check_sum_like(mine.reshape(-1), s.sum(1), scale, depth, lib.F32)
    for op, name in [(lib.RMAX, "argmax"), (lib.RMIN, "argmin")]:
        want = oracle.arg_reduce(lib.F32, flat, [64, 128, 1024], 0, [131072, 1024, 1], 1, op)
        assert np.array_equal(getattr(t, name)(1).to_numpy(), want)


def test_reductions_past_the_infinity_cache():
    # 320 MiB, over the 256 MiB Infinity Cache: the row and column kernels
    # stream with nontemporal loads.  Max and the arg indices stay bit-exact
    # (numpy's max and first-index argmax are the Host rule on NaN-free
    # data); sums and variances stay within the accumulated-rounding bound.
    rng = np.random.default_rng(14)
    x = rng.standard_normal((80, 1024, 1024), dtype=np.float32)
    t = Tensor.from_numpy(x)
    assert bits_equal(t.max_axes([2]).to_numpy(), x.max(2))
    assert bits_equal(t.min_axes([0]).to_numpy(), x.min(0))
    assert np.array_equal(t.argmax(2).to_numpy(), x.argmax(2))
    assert np.array_equal(t.argmin(0).to_numpy(), x.argmin(0))
    for axes in ([2], [0]):
        s = slices(x, axes)
        depth = s.shape[1]
        check_sum_like(t.sum_axes(axes).to_numpy().reshape(-1), s.sum(1), np.abs(s).sum(1), depth, lib.F32, axes)
        dev = s - s.mean(1, keepdims=True)
        want = (dev ** 2).sum(1) / depth
        check_sum_like(t.var_axes(axes).to_numpy().reshape(-1), want, want + np.abs(s).max(1) ** 2 / depth, depth,
                       lib.F32, axes)
        del s, dev


def test_whole_vector_reduce_and_dot():
    rng = np.random.default_rng(12)
    for n in [1, 15, 16, 1000, 1 << 20]:
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        da, db = lib.Buffer.of(a), lib.Buffer.of(b)
        result = lib.Buffer(4)
        for op, want in [(lib.RMAX, a.max()), (lib.RMIN, a.min())]:
            lib.call("tc_vector_reduce", lib.F32, da.ptr, n, op, result.ptr)
            assert result.download(np.float32)[0] == want
        lib.call("tc_vector_reduce", lib.F32, da.ptr, n, lib.SUM, result.ptr)
        want = a.astype(np.float64).sum()
        assert abs(result.download(np.float32)[0] - want) <= 2.0 ** -24 * 4 * np.sqrt(n) * np.abs(a).sum()
        lib.call("tc_dot", lib.F32, da.ptr, db.ptr, n, result.ptr)
        want = np.dot(a.astype(np.float64), b)
        assert abs(result.download(np.float32)[0] - want) <= 2.0 ** -24 * 4 * np.sqrt(n) * np.abs(a * b).sum()


def test_split_column_reductions_replay_from_a_graph_with_the_eager_bits():
    # A column reduction split across blocks writes partial states to
    # scratch and merges them in a second kernel, in a fixed order.  Captured
    # into a HIP graph (on a thread of its own, so on a stream of its own) and
    # replayed three times, with the program's own downloads between the
    # replays, it gives the eager bits every time.
    import threading

    rng = np.random.default_rng(15)
    x = rng.standard_normal((8192, 1024), dtype=np.float32)
    eager = Tensor.from_numpy(x)
    want = [eager.sum_axes([0]).to_numpy(), eager.var_axes([0]).to_numpy(), eager.max_axes([0]).to_numpy(),
            eager.argmax(0).to_numpy()]
    assert bits_equal(want[2], x.max(0))
    assert np.array_equal(want[3], x.argmax(0))
    failures = []

    def captured():
        try:
            lib.call("tc_init", 0)
            t = Tensor.from_numpy(x)
            lib.sync()
            graph = CapturedGraph(lambda: [t.sum_axes([0]), t.var_axes([0]), t.max_axes([0]), t.argmax(0)])
            for replay in range(3):
                graph.replay()
                for k, (got, expected) in enumerate(zip(graph.result, want)):
                    if not bits_equal(got.to_numpy(), expected):
                        failures.append((replay, k))
            graph.close()
        except Exception as error:  # reported on the test's thread
            failures.append(repr(error))

    worker = threading.Thread(target=captured)
    worker.start()
    worker.join()
    assert not failures, failures
