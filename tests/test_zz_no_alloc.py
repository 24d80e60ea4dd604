"""`tc_vector_reduce_noalloc`, the whole-buffer fold that allocates nothing,
against `tc_vector_reduce` (Kernels::vector_reduce, kernels.rs:867), which
runs the same kernels over storage from the cache: results must be the same
bits, for every type and fold, on calls in a row whose second is smaller
(the library's array then still holds the first call's partials past the
ones the second writes); and a call from a second stream while the array's
last use is still queued is refused."""

import ctypes

import numpy as np
import pytest

from tensorcrate_amd import lib
from tests.common import KINDS, KIND_NAMES, to_kind

pytestmark = pytest.mark.gpu


def fold(name, kind, buffer, n, op):
    out = lib.Buffer(4)
    lib.call(name, kind, buffer.ptr, n, op, out.ptr)
    return out.download(np.float32, 1)[0]


@pytest.mark.parametrize("kind", KINDS, ids=[KIND_NAMES[k] for k in KINDS])
@pytest.mark.parametrize("op", [lib.SUM, lib.RMIN, lib.RMAX], ids=["sum", "min", "max"])
def test_the_noalloc_fold_is_the_allocating_one(kind, op):
    rng = np.random.default_rng(17 + kind * 3 + op)
    for n in (48_000_003, 1_000_001, 5000, 1):
        x = to_kind(rng.standard_normal(n).astype(np.float32), kind)
        buffer = lib.Buffer.of(x)
        want = fold("tc_vector_reduce", kind, buffer, n, op)
        got = fold("tc_vector_reduce_noalloc", kind, buffer, n, op)
        assert np.array_equal(np.float32(got).view(np.uint32), np.float32(want).view(np.uint32)), (n, got, want)
        buffer.free()


def test_the_noalloc_fold_refuses_an_unknown_fold():
    buffer = lib.Buffer(16)
    out = lib.Buffer(4)
    with pytest.raises(lib.HipError, match="no Reduce 3"):
        lib.call("tc_vector_reduce_noalloc", lib.F32, buffer.ptr, 4, 3, out.ptr)


def test_the_noalloc_fold_over_nothing_is_the_identity():
    out = lib.Buffer(4)
    lib.call("tc_vector_reduce_noalloc", lib.F32, None, 0, lib.SUM, out.ptr)
    assert out.download(np.float32, 1)[0] == 0.0
    lib.call("tc_vector_reduce_noalloc", lib.F32, None, 0, lib.RMAX, out.ptr)
    assert out.download(np.float32, 1)[0] == -np.inf


def test_a_call_from_another_stream_is_refused_while_the_array_is_in_use():
    # The array belongs to the stream of its last call.  Another thread (its
    # own stream) queues a fold behind about 4 ms of copies; while that fold
    # is queued, a fold from this thread's stream is refused instead of
    # racing on the array, and once the other stream has drained it runs
    # and gives the allocating fold's bits.
    import threading

    n = 1 << 20
    x = lib.Buffer.of(np.random.default_rng(5).standard_normal(n).astype(np.float32))
    want = fold("tc_vector_reduce", lib.F32, x, n, lib.SUM)
    big = 4 << 30
    src, dst = lib.Buffer(big), lib.Buffer(big)
    theirs, ours = lib.Buffer(4), lib.Buffer(4)
    queued, go = threading.Event(), threading.Event()
    failure = []

    def other():
        try:
            for _ in range(3):
                lib.call("tc_copy", dst.ptr, src.ptr, big)
            lib.call("tc_vector_reduce_noalloc", lib.F32, x.ptr, n, lib.SUM, theirs.ptr)
        except Exception as error:  # reported by the main thread
            failure.append(error)
        queued.set()
        go.wait()
        lib.call("tc_sync")

    worker = threading.Thread(target=other)
    worker.start()
    try:
        assert queued.wait(60)
        assert not failure, failure
        with pytest.raises(lib.HipError, match="in use by another stream"):
            lib.call("tc_vector_reduce_noalloc", lib.F32, x.ptr, n, lib.SUM, ours.ptr)
    finally:
        go.set()
        worker.join()
    lib.call("tc_vector_reduce_noalloc", lib.F32, x.ptr, n, lib.SUM, ours.ptr)
    for out in (theirs, ours):
        got = out.download(np.float32, 1)[0]
        assert np.float32(got).view(np.uint32) == np.float32(want).view(np.uint32)
    for buffer in (x, src, dst, theirs, ours):
        buffer.free()
