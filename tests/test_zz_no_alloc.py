"""`tc_vector_reduce_noalloc`, the whole-buffer fold that allocates nothing,
against `tc_vector_reduce` (Kernels::vector_reduce, kernels.rs:867), which
runs the same kernels over storage from the cache: results must be the same
bits, for every type and fold, on calls in a row whose second is smaller
(the library's array then still holds the first call's partials past the
ones the second writes)."""

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
