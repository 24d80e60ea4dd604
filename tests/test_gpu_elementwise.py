"""Elementwise and broadcasting operations on the GPU against the oracle, bit
for bit, in every element type (kernels.rs:832-863, :912-938, :1162-1166;
tests/broadcast_reduce.rs:80-233 and tests/half.rs:115-185 are the
reference's versions)."""

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib
from tensorcrate_amd.tensor import Tensor
from tests.common import KINDS, bits_equal, filler, same, same_bits, to_kind, widen

pytestmark = pytest.mark.gpu

ARITH = [lib.ADD, lib.SUB, lib.MUL, lib.DIV, lib.REM]
CMP = [lib.MIN, lib.MAX, lib.MAX_SHARE, lib.LESS, lib.LESS_EQUAL, lib.GREATER, lib.GREATER_EQUAL]


def inputs(kind, n, seed):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal(n).astype(np.float32) * 4
    b = rng.standard_normal(n).astype(np.float32) * 2
    b[::7] = a[::7]  # ties for the comparisons
    a[::97] = np.nan
    return to_kind(a, kind), to_kind(b, kind)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n", [1, 7, 8, 9, 1001, 65536 + 3])
def test_same_shape_operations_are_bit_exact(kind, n):
    a, b = inputs(kind, n, n)
    da, db = lib.Buffer.of(a), lib.Buffer.of(b)
    out = lib.Buffer(a.nbytes)
    host = a.dtype
    for op in ARITH:
        lib.call("tc_elementwise", kind, op, da.ptr, db.ptr, out.ptr, n)
        assert same_bits(out.download(host, n), oracle.elementwise(kind, lib.ARITHMETIC, op, a, b), kind), op
    for op in CMP:
        lib.call("tc_compare", kind, op, da.ptr, db.ptr, out.ptr, n)
        got = widen(kind, out.download(host, n))
        assert same(got, widen(kind, oracle.elementwise(kind, lib.COMPARE, op, a, b))), op
    for left in (0, 1):
        for op in ARITH:
            lib.call("tc_broadcast", kind, op, da.ptr, 1.5, left, out.ptr, n)
            assert same_bits(out.download(host, n), oracle.scalar(kind, lib.ARITHMETIC, op, a, 1.5, left), kind), op
        for op in CMP:
            lib.call("tc_compare_scalar", kind, op, da.ptr, 0.0, left, out.ptr, n)
            got = widen(kind, out.download(host, n))
            assert same(got, widen(kind, oracle.scalar(kind, lib.COMPARE, op, a, 0.0, left))), op
    lib.call("tc_clamp", kind, da.ptr, -1.0, 2.0, out.ptr, n)
    assert same(widen(kind, out.download(host, n)), widen(kind, oracle.clamp(kind, a, -1.0, 2.0)))


@pytest.mark.parametrize("kind,n", [(lib.F32, (24 << 20) + 3), (lib.BF16, (48 << 20) + 5)])
def test_same_shape_operations_past_the_infinity_cache(kind, n):
    # Three operands of 96 MiB or more stream (non-temporal loads, plain
    # stores); the bits are the oracle's, tail elements included.
    a, b = inputs(kind, n, 3)
    da, db = lib.Buffer.of(a), lib.Buffer.of(b)
    out = lib.Buffer(a.nbytes)
    for op in ARITH:
        lib.call("tc_elementwise", kind, op, da.ptr, db.ptr, out.ptr, n)
        assert same_bits(out.download(a.dtype, n), oracle.elementwise(kind, lib.ARITHMETIC, op, a, b), kind), op


def test_unaligned_operands():
    # Views into the middle of a buffer: the element path, still exact.
    a, b = inputs(lib.F32, 1000, 5)
    da, db = lib.Buffer.of(a), lib.Buffer.of(b)
    out = lib.Buffer(a.nbytes)
    lib.call("tc_elementwise", lib.F32, lib.MUL, da.ptr + 4, db.ptr + 8, out.ptr + 4, 990)
    got = out.download(np.float32)[1:991]
    assert bits_equal(got, oracle.elementwise(lib.F32, lib.ARITHMETIC, lib.MUL, a[1:991], b[2:992]))


def broadcast_case(a_shape, b_shape, kind, shift=0.5):
    a = to_kind(filler(a_shape), kind) if a_shape else to_kind(np.array(2.5, np.float32), kind)
    b = to_kind(filler(b_shape) + np.float32(shift), kind) if b_shape else to_kind(np.array(2.5, np.float32), kind)
    return Tensor.from_numpy(a, kind), Tensor.from_numpy(b, kind), a, b


def check_broadcast(ta, tb, kind):
    va, vb = ta if not isinstance(ta, Tensor) else ta.view(), tb if not isinstance(tb, Tensor) else tb.view()
    shape = list(np.broadcast_shapes(va.shape, vb.shape))
    ba, bb = va.broadcast_to(shape), vb.broadcast_to(shape)
    a_host, b_host = va.storage.as_slice(), vb.storage.as_slice()
    for k, ops in [(lib.ARITHMETIC, ARITH), (lib.COMPARE, CMP)]:
        for op in ops:
            got = va.zip(vb, k, op).to_numpy()
            want = oracle.binary(kind, k, op, shape, a_host, ba.offset, list(ba.strides), b_host, bb.offset,
                                 list(bb.strides))
            assert same(widen(kind, got), widen(kind, want)), (k, op, shape)


@pytest.mark.parametrize("kind", KINDS)
def test_shapes_broadcast_from_the_last_axis(kind):
    # tests/broadcast_reduce.rs:109-124.
    for a_shape, b_shape in [([2, 3, 4], [4]), ([4], [2, 3, 4]), ([2, 3, 1], [1, 4]), ([2, 3, 4], []), ([], []),
                             ([2, 3, 5, 5], [5, 5]), ([2, 5, 4], [4]), ([2, 3, 5, 5], [2, 1, 1, 5])]:
        ta, tb, _, _ = broadcast_case(a_shape, b_shape, kind)
        check_broadcast(ta, tb, kind)


def test_broadcast_operands_may_be_non_contiguous_views():
    # tests/broadcast_reduce.rs:164-176.
    x = Tensor.from_numpy(filler([4, 3, 2]))
    xt = x.permute([2, 1, 0])
    wide = Tensor.from_numpy(filler([3, 8]) + np.float32(0.5))
    check_broadcast(xt, wide.narrow(1, 2, 4), lib.F32)
    check_broadcast(xt, wide.select(1, 5).unsqueeze(1), lib.F32)
    check_broadcast(xt, xt, lib.F32)


def test_power_is_within_tolerance():
    # `powf` is not correctly rounded on either side: a tolerance, pinned by
    # numpy in f64.
    rng = np.random.default_rng(9)
    a = rng.uniform(0.1, 3, (5, 33)).astype(np.float32)
    b = rng.uniform(-2, 2, (33,)).astype(np.float32)
    got = Tensor.from_numpy(a).power(Tensor.from_numpy(b)).to_numpy()
    want = a.astype(np.float64) ** b.astype(np.float64)
    assert np.allclose(got, want, rtol=4e-7)


def test_config3_broadcast_chain_at_full_size():
    # out = x * y + z with x [256, 512, 512] N(0,1), y [1, 512, 1], z [256, 1, 512]
    # U(-1, 1), seed 2: each step is one rounding, so numpy's own float32
    # arithmetic is the oracle's at this size.
    rng = np.random.default_rng(2)
    x = rng.standard_normal((256, 512, 512), dtype=np.float32)
    y = rng.uniform(-1, 1, (1, 512, 1)).astype(np.float32)
    z = rng.uniform(-1, 1, (256, 1, 512)).astype(np.float32)
    got = ((Tensor.from_numpy(x) * Tensor.from_numpy(y)) + Tensor.from_numpy(z)).to_numpy()
    assert np.array_equal(got, (x * y) + z)
    # The oracle itself, on a slab of the same layout.
    xs = x[:2]
    want = oracle.binary(lib.F32, lib.ARITHMETIC, lib.MUL, [2, 512, 512], xs, 0, [262144, 512, 1], y, 0, [0, 1, 0])
    assert np.array_equal(got[:2], oracle.binary(lib.F32, lib.ARITHMETIC, lib.ADD, [2, 512, 512], want, 0,
                                                 [262144, 512, 1], z, 0, [512, 0, 1]))


def test_fill_and_duplicate():
    for width, dtype in [(1, np.uint8), (2, np.uint16), (4, np.uint32), (8, np.uint64)]:
        for n in [1, 5, 16, 1000, 4099]:
            buffer = lib.Buffer(n * width + 16)
            value = np.array([0x5A], dtype)
            lib.call("tc_fill", buffer.ptr + width, n, width, value.ctypes.data)
            assert np.all(buffer.download(dtype, n + 1)[1:] == value[0])
    a = lib.Buffer.of(np.arange(100, dtype=np.float32))
    b = lib.Buffer(400)
    lib.call("tc_copy", b.ptr, a.ptr, 400)
    assert np.array_equal(b.download(np.float32), np.arange(100, dtype=np.float32))


def test_clamp_bounds_follow_the_reference():
    # A NaN bound is inert and only low > high is refused (shape.rs:30-43).
    a = np.array([-3.0, -0.5, 0.0, 0.5, 3.0, np.nan], np.float32)
    da, out = lib.Buffer.of(a), lib.Buffer(a.nbytes)
    lib.call("tc_clamp", lib.F32, da.ptr, float("nan"), 1.0, out.ptr, a.size)
    assert same(out.download(np.float32), np.fmin(np.fmax(a, np.nan), np.float32(1.0)))
    lib.call("tc_clamp", lib.F32, da.ptr, -1.0, float("nan"), out.ptr, a.size)
    assert same(out.download(np.float32), oracle.clamp(lib.F32, a, -1.0, float("nan")))
    with pytest.raises(lib.HipError, match="lower bound exceeds the upper"):
        lib.call("tc_clamp", lib.F32, da.ptr, 2.0, 1.0, out.ptr, a.size)
