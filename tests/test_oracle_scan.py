"""The oracle's prefix sum and sort (`Kernels::vector_prefix_sum`,
`vector_sort`, kernels.rs:870-873) pinned on the reference's own answers
(tests/ordering.rs:99-135, tests/dtypes.rs:95-124), on closed forms (running
totals of ones, exact in f32 and rounded once per output), on numpy's sort
for NaN-free inputs, and on the totalOrder facts numpy's sort cannot see
(-0 before +0, NaNs at the ends by sign)."""

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib
from tests.common import KINDS, to_kind, widen

ASCENDING, DESCENDING = 0, 1
NAN_BITS = 0x7FC00000


def ordering_values(length):
    # tests/ordering.rs:14-18.
    return np.array([(i * 37 % 23) * 0.5 - 5.0 for i in range(length)], np.float32)


@pytest.mark.parametrize("length", [0, 1, 5, 15, 16, 17, 64, 100])
def test_prefix_sum_is_the_running_total(length):
    # tests/ordering.rs:99-108.
    values = ordering_values(length)
    got = oracle.prefix_sum(lib.F32, values)
    running = np.float32(0)
    for i, v in enumerate(values):
        running = np.float32(running + v)
        assert abs(got[i] - running) <= 1e-4


@pytest.mark.parametrize("kind", KINDS)
def test_prefix_sums_of_ones_round_each_total_once(kind):
    # dtypes.rs:121-123: 3000 f16 ones end at 3000.  Every running total of
    # ones is an integer below 2^24, exact in f32, so output i is i + 1
    # rounded once to the type (ties to even: bf16 gives 256 for 257 and 260 for 259).
    n = 10_000
    got = widen(kind, oracle.prefix_sum(kind, to_kind(np.ones(n), kind)))
    want = widen(kind, to_kind(np.arange(1, n + 1, dtype=np.float32), kind))
    assert np.array_equal(got, want)
    if kind == lib.F16:
        assert got[2999] == 3000.0
    if kind == lib.BF16:
        assert got[256] == 256.0 and got[258] == 260.0


def test_prefix_sum_against_f64():
    # A dropped or doubled term, or an exclusive scan, moves a total by a
    # whole element; the f32 left-to-right error is at most i u sum |x|.
    rng = np.random.default_rng(9)
    x = rng.uniform(-1, 1, 5000).astype(np.float32)
    got = oracle.prefix_sum(lib.F32, x).astype(np.float64)
    exact = np.cumsum(x.astype(np.float64))
    bound = np.arange(1, x.size + 1) * 2.0 ** -24 * np.cumsum(np.abs(x.astype(np.float64)))
    assert np.all(np.abs(got - exact) <= bound)


def test_sort_known_answers():
    # tests/ordering.rs:122-135: -NaN first, then -inf, -0 before +0, +NaN last.
    awkward = np.array([np.nan, 0.0, -0.0, -np.nan, 1.0, -np.inf], np.float32)
    awkward.view(np.uint32)[0] = NAN_BITS
    awkward.view(np.uint32)[3] = NAN_BITS | 0x80000000
    bits = oracle.sort(lib.F32, awkward, ASCENDING).view(np.uint32).tolist()
    assert bits == [NAN_BITS | 0x80000000, 0xFF800000, 0x80000000, 0, 0x3F800000, NAN_BITS]
    # tests/dtypes.rs:95-111 (in f32): the NaN sorts last ascending, first
    # descending.
    v = np.array([2.0, -0.0, np.nan, 0.0, -1.0, -np.inf], np.float32)
    v.view(np.uint32)[2] = NAN_BITS
    up = oracle.sort(lib.F32, v, ASCENDING)
    assert up.view(np.uint32).tolist() == [0xFF800000, 0xBF800000, 0x80000000, 0, 0x40000000, NAN_BITS]
    assert np.array_equal(oracle.sort(lib.F32, v, DESCENDING).view(np.uint32), up.view(np.uint32)[::-1])
    # tests/dtypes.rs:113-118: bf16 [1, 3, 2] descending.
    h = to_kind([1.0, 3.0, 2.0], lib.BF16)
    assert widen(lib.BF16, oracle.sort(lib.BF16, h, DESCENDING)).tolist() == [3.0, 2.0, 1.0]


@pytest.mark.parametrize("length", [0, 1, 5, 15, 16, 17, 64, 100])
@pytest.mark.parametrize("order", [ASCENDING, DESCENDING])
def test_sort_follows_the_ordering_fixture(length, order):
    # tests/ordering.rs:111-120: NaN-free values, so Python's `<` order is
    # the total order there.
    values = ordering_values(length)
    want = sorted(values.tolist(), reverse=order == DESCENDING)
    assert oracle.sort(lib.F32, values, order).tolist() == want


@pytest.mark.parametrize("kind", KINDS)
def test_sort_against_numpy_and_the_total_order_facts(kind):
    rng = np.random.default_rng(21 + kind)
    x = to_kind(rng.standard_normal(20_000) * np.exp(rng.uniform(-20, 20, 20_000)), kind)
    zeros = to_kind(np.array([0.0, -0.0] * 50, np.float32), kind)
    infs = to_kind(np.array([np.inf, -np.inf] * 5, np.float32), kind)
    x = np.concatenate([x, zeros, infs, x[:500]])  # duplicates too
    rng.shuffle(x)
    up = oracle.sort(kind, x, ASCENDING)
    wide = widen(kind, up)
    assert np.array_equal(wide, np.sort(widen(kind, x)))  # as numbers (-0 == +0)
    raw = up.view(np.uint32 if kind == lib.F32 else np.uint16)
    sign = 0x80000000 if kind == lib.F32 else 0x8000
    zero_at = np.flatnonzero(wide == 0)
    negative_zero = (raw[zero_at] & sign) != 0
    source = x.view(raw.dtype)
    count = int(np.sum(source == sign))  # -0 patterns in the input (underflows too)
    assert count >= 50 and negative_zero.sum() == count and negative_zero[:count].all()  # -0 first
    assert np.array_equal(np.sort(raw), np.sort(x.view(raw.dtype)))  # a permutation
    down = oracle.sort(kind, x, DESCENDING)
    assert np.array_equal(down.view(raw.dtype), raw[::-1])


@pytest.mark.parametrize("kind", [lib.F16, lib.BF16])
def test_sort_of_every_16_bit_pattern(kind):
    # All 65536 patterns: the NaNs with the sign set (0xFFFF down to the
    # first one past -inf) lead, the positive NaNs trail, and the numbers
    # between are in numeric order.
    x = np.arange(65536, dtype=np.uint16)
    np.random.default_rng(5).shuffle(x)
    host = x.view(np.float16) if kind == lib.F16 else x
    up = oracle.sort(kind, host, ASCENDING).view(np.uint16).astype(np.int64)
    exponent = 0x7C00 if kind == lib.F16 else 0x7F80
    negative_nans = np.arange(0xFFFF, 0x8000 | exponent, -1)
    positive_nans = np.arange(exponent + 1, 0x8000)
    assert np.array_equal(up[:negative_nans.size], negative_nans)
    assert np.array_equal(up[-positive_nans.size:], positive_nans)
    middle = up[negative_nans.size:65536 - positive_nans.size]
    numbers = widen(kind, middle.astype(np.uint16).view(np.float16) if kind == lib.F16 else middle.astype(np.uint16))
    assert np.all(np.diff(numbers) >= 0)
    assert middle[0] == 0x8000 | exponent and middle[-1] == exponent
