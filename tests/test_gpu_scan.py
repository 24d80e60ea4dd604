"""The prefix sum and the sort on the GPU (`tc_prefix_sum`, `tc_sort`;
`Kernels::vector_prefix_sum`, `vector_sort`, kernels.rs:870-873) against the
oracle.  The sort is bit-exact in totalOrder, NaNs and signed zeros
included.  The prefix sum adds in a fixed tree order, not the host's left to
right: it is bit-exact where every running total is exact in f32 (the
reference's own case, tests/half.rs:390-391), bit-identical from run to run,
and otherwise within D 2^-24 sum_{j<=i} |x_j| of the exact total, D = 64 +
n / 2^20 bounding the additions on any path, plus the one rounding to the
type (tests/half.rs:263-268 compare the two within 1 ulp at 300 elements)."""

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib
from tests.common import KINDS, to_kind, widen

pytestmark = pytest.mark.gpu

HOST = {lib.F32: np.float32, lib.F16: np.float16, lib.BF16: np.uint16}
UNIT = {lib.F32: 2.0 ** -24, lib.F16: 2.0 ** -11, lib.BF16: 2.0 ** -8}
ASCENDING, DESCENDING = 0, 1


def device_prefix_sum(kind, x):
    a = lib.Buffer.of(x) if x.size else lib.Buffer(16)
    out = lib.Buffer(max(x.nbytes, 16))
    lib.call("tc_prefix_sum", kind, a.ptr, out.ptr, x.size)
    return out.download(HOST[kind], x.size)


def device_sort(kind, x, order):
    a = lib.Buffer.of(x) if x.size else lib.Buffer(16)
    out = lib.Buffer(max(x.nbytes, 16))
    lib.call("tc_sort", kind, a.ptr, out.ptr, x.size, order)
    return out.download(HOST[kind], x.size)


@pytest.mark.parametrize("kind", KINDS)
def test_prefix_sum_of_ones_is_exact(kind):
    n = 10_000
    ones = to_kind(np.ones(n), kind)
    got = device_prefix_sum(kind, ones)
    assert np.array_equal(got.view(np.uint8), oracle.prefix_sum(kind, ones).view(np.uint8))
    if kind == lib.F16:
        assert widen(kind, got)[2999] == 3000.0


@pytest.mark.parametrize("n", [0, 1, 5, 15, 16, 17, 64, 100, 4095, 4096, 4097, 300_001])
def test_prefix_sum_of_half_integers_matches_the_host(n):
    # tests/ordering.rs:14-18's values: multiples of 0.5 whose totals stay
    # exact in f32, so any order of adding gives the host's bits.
    x = np.array([(i * 37 % 23) * 0.5 - 5.0 for i in range(n)], np.float32)
    assert np.array_equal(device_prefix_sum(lib.F32, x), oracle.prefix_sum(lib.F32, x))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("special", ["inf", "-inf", "nan", "inf_then_minus_inf", "spike"])
def test_prefix_sum_keeps_specials_out_of_earlier_outputs(kind, special):
    # An infinity, a NaN or a very large element part-way into a tile (and in
    # a later tile) must not reach the outputs before it: the host's running
    # total is finite up to there (vector.rs:578-589).  Where the special
    # sits and what follows it match the host's classes exactly; finite
    # outputs stay within the f64 bound of the other prefix-sum tests.
    n = 3 * 4096 + 123
    x = np.full(n, 0.1, np.float32)
    spots = [2050, 4096 + 3000]
    if special == "spike":
        x[spots[0]] = 1e9 if kind == lib.F32 else (60000.0 if kind == lib.F16 else 1e9)
    elif special == "inf_then_minus_inf":
        x[spots[0]], x[spots[1]] = np.inf, -np.inf
    else:
        x[spots[0]] = {"inf": np.inf, "-inf": -np.inf, "nan": np.nan}[special]
    x = to_kind(x, kind)
    got = widen(kind, device_prefix_sum(kind, x)).astype(np.float64)
    host = widen(kind, oracle.prefix_sum(kind, x)).astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(host))
    assert np.array_equal(np.isposinf(got), np.isposinf(host)) and np.array_equal(np.isneginf(got), np.isneginf(host))
    assert np.all(np.isfinite(got[:spots[0]]))
    finite = np.isfinite(host)
    wide = widen(kind, x).astype(np.float64)
    with np.errstate(invalid="ignore"):
        exact = np.cumsum(np.where(np.isfinite(wide), wide, 0.0))
        scale = np.cumsum(np.abs(np.where(np.isfinite(wide), wide, 0.0)))
    depth = 64 + n / 2 ** 20
    bound = depth * 2.0 ** -24 * scale + UNIT[kind] * (np.abs(exact) + depth * 2.0 ** -24 * scale) + 2.0 ** -24
    assert np.all(np.abs(got[finite] - exact[finite]) <= bound[finite])


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n", [1, 300, 4097, 1 << 20, (1 << 22) + 17, (1 << 26) + 5])
def test_prefix_sum_against_f64(kind, n):
    if kind != lib.F32 and n > (1 << 22) + 17:
        pytest.skip("the f32 case covers the multi-chunk offsets at this size")
    rng = np.random.default_rng(n + kind)
    x = to_kind(rng.uniform(-1, 1, n).astype(np.float32), kind)
    got = device_prefix_sum(kind, x)
    wide = widen(kind, x).astype(np.float64)
    exact = np.cumsum(wide)
    scale = np.cumsum(np.abs(wide))
    depth = 64 + n / 2 ** 20
    bound = depth * 2.0 ** -24 * scale + UNIT[kind] * (np.abs(exact) + depth * 2.0 ** -24 * scale) + 2.0 ** -24
    g = widen(kind, got).astype(np.float64)
    assert np.all(np.abs(g - exact) <= bound)
    if n <= (1 << 20):
        # The host's left-to-right total within its own bound i u sum |x|.
        host = widen(kind, oracle.prefix_sum(kind, x)).astype(np.float64)
        left_to_right = np.arange(1, n + 1) * 2.0 ** -24 * scale
        assert np.all(np.abs(host - exact) <= left_to_right + UNIT[kind] * (np.abs(exact) + left_to_right) + 2.0 ** -24)
    again = device_prefix_sum(kind, x)
    assert np.array_equal(got.view(np.uint8), again.view(np.uint8))  # deterministic


def special_values(kind, n, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * np.exp(rng.uniform(-30, 30, n))).astype(np.float32)
    picks = rng.integers(0, n, size=min(n, 64))
    x[picks[: len(picks) // 2]] = rng.choice(np.array([0.0, -0.0, np.inf, -np.inf], np.float32), len(picks) // 2)
    x = to_kind(x, kind)
    if n >= 8:
        raw = x.view(np.uint32 if kind == lib.F32 else np.uint16)
        nan = 0x7FC00001 if kind == lib.F32 else (0x7E01 if kind == lib.F16 else 0x7FC1)
        sign = 0x80000000 if kind == lib.F32 else 0x8000
        raw[picks[-4:]] = [nan, nan | sign, nan + 2, (nan + 2) | sign]
        raw[picks[-8:-4]] = raw[picks[:4]]  # duplicates
    return x


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n", [0, 1, 2, 17, 1000, 4097, (1 << 20) + 7, (1 << 24) + 3])
def test_sort_is_the_total_order_exactly(kind, n):
    if kind != lib.F32 and n > (1 << 20) + 7:
        pytest.skip("16-bit keys are covered by every pattern below")
    x = special_values(kind, n, n + 7 * kind)
    for order in [ASCENDING, DESCENDING]:
        got = device_sort(kind, x, order)
        want = oracle.sort(kind, x, order)
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), order


@pytest.mark.parametrize("kind", [lib.F16, lib.BF16])
def test_sort_of_every_16_bit_pattern(kind):
    x = np.tile(np.arange(65536, dtype=np.uint16), 3)
    np.random.default_rng(kind).shuffle(x)
    host = x.view(np.float16) if kind == lib.F16 else x
    for order in [ASCENDING, DESCENDING]:
        got = device_sort(kind, host, order)
        assert np.array_equal(got.view(np.uint16), oracle.sort(kind, host, order).view(np.uint16)), order


def test_sort_rejects_an_unknown_order():
    x = np.ones(4, np.float32)
    with pytest.raises(lib.HipError, match="no SortOrder 2"):
        device_sort(lib.F32, x, 2)
