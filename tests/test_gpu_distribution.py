"""Distribution functions on the GPU (`tc_distribution`,
`tc_axis_distribution`; `Kernels::vector_distribution`,
`matrix_distribution`, `matrix_axis_distribution`, kernels.rs:1046-1070)
against the oracle.  Both evaluate the Host's f64 methods in the Host's order
and round once to f32 (then to the type); they differ only where the GPU's
f64 `exp`/`log` differ from the C library's by an ulp of f64, so every
element is within one ulp of the element type, NaN for NaN, and all but a few
in ten thousand are bit-identical.  (The reference's Metal tier, computing in
f32, is held to 1e-5 .. 1e-3 relative, tests/statistics.rs:653-735.)"""

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib
from tests.common import KINDS, ordered_bits, to_kind

pytestmark = pytest.mark.gpu

HOST = {lib.F32: np.float32, lib.F16: np.float16, lib.BF16: np.uint16}
N, IG = oracle.NORMAL, oracle.INVERSE_GAUSSIAN
PDF, CDF, PPF = oracle.PDF, oracle.CDF, oracle.PPF
STATISTICS = [PDF, CDF, PPF]


def agree(kind, got, want):
    g, w = got.view(HOST[kind]), want.view(HOST[kind])
    nan_g = np.isnan(g.astype(np.float32)) if kind != lib.BF16 else (g & 0x7FFF) > 0x7F80
    nan_w = np.isnan(w.astype(np.float32)) if kind != lib.BF16 else (w & 0x7FFF) > 0x7F80
    assert np.array_equal(nan_g, nan_w)
    keep = ~nan_w
    distance = np.abs(ordered_bits(g[keep]) - ordered_bits(w[keep]))
    assert distance.max(initial=0) <= 1
    assert np.count_nonzero(distance) <= max(2, distance.size // 2000)


def inputs(kind, family, statistic, n, seed):
    rng = np.random.default_rng(seed)
    if statistic == PPF:
        x = rng.uniform(0, 1, n).astype(np.float32)
        specials = [0.0, 1.0, -0.5, 1.5, 1e-30, 1 - 2 ** -24, np.nan, 0.5]
    elif family == N:
        x = rng.uniform(-9, 9, n).astype(np.float32)
        specials = [0.0, -0.0, np.inf, -np.inf, np.nan, 40.0, -40.0, 1e-30]
    else:
        x = rng.uniform(-1, 12, n).astype(np.float32)
        specials = [0.0, -1.0, np.inf, np.nan, 1e-30, 200.0, 0.5, 1e-3]
    x[: min(n, len(specials))] = specials[: min(n, len(specials))]
    return to_kind(x, kind)


def device_distribution(kind, family, statistic, x, first, second):
    a = lib.Buffer.of(x)
    out = lib.Buffer(x.nbytes)
    lib.call("tc_distribution", kind, family, statistic, a.ptr, out.ptr, x.size, first, second)
    return out.download(HOST[kind], x.size)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("family,first,second", [(N, 0.0, 1.0), (N, 2.0, 3.0), (IG, 2.0, 3.0), (IG, 1.0, 100.0)])
@pytest.mark.parametrize("statistic", STATISTICS)
def test_distribution_against_the_oracle(kind, family, first, second, statistic):
    n = 40_000 if family == IG and statistic == PPF else 300_000
    x = inputs(kind, family, statistic, n, 17 * kind + 5 * statistic + family)
    got = device_distribution(kind, family, statistic, x, first, second)
    agree(kind, got, oracle.distribution(kind, family, statistic, x, first, second))


@pytest.mark.parametrize("family", [N, IG])
def test_parameters_that_are_not_positive_give_nans(family):
    x = np.linspace(0.1, 0.9, 9).astype(np.float32)
    for first, second in [(1.0, 0.0), (1.0, -2.0), (1.0, float("nan"))] + ([(-1.0, 1.0)] if family == IG else []):
        for statistic in STATISTICS:
            got = device_distribution(lib.F32, family, statistic, x, first, second)
            assert np.all(np.isnan(got)), (first, second, statistic)


def test_reference_values_in_f32():
    # tests/statistics.rs:334-390, :393-408 through the kernel.
    x = np.array([-1.0, 0.0, 1.0], np.float32)
    p = device_distribution(lib.F32, N, CDF, x, 0.0, 1.0)
    assert p[1] == 0.5 and abs(p[0] - 0.1586552539314571) < 1e-8 and abs(p[2] - 0.8413447460685429) < 1e-8
    back = device_distribution(lib.F32, N, PPF, p, 0.0, 1.0)
    assert np.allclose(back, x, atol=1e-6)
    grid = np.arange(-40, 40, dtype=np.float32) / np.float32(10)
    cdf = device_distribution(lib.F32, N, CDF, grid, 0.0, 1.0)
    want = np.array([oracle.evaluate(N, CDF, float(v), 0.0, 1.0) for v in grid])
    assert np.all(np.abs(cdf - want) < 1e-7)
    wald = device_distribution(lib.F32, IG, CDF, np.array([1.0], np.float32), 1.0, 1e6)
    assert 0.0 <= wald[0] <= 1.0 and abs(wald[0] - 0.5) < 1e-3


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("family", [N, IG])
@pytest.mark.parametrize("rows,cols", [(1, 1), (16, 24), (300, 1031), (5000, 7)])
def test_axis_distribution_against_the_oracle(kind, axis, family, rows, cols):
    rng = np.random.default_rng(rows * cols + axis)
    extent = rows if axis == 0 else cols
    first = to_kind(rng.uniform(0.5, 3, extent).astype(np.float32), kind)
    second = to_kind(rng.uniform(0.5, 4, extent).astype(np.float32), kind)
    if extent > 3:
        second[2] = to_kind(np.array([0.0], np.float32), kind)[0]  # a degenerate slice is NaNs
    for statistic in STATISTICS:
        if statistic == PPF:
            m = to_kind(rng.uniform(0, 1, (rows, cols)).astype(np.float32), kind)
        else:
            m = to_kind(rng.uniform(-2, 8, (rows, cols)).astype(np.float32), kind)
        if family == IG and statistic == PPF and rows * cols > 100_000:
            m = m[: 100_000 // cols]
        r = m.shape[0]
        f = first[:r] if axis == 0 else first
        s = second[:r] if axis == 0 else second
        dm, df, ds = lib.Buffer.of(m), lib.Buffer.of(f), lib.Buffer.of(s)
        out = lib.Buffer(m.nbytes)
        lib.call("tc_axis_distribution", kind, family, statistic, dm.ptr, r, cols, axis, df.ptr, ds.ptr, out.ptr)
        got = out.download(HOST[kind], m.size).reshape(m.shape)
        agree(kind, got.reshape(-1), oracle.axis_distribution(kind, family, statistic, m, axis, f, s).reshape(-1))


def test_unknown_codes_are_errors():
    x = lib.Buffer.of(np.ones(4, np.float32))
    out = lib.Buffer(16)
    with pytest.raises(lib.HipError, match="no Family 2"):
        lib.call("tc_distribution", lib.F32, 2, 0, x.ptr, out.ptr, 4, 0.0, 1.0)
    with pytest.raises(lib.HipError, match="no Statistic 3"):
        lib.call("tc_distribution", lib.F32, 0, 3, x.ptr, out.ptr, 4, 0.0, 1.0)
    with pytest.raises(lib.HipError, match="no Axis 2"):
        lib.call("tc_axis_distribution", lib.F32, 0, 0, x.ptr, 2, 2, 2, x.ptr, x.ptr, out.ptr)
