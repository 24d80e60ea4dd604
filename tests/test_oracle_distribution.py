"""The oracle's distribution functions (`Kernels::vector_distribution`,
`matrix_axis_distribution`, kernels.rs:1046-1070; the Host's special
functions, statistics/special.rs) pinned on the reference's published values
and round trips (tests/statistics.rs:84-196, :334-408, :451-505) and on
scipy's independent implementations: erf/erfc against `scipy.special`, the
normal against `scipy.stats.norm`, the inverse Gaussian (mean mu, shape
lambda) against `scipy.stats.invgauss(mu / lambda, scale=lambda)`.  A wrong
digit in a coefficient table moves a value far beyond these tolerances."""

import math

import numpy as np
import pytest
from scipy import special, stats

from oracle import binding as oracle
from tensorcrate_amd import lib
from tests.common import KINDS, to_kind, widen

N, IG = oracle.NORMAL, oracle.INVERSE_GAUSSIAN
PDF, CDF, PPF = oracle.PDF, oracle.CDF, oracle.PPF


def close(a, b, tolerance):
    # tests/statistics.rs:7-9.
    return abs(a - b) <= tolerance * max(abs(b), 1.0)


def relative(a, b):
    return abs(a - b) / abs(b) if b != 0 else abs(a)


def test_error_function_against_scipy():
    for x in np.linspace(-6, 6, 2401):
        assert close(oracle.load().or_erf(x), special.erf(x), 1e-15), x
    for x in np.linspace(-3, 26.5, 2951):
        assert relative(oracle.load().or_erfc(x), special.erfc(x)) <= 1e-13, x
    # tests/statistics.rs:75-79.
    assert oracle.load().or_erf(0.0) == 0.0 and oracle.load().or_erfc(0.0) == 1.0
    assert math.isnan(oracle.load().or_erf(math.nan))
    assert oracle.load().or_erfc(-30.0) == 2.0 and oracle.load().or_erfc(30.0) == 0.0


def test_normal_published_values():
    # tests/statistics.rs:84-118.
    for z, want in [(0.0, 0.5), (1.0, 0.8413447460685429), (-1.0, 0.1586552539314571),
                    (1.96, 0.9750021048517795), (-3.0, 0.001349898031630095)]:
        assert close(oracle.evaluate(N, CDF, z, 0.0, 1.0), want, 1e-14)
    for p, want in [(0.95, 1.6448536269514722), (0.975, 1.959963984540054), (0.99, 2.326347874040841), (0.5, 0.0)]:
        assert close(oracle.evaluate(N, PPF, p, 0.0, 1.0), want, 1e-14)
    assert oracle.evaluate(N, PPF, 0.0, 0.0, 1.0) == -math.inf
    assert oracle.evaluate(N, PPF, 1.0, 0.0, 1.0) == math.inf
    assert math.isnan(oracle.evaluate(N, PPF, 1.5, 0.0, 1.0))
    assert math.isnan(oracle.evaluate(N, PPF, -0.5, 0.0, 1.0))
    # tests/statistics.rs:375-389.
    assert oracle.evaluate(N, CDF, 10.0, 10.0, 2.0) == 0.5
    assert close(oracle.evaluate(N, CDF, 12.0, 10.0, 2.0), 0.8413447460685429, 1e-14)
    assert close(oracle.evaluate(N, PPF, 0.975, 10.0, 2.0), 10.0 + 2.0 * 1.959963984540054, 1e-13)
    assert math.isnan(oracle.evaluate(N, CDF, 1.0, 0.0, 0.0))
    assert close(oracle.evaluate(N, PDF, 0.0, 0.0, 1.0), 1 / math.sqrt(2 * math.pi), 1e-15)


def test_normal_quantile_inverts_the_distribution_function():
    # tests/statistics.rs:122-143.
    for i in range(1, 10_000, 7):
        p = i / 10_000
        assert close(oracle.evaluate(N, CDF, oracle.evaluate(N, PPF, p, 0, 1), 0, 1), p, 1e-13)
    for p in [1e-300, 1e-100, 1e-20, 1e-8, 1e-3]:
        assert close(oracle.evaluate(N, CDF, oracle.evaluate(N, PPF, p, 0, 1), 0, 1), p, 1e-12)
    erf_inv = oracle.load().or_normal_quantile(0.5 * (oracle.load().or_erf(0.75) + 1.0)) * math.sqrt(0.5)
    assert close(erf_inv, 0.75, 1e-14)


@pytest.mark.parametrize("mean,stddev", [(0.0, 1.0), (2.0, 3.0), (-5.0, 0.25)])
def test_normal_against_scipy(mean, stddev):
    law = stats.norm(mean, stddev)
    for x in np.linspace(mean - 9 * stddev, mean + 9 * stddev, 301):
        assert relative(oracle.evaluate(N, PDF, x, mean, stddev), law.pdf(x)) <= 1e-13
        assert relative(oracle.evaluate(N, CDF, x, mean, stddev), law.cdf(x)) <= 1e-13
    for p in np.concatenate([np.linspace(0.001, 0.999, 333), [1e-10, 1e-30, 1 - 1e-12]]):
        assert close(oracle.evaluate(N, PPF, p, mean, stddev), law.ppf(p), 1e-13)


@pytest.mark.parametrize("mean,shape", [(1.0, 1.0), (1.0, 3.0), (2.0, 0.5), (0.5, 20.0), (1.0, 100.0)])
def test_inverse_gaussian_against_scipy_and_its_quantile(mean, shape):
    law = stats.invgauss(mean / shape, scale=shape)
    for x in np.linspace(0.01, 6 * mean, 200):
        assert relative(oracle.evaluate(IG, PDF, x, mean, shape), law.pdf(x)) <= 1e-12
        assert close(oracle.evaluate(IG, CDF, x, mean, shape), law.cdf(x), 1e-12)
    # tests/statistics.rs:147-180: the quantile inverts the distribution.
    for i in range(1, 500, 3):
        p = i / 500
        x = oracle.evaluate(IG, PPF, p, mean, shape)
        assert close(oracle.evaluate(IG, CDF, x, mean, shape), p, 1e-12)
        assert close(x, law.ppf(p), 1e-9)


def test_inverse_gaussian_edges():
    # tests/statistics.rs:182-192.
    assert oracle.evaluate(IG, CDF, 0.0, 1.0, 1.0) == 0.0
    assert oracle.evaluate(IG, PDF, -1.0, 1.0, 1.0) == 0.0
    assert oracle.evaluate(IG, PPF, 0.0, 1.0, 1.0) == 0.0
    assert oracle.evaluate(IG, PPF, 1.0, 1.0, 1.0) == math.inf
    assert math.isnan(oracle.evaluate(IG, CDF, 1.0, -1.0, 1.0))
    extreme = oracle.evaluate(IG, CDF, 1.0, 1.0, 1e6)
    assert 0.0 <= extreme <= 1.0 and close(extreme, 0.5, 1e-3)


def test_single_precision_keeps_full_single_precision_accuracy():
    # tests/statistics.rs:393-408.
    x = np.arange(-40, 40, dtype=np.float32) / np.float32(10)
    got = oracle.distribution(lib.F32, N, CDF, x, 0.0, 1.0)
    want = stats.norm.cdf(x.astype(np.float64))
    assert np.all(np.abs(got - want) < 1e-7)


@pytest.mark.parametrize("kind", KINDS)
def test_results_round_through_f32(kind):
    # The Host's `cast` (statistics/mod.rs:292-297) for f16/bf16 goes through
    # f32: the element result is the f64 value rounded to f32, then to the type.
    rng = np.random.default_rng(kind)
    x = to_kind(rng.uniform(-4, 4, 500).astype(np.float32), kind)
    got = oracle.distribution(kind, N, CDF, x, 0.5, 1.5)
    wide = widen(kind, x).astype(np.float64)
    want = to_kind(np.array([oracle.evaluate(N, CDF, v, 0.5, 1.5) for v in wide], np.float32), kind)
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))


def test_axis_distributions_use_one_pair_per_row_or_column():
    # tests/statistics.rs:451-505 in f32: rows on scales 1 and 1000 land on
    # the same probabilities; columns mirror; the quantile takes them back.
    m = np.array([[1, 2, 3, 4, 5], [1000, 2000, 3000, 4000, 5000]], np.float32)
    means = m.mean(axis=1).astype(np.float32)
    stds = m.std(axis=1).astype(np.float32)
    p = oracle.axis_distribution(lib.F32, N, CDF, m, 0, means, stds)
    assert close(p[0, 2], 0.5, 1e-7) and close(p[1, 2], 0.5, 1e-7)
    assert np.allclose(p[0], p[1], rtol=0, atol=2e-7)
    back = oracle.axis_distribution(lib.F32, N, PPF, p, 0, means, stds)
    assert np.allclose(back, m, rtol=2e-6)
    col_means = m.mean(axis=0).astype(np.float32)
    col_stds = m.std(axis=0).astype(np.float32)
    assert col_means[0] == 500.5
    by_column = oracle.axis_distribution(lib.F32, N, CDF, m, 1, col_means, col_stds)
    assert np.allclose(by_column[0], 1 - by_column[1], atol=2e-7)
    for r in range(2):
        want = oracle.distribution(lib.F32, N, CDF, m[r], float(means[r]), float(stds[r]))
        assert np.array_equal(p[r], want)
