"""Whole-buffer and per-axis moments on the GPU (`tc_moments`,
`tc_axis_moments`; `Kernels::vector_moments`, `matrix_moments`,
`matrix_axis_moments`, kernels.rs:1035-1042) against the oracle: the mean
and the sum of squared deviations, within the accumulated-rounding bound of
folds taken in a different order; NaNs where there is nothing to fold."""

import math

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib
from tests.common import identity_place, to_kind, widen

pytestmark = pytest.mark.gpu

HOST = {lib.F32: np.float32, lib.F16: np.float16, lib.BF16: np.uint16}


def device_moments(kind, x):
    a = lib.Buffer.of(x) if x.size else lib.Buffer(16)
    out = lib.Buffer(8)
    lib.call("tc_moments", kind, a.ptr, x.size, out.ptr)
    mean, devs = out.download(np.float32, 2)
    return float(mean), float(devs)


@pytest.mark.parametrize("kind", [lib.F32, lib.F16, lib.BF16])
@pytest.mark.parametrize("n", [1, 7, 64, 1000, 1 << 20, 25_000_003])
def test_moments_against_the_oracle(kind, n):
    rng = np.random.default_rng(n)
    x = to_kind(rng.uniform(-3, 3, n) + 1.5, kind)
    got_mean, got_devs = device_moments(kind, x)
    want_mean, want_devs = oracle.moments(kind, x)
    wide = widen(kind, x).astype(np.float64)
    scale = np.abs(wide).mean()
    exact_mean = wide.mean()
    exact_devs = ((wide - exact_mean) ** 2).sum()
    # The device's tree of folds is held to the sqrt(n) bound against the
    # exact moments; the oracle's left-to-right fold, as the host's, only to
    # the n bound (it drifts by 1% over 25 M elements), so the two are
    # compared through the exact values rather than with each other.
    assert abs(got_mean - exact_mean) <= 8 * math.sqrt(n) * 2.0 ** -24 * scale + 1e-30
    assert abs(got_devs - exact_devs) <= 16 * math.sqrt(n) * 2.0 ** -24 * exact_devs + 1e-30
    assert abs(want_mean - exact_mean) <= n * 2.0 ** -24 * scale + 1e-30
    assert abs(want_devs - exact_devs) <= 2 * n * 2.0 ** -24 * exact_devs + 1e-30


def test_moments_of_nothing_are_nans_and_unaligned_starts_fold_every_element():
    mean, devs = device_moments(lib.F32, np.zeros(0, np.float32))
    assert math.isnan(mean) and math.isnan(devs)
    x = np.arange(1, 1027, dtype=np.float32)
    a = lib.Buffer.of(x)
    out = lib.Buffer(8)
    lib.call("tc_moments", lib.F32, a.ptr + 4, x.size - 1, out.ptr)
    mean, devs = out.download(np.float32, 2)
    want = x[1:].astype(np.float64)
    assert abs(mean - want.mean()) <= 1e-4 and abs(devs - ((want - want.mean()) ** 2).sum()) <= 1e-6 * devs


@pytest.mark.parametrize("kind", [lib.F32, lib.BF16])
@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 300), (300, 7), (1024, 1024), (64, 100000)])
@pytest.mark.parametrize("axis", [0, 1])
def test_axis_moments_against_the_oracle(kind, rows, cols, axis):
    rng = np.random.default_rng(rows + cols + axis)
    x = to_kind(rng.uniform(-2, 2, rows * cols), kind)
    size = 4 if kind == lib.F32 else 2
    n = rows if axis == 0 else cols
    a, means, devs = lib.Buffer.of(x), lib.Buffer(n * size), lib.Buffer(n * size)
    lib.call("tc_axis_moments", kind, a.ptr, rows, cols, axis, means.ptr, devs.ptr)
    place = identity_place(rows, cols) if axis == 0 else (0, cols, 1, [cols], [1])
    want_mean, want_devs = oracle.row_moments(kind, kind, x, place, n, cols if axis == 0 else rows)
    depth = cols if axis == 0 else rows
    unit = 2.0 ** -24 if kind == lib.F32 else 2.0 ** -8
    gm, wm = widen(kind, means.download(HOST[kind], n)), widen(kind, want_mean)
    gd, wd = widen(kind, devs.download(HOST[kind], n)), widen(kind, want_devs)
    root = math.sqrt(depth)
    assert np.all(np.abs(gm - wm) <= 8 * root * 2.0 ** -24 * 2 + 2 * unit * np.abs(wm))
    assert np.all(np.abs(gd - wd) <= 16 * root * 2.0 ** -24 * (wd + depth) + 2 * unit * wd)


def test_axis_moments_along_an_empty_axis_are_nans():
    a, means, devs = lib.Buffer(16), lib.Buffer(16), lib.Buffer(16)
    lib.call("tc_axis_moments", lib.F32, a.ptr, 3, 0, 0, means.ptr, devs.ptr)
    assert np.all(np.isnan(means.download(np.float32, 3))) and np.all(np.isnan(devs.download(np.float32, 3)))
