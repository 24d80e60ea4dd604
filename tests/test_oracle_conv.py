"""The oracle's correlation, padding and flipping (`Kernels::correlate`,
`correlate_input_gradient`, `pad`, `flip`; kernels.rs:990-1029) pinned on the
reference's hand-worked answers (tests/conv.rs:48-130), against numpy in
f64, and the input gradient against the adjoint identity
<correlate(X, K), Ȳ> = <X, input_gradient(Ȳ, K)>."""

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib


def test_correlation_known_answers():
    x = np.array([[1, 2, 3], [4, 5, 6], [7, 8, 9]], np.float32)
    taps = np.array([[1, 10], [100, 1000]], np.float32)
    assert oracle.correlate(lib.F32, x, taps, False).tolist() == [[5421.0, 6532.0], [8754.0, 9865.0]]
    assert oracle.correlate(lib.F32, x, taps, True).tolist() == [[1245.0, 2356.0], [4578.0, 5689.0]]
    scale = np.array([[3.0]], np.float32)
    assert np.array_equal(oracle.correlate(lib.F32, x, scale, False), 3 * x)


def test_padding_and_flipping_known_answers():
    x = np.array([[1, 2], [3, 4]], np.float32)
    assert oracle.pad(x, 1, 1).tolist() == [[0, 0, 0, 0], [0, 1, 2, 0], [0, 3, 4, 0], [0, 0, 0, 0]]
    assert oracle.pad(x, 0, 2).tolist() == [[0, 0, 1, 2, 0, 0], [0, 0, 3, 4, 0, 0]]
    assert np.array_equal(oracle.pad(x, 0, 0), x)
    assert oracle.flip(x).tolist() == [[4, 3], [2, 1]]
    assert np.array_equal(oracle.flip(oracle.flip(x)), x)


@pytest.mark.parametrize("flip", [False, True])
def test_correlation_against_f64_and_the_flip_identity(flip):
    rng = np.random.default_rng(4)
    x = rng.uniform(-1, 1, (17, 23)).astype(np.float32)
    k = rng.uniform(-1, 1, (4, 6)).astype(np.float32)
    got = oracle.correlate(lib.F32, x, k, flip)
    kk = k[::-1, ::-1] if flip else k
    want = np.array([[(x[r:r + 4, c:c + 6].astype(np.float64) * kk).sum() for c in range(18)] for r in range(14)])
    assert np.allclose(got, want, atol=1e-5)
    # Convolution is correlation with the flipped window (tests/conv.rs:119-128).
    assert np.array_equal(oracle.correlate(lib.F32, x, k, True), oracle.correlate(lib.F32, x, oracle.flip(k), False))


@pytest.mark.parametrize("flip", [False, True])
def test_input_gradient_is_the_adjoint_of_correlation(flip):
    rng = np.random.default_rng(5)
    x = rng.uniform(-1, 1, (12, 15)).astype(np.float64)
    k = rng.uniform(-1, 1, (3, 5)).astype(np.float32)
    adj = rng.uniform(-1, 1, (10, 11)).astype(np.float32)
    y = oracle.correlate(lib.F32, x.astype(np.float32), k, flip).astype(np.float64)
    g = oracle.correlate_input_gradient(lib.F32, adj, k, flip).astype(np.float64)
    assert g.shape == x.shape
    assert abs((y * adj).sum() - (x * g).sum()) <= 1e-4 * np.abs(y * adj).sum()
