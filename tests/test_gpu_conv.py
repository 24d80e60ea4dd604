"""Correlation, its input gradient, padding and flipping on the GPU
(`tc_correlate`, `tc_correlate_input_gradient`, `tc_pad`, `tc_flip`;
kernels.rs:990-1029) against the oracle: bit for bit, since each output is
the host's own sequence of f32 multiplies and adds (f16 and bf16 widened and
rounded once), and padding and flipping move bits."""

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib
from tests.common import to_kind

pytestmark = pytest.mark.gpu

HOST = {lib.F32: np.float32, lib.F16: np.float16, lib.BF16: np.uint16}


def device_correlate(kind, x, k, flip):
    (rows, cols), (wr, wc) = x.shape, k.shape
    out_shape = (rows - wr + 1, cols - wc + 1)
    dx, dk, out = lib.Buffer.of(x), lib.Buffer.of(k), lib.Buffer(max(out_shape[0] * out_shape[1] * x.itemsize, 1))
    lib.call("tc_correlate", kind, dx.ptr, rows, cols, dk.ptr, wr, wc, int(flip), out.ptr)
    return out.download(HOST[kind], out_shape[0] * out_shape[1]).reshape(out_shape)


def test_known_answers():
    x = np.array([[1, 2, 3], [4, 5, 6], [7, 8, 9]], np.float32)
    taps = np.array([[1, 10], [100, 1000]], np.float32)
    assert device_correlate(lib.F32, x, taps, False).tolist() == [[5421.0, 6532.0], [8754.0, 9865.0]]
    assert device_correlate(lib.F32, x, taps, True).tolist() == [[1245.0, 2356.0], [4578.0, 5689.0]]


@pytest.mark.parametrize("kind", [lib.F32, lib.F16, lib.BF16])
@pytest.mark.parametrize("shape,window", [((17, 23), (4, 6)), ((256, 300), (5, 5)), ((1000, 1000), (3, 3)),
                                          ((64, 64), (64, 64)), ((9, 9), (1, 1)), ((40, 30), (1, 30))])
@pytest.mark.parametrize("flip", [False, True])
def test_correlation_is_the_hosts_bits(kind, shape, window, flip):
    rng = np.random.default_rng(shape[0] + window[1])
    x = to_kind(rng.uniform(-1, 1, shape), kind)
    k = to_kind(rng.uniform(-1, 1, window), kind)
    got = device_correlate(kind, x, k, flip)
    want = oracle.correlate(kind, x, k, flip)
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))


@pytest.mark.parametrize("kind", [lib.F32, lib.BF16])
@pytest.mark.parametrize("adjoint_shape,window", [((10, 11), (3, 5)), ((300, 200), (7, 4)), ((1, 1), (5, 5))])
@pytest.mark.parametrize("flip", [False, True])
def test_input_gradient_is_the_hosts_bits(kind, adjoint_shape, window, flip):
    rng = np.random.default_rng(adjoint_shape[1] + window[0])
    adj = to_kind(rng.uniform(-1, 1, adjoint_shape), kind)
    k = to_kind(rng.uniform(-1, 1, window), kind)
    (ar, ac), (wr, wc) = adj.shape, k.shape
    da, dk = lib.Buffer.of(adj), lib.Buffer.of(k)
    out = lib.Buffer((ar + wr - 1) * (ac + wc - 1) * adj.itemsize)
    lib.call("tc_correlate_input_gradient", kind, da.ptr, ar, ac, dk.ptr, wr, wc, int(flip), out.ptr)
    got = out.download(HOST[kind], (ar + wr - 1) * (ac + wc - 1))
    want = oracle.correlate_input_gradient(kind, adj, k, flip).reshape(-1)
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))


def test_a_window_larger_than_the_input_is_refused():
    x, k = lib.Buffer(64), lib.Buffer(64)
    with pytest.raises(lib.HipError, match="a 3×2 window does not fit in a 2×4 input"):
        lib.call("tc_correlate", lib.F32, x.ptr, 2, 4, k.ptr, 3, 2, 0, x.ptr)


@pytest.mark.parametrize("dtype", [np.uint8, np.uint16, np.float32, np.float64])
@pytest.mark.parametrize("shape,pads", [((2, 2), (1, 1)), ((2, 2), (0, 2)), ((333, 517), (3, 0)), ((1, 1), (0, 0))])
def test_pad_and_flip_move_bits(dtype, shape, pads):
    rng = np.random.default_rng(shape[1])
    x = rng.integers(0, 250, shape).astype(dtype)
    dx = lib.Buffer.of(x)
    rows, cols = shape
    out_shape = (rows + 2 * pads[0], cols + 2 * pads[1])
    out = lib.Buffer(out_shape[0] * out_shape[1] * x.itemsize)
    lib.call("tc_pad", x.itemsize, dx.ptr, rows, cols, pads[0], pads[1], out.ptr)
    assert np.array_equal(out.download(dtype, out_shape[0] * out_shape[1]).reshape(out_shape),
                          oracle.pad(x, pads[0], pads[1]))
    flipped = lib.Buffer(x.nbytes)
    lib.call("tc_flip", x.itemsize, dx.ptr, rows, cols, flipped.ptr)
    assert np.array_equal(flipped.download(dtype, x.size).reshape(shape), oracle.flip(x))
