"""Strided copies on the GPU against the oracle, bit for bit
(Backend::strided_copy / assemble / strided_write, backend.rs:141-323;
tests/nd_tensor.rs:113-292 and metal/tests.rs:327-412 are the reference's
versions of these checks)."""

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib
from tensorcrate_amd.tensor import Tensor
from tests.common import bits_equal, filler

pytestmark = pytest.mark.gpu


def test_permute_matches_the_reference_known_answer():
    # metal/tests.rs:327-412: [2, 3, 4] permuted to [4, 2, 3] reads strides [1, 12, 4].
    x = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    view = Tensor.from_numpy(x).permute([2, 0, 1])
    assert view.strides == (1, 12, 4)
    assert bits_equal(view.contiguous().to_numpy(), oracle.strided_copy(x.reshape(-1), [4, 2, 3], 0, [1, 12, 4]))


@pytest.mark.parametrize("axes", [[0, 2, 1], [2, 1, 0], [1, 0, 2], [2, 0, 1]])
@pytest.mark.parametrize("shape", [(5, 67, 70), (3, 68, 132), (2, 64, 256)])
def test_permutes_of_every_width(axes, shape):
    # Every element width moves by its bits (tests/nd_tensor.rs:712-744);
    # extents that are multiples of four take the 16-byte tile path for
    # 4-byte elements, with partial tiles at the edges.
    for kind, dtype in [("u8", np.uint8), ("u16", np.uint16), ("f32", np.float32), ("u64", np.uint64)]:
        x = (np.arange(np.prod(shape)) % 251).astype(dtype).reshape(shape)
        buffer = lib.Buffer.of(x)
        strides = [s // x.itemsize for s in x.strides]
        out_shape = [shape[a] for a in axes]
        out = lib.Buffer(x.nbytes)
        lib.call("tc_strided_copy", x.itemsize, buffer.ptr, x.size, 3, lib.dims(out_shape),
                 lib.ctypes.byref(lib.strided(0, [strides[a] for a in axes])), out.ptr)
        got = out.download(dtype, x.size).reshape(out_shape)
        want = oracle.strided_copy(x.reshape(-1), out_shape, 0, [strides[a] for a in axes])
        assert bits_equal(got, want), kind


def test_sixteen_byte_elements():
    x = np.arange(2 * 3 * 8 * 2, dtype=np.uint64).reshape(2, 3, 8, 2)  # 16-byte elements: pairs
    buffer = lib.Buffer.of(x)
    out = lib.Buffer(x.nbytes)
    lib.call("tc_strided_copy", 16, buffer.ptr, 2 * 3 * 8, 3, lib.dims([8, 2, 3]),
             lib.ctypes.byref(lib.strided(0, [1, 24, 8])), out.ptr)
    got = out.download(np.uint64).reshape(8, 2, 3, 2)
    assert np.array_equal(got, x.transpose(2, 0, 1, 3))


def test_views_slices_and_broadcasts():
    x = filler([3, 4, 5, 6])
    t = Tensor.from_numpy(x)
    cases = [
        t.narrow(3, 1, 4).transpose(0, 2),
        t.select(1, 2).slice(2, 1, 5),
        t.permute([3, 1, 0, 2]),
        t.slice(0, 1, 3).broadcast_to([7, 2, 4, 5, 6]),
        t.select(3, 5).unsqueeze(0).broadcast_to([4, 3, 4, 5]),
    ]
    for view in cases:
        got = view.contiguous().to_numpy()
        want = oracle.strided_copy(x.reshape(-1), list(view.shape), view.offset, list(view.strides))
        assert bits_equal(got, want), view.shape


def test_concat_stack_and_write_slice():
    # tensor.rs:392-399 and :495-500 known answers, then the config-3 shapes.
    a = Tensor.from_numpy(np.array([[1.0], [2.0]], np.float32))
    b = Tensor.from_numpy(np.array([[3.0, 4.0], [5.0, 6.0]], np.float32))
    assert Tensor.concat([a, b], 1).to_numpy().tolist() == [[1, 3, 4], [2, 5, 6]]
    cache = Tensor.filled([2, 4], 0.0)
    cache.write_slice(1, 2, Tensor.from_numpy(np.array([[7.0], [8.0]], np.float32)))
    assert cache.to_numpy().reshape(-1).tolist() == [0, 0, 7, 0, 0, 0, 8, 0]
    x = filler([4, 6, 5])
    t = Tensor.from_numpy(x)
    stacked = Tensor.stack([t.select(1, 0), t.select(1, 3), t.select(1, 5)], 1).to_numpy()
    assert bits_equal(stacked, x[:, [0, 3, 5], :])
    halves = t.chunk(1, 2)
    assert bits_equal(Tensor.concat([halves[1], halves[0]], 1).to_numpy(), np.concatenate([x[:, 3:], x[:, :3]], 1))


def test_config3_permute_slice_concat_at_full_size():
    # x [256, 512, 512]: permute(0, 2, 1) materialised, slice [:, 128:384, :],
    # concat of the two halves on axis 1.  Checked through exact index
    # identities on sampled coordinates and a checksum against numpy.
    rng = np.random.default_rng(2)
    x = rng.standard_normal((256, 512, 512), dtype=np.float32)
    t = Tensor.from_numpy(x)
    p = t.permute([0, 2, 1]).contiguous()
    got = p.to_numpy()
    assert np.array_equal(got, x.transpose(0, 2, 1))
    s = p.slice(1, 128, 384).contiguous().to_numpy()
    assert np.array_equal(s, got[:, 128:384, :])
    halves = p.chunk(1, 2)
    c = Tensor.concat(halves, 1).to_numpy()
    assert np.array_equal(c, got)


def test_transpose_of_every_width():
    for dtype in [np.uint16, np.float32, np.uint64]:
        for rows, cols in [(1, 1), (3, 5), (64, 64), (130, 257), (1000, 3)]:
            x = (np.arange(rows * cols) % 65521).astype(dtype).reshape(rows, cols)
            src, dst = lib.Buffer.of(x), lib.Buffer(x.nbytes)
            lib.call("tc_transpose", x.itemsize, rows, cols, src.ptr, dst.ptr)
            assert bits_equal(dst.download(dtype, x.size).reshape(cols, rows), oracle.transpose(x))


def test_a_transpose_past_the_infinity_cache():
    # 8192 x 8192 f32 moves 512 MiB: the tiled kernel streams its loads and
    # stores plainly; the bits are numpy's transpose.
    x = np.random.default_rng(8).standard_normal((8192, 8192), dtype=np.float32)
    src, dst = lib.Buffer.of(x), lib.Buffer(x.nbytes)
    lib.call("tc_transpose", 4, 8192, 8192, src.ptr, dst.ptr)
    assert bits_equal(dst.download(np.float32, x.size).reshape(8192, 8192), x.T)


def test_a_layout_past_its_storage_is_refused():
    x = Tensor.from_numpy(np.zeros(10, np.float32))
    with pytest.raises(lib.HipError, match="reaches past 10 elements"):
        lib.call("tc_strided_copy", 4, x.storage.ptr, 10, 2, lib.dims([2, 3]),
                 lib.ctypes.byref(lib.strided(5, [3, 1])), x.storage.ptr)
