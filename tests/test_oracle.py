"""The oracle pinned against the reference's own known answers and against
brute force and closed forms (CPU only).

Every check here is chosen so a plausible slip in the restatement — a
dropped term, a wrong stride, a transposed operand, a wrong rounding rule —
fails it.  The reference's tests quoted are under arthurmburke/tensorcrate.
"""

import itertools

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib
from tests.common import Lcg, filler, same, to_kind, torch, widen


def walk(shape, offset, strides):
    """The storage positions a layout visits, in order: a strided copy of
    the identity (layout.rs:504-510)."""
    size = 64
    source = np.arange(size, dtype=np.uint32)
    return oracle.strided_copy(source, shape, offset, strides).reshape(-1).tolist()


# ---- layout (layout.rs:512-593) ------------------------------------------------

def test_a_contiguous_layout_walks_in_order():
    assert walk([2, 3, 4], 5, [12, 4, 1]) == list(range(5, 29))


def test_a_permuted_layout_walks_in_the_permuted_order():
    assert walk([3, 2], 0, [1, 3]) == [0, 3, 1, 4, 2, 5]
    assert walk([], 7, []) == [7]
    assert walk([3, 0, 2], 0, [0, 0, 0]) == []


def test_broadcast_strides_repeat():
    # A [3, 1] column read as [2, 3, 4] (layout.rs:569-570: strides [0, 1, 0]).
    got = walk([2, 3, 4], 0, [0, 1, 0])
    assert got == [r for _ in range(2) for r in range(3) for _ in range(4)]


# ---- element conversions (half 2.7.1) -----------------------------------------

SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 65504.0, 65519.99, 65520.0, 1e-8, 6e-8,
                     5.960464477539063e-08, 2.98e-08, 3.0e-08, 6.103515625e-05, 6.1035156e-05, 3.4e38, 1.17549435e-38,
                     1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -9, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -12], np.float32)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    values = np.concatenate([SPECIALS, rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
                             rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    got = oracle.bf16_from_f32(values)
    want = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    finite = ~np.isnan(values)
    assert np.array_equal(got[finite], want[finite])
    # NaNs stay NaNs, quieted, with their sign.
    nan_bits = got[~finite]
    assert np.all((nan_bits & 0x7F80) == 0x7F80) and np.all((nan_bits & 0x0040) != 0)


def test_f16_rounding_matches_numpy():
    rng = np.random.default_rng(1)
    values = np.concatenate([SPECIALS, (rng.standard_normal(50000) * 10.0 ** rng.uniform(-9, 6, 50000)).astype(np.float32)])
    got = oracle.f16_from_f32(values)
    want = values.astype(np.float16)
    finite = ~np.isnan(values)
    assert np.array_equal(got[finite].view(np.uint16), want[finite].view(np.uint16))
    back = oracle.widen(lib.F16, got.view(np.uint16))
    assert np.array_equal(back[finite], want[finite].astype(np.float32))


# ---- strided copies (backend.rs:255-323) --------------------------------------

def test_strided_copy_is_numpy_indexing():
    x = np.arange(3 * 4 * 5 * 6, dtype=np.float32).reshape(3, 4, 5, 6)
    flat = x.reshape(-1)
    s = [120, 30, 6, 1]
    # permute(2, 0, 3, 1)
    got = oracle.strided_copy(flat, [5, 3, 6, 4], 0, [s[2], s[0], s[3], s[1]])
    assert np.array_equal(got, x.transpose(2, 0, 3, 1))
    # narrow(3, 1, 4).transpose(0, 2)
    got = oracle.strided_copy(flat, [5, 4, 3, 4], 1, [6, 30, 120, 1])
    assert np.array_equal(got, x[:, :, :, 1:5].transpose(2, 1, 0, 3))
    # every element width moves by its bits
    for dtype in [np.uint8, np.uint16, np.uint32, np.uint64]:
        y = np.arange(24, dtype=dtype).reshape(2, 3, 4)
        assert np.array_equal(oracle.strided_copy(y.reshape(-1), [4, 2, 3], 0, [1, 12, 4]), y.transpose(2, 0, 1))


def test_strided_write_leaves_the_rest():
    target = np.zeros(8, np.float32)
    step = np.array([7.0, 8.0], np.float32)
    # tensor.rs:495-500: a [2, 1] step written at column 2 of a [2, 4] cache.
    oracle.strided_write(step, target, [2, 1], 0, [1, 1], 2, [4, 1])
    assert target.tolist() == [0, 0, 7, 0, 0, 0, 8, 0]


# ---- broadcast binary (strided.rs:29-78, kernels.rs:431-441) -------------------

def naive_broadcast(a, b, op):
    shape = np.broadcast_shapes(a.shape, b.shape)
    aa, bb = np.broadcast_to(a, shape), np.broadcast_to(b, shape)
    out = np.empty(shape, np.float32)
    for index in itertools.product(*[range(n) for n in shape]):
        out[index] = op(np.float32(aa[index]), np.float32(bb[index]))
    return out


ARITHMETIC = [(lib.ADD, lambda x, y: x + y), (lib.SUB, lambda x, y: x - y), (lib.MUL, lambda x, y: x * y),
              (lib.DIV, lambda x, y: x / y), (lib.REM, lambda x, y: np.fmod(x, y))]
COMPARE = [(lib.MIN, lambda x, y: np.fmin(x, y)), (lib.MAX, lambda x, y: np.fmax(x, y)),
           (lib.MAX_SHARE, lambda x, y: 1.0 if x > y else (0.0 if x < y else 0.5)),
           (lib.LESS, lambda x, y: float(x < y)), (lib.LESS_EQUAL, lambda x, y: float(x <= y)),
           (lib.GREATER, lambda x, y: float(x > y)), (lib.GREATER_EQUAL, lambda x, y: float(x >= y))]


def broadcast_layout(x, shape):
    strides = [0] * len(shape)
    added = len(shape) - x.ndim
    for axis in range(x.ndim):
        strides[added + axis] = 0 if x.shape[axis] == 1 else int(np.prod(x.shape[axis + 1:], dtype=np.int64))
    return strides


@pytest.mark.parametrize("a_shape,b_shape", [([2, 3, 4], [4]), ([4], [2, 3, 4]), ([2, 3, 1], [1, 4]), ([2, 3, 4], []),
                                             ([], [])])
def test_broadcast_matches_the_naive_reference(a_shape, b_shape):
    # tests/broadcast_reduce.rs:109-124, with `with_scalar(0.5, Add)` shifts.
    a = filler(a_shape)
    b = filler(b_shape) + np.float32(0.5) if b_shape else np.array(2.5, np.float32)
    if not a_shape:
        a = np.array(2.5, np.float32)
    shape = list(np.broadcast_shapes(a.shape, b.shape))
    for kind, cases in [(lib.ARITHMETIC, ARITHMETIC), (lib.COMPARE, COMPARE)]:
        for op, f in cases:
            got = oracle.binary(lib.F32, kind, op, shape, a, 0, broadcast_layout(a, shape), b, 0,
                                broadcast_layout(b, shape))
            assert same(got, naive_broadcast(a, b, f)), (kind, op)


def test_compact_elementwise_rounds_once():
    # A bf16 or f16 result is the f32 result rounded once (compact.rs:5-13):
    # check against torch's own bf16/f16 arithmetic.
    rng = np.random.default_rng(2)
    for kind, ttype in [(lib.BF16, torch.bfloat16), (lib.F16, torch.float16)]:
        a = to_kind(rng.standard_normal(4096).astype(np.float32) * 3, kind)
        b = to_kind(rng.standard_normal(4096).astype(np.float32) + 4, kind)
        ta = torch.from_numpy(widen(kind, a)).to(ttype)
        tb = torch.from_numpy(widen(kind, b)).to(ttype)
        for op, tf in [(lib.ADD, torch.add), (lib.SUB, torch.sub), (lib.MUL, torch.mul), (lib.DIV, torch.div)]:
            got = widen(kind, oracle.elementwise(kind, lib.ARITHMETIC, op, a, b))
            want = tf(ta, tb).float().numpy()
            assert np.array_equal(got, want), (kind, op)


# ---- reductions (strided.rs:80-225) -------------------------------------------

def naive_slices(x, axes):
    kept = [k for k in range(x.ndim) if k not in axes]
    moved = np.transpose(x, kept + list(axes))
    return moved.reshape(int(np.prod([x.shape[k] for k in kept], dtype=np.int64)), -1)


def test_reductions_over_every_subset_of_axes():
    # tests/broadcast_reduce.rs:385-399: the filler's sums are exact in f32.
    x = filler([2, 3, 4, 5])
    flat = x.reshape(-1)
    strides = [60, 20, 5, 1]
    for r in range(1, 5):
        for axes in itertools.combinations(range(4), r):
            slices = naive_slices(x, axes).astype(np.float64)
            kept = [x.shape[k] for k in range(4) if k not in axes]
            n = slices.shape[1]
            for kind, op, want in [(lib.FOLD, lib.SUM, slices.sum(1)), (lib.FOLD, lib.RMIN, slices.min(1)),
                                   (lib.FOLD, lib.RMAX, slices.max(1)), (lib.MEAN, 0, slices.sum(1) / n)]:
                got = oracle.reduce(lib.F32, flat, x.shape, 0, strides, list(axes), kind, op)
                assert np.allclose(got.reshape(-1), want, rtol=1e-6, atol=0), (axes, kind, op)
            for divisor in [n, n - 1]:
                got = oracle.reduce(lib.F32, flat, x.shape, 0, strides, list(axes), lib.VARIANCE, 0, divisor)
                want = ((slices - slices.mean(1, keepdims=True)) ** 2).sum(1) / divisor
                assert np.allclose(got.reshape(-1), want, rtol=1e-5, atol=1e-6), (axes, divisor)
            assert got.shape == tuple(kept)


def test_the_sum_folds_left_to_right_in_f32():
    # The host folds each slice in its own row-major order in an f32
    # accumulator (strided.rs:113-118): check the exact bits against that
    # definition on values whose sums do round.
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 50, 7)).astype(np.float32)
    got = oracle.reduce(lib.F32, x.reshape(-1), x.shape, 0, [350, 7, 1], [0, 2], lib.FOLD, lib.SUM)
    for j in range(50):
        total = np.float32(0)
        for i in range(3):
            for k in range(7):
                total = np.float32(total + x[i, j, k])
        assert got[j] == total


def test_extremes_pass_over_nans():
    # tests/broadcast_reduce.rs:505-519.
    nan = np.nan
    x = np.array([1.0, nan, 3.0, nan, nan, nan, -2.0, 5.0, nan], np.float32)
    r = lambda axes, op: oracle.reduce(lib.F32, x, [3, 3], 0, [3, 1], axes, lib.FOLD, op).tolist()
    assert r([1], lib.RMAX) == [3.0, -np.inf, 5.0]
    assert r([1], lib.RMIN) == [1.0, np.inf, -2.0]
    assert r([0], lib.RMAX) == [1.0, 5.0, 3.0]
    arg = lambda axis, op: oracle.arg_reduce(lib.F32, x, [3, 3], 0, [3, 1], axis, op).tolist()
    assert arg(1, lib.RMAX) == [2, 0, 1]
    assert arg(1, lib.RMIN) == [0, 0, 0]
    assert arg(0, lib.RMAX) == [0, 2, 0]
    assert np.isnan(r([1], lib.SUM)[0])


def test_ties_go_to_the_first_position():
    # tests/broadcast_reduce.rs:564-570.
    tied = np.array([1.0, 7.0, 7.0, 2.0, -3.0, -3.0, 0.0, -3.0], np.float32)
    assert oracle.arg_reduce(lib.F32, tied, [2, 4], 0, [4, 1], 1, lib.RMAX).tolist() == [1, 2]
    assert oracle.arg_reduce(lib.F32, tied, [2, 4], 0, [4, 1], 1, lib.RMIN).tolist() == [0, 0]


def test_arg_extremes_along_every_axis():
    # tests/broadcast_reduce.rs:521-562: brute force over every axis of a
    # permuted view, the filler giving many ties.
    x = filler([2, 3, 4, 5])
    view = x.transpose(3, 1, 0, 2)
    strides = [1, 20, 60, 5]
    for axis in range(4):
        slices = naive_slices(view, [axis])
        for op, pick in [(lib.RMAX, np.argmax), (lib.RMIN, np.argmin)]:
            got = oracle.arg_reduce(lib.F32, x.reshape(-1), view.shape, 0, strides, axis, op)
            assert got.reshape(-1).tolist() == [int(pick(s)) for s in slices]


def test_compact_sums_accumulate_in_f32():
    # tests/broadcast_reduce.rs:494-503.
    ones = to_kind(np.ones(2 * 10000, np.float32), lib.F16)
    got = oracle.reduce(lib.F16, ones, [2, 10000], 0, [10000, 1], [1], lib.FOLD, lib.SUM)
    assert widen(lib.F16, got).tolist() == [10000.0, 10000.0]
    ones = to_kind(np.ones(3000, np.float32), lib.BF16)
    got = oracle.reduce(lib.BF16, ones, [3, 1000], 0, [1000, 1], [1], lib.MEAN)
    assert widen(lib.BF16, got).tolist() == [1.0, 1.0, 1.0]


def test_variance_closed_form():
    # The population variance of 0..n-1 is (n^2 - 1) / 12 (metal/tests.rs:879-957
    # checks 143/12 for n = 12).
    x = np.arange(12, dtype=np.float32)
    got = oracle.reduce(lib.F32, x, [12], 0, [1], [0], lib.VARIANCE, 0, 12)
    assert got.reshape(-1).tolist() == [np.float32(143.0 / 12.0)]


# ---- products (matrix.rs:580-745) ----------------------------------------------

def test_matmul_matches_triple_loop():
    # tests/simd.rs:89-119, within 1e-4.
    m, k, n = 5, 6, 7
    a = (np.arange(m * k) * 0.1).astype(np.float32)
    b = (np.arange(k * n) * 0.2 - 1.0).astype(np.float32)
    addend = (np.arange(m * n) * -0.3 + 2.0).astype(np.float32)
    want = a.reshape(m, k).astype(np.float64) @ b.reshape(k, n).astype(np.float64)
    assert np.allclose(oracle.matmul(lib.F32, a, b, m, k, n), want, atol=1e-4)
    assert np.allclose(oracle.matmul(lib.F32, a, b, m, k, n, addend=addend), want + addend.reshape(m, n), atol=1e-4)


def relative_error(got, a, b, want):
    """|c - c_ref| / sum_k |a_ik b_kj|: the per-element error scale of a sum
    of products, which cancellation cannot shrink."""
    scale = np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))
    return np.max(np.abs(got.astype(np.float64) - want) / np.maximum(scale, 1e-30))


@pytest.mark.parametrize("m,k,n", [(96, 96, 96), (33, 70, 65), (1, 300, 40)])
def test_f32_matmul_is_within_f32_tolerance_of_f64(m, k, n):
    rng = np.random.default_rng(4)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    want = a.astype(np.float64) @ b.astype(np.float64)
    assert relative_error(oracle.matmul(lib.F32, a, b, m, k, n), a, b, want) <= 1e-5 * np.sqrt(k)


def test_the_f32_product_is_the_fma_chain():
    # matmul_avx (simd_x86.rs:1302-1327): each output is
    # fma(a_ip, b_pj, acc) over p in order for the 8-lane columns, and
    # acc + a_ip * b_pj on the tail.  torch's CPU float64 -> float32 of an
    # exact product plus a float32 accumulator is that single rounding when
    # the sum's exponent range is narrow, which holds for these inputs.
    rng = np.random.default_rng(5)
    m, k, n = 4, 40, 11
    a = (rng.integers(-64, 64, (m, k)) / 8).astype(np.float32)
    b = (rng.integers(-64, 64, (k, n)) / 8).astype(np.float32)
    got = oracle.matmul(lib.F32, a, b, m, k, n)
    want = np.zeros((m, n), np.float32)
    for p in range(k):
        want = (want.astype(np.float64) + a[:, p:p + 1].astype(np.float64) * b[p].astype(np.float64)).astype(np.float32)
    assert np.array_equal(got, want)


def test_compact_matmul_widens_and_rounds_once():
    # compact.rs:232-253: bf16 operands, the f32 product, one rounding.
    rng = np.random.default_rng(6)
    m, k, n = 16, 64, 24
    a = to_kind(rng.standard_normal((m, k)), lib.BF16)
    b = to_kind(rng.standard_normal((k, n)), lib.BF16)
    f32_product = oracle.matmul(lib.F32, widen(lib.BF16, a), widen(lib.BF16, b), m, k, n)
    assert np.array_equal(oracle.matmul(lib.BF16, a, b, m, k, n), to_kind(f32_product, lib.BF16))
    assert np.array_equal(oracle.matmul(lib.BF16, a, b, m, k, n, out_dtype=lib.F32), f32_product)


def test_matvec_vecmat_and_dot():
    rng = np.random.default_rng(7)
    m = rng.uniform(-1, 1, (37, 53)).astype(np.float32)
    v = rng.uniform(-1, 1, 53).astype(np.float32)
    w = rng.uniform(-1, 1, 37).astype(np.float32)
    assert np.allclose(oracle.matvec(lib.F32, m, v), m.astype(np.float64) @ v, atol=1e-5)
    assert np.allclose(oracle.matvec(lib.F32, m, v, addend=w), m.astype(np.float64) @ v + w, atol=1e-5)
    assert np.allclose(oracle.vecmat(lib.F32, w, m), w.astype(np.float64) @ m, atol=1e-5)
    # Below 16 elements the dot is the plain left-to-right loop (vector.rs:478-482).
    x, y = v[:15], v[15:30]
    total = np.float32(0)
    for p, q in zip(x, y):
        total = np.float32(total + np.float32(p * q))
    assert oracle.dot(lib.F32, x, y) == total
    assert np.isclose(oracle.dot(lib.F32, v, v), np.dot(v.astype(np.float64), v), rtol=1e-6)


def test_transpose():
    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    assert np.array_equal(oracle.transpose(x), x.T)


# ---- fused programs (fused/mod.rs:19-38) -------------------------------------

def test_fused_interpreter_known_answer():
    # fused/mod.rs:23-37: y = sqrt(a * w + 1) over [3, 0] and [1, 5] is [2, 1].
    code = [(0, 0, 0, 0, lib.F32, 0, 0.0), (0, 1, 1, 1, lib.F32, 0, 0.0), (2, lib.MUL, 2, 0, 1, 0, 0.0),
            (1, 0, 3, 0, 0, 0, 1.0), (2, lib.ADD, 4, 2, 3, 0, 0.0), (3, 13, 5, 4, 0, 0, 0.0),
            (5, 0, 0, 5, lib.F32, 0, 0.0)]
    identity = (0, 1, 1, [1], [2])
    a = np.array([3.0, 0.0], np.float32)
    w = np.array([1.0, 5.0], np.float32)
    y = np.zeros(2, np.float32)
    oracle.fused(lib.F32, code, [identity, identity], [a, w], [y], 1, 2)
    assert y.tolist() == [2.0, 1.0]
