"""Matrix products on the GPU's matrix cores against the oracle and f64
(Kernels::matmul / matmul_add / matmul_transposed_add / matvec / vecmat,
kernels.rs:897-987; tests/backend.rs:221-334 and tests/simd.rs:89-119 are the
reference's versions).

Tolerances (per element, relative to sum_k |a_ik b_kj|, which cancellation
cannot shrink): f32 1e-5 sqrt(K); f16 and bf16 inputs, compared with the f64
product of the same rounded inputs, 2^-7 sqrt(K) for a 16-bit output and
1e-5 sqrt(K) for the f32 (`matmul_f32`) output.
"""

import numpy as np
import pytest

from oracle import binding as oracle
from tensorcrate_amd import lib
from tests.common import to_kind, widen

pytestmark = pytest.mark.gpu

HOST = {lib.F32: np.float32, lib.F16: np.float16, lib.BF16: np.uint16}


def error(got, a, b, want):
    scale = np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))
    return np.max(np.abs(got.astype(np.float64) - want) / np.maximum(scale, 1e-30))


def product(in_kind, out_kind, transposed, a, b, m, k, n, addend=None):
    da, db = lib.Buffer.of(a), lib.Buffer.of(b)
    size = 4 if out_kind == lib.F32 else 2
    dc = lib.Buffer.of(addend) if addend is not None else lib.Buffer(m * n * size)
    lib.call("tc_matmul", in_kind, out_kind, transposed, int(addend is not None), m, k, n, da.ptr, db.ptr, dc.ptr)
    return dc.download(HOST[out_kind], m * n).reshape(m, n)


def tolerance(in_kind, out_kind, k):
    return (1e-5 if out_kind == lib.F32 else 2.0 ** -7) * np.sqrt(max(k, 1))


SHAPES = [(1, 1, 1), (5, 6, 7), (96, 96, 96), (33, 70, 65), (256, 128, 64), (300, 257, 129), (17, 1000, 3),
          (512, 512, 512)]


@pytest.mark.parametrize("in_kind,out_kind", [(lib.F32, lib.F32), (lib.BF16, lib.BF16), (lib.BF16, lib.F32),
                                              (lib.F16, lib.F16), (lib.F16, lib.F32)])
@pytest.mark.parametrize("m,k,n", SHAPES)
def test_matmul_against_the_oracle(in_kind, out_kind, m, k, n):
    rng = np.random.default_rng(m * 10000 + k * 100 + n)
    a = to_kind(rng.uniform(-1, 1, (m, k)), in_kind)
    b = to_kind(rng.uniform(-1, 1, (k, n)), in_kind)
    wa, wb = widen(in_kind, a), widen(in_kind, b)
    exact = wa.astype(np.float64) @ wb.astype(np.float64)
    tol = tolerance(in_kind, out_kind, k)
    got = widen(out_kind, product(in_kind, out_kind, lib.PLAIN, a, b, m, k, n))
    assert error(got, wa, wb, exact) <= tol
    want = widen(out_kind, oracle.matmul(in_kind, a, b, m, k, n, out_dtype=out_kind))
    assert error(got, wa, wb, want) <= 2 * tol


@pytest.mark.parametrize("kind", [lib.F32, lib.BF16])
@pytest.mark.parametrize("m,k,n", [(64, 48, 80), (130, 257, 33), (4, 4, 4), (96, 64, 131), (300, 128, 258)])
def test_transposed_products_accumulate(kind, m, k, n):
    # C + A^T B (A stored k x m) and C + A B^T (B stored n x k): the matmul
    # backward's two products (tape/mod.rs:1199-1214).
    rng = np.random.default_rng(k)
    at = to_kind(rng.uniform(-1, 1, (k, m)), kind)
    b = to_kind(rng.uniform(-1, 1, (k, n)), kind)
    bt = to_kind(rng.uniform(-1, 1, (n, k)), kind)
    a = to_kind(rng.uniform(-1, 1, (m, k)), kind)
    c = to_kind(rng.uniform(-1, 1, (m, n)), kind)
    tol = tolerance(kind, kind, k) + (2.0 ** -8 if kind == lib.BF16 else 0)
    got = widen(kind, product(kind, kind, lib.LEFT, at, b, m, k, n, addend=c))
    want = widen(kind, c) + widen(kind, at).T.astype(np.float64) @ widen(kind, b)
    assert error(got, widen(kind, at).T, widen(kind, b), want) <= tol * 2
    got = widen(kind, product(kind, kind, lib.RIGHT, a, bt, m, k, n, addend=c))
    want = widen(kind, c) + widen(kind, a).astype(np.float64) @ widen(kind, bt).T
    assert error(got, widen(kind, a), widen(kind, bt).T, want) <= tol * 2
    got = widen(kind, product(kind, kind, lib.PLAIN, a, b, m, k, n, addend=c))
    want = oracle.matmul(kind, a, b, m, k, n, addend=c)
    assert error(got, widen(kind, a), widen(kind, b), widen(kind, want)) <= tol * 2


@pytest.mark.parametrize("kind", [lib.F32, lib.BF16])
@pytest.mark.parametrize("m,k,n", [(300, 1, 1024), (257, 1, 33), (64, 3, 130), (129, 7, 64)])
def test_short_inner_dimensions(kind, m, k, n):
    # K below 8 takes the write-bound kernel (K = 1 is the tape's bias
    # broadcast, `outer`, tape/mod.rs:1000-1006), in every form and with an
    # addend.  An outer product is each a_i b_j rounded once, as the host
    # forms it: bit-exact.
    rng = np.random.default_rng(m + k + n)
    a = to_kind(rng.uniform(-1, 1, (m, k)), kind)
    b = to_kind(rng.uniform(-1, 1, (k, n)), kind)
    c = to_kind(rng.uniform(-1, 1, (m, n)), kind)
    wa, wb = widen(kind, a), widen(kind, b)
    tol = tolerance(kind, kind, k) + (2.0 ** -8 if kind == lib.BF16 else 0)
    exact = wa.astype(np.float64) @ wb.astype(np.float64)
    forms = [(lib.PLAIN, a, b), (lib.LEFT, np.ascontiguousarray(a.T), b), (lib.RIGHT, a, np.ascontiguousarray(b.T))]
    for form, x, y in forms:
        got = widen(kind, product(kind, kind, form, x, y, m, k, n))
        if k == 1:
            want = to_kind(wa.astype(np.float32) * wb.astype(np.float32), kind)
            assert np.array_equal(got, widen(kind, want)), form
        assert error(got, wa, wb, exact) <= tol, form
        got = widen(kind, product(kind, kind, form, x, y, m, k, n, addend=c))
        wc = widen(kind, c).astype(np.float64)
        scale = np.abs(wa.astype(np.float64)) @ np.abs(wb.astype(np.float64)) + np.abs(wc)
        assert np.max(np.abs(got - (exact + wc)) / scale) <= tol * 2, form


def test_an_empty_inner_dimension_gives_zeros_or_the_addend():
    # ops.rs:163-168, tests/backend.rs:259-266.
    a = np.zeros((3, 0), np.float32)
    b = np.zeros((0, 4), np.float32)
    assert np.array_equal(product(lib.F32, lib.F32, lib.PLAIN, a, b, 3, 0, 4), np.zeros((3, 4)))
    c = np.arange(12, dtype=np.float32).reshape(3, 4)
    assert np.array_equal(product(lib.F32, lib.F32, lib.PLAIN, a, b, 3, 0, 4, addend=c), c)


def check_matvec_vecmat(kind, rows, cols, rng):
    """matvec, matvec with an addend and vecmat of one matrix against f64."""
    m = to_kind(rng.uniform(-1, 1, (rows, cols)).astype(np.float32), kind)
    v = to_kind(rng.uniform(-1, 1, cols), kind)
    w = to_kind(rng.uniform(-1, 1, rows), kind)
    dm, dv, dw = lib.Buffer.of(m), lib.Buffer.of(v), lib.Buffer.of(w)
    out = lib.Buffer(rows * 4)
    lib.call("tc_matvec", kind, 0, rows, cols, dm.ptr, dv.ptr, out.ptr)
    got = widen(kind, out.download(HOST[kind], rows))
    wm, wv, ww = widen(kind, m), widen(kind, v), widen(kind, w)
    want = wm.astype(np.float64) @ wv
    scale = np.abs(wm).astype(np.float64) @ np.abs(wv)
    unit = 2.0 ** -24 if kind == lib.F32 else (2.0 ** -11 if kind == lib.F16 else 2.0 ** -8)
    assert np.all(np.abs(got - want) <= 1e-5 * np.sqrt(cols) * scale + unit * np.abs(want) + 1e-30)
    lib.call("tc_matvec", kind, 1, rows, cols, dm.ptr, dv.ptr, dw.ptr)
    got = widen(kind, dw.download(HOST[kind], rows))
    assert np.all(np.abs(got - (want + ww)) <= 1e-5 * np.sqrt(cols) * scale + unit * (np.abs(want) + 1) + 1e-30)
    out = lib.Buffer(cols * 4)
    lib.call("tc_vecmat", kind, rows, cols, dw.ptr, dm.ptr, out.ptr)
    got = widen(kind, out.download(HOST[kind], cols))
    w2 = widen(kind, dw.download(HOST[kind], rows))
    want = w2.astype(np.float64) @ wm
    scale = np.abs(w2).astype(np.float64) @ np.abs(wm)
    assert np.all(np.abs(got - want) <= 1e-5 * np.sqrt(rows) * scale + unit * np.abs(want) + 1e-30)


def test_matvec_vecmat():
    rng = np.random.default_rng(13)
    for kind in [lib.F32, lib.BF16, lib.F16]:
        for rows, cols in [(1, 1), (37, 53), (1000, 64), (8, 8192), (513, 1031), (300, 5000), (64, 8200), (2000, 4096)]:
            check_matvec_vecmat(kind, rows, cols, rng)


@pytest.mark.parametrize("kind,rows,cols", [(lib.F32, 8192, 8192), (lib.F32, 8191, 8196), (lib.BF16, 8192, 16384),
                                            (lib.F16, 16390, 8196)])
def test_matvec_vecmat_of_matrices_as_large_as_the_infinity_cache(kind, rows, cols):
    # Matrices of 256 MiB and more are read with non-temporal loads, and
    # vecmat takes two packs a lane there: whole and ragged column tiles,
    # ragged row splits.
    check_matvec_vecmat(kind, rows, cols, np.random.default_rng(rows + cols))


def test_config1_f32_512_cubed():
    # f32 C = A @ B, A and B 512 x 512 U(-1, 1), seed 0, against the oracle.
    rng = np.random.default_rng(0)
    a = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    b = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    got = product(lib.F32, lib.F32, lib.PLAIN, a, b, 512, 512, 512)
    want = oracle.matmul(lib.F32, a, b, 512, 512, 512)
    assert error(got, a, b, want) <= 1e-5 * np.sqrt(512)
    assert error(got, a, b, a.astype(np.float64) @ b) <= 1e-5 * np.sqrt(512)


@pytest.mark.parametrize("in_kind,m,k,n", [(lib.BF16, 8192, 8192, 8192), (lib.F32, 4096, 4096, 4096),
                                           (lib.F16, 16384, 4096, 1024), (lib.F16, 16384, 1024, 4096)])
def test_config4_sweep_on_sampled_entries(in_kind, m, k, n):
    # The dense sweep at full size, seed 3: bf16 A, B ~ N(0, 1/sqrt(K)) (the
    # second parameter read as the standard deviation), f32 U(-1, 1), f16
    # N(0, 1/sqrt(K)); 64 sampled rows against the f64 product.  The f16
    # "skinny" product is checked both ways round: K = 4096 with N = 1024,
    # and K = 1024 with N = 4096, the orientation bench.py times.
    rng = np.random.default_rng(3)
    if in_kind == lib.F32:
        a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
        b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    else:
        sigma = 1 / np.sqrt(k)
        a = to_kind((rng.standard_normal((m, k), dtype=np.float32) * sigma), in_kind)
        b = to_kind((rng.standard_normal((k, n), dtype=np.float32) * sigma), in_kind)
    got = product(in_kind, in_kind, lib.PLAIN, a, b, m, k, n)
    rows = np.sort(rng.choice(m, 64, replace=False))
    wa, wb = widen(in_kind, a[rows]), widen(in_kind, b)
    want = wa.astype(np.float64) @ wb.astype(np.float64)
    assert error(widen(in_kind, got[rows]), wa, wb, want) <= tolerance(in_kind, in_kind, k)


def sampled_form(kind, form, m, k, n, rng, addend):
    """A product in `form` on the GPU, and its f64 value on 48 sampled rows."""
    a = to_kind(rng.standard_normal((m, k), dtype=np.float32) / np.float32(np.sqrt(k)), kind)
    b = to_kind(rng.standard_normal((k, n), dtype=np.float32) / np.float32(np.sqrt(k)), kind)
    c = to_kind(rng.uniform(-1, 1, (m, n)), kind) if addend else None
    x = np.ascontiguousarray(a.T) if form == lib.LEFT else a
    y = np.ascontiguousarray(b.T) if form == lib.RIGHT else b
    got = product(kind, kind, form, x, y, m, k, n, addend=c)
    rows = np.sort(rng.choice(m, 48, replace=False))
    rows = np.unique(np.concatenate([rows, [0, m - 1]]))
    wa, wb = widen(kind, a[rows]).astype(np.float64), widen(kind, b).astype(np.float64)
    want = wa @ wb
    scale = np.abs(wa) @ np.abs(wb)
    if addend:
        wc = widen(kind, c[rows]).astype(np.float64)
        want, scale = want + wc, scale + np.abs(wc)
    return widen(kind, got[rows]).astype(np.float64), want, scale


@pytest.mark.parametrize("kind", [lib.BF16, lib.F16], ids=["bf16", "f16"])
@pytest.mark.parametrize("form", [lib.PLAIN, lib.LEFT, lib.RIGHT], ids=["plain", "left", "right"])
@pytest.mark.parametrize("addend", [False, True], ids=["product", "accumulate"])
@pytest.mark.parametrize("m,k,n", [(4200, 128, 4200), (4200, 192, 4200), (4352, 1024, 4352), (4100, 1024, 4200),
                                   (4104, 2120, 4200), (4200, 2176, 4104), (4352, 4096, 4352)])
def test_products_with_more_tiles_than_compute_units(kind, form, addend, m, k, n):
    # More 256 x 256 tiles than the part's 256 CUs.  An even step count
    # takes the persistent kernel, where a block walks several tiles in turn,
    # including a K tail that is not a whole 64-deep step (2120 = 33 x 64 +
    # 8, 34 steps); an odd step count (192, 2176) takes the one-tile kernel.  Ragged edges in both
    # dimensions (4200 = 16 x 256 + 104), whole tiles only (4352 = 17 x 256),
    # and a ragged M with whole-tile columns; every form the tape's backward
    # products take (LEFT is Aᵀ·B, RIGHT is A·Bᵀ, tape/mod.rs:1195-1246),
    # with and without an addend.  The first and last rows are always
    # sampled, so the edge tiles are checked.
    rng = np.random.default_rng(m + 3 * k + 7 * n + 11 * form + int(addend))
    got, want, scale = sampled_form(kind, form, m, k, n, rng, addend)
    tol = tolerance(kind, kind, k) + (2.0 ** -8 if addend else 0.0)
    assert np.max(np.abs(got - want) / scale) <= tol


@pytest.mark.parametrize("in_kind,out_kind", [(lib.BF16, lib.BF16), (lib.F16, lib.F16), (lib.BF16, lib.F32),
                                              (lib.F16, lib.F32)])
@pytest.mark.parametrize("form", [lib.PLAIN, lib.LEFT, lib.RIGHT], ids=["plain", "left", "right"])
@pytest.mark.parametrize("m,k,n", [(4352, 128, 4352), (4100, 128, 4200)], ids=["whole", "ragged"])
def test_every_element_of_a_persistent_product(in_kind, out_kind, form, m, k, n):
    # 4352 x 128 x 4352: 289 whole 256 x 256 tiles on 256 CUs, so some blocks
    # walk two tiles, each of two steps; 4100 x 128 x 4200 the same count
    # with a ragged last tile row and column.  A 16-bit C runs the four-wave
    # kernel, whose staged whole-row stores skip the 16-byte pieces outside
    # C; an f32 C runs the eight-wave kernel and leaves through the
    # accumulators' own stores.  Every element is checked against the oracle
    # and f64, so a misplaced row or chunk of the staging, or a store past an
    # edge, cannot hide between sampled rows.
    rng = np.random.default_rng(m + n + out_kind + 5 * form)
    a = to_kind(rng.uniform(-1, 1, (m, k)), in_kind)
    b = to_kind(rng.uniform(-1, 1, (k, n)), in_kind)
    x = np.ascontiguousarray(a.T) if form == lib.LEFT else a
    y = np.ascontiguousarray(b.T) if form == lib.RIGHT else b
    wa, wb = widen(in_kind, a), widen(in_kind, b)
    # C is followed by 256 rows of a sentinel that no store may touch.
    guard = 256 * n
    if out_kind == lib.F32:
        sentinel = np.full(m * n + guard, 12345.5, dtype=np.float32)
    else:
        sentinel = np.full(m * n + guard, 0x7777, dtype=np.uint16).view(HOST[out_kind])
    da, db, dc = lib.Buffer.of(x), lib.Buffer.of(y), lib.Buffer.of(sentinel)
    lib.call("tc_matmul", in_kind, out_kind, form, 0, m, k, n, da.ptr, db.ptr, dc.ptr)
    whole = dc.download(HOST[out_kind], m * n + guard)
    assert np.array_equal(whole[m * n:].view(np.uint8), sentinel[m * n:].view(np.uint8))
    got = widen(out_kind, whole[: m * n].reshape(m, n))
    tol = tolerance(in_kind, out_kind, k)
    assert error(got, wa, wb, wa.astype(np.float64) @ wb.astype(np.float64)) <= tol
    want = widen(out_kind, oracle.matmul(in_kind, a, b, m, k, n, out_dtype=out_kind))
    assert error(got, wa, wb, want) <= 2 * tol


@pytest.mark.parametrize("kind", [lib.F32, lib.BF16, lib.F16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("form", [lib.PLAIN, lib.LEFT, lib.RIGHT], ids=["plain", "left", "right"])
@pytest.mark.parametrize("m,k,n", [(3000, 700, 1), (1, 700, 3000), (1, 4096, 1), (257, 8, 1), (1, 33, 129)])
def test_one_row_or_one_column_products(kind, form, m, k, n):
    # A product with one column or one row of output runs on the
    # matrix-vector kernels (MetalBuffer::product_into, metal/ops.rs:176-200),
    # in every form and with an addend, against f64.
    rng = np.random.default_rng(m + 7 * k + 11 * n + form)
    a = to_kind(rng.uniform(-1, 1, (m, k)), kind)
    b = to_kind(rng.uniform(-1, 1, (k, n)), kind)
    c = to_kind(rng.uniform(-1, 1, (m, n)), kind)
    x = np.ascontiguousarray(a.T) if form == lib.LEFT else a
    y = np.ascontiguousarray(b.T) if form == lib.RIGHT else b
    wa, wb, wc = (widen(kind, v).astype(np.float64) for v in (a, b, c))
    unit = {lib.F32: 2.0 ** -24, lib.F16: 2.0 ** -11, lib.BF16: 2.0 ** -8}[kind]
    scale = np.abs(wa) @ np.abs(wb)
    got = widen(kind, product(kind, kind, form, x, y, m, k, n)).astype(np.float64)
    want = wa @ wb
    assert np.all(np.abs(got - want) <= 1e-5 * np.sqrt(k) * scale + unit * np.abs(want) + 1e-30)
    got = widen(kind, product(kind, kind, form, x, y, m, k, n, addend=c)).astype(np.float64)
    want = want + wc
    assert np.all(np.abs(got - want) <= 1e-5 * np.sqrt(k) * scale + unit * (np.abs(want) + np.abs(wc)) + 1e-30)
