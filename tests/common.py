"""Helpers shared by the tests: the reference's deterministic generators and
element-type conversions."""

from __future__ import annotations

import numpy as np

from oracle import binding as oracle
from tensorcrate_amd import lib

class _Torch:
    """torch, imported on first use.  Only CPU tests use it (as an independent
    reference for rounding); importing it at collection would put its bundled
    ROCm runtime and code-object compiler into every test process, GPU ones
    included, where they share their sonames with the system ROCm the
    library is built against and whichever loads first is the one used."""

    def __getattr__(self, name):
        if name.startswith("__"):  # collection probes objects for dunders
            raise AttributeError(name)
        import torch as module

        return getattr(module, name)


torch = _Torch()

KINDS = [lib.F32, lib.F16, lib.BF16]
KIND_NAMES = {lib.F32: "f32", lib.F16: "f16", lib.BF16: "bf16"}


class Lcg:
    """The test generator of tests/half.rs:20-40: a 64-bit LCG, top 31 bits."""

    def __init__(self, seed: int):
        self.state = seed & (2**64 - 1)

    def next(self) -> int:
        self.state = (self.state * 6364136223846793005 + 1442695040888963407) & (2**64 - 1)
        return self.state >> 33

    def uniform(self, low: float, high: float, n: int) -> np.ndarray:
        return np.array([low + (high - low) * (self.next() / float(1 << 31)) for _ in range(n)])


def filler(shape) -> np.ndarray:
    """``value(i) = ((7i + 3) mod 23) - 11`` (tests/broadcast_reduce.rs:12-14):
    integral and mixed-sign, so sums are exact in any order."""
    n = int(np.prod(shape, dtype=np.int64)) if len(shape) else 1
    i = np.arange(n, dtype=np.int64)
    return (((i * 7 + 3) % 23) - 11).astype(np.float32).reshape(shape)


def to_kind(values, kind) -> np.ndarray:
    """f32 values in the host form of `kind`, rounded once to nearest even."""
    values = np.asarray(values, np.float32)
    if kind == lib.F32:
        return values.copy()
    return oracle.narrow(kind, values)


def widen(kind, values) -> np.ndarray:
    values = np.asarray(values)
    if kind == lib.F32:
        return values.astype(np.float32)
    return oracle.widen(kind, values)


def same(got, want) -> bool:
    """Equal element for element, a NaN matching a NaN
    (tests/broadcast_reduce.rs:65-74)."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return got.shape == want.shape and bool(np.all((got == want) | (np.isnan(got) & np.isnan(want))))


def bits_equal(got: np.ndarray, want: np.ndarray) -> bool:
    got, want = np.ascontiguousarray(got), np.ascontiguousarray(want)
    return got.shape == want.shape and got.tobytes() == want.tobytes()


def _nan_mask(values: np.ndarray, kind) -> np.ndarray:
    bits = values.view(np.uint32 if kind == lib.F32 else np.uint16).astype(np.uint64)
    if kind == lib.F32:
        return (bits & 0x7FFFFFFF) > 0x7F800000
    if kind == lib.F16:
        return (bits & 0x7FFF) > 0x7C00
    return (bits & 0x7FFF) > 0x7F80


def same_bits(got: np.ndarray, want: np.ndarray, kind) -> bool:
    """Bit for bit, except that any NaN matches any NaN: a NaN's sign and
    payload are not pinned (x86 produces a negative default NaN where the
    GPU's is positive), as the reference's own `assert_same` allows
    (tests/broadcast_reduce.rs:65-74)."""
    got, want = np.ascontiguousarray(got).reshape(-1), np.ascontiguousarray(want).reshape(-1)
    if got.shape != want.shape:
        return False
    gn, wn = _nan_mask(got, kind), _nan_mask(want, kind)
    if not np.array_equal(gn, wn):
        return False
    return got[~gn].tobytes() == want[~wn].tobytes()


class CapturedGraph:
    """The calls `fn` makes on the library's stream, captured (relaxed mode)
    into one HIP graph that `replay()` launches and waits for."""

    def __init__(self, fn):
        import ctypes

        hip = ctypes.CDLL("libamdhip64.so")
        vp = ctypes.c_void_p
        hip.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
        hip.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
        hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t]
        hip.hipGraphLaunch.argtypes = [vp, vp]
        hip.hipGraphExecDestroy.argtypes = [vp]
        hip.hipGraphDestroy.argtypes = [vp]
        self._hip = hip
        self._stream = vp()
        lib.call("tc_stream", ctypes.byref(self._stream))
        self._graph, self._exec = vp(), vp()
        assert hip.hipStreamBeginCapture(self._stream, 2) == 0
        try:
            self.result = fn()
        finally:
            assert hip.hipStreamEndCapture(self._stream, ctypes.byref(self._graph)) == 0
        assert hip.hipGraphInstantiate(ctypes.byref(self._exec), self._graph, None, None, 0) == 0

    def replay(self) -> None:
        assert self._hip.hipGraphLaunch(self._exec, self._stream) == 0
        lib.sync()

    def close(self) -> None:
        self._hip.hipGraphExecDestroy(self._exec)
        self._hip.hipGraphDestroy(self._graph)


class Code:
    """A fused program's encoded instructions, (kind, op, dst, a, b, aux,
    value) tuples in order (`Encoded`, fused/mod.rs:1391-1410); each value
    takes a fresh register unless `dst` names one to reuse."""

    def __init__(self):
        self.code = []
        self._next = 0

    def _dst(self, dst):
        if dst is None:
            dst = self._next
            self._next += 1
        assert dst < 16, "the kernels hold 16 registers"
        return dst

    def load(self, place, slot, dtype, dst=None):
        d = self._dst(dst)
        self.code.append((0, place, d, slot, dtype, 0, 0.0))
        return d

    def const(self, value, dst=None):
        d = self._dst(dst)
        self.code.append((1, 0, d, 0, 0, 0, float(value)))
        return d

    def binary(self, op, a, b, dst=None):
        d = self._dst(dst)
        self.code.append((2, op, d, a, b, 0, 0.0))
        return d

    def unary(self, op, a, dst=None):
        d = self._dst(dst)
        self.code.append((3, op, d, a, 0, 0, 0.0))
        return d

    def compare(self, op, a, b, dst=None):
        d = self._dst(dst)
        self.code.append((4, op, d, a, b, 0, 0.0))
        return d

    def store(self, a, dtype, slot):
        self.code.append((5, 0, 0, a, dtype, slot, 0.0))


def identity_place(rows, cols):
    """Element (row, col) of a row-major rows x cols operand."""
    return (0, 1, 1, [rows], [cols])


def row_broadcast(cols):
    """A length-`cols` vector read by every row."""
    return (0, 1, 0, [], [])


def column_broadcast(rows):
    """A length-`rows` vector, one value per row."""
    return (0, 0, 1, [rows], [1])


EXP, SQRT = 8, 13  # `Analytic` (kernels.rs:334-354)


def ordered_bits(values: np.ndarray) -> np.ndarray:
    """Float bit patterns mapped to integers in the same order as the values,
    so that differences count ulps (f32, or raw 16-bit f16/bf16 patterns)."""
    if values.dtype == np.float32:
        bits = values.view(np.int32).astype(np.int64)
        return np.where(bits < 0, -(bits & 0x7FFFFFFF), bits)
    bits = values.view(np.uint16).astype(np.int64)
    return np.where(bits & 0x8000, -(bits & 0x7FFF), bits)


def ulps(got: np.ndarray, want: np.ndarray) -> np.ndarray:
    """Ulps between two arrays of one storage type; NaN against NaN is 0,
    NaN against a number is huge."""
    wide_got = got.astype(np.float32) if got.dtype != np.uint16 else None
    gap = np.abs(ordered_bits(got) - ordered_bits(want))
    if got.dtype == np.uint16:
        nan_g = ((got & 0x7F80) == 0x7F80) & ((got & 0x7F) != 0)
        nan_w = ((want & 0x7F80) == 0x7F80) & ((want & 0x7F) != 0)
    else:
        nan_g, nan_w = np.isnan(wide_got), np.isnan(want.astype(np.float32))
    gap = np.where(nan_g & nan_w, 0, gap)
    return np.where(nan_g != nan_w, 1 << 40, gap)


def run_form_program(rows, skew=0):
    """max(scale[row] * x + bias[col] - s, 0) as bf16 and (that sum > bias)
    as f32: a row-broadcast f16 vector `bias` (its place `skew` elements
    on), one bf16 value a row, a contiguous f32 matrix and an f32 scalar,
    each a kind of load the run form takes.  Returns (code, places) with
    places for `rows` rows."""
    from tensorcrate_amd import lib

    code = [(0, 0, 0, 0, lib.F16, 0, 0.0), (0, 1, 1, 1, lib.BF16, 0, 0.0), (0, 2, 2, 2, lib.F32, 0, 0.0),
            (0, 3, 4, 3, lib.F32, 0, 0.0), (2, lib.MUL, 3, 1, 2, 0, 0.0), (2, lib.ADD, 3, 3, 0, 0, 0.0),
            (2, lib.SUB, 3, 3, 4, 0, 0.0), (1, 0, 6, 0, 0, 0, 0.0), (4, lib.MAX, 7, 3, 6, 0, 0.0),
            (4, lib.GREATER, 5, 3, 0, 0, 0.0), (5, 0, 0, 7, lib.BF16, 0, 0.0), (5, 0, 0, 5, lib.F32, 1, 0.0)]
    places = [(skew, 1, 0, [], []), (0, 0, 1, [rows], [1]), None, (0, 0, 0, [], [])]
    return code, places
