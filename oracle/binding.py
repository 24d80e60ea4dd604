"""ctypes binding of ``liboracle.so``, the CPU restatement of the Host backend.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg, as the checker and the timed CPU
baseline.  The product (``tensorcrate_amd``) never imports it.  Each wrapper
takes numpy arrays in the element type's host form (bf16 as uint16 bits) and
returns numpy arrays.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "liboracle.so"

F32, F16, BF16 = 0, 1, 2
NUMPY = {F32: np.float32, F16: np.float16, BF16: np.uint16}
MAX_RANK = 6

u32, u64, vp, f32, i32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_float, ctypes.c_int
f64 = ctypes.c_double


class Encoded(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_uint16), ("op", ctypes.c_uint16), ("dst", ctypes.c_uint8), ("a", ctypes.c_uint8),
                ("b", ctypes.c_uint8), ("aux", ctypes.c_uint8), ("value", ctypes.c_float)]


class Place(ctypes.Structure):
    _fields_ = [("offset", u64), ("col_step", u64), ("lead", u32), ("dims", u64 * 5), ("steps", u64 * 5)]


_SIGNATURES = {
    "or_bf16_from_f32": ([f32], ctypes.c_uint16),
    "or_f16_from_f32": ([f32], ctypes.c_uint16),
    "or_f16_to_f32": ([ctypes.c_uint16], f32),
    "or_narrow": ([u32, vp, vp, u64], None),
    "or_widen": ([u32, vp, vp, u64], None),
    "or_strided_copy": ([u32, vp, u32, vp, u64, vp, vp], u64),
    "or_strided_write": ([u32, vp, vp, u32, vp, u64, vp, u64, vp], None),
    "or_binary": ([u32, u32, u32, u32, vp, vp, u64, vp, vp, u64, vp, vp], None),
    "or_elementwise": ([u32, u32, u32, vp, vp, vp, u64], None),
    "or_scalar": ([u32, u32, u32, vp, f32, i32, vp, u64], None),
    "or_clamp": ([u32, vp, f32, f32, vp, u64], None),
    "or_reduce": ([u32, vp, u32, vp, u64, vp, u32, vp, u32, u32, u64, vp], None),
    "or_arg_reduce": ([u32, vp, u32, vp, u64, vp, u32, u32, vp], None),
    "or_matmul_f32": ([vp, vp, u64, u64, u64, vp, i32], None),
    "or_matmul": ([u32, u32, vp, vp, u64, u64, u64, vp, i32], None),
    "or_transpose": ([u32, vp, u64, u64, vp], None),
    "or_dot": ([u32, vp, vp, u64], f32),
    "or_matvec": ([u32, vp, vp, u64, u64, vp, i32], None),
    "or_vecmat": ([u32, vp, vp, u64, u64, vp], None),
    "or_fused": ([u32, vp, u32, vp, vp, vp, u64, u64], None),
    "or_row_moments": ([u32, u32, vp, vp, u64, u64, vp, vp], None),
    "or_unary": ([u32, u32, vp, vp, u64], None),
    "or_moments": ([u32, vp, u64, vp], None),
    "or_correlate": ([u32, vp, u64, u64, vp, u64, u64, i32, vp], None),
    "or_correlate_input_gradient": ([u32, vp, u64, u64, vp, u64, u64, i32, vp], None),
    "or_pad": ([u32, vp, u64, u64, u64, u64, vp], None),
    "or_flip": ([u32, vp, u64, u64, vp], None),
    "or_prefix_sum": ([u32, vp, u64, vp], None),
    "or_sort": ([u32, vp, u64, u32, vp], None),
    "or_erf": ([f64], f64),
    "or_erfc": ([f64], f64),
    "or_normal_quantile": ([f64], f64),
    "or_evaluate": ([u32, u32, f64, f64, f64], f64),
    "or_distribution": ([u32, u32, u32, vp, vp, u64, f32, f32], None),
    "or_axis_distribution": ([u32, u32, u32, vp, u64, u64, u32, vp, vp, vp], None),
    "or_unary_dual": ([u32, u32, vp, vp, vp, vp, u64], None),
    "or_power": ([u32, vp, vp, vp, u64], None),
    "or_power_scalar": ([u32, vp, f32, i32, vp, u64], None),
    "or_fused_sum": ([u32, vp, u32, vp, vp, u64, u64, u32, vp], None),
    "or_matmul_epilogue": ([u32, vp, u32, vp, vp, vp, u64, u64, u64, vp, u32, vp], None),
}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIBRARY


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        lib = ctypes.CDLL(str(LIBRARY))
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes, fn.restype = args, res
        _lib = lib
    return _lib


def _p(array: np.ndarray) -> int:
    return array.ctypes.data


def _dims(values) -> np.ndarray:
    out = np.zeros(MAX_RANK, np.uint64)
    out[: len(values)] = values
    return out


def bf16_from_f32(values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, np.float32)
    out = np.empty(values.shape, np.uint16)
    load().or_narrow(BF16, _p(values), _p(out), values.size)
    return out


def f16_from_f32(values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, np.float32)
    out = np.empty(values.shape, np.uint16)
    load().or_narrow(F16, _p(values), _p(out), values.size)
    return out.view(np.float16)


def widen(dtype: int, values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values)
    out = np.empty(values.shape, np.float32)
    load().or_widen(dtype, _p(values), _p(out), values.size)
    return out


def narrow(dtype: int, values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, np.float32)
    out = np.empty(values.shape, NUMPY[dtype])
    load().or_narrow(dtype, _p(values), _p(out), values.size)
    return out


def strided_copy(src: np.ndarray, shape, offset, strides) -> np.ndarray:
    src = np.ascontiguousarray(src).reshape(-1)
    count = int(np.prod(shape, dtype=np.int64)) if len(shape) else 1
    out = np.empty(count, src.dtype)
    d_shape, d_strides = _dims(shape), _dims(strides)
    load().or_strided_copy(src.itemsize, _p(src), len(shape), _p(d_shape), offset, _p(d_strides), _p(out))
    return out.reshape(shape)


def strided_write(src: np.ndarray, target: np.ndarray, shape, from_offset, from_strides, to_offset, to_strides):
    src = np.ascontiguousarray(src).reshape(-1)
    assert target.flags.c_contiguous and target.dtype == src.dtype
    d_shape, d_from, d_to = _dims(shape), _dims(from_strides), _dims(to_strides)
    load().or_strided_write(src.itemsize, _p(src), _p(target), len(shape), _p(d_shape), from_offset, _p(d_from),
                            to_offset, _p(d_to))


def binary(dtype, kind, op, shape, a, a_offset, a_strides, b, b_offset, b_strides) -> np.ndarray:
    a = np.ascontiguousarray(a).reshape(-1)
    b = np.ascontiguousarray(b).reshape(-1)
    count = int(np.prod(shape, dtype=np.int64)) if len(shape) else 1
    out = np.empty(count, NUMPY[dtype])
    d_shape, d_a, d_b = _dims(shape), _dims(a_strides), _dims(b_strides)
    load().or_binary(dtype, kind, op, len(shape), _p(d_shape), _p(a), a_offset, _p(d_a), _p(b), b_offset, _p(d_b),
                     _p(out))
    return out.reshape(shape)


def elementwise(dtype, kind, op, a, b) -> np.ndarray:
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    out = np.empty(a.shape, NUMPY[dtype])
    load().or_elementwise(dtype, kind, op, _p(a), _p(b), _p(out), a.size)
    return out


def scalar(dtype, kind, op, a, value, scalar_left) -> np.ndarray:
    a = np.ascontiguousarray(a)
    out = np.empty(a.shape, NUMPY[dtype])
    load().or_scalar(dtype, kind, op, _p(a), value, int(scalar_left), _p(out), a.size)
    return out


def clamp(dtype, a, low, high) -> np.ndarray:
    a = np.ascontiguousarray(a)
    out = np.empty(a.shape, NUMPY[dtype])
    load().or_clamp(dtype, _p(a), low, high, _p(out), a.size)
    return out


def reduce(dtype, values, shape, offset, strides, axes, kind, op=0, divisor=0) -> np.ndarray:
    values = np.ascontiguousarray(values).reshape(-1)
    kept = [shape[k] for k in range(len(shape)) if k not in axes]
    count = int(np.prod(kept, dtype=np.int64)) if kept else 1
    out = np.empty(count, NUMPY[dtype])
    axes_array = np.array(sorted(axes), np.uint32)
    d_shape, d_strides = _dims(shape), _dims(strides)
    load().or_reduce(dtype, _p(values), len(shape), _p(d_shape), offset, _p(d_strides), len(axes), _p(axes_array),
                     kind, op, divisor, _p(out))
    return out.reshape(kept)


def arg_reduce(dtype, values, shape, offset, strides, axis, op) -> np.ndarray:
    values = np.ascontiguousarray(values).reshape(-1)
    kept = [shape[k] for k in range(len(shape)) if k != axis]
    count = int(np.prod(kept, dtype=np.int64)) if kept else 1
    out = np.empty(count, np.uint32)
    d_shape, d_strides = _dims(shape), _dims(strides)
    load().or_arg_reduce(dtype, _p(values), len(shape), _p(d_shape), offset, _p(d_strides), axis, op, _p(out))
    return out.reshape(kept)


def matmul(in_dtype, a, b, m, k, n, out_dtype=None, addend=None) -> np.ndarray:
    out_dtype = in_dtype if out_dtype is None else out_dtype
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    out = (np.array(addend, NUMPY[out_dtype]).reshape(-1).copy() if addend is not None
           else np.empty(m * n, NUMPY[out_dtype]))
    load().or_matmul(in_dtype, out_dtype, _p(a), _p(b), m, k, n, _p(out), int(addend is not None))
    return out.reshape(m, n)


def transpose(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    rows, cols = a.shape
    out = np.empty((cols, rows), a.dtype)
    load().or_transpose(a.itemsize, _p(a), rows, cols, _p(out))
    return out


def dot(dtype, a, b) -> float:
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return load().or_dot(dtype, _p(a), _p(b), a.size)


def matvec(dtype, m, v, addend=None) -> np.ndarray:
    m, v = np.ascontiguousarray(m), np.ascontiguousarray(v)
    rows, cols = m.shape
    out = np.array(addend, NUMPY[dtype]).copy() if addend is not None else np.empty(rows, NUMPY[dtype])
    load().or_matvec(dtype, _p(m), _p(v), rows, cols, _p(out), int(addend is not None))
    return out


def vecmat(dtype, v, m) -> np.ndarray:
    m, v = np.ascontiguousarray(m), np.ascontiguousarray(v)
    rows, cols = m.shape
    out = np.empty(cols, NUMPY[dtype])
    load().or_vecmat(dtype, _p(v), _p(m), rows, cols, _p(out))
    return out


def _program(code, places):
    enc = (Encoded * max(len(code), 1))(*[Encoded(*c) for c in code])
    pl = (Place * max(len(places), 1))()
    for k, (offset, col_step, lead, dims, steps) in enumerate(places):
        pl[k].offset, pl[k].col_step, pl[k].lead = offset, col_step, lead
        for d in range(len(dims)):
            pl[k].dims[d], pl[k].steps[d] = dims[d], steps[d]
    return enc, pl


def fused(dtype, code, places, inputs, outputs, rows, cols) -> None:
    """Run an encoded program; ``code`` is a list of (kind, op, dst, a, b, aux,
    value) and ``places`` of (offset, col_step, lead, dims, steps)."""
    enc, pl = _program(code, places)
    ins = (vp * max(len(inputs), 1))(*[_p(x) for x in inputs])
    outs = (vp * max(len(outputs), 1))(*[_p(x) for x in outputs])
    load().or_fused(dtype, enc, len(code), pl, ins, outs, rows, cols)


def row_moments(dtype, input_dtype, values, place, rows, cols):
    """Each row's (mean, sum of squared deviations) of the matrix ``place``
    reads, as arrays of ``dtype``'s storage type."""
    values = np.ascontiguousarray(values)
    _, pl = _program([], [place])
    means = np.zeros(max(rows, 1), NUMPY[dtype])[:rows]
    devs = np.zeros(max(rows, 1), NUMPY[dtype])[:rows]
    load().or_row_moments(dtype, input_dtype, _p(values), pl, rows, cols, _p(means), _p(devs))
    return means, devs


def fused_sum(dtype, code, places, inputs, rows, cols, axis) -> np.ndarray:
    """The program's one output summed along ``axis`` (0 rows, 1 columns)."""
    enc, pl = _program(code, places)
    ins = (vp * max(len(inputs), 1))(*[_p(x) for x in inputs])
    out = np.zeros(max(rows if axis == 0 else cols, 1), NUMPY[dtype])[:rows if axis == 0 else cols]
    load().or_fused_sum(dtype, enc, len(code), pl, ins, rows, cols, axis, _p(out))
    return out


def matmul_epilogue(dtype, code, places, a, b, m, k, n, inputs, outputs) -> None:
    """The product ``a @ b`` as the program's input 0, ``inputs`` from slot 1."""
    enc, pl = _program(code, places)
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    ins = (vp * max(len(inputs), 1))(*[_p(x) for x in inputs])
    outs = (vp * max(len(outputs), 1))(*[_p(x) for x in outputs])
    load().or_matmul_epilogue(dtype, enc, len(code), pl, _p(a), _p(b), m, k, n, ins, len(inputs), outs)


def unary(dtype, op, a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    out = np.zeros_like(a)
    load().or_unary(dtype, op, _p(a), _p(out), a.size)
    return out


def unary_dual(dtype, op, value, tangent):
    value, tangent = np.ascontiguousarray(value), np.ascontiguousarray(tangent)
    out_value, out_tangent = np.zeros_like(value), np.zeros_like(value)
    load().or_unary_dual(dtype, op, _p(value), _p(tangent), _p(out_value), _p(out_tangent), value.size)
    return out_value, out_tangent


def power(dtype, a, b) -> np.ndarray:
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    out = np.zeros_like(a)
    load().or_power(dtype, _p(a), _p(b), _p(out), a.size)
    return out


def power_scalar(dtype, a, scalar, scalar_left) -> np.ndarray:
    a = np.ascontiguousarray(a)
    out = np.zeros_like(a)
    load().or_power_scalar(dtype, _p(a), scalar, int(scalar_left), _p(out), a.size)
    return out


def moments(dtype, a):
    """(mean, sum of squared deviations) as f32, unrounded."""
    a = np.ascontiguousarray(a)
    out = np.zeros(2, np.float32)
    load().or_moments(dtype, _p(a), a.size, _p(out))
    return float(out[0]), float(out[1])


def correlate(dtype, x, window, flip) -> np.ndarray:
    x, window = np.ascontiguousarray(x), np.ascontiguousarray(window)
    (rows, cols), (wr, wc) = x.shape, window.shape
    out = np.zeros((rows - wr + 1, cols - wc + 1), x.dtype)
    load().or_correlate(dtype, _p(x), rows, cols, _p(window), wr, wc, int(flip), _p(out))
    return out


def correlate_input_gradient(dtype, adjoint, window, forward_flip) -> np.ndarray:
    adjoint, window = np.ascontiguousarray(adjoint), np.ascontiguousarray(window)
    (ar, ac), (wr, wc) = adjoint.shape, window.shape
    out = np.zeros((ar + wr - 1, ac + wc - 1), adjoint.dtype)
    load().or_correlate_input_gradient(dtype, _p(adjoint), ar, ac, _p(window), wr, wc, int(forward_flip), _p(out))
    return out


def pad(x, pad_rows, pad_cols) -> np.ndarray:
    x = np.ascontiguousarray(x)
    rows, cols = x.shape
    out = np.ones((rows + 2 * pad_rows, cols + 2 * pad_cols), x.dtype)
    load().or_pad(x.itemsize, _p(x), rows, cols, pad_rows, pad_cols, _p(out))
    return out


def flip(x) -> np.ndarray:
    x = np.ascontiguousarray(x)
    out = np.zeros_like(x)
    load().or_flip(x.itemsize, _p(x), x.shape[0], x.shape[1], _p(out))
    return out


def prefix_sum(dtype, a) -> np.ndarray:
    """Inclusive running total in f32, each output rounded to the type."""
    a = np.ascontiguousarray(a)
    out = np.zeros_like(a)
    load().or_prefix_sum(dtype, _p(a), a.size, _p(out))
    return out


def sort(dtype, a, order) -> np.ndarray:
    """`a` in IEEE totalOrder, `order` 0 ascending or 1 descending."""
    a = np.ascontiguousarray(a)
    out = np.zeros_like(a)
    load().or_sort(dtype, _p(a), a.size, order, _p(out))
    return out


NORMAL, INVERSE_GAUSSIAN = 0, 1
PDF, CDF, PPF = 0, 1, 2


def evaluate(family, statistic, x, first, second) -> float:
    """One distribution function in f64, unrounded."""
    return load().or_evaluate(family, statistic, x, first, second)


def distribution(dtype, family, statistic, a, first, second) -> np.ndarray:
    a = np.ascontiguousarray(a)
    out = np.zeros_like(a)
    load().or_distribution(dtype, family, statistic, _p(a), _p(out), a.size, first, second)
    return out


def axis_distribution(dtype, family, statistic, a, axis, first, second) -> np.ndarray:
    a, first, second = (np.ascontiguousarray(v) for v in (a, first, second))
    rows, cols = a.shape
    out = np.zeros_like(a)
    load().or_axis_distribution(dtype, family, statistic, _p(a), rows, cols, axis, _p(first), _p(second), _p(out))
    return out
