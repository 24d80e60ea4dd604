"""ctypes binding of ``libtchip.so``, the C ABI declared in ``include/tchip.h``.

This is the thin driver the parity tests and the benchmark use to reach the
HIP kernels.  Loading fails loudly when the library has not been built: there
is no other implementation behind these calls to fall back on.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

PACKAGE = Path(__file__).resolve().parent
LIBRARY = PACKAGE / "libtchip.so"

MAX_RANK = 6
FUSED_LEAD = 5

# Status codes (tc_status).
OK, INVALID, UNSUPPORTED, DEVICE, OUT_OF_MEMORY, FORMAT, IO = range(7)
# Element types (fused::DType, fused/mod.rs:145-150).
F32, F16, BF16, F64 = range(4)
# BinaryOp (kernels.rs:32-38).
ADD, SUB, MUL, DIV, REM = range(5)
# Compare (kernels.rs:106-122).
MIN, MAX, MAX_SHARE, LESS, LESS_EQUAL, GREATER, GREATER_EQUAL = range(7)
# Reduce (kernels.rs:183-187).
SUM, RMIN, RMAX = range(3)
# Pairwise kinds (kernels.rs:411-415).
ARITHMETIC, COMPARE, POWER = range(3)
# AxisReduction (kernels.rs:449-457).
FOLD, MEAN, VARIANCE = range(3)
# Transposed (kernels.rs:462-467), plus PLAIN.
PLAIN, LEFT, RIGHT = range(3)

DTYPE_SIZE = {F32: 4, F16: 2, BF16: 2}
# How each element type is held on the host: bf16 as its raw bits.
NUMPY_TYPE = {F32: np.float32, F16: np.float16, BF16: np.uint16}


class Strided(ctypes.Structure):
    _fields_ = [("offset", ctypes.c_uint64), ("strides", ctypes.c_uint64 * MAX_RANK)]


class Region(ctypes.Structure):
    _fields_ = [
        ("source", ctypes.c_void_p),
        ("source_len", ctypes.c_uint64),
        ("rank", ctypes.c_uint32),
        ("shape", ctypes.c_uint64 * MAX_RANK),
        ("src", Strided),
        ("dst", Strided),
    ]


class Split(ctypes.Structure):
    _fields_ = [
        ("offset", ctypes.c_uint64),
        ("kept_rank", ctypes.c_uint32),
        ("kept", ctypes.c_uint64 * MAX_RANK),
        ("kept_strides", ctypes.c_uint64 * MAX_RANK),
        ("folded_rank", ctypes.c_uint32),
        ("folded", ctypes.c_uint64 * MAX_RANK),
        ("folded_strides", ctypes.c_uint64 * MAX_RANK),
    ]


class Encoded(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_uint16),
        ("op", ctypes.c_uint16),
        ("dst", ctypes.c_uint8),
        ("a", ctypes.c_uint8),
        ("b", ctypes.c_uint8),
        ("aux", ctypes.c_uint8),
        ("value", ctypes.c_float),
    ]


class Place(ctypes.Structure):
    _fields_ = [
        ("offset", ctypes.c_uint64),
        ("col_step", ctypes.c_uint64),
        ("lead", ctypes.c_uint32),
        ("dims", ctypes.c_uint64 * FUSED_LEAD),
        ("steps", ctypes.c_uint64 * FUSED_LEAD),
    ]


class Statistic(ctypes.Structure):
    """``tc_row_stat``: one row statistic a program reads."""
    _fields_ = [
        ("source", ctypes.c_void_p),
        ("source_len", ctypes.c_uint64),
        ("source_dtype", ctypes.c_uint32),
        ("which", ctypes.c_uint32),
        ("place", Place),
    ]


STAT_MEAN, STAT_DEVIATIONS = 0, 1


class HipError(RuntimeError):
    """A failed call: the status code and the library's message."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


_lib: ctypes.CDLL | None = None

u32, u64, vp, i32, f32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int, ctypes.c_float


class Tcr1(ctypes.Structure):
    """`tc_tcr1`: a TCR1 record's header as the loader parsed it."""
    _fields_ = [("kind", u32), ("rank", u32), ("shape", u64 * MAX_RANK), ("count", u64), ("element_bytes", u64),
                ("data_offset", u64), ("end_offset", u64)]


# Every entry point of include/tchip.h with its argument types.
SIGNATURES = {
    "tc_init": [i32],
    "tc_last_error": [],
    "tc_sync": [],
    "tc_stream": [ctypes.POINTER(vp)],
    "tc_device_info": [ctypes.c_char_p, ctypes.c_size_t, ctypes.c_char_p, ctypes.c_size_t],
    "tc_timer_begin": [],
    "tc_timer_end": [ctypes.POINTER(f32)],
    "tc_alloc": [ctypes.c_size_t, ctypes.POINTER(vp)],
    "tc_free": [vp],
    "tc_empty_cache": [],
    "tc_release_graph_memory": [],
    "tc_graph_memory": [ctypes.POINTER(u64), ctypes.POINTER(u64)],
    "tc_activity": [ctypes.POINTER(u64), ctypes.POINTER(u64)],
    "tc_upload": [vp, vp, ctypes.c_size_t],
    "tc_download": [vp, vp, ctypes.c_size_t],
    "tc_copy": [vp, vp, ctypes.c_size_t],
    "tc_fill": [vp, u64, u32, vp],
    "tc_strided_copy": [u32, vp, u64, u32, ctypes.POINTER(u64), ctypes.POINTER(Strided), vp],
    "tc_assemble": [u32, vp, u64, ctypes.POINTER(Region), u32],
    "tc_strided_write": [u32, vp, u64, ctypes.POINTER(Region)],
    "tc_elementwise": [u32, u32, vp, vp, vp, u64],
    "tc_broadcast": [u32, u32, vp, f32, i32, vp, u64],
    "tc_compare": [u32, u32, vp, vp, vp, u64],
    "tc_compare_scalar": [u32, u32, vp, f32, i32, vp, u64],
    "tc_clamp": [u32, vp, f32, f32, vp, u64],
    "tc_unary": [u32, u32, vp, vp, u64],
    "tc_unary_dual": [u32, u32, vp, vp, vp, vp, u64],
    "tc_power": [u32, vp, vp, vp, u64],
    "tc_power_scalar": [u32, vp, f32, i32, vp, u64],
    "tc_strided_binary": [u32, u32, u32, u32, ctypes.POINTER(u64), vp, u64, ctypes.POINTER(Strided), vp, u64,
                          ctypes.POINTER(Strided), vp],
    "tc_reduce_axes": [u32, vp, u64, ctypes.POINTER(Split), u32, u32, u64, vp],
    "tc_arg_reduce": [u32, vp, u64, ctypes.POINTER(Split), u32, vp],
    "tc_vector_reduce": [u32, vp, u64, u32, vp],
    "tc_vector_reduce_noalloc": [u32, vp, u64, u32, vp],
    "tc_dot": [u32, vp, vp, u64, vp],
    "tc_moments": [u32, vp, u64, vp],
    "tc_prefix_sum": [u32, vp, vp, u64],
    "tc_upload_staged": [vp, vp, ctypes.c_size_t],
    "tc_read_async": [vp, ctypes.c_size_t, ctypes.POINTER(u64)],
    "tc_read_wait": [u64, vp, ctypes.c_size_t],
    "tc_download_staged": [vp, vp, ctypes.c_size_t],
    "tc_tcr1_read_header": [ctypes.c_char_p, u64, ctypes.c_char_p, u32, u32, vp],
    "tc_tcr1_load": [ctypes.c_char_p, vp, vp],
    "tc_tcr1_save": [ctypes.c_char_p, i32, u32, u32, vp, ctypes.c_char_p, u32, vp],
    "tc_distribution": [u32, u32, u32, vp, vp, u64, f32, f32],
    "tc_axis_distribution": [u32, u32, u32, vp, u64, u64, u32, vp, vp, vp],
    "tc_sort": [u32, vp, vp, u64, u32],
    "tc_correlate": [u32, vp, u64, u64, vp, u64, u64, i32, vp],
    "tc_correlate_input_gradient": [u32, vp, u64, u64, vp, u64, u64, i32, vp],
    "tc_pad": [u32, vp, u64, u64, u64, u64, vp],
    "tc_flip": [u32, vp, u64, u64, vp],
    "tc_axis_moments": [u32, vp, u64, u64, u32, vp, vp],
    "tc_matmul": [u32, u32, u32, i32, u64, u64, u64, vp, vp, vp],
    "tc_matvec": [u32, i32, u64, u64, vp, vp, vp],
    "tc_vecmat": [u32, u64, u64, vp, vp, vp],
    "tc_transpose": [u32, u64, u64, vp, vp],
    "tc_fused": [u32, ctypes.POINTER(Encoded), u32, ctypes.POINTER(Place), u32, ctypes.POINTER(vp),
                 ctypes.POINTER(u64), u32, ctypes.POINTER(vp), ctypes.POINTER(u64), u32, u64, u64],
    "tc_fused_compiled": [ctypes.POINTER(u64)],
    "tc_fused_resident": [u64, ctypes.POINTER(u64), ctypes.POINTER(u64)],
    "tc_matmul_epilogue_source": [u32, vp, u32, vp, u32, u32, ctypes.c_char_p, u64, ctypes.POINTER(u64)],
    "tc_fused_source": [u32, vp, u32, vp, u32, vp, u32, u64, u64, ctypes.c_char_p, u64, ctypes.POINTER(u64)],
    "tc_fused_with_statistics_source": [u32, vp, u32, vp, u32, ctypes.POINTER(vp), u32, u64, u64, vp, u32,
                                        ctypes.c_char_p, u64, ctypes.POINTER(u64)],
    "tc_row_moments": [u32, u32, vp, u64, ctypes.POINTER(Place), u64, u64, vp, vp],
    "tc_fused_with_statistics": [u32, ctypes.POINTER(Encoded), u32, ctypes.POINTER(Place), u32, ctypes.POINTER(vp),
                                 ctypes.POINTER(u64), u32, ctypes.POINTER(vp), ctypes.POINTER(u64), u32, u64, u64,
                                 ctypes.POINTER(Statistic), u32],
    "tc_fused_sum": [u32, ctypes.POINTER(Encoded), u32, ctypes.POINTER(Place), u32, ctypes.POINTER(vp),
                     ctypes.POINTER(u64), u32, u64, u64, u32, vp],
    "tc_matmul_epilogue": [u32, ctypes.POINTER(Encoded), u32, ctypes.POINTER(Place), u32, u64, u64, u64, vp, vp,
                           ctypes.POINTER(vp), ctypes.POINTER(u64), u32, ctypes.POINTER(vp), ctypes.POINTER(u64),
                           u32],
}


def load() -> ctypes.CDLL:
    """The loaded library, with every signature set; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(os.environ.get("TCHIP_LIBRARY", LIBRARY))
    if not path.exists():
        raise RuntimeError(
            f"{path} is not built: run __graft_entry__.build() first; the Hip backend has no "
            "other implementation to fall back on"
        )
    lib = ctypes.CDLL(str(path))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_char_p if name == "tc_last_error" else ctypes.c_int
    _lib = lib
    return lib


def check(status: int) -> None:
    if status != OK:
        message = load().tc_last_error().decode()
        raise HipError(status, message)


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))


def sync() -> None:
    call("tc_sync")


def activity() -> tuple[int, int]:
    """This thread's (operations queued, host waits) so far (`tc_activity`)."""
    dispatches, waits = u64(), u64()
    call("tc_activity", ctypes.byref(dispatches), ctypes.byref(waits))
    return dispatches.value, waits.value


def graph_memory() -> tuple[int, int]:
    """Bytes of (live, retired) storage that captured graphs may touch."""
    live, retired = u64(), u64()
    call("tc_graph_memory", ctypes.byref(live), ctypes.byref(retired))
    return live.value, retired.value


def device_info() -> tuple[str, str]:
    name = ctypes.create_string_buffer(256)
    arch = ctypes.create_string_buffer(64)
    call("tc_device_info", name, 256, arch, 64)
    return name.value.decode(), arch.value.decode()


class Buffer:
    """Device storage from the library's stream-ordered cache."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        pointer = vp()
        call("tc_alloc", max(self.nbytes, 1), ctypes.byref(pointer))
        self.ptr = pointer.value

    @classmethod
    def of(cls, array: np.ndarray) -> "Buffer":
        array = np.ascontiguousarray(array)
        buffer = cls(array.nbytes)
        if array.nbytes:
            call("tc_upload", buffer.ptr, array.ctypes.data, array.nbytes)
        return buffer

    def download(self, dtype, count: int | None = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(count, dtype)
        if out.nbytes:
            call("tc_download", out.ctypes.data, self.ptr, out.nbytes)
        return out

    def free(self) -> None:
        if self.ptr is not None:
            load().tc_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def strided(offset: int, strides) -> Strided:
    s = Strided()
    s.offset = offset
    for k, v in enumerate(strides):
        s.strides[k] = v
    return s


def dims(values) -> ctypes.Array:
    array = (u64 * MAX_RANK)()
    for k, v in enumerate(values):
        array[k] = v
    return array


def split(offset: int, kept, kept_strides, folded, folded_strides) -> Split:
    s = Split()
    s.offset = offset
    s.kept_rank = len(kept)
    s.folded_rank = len(folded)
    for k, (e, st) in enumerate(zip(kept, kept_strides)):
        s.kept[k], s.kept_strides[k] = e, st
    for k, (e, st) in enumerate(zip(folded, folded_strides)):
        s.folded[k], s.folded_strides[k] = e, st
    return s


def _program(code, places):
    enc = (Encoded * max(len(code), 1))(*[Encoded(*c) for c in code])
    pl = (Place * max(len(places), 1))()
    for k, (offset, col_step, lead, dims_, steps) in enumerate(places):
        pl[k].offset, pl[k].col_step, pl[k].lead = offset, col_step, lead
        for d in range(len(dims_)):
            pl[k].dims[d], pl[k].steps[d] = dims_[d], steps[d]
    return enc, pl


def _buffers(pairs):
    ptrs = (vp * max(len(pairs), 1))(*[b.ptr for b, _ in pairs])
    lens = (u64 * max(len(pairs), 1))(*[n for _, n in pairs])
    return ptrs, lens


def fused(dtype: int, code, places, inputs, outputs, rows: int, cols: int) -> None:
    """``tc_fused`` over Python lists: ``code`` of (kind, op, dst, a, b, aux,
    value) tuples, ``places`` of (offset, col_step, lead, dims, steps), and
    ``inputs``/``outputs`` of (Buffer, element count) pairs."""
    enc, pl = _program(code, places)
    ins, in_lens = _buffers(inputs)
    outs, out_lens = _buffers(outputs)
    call("tc_fused", dtype, enc, len(code), pl, len(places), ins, in_lens, len(inputs), outs, out_lens, len(outputs),
         rows, cols)


def row_moments(dtype: int, input_dtype: int, source, source_len: int, place, rows: int, cols: int,
                means, deviations) -> None:
    """``tc_row_moments``: ``source``, ``means`` and ``deviations`` are
    Buffers; ``place`` is (offset, col_step, lead, dims, steps)."""
    _, pl = _program([], [place])
    call("tc_row_moments", dtype, input_dtype, source.ptr, source_len, pl, rows, cols, means.ptr, deviations.ptr)


def fused_sum(dtype: int, code, places, inputs, rows: int, cols: int, axis: int, out) -> None:
    """``tc_fused_sum`` into the Buffer ``out``."""
    enc, pl = _program(code, places)
    ins, in_lens = _buffers(inputs)
    call("tc_fused_sum", dtype, enc, len(code), pl, len(places), ins, in_lens, len(inputs), rows, cols, axis,
         out.ptr)


def fused_with_statistics(dtype: int, code, places, inputs, outputs, rows: int, cols: int, statistics) -> None:
    """``tc_fused_with_statistics`` (``Kernels::fused_with_statistics``,
    kernels.rs:1103-1113): the program runs over ``inputs`` followed by its
    row statistics, statistic i being input slot ``len(inputs) + i``.

    ``statistics`` lists, in slot order, (source Buffer, element count,
    storage dtype, place, "mean" | "deviations").  The library computes each
    distinct source's moments once (``tc_row_moments``) and runs the program
    with them, or, from the program's second appearance, runs one compiled
    kernel that never stores them."""
    enc, pl = _program(code, places)
    ins, in_lens = _buffers(inputs)
    outs, out_lens = _buffers(outputs)
    stats = (Statistic * max(len(statistics), 1))()
    for i, (source, source_len, source_dtype, place, which) in enumerate(statistics):
        _, spl = _program([], [place])
        stats[i].source, stats[i].source_len, stats[i].source_dtype = source.ptr, source_len, source_dtype
        stats[i].which = {"mean": STAT_MEAN, "deviations": STAT_DEVIATIONS}[which]
        stats[i].place = spl[0]
    call("tc_fused_with_statistics", dtype, enc, len(code), pl, len(places), ins, in_lens, len(inputs), outs,
         out_lens, len(outputs), rows, cols, stats, len(statistics))


def matmul_epilogue(dtype: int, code, places, a, b, m: int, k: int, n: int, inputs, outputs) -> None:
    """``tc_matmul_epilogue``: ``a``, ``b`` Buffers; ``inputs`` (slots 1 on)
    and ``outputs`` (Buffer, element count) pairs."""
    enc, pl = _program(code, places)
    ins, in_lens = _buffers(inputs)
    outs, out_lens = _buffers(outputs)
    call("tc_matmul_epilogue", dtype, enc, len(code), pl, len(places), m, k, n, a.ptr, b.ptr, ins, in_lens,
         len(inputs), outs, out_lens, len(outputs))


def region(source: Buffer | int, source_len: int, shape, src_offset, src_strides, dst_offset,
           dst_strides) -> Region:
    r = Region()
    r.source = source.ptr if isinstance(source, Buffer) else source
    r.source_len = source_len
    r.rank = len(shape)
    for k, v in enumerate(shape):
        r.shape[k] = v
    r.src = strided(src_offset, src_strides)
    r.dst = strided(dst_offset, dst_strides)
    return r


# ---- the C++ host mirror (include/tchip_host.h) -------------------------------

HOST_LIBRARY = PACKAGE / "libtchip_host.so"

HOST_SIGNATURES = {
    "tch_last_error": [],
    "tch_mlp_create": [u32, ctypes.POINTER(u64), u64, ctypes.POINTER(vp), ctypes.POINTER(vp), vp, vp, f32,
                       ctypes.POINTER(vp)],
    "tch_mlp_step": [vp, i32],
    "tch_mlp_loss": [vp, ctypes.POINTER(f32)],
    "tch_mlp_parameters": [vp, u32, vp, vp],
    "tch_mlp_gradients": [vp, u32, vp, vp],
    "tch_mlp_destroy": [vp],
    "tch_tape_create": [ctypes.POINTER(vp)],
    "tch_tape_destroy": [vp],
    "tch_tape_tensor": [vp, u32, ctypes.POINTER(u64), vp, ctypes.POINTER(u32)],
    "tch_tape_binary": [vp, u32, u32, u32, ctypes.POINTER(u32)],
    "tch_tape_matvec_add": [vp, u32, u32, u32, ctypes.POINTER(u32)],
    "tch_tape_unary": [vp, u32, u32, f32, f32, ctypes.POINTER(u32)],
    "tch_tape_layout": [vp, u32, u32, u32, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(u32)],
    "tch_tape_reduce": [vp, u32, u32, u32, ctypes.POINTER(ctypes.c_int64), i32, ctypes.POINTER(u32)],
    "tch_tape_split": [vp, u32, ctypes.c_int64, u32, ctypes.POINTER(u64), ctypes.POINTER(u32)],
    "tch_tape_join": [vp, u32, u32, ctypes.POINTER(u32), ctypes.c_int64, ctypes.POINTER(u32)],
    "tch_tape_add_scalars": [vp, u32, u32, ctypes.POINTER(u32)],
    "tch_tape_backward": [vp, u32, vp],
    "tch_tape_shape": [vp, u32, ctypes.POINTER(u32), ctypes.POINTER(u64)],
    "tch_tape_read": [vp, u32, i32, vp],
    "tch_tape_zero_grad": [vp],
}

HOST_VOID = {"tch_mlp_destroy", "tch_tape_destroy"}

_host: ctypes.CDLL | None = None


def load_host() -> ctypes.CDLL:
    """``libtchip_host.so``, after ``libtchip.so`` (which it links, so both
    share one runtime state); raises if it is not built."""
    global _host
    if _host is not None:
        return _host
    load()
    if not HOST_LIBRARY.exists():
        raise RuntimeError(f"{HOST_LIBRARY} is not built: run __graft_entry__.build() first")
    host = ctypes.CDLL(str(HOST_LIBRARY))
    for name, argtypes in HOST_SIGNATURES.items():
        fn = getattr(host, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_char_p if name == "tch_last_error" else (None if name in HOST_VOID else ctypes.c_int)
    _host = host
    return host


def host_call(name: str, *args) -> None:
    status = getattr(load_host(), name)(*args)
    if status != OK:
        raise HipError(status, load_host().tch_last_error().decode())


class Mlp:
    """The training step of tensorcrate's benchmark harness (``mlp_step``,
    benches/nn_ops.rs:875-921) on the C++ tape, through ``tch_mlp_*``."""

    def __init__(self, widths, batch: int, weights, biases, inputs, targets, rate: float):
        self.widths, self.batch = list(widths), int(batch)
        layers = len(self.widths) - 1
        keep = [np.ascontiguousarray(a, np.float32) for a in (*weights, *biases, inputs, targets)]
        ws, bs, x, y = keep[:layers], keep[layers:2 * layers], keep[-2], keep[-1]
        dims = (u64 * (layers + 1))(*self.widths)
        wp = (vp * layers)(*[a.ctypes.data for a in ws])
        bp = (vp * layers)(*[a.ctypes.data for a in bs])
        handle = vp()
        host_call("tch_mlp_create", layers, dims, self.batch, wp, bp, x.ctypes.data, y.ctypes.data, rate,
                  ctypes.byref(handle))
        self.handle = handle.value

    def step(self, update: bool = True) -> None:
        host_call("tch_mlp_step", self.handle, int(update))

    def loss(self) -> float:
        value = f32()
        host_call("tch_mlp_loss", self.handle, ctypes.byref(value))
        return value.value

    def _read(self, name: str, layer: int):
        w = np.empty((self.widths[layer + 1], self.widths[layer]), np.float32)
        b = np.empty(self.widths[layer + 1], np.float32)
        host_call(name, self.handle, layer, w.ctypes.data, b.ctypes.data)
        return w, b

    def parameters(self, layer: int):
        return self._read("tch_mlp_parameters", layer)

    def gradients(self, layer: int):
        return self._read("tch_mlp_gradients", layer)

    def close(self) -> None:
        if self.handle is not None:
            load_host().tch_mlp_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ``tch_binary``, ``tch_unary``, ``tch_layout``, ``tch_reduction`` (include/tchip_host.h).
TAPE_BINARY = {"add": 0, "sub": 1, "mul": 2, "div": 3, "maximum": 4, "minimum": 5, "power": 6, "matmul": 7,
               "vector_mul": 8, "matvec": 9}
TAPE_UNARY = {"clamp_min": 0, "clamp_max": 1, "clamp": 2, "relu": 3, "abs": 4, "neg": 5, "scale": 6, "shift": 7,
              "power_scalar": 8, "power_scalar_left": 9, "contiguous": 10}
TAPE_ANALYTIC = 32
TAPE_LAYOUT = {"reshape": 0, "permute": 1, "transpose": 2, "broadcast_to": 3, "narrow": 4, "select": 5, "slice": 6,
               "squeeze": 7, "unsqueeze": 8}
TAPE_JOIN = {"concat": 0, "stack": 1}
TAPE_REDUCE = {"sum_axes": 0, "mean_axes": 1, "var_axes": 2, "var_axes_sample": 3, "max_axes": 4, "min_axes": 5,
               "sum": 6, "mean": 7}


class Tape:
    """A tape of tensor variables on the C++ mirror of tape/tensor.rs,
    through ``tch_tape_*``: ``tensor`` records a leaf, the methods of
    ``TapeVar`` record operations, ``backward`` runs the rules."""

    def __init__(self):
        handle = vp()
        host_call("tch_tape_create", ctypes.byref(handle))
        self.handle = handle.value

    def _out(self, name, *args) -> "TapeVar":
        out = u32()
        host_call(name, self.handle, *args, ctypes.byref(out))
        return TapeVar(self, out.value)

    def tensor(self, values) -> "TapeVar":
        values = np.array(values, np.float32, order="C")  # keeps a 0-d shape, which ascontiguousarray does not
        dims = (u64 * max(values.ndim, 1))(*values.shape)
        return self._out("tch_tape_tensor", values.ndim, dims, values.ctypes.data)

    def join(self, op: str, pieces, axis: int) -> "TapeVar":
        handles = (u32 * max(len(pieces), 1))(*[p.handle for p in pieces])
        return self._out("tch_tape_join", TAPE_JOIN[op], len(pieces), handles, axis)

    def zero_grad(self) -> None:
        host_call("tch_tape_zero_grad", self.handle)

    def close(self) -> None:
        if self.handle is not None:
            load_host().tch_tape_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _axes(axes):
    axes = [axes] if isinstance(axes, int) else list(axes)
    return len(axes), (ctypes.c_int64 * max(len(axes), 1))(*axes)


class TapeVar:
    """One variable of a ``Tape``: a tensor, or a scalar from ``sum``/``mean``."""

    def __init__(self, tape: Tape, handle: int):
        self.tape, self.handle = tape, handle

    @property
    def shape(self) -> tuple[int, ...]:
        rank, dims = u32(), (u64 * 8)()
        host_call("tch_tape_shape", self.tape.handle, self.handle, ctypes.byref(rank), dims)
        return tuple(dims[k] for k in range(rank.value))

    def _read(self, gradient: int):
        shape = self.shape
        out = np.empty(shape, np.float32)
        host_call("tch_tape_read", self.tape.handle, self.handle, gradient, out.ctypes.data)
        return out if shape else float(out)

    def value(self):
        return self._read(0)

    def grad(self):
        return self._read(1)

    def binary(self, other: "TapeVar", op: str) -> "TapeVar":
        return self.tape._out("tch_tape_binary", TAPE_BINARY[op], self.handle, other.handle)

    __add__ = lambda self, o: self.binary(o, "add")
    __sub__ = lambda self, o: self.binary(o, "sub")
    __mul__ = lambda self, o: self.binary(o, "mul")
    __truediv__ = lambda self, o: self.binary(o, "div")

    def unary(self, op, first: float = 0.0, second: float = 0.0) -> "TapeVar":
        code = op if isinstance(op, int) else TAPE_UNARY[op]
        return self.tape._out("tch_tape_unary", code, self.handle, first, second)

    def analytic(self, f: int) -> "TapeVar":
        return self.unary(TAPE_ANALYTIC + f)

    def layout(self, op: str, values) -> "TapeVar":
        count, array = _axes(values)
        return self.tape._out("tch_tape_layout", TAPE_LAYOUT[op], self.handle, count, array)

    def reduce(self, op: str, axes=(), keep_dims: bool = False) -> "TapeVar":
        count, array = _axes(axes)
        return self.tape._out("tch_tape_reduce", TAPE_REDUCE[op], self.handle, count, array, int(keep_dims))

    def split(self, axis: int, sizes=None, parts: int = 0) -> list["TapeVar"]:
        """Pieces of ``sizes`` along ``axis``, or ``parts`` equal ones."""
        count = len(sizes) if sizes is not None else parts
        out = (u32 * max(count, 1))()
        array = (u64 * max(count, 1))(*sizes) if sizes is not None else None
        host_call("tch_tape_split", self.tape.handle, self.handle, axis, count, array, out)
        return [TapeVar(self.tape, out[k]) for k in range(count)]

    def matvec_add(self, v: "TapeVar", addend: "TapeVar") -> "TapeVar":
        return self.tape._out("tch_tape_matvec_add", self.handle, v.handle, addend.handle)

    def add_scalar(self, other: "TapeVar") -> "TapeVar":
        return self.tape._out("tch_tape_add_scalars", self.handle, other.handle)

    def backward(self, seed=None) -> None:
        if seed is None:
            host_call("tch_tape_backward", self.tape.handle, self.handle, None)
            return
        seed = np.array(seed, np.float32, order="C")
        host_call("tch_tape_backward", self.tape.handle, self.handle, seed.ctypes.data)
