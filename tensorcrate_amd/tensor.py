"""Host-side mirror of tensorcrate's shaped types over the Hip backend.

``Tensor`` and ``TensorView`` follow the reference's ``Tensor``/``TensorView``
(src/tensors/tensor.rs, view.rs, reduction.rs, tensor_ops.rs): a view is a
shape, strides and an offset over one device storage, zero-copy reshaping
happens here, and every element-touching operation is one call into
``libtchip`` — ``strided_copy``, ``assemble``, ``strided_write``,
``strided_binary``, ``reduce_axes``, ``arg_reduce``.  Shape mistakes raise
``ValueError`` with the reference's panic wording before anything reaches the
device.  This layer exists so the parity tests read like the reference's own
(tests/nd_tensor.rs, tests/broadcast_reduce.rs); a Rust build binds the same
entry points from ``Backend``/``Kernels`` instead.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import halfconv, lib

MAX_RANK = lib.MAX_RANK

# Element kinds this mirror stores: the three float types and u32 indices.
U32 = "u32"
_WIDTH = {lib.F32: 4, lib.F16: 2, lib.BF16: 2, U32: 4}
_NUMPY = {lib.F32: np.float32, lib.F16: np.float16, lib.BF16: np.uint16, U32: np.uint32}


def contiguous_strides(shape) -> tuple[int, ...]:
    """Row-major strides (layout.rs:106-117)."""
    strides, step = [0] * len(shape), 1
    for axis in range(len(shape) - 1, -1, -1):
        strides[axis] = step
        step *= shape[axis]
    return tuple(strides)


def broadcast_shape(left, right) -> tuple[int, ...]:
    """numpy broadcasting from the last axis (layout.rs:316-340)."""
    rank = max(len(left), len(right))
    out = []
    for axis in range(rank):
        from_end = rank - axis
        l = left[len(left) - from_end] if len(left) >= from_end else 1
        r = right[len(right) - from_end] if len(right) >= from_end else 1
        if l == r or r == 1:
            out.append(l)
        elif l == 1:
            out.append(r)
        else:
            raise ValueError(f"shapes {list(left)} and {list(right)} do not broadcast")
    return tuple(out)


def _resolve(axis: int, rank: int, operation: str, shape) -> int:
    resolved = axis + rank if axis < 0 else axis
    if not 0 <= resolved < rank:
        raise ValueError(f"{operation}: axis {axis} is out of range for shape {list(shape)} ({rank} axes)")
    return resolved


class Storage:
    """A flat device allocation of ``len`` elements of one kind (``Backend::Storage``)."""

    def __init__(self, kind, length: int, buffer: lib.Buffer | None = None):
        self.kind = kind
        self.len = int(length)
        self.width = _WIDTH[kind]
        self.buffer = buffer if buffer is not None else lib.Buffer(self.len * self.width)

    @property
    def ptr(self) -> int:
        return self.buffer.ptr

    @classmethod
    def store(cls, kind, values: np.ndarray) -> "Storage":
        """``Backend::store`` (backend.rs:89): one upload."""
        values = np.ascontiguousarray(values, dtype=_NUMPY[kind]).reshape(-1)
        return cls(kind, values.size, lib.Buffer.of(values))

    def as_slice(self) -> np.ndarray:
        """``Backend::as_slice`` (backend.rs:99): waits for queued work, then reads."""
        return self.buffer.download(_NUMPY[self.kind], self.len)

    def duplicate(self) -> "Storage":
        """``Backend::duplicate`` (backend.rs:111): a device-side copy."""
        out = Storage(self.kind, self.len)
        lib.call("tc_copy", out.ptr, self.ptr, self.len * self.width)
        return out

    @classmethod
    def filled(cls, kind, length: int, value) -> "Storage":
        """``Vector::filled`` (vector.rs:101) without a host upload."""
        out = cls(kind, length)
        if kind == lib.BF16:
            scalar = halfconv.bf16_bits(np.array([value], np.float32))
        else:
            scalar = np.array([value], dtype=_NUMPY[kind])
        lib.call("tc_fill", out.ptr, out.len, out.width, scalar.ctypes.data)
        return out


@dataclass
class TensorView:
    """A layout over a storage (view.rs:31): element [i...] is
    ``storage[offset + sum(i_k * strides[k])]``."""

    storage: Storage
    shape: tuple
    strides: tuple
    offset: int = 0

    # ---- shape ----------------------------------------------------------
    @property
    def rank(self) -> int:
        return len(self.shape)

    def __len__(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    @property
    def kind(self):
        return self.storage.kind

    def _with(self, shape, strides, offset) -> "TensorView":
        if len(shape) > MAX_RANK:
            raise ValueError(f"shape {list(shape)} has {len(shape)} axes, more than the {MAX_RANK} a tensor may have")
        return TensorView(self.storage, tuple(shape), tuple(strides), offset)

    def permute(self, axes) -> "TensorView":
        """view.rs:146-170."""
        if sorted(axes) != list(range(self.rank)):
            raise ValueError(f"permute: {list(axes)} is not an order of the {self.rank} axes of shape {list(self.shape)}")
        return self._with([self.shape[a] for a in axes], [self.strides[a] for a in axes], self.offset)

    def transpose(self, a: int, b: int) -> "TensorView":
        """view.rs:180-188."""
        a, b = _resolve(a, self.rank, "transpose", self.shape), _resolve(b, self.rank, "transpose", self.shape)
        axes = list(range(self.rank))
        axes[a], axes[b] = axes[b], axes[a]
        return self.permute(axes)

    def narrow(self, axis: int, start: int, length: int) -> "TensorView":
        """view.rs:196-201: ``length`` elements of ``axis`` from ``start``."""
        axis = _resolve(axis, self.rank, "narrow", self.shape)
        end = start + length
        if not (start <= end <= self.shape[axis]):
            raise ValueError(f"narrow: {start}..{end} reaches past axis {axis}'s extent of {self.shape[axis]}")
        shape = list(self.shape)
        shape[axis] = length
        return self._with(shape, self.strides, self.offset + start * self.strides[axis])

    def slice(self, axis: int, start: int, end: int) -> "TensorView":
        """view.rs:209: the elements ``start..end`` of ``axis``."""
        return self.narrow(axis, start, end - start)

    def select(self, axis: int, index: int) -> "TensorView":
        """view.rs:233: ``axis`` fixed at ``index`` and removed."""
        axis = _resolve(axis, self.rank, "select", self.shape)
        one = self.narrow(axis, index, 1)
        return self._with(one.shape[:axis] + one.shape[axis + 1:], one.strides[:axis] + one.strides[axis + 1:],
                          one.offset)

    def chunk(self, axis: int, parts: int) -> list["TensorView"]:
        """view.rs:283: ``parts`` pieces of ``axis``, the last possibly shorter."""
        axis = _resolve(axis, self.rank, "chunk", self.shape)
        size = -(-self.shape[axis] // parts)
        return [self.narrow(axis, s, min(size, self.shape[axis] - s)) for s in range(0, self.shape[axis], size)]

    def unsqueeze(self, axis: int) -> "TensorView":
        """view.rs:323: a new axis of extent one before ``axis``."""
        axis = _resolve(axis, self.rank + 1, "unsqueeze", self.shape)
        stride = self.strides[axis] * self.shape[axis] if axis < self.rank else 1
        return self._with(self.shape[:axis] + (1,) + self.shape[axis:],
                          self.strides[:axis] + (stride,) + self.strides[axis:], self.offset)

    def broadcast_to(self, shape) -> "TensorView":
        """view.rs:370 with ``broadcast_strides`` (layout.rs:347-363)."""
        shape = tuple(shape)
        added = len(shape) - self.rank
        if added < 0:
            raise ValueError(f"broadcast: shape {list(self.shape)} does not broadcast to {list(shape)}")
        strides = [0] * len(shape)
        for axis in range(self.rank):
            wanted = shape[added + axis]
            if self.shape[axis] == wanted:
                strides[added + axis] = self.strides[axis]
            elif self.shape[axis] == 1:
                strides[added + axis] = 0
            else:
                raise ValueError(f"broadcast: shape {list(self.shape)} does not broadcast to {list(shape)}")
        return self._with(shape, strides, self.offset)

    def is_contiguous(self) -> bool:
        """layout.rs:122-134."""
        if 0 in self.shape:
            return True
        step = 1
        for extent, stride in zip(reversed(self.shape), reversed(self.strides)):
            if extent != 1 and stride != step:
                return False
            step *= extent
        return True

    # ---- copies ---------------------------------------------------------
    def contiguous(self) -> "Tensor":
        """``TensorView::contiguous`` (view.rs:407) = ``Backend::strided_copy``."""
        out = Storage(self.kind, len(self))
        from_ = lib.strided(self.offset, self.strides)
        lib.call("tc_strided_copy", self.storage.width, self.storage.ptr, self.storage.len, self.rank,
                 lib.dims(self.shape), ctypes.byref(from_), out.ptr)
        return Tensor(out, self.shape)

    def region(self, to_offset: int, to_strides) -> lib.Region:
        """``TensorView::region`` (view.rs:466): this view as the source of a copy."""
        return lib.region(self.storage.ptr, self.storage.len, self.shape, self.offset, self.strides, to_offset,
                          to_strides)

    def to_numpy(self) -> np.ndarray:
        return self.contiguous().to_numpy()

    # ---- arithmetic (tensor_ops.rs:54-199) ------------------------------
    def zip(self, other: "TensorView", kind: int, op: int) -> "Tensor":
        """``TensorView::zip`` (tensor_ops.rs:71-91): whole same-shape tensors
        take the vector kernel, anything else broadcasts and reads in place."""
        if self.kind != other.kind:
            raise ValueError("elementwise: operands of different element types")
        if (self.shape == other.shape and self.is_whole() and other.is_whole()):
            out = Storage(self.kind, len(self))
            name = "tc_elementwise" if kind == lib.ARITHMETIC else "tc_compare"
            if kind == lib.POWER:
                return self._strided(other, kind, op, self.shape)
            lib.call(name, self.kind, op, self.storage.ptr, other.storage.ptr, out.ptr, len(self))
            return Tensor(out, self.shape)
        shape = broadcast_shape(self.shape, other.shape)
        return self.broadcast_to(shape)._strided(other.broadcast_to(shape), kind, op, shape)

    def _strided(self, other: "TensorView", kind: int, op: int, shape) -> "Tensor":
        out = Storage(self.kind, int(np.prod(shape, dtype=np.int64)) if shape else 1)
        a_at, b_at = lib.strided(self.offset, self.strides), lib.strided(other.offset, other.strides)
        lib.call("tc_strided_binary", self.kind, kind, op, len(shape), lib.dims(shape), self.storage.ptr,
                 self.storage.len, ctypes.byref(a_at), other.storage.ptr, other.storage.len, ctypes.byref(b_at),
                 out.ptr)
        return Tensor(out, shape)

    def is_whole(self) -> bool:
        return self.offset == 0 and self.is_contiguous() and len(self) == self.storage.len

    def elementwise(self, other, op: int) -> "Tensor":
        return self.zip(as_view(other), lib.ARITHMETIC, op)

    def compare(self, other, op: int) -> "Tensor":
        return self.zip(as_view(other), lib.COMPARE, op)

    def power(self, other) -> "Tensor":
        return self.zip(as_view(other), lib.POWER, 0)

    __add__ = lambda self, o: self.elementwise(o, lib.ADD)
    __sub__ = lambda self, o: self.elementwise(o, lib.SUB)
    __mul__ = lambda self, o: self.elementwise(o, lib.MUL)
    __truediv__ = lambda self, o: self.elementwise(o, lib.DIV)
    __mod__ = lambda self, o: self.elementwise(o, lib.REM)

    # ---- reductions (reduction.rs:98-312) --------------------------------
    def _axes(self, axes, operation: str) -> list[int]:
        if isinstance(axes, int):
            axes = [axes]
        if axes is None:
            axes = list(range(self.rank))
        resolved = sorted(_resolve(a, self.rank, operation, self.shape) for a in axes)
        if len(set(resolved)) != len(resolved):
            raise ValueError(f"{operation}: axes {list(axes)} are not distinct axes of shape {list(self.shape)}")
        return resolved

    def split_for(self, axes) -> lib.Split:
        """``Split::new`` (layout.rs:382-401)."""
        kept = [k for k in range(self.rank) if k not in axes]
        return lib.split(self.offset, [self.shape[k] for k in kept], [self.strides[k] for k in kept],
                         [self.shape[k] for k in axes], [self.strides[k] for k in axes])

    def _reduction(self, axes, keep_dims, operation, kind, op, divisor_of, empty) -> "Tensor":
        axes = self._axes(axes, operation)
        shape = tuple((1,) if k in axes else (self.shape[k],) for k in range(self.rank) if keep_dims or k not in axes)
        shape = tuple(s[0] for s in shape)
        depth = int(np.prod([self.shape[k] for k in axes], dtype=np.int64)) if axes else 1
        divisor = divisor_of(depth)
        results = int(np.prod(shape, dtype=np.int64)) if shape else 1
        if divisor is None or depth == 0 or 0 in shape:
            return Tensor(Storage.filled(self.kind, results, empty), shape)
        out = Storage(self.kind, results)
        split = self.split_for(axes)
        lib.call("tc_reduce_axes", self.kind, self.storage.ptr, self.storage.len, ctypes.byref(split), kind, op,
                 divisor, out.ptr)
        return Tensor(out, shape)

    def sum_axes(self, axes, keep_dims=False) -> "Tensor":
        return self._reduction(axes, keep_dims, "sum_axes", lib.FOLD, lib.SUM, lambda d: 0, 0.0)

    def max_axes(self, axes, keep_dims=False) -> "Tensor":
        return self._reduction(axes, keep_dims, "max_axes", lib.FOLD, lib.RMAX, lambda d: 0, -np.inf)

    def min_axes(self, axes, keep_dims=False) -> "Tensor":
        return self._reduction(axes, keep_dims, "min_axes", lib.FOLD, lib.RMIN, lambda d: 0, np.inf)

    def mean_axes(self, axes, keep_dims=False) -> "Tensor":
        return self._reduction(axes, keep_dims, "mean_axes", lib.MEAN, 0, lambda d: 0, np.nan)

    def var_axes(self, axes, correction="population", keep_dims=False) -> "Tensor":
        """``Correction::divisor`` (statistics/mod.rs:96-101): n, or n - 1
        for ``sample``; too few elements give NaN."""
        def divisor(n):
            if correction == "sample":
                return n - 1 if n >= 2 else None
            return n if n >= 1 else None
        return self._reduction(axes, keep_dims, "var_axes", lib.VARIANCE, 0, divisor, np.nan)

    def _arg(self, axis, keep_dims, op, operation) -> "Tensor":
        axis = _resolve(axis, self.rank, operation, self.shape)
        extent = self.shape[axis]
        if extent == 0:
            raise ValueError(f"{operation}: axis {axis} of shape {list(self.shape)} is empty")
        if extent > 0xFFFFFFFF:
            raise ValueError(f"{operation}: axis {axis} of shape {list(self.shape)} is longer than a u32 index reaches")
        shape = tuple(1 if k == axis else self.shape[k] for k in range(self.rank) if keep_dims or k != axis)
        results = int(np.prod(shape, dtype=np.int64)) if shape else 1
        if 0 in shape:
            return Tensor(Storage.filled(U32, 0, 0), shape)
        out = Storage(U32, results)
        split = self.split_for([axis])
        lib.call("tc_arg_reduce", self.kind, self.storage.ptr, self.storage.len, ctypes.byref(split), op, out.ptr)
        return Tensor(out, shape)

    def argmax(self, axis, keep_dims=False) -> "Tensor":
        return self._arg(axis, keep_dims, lib.RMAX, "argmax")

    def argmin(self, axis, keep_dims=False) -> "Tensor":
        return self._arg(axis, keep_dims, lib.RMIN, "argmin")


class Tensor:
    """An owned row-major tensor (tensor.rs:50): a shape over one storage."""

    def __init__(self, storage: Storage, shape):
        self.storage = storage
        self.shape = tuple(int(s) for s in shape)

    @classmethod
    def from_numpy(cls, array: np.ndarray, kind=lib.F32) -> "Tensor":
        return cls(Storage.store(kind, array), array.shape)

    @classmethod
    def filled(cls, shape, value, kind=lib.F32) -> "Tensor":
        return cls(Storage.filled(kind, int(np.prod(shape, dtype=np.int64)) if shape else 1, value), shape)

    @property
    def kind(self):
        return self.storage.kind

    def view(self) -> TensorView:
        return TensorView(self.storage, self.shape, contiguous_strides(self.shape), 0)

    def to_numpy(self) -> np.ndarray:
        return self.storage.as_slice().reshape(self.shape)

    def __getattr__(self, name):
        # Every view operation is available on the owned tensor, as the
        # reference's `Deref`-style forwarding gives.
        return getattr(self.view(), name)

    def __add__(self, o):
        return self.view() + o

    def __sub__(self, o):
        return self.view() - o

    def __mul__(self, o):
        return self.view() * o

    def __truediv__(self, o):
        return self.view() / o

    def __mod__(self, o):
        return self.view() % o

    @staticmethod
    def concat(pieces, axis: int) -> "Tensor":
        """tensor.rs:409-449: one region per piece, one ``assemble``."""
        pieces = [as_view(p) for p in pieces]
        if not pieces:
            raise ValueError("concat: there are no tensors to join")
        first = pieces[0]
        axis = _resolve(axis, first.rank, "concat", first.shape)
        extent = 0
        for piece in pieces:
            if piece.rank != first.rank or any(k != axis and piece.shape[k] != first.shape[k]
                                               for k in range(first.rank)):
                raise ValueError(f"concat: shapes {list(first.shape)} and {list(piece.shape)} differ outside axis {axis}")
            extent += piece.shape[axis]
        shape = list(first.shape)
        shape[axis] = extent
        strides = contiguous_strides(shape)
        length = int(np.prod(shape, dtype=np.int64))
        regions, start = [], 0
        for piece in pieces:
            regions.append(piece.region(start * strides[axis], strides))
            start += piece.shape[axis]
        out = Storage(first.kind, length)
        array = (lib.Region * len(regions))(*regions)
        lib.call("tc_assemble", out.width, out.ptr, length, array, len(regions))
        return Tensor(out, shape)

    @staticmethod
    def stack(pieces, axis: int) -> "Tensor":
        """tensor.rs:459-483: concat of the pieces each with a new axis."""
        pieces = [as_view(p) for p in pieces]
        if not pieces:
            raise ValueError("stack: there are no tensors to stack")
        for piece in pieces:
            if piece.shape != pieces[0].shape:
                raise ValueError(f"stack: shapes {list(pieces[0].shape)} and {list(piece.shape)} differ")
        axis = _resolve(axis, pieces[0].rank + 1, "stack", pieces[0].shape)
        return Tensor.concat([p.unsqueeze(axis) for p in pieces], axis)

    def write_slice(self, axis: int, start: int, source) -> None:
        """tensor.rs:504-529: one ``strided_write`` into this tensor."""
        source = as_view(source)
        axis = _resolve(axis, len(self.shape), "write_slice", self.shape)
        rank = len(self.shape)
        fits = (source.rank == rank and all(k == axis or source.shape[k] == self.shape[k] for k in range(rank))
                and start + source.shape[axis] <= self.shape[axis])
        if not fits:
            raise ValueError(f"write_slice: a {list(source.shape)} source does not fit shape {list(self.shape)} "
                             f"from {start} along axis {axis}")
        strides = contiguous_strides(self.shape)
        region = source.region(start * strides[axis], strides)
        lib.call("tc_strided_write", self.storage.width, self.storage.ptr, self.storage.len, ctypes.byref(region))


def as_view(x) -> TensorView:
    return x.view() if isinstance(x, Tensor) else x
