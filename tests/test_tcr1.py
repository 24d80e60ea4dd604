"""The TCR1 tensor format (persist.rs:44-93): the checker's restatement
pinned on the reference's documented layout and tags (persist.rs:44-80,
:505-541), and the library's header checks through the C-ABI (host code
only, no device) against the reference's own cases (tests/persist.rs:35-330):
the stored shape is the loaded shape, a wrong element type, kind, magic or
version is a format error naming what it found, a short file an I/O error,
trailing bytes ignored and records concatenated in one stream."""

import ctypes
import struct

import numpy as np
import pytest

from oracle import tcr1
from tensorcrate_amd import lib

F64, F32, I64 = tcr1.tag("f64"), tcr1.tag("f32"), tcr1.tag("i64")


def sample_vector_bytes():
    # tests/persist.rs:35-41: Vector::new([1.5f64, -2.5]).
    return tcr1.record(tcr1.VECTOR, [2], F64, np.array([1.5, -2.5], "<f8").tobytes())


def header(path, tag, kind, offset=0):
    out = lib.Tcr1()
    status = lib.load().tc_tcr1_read_header(str(path).encode(), offset, tag, len(tag), kind, ctypes.byref(out))
    return status, out


def test_the_checker_writes_the_documented_layout():
    # persist.rs:51-61: magic, version, kind, tag length, tag, rows, cols.
    want = (b"TCR1" + bytes([1, 0, 1, 0x11]) + struct.pack("<QQ", 2, 1) + struct.pack("<dd", 1.5, -2.5))
    assert sample_vector_bytes() == want
    kind, shape, element_tag, payload, end = tcr1.parse(want + b"and then some")
    assert (kind, shape, element_tag, end) == (0, [2], F64, len(want))
    # persist.rs:65-69: a tensor stores its rank, then one extent per axis.
    t = tcr1.record(tcr1.TENSOR, [2, 3, 4], F32, bytes(96))
    assert t[8:8 + 32] == struct.pack("<QQQQ", 3, 2, 3, 4)


def test_tags_are_a_prefix_code():
    # persist.rs:505-522.
    assert tcr1.tag("f64") == bytes([0x11])
    assert tcr1.tag("Complex", "f64") == bytes([0x20, 0x11])
    assert tcr1.tag("Complex", "Dual", "f64") == bytes([0x20, 0x21, 0x11])
    assert tcr1.tag("Dual", "Complex", "f32") == bytes([0x21, 0x20, 0x10])
    assert tcr1.element_size(tcr1.tag("Complex", "Dual", "f64")) == 32
    assert tcr1.element_size(tcr1.tag("FixedPoint", 16)) == 8


def test_the_stored_shape_is_the_shape_that_is_loaded(tmp_path):
    # tests/persist.rs:158-188.
    p = tmp_path / "v.tcr"
    p.write_bytes(sample_vector_bytes())
    status, h = header(p, F64, tcr1.VECTOR)
    assert status == lib.OK
    assert (h.kind, h.rank, h.shape[0], h.count, h.element_bytes) == (0, 1, 2, 2, 8)
    assert (h.data_offset, h.end_offset) == (7 + 1 + 16, 7 + 1 + 16 + 16)
    for rows, cols in [(2, 2), (1, 4), (0, 5), (3, 1)]:
        q = tmp_path / f"m{rows}x{cols}.tcr"
        q.write_bytes(tcr1.record(tcr1.MATRIX, [rows, cols], F32, bytes(4 * rows * cols)))
        status, h = header(q, F32, tcr1.MATRIX)
        assert status == lib.OK and (h.rank, h.shape[0], h.shape[1], h.count) == (2, rows, cols, rows * cols)
    # A tensor target reads tensor, matrix and vector records (persist.rs:453-480).
    r = tmp_path / "t.tcr"
    r.write_bytes(tcr1.record(tcr1.TENSOR, [2, 3, 4], F32, bytes(96)))
    status, h = header(r, F32, tcr1.TENSOR)
    assert status == lib.OK and (h.rank, list(h.shape[:3]), h.count, h.data_offset) == (3, [2, 3, 4], 24, 8 + 32)
    assert header(p, F64, tcr1.TENSOR)[0] == lib.OK


def expect(path, tag, kind, status, *fragments):
    got, _ = header(path, tag, kind)
    message = lib.load().tc_last_error().decode()
    assert got == status, message
    for fragment in fragments:
        assert fragment in message, message


def test_a_wrong_element_type_is_a_format_error(tmp_path):
    # tests/persist.rs:191-220.
    p = tmp_path / "v.tcr"
    p.write_bytes(sample_vector_bytes())
    expect(p, I64, tcr1.VECTOR, lib.FORMAT, "element type is f64, but the target holds i64")
    q = tmp_path / "c.tcr"
    q.write_bytes(tcr1.record(tcr1.VECTOR, [1], tcr1.tag("Complex", "f64"), bytes(16)))
    expect(q, tcr1.tag("Dual", "f64"), tcr1.VECTOR, lib.FORMAT, "Complex<f64>", "Dual<f64>")


def test_a_vector_and_a_matrix_are_not_interchangeable(tmp_path):
    # tests/persist.rs:223-245.
    p = tmp_path / "v.tcr"
    p.write_bytes(sample_vector_bytes())
    expect(p, F64, tcr1.MATRIX, lib.FORMAT, "expected a matrix, found a vector")
    q = tmp_path / "m.tcr"
    q.write_bytes(tcr1.record(tcr1.MATRIX, [2, 1], F64, bytes(16)))
    expect(q, F64, tcr1.VECTOR, lib.FORMAT, "expected a vector, found a matrix")


def test_foreign_and_future_data_is_rejected(tmp_path):
    # tests/persist.rs:248-262.
    wrong_magic = bytearray(sample_vector_bytes())
    wrong_magic[0] = ord("X")
    p = tmp_path / "x.tcr"
    p.write_bytes(bytes(wrong_magic))
    expect(p, F64, tcr1.VECTOR, lib.FORMAT, "not a tensor file", "[84, 67, 82, 49]", "[88, 67, 82, 49]")
    future = bytearray(sample_vector_bytes())
    future[4] = 99
    p.write_bytes(bytes(future))
    expect(p, F64, tcr1.VECTOR, lib.FORMAT, "99")
    deep = tcr1.record(tcr1.TENSOR, [1] * 7, F32, bytes(4))
    p.write_bytes(deep)
    expect(p, F32, tcr1.TENSOR, lib.FORMAT, "stored tensor has 7 axes; a tensor may have at most 6")


def test_truncated_input_is_an_io_error(tmp_path):
    # tests/persist.rs:265-285.
    data = sample_vector_bytes()
    p = tmp_path / "t.tcr"
    for cut in [data[:5], data[:-4], b""]:
        p.write_bytes(cut)
        expect(p, F64, tcr1.VECTOR, lib.IO, "failed to fill whole buffer")
    expect(tmp_path / "missing.tcr", F64, tcr1.VECTOR, lib.IO, "missing.tcr")


def test_trailing_bytes_are_ignored_and_records_follow_one_another(tmp_path):
    # tests/persist.rs:288-330.
    first = sample_vector_bytes()
    second = tcr1.record(tcr1.MATRIX, [1, 3], F32, np.array([1, 2, 3], "<f4").tobytes())
    p = tmp_path / "s.tcr"
    p.write_bytes(first + second + b"and then some")
    status, h = header(p, F64, tcr1.VECTOR)
    assert status == lib.OK and h.end_offset == len(first)
    status, h2 = header(p, F32, tcr1.MATRIX, offset=h.end_offset)
    assert status == lib.OK and (h2.shape[0], h2.shape[1]) == (1, 3)
    assert h2.end_offset == len(first) + len(second)
