"""A restatement of the reference's TCR1 tensor format (persist.rs:44-93,
:105-189, :226-480) in plain Python, as the checker for the library's
loader and writer.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker; the product
(``tensorcrate_amd``) never imports it.

A record: b"TCR1", version 1, kind (0 vector, 1 matrix, 2 tensor), the
element tag's length and bytes, then the extents as little-endian u64 (a
vector's length and 1; a matrix's rows and columns; a tensor's rank and one
extent per axis), then the elements, row-major, little-endian.
"""

from __future__ import annotations

import struct

MAGIC = b"TCR1"
VERSION = 1
VECTOR, MATRIX, TENSOR = 0, 1, 2

# persist.rs:134-139 (leaves) and :141-189 (Complex, Dual, FixedPoint).
LEAVES = {"i8": (0x01, 1), "u8": (0x02, 1), "i16": (0x03, 2), "u16": (0x04, 2), "i32": (0x05, 4), "u32": (0x06, 4),
          "i64": (0x07, 8), "u64": (0x08, 8), "f32": (0x10, 4), "f64": (0x11, 8), "f16": (0x12, 2),
          "bf16": (0x13, 2)}
COMPLEX, DUAL, FIXED_POINT = 0x20, 0x21, 0x30


def tag(*path) -> bytes:
    """The tag of a nested type, outermost first: tag("Complex", "Dual",
    "f64") is Complex<Dual<f64>>; ("FixedPoint", 16) is FixedPoint<16>."""
    out = bytearray()
    for part in path:
        if part == "Complex":
            out.append(COMPLEX)
        elif part == "Dual":
            out.append(DUAL)
        elif part == "FixedPoint":
            out.append(FIXED_POINT)
        elif isinstance(part, int):
            out.append(part)
        else:
            out.append(LEAVES[part][0])
    return bytes(out)


def element_size(code: bytes) -> int:
    def walk(at):
        c = code[at]
        if c in (COMPLEX, DUAL):
            size, end = walk(at + 1)
            return 2 * size, end
        if c == FIXED_POINT:
            return 8, at + 2
        return next(size for value, size in LEAVES.values() if value == c), at + 1
    size, end = walk(0)
    assert end == len(code)
    return size


def record(kind: int, shape, element_tag: bytes, payload: bytes) -> bytes:
    """`write_to` (persist.rs:350-430): the header, then the payload."""
    head = MAGIC + bytes([VERSION, kind, len(element_tag)]) + element_tag
    if kind == TENSOR:
        head += struct.pack("<Q", len(shape)) + b"".join(struct.pack("<Q", e) for e in shape)
    else:
        rows = shape[0]
        cols = shape[1] if kind == MATRIX else 1
        head += struct.pack("<QQ", rows, cols)
    return head + payload


def parse(data: bytes, offset: int = 0):
    """(kind, shape, tag, payload, end) of the record at `offset`; raises
    ValueError on a malformed record and EOFError on a short one."""
    def take(n):
        nonlocal offset
        if offset + n > len(data):
            raise EOFError("failed to fill whole buffer")
        out = data[offset:offset + n]
        offset += n
        return out
    magic = take(4)
    if magic != MAGIC:
        raise ValueError(f"not a tensor file: found {list(magic)}")
    version, kind, length = take(3)
    if version != VERSION:
        raise ValueError(f"format version {version} is not supported")
    element_tag = take(length)
    if kind == TENSOR:
        (rank,) = struct.unpack("<Q", take(8))
        shape = [struct.unpack("<Q", take(8))[0] for _ in range(rank)]
    else:
        rows, cols = struct.unpack("<QQ", take(16))
        shape = [rows] if kind == VECTOR else [rows, cols]
    count = 1
    for e in shape:
        count *= e
    payload = take(count * element_size(element_tag))
    return kind, shape, element_tag, payload, offset
