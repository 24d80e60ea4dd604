"""TCR1 records straight to and from HBM (`tc_tcr1_load`, `tc_tcr1_save`;
persist.rs:44-93, :350-480) and the pinned staged transfers under them
(`tc_upload_staged`, `tc_download_staged`), against the format's restatement
in oracle/tcr1.py: payload bytes survive exactly (NaN payloads, signed zeros,
every element width, nested element types, sizes across several 16 MiB
staging chunks), and records written from the device parse as the reference
writes them, one after another in a stream."""

import ctypes

import numpy as np
import pytest

from oracle import tcr1
from tensorcrate_amd import lib

pytestmark = pytest.mark.gpu


def load(path, tag, kind, offset=0):
    h = lib.Tcr1()
    lib.call("tc_tcr1_read_header", str(path).encode(), offset, tag, len(tag), kind, ctypes.byref(h))
    nbytes = h.count * h.element_bytes
    dst = lib.Buffer(max(nbytes, 16))
    lib.call("tc_tcr1_load", str(path).encode(), ctypes.byref(h), dst.ptr)
    return h, dst.download(np.uint8, nbytes).tobytes()


def f32_specials(rng):
    x = rng.standard_normal(1001).astype("<f4")
    x.view("<u4")[:4] = [0x7FC00001, 0xFFC12345, 0x80000000, 0x7F800000]  # NaN payloads, -0, inf
    return x.tobytes()


# (name, tag, payload maker): made inside the test, not at collection.
PAYLOADS = [
    ("f32 specials", tcr1.tag("f32"), f32_specials),
    ("bf16", tcr1.tag("bf16"), lambda rng: rng.integers(0, 1 << 16, 777, dtype=np.uint16).astype("<u2").tobytes()),
    ("f16", tcr1.tag("f16"), lambda rng: rng.standard_normal(300).astype("<f2").tobytes()),
    ("f64", tcr1.tag("f64"), lambda rng: rng.standard_normal(129).astype("<f8").tobytes()),
    ("Complex<f32>", tcr1.tag("Complex", "f32"), lambda rng: rng.standard_normal(100).astype("<f4").tobytes()),
    ("Complex<Dual<f64>>", tcr1.tag("Complex", "Dual", "f64"),
     lambda rng: rng.standard_normal(36).astype("<f8").tobytes()),
    ("i64", tcr1.tag("i64"), lambda rng: rng.integers(-2**62, 2**62, 33, dtype=np.int64).astype("<i8").tobytes()),
    ("FixedPoint<16>", tcr1.tag("FixedPoint", 16),
     lambda rng: rng.integers(-2**40, 2**40, 12, dtype=np.int64).astype("<i8").tobytes()),
    ("u8, 40 MiB + 3", tcr1.tag("u8"), lambda rng: rng.integers(0, 256, (40 << 20) + 3, dtype=np.uint8).tobytes()),
    ("f32, 100 MiB", tcr1.tag("f32"), lambda rng: rng.standard_normal(25 << 20, dtype=np.float32).tobytes()),
]


@pytest.mark.parametrize("name,tag,make", PAYLOADS, ids=[p[0] for p in PAYLOADS])
def test_a_record_loads_into_hbm_bit_for_bit(tmp_path, name, tag, make):
    payload = make(np.random.default_rng(3))
    size = tcr1.element_size(tag)
    count = len(payload) // size
    p = tmp_path / "r.tcr"
    p.write_bytes(tcr1.record(tcr1.VECTOR, [count], tag, payload) + b"trailing")
    h, got = load(p, tag, tcr1.VECTOR)
    assert (h.count, h.element_bytes) == (count, size)
    assert got == payload


def test_tensor_and_matrix_records_load_with_their_shapes(tmp_path):
    x = np.arange(2 * 3 * 4, dtype="<f4")
    p = tmp_path / "t.tcr"
    p.write_bytes(tcr1.record(tcr1.TENSOR, [2, 3, 4], tcr1.tag("f32"), x.tobytes()) +
                  tcr1.record(tcr1.MATRIX, [3, 8], tcr1.tag("f32"), x.tobytes()))
    h, got = load(p, tcr1.tag("f32"), tcr1.TENSOR)
    assert (h.rank, list(h.shape[:3])) == (3, [2, 3, 4]) and got == x.tobytes()
    h2, got2 = load(p, tcr1.tag("f32"), tcr1.MATRIX, offset=h.end_offset)
    assert (h2.shape[0], h2.shape[1]) == (3, 8) and got2 == x.tobytes()


@pytest.mark.parametrize("kind,shape", [(tcr1.VECTOR, [5]), (tcr1.MATRIX, [3, 7]), (tcr1.TENSOR, [2, 3, 5]),
                                        (tcr1.TENSOR, []), (tcr1.MATRIX, [4096, 4097])])
def test_records_written_from_hbm_parse_as_the_reference_writes_them(tmp_path, kind, shape):
    count = int(np.prod(shape)) if shape else 1
    rng = np.random.default_rng(count)
    x = rng.standard_normal(count).astype("<f4")
    src = lib.Buffer.of(x)
    p = tmp_path / "w.tcr"
    tag = tcr1.tag("f32")
    dims = (ctypes.c_uint64 * 6)(*shape)
    lib.call("tc_tcr1_save", str(p).encode(), 0, kind, len(shape), dims, tag, len(tag), src.ptr)
    lib.call("tc_tcr1_save", str(p).encode(), 1, kind, len(shape), dims, tag, len(tag), src.ptr)
    data = p.read_bytes()
    expected = tcr1.record(kind, shape, tag, x.tobytes())
    assert data == expected + expected
    k, s, t, payload, end = tcr1.parse(data, len(expected))
    assert (k, t, payload, end) == (kind, tag, x.tobytes(), len(data))


@pytest.mark.parametrize("nbytes", [0, 1, 4095, 16 << 20, (16 << 20) + 3, (50 << 20) + 7])
def test_staged_transfers_round_trip(nbytes):
    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 256, nbytes, dtype=np.uint8)
    dev = lib.Buffer(max(nbytes, 16))
    lib.call("tc_upload_staged", dev.ptr, host.ctypes.data, nbytes)
    back = np.zeros(nbytes, np.uint8)
    lib.call("tc_download_staged", back.ctypes.data, dev.ptr, nbytes)
    assert np.array_equal(back, host)
    assert np.array_equal(dev.download(np.uint8, nbytes), host)


def test_queued_small_reads_wait_for_themselves_only():
    # The tape's unread loss (tape/mod.rs:253-295): a read queued behind the
    # work that produces it, waited for when the value is wanted, in any order.
    values = np.arange(10, dtype=np.float32) * 1.5 - 3
    dev = lib.Buffer.of(values)
    tickets = []
    for k in range(10):
        t = ctypes.c_uint64()
        lib.call("tc_read_async", dev.ptr + 4 * k, 4, ctypes.byref(t))
        tickets.append(t.value)
    for k in reversed(range(10)):
        got = ctypes.c_float()
        lib.call("tc_read_wait", tickets[k], ctypes.byref(got), 4)
        assert got.value == values[k]
    # A ticket whose slot 1024 later reads reused, and one never issued.
    for _ in range(1024):
        t = ctypes.c_uint64()
        lib.call("tc_read_async", dev.ptr, 4, ctypes.byref(t))
    with pytest.raises(lib.HipError, match="reused by 1024 later reads"):
        lib.call("tc_read_wait", tickets[0], ctypes.byref(ctypes.c_float()), 4)
    with pytest.raises(lib.HipError, match="never issued"):
        lib.call("tc_read_wait", t.value + 5, ctypes.byref(ctypes.c_float()), 4)
    with pytest.raises(lib.HipError, match="over 64"):
        lib.call("tc_read_async", dev.ptr, 65, ctypes.byref(t))
