"""The C ABI library loads and exports every entry point include/tchip.h
declares, with the struct layouts the header fixes (CPU only: no call here
touches a device)."""

import ctypes
import re
import subprocess
from pathlib import Path

from tensorcrate_amd import lib

ROOT = Path(__file__).resolve().parent.parent


def declared_functions(name="tchip.h", prefix="tc_"):
    header = (ROOT / "include" / name).read_text()
    header = re.sub(r"/\*.*?\*/", "", header, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|void|const char\*)\s+(" + prefix + r"\w+)\s*\(", header,
                                 flags=re.M)))


def test_the_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 30
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib.LIBRARY)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [name for name in names if name not in exported]
    assert not missing, missing
    # The binding names exactly the declared set.
    assert sorted(lib.SIGNATURES) == names


def test_the_host_mirror_exports_every_declared_symbol():
    names = declared_functions("tchip_host.h", "tch_")
    assert len(names) >= 7
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib.HOST_LIBRARY)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert not [name for name in names if name not in exported]
    assert sorted(lib.HOST_SIGNATURES) == names
    lib.load_host()


def test_the_library_loads_and_binds():
    loaded = lib.load()
    for name in declared_functions():
        assert getattr(loaded, name) is not None


def test_struct_layouts_match_the_header():
    # Natural C alignment of the header's structs, as a Rust #[repr(C)]
    # mirror would lay them out.
    assert ctypes.sizeof(lib.Strided) == 8 + 6 * 8
    assert ctypes.sizeof(lib.Encoded) == 12
    assert lib.Region.rank.offset == 16 and lib.Region.shape.offset == 24
    assert ctypes.sizeof(lib.Region) == 24 + 48 + 2 * 56
    assert lib.Split.kept.offset == 16
    assert ctypes.sizeof(lib.Place) == 8 + 8 + 8 + 40 + 40
    assert ctypes.sizeof(lib.Statistic) == 8 + 8 + 4 + 4 + ctypes.sizeof(lib.Place)


def test_errors_are_reported_not_raised_on_the_device():
    # A layout reaching past its storage is refused on the host, with the
    # reference's wording (backend.rs:245-250), before any device work; the
    # check needs no device.
    loaded = lib.load()
    shape = lib.dims([2, 3])
    from_ = lib.strided(5, [3, 1])
    status = loaded.tc_strided_copy(4, None, 10, 2, shape, ctypes.byref(from_), None)
    assert status == lib.INVALID
    assert loaded.tc_last_error().decode() == (
        "strided copy: shape [2, 3] with strides [3, 1] from offset 5 reaches past 10 elements")


def test_null_operands_are_refused_before_any_device_work():
    # A product or matrix-vector call with work to do and a null operand is
    # refused on the host, before any device work (a kernel would read
    # address 0).
    loaded = lib.load()
    assert loaded.tc_matmul(lib.F32, lib.F32, lib.PLAIN, 0, 4, 4, 4, None, None, None) == lib.INVALID
    assert loaded.tc_last_error().decode() == "matmul: a null operand"
    assert loaded.tc_matvec(lib.F32, 0, 8, 8, None, None, None) == lib.INVALID
    assert loaded.tc_last_error().decode() == "matvec: a null operand"
    assert loaded.tc_vecmat(lib.F32, 8, 8, None, None, None) == lib.INVALID
    assert loaded.tc_last_error().decode() == "vecmat: a null operand"
    # The same refusal across the other compute entry points that read or
    # write device memory.
    assert loaded.tc_elementwise(lib.F32, lib.ADD, None, None, None, 16) == lib.INVALID
    assert loaded.tc_last_error().decode() == "elementwise: a null operand"
    assert loaded.tc_unary(lib.F32, 0, None, None, 16) == lib.INVALID
    result = ctypes.c_float()
    assert loaded.tc_dot(lib.F32, None, None, 16, ctypes.byref(result)) == lib.INVALID
    assert loaded.tc_vector_reduce(lib.F32, None, 16, 0, ctypes.byref(result)) == lib.INVALID
    shape = lib.dims([2, 3])
    at = lib.strided(0, [3, 1])
    assert loaded.tc_strided_copy(4, None, 6, 2, shape, ctypes.byref(at), None) == lib.INVALID
    assert loaded.tc_last_error().decode() == "strided copy: a null operand"
    code = [(0, 0, 0, 0, lib.F32, 0, 0.0), (5, 0, 0, 0, lib.F32, 0, 0.0)]
    enc, places = lib._program(code, [(0, 1, 1, [2], [3])])
    ins = (ctypes.c_void_p * 1)(None)
    outs = (ctypes.c_void_p * 1)(None)
    lens = (ctypes.c_uint64 * 1)(6)
    assert loaded.tc_fused(lib.F32, enc, 2, places, 1, ins, lens, 1, outs, lens, 1, 2, 3) == lib.INVALID
    assert loaded.tc_last_error().decode() == "fused program: a null operand"
