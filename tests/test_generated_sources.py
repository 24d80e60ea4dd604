"""The kernels the runtime compiler builds from a program, compiled on the
CPU from the library's own generated source (hipcc cross-compiles for
gfx950) with the flags it hands the runtime compiler: every instance must
compile, and none may keep anything in scratch memory.

`tc_fused_with_statistics` (Kernels::fused_with_statistics,
kernels.rs:1103-1113) compiles a program with its row statistics into one
kernel from the program's second appearance; for a statistic of a
row-major matrix the kernel holds each row in registers, reads it once, and
feeds the program's loads of that matrix from the registers.  These check
the source of both forms."""

import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from tensorcrate_amd import _build, lib
from tests.common import Code, column_broadcast, identity_place, row_broadcast, run_form_program

CSRC = Path(__file__).resolve().parent.parent / "tensorcrate_amd" / "csrc"
RUNTIME_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-Xclang", "-target-feature",
                 "-Xclang", "-packed-fp32-ops"]


def layer_norm(dtype, cols):
    """(x - mean) / sqrt(deviations / cols + 1e-5) * gamma, gamma a row
    vector: the bench's program."""
    code = Code()
    x = code.load(0, 0, dtype)
    gamma = code.load(1, 1, dtype)
    mean = code.load(2, 2, dtype)
    deviations = code.load(2, 3, dtype)
    variance = code.binary(lib.ADD, code.binary(lib.MUL, deviations, code.const(np.float32(1.0 / cols))),
                           code.const(1e-5))
    root = code.unary(13, variance)
    code.store(code.binary(lib.MUL, code.binary(lib.DIV, code.binary(lib.SUB, x, mean), root), gamma), dtype, 0)
    return code.code


def statistics_source(dtype, code, places, rows, cols, source_ptr, stats):
    enc, pl = lib._program(code, places)
    inputs = (ctypes.c_void_p * 2)(source_ptr, 0x2000)
    table = (lib.Statistic * len(stats))()
    for i, (which, place) in enumerate(stats):
        _, spl = lib._program([], [place])
        table[i].source, table[i].source_len, table[i].source_dtype = source_ptr, rows * cols, dtype
        table[i].which = which
        table[i].place = spl[0]
    length = ctypes.c_uint64()
    lib.call("tc_fused_with_statistics_source", dtype, enc, len(code), pl, len(places), inputs, 2, rows, cols,
             table, len(stats), None, 0, ctypes.byref(length))
    out = ctypes.create_string_buffer(length.value + 1)
    lib.call("tc_fused_with_statistics_source", dtype, enc, len(code), pl, len(places), inputs, 2, rows, cols,
             table, len(stats), out, length.value + 1, ctypes.byref(length))
    return out.value.decode()


def compile_kernel(tmp_path, name, source):
    try:
        compiler = _build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc is not installed")
    path = tmp_path / f"{name}.hip"
    path.write_text("#include <hip/hip_runtime.h>\n" + source)
    target = tmp_path / f"{name}.s"
    result = subprocess.run([compiler, *RUNTIME_FLAGS, f"-I{CSRC}", "--cuda-device-only", "-S", str(path), "-o",
                             str(target)], capture_output=True, text=True)
    assert result.returncode == 0, result.stderr[-4000:]
    return target.read_text()


@pytest.mark.parametrize("dtype,cols,held,waves", [
    (lib.F32, 8192, True, 4), (lib.F32, 4100, True, 4), (lib.BF16, 1024, True, 1), (lib.F16, 8192, True, 4),
    (lib.F32, 3000, True, 2), (lib.F32, 8300, True, 4), (lib.F32, 16384, True, 4), (lib.F32, 777, False, 0),
    (lib.F32, 16400, False, 0)])
def test_statistics_kernels_compile_without_scratch(tmp_path, dtype, cols, held, waves):
    # Rows of up to 2048 elements take a wave each, up to 4096 two, longer
    # ones four, up to 64 values a lane (16384 elements); rows not whole
    # 16-byte packs, or longer, take the general form.  The held form reads
    # gamma, which every row reads alike, once for each of a lane's packs
    # before the program.
    rows = 64
    places = [identity_place(rows, cols), (0, 1, 0, [], []), column_broadcast(rows)]
    whole = identity_place(rows, cols)
    source = statistics_source(dtype, layer_norm(dtype, cols), places, rows, cols, 0x10000,
                               [(lib.STAT_MEAN, whole), (lib.STAT_DEVIATIONS, whole)])
    # The held form reads the row as 16-byte packs and feeds the program's
    # load of x from them.
    assert ("const float (&held)" in source) == held
    if held:
        assert re.search(r"v\d+\[e\] = held\[e\];", source)
        assert f"// {waves} wave(s) a row, {4 // waves} row(s) a block" in source
        assert ("__syncthreads();" in source) == (waves > 1)
        assert "p.invariant(inv[k], col < cols, col);" in source and re.search(r"v\d+\[e\] = inv\.i\d+\[e\];", source)
    text = compile_kernel(tmp_path, "statistics", source)
    assert re.findall(r"\.private_segment_fixed_size:\s+(\d+)", text) == ["0"]


def test_a_misaligned_or_offset_source_takes_the_general_form(tmp_path):
    rows, cols = 16, 1024
    places = [identity_place(rows, cols), (0, 1, 0, [], []), column_broadcast(rows)]
    whole = identity_place(rows, cols)
    stats = [(lib.STAT_MEAN, whole), (lib.STAT_DEVIATIONS, whole)]
    aligned = statistics_source(lib.F32, layer_norm(lib.F32, cols), places, rows, cols, 0x10000, stats)
    misaligned = statistics_source(lib.F32, layer_norm(lib.F32, cols), places, rows, cols, 0x10004, stats)
    assert "const float (&held)" in aligned and "const float (&held)" not in misaligned


def fused_source(dtype, code, places, rows, cols, pointers):
    enc, pl = lib._program(code, places)
    inputs = (ctypes.c_void_p * len(pointers))(*pointers)
    length = ctypes.c_uint64()
    lib.call("tc_fused_source", dtype, enc, len(code), pl, len(places), inputs, len(pointers), rows, cols, None, 0,
             ctypes.byref(length))
    out = ctypes.create_string_buffer(length.value + 1)
    lib.call("tc_fused_source", dtype, enc, len(code), pl, len(places), inputs, len(pointers), rows, cols, out,
             length.value + 1, ctypes.byref(length))
    return out.value.decode()


@pytest.mark.parametrize("dtype", [lib.F32, lib.F16, lib.BF16])
@pytest.mark.parametrize("cols,skew,form", [(1000, 0, "tc_fused_runs"), (1004, 0, "tc_fused_runs"),
                                            (70, 0, "tc_fused_general"), (1000, 1, "tc_fused_general")],
                         ids=["runs", "runs-of-four", "cols-not-whole-runs", "misaligned-bias"])
def test_broadcast_programs_compile_in_the_form_their_operands_allow(tmp_path, dtype, cols, skew, form):
    # A program with broadcast operands runs in runs of columns when cols is
    # a multiple of 4 and its operands start on whole pieces (here the f16
    # bias one element off does not), else in the general form; both
    # compile, without scratch.
    rows = 4099
    code, places = run_form_program(rows, skew)
    places[2] = identity_place(rows, cols)
    source = fused_source(dtype, code, places, rows, cols, [0x10000, 0x20000, 0x30000, 0x40000])
    assert f"void __launch_bounds__(256) {form}(" in source
    if form == "tc_fused_runs":
        # The program stores an f32 output, so a thread takes four columns:
        # each f32 store one 16-byte piece.
        assert "tc::load_run<4>(in[2]" in source and "tc::store_run<4, false>(out[1], 0u" in source
    text = compile_kernel(tmp_path, form, source)
    assert re.findall(r"\.private_segment_fixed_size:\s+(\d+)", text) == ["0"]


@pytest.mark.parametrize("cols,width", [(1000, 8), (1004, 4)])
def test_a_program_storing_only_16_bit_outputs_runs_eight_columns_a_thread(tmp_path, cols, width):
    # Without an f32 store, a thread of the run form takes eight columns:
    # 16-byte loads and stores of the 16-bit operands; four (8-byte pieces)
    # when cols is a multiple of 4 but not of 8.
    rows = 4099
    code, places = run_form_program(rows, 0)
    places[2] = identity_place(rows, cols)
    source = fused_source(lib.BF16, code[:-1], places, rows, cols, [0x10000, 0x20000, 0x30000, 0x40000])
    if width == 8:
        assert "tc::load_wide<8>(in[0]" in source and "tc::store_wide<8, false>(out[0]" in source
    else:
        assert "tc::load_run<4>(in[0]" in source and "tc::store_run<4, false>(out[0]" in source
    text = compile_kernel(tmp_path, f"runs_{width}", source)
    assert re.findall(r"\.private_segment_fixed_size:\s+(\d+)", text) == ["0"]


def test_the_composed_layer_norm_program_runs_in_runs(tmp_path):
    # The program pass of the composed layer norm: x and gamma in runs, the
    # row's two statistics one load a run.
    rows, cols = 8192, 8192
    places = [identity_place(rows, cols), (0, 1, 0, [], []), column_broadcast(rows)]
    source = fused_source(lib.F32, layer_norm(lib.F32, cols), places, rows, cols, [0x10000, 0x20000, 0x30000, 0x40000])
    assert "tc_fused_runs(" in source
    text = compile_kernel(tmp_path, "layer_norm_runs", source)
    assert re.findall(r"\.private_segment_fixed_size:\s+(\d+)", text) == ["0"]


def epilogue_source(kind, code, places, runs):
    enc, pl = lib._program(code, places)
    length = ctypes.c_uint64()
    lib.call("tc_matmul_epilogue_source", kind, enc, len(code), pl, len(places), runs, None, 0, ctypes.byref(length))
    out = ctypes.create_string_buffer(length.value + 1)
    lib.call("tc_matmul_epilogue_source", kind, enc, len(code), pl, len(places), runs, out, length.value + 1,
             ctypes.byref(length))
    return out.value.decode()


@pytest.mark.parametrize("runs", [1, 0])
def test_the_f32_product_epilogue_compiles_in_runs_of_four(tmp_path, runs):
    # relu(x w + b) over an f32 product: in the run form the f32 kernel hands
    # the program runs of four columns (one 16-byte piece, stored plainly),
    # the bias loaded once for a thread's columns; both forms compile into
    # the f32 kernel without scratch.
    m, n = 64, 96
    code = Code()
    total = code.binary(lib.ADD, code.load(0, 0, lib.F32), code.load(1, 1, lib.F32))
    code.store(code.compare(lib.MAX, total, code.const(0.0)), lib.F32, 0)
    places = [identity_place(m, n), row_broadcast(n)]
    source = epilogue_source(lib.F32, code.code, places, runs)
    assert f"static constexpr bool kRuns = {'true' if runs else 'false'};" in source
    if runs:
        assert "tc::load_run<4>(in[1]" in source and "tc::store_run<4, false>(out[0]" in source
    text = compile_kernel(tmp_path, f"f32_epilogue_{runs}", source +
                          "template __global__ void tc::inplace32_kernel<float, true, false, 128, 128, CompiledStore>("
                          "const float*, const float*, float*, uint32_t, uint32_t, uint32_t, bool, CompiledStore);\n")
    assert re.findall(r"\.private_segment_fixed_size:\s+(\d+)", text) == ["0"]
