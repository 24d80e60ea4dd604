"""The four-wave product kernel's hazard cover, checked in its gfx950 assembly.

`gemm16x16_wide_kernel` (csrc/gemm_kernels.hpp) writes each matrix-core step
as one inline-assembly instruction on an in-place AGPR accumulator, so the
compiler's hazard recognizer does not know those instructions are
matrix-core steps and inserts no wait states around them.  The kernel relies
on three facts instead:

- a step's A and B operand registers are written by LDS loads only, whose
  wait counts cover them, never by another vector instruction shortly
  before the step reads them;
- the zeroed accumulators stand several wait states before the first step
  reads them;
- 42 wait states separate the last step from the first read of its results.

This compiles every instance the library launches, and one with a program
epilogue, to assembly with the library's own flags, and checks those facts
(and that nothing spills) by a straight-line scan of each kernel.  The same
scan runs over the instances the runtime compiler builds for product
epilogues (`tc_matmul_epilogue` from a program's second appearance): their
source is the library's own (`tc_matmul_epilogue_source`), compiled with the
flags it hands the runtime compiler, for a dense layer's bias + relu and for
a program with more inputs, places and outputs.  A compiler that moved a
register copy next to a step would fail here, on the CPU, rather than give
wrong products on the GPU.  Runs on the CPU: hipcc cross-compiles for
gfx950.
"""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from tensorcrate_amd import _build, lib
from tests.common import EXP, Code, column_broadcast, identity_place, row_broadcast

CSRC = Path(__file__).resolve().parent.parent / "tensorcrate_amd" / "csrc"
INSTANCES = [(t, f) for t in ("tc::bf16_t", "_Float16") for f in ("true, true", "true, false", "false, false")]
SOURCE = """#include <hip/hip_runtime.h>
#include "gemm_kernels.hpp"
struct RowStore {
  static constexpr bool kProgram = true;
  static constexpr int kElems = 16;
  float* out;
  const float* bias;
  __device__ __forceinline__ void group(const bool (&live)[16], const uint32_t (&row)[16], const uint32_t (&col)[16],
                                        uint32_t N, const float (&product)[16]) const {
    for (int e = 0; e < 16; e++)
      if (live[e]) out[row[e] * N + col[e]] = fmaxf(product[e] + bias[col[e]], 0.0f);
  }
};
namespace tc {
%s
}
"""
# Wait states a non-matrix-core vector write must stand before a step reads
# the register, and a step's result before anything else reads it.
BEFORE_STEP = 12
AFTER_STEP = 18


def instance(t, forms, epi="PlainStore"):
    return (f"template __global__ void gemm16x16_wide_kernel<{t}, {t}, {forms}, {epi}>(const {t}*, const {t}*, "
            f"{t}*, uint32_t, uint32_t, uint32_t, bool, {epi});")


def registers(token, kind):
    m = re.fullmatch(kind + r"\[(\d+):(\d+)\]", token)
    if m:
        return range(int(m.group(1)), int(m.group(2)) + 1)
    m = re.fullmatch(kind + r"(\d+)", token)
    return range(int(m.group(1)), int(m.group(1)) + 1) if m else range(0)


def scan(body):
    """Problems in one kernel's instructions, in program order."""
    last = {}  # (file, register) -> (position, "step" | "vector" | "memory", text)
    position, steps, problems = 0, 0, []
    for raw in body.split("\n"):
        line = raw.split(";")[0].strip()
        if not line or line.startswith(".") or line.endswith(":"):
            continue
        parts = line.replace(",", " ").split()
        op = parts[0]
        if op == "s_nop":
            position += int(parts[1], 0) + 1
            continue
        position += 1
        if op.startswith("v_mfma"):
            steps += 1
            reads = [("v", r) for r in [*registers(parts[2], "v"), *registers(parts[3], "v")]]
            reads += [("a", r) for r in registers(parts[4], "a")]
            for reg in reads:
                if reg in last and last[reg][1] == "vector" and position - last[reg][0] < BEFORE_STEP:
                    problems.append(f"{last[reg][2]!r} then {line!r} {position - last[reg][0]} states later")
            for kind in ("a", "v"):
                for r in registers(parts[1], kind):
                    last[(kind, r)] = (position, "step", line)
            continue
        if op.startswith("v_") or op.startswith(("ds_write", "buffer_store", "global_store", "scratch_store")):
            sources = parts[2:] if op.startswith("v_") else parts[1:]
            for token in sources:
                for kind in ("a", "v"):
                    for r in registers(token, kind):
                        reg = (kind, r)
                        if reg in last and last[reg][1] == "step" and position - last[reg][0] < AFTER_STEP:
                            problems.append(f"{last[reg][2]!r} then {line!r} {position - last[reg][0]} states later")
        if op.startswith("v_") and len(parts) > 1:
            for kind in ("a", "v"):
                for r in registers(parts[1], kind):
                    last[(kind, r)] = (position, "vector", line)
        elif op.startswith(("ds_read", "buffer_load", "global_load", "scratch_load")) and len(parts) > 1:
            if not line.endswith(" lds"):  # a load into LDS writes no register
                for r in registers(parts[1], "v"):
                    last[("v", r)] = (position, "memory", line)
    return steps, problems


@pytest.fixture(scope="module")
def assembly(tmp_path_factory):
    try:
        compiler = _build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc is not installed")
    work = tmp_path_factory.mktemp("asm")
    source = work / "wide.hip"
    lines = [instance(t, f) for t, f in INSTANCES] + [instance("tc::bf16_t", "true, false", "::RowStore")]
    source.write_text(SOURCE % "\n".join(lines))
    target = work / "wide.s"
    flags = [f for f in _build.HIP_FLAGS if f != "-fPIC"]
    result = subprocess.run([compiler, *flags, f"-I{CSRC}", "--cuda-device-only", "-S", str(source), "-o",
                             str(target)], capture_output=True, text=True)
    assert result.returncode == 0, result.stderr[-4000:]
    return target.read_text()


def kernels(text):
    for chunk in re.split(r"\n(?=_Z\S*:)", text):
        name = chunk.split(":", 1)[0]
        if name.startswith("_Z") and "gemm16x16_wide_kernel" in name:
            yield name, chunk


def test_every_instance_is_there_and_nothing_spills(assembly):
    names = [name for name, _ in kernels(assembly)]
    assert len(names) == len(INSTANCES) + 1
    spills = re.findall(r"\.name:\s+(\S*gemm16x16_wide_kernel\S*)\n(?:.*\n)*?\s+\.vgpr_spill_count:\s+(\d+)", assembly)
    assert len(spills) == len(names)
    assert all(count == "0" for _, count in spills), spills
    agprs = re.findall(r"\.agpr_count:\s+(\d+)\n(?:.*\n)*?\s+\.name:\s+\S*gemm16x16_wide_kernel", assembly)
    assert agprs and all(count == "256" for count in agprs), agprs


def test_no_vector_write_stands_close_before_a_matrix_core_step(assembly):
    for name, body in kernels(assembly):
        steps, problems = scan(body)
        assert steps == 256, (name, steps)  # two 64-deep steps of 2 x 64 matrix-core steps
        assert not problems, (name, problems[:5])


def test_the_scan_finds_a_planted_hazard():
    # The same scan over a made-up sequence: a copy into an operand register
    # one instruction before the step that reads it, and an accumulator read
    # right after the step that writes it.
    body = "\n".join([
        "v_mov_b32_e32 v4, v9",
        "v_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]",
        "v_accvgpr_read_b32 v20, a1",
        "s_nop 7", "s_nop 7", "s_nop 7",
        "v_mfma_f32_16x16x32_bf16 a[4:7], v[12:15], v[8:11], a[4:7]",
    ])
    steps, problems = scan(body)
    assert steps == 2 and len(problems) == 2


# The runtime compiler's flags for generated kernels (csrc/fused.hip,
# kCompileFlags).
RUNTIME_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-Xclang", "-target-feature",
                 "-Xclang", "-packed-fp32-ops"]


def bias_relu(kind):
    code = Code()
    p = code.load(0, 0, kind)
    b = code.load(1, 1, kind)
    code.store(code.compare(lib.MAX, code.binary(lib.ADD, p, b), code.const(0.0)), kind, 0)
    return code.code


def scaled_two_outputs(kind):
    # out0 = product * scale[row] + bias[col] (+ 0.5); out1 = exp(product) in
    # f32: three places, two inputs, the product read twice, two outputs.
    code = Code()
    p = code.load(0, 0, kind)
    s = code.load(2, 2, kind)
    b = code.load(1, 1, kind)
    shifted = code.binary(lib.ADD, code.binary(lib.ADD, code.binary(lib.MUL, p, s), b), code.const(0.5))
    code.store(shifted, kind, 0)
    code.store(code.unary(EXP, code.load(0, 0, kind)), lib.F32, 1)
    return code.code


def generated_source(kind, code, places, runs):
    enc, pl = lib._program(code, places)
    length = ctypes.c_uint64()
    lib.call("tc_matmul_epilogue_source", kind, enc, len(code), pl, len(places), runs, None, 0,
             ctypes.byref(length))
    out = ctypes.create_string_buffer(length.value + 1)
    lib.call("tc_matmul_epilogue_source", kind, enc, len(code), pl, len(places), runs, out, length.value + 1,
             ctypes.byref(length))
    return out.value.decode()


@pytest.fixture(scope="module")
def generated_assembly(tmp_path_factory):
    try:
        compiler = _build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc is not installed")
    work = tmp_path_factory.mktemp("generated")
    m = n = 8192
    places = [identity_place(m, n), row_broadcast(n), column_broadcast(m)]
    out = []
    for name, program in (("bias_relu", bias_relu), ("scaled_two_outputs", scaled_two_outputs)):
        for kind, t in ((lib.BF16, "tc::bf16_t"), (lib.F16, "_Float16")):
            # The four-wave kernel takes only the run form; a launch whose
            # operands do not allow it compiles no four-wave instance.
            assert "kRuns = false" in generated_source(kind, program(kind), places, 0)
            source = generated_source(kind, program(kind), places, 1)
            assert "kRuns = true" in source, (name, kind)
            # The library asks the runtime compiler for this instance by
            # name; here it is instantiated explicitly.
            text = ("#include <hip/hip_runtime.h>\n" + source +
                    f"template __global__ void tc::gemm16x16_wide_kernel<{t}, {t}, true, false, CompiledStore>("
                    f"const {t}*, const {t}*, {t}*, uint32_t, uint32_t, uint32_t, bool, CompiledStore);\n")
            path = work / f"{name}_{kind}.hip"
            path.write_text(text)
            target = work / f"{name}_{kind}.s"
            result = subprocess.run([compiler, *RUNTIME_FLAGS, "-Rpass-analysis=kernel-resource-usage", f"-I{CSRC}",
                                     "--cuda-device-only", "-S", str(path), "-o", str(target)],
                                    capture_output=True, text=True)
            assert result.returncode == 0, result.stderr[-4000:]
            # The report the library reads to decide whether to launch it.
            vgprs = [int(v) for v in re.findall(r"remark:\s+VGPRs: (\d+)", result.stderr)]
            scratch = [int(v) for v in re.findall(r"ScratchSize \[bytes/lane\]: (\d+)", result.stderr)]
            out.append((name, kind, target.read_text(), vgprs, scratch))
    return out


def test_generated_epilogue_instances_keep_the_hazard_cover(generated_assembly):
    # A generated epilogue may hold more values than the registers the
    # accumulators leave; what it spills must stay out of the matrix-core
    # step sequence (no scratch access between its first and last step), and
    # the hazard scan must pass with the spill stores counted as readers.
    for name, kind, text, vgprs, scratch in generated_assembly:
        # Within what the library launches (gemm.hip's kWideVgprLimit).
        assert scratch == [0] and len(vgprs) == 1 and vgprs[0] <= 224, (name, kind, vgprs, scratch)
        found = list(kernels(text))
        assert len(found) == 1, (name, kind)
        agprs = re.findall(r"\.agpr_count:\s+(\d+)", text)
        assert agprs == ["256"], (name, kind, agprs)
        lines = [line.split(";")[0].strip() for line in found[0][1].split("\n")]
        steps_at = [i for i, line in enumerate(lines) if line.startswith("v_mfma")]
        inside = [line for line in lines[steps_at[0]:steps_at[-1]] if line.startswith("scratch_")]
        assert not inside, (name, kind, inside[:3])
        steps, problems = scan(found[0][1])
        assert steps == 256, (name, kind, steps)
        assert not problems, (name, kind, problems[:5])
