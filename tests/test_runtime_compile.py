"""The headers the runtime compiler reads must compile under hiprtc.

The library embeds `scalar_ops.h`, `device.hpp` and `gemm_kernels.hpp` and
compiles fused programs and product epilogues from them at run time; a
construct hiprtc lacks (a type only the full toolchain's headers define, say)
would make every such compile fail, and the library would quietly keep
interpreting.  hiprtc compiles for gfx950 without a GPU, so this runs on the
CPU, with the library's own flags (`kCompileFlags`, csrc/fused.hip).

The compile runs in a child interpreter: other tests import torch, whose
bundled ROCm carries an older code-object compiler under the same soname as
the system's, and in a process that has loaded it hiprtc compiles with that
one instead.
"""

import ctypes
import subprocess
import sys
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parent.parent / "tensorcrate_amd" / "csrc"
HEADERS = ["scalar_ops.h", "device.hpp", "gemm_kernels.hpp"]
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops"]
KERNELS = [
    "tc::gemm16x16_kernel<tc::bf16_t, tc::bf16_t, true, false, tc::PlainStore>",
    "tc::gemm16x16_kernel<_Float16, _Float16, true, false, tc::PlainStore>",
    "tc::gemm16x16_persistent_kernel<tc::bf16_t, tc::bf16_t, true, false>",
    "tc::gemm16x16_persistent_kernel<_Float16, float, false, false>",
    "tc::direct16_kernel<tc::bf16_t, tc::bf16_t, true, false, 128, 128, 2, 2, 64, 2, tc::PlainStore>",
    "tc::inplace32_kernel<float, true, false, 128, 128, tc::PlainStore>",
    "tc::gemm16x16_persistent_kernel<tc::bf16_t, tc::bf16_t, true, false, RowStore>",
    "tc::gemm16x16_kernel<_Float16, _Float16, true, false, RowStore>",
    "tc::gemm16x16_wide_kernel<tc::bf16_t, tc::bf16_t, true, false>",
    "tc::gemm16x16_wide_kernel<_Float16, _Float16, false, false, RowStore>",
]
# A program epilogue of the shape the library generates (csrc/gemm.hip,
# run_compiled_epilogue): sixteen elements a thread, stored where live.
SOURCE = b"""#include "gemm_kernels.hpp"
struct RowStore {
  static constexpr bool kProgram = true;
  static constexpr int kElems = 16;
  float* out;
  __device__ __forceinline__ void group(const bool (&live)[16], const uint32_t (&row)[16], const uint32_t (&col)[16],
                                        uint32_t N, const float (&product)[16]) const {
    for (int e = 0; e < 16; e++) if (live[e]) out[row[e] * N + col[e]] = product[e];
  }
};
"""


def compile_headers() -> str:
    """Compile the headers with every kernel of KERNELS; the log, or "" when
    it compiled."""
    rtc = ctypes.CDLL("libhiprtc.so")
    program = ctypes.c_void_p()
    sources = (ctypes.c_char_p * len(HEADERS))(*[(CSRC / name).read_bytes() for name in HEADERS])
    names = (ctypes.c_char_p * len(HEADERS))(*[name.encode() for name in HEADERS])
    assert rtc.hiprtcCreateProgram(ctypes.byref(program), SOURCE, b"headers.hip",
                                   len(HEADERS), sources, names) == 0
    try:
        for kernel in KERNELS:
            assert rtc.hiprtcAddNameExpression(program, kernel.encode()) == 0
        flags = (ctypes.c_char_p * len(FLAGS))(*[flag.encode() for flag in FLAGS])
        status = rtc.hiprtcCompileProgram(program, len(FLAGS), flags)
        size = ctypes.c_size_t()
        rtc.hiprtcGetProgramLogSize(program, ctypes.byref(size))
        log = ctypes.create_string_buffer(size.value + 1)
        rtc.hiprtcGetProgramLog(program, log)
        return "" if status == 0 else log.value.decode(errors="replace")[:4000] or f"hiprtc status {status}"
    finally:
        rtc.hiprtcDestroyProgram(ctypes.byref(program))


def test_the_embedded_headers_compile_under_hiprtc():
    try:
        ctypes.CDLL("libhiprtc.so")
    except OSError:
        pytest.skip("libhiprtc.so is not installed")
    root = Path(__file__).resolve().parent.parent
    child = subprocess.run(
        [sys.executable, "-c", "import sys; from tests.test_runtime_compile import compile_headers; "
                               "log = compile_headers(); print(log); sys.exit(1 if log else 0)"],
        cwd=root, capture_output=True, text=True, timeout=600)
    assert child.returncode == 0, child.stdout[-4000:] + child.stderr[-2000:]
