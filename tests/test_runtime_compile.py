"""The headers the runtime compiler reads must compile under hiprtc.

The library embeds `scalar_ops.h`, `device.hpp` and `gemm_kernels.hpp` and
compiles fused programs and product epilogues from them at run time; a
construct hiprtc lacks (a type only the full toolchain's headers define, say)
would make every such compile fail, and the library would quietly keep
interpreting.  hiprtc compiles for gfx950 without a GPU, so this runs on the
CPU, with the library's own flags (`kCompileFlags`, csrc/fused.hip).
"""

import ctypes
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
    "tc::inplace32_kernel<float, true, false, 256, 128, tc::PlainStore>",
]


def test_the_embedded_headers_compile_under_hiprtc():
    try:
        rtc = ctypes.CDLL("libhiprtc.so")
    except OSError:
        pytest.skip("libhiprtc.so is not installed")
    program = ctypes.c_void_p()
    sources = (ctypes.c_char_p * len(HEADERS))(*[(CSRC / name).read_bytes() for name in HEADERS])
    names = (ctypes.c_char_p * len(HEADERS))(*[name.encode() for name in HEADERS])
    assert rtc.hiprtcCreateProgram(ctypes.byref(program), b'#include "gemm_kernels.hpp"\n', b"headers.hip",
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
        assert status == 0, log.value.decode(errors="replace")[:4000]
    finally:
        rtc.hiprtcDestroyProgram(ctypes.byref(program))
