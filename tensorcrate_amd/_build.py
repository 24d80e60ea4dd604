"""Build recipes for the native parts of the backend.

``build_library()`` compiles the HIP sources under ``csrc/`` for gfx950 and
links ``libtchip.so`` in place, next to this file; ``build_host()`` compiles
the C++ host mirror under ``host/`` into ``libtchip_host.so`` against it.
Both drive ``hipcc`` directly: one object per source, compiled in parallel,
then one link.  Nothing here runs at import time.
"""

from __future__ import annotations

import concurrent.futures
import json
import os
import shutil
import subprocess
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
HOST = PACKAGE / "host"
INCLUDE = ROOT / "include"
OBJECTS = PACKAGE / "_build"
LIBRARY = PACKAGE / "libtchip.so"
HOST_LIBRARY = PACKAGE / "libtchip_host.so"

ARCH = os.environ.get("TC_OFFLOAD_ARCH", "gfx950")

# -ffp-contract=off keeps every elementwise operation one IEEE rounding, as
# the reference's host kernels are; packed-fp32 instructions are disabled for
# every kernel.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc was not found; the HIP backend cannot be built")
    return found


def _run(command: list[str]) -> None:
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(
            "command failed: " + " ".join(command) + "\n" + result.stdout + result.stderr
        )


def _compile(source: Path, flags: list[str]) -> Path:
    OBJECTS.mkdir(exist_ok=True)
    target = OBJECTS / (source.stem + ".o")
    _run([hipcc(), *flags, "-c", str(source), "-o", str(target)])
    return target


# The headers the runtime compiler reads, each embedded as a C string: the
# scalar operations every generated kernel calls, the element types and
# operand addressing, and the product kernels a compiled epilogue is built
# into.
EMBEDDED = {"scalar_ops.h": "tc_scalar_ops_source", "device.hpp": "tc_device_source",
            "gemm_kernels.hpp": "tc_gemm_kernels_source"}


def _embedded_sources() -> Path:
    """The headers of ``EMBEDDED`` as C strings, for hiprtc at run time."""
    OBJECTS.mkdir(exist_ok=True)
    target = OBJECTS / "embedded_sources.cpp"
    parts = []
    for header, symbol in EMBEDDED.items():
        text = (CSRC / header).read_text()
        body = "".join(f"    {json.dumps(line + chr(10))}\n" for line in text.splitlines())
        parts.append(f'extern "C" const char {symbol}[] =\n' + body + "    ;\n")
    target.write_text("".join(parts))
    return target


def build_library(jobs: int | None = None) -> Path:
    """Compile every ``csrc/*.hip`` for gfx950 and link ``libtchip.so``
    (with hiprtc, which compiles fused programs at run time)."""
    sources = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 8)
    # The ROCm whose code-object compiler the runtime compiler should find
    # loaded: the one hipcc belongs to (csrc/fused.hip, runtime_compiler_is_ours).
    rocm_lib = Path(hipcc()).resolve().parent.parent / "lib"
    flags = HIP_FLAGS + [f'-DTC_ROCM_LIB="{rocm_lib}"']
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        objects = list(pool.map(lambda s: _compile(s, flags), sources))
    embedded = OBJECTS / "embedded_sources.o"
    _run(["g++", "-O2", "-fPIC", "-c", str(_embedded_sources()), "-o", str(embedded)])
    staged = LIBRARY.with_suffix(".so.tmp")
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), str(embedded), "-lhiprtc",
          "-ldl", "-o", str(staged)])
    os.replace(staged, LIBRARY)
    return LIBRARY


def build_host() -> Path | None:
    """Compile the C++ host mirror (``host/*.cpp``) against ``libtchip.so``."""
    sources = sorted(HOST.glob("*.cpp"))
    if not sources:
        return None
    staged = HOST_LIBRARY.with_suffix(".so.tmp")
    _run([
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", f"-I{INCLUDE}", f"-I{HOST}",
        *map(str, sources), f"-L{PACKAGE}", "-ltchip", "-Wl,-rpath,$ORIGIN", "-o", str(staged),
    ])
    os.replace(staged, HOST_LIBRARY)
    return HOST_LIBRARY


def build_all() -> None:
    build_library()
    build_host()


if __name__ == "__main__":
    build_all()
    print(LIBRARY)
