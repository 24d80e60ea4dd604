"""The quotient that compiled programs use to divide by a value shared by a
group of elements (a function of the row's statistics or of constants,
`tc::div_uniform` in csrc/device.hpp): one f64 reciprocal, then an f64
product rounded to f32 per element, with the f32 division kept for every
result that is not a normal float.  Its exactness rests on x / d lying at
least 2^-49 (relatively) from every f32 midpoint, against the product's
2^-52; `uniform_division_check.c` checks the bits against the CPU's f32
division over a stride of every x for twenty divisors and over random
pairs.  The GPU tests of the compiled programs (Adam's bias corrections,
the layer norm's normalisation) hold the device code to the oracle's bits."""

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


def test_the_uniform_divisor_quotient_is_the_f32_division(tmp_path):
    compiler = shutil.which("gcc")
    if compiler is None:
        pytest.skip("gcc is not installed")
    binary = tmp_path / "uniform_division_check"
    build = subprocess.run([compiler, "-O2", "-o", str(binary), str(HERE / "uniform_division_check.c"), "-lm"],
                           capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([str(binary)], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "mismatches 0" in run.stdout
