"""The FP8 encoders and the INT8 row quantizers divide by the scale through
one correctly rounded reciprocal per group or row and two fused residual
corrections per value (drama3-studio_amd/csrc/common.hpp quotient_by_scale).
That quotient must be the IEEE quotient bit for bit, or encoded bytes drift
from the reference's true division (native/src/fp8_reference.cpp:19-36,
quantized_kernels.py:15-45).  The method is restated
in C (tests/quotient_check.c) and compared with IEEE division on the CPU over
random groups and adversarial values next to every E4M3 value and midpoint."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_reciprocal_quotient_is_the_ieee_quotient(tmp_path):
    exe = tmp_path / "quotient_check"
    subprocess.run(["gcc", "-std=c11", "-O2", "-ffp-contract=off", "-Wall", "-Werror",
                    str(ROOT / "tests" / "quotient_check.c"), "-o", str(exe), "-lm"], check=True)
    run = subprocess.run([str(exe), "2000000"], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.startswith("ok ")


def _planted(tmp_path, one_correction):
    """The check must catch a broken quotient: plant a mistake in a copy."""
    src = (ROOT / "tests" / "quotient_check.c").read_text()
    if one_correction:  # dropped term: the residual left out of the first correction
        src = src.replace("fmaf(fmaf(-q0, scale, v), y, q0)", "q0")
        src = src.replace("return fmaf(fmaf(-q1, scale, v), y, q1);", "return q1;")
    else:  # wrong sign in the residual
        src = src.replace("fmaf(fmaf(-q1, scale, v), y, q1)", "fmaf(fmaf(q1, scale, v), y, q1)")
    path = tmp_path / "planted.c"
    path.write_text(src)
    exe = tmp_path / "planted"
    subprocess.run(["gcc", "-std=c11", "-O2", "-ffp-contract=off", str(path), "-o", str(exe), "-lm"], check=True)
    return subprocess.run([str(exe), "200000"], capture_output=True, text=True, timeout=120)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
@pytest.mark.parametrize("one_correction", [True, False])
def test_quotient_check_catches_a_planted_mistake(tmp_path, one_correction):
    run = _planted(tmp_path, one_correction)
    assert run.returncode != 0 and "differ" in run.stdout
