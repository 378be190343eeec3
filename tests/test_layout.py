"""Workspace layouts of the C ABI, checked on the CPU: the layout arithmetic
(drama3-studio_amd/csrc/layout.hpp) is plain C++, built here with g++ and run
over a sweep of geometries (tests/layout_check.cpp)."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "drama3-studio_amd" / "csrc"


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_every_layout_keeps_the_head_to_itself(tmp_path):
    exe = tmp_path / "layout_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I", str(CSRC),
                    str(ROOT / "tests" / "layout_check.cpp"), "-o", str(exe)], check=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.startswith("ok ")
