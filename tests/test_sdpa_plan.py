"""Host test of the exact SDPA's launch plan (csrc/sdpa_plan.h).

The plan decides which query tiles run whole and how the tiles of a partial
last round are cut into key ranges whose partial results a merge kernel
combines.  tests/sdpa_plan_check.cpp walks head counts, query-tile counts
(full and ragged last tiles), key lengths and the kernels' tile shapes on a
256-CU device and checks that every tile runs once, the key ranges cover the
keys once, the pieces stay within 2 * CUs - 1, the scratch fits the
no-allocation entry point's 66 MiB array, and a scratch one byte short is
refused (the -8 path).
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
CSRC = HERE.parent / "triposplat-cpu-avx512_amd" / "csrc"


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs a host C++ compiler")
def test_sdpa_launch_plan(tmp_path):
    exe = tmp_path / "sdpa_plan_check"
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-Werror", "-I", str(CSRC),
                    str(HERE / "sdpa_plan_check.cpp"), "-o", str(exe)], check=True, timeout=120)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok "), r.stdout
    assert int(r.stdout.split()[1]) > 100000
