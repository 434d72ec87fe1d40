"""Host test of the device-workspace policy (csrc/workspace_pool.h).

The policy decides when a per-stream scratch buffer is reused, grown, freed
or retired.  Retiring matters for HIP graphs: a graph that captured a
few-row GEMM or a key-split SDPA holds the buffer's address, so the buffer
must outlive any later growth on that stream.  The C++ driver
tests/workspace_pool_check.cpp runs the policy over fake device operations
and checks each scenario (growth frees only after the stream, a captured
buffer is never freed, keys are independent, release, failure paths).
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
CSRC = HERE.parent / "triposplat-cpu-avx512_amd" / "csrc"


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs a host C++ compiler")
def test_workspace_pool_policy(tmp_path):
    exe = tmp_path / "workspace_pool_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-fsanitize=address,undefined",
                    "-I", str(CSRC), str(HERE / "workspace_pool_check.cpp"), "-o", str(exe)],
                   check=True, timeout=120)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip() == "ok"
