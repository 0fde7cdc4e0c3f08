"""The kernels' grid arithmetic (pseudobrain_amd/csrc/schedule.hpp) for device
shapes other than the full MI355X (32/64/80/128/256 CUs, 1/2/4/8 XCDs): the
XCD grouping of the scan, wide-scan and backward grids is a bijection, every
prep item has exactly one workgroup, and the scan's sequence groups stay within
the CUs. Compiled for the host with g++ (no GPU)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs a host C++ compiler")
def test_schedule_arithmetic(tmp_path):
    exe = tmp_path / "schedule_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-D__host__=", "-D__device__=",
                    "-I", os.path.join(ROOT, "pseudobrain_amd", "csrc"),
                    os.path.join(ROOT, "tests", "schedule_check.cpp"), "-o", str(exe)], check=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout[-2000:]
    assert run.stdout.strip().startswith("ok")
