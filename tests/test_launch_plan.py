"""The launch planner (velograd_amd/csrc/launch_plan.h) compiled for the CPU with AddressSanitizer
and UBSan and checked against the index facts the kernels rely on (tests/plan_check.cpp)."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_launch_planner_invariants(tmp_path):
    exe = tmp_path / "plan_check"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-I", os.path.join(REPO, "velograd_amd", "csrc"),
           os.path.join(HERE, "plan_check.cpp"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-4000:]
    assert "plan_check ok" in out.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
@pytest.mark.parametrize("opt", ["-O0", "-O3"])
def test_nv8_incident_plan_and_accesses(tmp_path, opt):
    """The host side of the tuning build whose one-wave-per-row forward (8 chunks per thread)
    faulted: its planner returns the launch that was intercepted in that build, and that launch's
    every load and store lies inside the tensors (tests/nv8_incident_check.cpp).  So neither a
    wrong plan nor an index outside the tensors explains the fault; 8 chunks per thread stay
    unplanned and uncompiled (launch_plan.h kMaxNV = 4)."""
    exe = tmp_path / "nv8"
    subprocess.run(["g++", "-std=c++17", opt, "-Wall", os.path.join(HERE, "nv8_incident_check.cpp"),
                    "-o", str(exe)], check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "plan: vec=1 nv=8 tpr=64 groups=4 block=256 grid=4096" in out.stdout
    assert "out of bounds: 0" in out.stdout and "in bounds" in out.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_nv8_incident_planner_overflow_is_real(tmp_path):
    """The same planner under UBSan reports the fifth write into `int order[4]`: the host bug
    that build carried (fixed in launch_plan.h, whose order array holds every entry)."""
    exe = tmp_path / "nv8_ubsan"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
                    "-fno-sanitize-recover=all", os.path.join(HERE, "nv8_incident_check.cpp"),
                    "-o", str(exe)], check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode != 0
    assert "index 4 out of bounds for type 'int [4]'" in out.stderr, out.stderr[-2000:]
