"""The guard of the static scan scratch, compiled and run on the CPU.

m3_hip_scan_views_static uses one device array per GPU, shared by every
handle of the process; the guard (m3.c_amd/csrc/hip/m3_scratch_guard.h)
makes a second, overlapping call on the same GPU fail with a message
instead of mixing the two calls' flags. tests/csrc/scratch_guard_check.cpp
checks its acquire/release rules and mutual exclusion under eight
contending threads.
"""
import os
import subprocess

from conftest import ROOT


def test_scratch_guard(tmp_path):
    binary = str(tmp_path / "scratch_guard_check")
    subprocess.run(["g++", "-std=c++17", "-O2", "-pthread",
                    "-I", os.path.join(ROOT, "m3.c_amd", "csrc", "hip"),
                    os.path.join(ROOT, "tests", "csrc",
                                 "scratch_guard_check.cpp"),
                    "-o", binary], check=True)
    result = subprocess.run([binary], capture_output=True, text=True,
                            timeout=120)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "violations 0" in result.stdout
