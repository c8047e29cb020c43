"""INTEGRATION.md route 2: the HIP backend's source compiles inside the
reference tree (CPU; needs the reference, so it is skipped elsewhere).

tests/route2_patch.py applies the route's header edits to copies of the
reference headers in a temporary directory outside the repository (pytest's
tmp_path); m3.c_amd/csrc/host/
m3_backend_hip.c, include/m3_hip.h and include/m3_backend_hip.h are
copied beside them, and gcc -fsyntax-only must accept the backend against
the patched reference headers alone. Against the unpatched headers it must
not: the patch is what the backend needs, no more.
"""
import os
import shutil
import subprocess

import pytest

from conftest import ROOT
from route2_patch import EDITS, apply_patch

REFERENCE = "/root/reference"

pytestmark = pytest.mark.skipif(
    not os.path.isdir(os.path.join(REFERENCE, "src")),
    reason="the reference tree is not present here")


def _compile(patched, tmp_path):
    out = str(tmp_path / ("route2" if patched else "route2_unpatched"))
    apply_patch(REFERENCE, out, edits=EDITS if patched else [])
    ours = os.path.join(out, "ours")
    os.makedirs(ours)
    for path in ("m3.c_amd/csrc/host/m3_backend_hip.c", "include/m3_hip.h",
                 "include/m3_backend_hip.h"):
        shutil.copy(os.path.join(ROOT, path), ours)
    return subprocess.run(
        ["gcc", "-std=c11", "-fsyntax-only", "-Wall", "-Wextra", "-Werror",
         "-D_POSIX_C_SOURCE=200809L", "-I", os.path.join(out, "src"),
         "-I", os.path.join(out, "include"), "-I", ours,
         os.path.join(ours, "m3_backend_hip.c")],
        capture_output=True, text=True)


def test_hip_backend_compiles_against_the_patched_reference(tmp_path):
    result = _compile(True, tmp_path)
    assert result.returncode == 0, result.stderr


def test_hip_backend_needs_the_patch(tmp_path):
    result = _compile(False, tmp_path)
    assert result.returncode != 0
    assert "M3_BACKEND_HIP" in result.stderr or "write" in result.stderr
