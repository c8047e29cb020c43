"""The C-ABI libraries load and export every function their headers declare
(CPU only: no compute call is made)."""
import ctypes
import os
import re
import subprocess

import pytest

from conftest import ROOT, m3

HEADERS = {
    "libm3.so": ["m3.h", "m3_backend.h", "m3_backend_hip.h", "m3_rng.h"],
    "libm3_hip.so": ["m3_hip.h"],
}


def declared_functions(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set()
    for match in re.finditer(r"\b(m3_\w+)\s*\(", text):
        name = match.group(1)
        before = text[:match.start()].rstrip()
        # declarations follow a return type, not an operator or '('
        if before.endswith(("(", ",", "=", "return")):
            continue
        if text[match.end():].lstrip().startswith("*"):
            continue  # a return type followed by a function-pointer name
        names.add(name)
    # function-pointer typedef names are not symbols
    return {n for n in names if n not in {"m3_backend_factory"}}


@pytest.mark.parametrize("library", sorted(HEADERS))
def test_library_exports_every_declared_function(library):
    lib = ctypes.CDLL(os.path.join(ROOT, "m3.c_amd", library))
    missing = []
    for header in HEADERS[library]:
        for name in sorted(declared_functions(header)):
            if not hasattr(lib, name):
                missing.append("%s (%s)" % (name, header))
    assert not missing, missing


def test_python_export_lists_cover_headers():
    declared = set()
    for header in HEADERS["libm3.so"]:
        declared |= declared_functions(header)
    assert declared <= set(m3.EXPORTS_M3), declared - set(m3.EXPORTS_M3)
    assert declared_functions("m3_hip.h") <= set(m3.EXPORTS_HIP)


def test_struct_layouts_match_ctypes_mirrors(tmp_path):
    """sizeof/offsetof of the public structs, compiled with gcc against
    include/, equal the ctypes mirrors used by the tests and bench."""
    source = tmp_path / "layout.c"
    source.write_text(r'''
#include "m3_backend.h"
#include "m3_hip.h"
#include "m3_rng.h"
#include <stddef.h>
#include <stdio.h>
int main(void) {
    printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\n",
           sizeof(m3_error), sizeof(m3_graph_value_desc),
           sizeof(m3_graph_node_desc), sizeof(m3_session_options),
           sizeof(m3_session_plan_info), sizeof(m3_tensor_view),
           sizeof(m3_command), sizeof(m3_hip_view),
           sizeof(m3_hip_kernel_time), sizeof(m3_rng),
           sizeof(m3_backend_info));
    printf("%zu %zu %zu %zu\n", offsetof(m3_graph_value_desc, role),
           offsetof(m3_graph_node_desc, parameters),
           offsetof(m3_tensor_view, storage),
           offsetof(m3_command, descriptor));
    return 0;
}
''')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"),
                    str(source), "-o", str(exe)], check=True)
    sizes, offsets = subprocess.run([str(exe)], check=True,
                                    capture_output=True,
                                    text=True).stdout.split("\n")[:2]
    c = [int(v) for v in sizes.split()]
    py = [ctypes.sizeof(t) for t in (
        m3.Error, m3.ValueDesc, m3.NodeDesc, m3.SessionOptions, m3.PlanInfo,
        m3.TensorView, m3.Command, m3.HipView, m3.HipKernelTime, m3.Rng,
        m3.BackendInfo)]
    assert c == py
    assert [int(v) for v in offsets.split()] == [
        m3.ValueDesc.role.offset, m3.NodeDesc.parameters.offset,
        m3.TensorView.storage.offset, m3.Command.descriptor.offset]


def test_device_count_without_gpu_is_safe():
    # Counting devices never fails; on a machine without a GPU it is 0.
    assert m3.hip_device_count() >= 0
