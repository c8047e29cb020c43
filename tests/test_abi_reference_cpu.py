"""include/*.h against the reference's own headers (CPU).

tests/golden/abi_reference.json holds sizeof/offsetof of every public and
plug-in struct, every enum value and the capacity macros of the
reference's headers (written by tests/golden/make_abi_fixture.py from
include/m3.h and src/m3_backend_internal.h of the reference tree). The
same probe compiled against this library's include/ must give the same
numbers; only the size of the backend vtable may grow, because this
library appends hooks after the reference's four.
"""
import json
import os
import sys

from conftest import ROOT

sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))

from abi_probe import GROWN, run_probe  # noqa: E402

FIXTURE = os.path.join(ROOT, "tests", "golden", "abi_reference.json")


def test_headers_match_the_reference_layouts_and_values():
    reference = json.load(open(FIXTURE))["values"]
    ours = run_probe([os.path.join(ROOT, "include")],
                     ["m3.h", "m3_backend.h"])
    assert set(ours) == set(reference)
    differ = {key: (ours[key], reference[key]) for key in reference
              if ours[key] != reference[key] and key not in GROWN}
    assert not differ, differ
    assert ours["sizeof m3_backend_vtable"] >= \
        reference["sizeof m3_backend_vtable"]


def test_probe_tells_layouts_apart(tmp_path):
    """A header with one field moved gives a different probe: the
    comparison above can fail."""
    header = tmp_path / "moved.h"
    source = open(os.path.join(ROOT, "include", "m3.h")).read()
    moved = source.replace("    bool allow_metal;\n    bool allow_cpu;",
                           "    bool allow_cpu;\n    bool allow_metal;")
    assert moved != source
    header.write_text(moved)
    (tmp_path / "m3.h").write_text(moved)
    ours = run_probe([str(tmp_path), os.path.join(ROOT, "include")],
                     ["m3.h", "m3_backend.h"])
    reference = json.load(open(FIXTURE))["values"]
    assert ours["offsetof m3_session_options.allow_metal"] != \
        reference["offsetof m3_session_options.allow_metal"]
