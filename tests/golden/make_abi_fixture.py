"""Writes tests/golden/abi_reference.json: the plug-in ABI (struct sizes
and offsets, enum values, capacities) of the reference's own headers,
probed by compiling tests/golden/abi_probe.py's program against
include/m3.h and src/m3_backend_internal.h of the reference tree (which
bring in src/m3_backend.h, src/m3_op.h, src/m3_tensor.h, src/m3_scratch.h
and src/m3_error.h). Run in a container that has the reference:

    python tests/golden/make_abi_fixture.py [/root/reference]
"""
import json
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from abi_probe import run_probe  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)),
                   "abi_reference.json")


def main():
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    values = run_probe([os.path.join(root, "include"),
                        os.path.join(root, "src")],
                       ["m3.h", "m3_backend_internal.h"])
    with open(OUT, "w") as handle:
        json.dump({"source": "reference include/m3.h, src/m3_backend.h, "
                             "src/m3_backend_internal.h, src/m3_op.h, "
                             "src/m3_tensor.h, src/m3_scratch.h, "
                             "src/m3_error.h; x86-64 gcc",
                   "values": values}, handle, indent=1, sort_keys=True)
        handle.write("\n")
    print("wrote %d entries to %s" % (len(values), OUT))


if __name__ == "__main__":
    main()
