"""Writes conversion_tables.json: hashes of the reference's own CAST tables.

Runs tests/csrc/numeric_tables.c in its "tables reference" mode against the
reference CPU provider compiled from its sources (oracle/_ref/libm3ref.so,
built by `make -C oracle ref` where the reference tree is present). The
tables are F32->F16 and F32->BF16 over all 2^32 F32 bit patterns and
F16->F32 and BF16->F32 over all 2^16 patterns; the hash is described in
numeric_tables.c. The fixture is data: it holds only the four hashes.

Usage: python tests/golden/make_conversion_tables.py
"""
import json
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(HERE))

from test_numeric_cpu import build_checker  # noqa: E402


def main():
    ref = os.path.join(ROOT, "oracle", "_ref", "libm3ref.so")
    if not os.path.exists(ref):
        print("oracle/_ref/libm3ref.so is not built", file=sys.stderr)
        return 1
    tool = build_checker()
    out = subprocess.run([tool, "tables", "reference", ref], check=True,
                         capture_output=True, text=True).stdout
    hashes = json.loads(out)
    fixture = {
        "description": "FNV-1a block hashes of the reference CPU provider's "
                       "CAST tables (src/m3_op_execute_basic.c:28-59 over "
                       "src/m3_op_numeric.c:27-130): F32->F16 and F32->BF16 "
                       "for all 2^32 inputs, F16->F32 and BF16->F32 for all "
                       "2^16 inputs",
        "generator": "tests/golden/make_conversion_tables.py",
        "hashes": hashes,
    }
    with open(os.path.join(HERE, "conversion_tables.json"), "w") as handle:
        json.dump(fixture, handle, indent=1)
        handle.write("\n")
    print(json.dumps(hashes))
    return 0


if __name__ == "__main__":
    sys.exit(main())
