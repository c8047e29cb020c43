"""CPU checks of the element conversions and libm restatements that the
gfx950 kernels are compiled from (m3.c_amd/csrc/hip/m3_numeric.h and
m3_libm.h), using tests/csrc/numeric_tables.c built for the host.

* The four full conversion tables of the kernels' header and of the oracle
  hash to the values the reference's own CAST produced for every input
  (tests/golden/conversion_tables.json, written by
  tests/golden/make_conversion_tables.py from the compiled reference).
* The kernels' header and the oracle agree value by value on all inputs.
* m3_expf, m3_sinf, m3_expf_any, m3_expm1f and m3_tanhf equal the C
  library's expf, sinf, expm1f and tanhf (the functions the reference calls
  at src/m3_op_execute_basic.c:113,156,172,188,227, tanhf through expm1f)
  on every 7th float.
"""
import json
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCE = os.path.join(HERE, "csrc", "numeric_tables.c")
HEADERS = [os.path.join(ROOT, "m3.c_amd", "csrc", "hip", name)
           for name in ("m3_numeric.h", "m3_libm.h", "m3_activation.h")]
TOOL = os.path.join(HERE, "_build", "numeric_tables")


def build_checker():
    """Builds numeric_tables when it is missing or older than its sources."""
    newest = max(os.path.getmtime(p) for p in [SOURCE] + HEADERS)
    if not os.path.exists(TOOL) or os.path.getmtime(TOOL) < newest:
        os.makedirs(os.path.dirname(TOOL), exist_ok=True)
        subprocess.run(
            ["gcc", "-O2", "-std=c11", "-fopenmp", "-ffp-contract=off",
             "-mfma", "-Wall", "-Wextra", "-Werror", "-D_GNU_SOURCE",
             "-I" + os.path.join(ROOT, "m3.c_amd", "csrc", "hip"),
             "-o", TOOL, SOURCE, "-ldl", "-lm"], check=True)
    return TOOL


def run(*args):
    result = subprocess.run([build_checker()] + list(args),
                            capture_output=True, text=True, timeout=600)
    assert result.returncode == 0, result.stdout + result.stderr
    return json.loads(result.stdout)


@pytest.fixture(scope="module")
def reference_hashes():
    with open(os.path.join(HERE, "golden", "conversion_tables.json")) as f:
        return json.load(f)["hashes"]


def oracle_library():
    path = os.path.join(ROOT, "oracle", "liboracle.so")
    if not os.path.exists(path):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")],
                       check=True, capture_output=True)
    return path


def test_kernel_conversion_tables_match_reference(reference_hashes):
    assert run("tables", "product") == reference_hashes


def test_oracle_conversion_tables_match_reference(reference_hashes):
    assert run("tables", "oracle", oracle_library()) == reference_hashes


def test_kernel_and_oracle_conversions_agree_everywhere():
    assert run("compare", oracle_library())["conversion_mismatches"] == 0


def test_libm_restatements_match_c_library():
    result = run("libm", "7")
    assert result["expf_checked"] > 400_000_000
    assert result["expf_mismatches"] == 0
    assert result["sinf_mismatches"] == 0
    assert result["sinf_magnitude_checked"] > 300_000_000
    assert result["sinf_magnitude_mismatches"] == 0
    assert result["all_checked"] > 600_000_000
    assert result["expf_any_mismatches"] == 0
    assert result["expm1f_mismatches"] == 0
    assert result["tanhf_mismatches"] == 0
    assert result["tanhf_uniform_mismatches"] == 0
    assert result["gated_silu_mismatches"] == 0
    assert result["silu_fast_mismatches"] == 0


def test_gated_silu_16bit_gates_match_c_statements():
    result = run("silu16")
    assert result["silu16_checked"] == 2 * 65536 * 8
    assert result["silu16_mismatches"] == 0


def test_hash_discriminates_a_planted_rounding_error(reference_hashes):
    """One F32->F16 entry rounded the wrong way (input 0x3f800fff) changes
    that table's hash and no other."""
    hashes = run("tables", "planted")
    assert hashes["f32_to_f16"] != reference_hashes["f32_to_f16"]
    for name in ("f32_to_bf16", "f16_to_f32", "bf16_to_f32"):
        assert hashes[name] == reference_hashes[name]
