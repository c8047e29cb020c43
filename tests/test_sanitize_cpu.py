"""The host layer under AddressSanitizer and UndefinedBehaviorSanitizer
(CPU).

`make -C m3.c_amd sanitize` rebuilds the C11 host layer (graph builder,
session compiler, liveness plan, fusion planner, scheduler, CPU provider,
staging, storage) with -fsanitize=address,undefined; the host-layer suites
then run again in a child Python that preloads the ASan runtime and loads
that build (M3_LIBRARY_DIR), with the oracle test backend built with the
same sanitizers. Any report stops the child with a nonzero status. The
kernels are not part of this run: GPU code is not built with sanitizers.
"""
import os
import subprocess
import sys

import pytest

from conftest import ROOT

SUITES = ["tests/test_graph_cpu.py", "tests/test_cpu_provider.py",
          "tests/test_storage_cpu.py"]


def _runtime(name):
    path = subprocess.run(["gcc", "-print-file-name=" + name],
                          capture_output=True, text=True).stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


def test_host_layer_under_asan_and_ubsan():
    asan = _runtime("libasan.so")
    if asan is None:
        pytest.skip("gcc has no ASan runtime here")
    subprocess.run(["make", "-C", os.path.join(ROOT, "m3.c_amd"), "-j8",
                    "sanitize"], check=True, stdout=subprocess.DEVNULL)
    env = dict(os.environ)
    env.update({
        "M3_LIBRARY_DIR": os.path.join(ROOT, "m3.c_amd", "_build",
                                       "sanitize"),
        "M3_SANITIZE": "1",
        "LD_PRELOAD": asan,
        # the interpreter's own allocations are not ours to audit
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=0",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
    })
    # the child really runs the sanitized build with the runtime active
    probe = subprocess.run(
        [sys.executable, "-c",
         "import ctypes, importlib.util, sys\n"
         "spec = importlib.util.spec_from_file_location('m3c_amd', "
         "'m3.c_amd/__init__.py')\n"
         "m = importlib.util.module_from_spec(spec)\n"
         "spec.loader.exec_module(m)\n"
         "m.load()\n"
         "maps = open('/proc/self/maps').read()\n"
         "print('sanitize/libm3.so' in maps, "
         "hasattr(ctypes.CDLL(None), '__asan_init'))\n"],
        cwd=ROOT, env=env, capture_output=True, text=True, timeout=300)
    assert probe.stdout.split() == ["True", "True"], probe.stdout + \
        probe.stderr[-3000:]
    result = subprocess.run(
        [sys.executable, "-m", "pytest", "-x", "-q", "-m", "not gpu",
         "-p", "no:cacheprovider"] + SUITES,
        cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    tail = (result.stdout + result.stderr)[-6000:]
    assert result.returncode == 0, tail
    assert "runtime error" not in result.stderr, tail
    assert "ERROR: AddressSanitizer" not in result.stderr, tail
