"""Every F32 input of TANH and of GATED_SILU's gate through the HIP provider
(GPU).

All 2^32 bit patterns, in chunks of 2^26, run through the vector kernels
(contiguous, aligned F32) and are compared bit for bit, NaN payloads
included, with the oracle, which calls the C library's tanhf and expf as the
reference's CPU provider does. GATED_SILU takes up = 1, so its output is
the activation itself. This pins the kernels' straight-line tanhf and their
division without operand scaling (m3_div_normal) on every input, beyond the
host-side checks of the same element functions in test_numeric_cpu.py,
which use the host's division.
"""
import sys
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from conftest import m3
from harness import HipFixture, ViewSpec, as_bytes, run_oracle

pytestmark = pytest.mark.gpu

CHUNK = 1 << 26
PIECES = 16  # oracle threads per chunk (ctypes releases the GIL)


@pytest.fixture(scope="module")
def hip(gpu):
    fixture = HipFixture()
    yield fixture
    fixture.close()


def oracle_chunk(pool, kind, arrays):
    """The oracle over one chunk, split into PIECES contiguous pieces."""
    step = CHUNK // PIECES

    def piece(index):
        part = [as_bytes(a[index * step:(index + 1) * step]) for a in arrays]
        part.append(np.zeros(4 * step, np.uint8))
        views = [ViewSpec(i, m3.F32, (step,)) for i in range(len(part))]
        status, out = run_oracle(kind, part, views)
        assert status == m3.OK
        return out[-1].view(np.uint32)

    return np.concatenate(list(pool.map(piece, range(PIECES))))


@pytest.mark.parametrize("kind", [m3.OP_TANH, m3.OP_GATED_SILU],
                         ids=["tanh", "gated_silu"])
def test_every_f32_input(hip, kind):
    ones = np.ones(CHUNK, np.float32)
    mismatches = 0
    with ThreadPoolExecutor(PIECES) as pool:
        for chunk in range((1 << 32) // CHUNK):
            start = chunk * CHUNK
            print("exhaustive kind", kind, "chunk", chunk, "of 64", flush=True,
                  file=sys.stderr)
            bits = (np.arange(CHUNK, dtype=np.uint64) + start).astype(
                np.uint32)
            arrays = [bits] if kind == m3.OP_TANH else [bits, ones]
            storages = [as_bytes(a) for a in arrays]
            storages.append(np.zeros(4 * CHUNK, np.uint8))
            views = [ViewSpec(i, m3.F32, (CHUNK,))
                     for i in range(len(storages))]
            status, out, message = hip.run(kind, storages, views)
            assert status == m3.OK, message
            expected = oracle_chunk(pool, kind, arrays)
            mismatches += int(np.count_nonzero(
                out[-1].view(np.uint32) != expected))
    assert mismatches == 0
