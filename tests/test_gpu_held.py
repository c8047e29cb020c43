"""The held forms of the F32 binary kernel and of the cheap casts (GPU).

Tensors large enough to fill the device, and small enough for all of its
workgroups to be resident at once, run a kernel that loads everything,
waits, then stores (m3_binary_held_kernel, m3_cast_held_kernel): on one
MI355X, F32 binaries of about 6.3M-12.6M elements and F16/BF16 -> F32 and
F32 -> BF16 casts of about 8.4M-16.8M elements. Smaller tensors (the other
parity tests) and larger ones run the streaming kernels. Every case here is
compared with the oracle bit for bit, NaN payloads, infinities, signed
zeros, subnormals and the tail of a count that is not a multiple of four
included; one cast above the held range checks the streaming form at the
same dtypes.
"""
import sys

import numpy as np
import pytest

from conftest import m3
from harness import HipFixture, ViewSpec, as_bytes, run_oracle

pytestmark = pytest.mark.gpu

SPECIALS32 = np.array([0x00000000, 0x80000000, 0x7f800000, 0xff800000,
                       0x7fc00000, 0xffc12345, 0x7f800001, 0x00000001,
                       0x807fffff, 0x3f800000, 0x477ff000, 0x477fefff,
                       0x38800000, 0x387fffff, 0x33000000, 0x7f7fffff,
                       0x3f808000, 0x3f818000], np.uint32)


@pytest.fixture(scope="module")
def hip(gpu):
    fixture = HipFixture()
    yield fixture
    fixture.close()


def compare(hip, kind, storages, views, name):
    print("gpu case", name, flush=True, file=sys.stderr)
    status, got, message = hip.run(kind, storages, views)
    ostatus, expected = run_oracle(kind, storages, views)
    assert status == ostatus, (name, m3.status_name(status), message)
    for index, (a, b) in enumerate(zip(got, expected)):
        if bytes(a) != bytes(b):
            diff = np.flatnonzero(a != b)
            raise AssertionError("%s: storage %d differs at %d bytes, first "
                                 "at byte %d" % (name, index, diff.size,
                                                 diff[0]))


def random_f32(rng, count, specials=0.05):
    values = (rng.standard_normal(count) * 4).astype(np.float32)
    bits = values.view(np.uint32)
    pick = rng.random(count) < specials
    bits[pick] = rng.choice(SPECIALS32, size=int(pick.sum()))
    return bits.view(np.float32)


BINARY_CASES = [
    # (left shape, right shape): both full with a tail of 3, a trailing
    # broadcast (the benchmark's class), a scalar
    ((9437187,), (9437187,)),
    ((3, 2048, 1539), (1539,)),
    ((7340033,), (1,)),
]


@pytest.mark.parametrize("op", [m3.OP_ADD, m3.OP_MUL, m3.OP_SUB, m3.OP_DIV])
@pytest.mark.parametrize("case", range(len(BINARY_CASES)))
def test_held_binary_f32(hip, op, case):
    rng = np.random.default_rng(7000 + 10 * op + case)
    left_shape, right_shape = BINARY_CASES[case]
    left = random_f32(rng, int(np.prod(left_shape)))
    right = random_f32(rng, int(np.prod(right_shape)))
    views = [ViewSpec(0, m3.F32, left_shape),
             ViewSpec(1, m3.F32, right_shape),
             ViewSpec(2, m3.F32, left_shape)]
    compare(hip, op, [as_bytes(left), as_bytes(right),
                      np.zeros(left.nbytes, np.uint8)], views,
            "held binary op%d %s x %s" % (op, left_shape, right_shape))


def sixteen_bit_source(rng, count):
    """Every 16-bit pattern, then random ones."""
    every = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    rest = rng.integers(0, 1 << 16, size=count - every.size,
                        dtype=np.uint32).astype(np.uint16)
    return np.concatenate([every, rest])


@pytest.mark.parametrize("count", [10000003, 20000001])
@pytest.mark.parametrize("pair", [(m3.F16, m3.F32), (m3.BF16, m3.F32),
                                  (m3.F32, m3.BF16), (m3.F32, m3.F16)])
def test_held_casts(hip, pair, count):
    rng = np.random.default_rng(8000 + 17 * pair[0] + pair[1] + count % 7)
    source_dtype, out_dtype = pair
    if source_dtype == m3.F32:
        source = as_bytes(random_f32(rng, count))
    else:
        source = as_bytes(sixteen_bit_source(rng, count))
    out_bytes = count * m3.DTYPE_SIZES[out_dtype]
    compare(hip, m3.OP_CAST, [source, np.zeros(out_bytes, np.uint8)],
            [ViewSpec(0, source_dtype, (count,)),
             ViewSpec(1, out_dtype, (count,))],
            "held cast %s %d" % (pair, count))
