"""The one-read softmax for rows of 2,049 to 32,768 columns (GPU).

m3_softmax_wide_kernel computes the reference's left-to-right F32 row sum
(src/m3_op_execute_basic.c:124-180) without a chain of one addition per
column: inside a binade of the running sum each step is an integer step on
that binade's grid, so most 64-column segments advance the sum by one
integer addition and the rest (the first one, binade crossings, exact
ties, wrong guesses) are summed column by column. Every case here is
checked against the oracle bit for bit, with rows built to exercise both
forms: ordinary logits at several spreads, causal masks, long runs of
zeros (equal maxima, e = 1, so the sum crosses many powers of two at
exact integers), a late maximum (tiny sums over a long prefix), values that
underflow to subnormal e, special rows (all -inf, +inf entries), 16-bit
input and output, padded and in-place rows.
"""
import os
import sys

import numpy as np
import pytest

from conftest import m3
from harness import HipFixture, ViewSpec, as_bytes, run_oracle

pytestmark = pytest.mark.gpu

WIDTHS = [2052, 3000, 4096, 4100, 6000, 8192, 8196, 12000, 16384, 16388,
          24000, 32768]


@pytest.fixture(scope="module")
def hip(gpu):
    fixture = HipFixture()
    yield fixture
    fixture.close()


def compare(hip, storages, views, name):
    print("gpu case", name, flush=True, file=sys.stderr)
    status, got, message = hip.run(m3.OP_SOFTMAX, storages, views)
    ostatus, expected = run_oracle(m3.OP_SOFTMAX, storages, views)
    assert status == ostatus, (name, m3.status_name(status), message)
    for index, (a, b) in enumerate(zip(got, expected)):
        if bytes(a) != bytes(b):
            diff = np.flatnonzero(a != b)
            raise AssertionError("%s: storage %d differs at %d bytes, first "
                                 "at byte %d" % (name, index, diff.size,
                                                 diff[0]))


def wide_rows(rng, rows, width):
    """Rows of every kind the kernel distinguishes, cycling through them."""
    out = np.empty((rows, width), np.float32)
    for r in range(rows):
        kind = r % 12
        row = out[r]
        if kind in (0, 1, 2):
            row[:] = rng.standard_normal(width) * (0.1, 3.0, 30.0)[kind]
        elif kind == 3:  # causal: a random number of finite entries
            row[:] = rng.standard_normal(width) * 3
            row[1 + int(rng.integers(0, width)):] = -np.inf
        elif kind == 4:  # equal maxima: e = 1 in every column
            row[:] = 0.0
        elif kind == 5:  # zeros and a few larger values
            row[:] = 0.0
            row[rng.integers(0, width, 8)] = 3.0
        elif kind == 6:  # the maximum last: tiny sums over the prefix
            row[:] = rng.standard_normal(width) * 2 - 40.0
            row[-1] = 5.0
        elif kind == 7:  # spread so wide that e underflows to subnormals
            row[:] = rng.standard_normal(width) * 60
        elif kind == 8:  # all -inf
            row[:] = -np.inf
        elif kind == 9:  # +inf entries
            row[:] = rng.standard_normal(width)
            row[rng.integers(0, width, 3)] = np.inf
        elif kind == 10:  # one finite entry
            row[:] = -np.inf
            row[int(rng.integers(0, width))] = -7.5
        else:  # logits on a coarse grid: e values with few bits
            row[:] = np.round(rng.standard_normal(width) * 4) * np.float32(
                np.log(2.0))
    return out


@pytest.mark.parametrize("width", WIDTHS)
def test_wide_rows_f32(hip, width):
    rng = np.random.default_rng(21000 + width)
    rows = 24
    logits = wide_rows(rng, rows, width)
    compare(hip, [as_bytes(logits), np.zeros(logits.nbytes, np.uint8)],
            [ViewSpec(0, m3.F32, (rows, width)),
             ViewSpec(1, m3.F32, (rows, width))],
            "softmax wide w=%d" % width)


def source_of(logits, dtype):
    if dtype == m3.F16:
        return as_bytes(logits.astype(np.float16).view(np.uint16))
    if dtype == m3.BF16:
        return as_bytes((logits.view(np.uint32) >> 16).astype(np.uint16))
    return as_bytes(logits)


@pytest.mark.parametrize("dtypes", [(m3.BF16, m3.BF16), (m3.F16, m3.F32),
                                    (m3.F32, m3.BF16)])
@pytest.mark.parametrize("width", [4096, 16384, 32768])
def test_wide_rows_16bit(hip, dtypes, width):
    rng = np.random.default_rng(22000 + width + 31 * dtypes[0] + dtypes[1])
    rows = 12
    logits = wide_rows(rng, rows, width)
    compare(hip, [source_of(logits, dtypes[0]),
                  np.zeros(rows * width * m3.DTYPE_SIZES[dtypes[1]],
                           np.uint8)],
            [ViewSpec(0, dtypes[0], (rows, width)),
             ViewSpec(1, dtypes[1], (rows, width))],
            "softmax wide %s w=%d" % (dtypes, width))


def test_wide_rows_padded_and_in_place(hip):
    rng = np.random.default_rng(23)
    width = 10000
    logits = wide_rows(rng, 12, width)
    padded = np.full((12, width + 64), 5.0, np.float32)
    padded[:, :width] = logits
    compare(hip, [as_bytes(padded), np.zeros(logits.nbytes, np.uint8)],
            [ViewSpec(0, m3.F32, (12, width), ((width + 64) * 4, 4)),
             ViewSpec(1, m3.F32, (12, width))], "softmax wide padded")
    compare(hip, [as_bytes(logits)],
            [ViewSpec(0, m3.F32, (12, width)),
             ViewSpec(0, m3.F32, (12, width))], "softmax wide in place")
    batched = wide_rows(rng, 3 * 4, 4096).reshape(3, 4, 4096)
    compare(hip, [as_bytes(batched), np.zeros(batched.nbytes, np.uint8)],
            [ViewSpec(0, m3.F32, (3, 4, 4096)),
             ViewSpec(1, m3.F32, (3, 4, 4096))], "softmax wide rank 3")


def test_wide_rows_subnormal_ties(hip):
    """Quotients on F32 subnormal rounding midpoints (e_j / sum =
    (2k+1) 2^-150) round to even in the wide kernel too."""
    from harness import subnormal_tie_rows
    rng = np.random.default_rng(24)
    logits = subnormal_tie_rows(rng, 24, 8192)
    compare(hip, [as_bytes(logits), np.zeros(logits.nbytes, np.uint8)],
            [ViewSpec(0, m3.F32, (24, 8192)),
             ViewSpec(1, m3.F32, (24, 8192))], "softmax wide ties")


def unstaged_rows(rng, rows, width, near=3600):
    """A maximum in column 0 (e = 1), then thousands of columns of e near
    5e-7, so that the running sum stays within 1/256 of 1 for `near` / 64
    64-column segments or more, then e near 0.05, so that the sum crosses
    2, 4, 8, ... in the segments after them."""
    out = np.empty((rows, width), np.float32)
    for r in range(rows):
        n1 = near + 300 * (r % 4)
        row = out[r]
        row[0] = 0.0
        row[1:n1] = -14.5 + 0.01 * rng.standard_normal(n1 - 1)
        row[n1:] = np.minimum(rng.standard_normal(width - n1) - 3.0, -1.0)
    return out


@pytest.mark.parametrize("width,lines,near", [(4096, 32, 2200),
                                              (16384, 48, 3600),
                                              (32768, 48, 3600)])
def test_wide_rows_unstaged_segments(hip, width, lines, near):
    """The kernel keeps in LDS the exponentials of at most 48 segments per
    row (32 for rows of at most 4,096 columns) that the in-order sum may
    have to add column by column (those whose estimated running sum lies
    within 1/256 of a power of two, or crosses one, and those holding a
    tie). These rows have more such segments than that, and the sum crosses
    powers of two in segments after them: the walk forms those segments'
    exponentials again from the input."""
    rng = np.random.default_rng(25000 + width)
    rows = 16
    logits = unstaged_rows(rng, rows, width, near)
    # the rows are what the test needs (float64 running sums suffice to
    # count segments near 1 and the powers of two crossed after them)
    e = np.exp(logits.astype(np.float64) - 0.0)
    s = np.cumsum(e, axis=1)[:, 63::64]
    assert ((s < 1.0 + 1.0 / 256.0).sum(axis=1) > lines).all()
    assert (np.floor(np.log2(s[:, -1])) >= 6).all()
    compare(hip, [as_bytes(logits), np.zeros(logits.nbytes, np.uint8)],
            [ViewSpec(0, m3.F32, (rows, width)),
             ViewSpec(1, m3.F32, (rows, width))],
            "softmax wide unstaged w=%d" % width)


@pytest.fixture(scope="module")
def hip_capped(gpu):
    """A HIP backend whose long-row softmax launches at most 37 workgroups
    (M3_HIP_SOFTMAX_WIDE_GRID, read when the device opens), so that each
    workgroup takes several rows in turn: its LDS words, lines, slot count
    and ready tags are used again from row to row, which launches of one
    workgroup per row (up to 2^20 rows) never do."""
    saved = os.environ.get("M3_HIP_SOFTMAX_WIDE_GRID")
    os.environ["M3_HIP_SOFTMAX_WIDE_GRID"] = "37"
    try:
        fixture = HipFixture()
    finally:
        if saved is None:
            del os.environ["M3_HIP_SOFTMAX_WIDE_GRID"]
        else:
            os.environ["M3_HIP_SOFTMAX_WIDE_GRID"] = saved
    yield fixture
    fixture.close()


@pytest.mark.parametrize("dtypes", [(m3.F32, m3.F32), (m3.BF16, m3.F32)])
@pytest.mark.parametrize("width", [2052, 8192, 16384, 32768])
def test_wide_rows_several_per_workgroup(hip_capped, dtypes, width):
    """150 rows of every kind (special rows among them) on 37 workgroups:
    each workgroup sums four or five rows one after another."""
    rng = np.random.default_rng(26000 + width + 7 * dtypes[0])
    rows = 150
    logits = wide_rows(rng, rows, width)
    compare(hip_capped, [source_of(logits, dtypes[0]),
                         np.zeros(logits.nbytes, np.uint8)],
            [ViewSpec(0, dtypes[0], (rows, width)),
             ViewSpec(1, dtypes[1], (rows, width))],
            "softmax wide, 37 workgroups %s w=%d" % (dtypes, width))


def test_wide_rows_full_size(hip):
    """[4096, 16384] F32 logits ~ N(0, 3), the benchmark's long-row shape,
    every element against the oracle."""
    logits = m3.rng_fill("normal", 4096 * 16384, seed=1, a=3.0).reshape(
        4096, 16384)
    compare(hip, [as_bytes(logits), np.zeros(logits.nbytes, np.uint8)],
            [ViewSpec(0, m3.F32, (4096, 16384)),
             ViewSpec(1, m3.F32, (4096, 16384))], "softmax wide full size")
