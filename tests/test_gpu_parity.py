"""Randomised parity of the HIP provider with the oracle (GPU).

Seeded inputs at sizes the oracle finishes in well under a second; every
launch path of every kernel family is hit (vector fast paths, tails,
broadcast classes, strided general paths, 16-bit dtypes, aliasing). The
bar is bit-exact output and equal status for every case, including NaN
payloads, infinities, signed zeros and subnormals in the inputs.
"""
import os
import sys

import numpy as np
import pytest

from conftest import m3
from harness import (HipFixture, ViewSpec, as_bytes, run_oracle,
                     subnormal_tie_rows)

pytestmark = pytest.mark.gpu

SPECIALS32 = np.array([0x00000000, 0x80000000, 0x7f800000, 0xff800000,
                       0x7fc00000, 0xffc12345, 0x7f800001, 0x00000001,
                       0x807fffff, 0x3f800000, 0x477ff000, 0x477fefff,
                       0x38800000, 0x387fffff, 0x33000000, 0x33000001,
                       0x7f7fffff, 0x3f801000, 0x3f803000], np.uint32)


@pytest.fixture(scope="module")
def hip(gpu):
    fixture = HipFixture()
    yield fixture
    fixture.close()


def random_f32(rng, count, scale=4.0, specials=0.05):
    values = (rng.standard_normal(count) * scale).astype(np.float32)
    bits = values.view(np.uint32)
    pick = rng.random(count) < specials
    bits[pick] = rng.choice(SPECIALS32, size=int(pick.sum()))
    return bits.view(np.float32)


def random_bits16(rng, count):
    return rng.integers(0, 1 << 16, size=count, dtype=np.uint32).astype(
        np.uint16)


def storage_for(rng, dtype, count, specials=0.05):
    if dtype == m3.F32:
        return as_bytes(random_f32(rng, count, specials=specials))
    if dtype == m3.I32:
        return as_bytes(rng.integers(-2**31, 2**31, size=count,
                                     dtype=np.int64).astype(np.int32))
    if dtype == m3.F16:
        values = (rng.standard_normal(count) * 4).astype(np.float16)
        bits = values.view(np.uint16)
        pick = rng.random(count) < specials
        bits[pick] = random_bits16(rng, int(pick.sum()))
        return as_bytes(bits)
    values = (rng.standard_normal(count) * 4).astype(np.float32)
    bits = (values.view(np.uint32) >> 16).astype(np.uint16)
    pick = rng.random(count) < specials
    bits[pick] = random_bits16(rng, int(pick.sum()))
    return as_bytes(bits)


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


def nbytes(spec):
    if spec.count() == 0:
        return 0
    last = spec.offset + sum((d - 1) * s for d, s in
                             zip(spec.shape, spec.byte_strides()))
    return last + m3.DTYPE_SIZES[spec.dtype]


# ---- binary -----------------------------------------------------------------

BINARY_LAYOUTS = [
    # (left shape, right shape, output shape)
    ((8, 64, 96), (96,), (8, 64, 96)),          # trailing broadcast
    ((8, 64, 96), (8, 64, 96), (8, 64, 96)),    # full x full
    ((8, 64, 96), (1,), (8, 64, 96)),           # scalar
    ((3, 40, 100), (40, 1), (3, 40, 100)),      # row broadcast, inner 100
    ((3, 40, 6), (40, 1), (3, 40, 6)),          # periodic, inner 6
    ((5, 7, 9), (7, 1), (5, 7, 9)),             # periodic, odd sizes
    ((4, 1, 33), (1, 5, 33), (4, 5, 33)),       # two-sided broadcast
    ((1000003,), (1000003,), (1000003,)),       # odd length, tail
    ((2, 3, 4, 5, 6), (1, 3, 1, 5, 1), (2, 3, 4, 5, 6)),  # general
    ((), (), ()),                               # rank zero
    ((7,), (), (7,)),                           # rank-zero right
    ((4, 262), (262,), (4, 262)),               # period not a multiple of 4
]


@pytest.mark.parametrize("op", [m3.OP_ADD, m3.OP_MUL, m3.OP_SUB, m3.OP_DIV])
@pytest.mark.parametrize("layout", range(len(BINARY_LAYOUTS)))
def test_binary_f32_layouts(hip, op, layout):
    rng = np.random.default_rng(1000 + 10 * op + layout)
    ls, rs, os_ = BINARY_LAYOUTS[layout]
    views = [ViewSpec(0, m3.F32, ls), ViewSpec(1, m3.F32, rs),
             ViewSpec(2, m3.F32, os_)]
    storages = [storage_for(rng, m3.F32, views[0].count()),
                storage_for(rng, m3.F32, views[1].count()),
                np.zeros(nbytes(views[2]), np.uint8)]
    compare(hip, op, storages, views, "binary op%d layout%d" % (op, layout))


@pytest.mark.parametrize("dtypes", [(m3.F16, m3.F16, m3.F16),
                                    (m3.BF16, m3.BF16, m3.BF16),
                                    (m3.F32, m3.BF16, m3.F16),
                                    (m3.F16, m3.F32, m3.BF16),
                                    (m3.BF16, m3.F16, m3.F32)])
@pytest.mark.parametrize("layout", [0, 1, 3, 4, 7, 8])
def test_binary_mixed_dtypes(hip, dtypes, layout):
    rng = np.random.default_rng(2000 + layout + 7 * sum(dtypes))
    ls, rs, os_ = BINARY_LAYOUTS[layout]
    views = [ViewSpec(0, dtypes[0], ls), ViewSpec(1, dtypes[1], rs),
             ViewSpec(2, dtypes[2], os_)]
    storages = [storage_for(rng, dtypes[0], views[0].count()),
                storage_for(rng, dtypes[1], views[1].count()),
                np.zeros(nbytes(views[2]), np.uint8)]
    for op in (m3.OP_ADD, m3.OP_MUL, m3.OP_SUB, m3.OP_DIV):
        compare(hip, op, storages, views,
                "binary %s layout%d op%d" % (dtypes, layout, op))


def test_binary_strided_and_offset_views(hip):
    rng = np.random.default_rng(3)
    # left: transposed [64, 48] view of a [48, 64] buffer at a 4-byte
    # offset; right: every other element of a [96] buffer.
    left = ViewSpec(0, m3.F32, (64, 48), (4, 256), 4)
    right = ViewSpec(1, m3.F32, (48,), (8,), 0)
    out = ViewSpec(2, m3.F32, (64, 48))
    storages = [storage_for(rng, m3.F32, 48 * 64 + 1),
                storage_for(rng, m3.F32, 96),
                np.zeros(nbytes(out), np.uint8)]
    for op in (m3.OP_ADD, m3.OP_MUL, m3.OP_SUB, m3.OP_DIV):
        compare(hip, op, storages, [left, right, out], "strided op%d" % op)


def test_binary_exact_alias_in_place(hip):
    rng = np.random.default_rng(4)
    shape = (16, 1000)
    storages = [storage_for(rng, m3.F32, 16000),
                storage_for(rng, m3.F32, 1000)]
    views = [ViewSpec(0, m3.F32, shape), ViewSpec(1, m3.F32, (1000,)),
             ViewSpec(0, m3.F32, shape)]
    compare(hip, m3.OP_MUL, storages, views, "in-place mul")


# ---- cast / copy -------------------------------------------------------------

DTYPES = [m3.F32, m3.F16, m3.BF16, m3.I32]


@pytest.mark.parametrize("src", DTYPES)
@pytest.mark.parametrize("dst", DTYPES)
@pytest.mark.parametrize("count", [1, 3, 4, 1021, 65536 + 7])
def test_cast_all_pairs(hip, src, dst, count):
    rng = np.random.default_rng(5000 + 97 * src + 13 * dst + count)
    storages = [storage_for(rng, src, count, specials=0.2),
                np.zeros(count * m3.DTYPE_SIZES[dst], np.uint8)]
    views = [ViewSpec(0, src, (count,)), ViewSpec(1, dst, (count,))]
    if src != m3.I32 and dst == m3.I32:
        # valid in-range values (the invalid case is a preflight test)
        values = rng.uniform(-2e9, 2e9, count).astype(np.float32)
        if src == m3.F32:
            storages[0] = as_bytes(values)
        elif src == m3.F16:
            storages[0] = as_bytes(rng.uniform(-6e4, 6e4, count).astype(
                np.float16).view(np.uint16))
        else:
            storages[0] = as_bytes((values.view(np.uint32) >> 16).astype(
                np.uint16))
    kind = m3.OP_COPY if src == dst else m3.OP_CAST
    compare(hip, kind, storages, views, "cast %d->%d n=%d" % (src, dst, count))


def test_cast_exhaustive_16bit_sources(hip):
    """All 65536 half and bfloat16 bit patterns to every other dtype."""
    bits = as_bytes(np.arange(1 << 16, dtype=np.uint32).astype(np.uint16))
    for src in (m3.F16, m3.BF16):
        for dst in (m3.F32, m3.F16, m3.BF16):
            if dst == src:
                continue
            views = [ViewSpec(0, src, (1 << 16,)),
                     ViewSpec(1, dst, (1 << 16,))]
            storages = [bits, np.zeros((1 << 16) * m3.DTYPE_SIZES[dst],
                                       np.uint8)]
            compare(hip, m3.OP_CAST, storages, views,
                    "exhaustive %d->%d" % (src, dst))


def test_cast_f32_dense_bit_sweep(hip):
    """Every 4099th F32 bit pattern (about a million, all classes) to F16
    and BF16."""
    bits = np.arange(0, 1 << 32, 4099, dtype=np.uint64).astype(np.uint32)
    for dst in (m3.F16, m3.BF16):
        views = [ViewSpec(0, m3.F32, (bits.size,)),
                 ViewSpec(1, dst, (bits.size,))]
        storages = [as_bytes(bits), np.zeros(bits.size * 2, np.uint8)]
        compare(hip, m3.OP_CAST, storages, views, "sweep ->%d" % dst)


def test_cast_strided_input(hip):
    rng = np.random.default_rng(6)
    for src, dst in ((m3.F32, m3.F16), (m3.BF16, m3.F32), (m3.I32, m3.BF16),
                     (m3.F16, m3.F16)):
        src_view = ViewSpec(0, src, (33, 17), (m3.DTYPE_SIZES[src],
                                               33 * m3.DTYPE_SIZES[src]))
        storages = [storage_for(rng, src, 33 * 17),
                    np.zeros(33 * 17 * m3.DTYPE_SIZES[dst], np.uint8)]
        kind = m3.OP_COPY if src == dst else m3.OP_CAST
        compare(hip, kind, storages, [src_view, ViewSpec(1, dst, (33, 17))],
                "strided cast %d->%d" % (src, dst))


# ---- softmax ------------------------------------------------------------------

def softmax_logits(rng, rows, width, causal=True, specials=True):
    values = (rng.standard_normal((rows, width)) * 3).astype(np.float32)
    if causal:
        mask = np.arange(width)[None, :] > (np.arange(rows)[:, None] %
                                            max(width, 1))
        values[mask] = -np.inf
    if specials and rows >= 4:
        values[0, :] = -np.inf
        values[1, ::3] = np.inf
        values[2, :] = 0.0
        values[3, :] = np.float32(1e-40)
    return values


@pytest.mark.parametrize("width", [1, 3, 4, 12, 64, 256, 260, 512, 1000,
                                   1024, 2048, 3000, 4096, 8192, 10000])
def test_softmax_widths(hip, width):
    rng = np.random.default_rng(7000 + width)
    rows = max(4, min(300, 300000 // width))
    logits = softmax_logits(rng, rows, width)
    views = [ViewSpec(0, m3.F32, (rows, width)),
             ViewSpec(1, m3.F32, (rows, width))]
    storages = [as_bytes(logits), np.zeros(logits.nbytes, np.uint8)]
    compare(hip, m3.OP_SOFTMAX, storages, views, "softmax w=%d" % width)


@pytest.mark.parametrize("dtypes", [(m3.F16, m3.F16), (m3.BF16, m3.BF16),
                                    (m3.F32, m3.F16), (m3.BF16, m3.F32)])
@pytest.mark.parametrize("width", [5, 256, 1024, 1500])
def test_softmax_dtypes(hip, dtypes, width):
    rng = np.random.default_rng(8000 + width + 17 * dtypes[0] + dtypes[1])
    rows = 64
    logits = softmax_logits(rng, rows, width)
    if dtypes[0] == m3.F16:
        source = as_bytes(logits.astype(np.float16).view(np.uint16))
    elif dtypes[0] == m3.BF16:
        source = as_bytes((logits.view(np.uint32) >> 16).astype(np.uint16))
    else:
        source = as_bytes(logits)
    views = [ViewSpec(0, dtypes[0], (rows, width)),
             ViewSpec(1, dtypes[1], (rows, width))]
    storages = [source, np.zeros(rows * width * m3.DTYPE_SIZES[dtypes[1]],
                                 np.uint8)]
    compare(hip, m3.OP_SOFTMAX, storages, views,
            "softmax %s w=%d" % (dtypes, width))


@pytest.mark.parametrize("width", [4, 200, 260, 1024, 2000, 4096, 6000])
def test_softmax_zero_tails(hip, width):
    """Rows whose e_j end in a run of zeros: -inf tails, finite tails that
    underflow expf to +0, masked blocks inside the row, and cut points at
    every offset inside a 256-column chunk."""
    rng = np.random.default_rng(11000 + width)
    rows = 96
    logits = (rng.standard_normal((rows, width)) * 3).astype(np.float32)
    for r in range(rows):
        cut = 1 + (r * 37 + int(rng.integers(0, width))) % width
        kind = r % 4
        if kind == 0:
            logits[r, cut:] = -np.inf
        elif kind == 1:
            logits[r, cut:] = np.float32(-200.0)
        elif kind == 2:
            logits[r, cut:] = -np.inf
            start = int(rng.integers(0, cut))
            logits[r, start:start + max(1, cut // 3)] = -np.inf
            logits[r, 0] = 1.0
        else:
            logits[r, : cut - 1] = -np.inf
    views = [ViewSpec(0, m3.F32, (rows, width)),
             ViewSpec(1, m3.F32, (rows, width))]
    storages = [as_bytes(logits), np.zeros(logits.nbytes, np.uint8)]
    compare(hip, m3.OP_SOFTMAX, storages, views, "softmax tails w=%d" % width)


@pytest.mark.parametrize("width", [100, 102, 128, 1024, 2048, 4096, 10000])
def test_softmax_subnormal_ties(hip, width):
    """Quotients that land exactly on a rounding midpoint of the F32
    subnormal range (e_j = sum * (2k+1) * 2^-150) round to even, as the
    reference's F32 division does, in every softmax kernel (widths 100,
    102 and 10000 run the general kernel, 128 to 2048 the rows kernel,
    4096 the tiled one)."""
    rng = np.random.default_rng(13000 + width)
    rows = 96
    logits = subnormal_tie_rows(rng, rows, width)
    views = [ViewSpec(0, m3.F32, (rows, width)),
             ViewSpec(1, m3.F32, (rows, width))]
    storages = [as_bytes(logits), np.zeros(logits.nbytes, np.uint8)]
    compare(hip, m3.OP_SOFTMAX, storages, views,
            "softmax subnormal ties w=%d" % width)


def softmax_source(logits, dtype):
    if dtype == m3.F16:
        return as_bytes(logits.astype(np.float16).view(np.uint16))
    if dtype == m3.BF16:
        return as_bytes((logits.view(np.uint32) >> 16).astype(np.uint16))
    return as_bytes(logits)


@pytest.mark.parametrize("width", [77, 1001, 2047, 2501, 9000, 9001, 16384,
                                   32768])
def test_softmax_any_width(hip, width):
    """Widths that are not a multiple of 4 move element by element (77,
    1001 and 2047 in registers, 2501 and 9001 streamed); rows wider than
    the LDS tile (9000, 16384, 32768) stream through three passes."""
    rng = np.random.default_rng(15000 + width)
    rows = max(6, min(96, 600000 // width))
    logits = softmax_logits(rng, rows, width)
    if rows >= 6:
        logits[4, width // 2:] = -np.inf
        logits[5, :] = -200.0
        logits[5, width - 1] = 0.0
    views = [ViewSpec(0, m3.F32, (rows, width)),
             ViewSpec(1, m3.F32, (rows, width))]
    storages = [as_bytes(logits), np.zeros(logits.nbytes, np.uint8)]
    compare(hip, m3.OP_SOFTMAX, storages, views, "softmax any w=%d" % width)


@pytest.mark.parametrize("dtypes", [(m3.F16, m3.F16), (m3.BF16, m3.F32),
                                    (m3.F32, m3.BF16)])
@pytest.mark.parametrize("width", [77, 1001, 16384])
def test_softmax_any_width_dtypes(hip, dtypes, width):
    rng = np.random.default_rng(16000 + width + 7 * dtypes[0] + dtypes[1])
    rows = 24
    logits = softmax_logits(rng, rows, width)
    views = [ViewSpec(0, dtypes[0], (rows, width)),
             ViewSpec(1, dtypes[1], (rows, width))]
    storages = [softmax_source(logits, dtypes[0]),
                np.zeros(rows * width * m3.DTYPE_SIZES[dtypes[1]], np.uint8)]
    compare(hip, m3.OP_SOFTMAX, storages, views,
            "softmax any %s w=%d" % (dtypes, width))


@pytest.mark.parametrize("width", [100, 1000, 12000])
def test_softmax_row_layouts(hip, width):
    """Row starts that are padded, unaligned, or not evenly spaced (outer
    axes that do not merge), for register-resident and streamed rows."""
    rng = np.random.default_rng(17000 + width)
    rows = 24
    logits = softmax_logits(rng, rows, width)
    out = np.zeros(logits.nbytes, np.uint8)
    # padded rows
    pitch = width + 13
    padded = np.full((rows, pitch), 5.0, np.float32)
    padded[:, :width] = logits
    compare(hip, m3.OP_SOFTMAX, [as_bytes(padded), out],
            [ViewSpec(0, m3.F32, (rows, width), (pitch * 4, 4)),
             ViewSpec(1, m3.F32, (rows, width))],
            "softmax padded odd pitch w=%d" % width)
    # a row start 4 bytes past a 16-byte boundary
    shifted = np.zeros(logits.size + 1, np.float32)
    shifted[1:] = logits.ravel()
    compare(hip, m3.OP_SOFTMAX, [as_bytes(shifted), out],
            [ViewSpec(0, m3.F32, (rows, width), None, 4),
             ViewSpec(1, m3.F32, (rows, width))],
            "softmax unaligned start w=%d" % width)
    # outer axes (4, 6) read from a (6, 4, width) layout: uneven row starts
    stack = logits.reshape(6, 4, width)
    compare(hip, m3.OP_SOFTMAX, [as_bytes(stack), out],
            [ViewSpec(0, m3.F32, (4, 6, width),
                      (width * 4, 4 * width * 4, 4)),
             ViewSpec(1, m3.F32, (4, 6, width))],
            "softmax uneven rows w=%d" % width)
    # the same with 16-bit input and output
    half = softmax_source(logits, m3.F16)
    compare(hip, m3.OP_SOFTMAX,
            [half, np.zeros(rows * width * 2, np.uint8)],
            [ViewSpec(0, m3.F16, (4, 6, width),
                      (width * 2, 4 * width * 2, 2)),
             ViewSpec(1, m3.BF16, (4, 6, width))],
            "softmax uneven rows f16->bf16 w=%d" % width)


def test_softmax_strided_and_in_place(hip):
    rng = np.random.default_rng(9)
    logits = softmax_logits(rng, 64, 1024)
    # rows with a padded stride, and a transposed view (column stride)
    padded = np.full((64, 1040), 7.0, np.float32)
    padded[:, :1024] = logits
    compare(hip, m3.OP_SOFTMAX, [as_bytes(padded),
                                 np.zeros(logits.nbytes, np.uint8)],
            [ViewSpec(0, m3.F32, (64, 1024), (4160, 4)),
             ViewSpec(1, m3.F32, (64, 1024))], "softmax padded rows")
    compare(hip, m3.OP_SOFTMAX, [as_bytes(logits.T.copy()),
                                 np.zeros(logits.nbytes, np.uint8)],
            [ViewSpec(0, m3.F32, (64, 1024), (4, 256)),
             ViewSpec(1, m3.F32, (64, 1024))], "softmax transposed")
    compare(hip, m3.OP_SOFTMAX, [as_bytes(logits)],
            [ViewSpec(0, m3.F32, (64, 1024)),
             ViewSpec(0, m3.F32, (64, 1024))], "softmax in place")
    batched = softmax_logits(rng, 4 * 32, 1024).reshape(4, 32, 1024)
    compare(hip, m3.OP_SOFTMAX, [as_bytes(batched),
                                 np.zeros(batched.nbytes, np.uint8)],
            [ViewSpec(0, m3.F32, (4, 32, 1024)),
             ViewSpec(1, m3.F32, (4, 32, 1024))], "softmax rank 3")


def lane_row_logits(rng, rows, width):
    """Causal logits with special rows (all -inf, +inf entries, all zero,
    subnormal) at every position within a wave of four rows."""
    logits = softmax_logits(rng, rows, width, specials=False)
    special = [lambda r: r.fill(-np.inf),
               lambda r: r.__setitem__(slice(None, None, 5), np.inf),
               lambda r: r.fill(0.0),
               lambda r: r.fill(np.float32(1e-40))]
    for k in range(min(rows, 40)):
        if k % 3 == 1:
            special[(k // 3) % 4](logits[k])
    if rows > 20:
        logits[17, :] = -np.inf
        logits[17, width - 1] = np.inf  # one +inf, last column
        logits[18, :] = -np.inf
        logits[18, width - 1] = 2.5  # a finite maximum in the last column
    return logits


@pytest.mark.parametrize("width", [516, 768, 1000, 1020, 1024])
@pytest.mark.parametrize("rows", [1, 2, 7, 258])
def test_softmax_lane_rows(hip, width, rows):
    """F32 rows of 513..1024 columns, four to a wave, one per 16 lanes:
    partial last waves (rows not a multiple of 4), widths that end inside
    a lane's block, and special rows at every position within a wave next
    to ordinary rows."""
    rng = np.random.default_rng(19000 + width * 7 + rows)
    logits = lane_row_logits(rng, rows, width)
    out = np.zeros(logits.nbytes, np.uint8)
    compare(hip, m3.OP_SOFTMAX, [as_bytes(logits), out],
            [ViewSpec(0, m3.F32, (rows, width)),
             ViewSpec(1, m3.F32, (rows, width))],
            "softmax lane rows w=%d rows=%d" % (width, rows))
    if rows == 258:
        # uneven row starts: outer axes (2, 129) read from (129, 2, width)
        stack = logits.reshape(129, 2, width)
        compare(hip, m3.OP_SOFTMAX, [as_bytes(stack), out],
                [ViewSpec(0, m3.F32, (2, 129, width),
                          (width * 4, 2 * width * 4, 4)),
                 ViewSpec(1, m3.F32, (2, 129, width))],
                "softmax lane rows uneven w=%d" % width)
        compare(hip, m3.OP_SOFTMAX, [as_bytes(logits)],
                [ViewSpec(0, m3.F32, (rows, width)),
                 ViewSpec(0, m3.F32, (rows, width))],
                "softmax lane rows in place w=%d" % width)


@pytest.mark.parametrize("dtypes", [(m3.F16, m3.F16), (m3.BF16, m3.F32),
                                    (m3.F32, m3.BF16)])
@pytest.mark.parametrize("width", [260, 300, 508, 512, 700, 1020, 1024])
@pytest.mark.parametrize("rows", [7, 258])
def test_softmax_lane_rows_dtypes(hip, dtypes, width, rows):
    """The lane-row kernel with 16-bit input or output, 8 float4 per lane
    (257..512 columns) and 16 (513..1024)."""
    rng = np.random.default_rng(21000 + width * 7 + rows + 3 * dtypes[0] +
                                dtypes[1])
    logits = lane_row_logits(rng, rows, width)
    out_size = 4 if dtypes[1] == m3.F32 else 2
    compare(hip, m3.OP_SOFTMAX,
            [softmax_source(logits, dtypes[0]),
             np.zeros(rows * width * out_size, np.uint8)],
            [ViewSpec(0, dtypes[0], (rows, width)),
             ViewSpec(1, dtypes[1], (rows, width))],
            "softmax lane rows %s w=%d rows=%d" % (dtypes, width, rows))


@pytest.fixture(scope="module")
def hip_late(gpu):
    """A HIP backend on which every wave of the lane-row softmax counts as
    late (M3_HIP_SOFTMAX_LATE_US=0, read when the device opens), so every
    sum runs the lane-to-lane form."""
    saved = os.environ.get("M3_HIP_SOFTMAX_LATE_US")
    os.environ["M3_HIP_SOFTMAX_LATE_US"] = "0"
    try:
        fixture = HipFixture()
    finally:
        if saved is None:
            del os.environ["M3_HIP_SOFTMAX_LATE_US"]
        else:
            os.environ["M3_HIP_SOFTMAX_LATE_US"] = saved
    yield fixture
    fixture.close()


@pytest.mark.parametrize("dtypes", [(m3.F32, m3.F32), (m3.F16, m3.F16),
                                    (m3.BF16, m3.F32)])
@pytest.mark.parametrize("width", [300, 516, 1000, 1024])
@pytest.mark.parametrize("rows", [7, 258])
def test_softmax_lane_rows_late_path(hip_late, dtypes, width, rows):
    """The lane-row kernel with every sum passed from lane to lane, the
    form that waves whose rows arrive late take: the same bits."""
    if dtypes == (m3.F32, m3.F32) and width <= 512:
        width += 512  # F32 rows of 257..512 columns take the rows kernel
    rng = np.random.default_rng(23000 + width * 7 + rows + 3 * dtypes[0] +
                                dtypes[1])
    logits = lane_row_logits(rng, rows, width)
    out_size = 4 if dtypes[1] == m3.F32 else 2
    compare(hip_late, m3.OP_SOFTMAX,
            [softmax_source(logits, dtypes[0]),
             np.zeros(rows * width * out_size, np.uint8)],
            [ViewSpec(0, dtypes[0], (rows, width)),
             ViewSpec(1, dtypes[1], (rows, width))],
            "softmax lane rows, late path %s w=%d rows=%d" % (dtypes, width,
                                                             rows))


# ---- snake1d -------------------------------------------------------------------

@pytest.mark.parametrize("shape", [(2, 16, 1024), (1, 3, 5), (3, 7, 12),
                                   (2, 96, 4096), (2, 40, 1200)])
def test_snake1d_layouts(hip, shape):
    rng = np.random.default_rng(10000 + sum(shape))
    count = int(np.prod(shape))
    x = random_f32(rng, count, scale=3.0, specials=0.01)
    x[:8] = np.array([200.0, -1e5, 3e38, 0.0, -0.0, 1e-30, 1e30, 125.0],
                     np.float32)[:min(8, count)]
    alpha = rng.uniform(0.1, 2.0, shape[1]).astype(np.float32)
    alpha[0] = np.uint32(0xb089705f).view(np.float32)  # -epsilon
    views = [ViewSpec(0, m3.F32, shape), ViewSpec(1, m3.F32, (1, shape[1], 1)),
             ViewSpec(2, m3.F32, shape)]
    storages = [as_bytes(x), as_bytes(alpha), np.zeros(x.nbytes, np.uint8)]
    compare(hip, m3.OP_SNAKE1D, storages, views, "snake %s" % (shape,))


def test_snake1d_large_grid(hip):
    """x[2,64,262144]: 8,192 workgroups of one tile each, every element
    compared with the oracle."""
    shape = (2, 64, 262144)
    rng = np.random.default_rng(10077)
    count = int(np.prod(shape))
    x = random_f32(rng, count, scale=3.0, specials=0.001)
    alpha = rng.uniform(0.1, 2.0, shape[1]).astype(np.float32)
    views = [ViewSpec(0, m3.F32, shape), ViewSpec(1, m3.F32, (1, shape[1], 1)),
             ViewSpec(2, m3.F32, shape)]
    storages = [as_bytes(x), as_bytes(alpha), np.zeros(x.nbytes, np.uint8)]
    compare(hip, m3.OP_SNAKE1D, storages, views, "snake %s" % (shape,))


def test_snake1d_strided_input_and_alias(hip):
    rng = np.random.default_rng(11)
    x = random_f32(rng, 2 * 8 * 64, scale=2.0, specials=0.0)
    alpha = rng.uniform(0.1, 2.0, 16).astype(np.float32)
    # input: channels-last buffer [2, 64, 8] viewed as [2, 8, 64]
    views = [ViewSpec(0, m3.F32, (2, 8, 64), (2048, 4, 32)),
             ViewSpec(1, m3.F32, (1, 8, 1), (32, 8, 4)),
             ViewSpec(2, m3.F32, (2, 8, 64))]
    storages = [as_bytes(x), as_bytes(alpha), np.zeros(x.nbytes, np.uint8)]
    compare(hip, m3.OP_SNAKE1D, storages, views, "snake strided")
    compare(hip, m3.OP_SNAKE1D, [as_bytes(x), as_bytes(alpha[:8])],
            [ViewSpec(0, m3.F32, (2, 8, 64)), ViewSpec(1, m3.F32, (1, 8, 1)),
             ViewSpec(0, m3.F32, (2, 8, 64))], "snake in place")


# ---- TANH -------------------------------------------------------------------

TANH_EDGES = np.array([0x41b00000, 0xc1b00000, 0x41afffff, 0x3f800000,
                       0x3f7fffff, 0xbf800000, 0x24000000, 0x23ffffff,
                       0xa3ffffff, 0x3eb17218, 0x3f851592, 0x33000000,
                       0x32ffffff, 0x7fc12345, 0xff812345, 0x7f800000,
                       0xff800000, 0x00000000, 0x80000000, 0x00000001],
                      np.uint32)

TANH_SHAPES = [(1,), (3,), (4,), (7,), (1021,), (8, 64, 96), (1000003,),
               (2, 1, 3, 1, 5, 1, 7, 2)]


@pytest.mark.parametrize("shape", TANH_SHAPES)
def test_tanh_layouts(hip, shape):
    rng = np.random.default_rng(20000 + int(np.prod(shape)))
    count = int(np.prod(shape))
    x = random_f32(rng, count, scale=3.0, specials=0.05)
    head = min(count, TANH_EDGES.size)
    x.view(np.uint32)[:head] = TANH_EDGES[:head]
    views = [ViewSpec(0, m3.F32, shape), ViewSpec(1, m3.F32, shape)]
    storages = [as_bytes(x), np.zeros(x.nbytes, np.uint8)]
    compare(hip, m3.OP_TANH, storages, views, "tanh %s" % (shape,))


def test_tanh_dense_bit_sweep(hip):
    """2^24 inputs spread over every exponent and sign: bit patterns
    k * 256 + r with a random low byte r."""
    rng = np.random.default_rng(21)
    bits = ((np.arange(1 << 24, dtype=np.uint64) << np.uint64(8)) |
            rng.integers(0, 256, 1 << 24, dtype=np.uint64)).astype(np.uint32)
    views = [ViewSpec(0, m3.F32, (1 << 24,)), ViewSpec(1, m3.F32, (1 << 24,))]
    storages = [as_bytes(bits), np.zeros(bits.nbytes, np.uint8)]
    compare(hip, m3.OP_TANH, storages, views, "tanh dense sweep")


def test_tanh_strided_offset_and_in_place(hip):
    rng = np.random.default_rng(22)
    x = random_f32(rng, 1001, scale=2.0)
    # every other element of a [10, 100] block, 4 bytes in
    views = [ViewSpec(0, m3.F32, (10, 50), (400, 8), 4),
             ViewSpec(1, m3.F32, (10, 50))]
    compare(hip, m3.OP_TANH, [as_bytes(x), np.zeros(2000, np.uint8)], views,
            "tanh strided")
    for offset in (0, 4):  # vector path, then the unaligned general path
        views = [ViewSpec(0, m3.F32, (997,), None, offset),
                 ViewSpec(0, m3.F32, (997,), None, offset)]
        compare(hip, m3.OP_TANH, [as_bytes(x)], views,
                "tanh in place offset %d" % offset)


# ---- GATED_SILU -------------------------------------------------------------

FLOAT_DTYPES = [m3.F32, m3.F16, m3.BF16]


def nan_heavy_f32(rng, count, fraction=0.45, scale=8.0):
    values = (rng.standard_normal(count) * scale).astype(np.float32)
    bits = values.view(np.uint32)
    pick = rng.random(count) < fraction
    payload = rng.integers(1, 1 << 23, count, dtype=np.uint32)
    sign = rng.integers(0, 2, count, dtype=np.uint32) << np.uint32(31)
    bits[pick] = (sign | np.uint32(0x7f800000) | payload)[pick]
    return values


@pytest.mark.parametrize("dtypes", [(g, u, o) for g in FLOAT_DTYPES
                                    for u in FLOAT_DTYPES
                                    for o in FLOAT_DTYPES])
@pytest.mark.parametrize("count", [5, 4099])
def test_gated_silu_dtypes(hip, dtypes, count):
    rng = np.random.default_rng(30000 + 100 * sum(dtypes) + count)
    views = [ViewSpec(i, d, (count,)) for i, d in enumerate(dtypes)]
    storages = [storage_for(rng, dtypes[0], count, specials=0.1),
                storage_for(rng, dtypes[1], count, specials=0.1),
                np.zeros(count * m3.DTYPE_SIZES[dtypes[2]], np.uint8)]
    compare(hip, m3.OP_GATED_SILU, storages, views,
            "gated silu %s count %d" % (dtypes, count))


@pytest.mark.parametrize("shape", [(8, 64, 96), (1000003,), (3, 1, 5, 7),
                                   ()])
def test_gated_silu_f32_layouts(hip, shape):
    rng = np.random.default_rng(31000 + int(np.prod(shape)))
    count = int(np.prod(shape))
    gate = random_f32(rng, count, scale=12.0, specials=0.05)
    up = random_f32(rng, count, scale=2.0, specials=0.05)
    views = [ViewSpec(i, m3.F32, shape) for i in range(3)]
    storages = [as_bytes(gate), as_bytes(up), np.zeros(4 * count, np.uint8)]
    compare(hip, m3.OP_GATED_SILU, storages, views,
            "gated silu %s" % (shape,))


@pytest.mark.parametrize("count", [4000, 4003])
def test_gated_silu_nan_operands(hip, count):
    """Both operands mostly NaN with random payloads and signs, plus the
    invalid cases (-inf gate; zero or infinite activation times an
    infinite or zero up)."""
    rng = np.random.default_rng(32000 + count)
    gate = nan_heavy_f32(rng, count)
    up = nan_heavy_f32(rng, count)
    gate.view(np.uint32)[:6] = [0xff800000, 0x7f800000, 0x00000000,
                                0xc2f00000, 0x7f800000, 0xff800000]
    up.view(np.uint32)[:6] = [0x7fa00005, 0x00000000, 0x7f800000,
                              0xff800000, 0x80000000, 0x3f800000]
    views = [ViewSpec(i, m3.F32, (count,)) for i in range(3)]
    storages = [as_bytes(gate), as_bytes(up), np.zeros(4 * count, np.uint8)]
    compare(hip, m3.OP_GATED_SILU, storages, views, "gated silu NaN")


def test_gated_silu_dense_gate_sweep(hip):
    rng = np.random.default_rng(33)
    gate = ((np.arange(1 << 24, dtype=np.uint64) << np.uint64(8)) |
            rng.integers(0, 256, 1 << 24, dtype=np.uint64)).astype(np.uint32)
    up = random_f32(rng, 1 << 24, scale=2.0, specials=0.02)
    views = [ViewSpec(i, m3.F32, (1 << 24,)) for i in range(3)]
    storages = [as_bytes(gate), as_bytes(up), np.zeros(4 << 24, np.uint8)]
    compare(hip, m3.OP_GATED_SILU, storages, views, "gated silu sweep")


@pytest.mark.parametrize("count", [16 << 16, (1 << 16) + 3])
def test_gated_silu_bf16_every_gate(hip, count):
    """Every BF16 gate bit pattern, so every entry of the BF16 kernel's
    activation table and every gate outside it (tiny, huge, subnormal,
    infinite, NaN), times random BF16 up bits (NaN, infinities and zeros
    included) and 1.0, through the vector path (with a 3-element tail for
    the odd count)."""
    rng = np.random.default_rng(35 + count)
    gate = (np.arange(count, dtype=np.uint32) & 0xffff).astype(np.uint16)
    up = random_bits16(rng, count)
    up[::7] = 0x3f80
    views = [ViewSpec(i, m3.BF16, (count,)) for i in range(3)]
    storages = [as_bytes(gate), as_bytes(up), np.zeros(2 * count, np.uint8)]
    compare(hip, m3.OP_GATED_SILU, storages, views,
            "gated silu BF16 every gate, count %d" % count)


def test_gated_silu_bf16_layouts_and_aliases(hip):
    """The BF16 kernel's neighbours: a 2-byte offset (the general kernel),
    the output over the gate and over up (the vector kernel in place)."""
    rng = np.random.default_rng(36)
    count = 4096
    gate = np.frombuffer(storage_for(rng, m3.BF16, count + 1, specials=0.1),
                         np.uint16).copy()
    up = np.frombuffer(storage_for(rng, m3.BF16, count + 1, specials=0.1),
                       np.uint16).copy()
    shifted = [ViewSpec(0, m3.BF16, (count,), None, 2),
               ViewSpec(1, m3.BF16, (count,)),
               ViewSpec(2, m3.BF16, (count,))]
    compare(hip, m3.OP_GATED_SILU,
            [as_bytes(gate), as_bytes(up), np.zeros(2 * count, np.uint8)],
            shifted, "gated silu BF16 offset gate")
    exact = [ViewSpec(0, m3.BF16, (count,)), ViewSpec(1, m3.BF16, (count,))]
    compare(hip, m3.OP_GATED_SILU, [as_bytes(gate), as_bytes(up)],
            exact + [exact[0]], "gated silu BF16 gate alias")
    compare(hip, m3.OP_GATED_SILU, [as_bytes(gate), as_bytes(up)],
            exact + [exact[1]], "gated silu BF16 up alias")


def test_gated_silu_strided_and_aliases(hip):
    rng = np.random.default_rng(34)
    gate = random_f32(rng, 2000, scale=6.0)
    up = random_f32(rng, 2000, scale=2.0)
    views = [ViewSpec(0, m3.F32, (20, 40), (320, 8), 4),
             ViewSpec(1, m3.F32, (20, 40), (160, 4), 0),
             ViewSpec(2, m3.F32, (20, 40))]
    compare(hip, m3.OP_GATED_SILU,
            [as_bytes(gate), as_bytes(up), np.zeros(3200, np.uint8)], views,
            "gated silu strided")
    exact = [ViewSpec(0, m3.F32, (1999,)), ViewSpec(1, m3.F32, (1999,))]
    compare(hip, m3.OP_GATED_SILU, [as_bytes(gate), as_bytes(up)],
            exact + [exact[0]], "gated silu gate alias")
    compare(hip, m3.OP_GATED_SILU, [as_bytes(gate), as_bytes(up)],
            exact + [exact[1]], "gated silu up alias")
    g16 = storage_for(rng, m3.BF16, 1001)
    u16 = storage_for(rng, m3.BF16, 1001)
    exact = [ViewSpec(0, m3.BF16, (1001,)), ViewSpec(1, m3.BF16, (1001,))]
    compare(hip, m3.OP_GATED_SILU, [g16, u16], exact + [exact[1]],
            "gated silu bf16 up alias")
