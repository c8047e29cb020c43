"""The oracle against the compiled reference on seeded random inputs (CPU).

oracle/_ref/libm3ref.so is the reference's own host op layer compiled from
its sources; every case here runs one command on it and on the oracle and
requires equal status and identical bytes in every storage, NaN payloads
included. Inputs mix normal values with the special classes (signed zeros,
infinities, NaNs with random payloads and signs, subnormals, overflow edges)
and, for the NaN rules of two-operand ops, with inputs where most elements
of both operands are NaN. Layouts cover contiguous, strided, offset,
broadcast and aliased views. SUB and DIV have no reference counterpart;
test_oracle_subdiv_cpu.py pins them to IEEE-754 subtraction and division
(numpy float32) and to the stated NaN payload rule.
"""
import numpy as np
import pytest

from conftest import m3
from harness import (ViewSpec, as_bytes, ref_available, run_oracle, run_ref,
                     subnormal_tie_rows)

pytestmark = pytest.mark.skipif(
    not ref_available(),
    reason="compiled reference (oracle/_ref) not built here")

SPECIALS32 = np.array([0x00000000, 0x80000000, 0x7f800000, 0xff800000,
                       0x7fc00000, 0xffc00000, 0x7f800001, 0x00000001,
                       0x807fffff, 0x3f800000, 0x42b17218, 0xc2b17218,
                       0x42b17217, 0xc2cff1b5, 0x41b00000, 0xc1b00000,
                       0x24000000, 0x23ffffff, 0x7f7fffff, 0xff7fffff],
                      np.uint32)


def nan_bits(rng, count):
    payload = rng.integers(1, 1 << 23, count, dtype=np.uint32)
    sign = rng.integers(0, 2, count, dtype=np.uint32) << np.uint32(31)
    return sign | np.uint32(0x7f800000) | payload


def f32_data(rng, count, scale=4.0, specials=0.1, nans=0.0):
    values = (rng.standard_normal(count) * scale).astype(np.float32)
    bits = values.view(np.uint32)
    pick = rng.random(count)
    special = pick < specials
    bits[special] = rng.choice(SPECIALS32, size=int(special.sum()))
    nan = (pick >= specials) & (pick < specials + nans)
    bits[nan] = nan_bits(rng, int(nan.sum()))
    return bits


def u16_data(rng, count, dtype, specials=0.1):
    if dtype == m3.F16:
        bits = (rng.standard_normal(count) * 4).astype(np.float16).view(
            np.uint16)
    else:
        bits = ((rng.standard_normal(count) * 4).astype(np.float32).view(
            np.uint32) >> 16).astype(np.uint16)
    pick = rng.random(count) < specials
    bits[pick] = rng.integers(0, 1 << 16, int(pick.sum())).astype(np.uint16)
    return bits


def storage(rng, dtype, count, **kw):
    if dtype == m3.F32:
        return as_bytes(f32_data(rng, count, **kw))
    if dtype == m3.I32:
        return as_bytes(rng.integers(-2**31, 2**31, count,
                                     dtype=np.int64).astype(np.int32))
    return as_bytes(u16_data(rng, count, dtype))


def span(spec):
    if spec.count() == 0:
        return 0
    return spec.offset + sum((d - 1) * s for d, s in
                             zip(spec.shape, spec.byte_strides())) + \
        m3.DTYPE_SIZES[spec.dtype]


def same(kind, storages, views):
    rstatus, rout = run_ref(kind, storages, views)
    ostatus, oout = run_oracle(kind, storages, views)
    assert rstatus == ostatus, (m3.status_name(rstatus),
                                m3.status_name(ostatus))
    for index, (a, b) in enumerate(zip(rout, oout)):
        if bytes(a) != bytes(b):
            diff = np.flatnonzero(a != b)
            raise AssertionError("storage %d differs at %d bytes, first at "
                                 "byte %d" % (index, diff.size, diff[0]))
    return rstatus


FLOATS = [m3.F32, m3.F16, m3.BF16]


@pytest.mark.parametrize("op", [m3.OP_ADD, m3.OP_MUL])
@pytest.mark.parametrize("layout", [
    ((6, 33, 40), (6, 33, 40)), ((6, 33, 40), (40,)), ((6, 33, 40), (33, 1)),
    ((4, 1, 9), (1, 5, 9)), ((7,), ()), ((), ())])
def test_binary_layouts_and_nan_operands(op, layout):
    rng = np.random.default_rng(10 + op)
    ls, rs = layout
    os_ = tuple(np.broadcast_shapes(ls, rs))
    views = [ViewSpec(0, m3.F32, ls), ViewSpec(1, m3.F32, rs),
             ViewSpec(2, m3.F32, os_)]
    for nans in (0.0, 0.6):
        storages = [storage(rng, m3.F32, views[0].count(), nans=nans),
                    storage(rng, m3.F32, views[1].count(), nans=nans),
                    np.zeros(span(views[2]), np.uint8)]
        assert same(op, storages, views) == m3.OK


@pytest.mark.parametrize("dtypes", [(a, b, c) for a in FLOATS for b in FLOATS
                                    for c in FLOATS])
def test_binary_mixed_dtypes(dtypes):
    rng = np.random.default_rng(sum(dtypes))
    shape = (5, 67)
    views = [ViewSpec(i, d, shape) for i, d in enumerate(dtypes)]
    storages = [storage(rng, dtypes[0], 335), storage(rng, dtypes[1], 335),
                np.zeros(span(views[2]), np.uint8)]
    same(m3.OP_MUL, storages, views)


def test_binary_strided_offset_and_alias():
    rng = np.random.default_rng(3)
    base = storage(rng, m3.F32, 4 * 30 * 2 + 8)
    other = storage(rng, m3.F32, 31)
    # strided, offset left; outputs are contiguous in the reference
    views = [ViewSpec(0, m3.F32, (4, 30), (240, 8), 16),
             ViewSpec(1, m3.F32, (30,), (4,), 4),
             ViewSpec(2, m3.F32, (4, 30))]
    assert same(m3.OP_ADD, [base, other, np.zeros(480, np.uint8)],
                views) == m3.OK
    # exact alias of an offset left input
    views = [ViewSpec(0, m3.F32, (4, 30), None, 16),
             ViewSpec(1, m3.F32, (30,), (4,), 4),
             ViewSpec(0, m3.F32, (4, 30), None, 16)]
    assert same(m3.OP_ADD, [base, other], views) == m3.OK


@pytest.mark.parametrize("src", FLOATS + [m3.I32])
@pytest.mark.parametrize("dst", FLOATS + [m3.I32])
def test_cast_pairs(src, dst):
    rng = np.random.default_rng(100 + 4 * src + dst)
    views = [ViewSpec(0, src, (3000,)), ViewSpec(1, dst, (3000,))]
    data = storage(rng, src, 3000, specials=0.02)
    if src == m3.F32 and dst == m3.I32:
        # in range, so that the preflight passes and conversion runs
        data = as_bytes((rng.standard_normal(3000) * 1e6).astype(np.float32))
    same(m3.OP_CAST, [data, np.zeros(span(views[1]), np.uint8)], views)


def test_cast_preflight_rejects_out_of_range():
    views = [ViewSpec(0, m3.F32, (3,)), ViewSpec(1, m3.I32, (3,))]
    data = as_bytes(np.array([1.0, 3e9, 2.0], np.float32))
    assert same(m3.OP_CAST, [data, np.zeros(12, np.uint8)], views) \
        == m3.OUT_OF_RANGE


@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("width", [1, 5, 64, 333])
def test_softmax_finite_rows(dtype, width):
    rng = np.random.default_rng(width + 7 * dtype)
    rows = 24
    values = (rng.standard_normal(rows * width) * 6).astype(np.float32)
    bits = values.view(np.uint32)
    pick = rng.random(rows * width)
    bits[pick < 0.05] = 0xff800000
    bits[(pick >= 0.05) & (pick < 0.07)] = 0x7f800000
    if dtype == m3.F32:
        data = as_bytes(bits)
    elif dtype == m3.F16:
        data = as_bytes(values.astype(np.float16))
    else:
        data = as_bytes((bits >> 16).astype(np.uint16))
    views = [ViewSpec(0, dtype, (rows, width)),
             ViewSpec(1, dtype, (rows, width))]
    same(m3.OP_SOFTMAX, [data, np.zeros(span(views[1]), np.uint8)], views)


def test_softmax_subnormal_ties():
    """Rows whose quotients fall exactly on subnormal rounding midpoints:
    the oracle equals the compiled reference, and the rows do contain
    quotients where RN_f32(e * RN_f64(1/sum)) (a product of the reciprocal
    in double) is not the F32 quotient, so the GPU test with the same rows
    (test_gpu_parity.py) tells the two apart."""
    import ctypes
    import ctypes.util

    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    rng = np.random.default_rng(13128)
    rows, width = 64, 128
    logits = subnormal_tie_rows(rng, rows, width)
    views = [ViewSpec(0, m3.F32, (rows, width)),
             ViewSpec(1, m3.F32, (rows, width))]
    same(m3.OP_SOFTMAX, [as_bytes(logits), np.zeros(logits.nbytes, np.uint8)],
         views)
    differ = 0
    for r in range(rows):
        zeros = int(np.count_nonzero(logits[r] == 0.0))
        for v in logits[r][np.isfinite(logits[r]) & (logits[r] != 0.0)]:
            e = np.float32(libm.expf(float(v)))
            quotient = e / np.float32(zeros)
            product = np.float32(np.float64(e) * (1.0 / np.float64(zeros)))
            differ += quotient.view(np.uint32) != product.view(np.uint32)
    assert differ > 100


def test_softmax_nan_preflight():
    data = as_bytes(np.array([1.0, np.nan, 2.0, 3.0], np.float32))
    views = [ViewSpec(0, m3.F32, (2, 2)), ViewSpec(1, m3.F32, (2, 2))]
    assert same(m3.OP_SOFTMAX, [data, np.zeros(16, np.uint8)], views) \
        == m3.OUT_OF_RANGE


def test_snake1d_random_and_special():
    rng = np.random.default_rng(5)
    shape = (2, 7, 50)
    views = [ViewSpec(0, m3.F32, shape), ViewSpec(1, m3.F32, (1, 7, 1)),
             ViewSpec(2, m3.F32, shape)]
    storages = [storage(rng, m3.F32, 700, scale=30.0),
                storage(rng, m3.F32, 7, specials=0.3),
                np.zeros(2800, np.uint8)]
    same(m3.OP_SNAKE1D, storages, views)


@pytest.mark.parametrize("scale", [0.3, 3.0, 40.0])
def test_tanh_random_and_special(scale):
    rng = np.random.default_rng(int(scale * 10))
    views = [ViewSpec(0, m3.F32, (50, 81)), ViewSpec(1, m3.F32, (50, 81))]
    storages = [storage(rng, m3.F32, 4050, scale=scale, nans=0.1),
                np.zeros(4050 * 4, np.uint8)]
    same(m3.OP_TANH, storages, views)


def test_tanh_strided_and_in_place():
    rng = np.random.default_rng(11)
    data = storage(rng, m3.F32, 200, nans=0.1)
    views = [ViewSpec(0, m3.F32, (10, 5), (80, 8), 4),
             ViewSpec(1, m3.F32, (10, 5))]
    same(m3.OP_TANH, [data, np.zeros(200, np.uint8)], views)
    views = [ViewSpec(0, m3.F32, (200,)), ViewSpec(0, m3.F32, (200,))]
    same(m3.OP_TANH, [data], views)


@pytest.mark.parametrize("dtypes", [(a, b, c) for a in FLOATS for b in FLOATS
                                    for c in FLOATS])
def test_gated_silu_dtypes(dtypes):
    rng = np.random.default_rng(200 + 9 * dtypes[0] + 3 * dtypes[1]
                                + dtypes[2])
    shape = (9, 130)
    views = [ViewSpec(i, d, shape) for i, d in enumerate(dtypes)]
    storages = [storage(rng, dtypes[0], 1170, scale=8.0),
                storage(rng, dtypes[1], 1170),
                np.zeros(span(views[2]), np.uint8)]
    same(m3.OP_GATED_SILU, storages, views)


@pytest.mark.parametrize("scale", [1.0, 30.0, 120.0])
def test_gated_silu_nan_operands(scale):
    """Both operands mostly NaN with random payloads and signs: pins which
    NaN each of the three operations of the activation passes on."""
    rng = np.random.default_rng(int(scale))
    views = [ViewSpec(i, m3.F32, (4000,)) for i in range(3)]
    storages = [storage(rng, m3.F32, 4000, scale=scale, nans=0.45),
                storage(rng, m3.F32, 4000, scale=scale, nans=0.45),
                np.zeros(16000, np.uint8)]
    same(m3.OP_GATED_SILU, storages, views)


def test_gated_silu_strided_and_aliases():
    rng = np.random.default_rng(13)
    gate = storage(rng, m3.F32, 400, nans=0.1)
    up = storage(rng, m3.F32, 400, nans=0.1)
    views = [ViewSpec(0, m3.F32, (20, 10), (80, 8), 0),
             ViewSpec(1, m3.F32, (20, 10), (40, 4), 4),
             ViewSpec(2, m3.F32, (20, 10))]
    same(m3.OP_GATED_SILU, [gate, up, np.zeros(800, np.uint8)], views)
    exact = [ViewSpec(0, m3.F32, (400,)), ViewSpec(1, m3.F32, (400,))]
    same(m3.OP_GATED_SILU, [gate, up], exact + [exact[0]])
    same(m3.OP_GATED_SILU, [gate, up], exact + [exact[1]])
