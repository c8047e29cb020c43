"""Command-list semantics of the HIP provider (GPU).

Restates the GPU-provider list contracts the reference tests for Metal:
data preflight of inputs that no command of the list writes is
list-atomic, and the first failing command in list order decides the
status (tests/test_metal_basic_softmax.c:242-357,
tests/test_metal_cast.c:294-424). A softmax or float-to-I32 cast whose
input IS written earlier in the list, which Metal rejects with UNSUPPORTED,
runs here with the reference CPU provider's order instead (preflight right
before the command, src/m3_op_execute_host.c:5-60): its producers run, its
input is scanned on the device, and a failing scan stops the list there
with OUT_OF_RANGE. Also covers the provider's cache of clean inputs: a
later host write or kernel output must be rescanned.
"""
import math
import sys

import numpy as np
import pytest

from conftest import m3
from harness import HipFixture, ViewSpec, as_bytes, run_oracle

pytestmark = pytest.mark.gpu


def f32(values):
    return np.asarray(values, dtype=np.float32)


@pytest.fixture()
def hip(gpu):
    fixture = HipFixture()
    yield fixture
    fixture.close()


def values(hip, handle, count, dtype=np.float32):
    out = np.empty(count, dtype=dtype)
    return hip.download([handle], [out])[0]


def write(hip, handle, array):
    lib, _ = m3.load()
    error = m3.Error()
    import ctypes
    m3.check(lib.m3_storage_write(handle, 0, array.ctypes.data_as(
        ctypes.c_void_p), array.nbytes, ctypes.byref(error)), error)


def test_softmax_preflight_order(hip):
    print("gpu case softmax_preflight_order", file=sys.stderr, flush=True)
    sentinel = f32([-9, -9, -9])
    arrays = [f32([3, 4, 5]), f32([2, 2, 2]), sentinel.copy(),
              f32([0, math.nan, 1]), sentinel.copy()]
    h = hip.upload(arrays)
    left, right, unrelated, sm_in, sm_out = hip.views(
        h, [ViewSpec(i, m3.F32, (3,)) for i in range(5)])
    # NaN softmax rejects the whole list; the MUL does not run either.
    status, _ = hip.execute([(m3.OP_MUL, [left, right, unrelated]),
                             (m3.OP_SOFTMAX, [sm_in, sm_out])])
    assert status == m3.OUT_OF_RANGE
    assert list(values(hip, h[2], 3)) == [-9, -9, -9]
    assert list(values(hip, h[4], 3)) == [-9, -9, -9]
    # A finite input commits both commands.
    write(hip, h[3], f32([0, 1, 2]))
    status, _ = hip.execute([(m3.OP_MUL, [left, right, unrelated]),
                             (m3.OP_SOFTMAX, [sm_in, sm_out])])
    assert status == m3.OK
    assert list(values(hip, h[2], 3)) == [6, 8, 10]
    # The softmax input is produced earlier in the list (over a NaN the host
    # wrote): the producer runs, the produced input is scanned on the
    # device, and the softmax runs on it.
    write(hip, h[3], f32([0, math.nan, 1]))
    write(hip, h[4], sentinel)
    status, message = hip.execute([(m3.OP_ADD, [left, right, sm_in]),
                                   (m3.OP_SOFTMAX, [sm_in, sm_out])])
    assert status == m3.OK, message
    assert list(values(hip, h[3], 3)) == [5, 6, 7]
    expected = softmax_oracle(f32([5, 6, 7]))
    assert np.array_equal(values(hip, h[4], 3).view(np.uint32),
                          expected.view(np.uint32))
    # A producer that writes a NaN: it runs, the softmax does not.
    write(hip, h[2], f32([1, math.nan, 1]))
    write(hip, h[4], sentinel)
    status, message = hip.execute([(m3.OP_MUL, [left, unrelated, sm_in]),
                                   (m3.OP_SOFTMAX, [sm_in, sm_out])])
    assert status == m3.OUT_OF_RANGE
    assert "NaN" in message
    got = values(hip, h[3], 3)
    assert got[0] == 3 and math.isnan(got[1]) and got[2] == 5
    assert list(values(hip, h[4], 3)) == [-9, -9, -9]
    # A softmax output is a producer too: softmax of a softmax.
    status, _ = hip.execute([(m3.OP_SOFTMAX, [left, sm_in]),
                             (m3.OP_SOFTMAX, [sm_in, sm_out])])
    assert status == m3.OK
    expected = softmax_oracle(softmax_oracle(f32([3, 4, 5])))
    assert np.array_equal(values(hip, h[4], 3).view(np.uint32),
                          expected.view(np.uint32))


def softmax_oracle(row):
    views = [ViewSpec(0, m3.F32, (row.size,)), ViewSpec(1, m3.F32, (row.size,))]
    status, out = run_oracle(m3.OP_SOFTMAX, [as_bytes(row),
                                             np.zeros(row.nbytes, np.uint8)],
                             views)
    assert status == m3.OK
    return out[1].view(np.float32)


def test_float_to_i32_cast_atomic(hip):
    print("gpu case float_to_i32_cast_atomic", file=sys.stderr, flush=True)
    arrays = [f32([1, math.nan, 2, math.inf]), f32([9, 8, 7, 6]),
              np.array([77, 78, 79, 80], np.int32)]
    h = hip.upload(arrays)
    src, middle = hip.views(h[:2], [ViewSpec(0, m3.F32, (4,)),
                                    ViewSpec(1, m3.F32, (4,))])
    (dst,) = hip.views([h[2]], [ViewSpec(0, m3.I32, (4,))])
    status, _ = hip.execute([(m3.OP_CAST, [src, dst])])
    assert status == m3.OUT_OF_RANGE
    assert list(values(hip, h[2], 4, np.int32)) == [77, 78, 79, 80]
    # Earlier invalid cast of a list input wins over a later dependent
    # one, and nothing runs.
    status, _ = hip.execute([(m3.OP_CAST, [src, dst]),
                             (m3.OP_COPY, [src, middle]),
                             (m3.OP_CAST, [middle, dst])])
    assert status == m3.OUT_OF_RANGE
    assert list(values(hip, h[1], 4)) == [9, 8, 7, 6]
    assert list(values(hip, h[2], 4, np.int32)) == [77, 78, 79, 80]
    # COPY then CAST of the copied (produced) invalid values: the COPY
    # runs, the CAST is rejected on the device scan and writes nothing.
    status, message = hip.execute([(m3.OP_COPY, [src, middle]),
                                   (m3.OP_CAST, [middle, dst])])
    assert status == m3.OUT_OF_RANGE
    assert "invalid" in message
    got = values(hip, h[1], 4)
    assert got[0] == 1 and math.isnan(got[1]) and got[2] == 2 and \
        math.isinf(got[3])
    assert list(values(hip, h[2], 4, np.int32)) == [77, 78, 79, 80]
    # Valid produced values are cast.
    write(hip, h[0], f32([1.5, -2.5, 3e9 / 2, -7.0]))
    status, message = hip.execute([(m3.OP_COPY, [src, middle]),
                                   (m3.OP_CAST, [middle, dst])])
    assert status == m3.OK, message
    assert list(values(hip, h[2], 4, np.int32)) == [1, -2, 1500000000, -7]


def test_clean_input_cache_sees_later_writes(hip):
    print("gpu case clean_input_cache", file=sys.stderr, flush=True)
    arrays = [f32([0, 1, 2, 3]), np.zeros(16, np.uint8), f32([1, 1, 1, 1])]
    h = hip.upload(arrays)
    sm_in, sm_out, other = hip.views(
        h, [ViewSpec(0, m3.F32, (4,)), ViewSpec(1, m3.F32, (4,)),
            ViewSpec(2, m3.F32, (4,))])
    assert hip.execute([(m3.OP_SOFTMAX, [sm_in, sm_out])])[0] == m3.OK
    assert hip.execute([(m3.OP_SOFTMAX, [sm_in, sm_out])])[0] == m3.OK
    # Host write of a NaN after a clean scan: must be rescanned.
    write(hip, h[0], f32([0, math.nan, 2, 3]))
    assert hip.execute([(m3.OP_SOFTMAX, [sm_in, sm_out])])[0] == \
        m3.OUT_OF_RANGE
    # Clean again, then a kernel writes a NaN into the input storage in a
    # separate list: must be rescanned.
    write(hip, h[0], f32([0, 1, 2, 3]))
    assert hip.execute([(m3.OP_SOFTMAX, [sm_in, sm_out])])[0] == m3.OK
    write(hip, h[2], f32([math.nan, 1, 1, 1]))
    assert hip.execute([(m3.OP_MUL, [sm_in, other, sm_in])])[0] == m3.OK
    assert hip.execute([(m3.OP_SOFTMAX, [sm_in, sm_out])])[0] == \
        m3.OUT_OF_RANGE


def test_write_starts_rescan_of_watched_inputs(hip):
    """A host write to an input the preflight has scanned starts its rescan
    on the device; the next list collects it. Whatever happens between the
    write and the run (a second write, a kernel writing the input, a NaN
    written and then overwritten), the run sees the data it reads."""
    print("gpu case write_starts_rescan", file=sys.stderr, flush=True)
    arrays = [f32([0, 1, 2, 3]), np.zeros(16, np.uint8), f32([1, 1, 1, 1])]
    h = hip.upload(arrays)
    sm_in, sm_out, other = hip.views(
        h, [ViewSpec(0, m3.F32, (4,)), ViewSpec(1, m3.F32, (4,)),
            ViewSpec(2, m3.F32, (4,))])
    assert hip.execute([(m3.OP_SOFTMAX, [sm_in, sm_out])])[0] == m3.OK
    expected = values(hip, h[1], 4)
    # clean write: the started scan passes and the run uses it
    write(hip, h[0], f32([0, 1, 2, 3]))
    assert hip.execute([(m3.OP_SOFTMAX, [sm_in, sm_out])])[0] == m3.OK
    assert list(values(hip, h[1], 4)) == list(expected)
    # NaN written, then overwritten before the run
    write(hip, h[0], f32([0, math.nan, 2, 3]))
    write(hip, h[0], f32([0, 1, 2, 3]))
    assert hip.execute([(m3.OP_SOFTMAX, [sm_in, sm_out])])[0] == m3.OK
    # clean written, then NaN before the run: rejected, output untouched
    write(hip, h[0], f32([0, 1, 2, 3]))
    write(hip, h[0], f32([math.nan, 1, 2, 3]))
    hip_out_before = list(values(hip, h[1], 4))
    assert hip.execute([(m3.OP_SOFTMAX, [sm_in, sm_out])])[0] == \
        m3.OUT_OF_RANGE
    assert list(values(hip, h[1], 4)) == hip_out_before
    # clean written (scan started), then a kernel writes a NaN into the
    # input in another list before the softmax runs
    write(hip, h[0], f32([0, 1, 2, 3]))
    write(hip, h[2], f32([math.nan, 1, 1, 1]))
    assert hip.execute([(m3.OP_MUL, [sm_in, other, sm_in])])[0] == m3.OK
    assert hip.execute([(m3.OP_SOFTMAX, [sm_in, sm_out])])[0] == \
        m3.OUT_OF_RANGE
    # and clean again
    write(hip, h[0], f32([3, 2, 1, 0]))
    assert hip.execute([(m3.OP_SOFTMAX, [sm_in, sm_out])])[0] == m3.OK
    assert list(values(hip, h[1], 4)) == list(expected[::-1])


def test_started_scans_through_the_c_abi(gpu):
    """m3_hip_scan_views_begin/collect: the flags of a started scan are
    those of the blocking scan of the same views, also with a blocking scan
    in between; only the last started scan can be collected."""
    from harness import HipScanFixture

    scan = HipScanFixture()
    try:
        rng = np.random.default_rng(13)
        clean = rng.standard_normal(1 << 20).astype(np.float32)
        dirty = clean.copy()
        dirty[123457] = np.nan
        a_clean, a_dirty = scan.upload(clean), scan.upload(dirty)
        v_clean = scan.view(a_clean, m3.F32, (1 << 20,))
        v_dirty = scan.view(a_dirty, m3.F32, (1 << 20,))
        v_odd = scan.view(a_dirty + 4, m3.F32, (1 << 19,), (8,))
        nan = 0
        code, ticket, message = scan.begin([nan, nan, nan],
                                           [v_dirty, v_clean, v_odd])
        assert code == 0, message
        code, flags, message = scan.scan("m3_hip_scan_views", [nan, nan],
                                         [v_clean, v_dirty])
        assert code == 0 and flags == [0, 1], message
        code, flags, message = scan.collect(ticket, 3)
        assert code == 0, message
        # 123457 is odd: the view from element 1 with stride 2 holds it
        assert flags == [1, 0, 1]
        code, first, message = scan.begin([nan], [v_clean])
        assert code == 0, message
        code, second, message = scan.begin([nan], [v_dirty])
        assert code == 0, message
        assert scan.collect(first, 1)[0] != 0
        code, flags, message = scan.collect(second, 1)
        assert code == 0 and flags == [1], message
        assert scan.collect(second, 2)[0] != 0
    finally:
        scan.close()


def test_scan_flags_follow_each_call(gpu):
    """m3_hip_scan_views through the C-ABI, call after call: flags are set
    exactly for the views that offend in that call (a NaN, or a value
    outside [-2^31, 2^31) for the I32 kind), in contiguous F32, strided
    and 16-bit views, whatever earlier calls found; an empty list and an
    empty view leave no trace."""
    from harness import HipScanFixture

    scan = HipScanFixture()
    try:
        rng = np.random.default_rng(12)
        clean = rng.standard_normal(1 << 20).astype(np.float32)
        dirty = clean.copy()
        dirty[777777] = np.nan
        big = np.full(4099, 3.0e9, np.float32)
        halves = rng.standard_normal(3001).astype(np.float16)
        halves_nan = halves.copy()
        halves_nan[3000] = np.float16("nan")
        a = {name: scan.upload(array) for name, array in
             (("clean", clean), ("dirty", dirty), ("big", big),
              ("halves", halves.view(np.uint16)),
              ("halves_nan", halves_nan.view(np.uint16)))}
        nan, rng32 = 0, 1
        v_clean = scan.view(a["clean"], m3.F32, (1 << 20,))
        v_dirty = scan.view(a["dirty"], m3.F32, (1 << 20,))
        # every other element: 777777 is odd, so this view misses the NaN
        v_even = scan.view(a["dirty"], m3.F32, (1 << 19,), (8,))
        v_big = scan.view(a["big"], m3.F32, (4099,))
        v_half = scan.view(a["halves"], m3.F16, (3001,))
        v_half_nan = scan.view(a["halves_nan"], m3.F16, (3001,))
        v_empty = scan.view(a["clean"], m3.F32, (0,))
        calls = [
            ([nan, nan, nan], [v_clean, v_dirty, v_even], [0, 1, 0]),
            ([nan, nan], [v_clean, v_clean], [0, 0]),
            ([rng32, rng32, nan], [v_big, v_clean, v_half_nan], [1, 0, 1]),
            ([nan, nan, rng32], [v_half, v_empty, v_clean], [0, 0, 0]),
            ([], [], []),
            ([nan] * 64, [v_dirty] * 63 + [v_clean], [1] * 63 + [0]),
            ([nan], [v_clean], [0]),
        ]
        for kinds, views, expected in calls:
            code, flags, message = scan.scan("m3_hip_scan_views", kinds,
                                             views)
            assert code == 0, message
            assert flags == expected, (kinds, flags, expected)
        code, _, message = scan.scan("m3_hip_scan_views", [nan] * 65,
                                     [v_clean] * 65)
        assert code != 0 and "64" in message
    finally:
        scan.close()
