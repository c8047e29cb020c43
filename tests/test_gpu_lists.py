"""Command-list semantics of the HIP provider (GPU).

Restates the GPU-provider list contracts the reference tests for Metal:
data preflight is list-atomic, a softmax or float-to-I32 cast whose input
is written earlier in the same list is rejected with UNSUPPORTED before
anything runs, and the first failing command in list order decides the
status (tests/test_metal_basic_softmax.c:242-357,
tests/test_metal_cast.c:294-424). Also covers the provider's cache of
clean inputs: a later host write or kernel output must be rescanned.
"""
import math
import sys

import numpy as np
import pytest

from conftest import m3
from harness import HipFixture, ViewSpec, as_bytes

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
    # A producer of the softmax input earlier in the list is rejected.
    write(hip, h[3], f32([0, math.nan, 1]))
    write(hip, h[4], sentinel)
    status, message = hip.execute([(m3.OP_ADD, [left, right, sm_in]),
                                   (m3.OP_SOFTMAX, [sm_in, sm_out])])
    assert status == m3.UNSUPPORTED
    assert "depends on an earlier output" in message
    got = values(hip, h[3], 3)
    assert got[0] == 0 and math.isnan(got[1]) and got[2] == 1
    assert list(values(hip, h[4], 3)) == [-9, -9, -9]
    # A softmax output is a prior writer too.
    status, _ = hip.execute([(m3.OP_SOFTMAX, [left, sm_in]),
                             (m3.OP_SOFTMAX, [sm_in, sm_out])])
    assert status == m3.UNSUPPORTED
    assert list(values(hip, h[4], 3)) == [-9, -9, -9]


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
    # COPY then CAST of the copied (produced) values: rejected, untouched.
    status, _ = hip.execute([(m3.OP_COPY, [src, middle]),
                             (m3.OP_CAST, [middle, dst])])
    assert status == m3.UNSUPPORTED
    assert list(values(hip, h[1], 4)) == [9, 8, 7, 6]
    assert list(values(hip, h[2], 4, np.int32)) == [77, 78, 79, 80]
    # Earlier invalid cast wins over a later dependent one.
    status, _ = hip.execute([(m3.OP_CAST, [src, dst]),
                             (m3.OP_COPY, [src, middle]),
                             (m3.OP_CAST, [middle, dst])])
    assert status == m3.OUT_OF_RANGE
    assert list(values(hip, h[1], 4)) == [9, 8, 7, 6]


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
