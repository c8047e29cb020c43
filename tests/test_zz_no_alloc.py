"""m3_hip_scan_views_static, the scan that allocates nothing (GPU).

It must give exactly what m3_hip_scan_views gives on the same views: two
calls in a row, the second with fewer views over a smaller input (so the
words the first call marked but the second does not use must not leak
into its results), NaN and I32-range kinds, contiguous, strided, F16, BF16
and zero-element views. More views than its static array holds is rejected
with a message. On a freshly opened handle, before any allocating scan has
made the device's flag words, the static scan changes the library's count
of device and pinned allocations (m3_hip_allocation_count) by nothing.
"""
import ctypes

import numpy as np
import pytest

from conftest import m3
from harness import HipScanFixture

pytestmark = pytest.mark.gpu

NAN, I32_RANGE = 0, 1


def allocations():
    _, hip = m3.load()
    count = ctypes.c_uint64(0)
    hip.m3_hip_allocation_count.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    assert hip.m3_hip_allocation_count(ctypes.byref(count)) == 0
    return count.value


def test_static_scan_allocates_nothing_on_a_fresh_handle(gpu):
    scan = HipScanFixture()
    try:
        rng = np.random.default_rng(5)
        data = rng.standard_normal(1 << 20).astype(np.float32)
        data[12345] = np.nan
        brain = (rng.standard_normal(999).astype(np.float32).view(np.uint32)
                 >> 16).astype(np.uint16)
        brain[7] = 0x7fc1  # a BF16 NaN
        a = scan.upload(data)
        b = scan.upload(brain)
        kinds = [NAN, NAN, I32_RANGE, NAN]
        views = [scan.view(a, m3.F32, (1 << 20,)),
                 scan.view(b, m3.BF16, (999,)),
                 scan.view(a, m3.F32, (0,)),
                 scan.view(b, m3.BF16, (7,))]
        before = allocations()
        code, got, message = scan.scan("m3_hip_scan_views_static", kinds,
                                       views)
        assert code == 0, message
        code, again, message = scan.scan("m3_hip_scan_views_static", kinds,
                                         views)
        assert code == 0, message
        assert allocations() == before
        assert got == again == [1, 1, 0, 0]
        # the allocating scan agrees (and makes its flag words now)
        code, want, message = scan.scan("m3_hip_scan_views", kinds, views)
        assert code == 0, message
        assert want == got
        assert allocations() > before
    finally:
        scan.close()


def test_static_scan_equals_the_allocating_scan(gpu):
    scan = HipScanFixture()
    try:
        rng = np.random.default_rng(21)
        big = rng.standard_normal(1 << 22).astype(np.float32)
        big_nan = big.copy()
        big_nan[(1 << 22) - 5] = np.nan
        huge = np.full(1 << 16, 5.0e9, np.float32)
        small = rng.standard_normal(1000).astype(np.float32)
        small_nan = small.copy()
        small_nan[3] = np.nan
        half = rng.standard_normal(777).astype(np.float16)
        a = {name: scan.upload(array) for name, array in
             (("big", big), ("big_nan", big_nan), ("huge", huge),
              ("small", small), ("small_nan", small_nan),
              ("half", half.view(np.uint16)))}
        first = ([NAN, NAN, I32_RANGE, NAN, I32_RANGE, NAN],
                 [scan.view(a["big"], m3.F32, (1 << 22,)),
                  scan.view(a["big_nan"], m3.F32, (1 << 22,)),
                  scan.view(a["huge"], m3.F32, (1 << 16,)),
                  scan.view(a["big_nan"], m3.F32, (1 << 21,), (8,)),
                  scan.view(a["big"], m3.F32, (1 << 22,)),
                  scan.view(a["half"], m3.F16, (777,))])
        # fewer views, smaller inputs; view 1 is now clean where the first
        # call's view 1 was not
        second = ([NAN, NAN, NAN],
                  [scan.view(a["small_nan"], m3.F32, (1000,)),
                   scan.view(a["small"], m3.F32, (1000,)),
                   scan.view(a["small"], m3.F32, (500,), (8,))])
        for kinds, views in (first, second):
            code, want, message = scan.scan("m3_hip_scan_views", kinds,
                                            views)
            assert code == 0, message
            code, got, message = scan.scan("m3_hip_scan_views_static",
                                           kinds, views)
            assert code == 0, message
            assert got == want
        assert scan.scan("m3_hip_scan_views_static", first[0],
                         first[1])[1] == [0, 1, 1, 0, 0, 0]
        assert scan.scan("m3_hip_scan_views_static", second[0],
                         second[1])[1] == [1, 0, 0]
        code, _, message = scan.scan(
            "m3_hip_scan_views_static", [NAN] * 65,
            [scan.view(a["small"], m3.F32, (1000,))] * 65)
        assert code != 0 and "64" in message
    finally:
        scan.close()
