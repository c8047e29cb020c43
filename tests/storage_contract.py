"""The storage contract of a backend, after the reference's own test of
its GPU backend's storage (tests/test_metal_runtime.c:40-172): allocation
statistics (live and peak), exact round trips at offset 0 and at nonzero
offsets, empty transfers at the boundary, OUT_OF_RANGE past it,
INVALID_ARGUMENT for a NULL buffer and a bad alignment (with the output
cleared), and statistics after frees. Shared by test_storage_cpu.py (host
backend) and test_gpu_storage.py (HIP backend).
"""
import ctypes

import numpy as np

from conftest import m3


def _stats(lib, backend):
    stats = m3.AllocationStats()
    error = m3.Error()
    assert lib.m3_backend_get_allocation_stats(backend, ctypes.byref(stats),
                                               ctypes.byref(error)) == m3.OK
    return (stats.live_allocated_bytes, stats.peak_allocated_bytes,
            stats.live_storage_count, stats.peak_storage_count)


def _ptr(array):
    return array.ctypes.data_as(ctypes.c_void_p)


def check_storage_contract(constructor, device_memory):
    lib, _ = m3.load()
    backend = ctypes.c_void_p()
    error = m3.Error()
    assert getattr(lib, constructor)(ctypes.byref(backend),
                                     ctypes.byref(error)) == m3.OK
    try:
        _check(lib, backend, device_memory)
    finally:
        lib.m3_backend_free(backend)


def _check(lib, backend, device_memory):
    size = 1000
    source = np.arange(size, dtype=np.uint32).astype(np.uint8)
    error = m3.Error()
    info = m3.BackendInfo()
    assert lib.m3_backend_get_info(backend, ctypes.byref(info),
                                   ctypes.byref(error)) == m3.OK
    assert info.maximum_storage_bytes >= size
    assert all(32 <= c < 127 for c in info.name.rstrip(b"\0"))
    assert _stats(lib, backend) == (0, 0, 0, 0)

    storage = ctypes.c_void_p()
    assert lib.m3_storage_allocate(backend, size, 16, ctypes.byref(storage),
                                   ctypes.byref(error)) == m3.OK
    assert lib.m3_storage_size(storage) == size
    assert lib.m3_storage_backend(storage) == backend.value
    # device memory has no host address; its backend address exists
    assert (lib.m3_storage_data(storage) is None) == device_memory
    assert lib.m3_storage_device_data(storage) is not None
    assert _stats(lib, backend) == (size, size, 1, 1)

    assert lib.m3_storage_write(storage, 0, _ptr(source), size,
                                ctypes.byref(error)) == m3.OK
    back = np.zeros(size, np.uint8)
    assert lib.m3_storage_read(storage, 0, _ptr(back), size,
                               ctypes.byref(error)) == m3.OK
    assert np.array_equal(back, source)

    # subranges at nonzero offsets: small writes (the HIP backend carries
    # writes of at most 256 bytes in a kernel's arguments) and large ones
    expected = source.copy()
    rng = np.random.default_rng(8)
    for offset, length in ((5, 7), (600, 256), (333, 257), (1, 400),
                           (size - 3, 3)):
        piece = rng.integers(0, 256, length, dtype=np.uint8)
        assert lib.m3_storage_write(storage, offset, _ptr(piece), length,
                                    ctypes.byref(error)) == m3.OK
        expected[offset:offset + length] = piece
        got = np.zeros(length, np.uint8)
        assert lib.m3_storage_read(storage, offset, _ptr(got), length,
                                   ctypes.byref(error)) == m3.OK
        assert np.array_equal(got, piece)
    assert lib.m3_storage_read(storage, 0, _ptr(back), size,
                               ctypes.byref(error)) == m3.OK
    assert np.array_equal(back, expected)

    assert lib.m3_storage_write(storage, size, None, 0,
                                ctypes.byref(error)) == m3.OK
    assert lib.m3_storage_write(storage, size, _ptr(source), 1,
                                ctypes.byref(error)) == m3.OUT_OF_RANGE
    assert lib.m3_storage_read(storage, size - 1, _ptr(back), 2,
                               ctypes.byref(error)) == m3.OUT_OF_RANGE
    assert lib.m3_storage_write(storage, 0, None, 1,
                                ctypes.byref(error)) == m3.INVALID_ARGUMENT

    temporary = ctypes.c_void_p(1)
    assert lib.m3_storage_allocate(backend, size, 3, ctypes.byref(temporary),
                                   ctypes.byref(error)) == \
        m3.INVALID_ARGUMENT
    assert temporary.value is None
    too_big = info.maximum_storage_bytes + 1
    if too_big < 2 ** 64:
        assert lib.m3_storage_allocate(backend, too_big, 16,
                                       ctypes.byref(temporary),
                                       ctypes.byref(error)) == \
            m3.OUT_OF_RANGE
    assert lib.m3_storage_allocate(backend, size, 16, ctypes.byref(temporary),
                                   ctypes.byref(error)) == m3.OK
    lib.m3_storage_free(temporary)
    assert _stats(lib, backend) == (size, 2 * size, 1, 2)
    lib.m3_storage_free(storage)
    assert _stats(lib, backend)[0::2] == (0, 0)
