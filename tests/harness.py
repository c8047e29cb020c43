"""Test harness: the same command on the oracle, the compiled reference and
the HIP provider.

A case is a list of host storages (numpy uint8 buffers) and views over them
(ViewSpec: storage index, dtype, shape, byte strides, byte offset). Views
that name the same storage alias exactly as they do in the reference.

* ``run_oracle``  - oracle/liboracle.so (CPU restatement of the reference)
* ``run_ref``     - oracle/_ref/libm3ref.so (the reference's own host code),
                    when it was built in this container
* ``HipFixture``  - the product: storages on the HIP backend, commands
                    through m3_backend_execute (include/m3_backend.h)
* ``HostFixture`` - the product's CPU provider, on the host backend
"""
import ctypes
import os
from dataclasses import dataclass, field

import numpy as np

from conftest import ROOT, m3

ORACLE_PATH = os.path.join(ROOT, "oracle", "liboracle.so")
REF_PATH = os.path.join(ROOT, "oracle", "_ref", "libm3ref.so")

NP_DTYPES = {m3.F32: np.float32, m3.F16: np.uint16, m3.BF16: np.uint16,
             m3.I32: np.int32}


@dataclass
class ViewSpec:
    storage: int
    dtype: int
    shape: tuple
    strides: tuple = None  # bytes; None means row-major
    offset: int = 0        # bytes

    def byte_strides(self):
        if self.strides is not None:
            return tuple(self.strides)
        size = m3.DTYPE_SIZES[self.dtype]
        out = []
        step = size
        for dim in reversed(self.shape):
            out.append(step)
            step *= dim
        count = int(np.prod(self.shape)) if self.shape else 1
        return tuple(reversed(out)) if count else tuple(0 for _ in self.shape)

    def count(self):
        return int(np.prod(self.shape)) if self.shape else 1


class OView(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("byte_offset", ctypes.c_uint64),
                ("dtype", ctypes.c_uint32), ("rank", ctypes.c_uint32),
                ("shape", ctypes.c_uint64 * 8),
                ("byte_strides", ctypes.c_uint64 * 8)]


class RefView(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("bytes", ctypes.c_size_t),
                ("byte_offset", ctypes.c_uint64), ("dtype", ctypes.c_uint32),
                ("rank", ctypes.c_uint32), ("shape", ctypes.c_uint64 * 8),
                ("byte_strides", ctypes.c_uint64 * 8)]


_ORACLE = None
_REF = None


def oracle():
    global _ORACLE
    if _ORACLE is None:
        lib = ctypes.CDLL(ORACLE_PATH)
        for name in ("oracle_f16_to_f32", "oracle_bf16_to_f32"):
            getattr(lib, name).restype = ctypes.c_uint32
            getattr(lib, name).argtypes = [ctypes.c_uint16]
        for name in ("oracle_f32_to_f16", "oracle_f32_to_bf16"):
            getattr(lib, name).restype = ctypes.c_uint16
            getattr(lib, name).argtypes = [ctypes.c_uint32]
        P = ctypes.POINTER(OView)
        lib.oracle_binary.argtypes = [ctypes.c_uint32, P, P, P]
        lib.oracle_cast.argtypes = [P, P]
        lib.oracle_copy.argtypes = [P, P]
        lib.oracle_softmax.argtypes = [P, P]
        lib.oracle_snake1d.argtypes = [P, P, P]
        lib.oracle_gated_silu.argtypes = [P, P, P]
        lib.oracle_tanh.argtypes = [P, P]
        lib.oracle_preflight_nan.argtypes = [P]
        lib.oracle_preflight_i32.argtypes = [P]
        for name in ("oracle_f32_to_f16_array", "oracle_f32_to_bf16_array",
                     "oracle_f16_to_f32_array"):
            getattr(lib, name).argtypes = [ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.c_size_t]
        _ORACLE = lib
    return _ORACLE


def ref_available():
    return os.path.exists(REF_PATH)


def ref():
    global _REF
    if _REF is None:
        lib = ctypes.CDLL(REF_PATH)
        lib.ref_execute.argtypes = [ctypes.c_int, ctypes.POINTER(RefView),
                                    ctypes.c_size_t, ctypes.c_char_p,
                                    ctypes.c_size_t]
        lib.ref_execute.restype = ctypes.c_int
        _REF = lib
    return _REF


def _fill(struct, spec, storages):
    struct.data = storages[spec.storage].ctypes.data
    struct.byte_offset = spec.offset
    struct.dtype = spec.dtype
    struct.rank = len(spec.shape)
    for i, (dim, stride) in enumerate(zip(spec.shape, spec.byte_strides())):
        struct.shape[i] = dim
        struct.byte_strides[i] = stride


OP_OF_KIND = {m3.OP_ADD: 0, m3.OP_MUL: 1, m3.OP_SUB: 2, m3.OP_DIV: 3}


def run_oracle(kind, storages, views):
    """Runs one command on the oracle; returns (status, new storages).

    Applies the reference's data preflight first (CPU provider order:
    preflight, then execute), so a failing input leaves outputs unchanged.
    """
    lib = oracle()
    out = [s.copy() for s in storages]
    structs = []
    for spec in views:
        s = OView()
        _fill(s, spec, out)
        structs.append(s)
    refs = [ctypes.byref(s) for s in structs]
    if kind == m3.OP_SOFTMAX and lib.oracle_preflight_nan(refs[0]):
        return m3.OUT_OF_RANGE, out
    if (kind == m3.OP_CAST and views[1].dtype == m3.I32 and
            views[0].dtype != m3.I32 and lib.oracle_preflight_i32(refs[0])):
        return m3.OUT_OF_RANGE, out
    if kind in OP_OF_KIND:
        lib.oracle_binary(OP_OF_KIND[kind], *refs)
    elif kind == m3.OP_CAST:
        lib.oracle_cast(*refs)
    elif kind == m3.OP_COPY:
        lib.oracle_copy(*refs)
    elif kind == m3.OP_SOFTMAX:
        lib.oracle_softmax(*refs)
    elif kind == m3.OP_SNAKE1D:
        lib.oracle_snake1d(*refs)
    elif kind == m3.OP_GATED_SILU:
        lib.oracle_gated_silu(*refs)
    elif kind == m3.OP_TANH:
        lib.oracle_tanh(*refs)
    else:
        raise ValueError(kind)
    return m3.OK, out


def run_ref(kind, storages, views):
    """Runs one command on the compiled reference; (status, new storages)."""
    lib = ref()
    out = [s.copy() for s in storages]
    structs = (RefView * len(views))()
    for i, spec in enumerate(views):
        _fill(structs[i], spec, out)
        structs[i].bytes = out[spec.storage].nbytes
    message = ctypes.create_string_buffer(256)
    status = lib.ref_execute(kind, structs, len(views), message, 256)
    return status, out


class BackendFixture:
    """Storages and views on one backend made by `constructor`, commands
    through m3_backend_execute."""

    def __init__(self, constructor):
        self.lib, _ = m3.load()
        self.backend = ctypes.c_void_p()
        error = m3.Error()
        make = getattr(self.lib, constructor)
        m3.check(make(ctypes.byref(self.backend), ctypes.byref(error)),
                 error)
        self.storages = []
        self.keep = []

    def upload(self, arrays):
        handles = []
        for array in arrays:
            storage = ctypes.c_void_p()
            error = m3.Error()
            m3.check(self.lib.m3_storage_allocate(self.backend, array.nbytes,
                                                  16, ctypes.byref(storage),
                                                  ctypes.byref(error)), error)
            if array.nbytes:
                m3.check(self.lib.m3_storage_write(
                    storage, 0, array.ctypes.data_as(ctypes.c_void_p),
                    array.nbytes, ctypes.byref(error)), error)
            handles.append(storage)
            self.storages.append(storage)
        return handles

    def views(self, handles, specs):
        out = []
        for spec in specs:
            view = m3.TensorView()
            self.lib.m3_tensor_view_init(ctypes.byref(view))
            shape = (ctypes.c_uint64 * 8)(*spec.shape)
            strides = (ctypes.c_size_t * 8)(*spec.byte_strides())
            error = m3.Error()
            m3.check(self.lib.m3_tensor_view_strided(
                ctypes.byref(view), handles[spec.storage], spec.dtype,
                len(spec.shape), shape, strides, spec.offset,
                ctypes.byref(error)), error)
            out.append(view)
        self.keep.append(out)
        return out

    def execute(self, commands):
        """commands: list of (kind, [TensorView, ...]). Returns (status,
        message)."""
        array = (m3.Command * len(commands))()
        for i, (kind, views) in enumerate(commands):
            array[i].kind = kind
            for j, view in enumerate(views):
                array[i].descriptor.views[j] = ctypes.pointer(view)
        error = m3.Error()
        status = self.lib.m3_backend_execute(self.backend, array,
                                             len(commands), None,
                                             ctypes.byref(error))
        return status, error.text()

    def download(self, handles, arrays):
        out = []
        for handle, array in zip(handles, arrays):
            result = np.empty_like(array)
            error = m3.Error()
            if array.nbytes:
                m3.check(self.lib.m3_storage_read(
                    handle, 0, result.ctypes.data_as(ctypes.c_void_p),
                    result.nbytes, ctypes.byref(error)), error)
            out.append(result)
        return out

    def run(self, kind, storages, views):
        handles = self.upload(storages)
        tensor_views = self.views(handles, views)
        status, message = self.execute([(kind, tensor_views)])
        return status, self.download(handles, storages), message

    def close(self):
        for storage in self.storages:
            self.lib.m3_storage_free(storage)
        self.storages = []
        if self.backend:
            self.lib.m3_backend_free(self.backend)
            self.backend = ctypes.c_void_p()


class HipFixture(BackendFixture):
    """The HIP backend (m3_backend_create_hip): the GPU provider."""

    def __init__(self):
        super().__init__("m3_backend_create_hip")


class HostFixture(BackendFixture):
    """The host backend (m3_backend_create_host): the CPU provider."""

    def __init__(self):
        super().__init__("m3_backend_create_host")


def as_bytes(array):
    """Raw bytes of a numpy array as a uint8 storage buffer."""
    return np.ascontiguousarray(array).view(np.uint8).reshape(-1).copy()


def f32_bits(values):
    return np.asarray(values, dtype=np.float32).view(np.uint32)


def bits_f32(bits):
    return np.asarray(bits, dtype=np.uint32).view(np.float32)


# Row sums z (a count of zero logits, each e = 1) for which RN_f64(1/z) is
# far enough from 1/z that RN_f32(e * RN_f64(1/z)) misses the tie of some
# subnormal quotients e / z = (2k+1) * 2^-150 (found by enumerating every
# even z below 300; smaller ones round back onto the tie).
TIE_SUMS = (98, 150, 154, 182, 186, 198)


def _tie_logits(rng, z, count):
    """Up to `count` logits v with expf(v) = e subnormal and e / z an exact
    rounding midpoint that the product with the reciprocal rounds the wrong
    way."""
    import ctypes
    import ctypes.util

    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    m = z // 2
    k = rng.integers(0, (1 << 16) // m, 8 * count + 64).astype(np.int64)
    a = m * (2 * k + 1)
    product = (a * 2.0 ** -149 * (1.0 / np.float64(z))).astype(np.float32)
    correct = np.where(k % 2 == 0, k, k + 1)  # the even neighbour
    wrong = a[product.view(np.uint32).astype(np.int64) != correct]
    found = []
    for target in wrong:
        guess = np.float32(np.log(float(target) * 2.0 ** -149))
        for step in range(-6, 7):
            v = np.uint32(int(guess.view(np.uint32)) + step).view(np.float32)
            e = np.float32(libm.expf(float(v)))
            if int(e.view(np.uint32)) == int(target):
                found.append(v)
                break
        if len(found) == count:
            break
    return np.array(found, np.float32)


def subnormal_tie_rows(rng, rows, width):
    """Softmax rows whose quotients e_j / sum fall exactly on rounding
    midpoints of the F32 subnormal range: z zeros (each e = 1, so sum = z
    exactly, z from TIE_SUMS) followed by logits whose e_j = expf(v) is a
    subnormal with e_j / z = (2k+1) * 2^-150, chosen where a product with
    the reciprocal in double rounds the other way, then -inf. Row 0 is
    [98 zeros, -0x1.892ae8p+6, -inf...] (147 * 2^-149 / 98 = 3 * 2^-150).
    Needs width >= 100."""
    sums = [z for z in TIE_SUMS if z + 2 <= width]
    assert sums, "tie rows need width >= 100"
    logits = np.full((rows, width), -np.inf, np.float32)
    for r in range(rows):
        z = sums[r % len(sums)]
        logits[r, :z] = 0.0
        ties = _tie_logits(rng, z, min(64, (width - z) * 3 // 4))
        logits[r, z:z + ties.size] = ties
        rng.shuffle(logits[r, :z + ties.size])
    logits[0, :] = -np.inf
    logits[0, :98] = 0.0
    logits[0, 98] = np.float32(float.fromhex("-0x1.892ae8p+6"))
    return logits


class HipScanFixture:
    """One HIP device handle and one arena, driven through the C-ABI
    (include/m3_hip.h): upload host arrays, describe them as m3_hip_view
    blocks, and call a data-scan entry point by name."""

    def __init__(self, arena_bytes=1 << 26):
        _, self.hip = m3.load()
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        self.hip.m3_hip_arena_reserve.argtypes = [vp, sz,
                                                  ctypes.POINTER(vp),
                                                  ctypes.c_char_p, sz]
        self.hip.m3_hip_arena_release.argtypes = [vp, vp]
        self.hip.m3_hip_copy_h2d.argtypes = [vp, vp, vp, sz,
                                             ctypes.c_char_p, sz]
        self.message = ctypes.create_string_buffer(256)
        self.device = ctypes.c_void_p()
        assert self.hip.m3_hip_device_open(0, ctypes.byref(self.device),
                                           self.message, 256) == 0
        self.base = ctypes.c_void_p()
        assert self.hip.m3_hip_arena_reserve(self.device, arena_bytes,
                                             ctypes.byref(self.base),
                                             self.message, 256) == 0
        self.size = arena_bytes
        self.used = 0

    def upload(self, array):
        """Copies `array` into the arena (256-byte aligned); its address."""
        data = np.ascontiguousarray(array)
        at = self.base.value + self.used
        assert self.used + data.nbytes <= self.size
        self.used += (data.nbytes + 255) // 256 * 256
        assert self.hip.m3_hip_copy_h2d(
            self.device, ctypes.c_void_p(at),
            data.ctypes.data_as(ctypes.c_void_p), data.nbytes,
            self.message, 256) == 0, self.message.value
        return at

    @staticmethod
    def view(address, dtype, shape, strides=None):
        size = m3.DTYPE_SIZES[dtype]
        view = m3.HipView()
        view.base = address
        view.rank = len(shape)
        view.dtype = dtype
        view.element_count = int(np.prod(shape)) if shape else 1
        step = size
        dense = []
        for dim in reversed(shape):
            dense.append(step)
            step *= dim
        dense = list(reversed(dense))
        for axis, dim in enumerate(shape):
            view.shape[axis] = dim
            view.byte_strides[axis] = (strides or dense)[axis]
        return view

    def scan(self, entry, kinds, views):
        """Calls entry(device, kinds, views, count, flags, ...); returns
        (code, flags, message)."""
        count = len(views)
        kind_array = (ctypes.c_uint32 * max(count, 1))(*kinds)
        view_array = (m3.HipView * max(count, 1))(*views)
        flags = (ctypes.c_uint32 * max(count, 1))(*([7] * max(count, 1)))
        code = getattr(self.hip, entry)(self.device, kind_array, view_array,
                                        count, flags, self.message, 256)
        return code, list(flags[:count]), self.message.value.decode()

    def begin(self, kinds, views):
        """m3_hip_scan_views_begin; returns (code, ticket, message)."""
        count = len(views)
        kind_array = (ctypes.c_uint32 * max(count, 1))(*kinds)
        view_array = (m3.HipView * max(count, 1))(*views)
        ticket = ctypes.c_uint32(0)
        code = self.hip.m3_hip_scan_views_begin(
            self.device, kind_array, view_array, count, ctypes.byref(ticket),
            self.message, 256)
        return code, ticket.value, self.message.value.decode()

    def collect(self, ticket, count):
        """m3_hip_scan_views_collect; returns (code, flags, message)."""
        flags = (ctypes.c_uint32 * max(count, 1))(*([7] * max(count, 1)))
        code = self.hip.m3_hip_scan_views_collect(
            self.device, ticket, count, flags, self.message, 256)
        return code, list(flags[:count]), self.message.value.decode()

    def close(self):
        if self.base.value:
            self.hip.m3_hip_arena_release(self.device, self.base)
        self.hip.m3_hip_device_close(self.device)
